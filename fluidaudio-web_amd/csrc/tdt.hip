// Greedy TDT decoding on the GPU (the step after the encoder): joint network,
// prediction network (2-layer LSTM) and the TDT token / duration loop for a
// batch of windows, reading the encoder's pre-projected frames in place.
//
// Restates rust/parakeet-decoder/src/lib.rs decode_proj (:285-318) in f32,
// operation by operation: the decoder's own polynomial expf (:47-54) with its
// floorf / ldexpf (:55-62), sigmoid and tanhf (:44, :63), 4-lane dot products
// summed lane by lane (:108-121), the iofc LSTM step (:124-137), the pred
// projection (:148-162), the joint logits accumulated over hidden units in
// order with zero activations skipped (:164-217), first-maximum argmax and the
// TDT advance (durations 0..4, at most 10 symbols per frame).  This file is
// compiled with -ffp-contract=off (no multiply-add is fused), so token ids and
// frames equal the reference's.
//
// The windows advance in lock-step, one decoding step per kernel sequence:
//   tdt_joint_kernel    logit m per thread, a group of 4 windows' accumulators
//                       in registers (the joint matrix is read once per step
//                       per window group); per-block argmax per window
//   tdt_update_kernel   per window: final argmax, token record, TDT advance,
//                       emit flag; H, C <- candidate state when a token was emitted
//   tdt_z_kernel        LSTM gate pre-activations: thread = (gate row, one of
//                       the dot's four lane sums), a group of windows per block
//   tdt_gates_kernel    LSTM cell -> candidate state
//   tdt_proj_kernel     pred projection (emitting windows) and the next joint
//                       input relu(frame + pred) (every active window)
// The reference's GPU decoder (src/engines/asr-parakeet/gpu-decoder.js) runs one
// workgroup per window that streams the whole joint matrix per step; batching
// the windows is what makes the matrix traffic one read per step here.
#include <algorithm>
#include <cstring>
#include <vector>

#include "fa_internal.h"
#include "attention.h"

namespace fa {

constexpr int TH = 640, TV = 8193, TL = 8198, TBLANK = 8192, TMAXSYM = 10;
constexpr int TG = 4;                      // windows per block (grid.y = window groups)
constexpr int TJB = 64;                    // joint logits per block
constexpr int TNB = (TL + TJB - 1) / TJB;  // joint blocks (129)

struct TdtWin {
  int t, T, emitted, n_out, emit, off, last;
  int cur;  // slot of the committed LSTM state; the candidate is in 1 - cur
};

struct TdtState {
  TdtWin *win;
  float *h, *c;            // [n][slot 2][layer 2][TH]: committed (cur) and candidate states
  float *pp, *j;           // [n][TH]
  float *z;                // [n][4 TH]
  float *pv;               // [n][TNB] token partial maxima
  int *pi;                 // [n][TNB]
  float *dv;               // [n]
  int *di;                 // [n]
  int *ids, *frs;          // [n][cap]
  int *alive;              // [n] window still has frames
};

__device__ __forceinline__ float tdt_floorf(float x) {
  const float i = (float)(int)x;
  return i > x ? i - 1.0f : i;
}
__device__ __forceinline__ float tdt_ldexpf(float x, int e) {
  float r = x;
  int n = e;
  while (n > 30) {
    r *= 1073741824.0f;
    n -= 30;
  }
  while (n < -30) {
    r *= 9.313225746154785e-10f;
    n += 30;
  }
  return r * __uint_as_float((unsigned)(127 + n) << 23);
}
__device__ __forceinline__ float tdt_expf(float x) {
  const float xc = x > 30.0f ? 30.0f : (x < -30.0f ? -30.0f : x);
  const float t = xc * 1.4426950408889634f;
  const float fl = tdt_floorf(t);
  const float frac = t - fl;
  const float p = 1.0f + frac * (0.6931472f + frac * (0.2402265f + frac * (0.0555041f + frac * 0.0096181f)));
  return tdt_ldexpf(p, (int)fl);
}
__device__ __forceinline__ float tdt_sigmoid(float x) { return 1.0f / (1.0f + tdt_expf(-x)); }
__device__ __forceinline__ float tdt_tanhf(float x) {
  const float e = tdt_expf(2.0f * x);
  return (e - 1.0f) / (e + 1.0f);
}
__device__ __forceinline__ bool better(float v, int i, float bv, int bi) { return v > bv || (v == bv && i < bi); }

// Block-wide (value, index) maximum, ties to the lower index (a sequential
// scan with a strict '>' keeps the first maximum).
__device__ void block_argmax(float v, int i, float *rv, int *ri, float &ov, int &oi) {
  const int tid = threadIdx.x;
  rv[tid] = v;
  ri[tid] = i;
  __syncthreads();
  for (int s = blockDim.x / 2; s > 0; s >>= 1) {
    if (tid < s && better(rv[tid + s], ri[tid + s], rv[tid], ri[tid])) {
      rv[tid] = rv[tid + s];
      ri[tid] = ri[tid + s];
    }
    __syncthreads();
  }
  ov = rv[0];
  oi = ri[0];
  __syncthreads();
}

// Block = 64 logits, one per thread; every thread keeps the accumulators of
// a group of windows and sums over hidden units n in order (the reference's
// axpy order), the weight column loads issued ahead of the adds.  The joint
// inputs are wave-uniform (scalar loads).  The reference skips n with
// j[n] == 0; with finite weights adding 0·w changes no value (at most the sign
// of an exact zero, which compares equal), so the sum here does not branch.
__global__ __launch_bounds__(64) void tdt_joint_kernel(const float *__restrict__ out_w, const float *__restrict__ out_b,
                                                       const float *__restrict__ jin, TdtState st, int n) {
  __shared__ float rv[64];
  __shared__ int ri[64];
  const int tid = threadIdx.x, m = blockIdx.x * TJB + tid;
  const bool valid = m < TL;
  const int w0 = blockIdx.y * TG;
  bool act[TG];
  bool any = false;
#pragma unroll
  for (int g = 0; g < TG; g++) {
    act[g] = w0 + g < n && st.win[w0 + g].t < st.win[w0 + g].T;
    any |= act[g];
  }
  if (!any) return;  // uniform: every thread reads the same flags
  const float *jw[TG];
#pragma unroll
  for (int g = 0; g < TG; g++) jw[g] = jin + (size_t)(act[g] ? w0 + g : w0) * TH;  // inactive: any valid row, never used
  float acc[TG];
  const float b = valid ? out_b[m] : 0.f;
#pragma unroll
  for (int g = 0; g < TG; g++) acc[g] = b;
  const float *col = out_w + (valid ? m : 0);
  for (int k0 = 0; k0 < TH; k0 += 32) {
    float wv[32];
#pragma unroll
    for (int u = 0; u < 32; u++) wv[u] = col[(size_t)(k0 + u) * TL];
#pragma unroll
    for (int u = 0; u < 32; u++)
#pragma unroll
      for (int g = 0; g < TG; g++) acc[g] = acc[g] + jw[g][k0 + u] * wv[u];
  }
  for (int g = 0; g < TG; g++) {
    const int w = w0 + g;
    if (!act[g]) continue;  // uniform
    float bv;
    int bi;
    block_argmax((valid && m < TV) ? acc[g] : -INFINITY, (valid && m < TV) ? m : 0x7fffffff, rv, ri, bv, bi);
    if (tid == 0) {
      st.pv[w * TNB + blockIdx.x] = bv;
      st.pi[w * TNB + blockIdx.x] = bi;
    }
    if (blockIdx.x == TNB - 1) {
      block_argmax((valid && m >= TV) ? acc[g] : -INFINITY, (valid && m >= TV) ? m - TV : 0x7fffffff, rv, ri, bv, bi);
      if (tid == 0) {
        st.dv[w] = bv;
        st.di[w] = bi;
      }
    }
  }
}

// Block = one window: argmax over the joint blocks' partials (largest value,
// ties to the lower index: the reference's in-order strict '>' scan), token
// record, TDT advance, and the commit of the candidate state when a token was
// emitted (commit_state, lib.rs:146).
__global__ __launch_bounds__(64) void tdt_update_kernel(TdtState st, int cap) {
  __shared__ float rv[64];
  __shared__ int ri[64];
  const int w = blockIdx.x, tid = threadIdx.x;
  TdtWin s = st.win[w];
  if (s.t >= s.T) {  // uniform
    if (tid == 0) {
      st.win[w].emit = 0;
      st.alive[w] = 0;
    }
    return;
  }
  float bv = -INFINITY;
  int bi = 0x7fffffff;
  for (int b = tid; b < TNB; b += 64)
    if (better(st.pv[w * TNB + b], st.pi[w * TNB + b], bv, bi)) {
      bv = st.pv[w * TNB + b];
      bi = st.pi[w * TNB + b];
    }
  float mv;
  int tok;
  block_argmax(bv, bi, rv, ri, mv, tok);
  if (tid == 0) {
    const int step = st.di[w];
    s.emit = 0;
    if (tok != TBLANK) {
      if (s.n_out < cap) {
        st.ids[(size_t)w * cap + s.n_out] = tok;
        st.frs[(size_t)w * cap + s.n_out] = s.t;
      }
      s.n_out++;
      s.emitted++;
      s.emit = 1;
      s.last = tok;
      s.cur ^= 1;  // commit_state: the candidate slot becomes the committed one
    }
    if (step > 0) {
      s.t += step;
      s.emitted = 0;
    } else if (tok == TBLANK || s.emitted >= TMAXSYM) {
      s.t += 1;
      s.emitted = 0;
    }
    st.win[w] = s;
    st.alive[w] = s.t < s.T;
  }
}

// Gate pre-activations of one LSTM layer for the windows that emitted:
// z[r] = ((b[r] + b[4H + r]) + W[r]·x) + R[r]·h.  The reference's dot keeps
// four lane sums (k = l mod 4, k ascending) added as ((s0 + s1) + s2) + s3, so
// each lane sum is one thread here: thread = (gate row r, lane l), 64 rows x
// 4 lanes per block, a group of windows per block (x and h staged in LDS); W
// and R are stored k-major (WT[k][r]) so the loads of a k are contiguous
// across rows.  Layer 0 reads x = embed[last token], layer 1 x = the layer-0
// candidate hidden state.
__global__ __launch_bounds__(256) void tdt_z_kernel(const float *__restrict__ WT, const float *__restrict__ RT, const float *__restrict__ B,
                                                    const float *__restrict__ embed, int layer, TdtState st, int n) {
  __shared__ float xs[TG][TH], hsm[TG][TH];
  __shared__ float part[2][TG][64][4];
  const int l = threadIdx.x & 3, rl = threadIdx.x >> 2, r = blockIdx.x * 64 + rl;  // 40 blocks
  const int w0 = blockIdx.y * TG;
  bool any = false;
  for (int g = 0; g < TG && w0 + g < n; g++) any |= st.win[w0 + g].emit != 0;
  if (!any) return;
  for (int e = threadIdx.x; e < TG * TH; e += 256) {
    const int g = e / TH, k = e % TH, w = w0 + g;
    float xv = 0.f, hv = 0.f;
    if (w < n && st.win[w].emit) {
      const int cur = st.win[w].cur;
      xv = layer == 0 ? embed[(size_t)st.win[w].last * TH + k] : st.h[(((size_t)w * 2 + (cur ^ 1)) * 2 + 0) * TH + k];
      hv = st.h[(((size_t)w * 2 + cur) * 2 + layer) * TH + k];
    }
    xs[g][k] = xv;
    hsm[g][k] = hv;
  }
  __syncthreads();
  float aw[TG], ar[TG];
#pragma unroll
  for (int g = 0; g < TG; g++) aw[g] = ar[g] = 0.f;
  for (int i0 = 0; i0 < TH / 4; i0 += 32) {
    float wv[32], rv[32];
#pragma unroll
    for (int u = 0; u < 32; u++) {
      const int k = 4 * (i0 + u) + l;
      wv[u] = WT[(size_t)k * 4 * TH + r];
      rv[u] = RT[(size_t)k * 4 * TH + r];
    }
#pragma unroll
    for (int u = 0; u < 32; u++) {
      const int k = 4 * (i0 + u) + l;
#pragma unroll
      for (int g = 0; g < TG; g++) {
        aw[g] = aw[g] + wv[u] * xs[g][k];
        ar[g] = ar[g] + rv[u] * hsm[g][k];
      }
    }
  }
#pragma unroll
  for (int g = 0; g < TG; g++) {
    part[0][g][rl][l] = aw[g];
    part[1][g][rl][l] = ar[g];
  }
  __syncthreads();
  if (l == 0) {
    const float b = B[r] + B[4 * TH + r];
    for (int g = 0; g < TG; g++) {
      const int w = w0 + g;
      if (w < n && st.win[w].emit) {
        const float *pw = part[0][g][rl], *pr = part[1][g][rl];
        const float dw = pw[0] + pw[1] + pw[2] + pw[3];
        const float dr = pr[0] + pr[1] + pr[2] + pr[3];
        st.z[(size_t)w * 4 * TH + r] = b + dw + dr;
      }
    }
  }
}

// LSTM cell of one layer: thread = (hidden unit, window).
__global__ __launch_bounds__(256) void tdt_gates_kernel(int layer, TdtState st) {
  const int w = blockIdx.y, g = blockIdx.x * 256 + threadIdx.x;
  if (g >= TH || !st.win[w].emit) return;
  const float *z = st.z + (size_t)w * 4 * TH;
  const float zi = z[g], zo = z[TH + g], zf = z[2 * TH + g], zc = z[3 * TH + g];
  const int cur = st.win[w].cur;
  const size_t o = (((size_t)w * 2 + cur) * 2 + layer) * TH + g, on = (((size_t)w * 2 + (cur ^ 1)) * 2 + layer) * TH + g;
  const float cc = tdt_sigmoid(zf) * st.c[o] + tdt_sigmoid(zi) * tdt_tanhf(zc);
  st.c[on] = cc;
  st.h[on] = tdt_sigmoid(zo) * tdt_tanhf(cc);
}

// Pred projection of one window if it emitted (pp[n] = b[n] + Σ_k dec[k] w[k][n],
// k in order; dec arrives as scalar loads), then its next joint input
// j = relu(frame[t] + pp) if it is still active.  Block = 64 output units x one
// window (10 x n blocks); weight loads issued ahead of the adds.
__global__ __launch_bounds__(64) void tdt_proj_kernel(const float *__restrict__ pw, const float *__restrict__ pb, const float *__restrict__ frames,
                                                      const float *__restrict__ hs, TdtState st) {
  const int u = blockIdx.x * 64 + threadIdx.x, w = blockIdx.y;
  const TdtWin s = st.win[w];
  if (__builtin_amdgcn_readfirstlane(s.emit)) {  // uniform
    const float *dec = hs + (((size_t)w * 2 + (__builtin_amdgcn_readfirstlane(s.cur) ^ 1)) * 2 + 1) * TH;
    float acc = pb[u];
    for (int k0 = 0; k0 < TH; k0 += 64) {
      float wv[64];
#pragma unroll
      for (int q = 0; q < 64; q++) wv[q] = pw[(size_t)(k0 + q) * TH + u];
#pragma unroll
      for (int q = 0; q < 64; q++) acc = acc + dec[k0 + q] * wv[q];
    }
    st.pp[(size_t)w * TH + u] = acc;
  }
  if (s.t < s.T) {
    const float v = frames[(size_t)(s.off + s.t) * TH + u] + st.pp[(size_t)w * TH + u];
    st.j[(size_t)w * TH + u] = v > 0.0f ? v : 0.0f;
  }
}

}  // namespace fa

using namespace fa;

struct fa_tdt {
  fa_ctx *ctx = nullptr;
  float *embed = nullptr, *lw[2] = {}, *lr[2] = {}, *lb[2] = {}, *pred_w = nullptr, *pred_b = nullptr, *out_w = nullptr, *out_b = nullptr;
  void *state = nullptr;
  size_t state_bytes = 0;
};

extern "C" {

int fa_tdt_load(fa_ctx *ctx, const float *const *w, fa_tdt **out) {
  if (!ctx || !w || !out) return FA_E_INVALID;
  static const size_t sizes[11] = {(size_t)TV * TH, 4u * TH * TH, 4u * TH * TH, 8u * TH, 4u * TH * TH, 4u * TH * TH, 8u * TH,
                                   (size_t)TH * TH, TH, (size_t)TH * TL, TL};
  for (int i = 0; i < 11; i++)
    if (!w[i]) return set_err(ctx, FA_E_INVALID, "tdtLoad: weight %d missing", i);
  fa_tdt *d = new fa_tdt();
  d->ctx = ctx;
  float **dst[11] = {&d->embed, &d->lw[0], &d->lr[0], &d->lb[0], &d->lw[1], &d->lr[1], &d->lb[1], &d->pred_w, &d->pred_b, &d->out_w, &d->out_b};
  for (int i = 0; i < 11; i++) {
    float *p = (float *)dev_alloc(ctx, sizes[i] * 4);
    if (!p) {
      fa_tdt_destroy(d);
      return FA_E_OOM;
    }
    *dst[i] = p;
    const float *src = w[i];
    std::vector<float> tr;
    if (i == 1 || i == 2 || i == 4 || i == 5) {  // LSTM W / R [4H][H] -> k-major [H][4H]
      tr.resize(sizes[i]);
      for (int r = 0; r < 4 * TH; r++)
        for (int k = 0; k < TH; k++) tr[(size_t)k * 4 * TH + r] = src[(size_t)r * TH + k];
      src = tr.data();
    }
    if (hipMemcpy(p, src, sizes[i] * 4, hipMemcpyHostToDevice) != hipSuccess) {
      fa_tdt_destroy(d);
      return set_err(ctx, FA_E_DEVICE, "tdtLoad: upload of weight %d failed", i);
    }
  }
  *out = d;
  return FA_OK;
}

void fa_tdt_destroy(fa_tdt *d) {
  if (!d) return;
  if (d->ctx) (void)hipStreamSynchronize(d->ctx->stream);
  float *ps[11] = {d->embed, d->lw[0], d->lr[0], d->lb[0], d->lw[1], d->lr[1], d->lb[1], d->pred_w, d->pred_b, d->out_w, d->out_b};
  for (float *p : ps)
    if (p) (void)hipFree(p);
  if (d->state) (void)hipFree(d->state);
  delete d;
}

int fa_tdt_decode(fa_tdt *d, fa_tensor frames, const int32_t *lens, int n, int cap, int32_t *ids, int32_t *frame_idx, int32_t *counts) {
  if (!d) return FA_E_INVALID;
  fa_ctx *ctx = d->ctx;
  TensorRec *rf;
  FA_TRY(need(ctx, frames, &rf, "tdtDecode"));
  if (rf->kind != S_F32 || rf->cols != TH) return set_err(ctx, FA_E_INVALID, "tdtDecode: frames must be f32 [rows, %d] (pre-projected)", TH);
  if (n <= 0 || n > kMaxWin) return set_err(ctx, FA_E_INVALID, "tdtDecode: %d windows (1..%d)", n, kMaxWin);
  if (cap <= 0) return set_err(ctx, FA_E_INVALID, "tdtDecode: capacity %d", cap);
  std::vector<TdtWin> win(n);
  long off = 0;
  int tmax = 0;
  for (int i = 0; i < n; i++) {
    if (lens[i] < 0) return set_err(ctx, FA_E_INVALID, "tdtDecode: window %d length %d", i, lens[i]);
    win[i] = TdtWin{0, lens[i], 0, 0, lens[i] > 0 ? 1 : 0, (int)off, TBLANK, 0};  // committed state in slot 0 (zero)
    off += lens[i];
    tmax = std::max(tmax, lens[i]);
  }
  if (off > rf->rows) return set_err(ctx, FA_E_INVALID, "tdtDecode: %ld frames in the windows, %d in the tensor", off, rf->rows);
  // state layout
  size_t o = 0;
  auto take = [&](size_t bytes) {
    const size_t at = o;
    o += (bytes + 255) & ~(size_t)255;
    return at;
  };
  const size_t o_win = take(sizeof(TdtWin) * n), o_h = take(4ul * n * 4 * TH), o_c = take(4ul * n * 4 * TH), o_pp = take(4ul * n * TH), o_j = take(4ul * n * TH), o_z = take(4ul * n * 4 * TH),
               o_pv = take(4ul * n * TNB), o_pi = take(4ul * n * TNB), o_dv = take(4ul * n), o_di = take(4ul * n), o_ids = take(4ul * n * cap),
               o_frs = take(4ul * n * cap), o_act = take(4ul * n);
  if (d->state_bytes < o) {
    if (d->state) {
      FA_HIP(ctx, hipStreamSynchronize(ctx->stream));
      (void)hipFree(d->state);
      d->state = nullptr;
      d->state_bytes = 0;
    }
    if (!(d->state = dev_alloc(ctx, o))) return FA_E_OOM;
    d->state_bytes = o;
  }
  char *base = (char *)d->state;
  TdtState st;
  st.win = (TdtWin *)(base + o_win);
  st.h = (float *)(base + o_h);
  st.c = (float *)(base + o_c);
  st.pp = (float *)(base + o_pp);
  st.j = (float *)(base + o_j);
  st.z = (float *)(base + o_z);
  st.pv = (float *)(base + o_pv);
  st.pi = (int *)(base + o_pi);
  st.dv = (float *)(base + o_dv);
  st.di = (int *)(base + o_di);
  st.ids = (int *)(base + o_ids);
  st.frs = (int *)(base + o_frs);
  st.alive = (int *)(base + o_act);
  rf = get(ctx, frames);
  const float *fr = (const float *)rf->ptr;
  const int ng = (n + TG - 1) / TG;  // window groups
  FA_HIP(ctx, hipMemsetAsync(base + o_h, 0, o_pp - o_h, ctx->stream));  // both state slots = 0
  FA_HIP(ctx, hipMemcpyAsync(st.win, win.data(), sizeof(TdtWin) * n, hipMemcpyHostToDevice, ctx->stream));
  auto predict = [&]() -> int {  // candidate state + pred projection for windows with emit set
    for (int layer = 0; layer < 2; layer++) {
      {
        ProfScope ps(ctx, "tdt_lstm_z");
        FA_LAUNCH(ps, tdt_z_kernel, dim3(4 * TH / 64, ng), dim3(256), 0, ctx->stream, d->lw[layer], d->lr[layer], d->lb[layer], d->embed, layer,
                  st, n);
      }
      ProfScope ps(ctx, "tdt_lstm_cell");
      FA_LAUNCH(ps, tdt_gates_kernel, dim3(cdiv(TH, 256), n), dim3(256), 0, ctx->stream, layer, st);
    }
    ProfScope ps(ctx, "tdt_proj");
    FA_LAUNCH(ps, tdt_proj_kernel, dim3(TH / 64, n), dim3(64), 0, ctx->stream, d->pred_w, d->pred_b, fr, (const float *)st.h, st);
    return check_launch(ctx, "tdt_predict");
  };
  FA_TRY(predict());  // predict(BLANK) from the zero state, then j for t = 0
  // steps in chunks; each step advances a window's frame or emits a token, and
  // a frame emits at most 10 tokens, so 11 * Tmax steps bound the loop
  const long max_steps = 11L * tmax + 1;
  constexpr int kChunk = 16;
  int active = 1;
  std::vector<int> alive(n);
  for (long s = 0; s < max_steps && active; s += kChunk) {
    for (int k = 0; k < kChunk; k++) {
      {
        ProfScope ps(ctx, "tdt_joint");
        FA_LAUNCH(ps, tdt_joint_kernel, dim3(TNB, ng), dim3(64), 0, ctx->stream, d->out_w, d->out_b, (const float *)st.j, st, n);
      }
      {
        ProfScope ps(ctx, "tdt_update");
        FA_LAUNCH(ps, tdt_update_kernel, dim3(n), dim3(64), 0, ctx->stream, st, cap);
      }
      FA_TRY(predict());
    }
    FA_HIP(ctx, hipMemcpyAsync(alive.data(), st.alive, 4ul * n, hipMemcpyDeviceToHost, ctx->stream));
    FA_HIP(ctx, hipStreamSynchronize(ctx->stream));
    active = 0;
    for (int i = 0; i < n; i++) active += alive[i];
  }
  if (active) return set_err(ctx, FA_E_DEVICE, "tdtDecode: windows still active after %ld steps", max_steps);
  std::vector<TdtWin> fin(n);
  FA_HIP(ctx, hipMemcpy(fin.data(), st.win, sizeof(TdtWin) * n, hipMemcpyDeviceToHost));
  FA_HIP(ctx, hipMemcpy(ids, st.ids, 4ul * n * cap, hipMemcpyDeviceToHost));
  FA_HIP(ctx, hipMemcpy(frame_idx, st.frs, 4ul * n * cap, hipMemcpyDeviceToHost));
  for (int i = 0; i < n; i++) counts[i] = fin[i].n_out;
  return FA_OK;
}

}  // extern "C"
