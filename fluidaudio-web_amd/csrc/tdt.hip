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
//   tdt_joint_kernel    joint logits: a 64-column slab of the joint matrix
//                       streamed through LDS once per step for up to 8 live
//                       windows (a wave each); per-slab argmax per window
//   tdt_update_kernel   per window: final argmax, token record, TDT advance,
//                       emit flag; the candidate state becomes the committed one
//                       when a token was emitted
//   tdt_z_kernel        LSTM gate partial dot products: thread = gate row, block
//                       = (matrix, one of the dot's four lane sums, a group of
//                       emitting windows)
//   tdt_gates_kernel    lane sums -> gate pre-activations -> LSTM cell ->
//                       candidate state
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
constexpr int TJB = 64;                    // joint / projection columns per block (one per lane)
constexpr int TNB = (TL + TJB - 1) / TJB;  // joint column slabs (129)
constexpr int TLP = TNB * TJB;             // padded row stride of the joint matrix on the device

struct TdtWin {
  int t, T, emitted, n_out, emit, off, last;
  int cur;  // slot of the committed LSTM state; the candidate is in 1 - cur
};

struct TdtState {
  TdtWin *win;
  float *h, *c;            // [n][slot 2][layer 2][TH]: committed (cur) and candidate states
  float *pp, *j;           // [n][TH]
  float *z;                // [n][matrix 2][lane 4][4 TH] partial dot products
  float *pv;               // [n][TNB] token partial maxima
  int *pi;                 // [n][TNB]
  float *dv;               // [n]
  int *di;                 // [n]
  int *ids, *frs;          // [n][cap]
  int *alive;              // [n] window still has frames (-1: no finite joint maximum)
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

// Window groups.  A 64-thread block (lane = window, n <= 64) finds the
// windows of its group among those selected by `pred` (ranks first ..
// first + G - 1 in window order) and returns how many there are; grid rows
// past the last group exit at once.  Grouping the selected windows (rather
// than fixed runs of windows) keeps the number of blocks, and the number of
// times a weight matrix is read, to what the live windows need.
__device__ __forceinline__ int tdt_group(bool pred, int first, int G, int *lst) {
  const unsigned long long m = __ballot(pred);
  const int lane = threadIdx.x;
  const int rank = __popcll(m & ((1ull << lane) - 1ull));
  if (pred && rank >= first && rank < first + G) lst[rank - first] = lane;
  __syncthreads();
  const int cnt = __popcll(m) - first;
  return cnt < 0 ? 0 : (cnt > G ? G : cnt);
}

// acc[g] = (...((acc[g] + w(0) x(g, 0)) + w(1) x(g, 1)) ... + w(N-1) x(g, N-1)):
// the in-order sums of the reference, one chain per (thread, g).  Two named
// register buffers of B loads alternate inside a loop step of 2B, so the
// loads of one buffer are in flight while the other is summed; the prefetch
// is unconditional (clamped to the last row) so that no buffer is copied
// between iterations (a copy would wait for every load in flight).
template <int N, int B, int G, typename LW, typename XV>
__device__ __forceinline__ void chain_dot(float (&acc)[G], LW lw, XV xv) {
  static_assert(N % (2 * B) == 0, "chain length must be a whole number of buffer pairs");
  float wa[B], wb[B];
#pragma unroll
  for (int u = 0; u < B; u++) wa[u] = lw(u);
#pragma unroll 1
  for (int i0 = 0; i0 < N; i0 += 2 * B) {
#pragma unroll
    for (int u = 0; u < B; u++) wb[u] = lw(i0 + B + u);
#pragma unroll
    for (int u = 0; u < B; u++)
#pragma unroll
      for (int g = 0; g < G; g++) acc[g] = acc[g] + wa[u] * xv(g, i0 + u);
    const int nx = i0 + 2 * B < N ? i0 + 2 * B : N - B;  // last step: a harmless reload
#pragma unroll
    for (int u = 0; u < B; u++) wa[u] = lw(nx + u);
#pragma unroll
    for (int u = 0; u < B; u++)
#pragma unroll
      for (int g = 0; g < G; g++) acc[g] = acc[g] + wb[u] * xv(g, i0 + B + u);
  }
}

// Weight loads through a buffer resource: the row offset of a strided column
// walk is a scalar operand, the lane's column a 32-bit vector offset.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t tdt_rsrc(const float *p, size_t n) {
  return __builtin_amdgcn_make_buffer_rsrc((void *)p, 0, (int)(n * 4), 0x00020000);
}
__device__ __forceinline__ float tdt_ld(__amdgpu_buffer_rsrc_t r, int voff, int soff) {
  return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, voff, soff, 0));
}


// ── joint logits and pred projection: in-order sums over 640 hidden units ──
// out[w][m] = init[m] + Σ_k x[w][k] W[k][m], k ascending (the reference's
// axpy order), for a column slab of TJB = 32 columns and up to 16 windows per
// block.  The slab's rows are streamed global->LDS by global_load_lds_dwordx4
// in chunks of 64 rows, RS_S chunks in flight (no VGPR staging, so the copy
// depth does not depend on register budget: each wave walking 640 dependent
// rows on its own is latency-bound); the windows' x vectors are staged in LDS
// once and read as broadcasts.  Lane = (column c, half h); window slot
// s = wave + 4 h + 8 q (q < 2) so few windows still spread over all waves.
// W rows must be 16-byte aligned and the slab must lie inside every row.
// The reference skips k with x[k] == 0; with finite weights adding 0·w changes
// no value (at most the sign of an exact zero, which compares equal), so the
// sum does not branch.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void tdt_dma16(const void *g, uint32_t lds_addr) {
  asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(g), "s"(lds_addr) : "memory", "m0");
}
#pragma clang diagnostic pop
template <int N>
__device__ __forceinline__ void tdt_wait_vmcnt() {  // gfx9 s_waitcnt: vmcnt [3:0]+[15:14], expcnt 7, lgkmcnt 15 = no wait
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

constexpr int RS_KC = 64, RS_S = 4, RS_SLOTS = 8;  // rows per chunk, chunks in flight, windows (waves) per block

// Wave = one selected window, lane = one column of a 64-column slab: every
// lane runs one in-order chain over the 640 hidden units.  The window's input
// vector is wave-uniform and is read with scalar loads (SGPR operands of the
// multiplies; measured 18.7 us per step against 29.0 with the vector staged
// in LDS and read as broadcasts); the slab's rows are streamed global->LDS by
// global_load_lds_dwordx4 in chunks of 64 rows, RS_S chunks in flight, and
// shared by the block's 8 windows.  W rows must be 16-byte aligned and the
// slab must lie inside every row.
// Selected = windows with frames left; per-slab token maximum, and the
// duration maximum in the last slab.
__global__ __launch_bounds__(64 * RS_SLOTS) void tdt_joint_kernel(const float *__restrict__ W, int ldw, int ncols, const float *__restrict__ bias,
                                                                  const float *__restrict__ xsrc, TdtState st, int n) {
  __shared__ __attribute__((aligned(1024))) float ws[RS_S][RS_KC][TJB];
  __shared__ int lst[RS_SLOTS], lcnt;
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int slab = blockIdx.x, col = slab * TJB + lane;
  if (wave == 0) {
    const bool sel = lane < n && st.win[lane].t < st.win[lane].T;
    const unsigned long long m = __ballot(sel);
    const int first = blockIdx.y * RS_SLOTS, rank = __popcll(m & ((1ull << lane) - 1ull));
    if (sel && rank >= first && rank < first + RS_SLOTS) lst[rank - first] = lane;
    if (lane == 0) lcnt = min(max(__popcll(m) - first, 0), RS_SLOTS);
  }
  __syncthreads();
  const int cnt = lcnt;
  if (cnt == 0) return;  // uniform
  const uint32_t sb = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(__attribute__((address_space(3))) char *)&ws[0][0][0]);
  // a chunk is 64 rows x 256 B = 16 copies of 1 KB (4 rows each), two per wave
  const float *wsrc = W + (size_t)(lane >> 4) * ldw + slab * TJB + (lane & 15) * 4;
  auto issue = [&](int ch) {
#pragma unroll
    for (int i = 0; i < 2; i++) {
      const int ins = wave * 2 + i;
      tdt_dma16(wsrc + (size_t)(ch * RS_KC + ins * 4) * ldw, sb + (ch % RS_S) * (RS_KC * TJB * 4) + ins * 1024);
    }
  };
  constexpr int NCH = TH / RS_KC;
#pragma unroll
  for (int ch = 0; ch < RS_S - 1; ch++) issue(ch);
  const bool work = wave < cnt;
  const int w = __builtin_amdgcn_readfirstlane(lst[work ? wave : 0]);
  const float *xw = xsrc + (size_t)w * TH;  // wave-uniform: scalar loads, SGPR operands
  const bool valid = col < ncols;
  float acc = valid ? bias[col] : 0.f;
  for (int ch = 0; ch < NCH; ch++) {
    const int newer = min(RS_S - 2, NCH - 1 - ch);  // copies issued after chunk ch, per wave: 2 each
    if (newer >= 2) tdt_wait_vmcnt<4>();
    else if (newer == 1) tdt_wait_vmcnt<2>();
    else tdt_wait_vmcnt<0>();
    __syncthreads();  // chunk ch visible to every wave; the stage of chunk ch - 1 is free
    if (ch + RS_S - 1 < NCH) issue(ch + RS_S - 1);
    if (work) {
      const float *wr = &ws[ch % RS_S][0][lane];
      const int k0 = ch * RS_KC;
      float wA[16], wB[16], xA[16], xB[16];
      auto ld = [&](int kk, float(&wv)[16], float(&xv)[16]) {
#pragma unroll
        for (int u = 0; u < 16; u++) wv[u] = wr[(kk + u) * TJB];
#pragma unroll
        for (int u = 0; u < 16; u++) xv[u] = xw[k0 + kk + u];
      };
      auto sum = [&](const float(&wv)[16], const float(&xv)[16]) {
#pragma unroll
        for (int u = 0; u < 16; u++) acc = acc + xv[u] * wv[u];
      };
      ld(0, wA, xA);
      ld(16, wB, xB);
      sum(wA, xA);
      ld(32, wA, xA);
      sum(wB, xB);
      ld(48, wB, xB);
      sum(wA, xA);
      sum(wB, xB);
    }
  }
  if (!work) return;
  {
    float bv = (valid && col < TV) ? acc : -INFINITY;
    int bi = (valid && col < TV) ? col : 0x7fffffff;
#pragma unroll
    for (int sh = 32; sh > 0; sh >>= 1) {
      const float ov = __shfl_xor(bv, sh);
      const int oi = __shfl_xor(bi, sh);
      if (better(ov, oi, bv, bi)) {
        bv = ov;
        bi = oi;
      }
    }
    if (lane == 0) {
      st.pv[w * TNB + slab] = bv;
      st.pi[w * TNB + slab] = bi;
    }
    if (slab == TNB - 1) {
      float dv = (valid && col >= TV) ? acc : -INFINITY;
      int di = (valid && col >= TV) ? col - TV : 0x7fffffff;
#pragma unroll
      for (int sh = 32; sh > 0; sh >>= 1) {
        const float ov = __shfl_xor(dv, sh);
        const int oi = __shfl_xor(di, sh);
        if (better(ov, oi, dv, di)) {
          dv = ov;
          di = oi;
        }
      }
      if (lane == 0) {
        st.dv[w] = dv;
        st.di[w] = di;
      }
    }
  }
}

// Pred projection of the windows that emitted, pp = pred_b + h1 · pred_w
// (in-order sums over the 640 hidden units), and the next joint input
// j = relu(frame[t] + pp).  Block = one wave = ZG emitting windows x 64
// columns.  pred_w is stored column-major on the device (WT[col][k]), so a
// lane's float4 load brings 4 consecutive k of its column: 160 loads per
// chain instead of 640, streamed with two register buffers of PB loads.  The
// windows' h vectors are staged in LDS and read as broadcasts (in-order LDS
// returns let the reads run ahead of their use; scalar loads would each be
// waited for in full); each lane runs ZG chains sharing its weight loads.  The last grid row refreshes
// j of the active windows that did not emit.
template <int ZG>
__global__ __launch_bounds__(64) void tdt_proj_kernel(const float *__restrict__ WT, const float *__restrict__ bias, const float *__restrict__ hsrc,
                                                      const float *__restrict__ frames, TdtState st, int n) {
  constexpr int PB = 20, NI = TH / 4;
  static_assert(NI % (2 * PB) == 0, "whole buffer pairs");
  __shared__ int lst[ZG];
  __shared__ __attribute__((aligned(16))) float xs[ZG][TH];
  const int tid = threadIdx.x, col = blockIdx.x * 64 + tid;
  if ((int)blockIdx.y == (int)gridDim.y - 1) {
    for (int w = 0; w < n; w++) {
      const TdtWin s = st.win[w];
      if (!s.emit && s.t < s.T) {
        const float v = frames[(size_t)(s.off + s.t) * TH + col] + st.pp[(size_t)w * TH + col];
        st.j[(size_t)w * TH + col] = v > 0.0f ? v : 0.0f;
      }
    }
    return;
  }
  const bool em = tid < n && st.win[tid].emit != 0;
  const int cnt = tdt_group(em, blockIdx.y * ZG, ZG, lst);
  if (cnt == 0) return;
  const float4 *wc = reinterpret_cast<const float4 *>(WT + (size_t)col * TH);
  float acc[ZG];
  const float b0 = bias[col];
#pragma unroll
  for (int g = 0; g < ZG; g++) acc[g] = b0;
  float4 wa[PB], wb[PB];
#pragma unroll
  for (int u = 0; u < PB; u++) wa[u] = wc[u];
  // the windows' h vectors -> LDS (read back as broadcasts)
  for (int e = tid; e < ZG * TH; e += 64) {
    const int g = e / TH, k = e - g * TH, w = lst[g < cnt ? g : 0];
    xs[g][k] = hsrc[(((size_t)w * 2 + (st.win[w].cur ^ 1)) * 2 + 1) * TH + k];
  }
  __syncthreads();
  // x in groups of 4 float4 (16 k) per window, two register sets: the LDS
  // reads of group q + 1 are issued before group q is summed
  auto ldx = [&](int i, float4(&xv)[ZG][4]) {
#pragma unroll
    for (int g = 0; g < ZG; g++)
#pragma unroll
      for (int v = 0; v < 4; v++) xv[g][v] = *reinterpret_cast<const float4 *>(&xs[g][4 * (i + v)]);
  };
  auto sum4 = [&](const float4(&wv)[PB], int u0, const float4(&xv)[ZG][4]) {
#pragma unroll
    for (int v = 0; v < 4; v++) {
      const float we[4] = {wv[u0 + v].x, wv[u0 + v].y, wv[u0 + v].z, wv[u0 + v].w};
#pragma unroll
      for (int g = 0; g < ZG; g++) {
        const float xe[4] = {xv[g][v].x, xv[g][v].y, xv[g][v].z, xv[g][v].w};
#pragma unroll
        for (int e = 0; e < 4; e++) acc[g] = acc[g] + xe[e] * we[e];
      }
    }
  };
  auto sum = [&](const float4(&wv)[PB], int i0) {
    static_assert(PB % 4 == 0, "groups of 4");
    float4 xA[ZG][4], xB[ZG][4];
    ldx(i0, xA);
#pragma unroll
    for (int q = 0; q < PB / 4; q += 2) {
      if (q + 1 < PB / 4) ldx(i0 + 4 * (q + 1), xB);
      sum4(wv, 4 * q, xA);
      if (q + 1 < PB / 4) {
        if (q + 2 < PB / 4) ldx(i0 + 4 * (q + 2), xA);
        sum4(wv, 4 * (q + 1), xB);
      }
    }
  };

#pragma unroll 1
  for (int i0 = 0; i0 < NI; i0 += 2 * PB) {
#pragma unroll
    for (int u = 0; u < PB; u++) wb[u] = wc[i0 + PB + u];
    sum(wa, i0);
    const int nx = i0 + 2 * PB < NI ? i0 + 2 * PB : NI - PB;  // last step: a harmless reload
#pragma unroll
    for (int u = 0; u < PB; u++) wa[u] = wc[nx + u];
    sum(wb, i0 + PB);
  }
#pragma unroll
  for (int g = 0; g < ZG; g++) {
    if (g >= cnt) break;
    const int w = lst[g];
    st.pp[(size_t)w * TH + col] = acc[g];
    const TdtWin s = st.win[w];
    if (s.t < s.T) {
      const float v = frames[(size_t)(s.off + s.t) * TH + col] + acc[g];
      st.j[(size_t)w * TH + col] = v > 0.0f ? v : 0.0f;
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
      if (st.alive[w] > 0) st.alive[w] = 0;  // a -1 flag stays
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
    if (tok < 0 || tok >= TV || step < 0 || step >= TL - TV) {
      // no finite maximum (non-finite logits): end the window and flag it, so
      // a bad value can never become an embedding row index
      s.t = s.T;
      st.win[w] = s;
      st.alive[w] = -1;
      return;
    }
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

// Gate pre-activations of one LSTM layer for the windows that emitted,
// z[r] = ((b[r] + b[4H + r]) + W[r]·x) + R[r]·h.  The reference's dot keeps
// four lane sums (k = l mod 4, k ascending) added as ((s0 + s1) + s2) + s3;
// each lane sum of each matrix is one chain here: block = 64 gate rows (one
// per thread) x one (matrix, lane l) x a group of ZG emitting windows, so a
// wave's weight loads (W and R stored k-major, WT[k][r]) are one contiguous
// row segment and its x / h operands are LDS broadcasts.  The partial sums
// go to zp[w][matrix][l][4H]; the cell kernel adds them in the reference's
// order.  Layer 0 reads x = embed[last token], layer 1 x = the layer-0
// candidate hidden state.
template <int ZG>
__global__ __launch_bounds__(64) void tdt_z_kernel(const float *__restrict__ WT, const float *__restrict__ RT, const float *__restrict__ embed,
                                                   int layer, TdtState st, int n) {
  __shared__ int lst[ZG];
  __shared__ float xs[ZG][TH / 4];
  const int tid = threadIdx.x, l = blockIdx.x & 3, mat = (blockIdx.x >> 2) & 1, r = (blockIdx.x >> 3) * 64 + tid;
  const bool em = tid < n && st.win[tid].emit != 0;
  const int cnt = tdt_group(em, blockIdx.y * ZG, ZG, lst);
  if (cnt == 0) return;
  for (int e = tid; e < ZG * (TH / 4); e += 64) {
    const int g = e / (TH / 4), i = e % (TH / 4), w = lst[g < cnt ? g : 0];
    const TdtWin s = st.win[w];
    const float *src = mat == 1 ? st.h + (((size_t)w * 2 + s.cur) * 2 + layer) * TH
                                : (layer == 0 ? embed + (size_t)s.last * TH : st.h + (((size_t)w * 2 + (s.cur ^ 1)) * 2 + 0) * TH);
    xs[g][i] = src[4 * i + l];
  }
  __syncthreads();
  const __amdgpu_buffer_rsrc_t rm = tdt_rsrc(mat == 0 ? WT : RT, (size_t)4 * TH * TH);
  const int voff = (l * 4 * TH + r) * 4;  // row k = 4 i + l
  float acc[ZG];
#pragma unroll
  for (int g = 0; g < ZG; g++) acc[g] = 0.f;
  chain_dot<TH / 4, 40, ZG>(acc, [&](int i) { return tdt_ld(rm, voff, i * 16 * TH * 4); }, [&](int g, int i) { return xs[g][i]; });
#pragma unroll
  for (int g = 0; g < ZG; g++)
    if (g < cnt) st.z[(((size_t)lst[g] * 2 + mat) * 4 + l) * 4 * TH + r] = acc[g];
}

// LSTM cell of one layer: thread = (hidden unit, window).
__global__ __launch_bounds__(256) void tdt_gates_kernel(const float *__restrict__ B, int layer, TdtState st) {
  const int w = blockIdx.y, g = blockIdx.x * 256 + threadIdx.x;
  if (g >= TH || !st.win[w].emit) return;
  const float *zp = st.z + (size_t)w * 8 * 4 * TH;
  auto zrow = [&](int r) {
    const float dw = ((zp[r] + zp[4 * TH + r]) + zp[8 * TH + r]) + zp[12 * TH + r];
    const float dr = ((zp[16 * TH + r] + zp[20 * TH + r]) + zp[24 * TH + r]) + zp[28 * TH + r];
    return ((B[r] + B[4 * TH + r]) + dw) + dr;
  };
  const float zi = zrow(g), zo = zrow(TH + g), zf = zrow(2 * TH + g), zc = zrow(3 * TH + g);
  const int cur = st.win[w].cur;
  const size_t o = (((size_t)w * 2 + cur) * 2 + layer) * TH + g, on = (((size_t)w * 2 + (cur ^ 1)) * 2 + layer) * TH + g;
  const float cc = tdt_sigmoid(zf) * st.c[o] + tdt_sigmoid(zi) * tdt_tanhf(zc);
  st.c[on] = cc;
  st.h[on] = tdt_sigmoid(zo) * tdt_tanhf(cc);
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
  // device sizes: the joint matrix rows are padded to TLP columns (zeros), so
  // every row is 16-byte aligned and every 32-column slab lies inside it
  size_t dsz[11];
  for (int i = 0; i < 11; i++) dsz[i] = sizes[i];
  dsz[9] = (size_t)TH * TLP;
  for (int i = 0; i < 11; i++) {
    float *p = (float *)dev_alloc(ctx, dsz[i] * 4);
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
    if (i == 7) {  // pred projection [H][H] (k-major) -> column-major [col][k]
      tr.resize(sizes[i]);
      for (int k = 0; k < TH; k++)
        for (int m = 0; m < TH; m++) tr[(size_t)m * TH + k] = src[(size_t)k * TH + m];
      src = tr.data();
    }
    if (i == 9) {  // joint [H][TL] -> [H][TLP]
      tr.assign(dsz[i], 0.f);
      for (int k = 0; k < TH; k++) memcpy(&tr[(size_t)k * TLP], src + (size_t)k * TL, TL * 4);
      src = tr.data();
    }
    if (hipMemcpy(p, src, dsz[i] * 4, hipMemcpyHostToDevice) != hipSuccess) {
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
  return fa::tdt_decode_dev(d, (const float *)rf->ptr, rf->rows, lens, n, cap, ids, frame_idx, counts);
}

}  // extern "C"

// The decode of n windows whose projected frames are rows of fr ([rows,
// 640] f32 on the device), on the context stream; the host waits for it.
int fa::tdt_decode_dev(fa_tdt *d, const float *fr, long rows, const int32_t *lens, int n, int cap, int32_t *ids, int32_t *frame_idx, int32_t *counts) {
  fa_ctx *ctx = d->ctx;
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
  if (off > rows) return set_err(ctx, FA_E_INVALID, "tdtDecode: %ld frames in the windows, %ld in the tensor", off, rows);
  // state layout
  size_t o = 0;
  auto take = [&](size_t bytes) {
    const size_t at = o;
    o += (bytes + 255) & ~(size_t)255;
    return at;
  };
  const size_t o_win = take(sizeof(TdtWin) * n), o_h = take(4ul * n * 4 * TH), o_c = take(4ul * n * 4 * TH), o_pp = take(4ul * n * TH), o_j = take(4ul * n * TH), o_z = take(4ul * n * 8 * 4 * TH),
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
  constexpr int zg = 2;  // emitting windows per LSTM block (measured: 2 < 4 < 8)
  FA_HIP(ctx, hipMemsetAsync(base + o_h, 0, o_pp - o_h, ctx->stream));  // both state slots = 0
  FA_HIP(ctx, hipMemsetAsync(st.alive, 0, 4ul * n, ctx->stream));
  FA_HIP(ctx, hipMemcpyAsync(st.win, win.data(), sizeof(TdtWin) * n, hipMemcpyHostToDevice, ctx->stream));
  auto predict = [&]() -> int {  // candidate state + pred projection for windows with emit set
    for (int layer = 0; layer < 2; layer++) {
      {
        ProfScope ps(ctx, "tdt_lstm_z");
        FA_LAUNCH(ps, tdt_z_kernel<zg>, dim3(4 * TH / 64 * 8, cdiv(n, zg)), dim3(64), 0, ctx->stream, d->lw[layer], d->lr[layer], d->embed, layer,
                  st, n);
      }
      ProfScope ps(ctx, "tdt_lstm_cell");
      FA_LAUNCH(ps, tdt_gates_kernel, dim3(cdiv(TH, 256), n), dim3(256), 0, ctx->stream, d->lb[layer], layer, st);
    }
    ProfScope ps(ctx, "tdt_proj");
    FA_LAUNCH(ps, tdt_proj_kernel<2>, dim3(TH / 64, cdiv(n, 2) + 1), dim3(64), 0, ctx->stream, d->pred_w, d->pred_b, (const float *)st.h, fr, st, n);
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
        FA_LAUNCH(ps, tdt_joint_kernel, dim3(TNB, cdiv(n, RS_SLOTS)), dim3(64 * RS_SLOTS), 0, ctx->stream, d->out_w, TLP, TL, d->out_b,
                  (const float *)st.j, st, n);
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
    for (int i = 0; i < n; i++) {
      if (alive[i] < 0) return set_err(ctx, FA_E_DEVICE, "tdtDecode: window %d: joint logits without a finite maximum", i);
      active += alive[i];
    }
  }
  if (active) return set_err(ctx, FA_E_DEVICE, "tdtDecode: windows still active after %ld steps", max_steps);
  std::vector<TdtWin> fin(n);
  FA_HIP(ctx, hipMemcpy(fin.data(), st.win, sizeof(TdtWin) * n, hipMemcpyDeviceToHost));
  FA_HIP(ctx, hipMemcpy(ids, st.ids, 4ul * n * cap, hipMemcpyDeviceToHost));
  FA_HIP(ctx, hipMemcpy(frame_idx, st.frs, 4ul * n * cap, hipMemcpyDeviceToHost));
  for (int i = 0; i < n; i++) counts[i] = fin[i].n_out;
  return FA_OK;
}


