// Fused Parakeet FastConformer encoder: loadParakeetEncoder + parakeetEncodeBatch
// (src/engines/asr-parakeet/raw-encoder.js:39-161, 177-222, 235-386) as one
// native forward over a batch of variable-length windows.
//
// HBM layout (rows = frames of all windows, packed back to back or padded to
// the batch's longest window; one row table per stage, see WinStage):
//   mel      [R0, melBins]     f32   time-major (the reference transposes on the host)
//   s2       [R2, 32, 2*Csub]  f16   c0+c1 output (c0 fused, never stored), hi/lo pairs
//   s2p      [R2, 32, Csub]    f32   pw c2 output before its ReLU
//   s3, s3p  [R3, 16, 2*Csub]  f16   dw c3 output, pw c4 output, hi/lo pairs
//   x        [R3, D]           f32   residual stream (the returned frames)
//   h        [R3, D]           f16   LayerNorm outputs (GEMM A operands)
//   u        [R3, max(DFF,3D)] f16   FF hidden / fused q|k|v
//   a, g     [R3, D]           f16   attention output, GLU output, dwconv output
// Channels-last front-end tensors make the 1x1 convs plain GEMMs over (t, f)
// rows and make the flatten to [T, Csub*Fsub] free: the linear's weight rows
// are permuted at load from the reference's c*F+f order to f*Csub+c.
//
// Per layer (M = R3 rows):  LN -> FF1 (W1+SiLU, W2·½ + x) -> LN -> QKV (one
// GEMM, N = 3D) -> fused rel-pos attention -> out-proj + x -> LN -> pw1 with
// the GLU in the GEMM epilogue -> depthwise k=9 + bias + SiLU (per window) ->
// pw2 + x -> LN -> FF2 -> LN.  Residual adds ride the GEMM epilogues (as the
// reference's `add` option, raw-encoder.js:282-284).
#include <cmath>
#include <functional>
#include <cstring>
#include <string>
#include <unordered_map>
#include <vector>

#include "fa_internal.h"
#include "fa_device.h"
#include "gemm.h"
#include "attention.h"
#include "ops.h"
#include "encoder_impl.h"

#include <array>

namespace fa {

// One stage's window table: rows [off[w], off[w]+len[w]) belong to window w
// (WinStage, encoder_impl.h).

// ── subsampling kernels (channels-last) ──────────────────────────────────
// One wavefront per output row (window, t) sweeping the frequency axis; lane l
// owns channels [CPL*l, CPL*l + CPL), so each lane's weights stay in registers
// for the whole sweep, inputs every lane shares (mel taps) are wave-uniform,
// and a row position's channels are one contiguous store.
//
// The activations that feed the pointwise-conv GEMMs are stored as exact f16
// pairs (hi = f16(v), lo = f16(v - hi), interleaved per channel) and those
// GEMMs read K = 2*Csub against duplicated weight rows: the front end then
// carries f32-accurate activations through f16 matrix cores.

template <int CPL>
__device__ __forceinline__ void store_hilo(_Float16 *dst, const float (&v)[CPL]) {
  _Float16 o[2 * CPL];
#pragma unroll
  for (int e = 0; e < CPL; e++) {
    const _Float16 hi = (_Float16)v[e];
    o[2 * e] = hi;
    o[2 * e + 1] = (_Float16)(v[e] - (float)hi);
  }
  if constexpr (CPL == 1) {
    *reinterpret_cast<h2 *>(dst) = h2{o[0], o[1]};
  } else if constexpr (CPL == 2) {
    *reinterpret_cast<h4 *>(dst) = h4{o[0], o[1], o[2], o[3]};
  } else {
#pragma unroll
    for (int e = 0; e < 2 * CPL; e += 8) *reinterpret_cast<h8 *>(dst + e) = h8{o[e], o[e + 1], o[e + 2], o[e + 3], o[e + 4], o[e + 5], o[e + 6], o[e + 7]};
  }
}

// c0 (conv2d 1 -> C, 3x3, stride 2, + bias, ReLU; raw-encoder.js:188) fused
// into c1 (depthwise 3x3, stride 2, + bias; raw-encoder.js:189): the c0 map
// never reaches memory.  Both convs pad pt rows on top and pl bins on the
// left (Parakeet: 1 and 1; the streaming models' subPad, raw-encoder.js:187-219);
// the bottom / right pads are implied by the stage lengths the host computes.
// c0 outputs outside [0,T1) x [0,F1) are c1's zero padding.  w0 [C][9], b0
// [C]; w1 [9][C] (tap-major), b1 [C].  Output: [rows of stage 2][F2][C] as
// hi/lo pairs (2C halfs per position).  src null: mel rows time-major
// [rows][MB], window at row s0.off; src set: the channel-major feature stream
// [MB][src->ttot], window at column src->start, read in place (no packed copy).
// LM = true (melBins + both frequency pads <= kC01MelStride): the block's 19
// mel rows (its 4 waves' 7-row spans overlap by 3) are staged in LDS once,
// zero-padded in time and frequency, and the c0 taps are LDS broadcasts
// instead of per-tap global loads.
constexpr int kC01MelStride = 132;  // LDS row: melBins + both frequency pads
template <int CPL, bool LM = false>
__global__ __launch_bounds__(256) void sub_c01_kernel(const float *__restrict__ mel, int MB, WinStage s0, WinStage s1, int F1, WinStage s2, int F2,
                                                      const float *__restrict__ w0, const float *__restrict__ b0, const float *__restrict__ w1,
                                                      const float *__restrict__ b1, _Float16 *__restrict__ y, int pt, int pl, const MelSrc *__restrict__ src) {
  constexpr int C = 64 * CPL;
  constexpr int kRows = 19;  // mel rows the block's 4 output rows read (4 * 3 + 7)
  __shared__ float smel[LM ? kRows : 1][LM ? kC01MelStride : 1];
  const int lane = threadIdx.x & 63, win = blockIdx.y, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int t2 = blockIdx.x * 4 + wave;
  if (blockIdx.x * 4 >= s2.len[win]) return;  // whole block idle
  // mel rows 4*t2 - 3*pt .. +6 feed this output row (c1 row t2 reads c0 rows
  // 2*t2 - pt .. +2, each reading mel rows 2*t1 - pt .. +2)
  const int rblk = 16 * blockIdx.x - 3 * pt;
  // the window's first mel frame: time-major row (element ti * MB + fi) or
  // channel-major stream column (element fi * ttot + ti)
  // (mel is null when the descriptor is given: no offset is applied to it then)
  const long ttot = src ? src->ttot : 0;
  const float *m = src ? src->ptr + src->start[win] : mel + (size_t)s0.off[win] * MB;
  const int T0 = s0.len[win], T1 = s1.len[win];
  if constexpr (LM) {  // slot [r][j] holds frame rblk + r, bin j - pl; zero outside the window
    for (int idx = threadIdx.x; idx < kRows * kC01MelStride; idx += 256) {
      int r, j;
      if (ttot) {  // consecutive lanes walk time within a bin (contiguous in the stream)
        j = idx / kRows;
        r = idx - j * kRows;
      } else {
        r = idx / kC01MelStride;
        j = idx - r * kC01MelStride;
      }
      const int ti = rblk + r, fi = j - pl;
      smel[r][j] = (ti >= 0 && ti < T0 && fi >= 0 && fi < MB) ? m[ttot ? (size_t)fi * ttot + ti : (size_t)ti * MB + fi] : 0.f;
    }
    __syncthreads();
  }
  if (t2 >= s2.len[win]) return;
  float k0[CPL][9], c0b[CPL], k1[9][CPL], c1b[CPL];
#pragma unroll
  for (int e = 0; e < CPL; e++) {
    const int ch = CPL * lane + e;
    c0b[e] = b0[ch];
    c1b[e] = b1[ch];
#pragma unroll
    for (int k = 0; k < 9; k++) {
      k0[e][k] = w0[ch * 9 + k];
      k1[k][e] = w1[k * C + ch];
    }
  }
  // c0 output (t1, f1) for this lane's channels; zero outside the c0 map
  auto c0 = [&](int t1, int f1, float (&o)[CPL]) {
    if (t1 < 0 || t1 >= T1 || f1 < 0 || f1 >= F1) {
#pragma unroll
      for (int e = 0; e < CPL; e++) o[e] = 0.f;
      return;
    }
    float x[9];
#pragma unroll
    for (int a = 0; a < 3; a++) {
      const int ti = 2 * t1 - pt + a;
#pragma unroll
      for (int bb = 0; bb < 3; bb++) {
        const int fi = 2 * f1 - pl + bb;
        if constexpr (LM)
          x[a * 3 + bb] = smel[ti - rblk][fi + pl];
        else
          x[a * 3 + bb] = (ti >= 0 && ti < T0 && fi >= 0 && fi < MB) ? m[ttot ? (size_t)fi * ttot + ti : (size_t)ti * MB + fi] : 0.f;
      }
    }
#pragma unroll
    for (int e = 0; e < CPL; e++) {
      float acc = c0b[e];
#pragma unroll
      for (int k = 0; k < 9; k++) acc += x[k] * k0[e][k];
      o[e] = fmaxf(acc, 0.f);
    }
  };
  // output columns [fb, fe): blockIdx.z of gridDim.z column groups (small
  // grids, a stream pass, spread a row's columns over more waves)
  const int fper = (F2 + gridDim.z - 1) / gridDim.z, fb = blockIdx.z * fper, fe = min(F2, fb + fper);
  float left[3][CPL];  // c0 column 2*f2-pl of rows 2*t2-pt .. 2*t2-pt+2 (the previous step's right column)
#pragma unroll
  for (int a = 0; a < 3; a++) c0(2 * t2 - pt + a, 2 * fb - pl, left[a]);
  _Float16 *yr = y + (size_t)(s2.off[win] + t2) * F2 * 2 * C + 2 * CPL * lane;
  for (int f2 = fb; f2 < fe; f2++) {
    float o[CPL];
#pragma unroll
    for (int e = 0; e < CPL; e++) o[e] = c1b[e];
#pragma unroll
    for (int a = 0; a < 3; a++) {
      float mid[CPL], right[CPL];
      c0(2 * t2 - pt + a, 2 * f2 - pl + 1, mid);
      c0(2 * t2 - pt + a, 2 * f2 - pl + 2, right);
#pragma unroll
      for (int e = 0; e < CPL; e++) {
        o[e] += left[a][e] * k1[a * 3][e];
        o[e] += mid[e] * k1[a * 3 + 1][e];
        o[e] += right[e] * k1[a * 3 + 2][e];
        left[a][e] = right[e];
      }
    }
    store_hilo<CPL>(yr + (size_t)f2 * 2 * C, o);
  }
}

// c3: depthwise conv2d 3x3, stride 2, pads pt / pl, + bias (raw-encoder.js:191) over
// the c2 GEMM's f32 pre-activation output, applying c2's ReLU on load.
// wt [9][C] (tap-major).  Output hi/lo pairs like sub_c01_kernel.
// With vrow set it also writes the encoder's row map for the transposed V
// buffer: vrow[out.off[win] + to] = win * vstride + to for the window's
// frames, -1 for the padding rows of a padded layout (to < vpad).
template <int CPL>
__global__ __launch_bounds__(256) void sub_dw_kernel(const float *__restrict__ x, WinStage in, int Fin, WinStage out, int Fout,
                                                     const float *__restrict__ wt, const float *__restrict__ b, _Float16 *__restrict__ y,
                                                     int *__restrict__ vrow, int vstride, int vpad, int pt, int pl) {
  constexpr int C = 64 * CPL;
  const int lane = threadIdx.x & 63, win = blockIdx.y;
  const int to = blockIdx.x * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  if (vrow && lane == 0 && blockIdx.z == 0 && (to < out.len[win] || to < vpad)) vrow[out.off[win] + to] = to < out.len[win] ? win * vstride + to : -1;
  if (to >= out.len[win]) return;
  float wr[9][CPL], br[CPL];
#pragma unroll
  for (int e = 0; e < CPL; e++) {
    br[e] = b[CPL * lane + e];
#pragma unroll
    for (int k = 0; k < 9; k++) wr[k][e] = wt[k * C + CPL * lane + e];
  }
  const int Ti = in.len[win];
  const float *xb = x + (size_t)in.off[win] * Fin * C + CPL * lane;
  auto ld = [&](int ti, int fi, float (&v)[CPL]) {
    if (ti >= 0 && ti < Ti && fi >= 0 && fi < Fin) {
      const float *src = xb + ((size_t)ti * Fin + fi) * C;
#pragma unroll
      for (int e = 0; e < CPL; e++) v[e] = fmaxf(src[e], 0.f);
    } else {
#pragma unroll
      for (int e = 0; e < CPL; e++) v[e] = 0.f;
    }
  };
  // output columns [fb, fe): blockIdx.z of gridDim.z column groups, as sub_c01_kernel
  const int fper = (Fout + gridDim.z - 1) / gridDim.z, fb = blockIdx.z * fper, fe = min(Fout, fb + fper);
  float left[3][CPL];  // input column 2*fo-pl of rows 2*to-pt .. 2*to-pt+2
#pragma unroll
  for (int a = 0; a < 3; a++) ld(2 * to - pt + a, 2 * fb - pl, left[a]);
  _Float16 *yr = y + (size_t)(out.off[win] + to) * Fout * 2 * C + 2 * CPL * lane;
  for (int fo = fb; fo < fe; fo++) {
    float o[CPL];
#pragma unroll
    for (int e = 0; e < CPL; e++) o[e] = br[e];
#pragma unroll
    for (int a = 0; a < 3; a++) {
      const int ti = 2 * to - pt + a;
      float mid[CPL], right[CPL];
      ld(ti, 2 * fo - pl + 1, mid);
      ld(ti, 2 * fo - pl + 2, right);
#pragma unroll
      for (int e = 0; e < CPL; e++) {
        o[e] += left[a][e] * wr[a * 3][e];
        o[e] += mid[e] * wr[a * 3 + 1][e];
        o[e] += right[e] * wr[a * 3 + 2][e];
        left[a][e] = right[e];
      }
    }
    store_hilo<CPL>(yr + (size_t)fo * 2 * C, o);
  }
}

// Front-end launches: C = 64 * CPL channels, grid (rows / 4, windows).
#define FA_CPL_SWITCH(C, CALL)                                        \
  switch ((C) / 64) {                                                 \
    case 1: CALL(1); break;                                           \
    case 2: CALL(2); break;                                           \
    case 4: CALL(4); break;                                           \
    case 8: CALL(8); break;                                           \
    default: return set_err(ctx, FA_E_UNSUPPORTED, "Csub=%d", (C)); \
  }
static int launch_c01(fa_ctx *ctx, ProfScope &ps, dim3 grid, const float *mel, int MB, WinStage s0, WinStage s1, int F1, WinStage s2, int F2,
                      const float *w0, const float *b0, const float *w1, const float *b1, _Float16 *y, int C, bool lds_mel, int pt, int pl, int pr,
                      const MelSrc *src) {
  if (MB + pl + pr <= kC01MelStride && lds_mel) {
#define FA_C01(K) FA_LAUNCH(ps, (sub_c01_kernel<K, true>), grid, dim3(256), 0, ctx->stream, mel, MB, s0, s1, F1, s2, F2, w0, b0, w1, b1, y, pt, pl, src)
    FA_CPL_SWITCH(C, FA_C01)
#undef FA_C01
    return FA_OK;
  }
#define FA_C01(K) FA_LAUNCH(ps, sub_c01_kernel<K>, grid, dim3(256), 0, ctx->stream, mel, MB, s0, s1, F1, s2, F2, w0, b0, w1, b1, y, pt, pl, src)
  FA_CPL_SWITCH(C, FA_C01)
#undef FA_C01
  return FA_OK;
}
static int launch_dw(fa_ctx *ctx, ProfScope &ps, dim3 grid, const float *x, WinStage in, int Fin, WinStage out, int Fout, const float *wt,
                     const float *b, _Float16 *y, int C, int *vrow, int vstride, int vpad, int pt, int pl) {
#define FA_DW(K) FA_LAUNCH(ps, sub_dw_kernel<K>, grid, dim3(256), 0, ctx->stream, x, in, Fin, out, Fout, wt, b, y, vrow, vstride, vpad, pt, pl)
  FA_CPL_SWITCH(C, FA_DW)
#undef FA_DW
  return FA_OK;
}
#undef FA_CPL_SWITCH

// LayerNorm over D = 256 * V columns (one wavefront per row, 4*V values per
// lane in registers) of the f32 residual stream into the f16 GEMM operand;
// with `lo` also the exact remainder plane lo = f16(y - f16(y)).  Statistics
// as the reference's layernorm (compute.js:519-529): mean, then the mean of
// squared deviations, eps inside the rsqrt.
// SILU = true: SiLU after the affine (the streaming models' conv-module
// LayerNorm of the depthwise output, raw-encoder.js:361-364).
template <int V, bool SILU = false>
__global__ __launch_bounds__(256) void enc_ln_kernel(const float *__restrict__ x, const float *__restrict__ gamma, const float *__restrict__ beta,
                                                     _Float16 *__restrict__ y, _Float16 *__restrict__ ylo, int rows, float eps) {
  constexpr int D = 256 * V;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (row >= rows) return;
  const float4 *xr = reinterpret_cast<const float4 *>(x + (size_t)row * D);
  float4 v[V];
  f4 gv[V], bv[V];
#pragma unroll
  for (int t = 0; t < V; t++) {  // gamma / beta loaded with the row: their latency overlaps the reductions
    v[t] = xr[lane + 64 * t];
    gv[t] = reinterpret_cast<const f4 *>(gamma)[lane + 64 * t];
    bv[t] = reinterpret_cast<const f4 *>(beta)[lane + 64 * t];
  }
#pragma unroll
  for (int t = 0; t < V; t++) asm volatile("" : "+v"(gv[t]), "+v"(bv[t]));  // loads issued here, not sunk below the reductions
  float s = 0.f;
#pragma unroll
  for (int t = 0; t < V; t++) s += v[t].x + v[t].y + v[t].z + v[t].w;
  const float mean = wave_sum(s) * (1.f / D);
  float q = 0.f;
#pragma unroll
  for (int t = 0; t < V; t++) {
    const float a = v[t].x - mean, b = v[t].y - mean, c = v[t].z - mean, d = v[t].w - mean;
    q += a * a + b * b + c * c + d * d;
  }
  const float inv = rsqrtf(wave_sum(q) * (1.f / D) + eps);
#pragma unroll
  for (int t = 0; t < V; t++) {
    const int j = lane + 64 * t;
    const f4 gm = gv[t], bt = bv[t];
    float o[4] = {(v[t].x - mean) * inv * gm.x + bt.x, (v[t].y - mean) * inv * gm.y + bt.y, (v[t].z - mean) * inv * gm.z + bt.z,
                  (v[t].w - mean) * inv * gm.w + bt.w};
    if constexpr (SILU) {
#pragma unroll
      for (int e = 0; e < 4; e++) o[e] = silu_f(o[e]);
    }
    h4 hi, lo;
#pragma unroll
    for (int e = 0; e < 4; e++) {
      hi[e] = (_Float16)o[e];
      lo[e] = (_Float16)(o[e] - (float)hi[e]);
    }
    reinterpret_cast<h4 *>(y + (size_t)row * D)[j] = hi;
    if (ylo) reinterpret_cast<h4 *>(ylo + (size_t)row * D)[j] = lo;
  }
}

// The layer's closing LayerNorm (norm_out) in place on the f32 residual
// stream, D = 256 * V (one wavefront per row, float4 loads and stores).
template <int V>
__global__ __launch_bounds__(256) void enc_ln_f32_kernel(float *__restrict__ x, const float *__restrict__ gamma, const float *__restrict__ beta, int rows,
                                                         float eps) {
  constexpr int D = 256 * V;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (row >= rows) return;
  float4 *xr = reinterpret_cast<float4 *>(x + (size_t)row * D);
  float4 v[V];
  float s = 0.f;
#pragma unroll
  for (int t = 0; t < V; t++) {
    v[t] = xr[lane + 64 * t];
    s += v[t].x + v[t].y + v[t].z + v[t].w;
  }
  const float mean = wave_sum(s) * (1.f / D);
  float q = 0.f;
#pragma unroll
  for (int t = 0; t < V; t++) {
    const float a = v[t].x - mean, b = v[t].y - mean, c = v[t].z - mean, d = v[t].w - mean;
    q += a * a + b * b + c * c + d * d;
  }
  const float inv = rsqrtf(wave_sum(q) * (1.f / D) + eps);
#pragma unroll
  for (int t = 0; t < V; t++) {
    const int j = lane + 64 * t;
    const float4 gm = reinterpret_cast<const float4 *>(gamma)[j], bt = reinterpret_cast<const float4 *>(beta)[j];
    xr[j] = make_float4((v[t].x - mean) * inv * gm.x + bt.x, (v[t].y - mean) * inv * gm.y + bt.y, (v[t].z - mean) * inv * gm.z + bt.z,
                        (v[t].w - mean) * inv * gm.w + bt.w);
  }
}

// A layer's norm_out fused with the next layer's first LayerNorm (norm_ff1):
// the row is read once, normalised in place on the f32 residual stream, and
// normalised again from registers into the f16 operand (and its lo plane when
// the next layer carries it exact).  Same arithmetic as enc_ln_f32_kernel
// followed by enc_ln_kernel.
template <int V>
__global__ __launch_bounds__(256) void enc_ln2_kernel(float *__restrict__ x, const float *__restrict__ g0, const float *__restrict__ b0,
                                                      const float *__restrict__ g1, const float *__restrict__ b1, _Float16 *__restrict__ y,
                                                      _Float16 *__restrict__ ylo, int rows, float eps) {
  constexpr int D = 256 * V;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (row >= rows) return;
  float4 *xr = reinterpret_cast<float4 *>(x + (size_t)row * D);
  float4 v[V];
#pragma unroll
  for (int t = 0; t < V; t++) v[t] = xr[lane + 64 * t];
#pragma unroll
  for (int pass = 0; pass < 2; pass++) {
    float s = 0.f;
#pragma unroll
    for (int t = 0; t < V; t++) s += v[t].x + v[t].y + v[t].z + v[t].w;
    const float mean = wave_sum(s) * (1.f / D);
    float q = 0.f;
#pragma unroll
    for (int t = 0; t < V; t++) {
      const float a = v[t].x - mean, b = v[t].y - mean, c = v[t].z - mean, d = v[t].w - mean;
      q += a * a + b * b + c * c + d * d;
    }
    const float inv = rsqrtf(wave_sum(q) * (1.f / D) + eps);
    const float *gamma = pass ? g1 : g0, *beta = pass ? b1 : b0;
#pragma unroll
    for (int t = 0; t < V; t++) {
      const int j = lane + 64 * t;
      const float4 gm = reinterpret_cast<const float4 *>(gamma)[j], bt = reinterpret_cast<const float4 *>(beta)[j];
      const float4 o = make_float4((v[t].x - mean) * inv * gm.x + bt.x, (v[t].y - mean) * inv * gm.y + bt.y, (v[t].z - mean) * inv * gm.z + bt.z,
                                   (v[t].w - mean) * inv * gm.w + bt.w);
      if (pass == 0) {
        xr[j] = o;
        v[t] = o;
      } else {
        const float oo[4] = {o.x, o.y, o.z, o.w};
        h4 hi, lo;
#pragma unroll
        for (int e = 0; e < 4; e++) {
          hi[e] = (_Float16)oo[e];
          lo[e] = (_Float16)(oo[e] - (float)hi[e]);
        }
        reinterpret_cast<h4 *>(y + (size_t)row * D)[j] = hi;
        if (ylo) reinterpret_cast<h4 *>(ylo + (size_t)row * D)[j] = lo;
      }
    }
  }
}

// Conv module depthwise conv over time, k taps, symmetric pad (k-1)/2,
// + bias (BatchNorm folded) + SiLU (raw-encoder.js:365-367), per window.
// Thread = CPT channels x TT consecutive frames; the TT+k-1 input rows are
// loaded once into registers (each input row is read (TT+k-1)/TT times).
// TI = float: the GLU output arrives in f32; ylo (optional) receives the exact
// f16 remainder of each output for a two-plane GEMM operand.
template <int KT, int TT, int CPT, typename TI>
__global__ __launch_bounds__(64) void dwconv_silu_kernel(const TI *__restrict__ x, _Float16 *__restrict__ y, _Float16 *__restrict__ ylo,
                                                          const float *__restrict__ wt, const float *__restrict__ b, int D, WinStage st) {
  static_assert(CPT == 4 || CPT == 8, "4 or 8 channels per thread");
  typedef _Float16 hv __attribute__((ext_vector_type(CPT)));
  const int win = blockIdx.y;
  const int T = st.len[win];
  const int t0 = blockIdx.x * TT;
  if (t0 >= T) return;
  const int c0 = (blockIdx.z * blockDim.x + threadIdx.x) * CPT;
  if (c0 >= D) return;
  constexpr int PAD = (KT - 1) / 2;
  const TI *xb = x + (size_t)st.off[win] * D + c0;
  _Float16 *yb = y + (size_t)st.off[win] * D + c0;
  float in[TT + KT - 1][CPT];
#pragma unroll
  for (int r = 0; r < TT + KT - 1; r++) {
    const int t = t0 - PAD + r;
    if (t >= 0 && t < T) {
      if constexpr (sizeof(TI) == 2) {
        const hv v = *reinterpret_cast<const hv *>(xb + (size_t)t * D);
#pragma unroll
        for (int e = 0; e < CPT; e++) in[r][e] = (float)v[e];
      } else {
#pragma unroll
        for (int q = 0; q < CPT / 4; q++) {
          const float4 a4 = reinterpret_cast<const float4 *>(xb + (size_t)t * D)[q];
          in[r][4 * q] = a4.x;
          in[r][4 * q + 1] = a4.y;
          in[r][4 * q + 2] = a4.z;
          in[r][4 * q + 3] = a4.w;
        }
      }
    } else {
#pragma unroll
      for (int e = 0; e < CPT; e++) in[r][e] = 0.f;
    }
  }
  float wk[KT][CPT];
#pragma unroll
  for (int k = 0; k < KT; k++)
#pragma unroll
    for (int e = 0; e < CPT; e++) wk[k][e] = wt[k * D + c0 + e];
  float bb[CPT];
#pragma unroll
  for (int e = 0; e < CPT; e++) bb[e] = b[c0 + e];
#pragma unroll
  for (int t = 0; t < TT; t++) {
    if (t0 + t >= T) break;
    hv o, ol;
#pragma unroll
    for (int e = 0; e < CPT; e++) {
      float acc = 0.f;
#pragma unroll
      for (int k = 0; k < KT; k++) acc += in[t + k][e] * wk[k][e];
      const float r = silu_f(acc + bb[e]);
      o[e] = (_Float16)r;
      ol[e] = (_Float16)(r - (float)o[e]);
    }
    *reinterpret_cast<hv *>(yb + (size_t)(t0 + t) * D) = o;
    if (ylo) *reinterpret_cast<hv *>(ylo + (size_t)st.off[win] * D + c0 + (size_t)(t0 + t) * D) = ol;
  }
}

// Depthwise conv over time (k = 9) for the streaming models and stream
// passes: causal (pad k-1 on the left, raw-encoder.js:279-280) or symmetric,
// + bias; taps before a window's first frame read `cache` when one is given
// (a stream pass: the k-1 GLU rows ahead of the pass, window 0 only) and zeros
// otherwise.  Then either SiLU into f16 (+ exact lo plane), or the raw f32
// value into y32 when the layer normalises the depthwise output first.
// Thread = 4 channels of one frame.
template <typename TI>
__global__ __launch_bounds__(64) void dwconv_gen_kernel(const TI *__restrict__ x, const CcSlots slots, int use_slots, size_t cco, WinStage st, int causal,
                                                        const float *__restrict__ wt, const float *__restrict__ b, int D, _Float16 *__restrict__ y,
                                                        _Float16 *__restrict__ ylo, float *__restrict__ y32) {
  constexpr int KT = 9;
  const int win = blockIdx.y, t = blockIdx.x, T = st.len[win];
  if (t >= T) return;
  const float *cache = use_slots ? slots.cc_in[win] + cco : nullptr;  // a stream pass: taps before the window's first frame
  const int c0 = (blockIdx.z * 64 + threadIdx.x) * 4;
  if (c0 >= D) return;
  const int pad = causal ? KT - 1 : (KT - 1) / 2;
  const size_t base = (size_t)st.off[win] * D + c0;
  float acc[4];
#pragma unroll
  for (int e = 0; e < 4; e++) acc[e] = 0.f;
#pragma unroll
  for (int k = 0; k < KT; k++) {
    const int ti = t - pad + k;
    float v[4] = {0.f, 0.f, 0.f, 0.f};
    if (ti >= 0 && ti < T) {
#pragma unroll
      for (int e = 0; e < 4; e++) v[e] = (float)x[base + (size_t)ti * D + e];
    } else if (ti < 0 && cache) {
#pragma unroll
      for (int e = 0; e < 4; e++) v[e] = cache[(size_t)(KT - 1 + ti) * D + c0 + e];
    }
#pragma unroll
    for (int e = 0; e < 4; e++) acc[e] += v[e] * wt[k * D + c0 + e];
  }
  h4 hi, lo;
#pragma unroll
  for (int e = 0; e < 4; e++) {
    const float r = acc[e] + b[c0 + e];
    if (y32) {
      y32[base + (size_t)t * D + e] = r;
    } else {
      const float sv = silu_f(r);
      hi[e] = (_Float16)sv;
      lo[e] = (_Float16)(sv - (float)hi[e]);
    }
  }
  if (!y32) {
    *reinterpret_cast<h4 *>(y + base + (size_t)t * D) = hi;
    if (ylo) *reinterpret_cast<h4 *>(ylo + base + (size_t)t * D) = lo;
  }
}

// Depthwise conv (k = 9, causal or symmetric, taps before the window's first
// frame from `cache` in a stream pass) + bias, then the conv-module LayerNorm
// (streaming models, raw-encoder.js:361-364) + SiLU into f16 (+ exact lo
// plane): block = one frame (256 threads x 4 channels, D <= 1024), the row
// statistics reduced over the block (mean, then mean of squared deviations,
// eps inside the rsqrt, as enc_ln_kernel).  In a stream pass block (0, 0)
// also writes the next pass's conv cache (rows nemit .. nemit + 7 of
// [cache ; GLU rows]).
template <typename TI>
__global__ __launch_bounds__(256) void dwconv_ln_kernel(const TI *__restrict__ x, const CcSlots slots, int use_slots, size_t cco, WinStage st, int causal,
                                                        const float *__restrict__ wt, const float *__restrict__ b, const float *__restrict__ gamma,
                                                        const float *__restrict__ beta, int D, _Float16 *__restrict__ y, _Float16 *__restrict__ ylo, int nemit) {
  constexpr int KT = 9;
  __shared__ float red[2][4];
  const int win = blockIdx.y, t = blockIdx.x, T = st.len[win];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int c0 = tid * 4;
  const bool act = c0 < D;
  // a stream pass: this window's stream caches (taps before its first frame, and the next pass's)
  const float *cache = use_slots ? slots.cc_in[win] + cco : nullptr;
  float *cc_out = use_slots ? slots.cc_out[win] + cco : nullptr;
  if (cc_out && t == 0 && act) {
    // every load issued before the first store (the stores could alias them for all the compiler knows)
    const TI *xw = x + (size_t)st.off[win] * D + c0;
    float4 rows[KT - 1];
#pragma unroll
    for (int r = 0; r < KT - 1; r++) {
      const int src = nemit + r;
      if (src < KT - 1) {
        rows[r] = *reinterpret_cast<const float4 *>(cache + (size_t)src * D + c0);
      } else {
        const TI *xr = xw + (size_t)(src - (KT - 1)) * D;
        rows[r] = make_float4((float)xr[0], (float)xr[1], (float)xr[2], (float)xr[3]);
      }
    }
#pragma unroll
    for (int r = 0; r < KT - 1; r++) *reinterpret_cast<float4 *>(cc_out + (size_t)r * D + c0) = rows[r];
  }
  if (t >= T) return;  // uniform per block
  const int pad = causal ? KT - 1 : (KT - 1) / 2;
  const size_t base = (size_t)st.off[win] * D + c0;
  float r[4] = {0.f, 0.f, 0.f, 0.f};
  if (act) {
    // every tap's inputs and weights are loaded before the first product
    // (one memory round trip, not one per tap)
    float v[KT][4], wk[KT][4];
#pragma unroll
    for (int k = 0; k < KT; k++) {
      const float4 w4 = *reinterpret_cast<const float4 *>(wt + k * D + c0);
      wk[k][0] = w4.x; wk[k][1] = w4.y; wk[k][2] = w4.z; wk[k][3] = w4.w;
      const int ti = t - pad + k;
      if (ti >= 0 && ti < T) {
        if constexpr (sizeof(TI) == 4) {
          const float4 a = *reinterpret_cast<const float4 *>(x + base + (size_t)ti * D);
          v[k][0] = a.x; v[k][1] = a.y; v[k][2] = a.z; v[k][3] = a.w;
        } else {
          const h4 a = *reinterpret_cast<const h4 *>(x + base + (size_t)ti * D);
#pragma unroll
          for (int e = 0; e < 4; e++) v[k][e] = (float)a[e];
        }
      } else if (ti < 0 && cache) {
        const float4 a = *reinterpret_cast<const float4 *>(cache + (size_t)(KT - 1 + ti) * D + c0);
        v[k][0] = a.x; v[k][1] = a.y; v[k][2] = a.z; v[k][3] = a.w;
      } else {
#pragma unroll
        for (int e = 0; e < 4; e++) v[k][e] = 0.f;
      }
    }
    float acc[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int k = 0; k < KT; k++)
#pragma unroll
      for (int e = 0; e < 4; e++) acc[e] += v[k][e] * wk[k][e];
#pragma unroll
    for (int e = 0; e < 4; e++) r[e] = acc[e] + b[c0 + e];
  }
  auto block_sum = [&](float v, int slot) {
    v = wave_sum(v);
    if (lane == 0) red[slot][wave] = v;
    __syncthreads();
    return (red[slot][0] + red[slot][1]) + (red[slot][2] + red[slot][3]);
  };
  const float mean = block_sum(act ? r[0] + r[1] + r[2] + r[3] : 0.f, 0) * (1.f / D);
  float q = 0.f;
  if (act)
#pragma unroll
    for (int e = 0; e < 4; e++) q += (r[e] - mean) * (r[e] - mean);
  const float inv = rsqrtf(block_sum(q, 1) * (1.f / D) + 1e-5f);
  if (!act) return;
  h4 hi, lo;
#pragma unroll
  for (int e = 0; e < 4; e++) {
    const float o = silu_f((r[e] - mean) * inv * gamma[c0 + e] + beta[c0 + e]);
    hi[e] = (_Float16)o;
    lo[e] = (_Float16)(o - (float)hi[e]);
  }
  *reinterpret_cast<h4 *>(y + base + (size_t)t * D) = hi;
  if (ylo) *reinterpret_cast<h4 *>(ylo + base + (size_t)t * D) = lo;
}

// Stream-pass depthwise-conv cache: row r < k-1 of the next cache is row
// nemit + r of [cache (k-1 rows) ; this pass's GLU rows] -- the k-1 GLU
// outputs ahead of the next pass's first frame.
template <typename TI>
__global__ __launch_bounds__(256) void stream_conv_cache_kernel(const CcSlots slots, size_t cco, const TI *__restrict__ g, int D, int nemit,
                                                                int nq) {
  constexpr int KT = 9;
  const int r = blockIdx.x, w = blockIdx.y, src = nemit + r;  // row r of window (stream) w's next cache
  const float *cc_in = slots.cc_in[w] + cco;
  float *cc_out = slots.cc_out[w] + cco;
  g += (size_t)w * nq * D;
  for (int c = threadIdx.x; c < D; c += 256)
    cc_out[(size_t)r * D + c] = src < KT - 1 ? cc_in[(size_t)src * D + c] : (float)g[(size_t)(src - (KT - 1)) * D + c];
}

// Attention of a stream pass (relShiftStream + softmax + bmmPV,
// compute.js:689-703, streaming-encoder.js:241-254): query i of the pass
// attends key j of [this layer's Lc cached keys ; the pass's nq keys], key j
// at position j - Lc relative to the pass's first frame (the pass starts on a
// chunk boundary); key j is visible iff j - Lc lies in [cs - left,
// cs + chunk - 1 + right], cs = chunk * floor(i / chunk), and its positional
// term uses table row clamp(dMax - (i - (j - Lc)), 0, Pn - 1).  One wave per
// (query, head): lanes over keys for the f32 scores, wave reductions for the
// softmax, lanes over head dims for P·V.  The head's K and V rows are staged
// in LDS once per block (4 queries) with every row load in flight at once
// (reading V from global one key after another cost ~76 us per layer); the
// first query block of each head also writes the head's part of the next
// pass's K / V caches from them.  Lk <= 256.
__global__ __launch_bounds__(256) void stream_attn_kernel(const _Float16 *__restrict__ u, int ldu, const KvSlots slots, size_t kvo,
                                                          int Lc, int nq, int D, const _Float16 *__restrict__ P, int Pn, int dMax,
                                                          const float *__restrict__ pbu, const float *__restrict__ pbv, int chunk, int left, int right,
                                                          _Float16 *__restrict__ out, _Float16 *__restrict__ out_lo, int nemit, int keep) {
  constexpr int HD = 128, MAXK = 256, KS = HD + 8;  // K rows padded: lanes read different keys' rows
  __shared__ float qs[4][2][HD];
  __shared__ float ps[4][MAXK];
  __shared__ __attribute__((aligned(16))) _Float16 vs[MAXK][HD];  // the head's V rows, shared by the block's 4 queries
  __shared__ __attribute__((aligned(16))) _Float16 ks[MAXK][KS];  // and its K rows
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, h = blockIdx.y, w = blockIdx.z;
  // window w = stream w of the batched pass: its nq rows of u / out, its caches
  u += (size_t)w * nq * ldu;
  out += (size_t)w * nq * D;
  if (out_lo) out_lo += (size_t)w * nq * D;
  const _Float16 *kc = slots.kc_in[w] + kvo, *vc = slots.vc_in[w] + kvo;
  _Float16 *kc_out = keep > 0 ? slots.kc_out[w] + kvo : nullptr, *vc_out = slots.vc_out[w] + kvo;
  const int Lk = Lc + nq;
  // A block has four waves.  With more than two queries (nq > 2) each wave
  // takes one query; otherwise each query's keys are split over two waves
  // (kh = 2: [jb, je) is this wave's half), whose maxima, sums and P.V
  // partial rows meet in LDS.  The grid is cdiv(nq, 4) blocks either way.
  const int kh = nq <= 2 ? 2 : 1;
  const int i = blockIdx.x * (4 / kh) + wave / kh, half = wave % kh;
  const int Lh = (Lk + kh - 1) / kh, jb = half * Lh, je = min(Lk, jb + Lh);
  const bool act = i < nq;
  // this wave's query row and the positional biases, loaded ahead of the staging
  float qv[2] = {0.f, 0.f}, bu[2] = {0.f, 0.f}, bv[2] = {0.f, 0.f};
  if (i < nq) {
#pragma unroll
    for (int e = 0; e < 2; e++) {
      const int d = lane + 64 * e;
      qv[e] = (float)u[(size_t)i * ldu + h * HD + d];
      bu[e] = pbu[h * HD + d];
      bv[e] = pbv[h * HD + d];
    }
  }
  // the positional rows of this lane's first two keys, also loaded ahead
  // (later keys, more than 128 in the wave's range, load theirs in the score loop)
  const int cs = chunk * (i / chunk);
  h8 pf[2][HD / 8];
#pragma unroll
  for (int t = 0; t < 2; t++) {
    const int j = jb + lane + 64 * t, rel = j - Lc;
    if (act && j < je && rel >= cs - left && rel <= cs + chunk - 1 + right) {
      const _Float16 *pp = P + (size_t)min(max(dMax - (i - rel), 0), Pn - 1) * D + h * HD;
#pragma unroll
      for (int d = 0; d < HD / 8; d++) pf[t][d] = *reinterpret_cast<const h8 *>(pp + 8 * d);
    }
  }
  // K / V rows to LDS: kStage 16-byte loads of each per thread are issued
  // before any of them is stored (one memory round trip per kStage * 256
  // pieces, not one per 256)
  constexpr int kStage = 8;
  const int npc = Lk * (HD / 8);
  for (int base = threadIdx.x; base < npc; base += 256 * kStage) {
    h8 kr[kStage], vr[kStage];
#pragma unroll
    for (int t = 0; t < kStage; t++) {
      const int idx = base + 256 * t;
      if (idx < npc) {
        const int j = idx >> 4, c8 = (idx & 15) * 8;
        const _Float16 *vsrc = j < Lc ? vc + (size_t)j * D + h * HD + c8 : u + (size_t)(j - Lc) * ldu + 2 * D + h * HD + c8;
        const _Float16 *ksrc = j < Lc ? kc + (size_t)j * D + h * HD + c8 : u + (size_t)(j - Lc) * ldu + D + h * HD + c8;
        vr[t] = *reinterpret_cast<const h8 *>(vsrc);
        kr[t] = *reinterpret_cast<const h8 *>(ksrc);
      }
    }
#pragma unroll
    for (int t = 0; t < kStage; t++) {
      const int idx = base + 256 * t;
      if (idx < npc) {
        const int j = idx >> 4, c8 = (idx & 15) * 8;
        *reinterpret_cast<h8 *>(&vs[j][c8]) = vr[t];
        *reinterpret_cast<h8 *>(&ks[j][c8]) = kr[t];
      }
    }
  }
  __syncthreads();
  if (blockIdx.x == 0 && kc_out) {
    // the next pass's caches for this head: rows Lc + nemit - keep .. of [cached ; new]
    // (the keys of the last `keep` emitted frames, streaming-encoder.js:254-257)
    for (int idx = threadIdx.x; idx < keep * (HD / 8); idx += 256) {
      const int r = idx >> 4, c8 = (idx & 15) * 8, src = Lc + nemit - keep + r;
      *reinterpret_cast<h8 *>(kc_out + (size_t)r * D + h * HD + c8) = *reinterpret_cast<const h8 *>(&ks[src][c8]);
      *reinterpret_cast<h8 *>(vc_out + (size_t)r * D + h * HD + c8) = *reinterpret_cast<const h8 *>(&vs[src][c8]);
    }
  }
  __shared__ float xmx[4], xsum[4];
  __shared__ float opart[4][HD];
  float mx = -INFINITY, sum = 0.f, o[2] = {0.f, 0.f};
  if (act) {
#pragma unroll
    for (int e = 0; e < 2; e++) {
      const int d = lane + 64 * e;
      qs[wave][0][d] = qv[e] + bu[e];
      qs[wave][1][d] = qv[e] + bv[e];
    }
    __builtin_amdgcn_s_waitcnt(0xc07f);
    __builtin_amdgcn_wave_barrier();
    auto score = [&](int j, const h8 *pv8) {  // pv8: the key's positional row, 8 halves per piece
      float acc = 0.f;
#pragma unroll
      for (int d = 0; d < HD; d += 8) {
        const h8 kv = *reinterpret_cast<const h8 *>(&ks[j][d]), pv = pv8[d / 8];
#pragma unroll
        for (int e = 0; e < 8; e++) acc += qs[wave][0][d + e] * (float)kv[e] + qs[wave][1][d + e] * (float)pv[e];
      }
      return acc;
    };
#pragma unroll
    for (int t = 0; t < 2; t++) {
      const int j = jb + lane + 64 * t, rel = j - Lc;
      if (j < je) {
        const float sc = rel >= cs - left && rel <= cs + chunk - 1 + right ? score(j, pf[t]) : -INFINITY;
        ps[wave][j] = sc;
        mx = fmaxf(mx, sc);
      }
    }
    for (int j = jb + lane + 128; j < je; j += 64) {
      const int rel = j - Lc;
      float sc = -INFINITY;
      if (rel >= cs - left && rel <= cs + chunk - 1 + right) {
        const _Float16 *pp = P + (size_t)min(max(dMax - (i - rel), 0), Pn - 1) * D + h * HD;
        h8 pv8[HD / 8];
#pragma unroll
        for (int d = 0; d < HD / 8; d++) pv8[d] = *reinterpret_cast<const h8 *>(pp + 8 * d);
        sc = score(j, pv8);
      }
      ps[wave][j] = sc;
      mx = fmaxf(mx, sc);
    }
    mx = wave_max(mx);  // one half may see only masked keys (-inf); the query's max is finite
  }
  if (kh == 2) {  // the query's max over both halves
    if (act && lane == 0) xmx[wave] = mx;
    __syncthreads();
    if (act) mx = fmaxf(mx, xmx[wave ^ 1]);
  }
  if (act) {
    for (int j = jb + lane; j < je; j += 64) {
      const float p = __expf(ps[wave][j] - mx);  // masked keys: exp(-inf) = 0
      ps[wave][j] = p;
      sum += p;
    }
    sum = wave_sum(sum);
    __builtin_amdgcn_s_waitcnt(0xc07f);
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int e = 0; e < 2; e++) {
      const int d = lane + 64 * e;
      float acc = 0.f;
#pragma unroll 8
      for (int j = jb; j < je; j++) acc += ps[wave][j] * (float)vs[j][d];  // masked keys carry p = 0
      o[e] = acc;
    }
  }
  if (kh == 2) {  // the second half's sum and P.V row join the first half's
    if (act && half) {
      if (lane == 0) xsum[wave] = sum;
#pragma unroll
      for (int e = 0; e < 2; e++) opart[wave][lane + 64 * e] = o[e];
    }
    __syncthreads();
    if (!act || half) return;
    sum += xsum[wave + 1];
#pragma unroll
    for (int e = 0; e < 2; e++) o[e] += opart[wave + 1][lane + 64 * e];
  } else if (!act) {
    return;
  }
  const float inv = 1.f / sum;
#pragma unroll
  for (int e = 0; e < 2; e++) {
    const int d = lane + 64 * e;
    const float v = o[e] * inv;
    const _Float16 hi = (_Float16)v;
    out[(size_t)i * D + h * HD + d] = hi;
    if (out_lo) out_lo[(size_t)i * D + h * HD + d] = (_Float16)(v - (float)hi);
  }
}

// Zero rows of a padded batch past each window's length (output contract).
// Plain 16-byte vector copy (graph-mode input / output staging).
__global__ __launch_bounds__(256) void copy_f4_kernel(const float4 *__restrict__ src, float4 *__restrict__ dst, long n4) {
  for (long i = (long)blockIdx.x * 256 + threadIdx.x; i < n4; i += (long)gridDim.x * 256) dst[i] = src[i];
}
static int copy_f4(fa_ctx *ctx, const void *src, void *dst, size_t bytes, const char *label) {
  const long n4 = (long)(bytes / 16);
  if (!n4) return FA_OK;
  ProfScope ps(ctx, label);
  FA_LAUNCH(ps, copy_f4_kernel, dim3((unsigned)std::min<long>(cdiv(n4, 256), 4096)), dim3(256), 0, ctx->stream, (const float4 *)src, (float4 *)dst, n4);
  return check_launch(ctx, label);
}

__global__ void zero_pad_rows_kernel(float *x, int D, WinStage st, int Tpad) {
  const int win = blockIdx.y;
  const int r = blockIdx.x;
  if (r < st.len[win] || r >= Tpad) return;
  float *row = x + (size_t)(st.off[win] + r) * D;
  for (int j = threadIdx.x; j < D; j += blockDim.x) row[j] = 0.f;
}

// f32 -> f16 conversion (load-time positional table)
__global__ void f32_to_f16_kernel(const float *x, _Float16 *y, long n) {
  for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (long)gridDim.x * blockDim.x) y[i] = (_Float16)x[i];
}

// ── host-side weight preparation ─────────────────────────────────────────
static uint16_t h_f32_to_f16(float f) { return __half_as_ushort(__float2half_rn(f)); }
static float h_f16_to_f32(uint16_t h) { return __half2float(__ushort_as_half(h)); }

}  // namespace fa

namespace fa {

template <typename T>
static T *dupload(fa_encoder *e, const T *host, size_t n) {
  T *d = (T *)dev_alloc(e->ctx, n * sizeof(T) + 16);
  if (!d) return nullptr;
  e->allocs.push_back(d);
  if (hipMemcpy(d, host, n * sizeof(T), hipMemcpyHostToDevice) != hipSuccess) return nullptr;
  return d;
}

// Per-output-column symmetric int8 of Bt [N][K] (row n = output column n):
// s = f32(max|w|)/127 (0 -> 1), q = clip(rint(w/s), -127, 127)
// (quantize-parakeet-encoder.py:31-36, computed in f32 as numpy does).
static void quantize_int8_km(const float *bt, int N, int K, int8_t *q, float *scale) {
  for (int n = 0; n < N; n++) {
    float mx = 0.f;
    for (int k = 0; k < K; k++) mx = std::fmax(mx, std::fabs(bt[(size_t)n * K + k]));
    float s = mx / 127.0f;
    if (s == 0.f) s = 1.f;
    for (int k = 0; k < K; k++) {
      float r = std::rint(bt[(size_t)n * K + k] / s);
      r = r < -127.f ? -127.f : (r > 127.f ? 127.f : r);
      q[(size_t)n * K + k] = (int8_t)r;
    }
    scale[n] = s;
  }
}

// Symmetric int4 group-32 of Bt [N][K] into [N][ceil(K/32)][16 B] (low nibble
// = even k, nibble = q + 8) with f16 scales f16(max|w|/7) (0 -> 1.0).
static void quantize_int4_km(const float *bt, int N, int K, uint8_t *q, uint16_t *sc) {
  const int nblk = (K + 31) / 32;
  for (int n = 0; n < N; n++)
    for (int b = 0; b < nblk; b++) {
      float mx = 0.f;
      for (int t = 0; t < 32 && b * 32 + t < K; t++) mx = std::fmax(mx, std::fabs(bt[(size_t)n * K + b * 32 + t]));
      uint16_t sh = h_f32_to_f16(mx / 7.0f);
      float s = h_f16_to_f32(sh);
      if (s == 0.f) {
        sh = 0x3c00;
        s = 1.f;
      }
      sc[(size_t)n * nblk + b] = sh;
      uint8_t *blk = &q[((size_t)n * nblk + b) * 16];
      std::memset(blk, 0x88, 16);
      for (int t = 0; t < 32 && b * 32 + t < K; t++) {
        float r = std::rint(bt[(size_t)n * K + b * 32 + t] / s);
        r = r < -8.f ? -8.f : (r > 7.f ? 7.f : r);
        const uint8_t nib = (uint8_t)((int)r + 8);
        blk[t / 2] = (t & 1) ? (uint8_t)((blk[t / 2] & 0x0f) | (nib << 4)) : (uint8_t)((blk[t / 2] & 0xf0) | nib);
      }
    }
}

// Build a linear from Bt [N][K] raw f32 values (column n of the reference's
// [K, N] matrix is row n here), a per-column fold factor, optional bias.
static int build_lin(fa_encoder *e, Lin &L, const std::vector<float> &bt, int N, int K, const std::vector<float> &fold, const std::vector<float> *bias,
                     const char *name) {
  fa_ctx *ctx = e->ctx;
  L.N = N;
  L.K = K;
  bool unit = true;
  for (float f : fold) unit &= (f == 1.f);
  if (bias) {
    std::vector<float> bb(N);
    for (int n = 0; n < N; n++) bb[n] = (float)((double)(*bias)[n] * fold[n]);
    if (!(L.bias = dupload(e, bb.data(), N))) return set_err(ctx, FA_E_OOM, "encoder load: %s bias", name);
  }
  if (e->format == FA_W_F16) {
    std::vector<uint16_t> h((size_t)N * K);
    for (int n = 0; n < N; n++)
      for (int k = 0; k < K; k++) h[(size_t)n * K + k] = h_f32_to_f16((float)((double)bt[(size_t)n * K + k] * fold[n]));
    if (!(L.w = dupload(e, h.data(), h.size()))) return set_err(ctx, FA_E_OOM, "encoder load: %s", name);
    L.bkind = B_F16;
    return FA_OK;
  }
  if (e->format == FA_W_INT8) {
    std::vector<int8_t> q((size_t)N * K);
    std::vector<float> cs(N);
    quantize_int8_km(bt.data(), N, K, q.data(), cs.data());
    for (int n = 0; n < N; n++) cs[n] = (float)((double)cs[n] * fold[n]);
    if (!(L.w = dupload(e, q.data(), q.size())) || !(L.colscale = dupload(e, cs.data(), N))) return set_err(ctx, FA_E_OOM, "encoder load: %s", name);
    L.bkind = B_I8;
    return FA_OK;
  }
  if (K % 32) return set_err(ctx, FA_E_UNSUPPORTED, "encoder load: %s K=%d not a multiple of 32 for int4", name, K);
  const int nblk = K / 32;
  std::vector<uint8_t> q((size_t)N * nblk * 16);
  std::vector<uint16_t> sc((size_t)N * nblk);
  quantize_int4_km(bt.data(), N, K, q.data(), sc.data());
  if (!(L.w = dupload(e, q.data(), q.size())) || !(L.scales = dupload(e, sc.data(), sc.size()))) return set_err(ctx, FA_E_OOM, "encoder load: %s", name);
  if (!unit && !(L.colscale = dupload(e, fold.data(), N))) return set_err(ctx, FA_E_OOM, "encoder load: %s", name);
  L.bkind = B_I4;
  return FA_OK;
}

// Quantise-dequantise raw Bt values the way the chosen format stores them
// (used for the pos weights, which only enter through the load-time table).
static void roundtrip_format(int format, std::vector<float> &bt, int N, int K) {
  if (format == FA_W_INT8) {
    std::vector<int8_t> q((size_t)N * K);
    std::vector<float> s(N);
    quantize_int8_km(bt.data(), N, K, q.data(), s.data());
    for (int n = 0; n < N; n++)
      for (int k = 0; k < K; k++) bt[(size_t)n * K + k] = (float)q[(size_t)n * K + k] * s[n];
  } else if (format == FA_W_INT4) {
    const int nblk = (K + 31) / 32;
    std::vector<uint8_t> q((size_t)N * nblk * 16);
    std::vector<uint16_t> sc((size_t)N * nblk);
    quantize_int4_km(bt.data(), N, K, q.data(), sc.data());
    for (int n = 0; n < N; n++)
      for (int k = 0; k < K; k++) {
        const uint8_t byte = q[((size_t)n * nblk + k / 32) * 16 + (k % 32) / 2];
        const int nib = (k & 1) ? (byte >> 4) : (byte & 0xf);
        bt[(size_t)n * K + k] = (float)(nib - 8) * h_f16_to_f32(sc[(size_t)n * nblk + k / 32]);
      }
  }
}

static void set_gemm_b(GemmArgs &p, const Lin &L) {
  p.B = L.w;
  p.bkind = L.bkind;
  p.bscale = L.scales;
  p.bscale_f32 = 0;
  p.colscale = L.colscale;
  p.bias = L.bias;
  p.N = L.N;
  p.K = L.K;
}

static int grow(fa_encoder *e, void **buf, size_t *cap, size_t need) {
  if (need <= *cap) return FA_OK;
  e->ws_gen++;
  if (*buf) {
    (void)hipDeviceSynchronize();  // the buffer may be in use on the context stream or a lane stream
    (void)hipFree(*buf);
    *buf = nullptr;
    *cap = 0;
  }
  *buf = dev_alloc(e->ctx, need);
  if (!*buf) return FA_E_OOM;
  *cap = need;
  return FA_OK;
}

// Default operand precision: the three cheap operands (attention output, GLU
// output, depthwise output) exact in every layer, and every operand but the
// FF hidden state exact in the last kExactTail layers.  Measured on MI355X
// over 24k frames of configs[2] (8 batches of 16 windows) against the fp32
// path: projected-argmax disagreement 0.145 % with plain f16 operands,
// 0.050 % with the FF hidden state exact too, 0.013 % with everything exact
// (40 % more time); rounding errors of early layers decay through the later
// ones, so the tail carries the most weight, and the FF hidden operand (the
// widest, K = 4 DFF) buys the least for its cost.  The counts are near-ties
// that move with any change of rounding: with the current kernels an 8-layer
// tail gave 0.096 % (6.78 ms per step), 10 layers 0.075 % (6.86 ms), 12
// layers 0.112 %; 10 keeps the widest measured margin under the 0.1 % bar.
// The quantised formats keep an 8-layer tail: with 10, int8 configs[4] went
// from 2 to 4 flips in 3008 frames (the bar allows 3).
static const unsigned kCheapExact = FA_EXACT_ATTN_OUT | FA_EXACT_GLU | FA_EXACT_DW_OUT;
static const unsigned kTailExact = 31u & ~(unsigned)FA_EXACT_FF_HIDDEN;
// The quantised formats keep every operand exact in the tail: their weight
// rounding already spends part of the argmax margin (configs[4] measured
// 4 / 3008 disagreements without the FF-hidden plane, 0-3 with it).
static const unsigned kTailExactQuant = 31u;
static const int kExactTail = 10, kExactTailQuant = 8;

static inline int stride2_len(int T) { return T <= 0 ? 0 : (T - 1) / 2 + 1; }
// Output length of a k=3 stride-2 conv with pads p0 / p1: floor((T + p0 + p1 - 3) / 2) + 1.
static inline int stride2_out(int T, int p0, int p1) {
  if (T <= 0) return 0;
  const int q = T + p0 + p1 - 3;
  const int o = (q >= 0 ? q / 2 : -((1 - q) / 2)) + 1;
  return o > 0 ? o : 0;
}
static inline int enc_tsub(const fa_encoder_opts &o, int T) {
  for (int i = 0; i < 3; i++) T = stride2_out(T, o.sub_pad_t, o.sub_pad_b);
  return T;
}

// Replay the captured graph for `key`, capturing `launch` first when the key
// is new (least recently used graphs are evicted past 16); `pre` runs on the
// stream just before the replay (input staging).
int encoder_graph_run(fa_ctx *ctx, fa_encoder *e, const std::vector<int64_t> &key, const std::function<int()> &launch,
                      const std::function<int()> &pre) {
  EncWs::Captured *hit = nullptr;
  for (auto &gr : e->W().graphs)
    if (gr.key == key) hit = &gr;
  if (!hit) {
    FA_HIP(ctx, hipStreamBeginCapture(ctx->stream, hipStreamCaptureModeThreadLocal));
    const int st = launch();
    hipGraph_t graph = nullptr;
    const hipError_t ce = hipStreamEndCapture(ctx->stream, &graph);
    if (st != FA_OK) {
      if (graph) (void)hipGraphDestroy(graph);
      return st;
    }
    if (ce != hipSuccess) return set_err(ctx, FA_E_DEVICE, "encoder: graph capture: %s", hipGetErrorString(ce));
    hipGraphExec_t exec = nullptr;
    const hipError_t ie = hipGraphInstantiateWithFlags(&exec, graph, 0);
    (void)hipGraphDestroy(graph);
    if (ie != hipSuccess) return set_err(ctx, FA_E_DEVICE, "encoder: graph instantiate: %s", hipGetErrorString(ie));
    constexpr size_t kMaxGraphs = 16;
    if (e->W().graphs.size() >= kMaxGraphs) {  // evict the least recently used
      size_t lru = 0;
      for (size_t i = 1; i < e->W().graphs.size(); i++)
        if (e->W().graphs[i].used < e->W().graphs[lru].used) lru = i;
      (void)hipDeviceSynchronize();  // the evicted graph may still be running (context or lane stream)
      (void)hipGraphExecDestroy(e->W().graphs[lru].exec);
      e->W().graphs.erase(e->W().graphs.begin() + lru);
    }
    e->W().graphs.push_back({key, exec, 0});
    hit = &e->W().graphs.back();
  }
  hit->used = ++e->W().graph_clock;
  if (pre) FA_TRY(pre());
  FA_HIP(ctx, hipGraphLaunch(hit->exec, ctx->stream));
  return FA_OK;
}

int encoder_grow(fa_encoder *e, void **buf, size_t *cap, size_t need) { return grow(e, buf, cap, need); }
void encoder_ws_free(EncWs &w) {
  for (auto &g : w.graphs)
    if (g.exec) (void)hipGraphExecDestroy(g.exec);
  w.graphs.clear();
  for (void *p : {w.hlo, w.ulo, w.alo, w.g32, w.vt, w.vrow, w.s2, w.s2p, w.s3, w.s3p, w.h, w.u, w.a, w.g, w.melw, w.xw, w.dw32, w.wdq, w.msrc, w.skp})
    if (p) (void)hipFree(p);
  w = EncWs();
}
int encoder_copy_f4(fa_ctx *ctx, const void *src, void *dst, size_t bytes, const char *label) { return copy_f4(ctx, src, dst, bytes, label); }

int pass_geometry(fa_ctx *ctx, const fa_encoder *e, const int32_t *lens, int n, int layout, int pt, int pb, PassGeom *g) {
  const fa_encoder_cfg &c = e->cfg;
  const fa_encoder_opts &o = e->opts;
  if (n <= 0 || n > kMaxWin) return set_err(ctx, FA_E_INVALID, "encoder pass: %d windows", n);
  g->n = n;
  g->layout = layout;
  g->pt = pt;
  g->pb = pb;
  g->F[0] = c.melBins;
  for (int s = 1; s < 4; s++) g->F[s] = stride2_out(g->F[s - 1], o.sub_pad_l, o.sub_pad_r);
  if (g->F[3] != c.Fsub) return set_err(ctx, FA_E_INVALID, "encoder pass: melBins %d gives %d freq bins, manifest has %d", c.melBins, g->F[3], c.Fsub);
  for (int s = 0; s < 4; s++) {
    g->s[s] = WinStage{};
    g->s[s].n = n;
    g->mx[s] = 0;
  }
  for (int i = 0; i < n; i++) {
    if (lens[i] <= 0) return set_err(ctx, FA_E_INVALID, "encoder pass: window %d has length %d", i, lens[i]);
    g->s[0].len[i] = lens[i];
    for (int s = 1; s < 4; s++) g->s[s].len[i] = stride2_out(g->s[s - 1].len[i], pt, pb);
    if (g->s[3].len[i] <= 0) return set_err(ctx, FA_E_INVALID, "encoder pass: window %d (%d mel frames) subsamples to no frame", i, lens[i]);
    if (g->s[3].len[i] > e->maxT) return set_err(ctx, FA_E_INVALID, "encoder pass: window %d subsamples to %d frames > max_T %d", i, g->s[3].len[i], e->maxT);
    for (int s = 0; s < 4; s++) g->mx[s] = std::max(g->mx[s], g->s[s].len[i]);
  }
  for (int s = 0; s < 4; s++) {
    int acc = 0;
    for (int i = 0; i < n; i++) {
      g->s[s].off[i] = layout == 0 ? acc : i * g->mx[s];
      acc += layout == 0 ? g->s[s].len[i] : g->mx[s];
    }
    g->R[s] = acc;
  }
  g->M = g->R[3];
  return FA_OK;
}

// Quantised weights at large batches: the fused-dequant GEMM routes widen
// every B fragment in each wave that reads it, which costs more VALU than the
// MFMAs they feed once M fills the chip.  From kDequantRows rows on, each
// layer's linears are first widened once into an f16 [N][K] scratch (the
// exact values the fused routes compute: q for int8, with the column scale
// left to the epilogue; f16((q - 8)·s) for int4) and the f16 GEMM runs on
// them; the scratch is L2 / MALL-hot when the GEMM reads it.
constexpr int kDequantRows = 512;

// One launch per layer widens all its quantised linears: blockIdx.y = the
// linear, each lane one 8-value chunk (int8: 8 bytes; int4: one 4-byte word
// of a group-32 block, with the block's scale) -> 16 contiguous output bytes,
// so a wave's stores cover 1 KB without gaps; four chunks per lane, every
// load issued before the first store.  item i has chunks[i] chunks.
constexpr int kWdqMax = 8;
struct WdqList {
  const uint8_t *w[kWdqMax];
  const _Float16 *s[kWdqMax];
  _Float16 *out[kWdqMax];
  long chunks[kWdqMax];
  int n, i4;
};
constexpr int kWdqPer = 4;  // chunks per lane
__global__ __launch_bounds__(256) void wdq_kernel(WdqList L) {
  const int i = blockIdx.y;
  const long n8 = L.chunks[i];
  const long c0 = (long)blockIdx.x * 256 * kWdqPer + threadIdx.x;
  if (c0 >= n8) return;
  h8 o[kWdqPer];
  if (L.i4) {
    const uint32_t *w = reinterpret_cast<const uint32_t *>(L.w[i]);
    uint32_t v[kWdqPer];
    _Float16 sc[kWdqPer];
#pragma unroll
    for (int r = 0; r < kWdqPer; r++) {
      const long c = c0 + r * 256;
      v[r] = c < n8 ? w[c] : 0u;
      sc[r] = c < n8 ? L.s[i][c >> 2] : (_Float16)0.f;  // a group-32 block is 4 chunks
    }
#pragma unroll
    for (int r = 0; r < kWdqPer; r++) o[r] = i4x8_to_h8(v[r], sc[r]);
  } else {
    const uint2 *w = reinterpret_cast<const uint2 *>(L.w[i]);
    uint2 v[kWdqPer];
#pragma unroll
    for (int r = 0; r < kWdqPer; r++) {
      const long c = c0 + r * 256;
      v[r] = c < n8 ? w[c] : uint2{0u, 0u};
    }
#pragma unroll
    for (int r = 0; r < kWdqPer; r++) o[r] = i8x8_to_h8(v[r]);
  }
  h8 *out = reinterpret_cast<h8 *>(L.out[i]);
#pragma unroll
  for (int r = 0; r < kWdqPer; r++) {
    const long c = c0 + r * 256;
    if (c < n8) out[c] = o[r];
  }
}

static inline std::array<const Lin *, kWdqMax> layer_lins(const fa_encoder::Layer &Ly) {
  return {&Ly.ff1w1, &Ly.ff1w2, &Ly.qkv, &Ly.out, &Ly.pw1, &Ly.pw2, &Ly.ff2w1, &Ly.ff2w2};
}

static size_t wdq_bytes(const fa_encoder *e) {
  size_t mx = 0;
  for (const auto &Ly : e->L) {
    size_t t = 0;
    for (const Lin *L : layer_lins(Ly))
      if (L->bkind != B_F16) t += (size_t)L->N * L->K * 2;
    mx = std::max(mx, t);
  }
  return mx;
}

int pass_workspace(fa_ctx *ctx, fa_encoder *e, const PassGeom &g, int layers, bool stream) {
  const fa_encoder_cfg &c = e->cfg;
  const int D = c.D, C = c.Csub, M = g.M;
  FA_TRY(grow(e, &e->W().s2, &e->W().cap_s2, (size_t)g.R[2] * g.F[2] * 2 * C * 2));  // hi/lo f16
  FA_TRY(grow(e, &e->W().s2p, &e->W().cap_s2p, (size_t)g.R[2] * g.F[2] * C * 4));    // f32 pre-ReLU
  FA_TRY(grow(e, &e->W().s3, &e->W().cap_s3, (size_t)g.R[3] * g.F[3] * 2 * C * 2));  // hi/lo f16
  FA_TRY(grow(e, &e->W().s3p, &e->W().cap_s3p, (size_t)g.R[3] * g.F[3] * 2 * C * 2));  // hi/lo f16
  const size_t need_m = (size_t)M * D * 2, need_u = (size_t)M * std::max(c.DFF, 3 * D) * 2;
  if (need_m > e->W().cap_m) {
    size_t c1 = 0, c2 = 0, c3 = 0;
    if (e->W().h) { (void)hipDeviceSynchronize(); (void)hipFree(e->W().h); (void)hipFree(e->W().a); (void)hipFree(e->W().g); e->W().h = e->W().a = e->W().g = nullptr; e->ws_gen++; }
    FA_TRY(grow(e, &e->W().h, &c1, need_m));
    FA_TRY(grow(e, &e->W().a, &c2, need_m));
    FA_TRY(grow(e, &e->W().g, &c3, need_m));
    e->W().cap_m = need_m;
  }
  FA_TRY(grow(e, &e->W().u, &e->W().cap_u, need_u));
  unsigned any = 0;
  bool cln = false;
  for (int li = 0; li < layers; li++) {
    any |= e->L[li].exact;
    cln |= e->L[li].cln[0] != nullptr;
  }
  if (any & FA_EXACT_LN_OUT) FA_TRY(grow(e, &e->W().hlo, &e->W().cap_hlo, (size_t)M * D * 2));
  if (any & FA_EXACT_FF_HIDDEN) FA_TRY(grow(e, &e->W().ulo, &e->W().cap_ulo, (size_t)M * c.DFF * 2));
  if (any & (FA_EXACT_ATTN_OUT | FA_EXACT_DW_OUT)) FA_TRY(grow(e, &e->W().alo, &e->W().cap_alo, (size_t)M * D * 2));
  if (any & FA_EXACT_GLU) FA_TRY(grow(e, &e->W().g32, &e->W().cap_g32, (size_t)M * D * 4));
  if (cln) FA_TRY(grow(e, &e->W().dw32, &e->W().cap_dw32, (size_t)M * D * 4));
  if (e->format != FA_W_F16 && M >= kDequantRows) FA_TRY(grow(e, &e->W().wdq, &e->W().cap_wdq, wdq_bytes(e)));
  if (stream) FA_TRY(grow(e, &e->W().skp, &e->W().cap_skp, skinny_split_bytes(std::min(2 * c.D, kSkinnySplitMaxN))));
  if (!stream) {
    // transposed V per (window, head), written by the q|k|v GEMM's epilogue
    // (or v_transpose_kernel).  Keys past a window's end are never written:
    // the buffer starts zeroed and afterwards holds only finite V values of
    // earlier forwards there, which the attention weights by exactly 0.
    const int Tp = (g.mx[3] + 63) / 64 * 64;
    const uint64_t gen = e->ws_gen;
    FA_TRY(grow(e, &e->W().vt, &e->W().cap_vt, (size_t)g.n * c.H * c.HD * Tp * 2));
    if (e->ws_gen != gen) FA_HIP(ctx, hipMemsetAsync(e->W().vt, 0, e->W().cap_vt, ctx->stream));
    FA_TRY(grow(e, &e->W().vrow, &e->W().cap_vrow, (size_t)M * 4));
  }
  return FA_OK;
}

// The whole forward of one pass as a fixed kernel sequence (captured into a
// hipGraph by the callers when it repeats).  mel: [R0, melBins] time-major
// rows; x: [M, D] f32, the residual stream and the pass's output.
// Column groups of the front end's c01 / depthwise launches: a grid of fewer
// blocks than the chip's 256 CUs (a stream pass: a few rows) spreads each
// row's frequency columns over 8 groups; larger grids keep one.
static unsigned front_groups(unsigned blocks) { return blocks < 256 ? 8u : 1u; }

int pass_launch(fa_ctx *ctx, fa_encoder *e, const PassGeom &g, const float *melp, float *x, int layers, const StreamPass *sp) {
  const fa_encoder_cfg &c = e->cfg;
  const fa_encoder_opts &o = e->opts;
  const int D = c.D, C = c.Csub, MB = c.melBins, M = g.M, n = g.n, layout = g.layout;
  const int F1 = g.F[1], F2 = g.F[2], F3 = g.F[3];
  const WinStage &s0 = g.s[0], &s1 = g.s[1], &s2 = g.s[2], &s3 = g.s[3];
  const int *mx = g.mx, *R = g.R;
  const int Tp = (mx[3] + 63) / 64 * 64;
  _Float16 *h = (_Float16 *)e->W().h, *u = (_Float16 *)e->W().u, *a = (_Float16 *)e->W().a, *gg = (_Float16 *)e->W().g;
  // ── subsampling ──
  {
    ProfScope ps(ctx, "sub_c01");
    FA_TRY(launch_c01(ctx, ps, dim3(cdiv(mx[2], 4), n, front_groups(cdiv(mx[2], 4) * n)), melp, MB, s0, s1, F1, s2, F2, e->c0w, e->c0b, e->c1w, e->c1b, (_Float16 *)e->W().s2, C, e->c01_lds,
                      g.pt, o.sub_pad_l, o.sub_pad_r, g.mel_src));
    FA_TRY(check_launch(ctx, "sub_c01"));
  }
  {
    GemmArgs p;  // c2 (1x1) + bias; its ReLU is applied by the c3 kernel's loads
    p.A = e->W().s2; p.lda = 2 * C; p.akind = A_F16;
    set_gemm_b(p, e->c2);
    p.C = e->W().s2p; p.ldc = C;
    p.M = R[2] * F2; p.allow_skinny = sp != nullptr;
    FA_TRY(gemm_mfma(ctx, p, "sub_pw2"));
  }
  {
    ProfScope ps(ctx, "sub_dw3");
    FA_TRY(launch_dw(ctx, ps, dim3(cdiv(mx[3], 4), n, front_groups(cdiv(mx[3], 4) * n)), (const float *)e->W().s2p, s2, F2, s3, F3, e->c3w, e->c3b, (_Float16 *)e->W().s3, C,
                     sp ? nullptr : (int *)e->W().vrow, c.H * c.HD * Tp, layout == 1 ? mx[3] : 0, g.pt, o.sub_pad_l));
    FA_TRY(check_launch(ctx, "sub_dw3"));
  }
  {
    GemmArgs p;  // c4 (1x1) + bias + ReLU, written as hi/lo pairs for the linear
    p.A = e->W().s3; p.lda = 2 * C; p.akind = A_F16;
    set_gemm_b(p, e->c4);
    p.C = e->W().s3p; p.ldc = 2 * C; p.out_f16 = 1; p.hilo = 1;
    p.M = R[3] * F3; p.allow_skinny = sp != nullptr;
    FA_TRY(gemm_mfma(ctx, p, "sub_pw4"));
  }
  {
    GemmArgs p;
    p.A = e->W().s3p; p.lda = 2 * C * F3; p.akind = A_F16;
    set_gemm_b(p, e->lin);
    p.C = x; p.ldc = D;
    p.M = M; p.allow_skinny = sp != nullptr;
    FA_TRY(gemm_mfma(ctx, p, "sub_linear"));
  }

  // ── conformer layers ──
  // A operand (with an optional exact lo plane) -> C (with an optional lo plane)
  // quantised weights, batches of >= kDequantRows rows: each layer's linears
  // are widened (one launch) right before the layer runs.  Widening the next
  // layer on a second stream during the current one was measured slower
  // (int8 7.84 -> 8.59 ms per configs[4] batch): the copy competes with the
  // GEMMs for HBM and CU slots and the GEMMs lose more than the copy takes.
  const bool dq = e->format != FA_W_F16 && M >= kDequantRows;
  WdqList wdq{};
  const Lin *wdq_src[kWdqMax] = {};
  auto dequant_layer = [&](const fa_encoder::Layer &Ly) -> int {
    WdqList &W = wdq;
    W = WdqList{};
    _Float16 *dst = (_Float16 *)e->W().wdq;
    long mx = 0;
    for (const Lin *L : layer_lins(Ly)) {
      if (L->bkind == B_F16) continue;
      W.w[W.n] = (const uint8_t *)L->w;
      W.s[W.n] = (const _Float16 *)L->scales;
      W.out[W.n] = dst;
      W.chunks[W.n] = (long)L->N * L->K / 8;
      mx = std::max(mx, W.chunks[W.n]);
      W.i4 = L->bkind == B_I4;
      wdq_src[W.n++] = L;
      dst += (size_t)L->N * L->K;
    }
    if (!W.n) return FA_OK;
    ProfScope ps(ctx, "dequant_w");
    FA_LAUNCH(ps, wdq_kernel, dim3(cdiv(mx, 256 * kWdqPer), W.n), dim3(256), 0, ctx->stream, W);
    return check_launch(ctx, "dequant_w");
  };
  // stream passes of <= 16 rows: the LayerNorm ahead of the q|k|v, pw1 and
  // FF2 W1 products is folded into their skinny GEMM (A built from the
  // residual rows in the kernel), one launch fewer each (FA_LN_FOLD=0: off).
  // Measured per 160 ms chunk, 24 layers: one stream 2.34 -> 2.22 ms; at 32
  // rows (16 batched streams) every workgroup's row statistics cost more
  // than the launch saved (617 -> 608 aggregate audio-s/wall-s), so not there.
  const char *lf = getenv("FA_LN_FOLD");
  const bool fold_ln = sp && M <= 16 && D == 1024 && e->format == FA_W_F16 && !(lf && lf[0] == '0');
  struct {
    const float *g = nullptr, *b = nullptr;
    bool lo = false;
  } lnf;
  auto gemm = [&](const void *A, const void *Alo, int lda, const Lin &L, void *Cp, void *Clo, int ldc, int out_f16, int act, const float *add, int glu,
                  const char *label) {
    GemmArgs p;
    p.A = A; p.Alo = Alo; p.lda = lda; p.akind = A_F16;
    if (lnf.g) {  // A = LayerNorm(x) (+ its lo plane), built in the GEMM
      p.A = nullptr; p.Alo = nullptr;
      p.ln_x = x; p.ln_g = lnf.g; p.ln_b = lnf.b; p.ln_eps = 1e-5f; p.ln_lo = lnf.lo;
      lnf.g = lnf.b = nullptr;
    }
    set_gemm_b(p, L);
    if (L.bkind != B_F16 && M >= kDequantRows) {  // the layer's widened copy (dequant_layer), f16 route
      const _Float16 *wf = nullptr;
      for (int i = 0; i < wdq.n; i++)
        if (wdq_src[i] == &L) wf = wdq.out[i];
      if (!wf) return set_err(ctx, FA_E_STATE, "%s: quantised weights were not widened for this layer", label);
      p.B = wf;
      p.bkind = B_F16;
      p.bscale = nullptr;
    }
    p.C = Cp; p.Clo = Clo; p.ldc = ldc; p.out_f16 = out_f16; p.act = act;
    p.add = add; p.ldadd = ldc; p.glu = glu;
    p.M = M; p.allow_skinny = sp != nullptr;
    if (sp) {
      p.skp = (float *)e->W().skp;
      p.skp_bytes = e->W().cap_skp;
    }
    return gemm_mfma(ctx, p, label);
  };
  _Float16 *hlo = (_Float16 *)e->W().hlo, *ulo = (_Float16 *)e->W().ulo, *alo = (_Float16 *)e->W().alo;
  float *g32 = (float *)e->W().g32;
  // LayerNorm of rows `src` into the f16 operand dst (+ lo plane); silu: the conv-module LayerNorm
  auto ln_into = [&](const float *src, const float *gm, const float *bt, _Float16 *dst, _Float16 *lo, bool silu, const char *label) -> int {
    if (D % 256 == 0 && D <= 2048) {
      ProfScope ps(ctx, label);
      const dim3 grid(cdiv(M, 4));
#define FA_LNK(V)                                                                                                                       \
  do {                                                                                                                                  \
    if (silu)                                                                                                                           \
      FA_LAUNCH(ps, (enc_ln_kernel<V, true>), grid, dim3(256), 0, ctx->stream, src, gm, bt, dst, lo, M, 1e-5f);                        \
    else                                                                                                                                \
      FA_LAUNCH(ps, (enc_ln_kernel<V, false>), grid, dim3(256), 0, ctx->stream, src, gm, bt, dst, lo, M, 1e-5f);                       \
  } while (0)
      switch (D / 256) {
        case 1: FA_LNK(1); break;
        case 2: FA_LNK(2); break;
        case 4: FA_LNK(4); break;
        case 8: FA_LNK(8); break;
        default: silu = false; break;
      }
#undef FA_LNK
      if (D / 256 == 1 || D / 256 == 2 || D / 256 == 4 || D / 256 == 8) return check_launch(ctx, label);
    }
    if (silu) return set_err(ctx, FA_E_UNSUPPORTED, "%s: conv-module LayerNorm needs D a multiple of 256 (<= 2048)", label);
    return layernorm_launch(ctx, src, gm, bt, dst, 1, M, D, D, D, 1e-5f, label);
  };
  auto ln = [&](int which, const fa_encoder::Layer &Ly, const char *label) -> int {
    return ln_into(x, Ly.ln[which][0], Ly.ln[which][1], h, (Ly.exact & FA_EXACT_LN_OUT) ? hlo : nullptr, false, label);
  };
  AttnArgs at;
  at.q = u; at.k = u + D; at.v = u + 2 * D;
  at.ldq = at.ldk = at.ldv = 3 * D;
  at.ldp = D; at.prows = 2 * e->maxT - 1; at.pcenter = e->maxT - 1;
  at.out = a; at.ldo = D;
  at.H = c.H; at.HD = c.HD;
  at.chunk = o.att_chunk; at.left = o.att_left; at.right = o.att_right;
  at.win.n = n;
  for (int i = 0; i < n; i++) {
    at.win.off[i] = s3.off[i];
    at.win.len[i] = s3.len[i];
  }
  const bool fuse_ln = D == 256 || D == 512 || D == 1024 || D == 2048;  // norm_out + the next layer's norm_ff1 in one pass
  const bool plain_dw = !o.conv_causal && !sp;  // the offline symmetric depthwise conv (BatchNorm folded)
  for (int li = 0; li < layers; li++) {
    auto &Ly = e->L[li];
    if (dq) FA_TRY(dequant_layer(Ly));
    const unsigned ex = Ly.exact;
    const void *hl = (ex & FA_EXACT_LN_OUT) ? hlo : nullptr;
    void *ul = (ex & FA_EXACT_FF_HIDDEN) ? ulo : nullptr;
    // FF1 (its LayerNorm ran with the previous layer's norm_out)
    if (li == 0 || !fuse_ln) FA_TRY(ln(0, Ly, hl ? "ln_ff1_x" : "ln_ff1"));
    FA_TRY(gemm(h, hl, D, Ly.ff1w1, u, ul, c.DFF, 1, FA_ACT_SILU, nullptr, 0, hl ? "ff1_w1_x" : (ul ? "ff1_w1_u" : "ff1_w1")));
    FA_TRY(gemm(u, ul, c.DFF, Ly.ff1w2, x, nullptr, D, 0, FA_ACT_NONE, x, 0, ul ? "ff1_w2_x" : "ff1_w2"));
    // attention
    if (!fold_ln) FA_TRY(ln(1, Ly, hl ? "ln_att_x" : "ln_att"));
    bool vt_fused = false;
    {
      // q|k|v; offline, V goes straight to the attention's transposed buffer
      // when the direct-to-LDS route runs it (FA_VT_FUSE=0 at load keeps v_transpose)
      GemmArgs p;
      p.A = h; p.Alo = hl; p.lda = D; p.akind = A_F16;
      set_gemm_b(p, Ly.qkv);
      p.C = u; p.ldc = 3 * D; p.out_f16 = 1;
      p.M = M; p.allow_skinny = sp != nullptr;
      if (fold_ln) {  // norm_att folded in
        p.A = nullptr; p.Alo = nullptr;
        p.ln_x = x; p.ln_g = Ly.ln[1][0]; p.ln_b = Ly.ln[1][1]; p.ln_eps = 1e-5f; p.ln_lo = hl != nullptr;
      }
      if (!sp && c.HD == 128 && e->vt_fuse && gemm_takes_direct(ctx, p)) {
        p.vt = (_Float16 *)e->W().vt; p.vrow = (const int *)e->W().vrow; p.vcol0 = 2 * D; p.vtp = Tp;
        vt_fused = true;
      }
      FA_TRY(gemm_mfma(ctx, p, hl ? "qkv_x" : "qkv"));
    }
    _Float16 *olo = (ex & FA_EXACT_ATTN_OUT) ? alo : nullptr;
    if (!sp) {
      at.pos = Ly.P;
      at.pbu = Ly.pbu;
      at.pbv = Ly.pbv;
      at.out_lo = olo;
      FA_TRY(relpos_attention_f16(ctx, at, mx[3], (_Float16 *)e->W().vt, olo ? "attention_x" : "attention", !vt_fused));
    } else {
      const size_t kvo = (size_t)li * sp->kv_ld * D;
      const int nq = M / n;  // frames per window (stream)
      {
        ProfScope ps(ctx, "stream_attention");
        FA_LAUNCH(ps, stream_attn_kernel, dim3(cdiv(nq, 4), c.H, n), dim3(256), 0, ctx->stream, u, 3 * D, sp->kv, kvo, sp->Lc, nq, D,
                  Ly.P + (size_t)(e->maxT - 1 - sp->dMax) * D, sp->Pn, sp->dMax, Ly.pbu, Ly.pbv, sp->chunk, sp->left, sp->right, a, olo, sp->nemit,
                  sp->keep);
        FA_TRY(check_launch(ctx, "stream_attention"));
      }
    }
    FA_TRY(gemm(a, olo, D, Ly.out, x, nullptr, D, 0, FA_ACT_NONE, x, 0, olo ? "attn_out_x" : "attn_out"));
    // conv module: pw1 + GLU (f16, or f32 when exact) -> depthwise (+ LayerNorm) + SiLU -> pw2
    if (fold_ln)  // norm_conv folded into pw1
      lnf = {Ly.ln[2][0], Ly.ln[2][1], hl != nullptr};
    else
      FA_TRY(ln(2, Ly, hl ? "ln_conv_x" : "ln_conv"));
    const bool glu32 = ex & FA_EXACT_GLU;
    FA_TRY(gemm(h, hl, D, Ly.pw1, glu32 ? (void *)g32 : (void *)gg, nullptr, D, glu32 ? 0 : 1, FA_ACT_NONE, nullptr, 1,
                hl ? "pw1_glu_x" : (glu32 ? "pw1_glu_f32" : "pw1_glu")));
    _Float16 *dlo = (ex & FA_EXACT_DW_OUT) ? alo : nullptr;
    if (plain_dw && !Ly.cln[0]) {
      ProfScope ps(ctx, glu32 ? (dlo ? "dwconv_x" : "dwconv_f32") : (dlo ? "dwconv_lo" : "dwconv"));
      // 4 channels x 16 frames per thread: inputs read 1.5x (24 rows per 16
      // outputs); measured 9.6 us against 10.9 for 8 channels x 4 frames (3x)
      const int thr = std::min(64, D / 4);
      const dim3 grid(cdiv(mx[3], 16), n, cdiv(D / 4, thr));
      if (glu32)
        FA_LAUNCH(ps, (dwconv_silu_kernel<9, 16, 4, float>), grid, dim3(thr), 0, ctx->stream, (const float *)g32, a, dlo, Ly.dww, Ly.dwb, D, s3);
      else
        FA_LAUNCH(ps, (dwconv_silu_kernel<9, 16, 4, _Float16>), grid, dim3(thr), 0, ctx->stream, (const _Float16 *)gg, a, dlo, Ly.dww, Ly.dwb, D, s3);
      FA_TRY(check_launch(ctx, "dwconv"));
    } else {
      static const CcSlots no_slots{};
      const CcSlots &slots = sp ? sp->cc : no_slots;  // a stream pass: per-window conv caches
      const int use_slots = sp != nullptr;
      const size_t cco = (size_t)li * 8 * D;
      float *y32 = Ly.cln[0] ? (float *)e->W().dw32 : nullptr;
      if (y32 && D % 4 == 0 && D <= 1024) {  // depthwise + conv-module LayerNorm + SiLU (+ the stream's conv cache) in one kernel
        ProfScope ps(ctx, "dwconv_ln");
        const dim3 grid(mx[3], n);
        if (glu32)
          FA_LAUNCH(ps, dwconv_ln_kernel<float>, grid, dim3(256), 0, ctx->stream, (const float *)g32, slots, use_slots, cco, s3, o.conv_causal, Ly.dww, Ly.dwb, Ly.cln[0],
                    Ly.cln[1], D, a, dlo, sp ? sp->nemit : 0);
        else
          FA_LAUNCH(ps, dwconv_ln_kernel<_Float16>, grid, dim3(256), 0, ctx->stream, (const _Float16 *)gg, slots, use_slots, cco, s3, o.conv_causal, Ly.dww, Ly.dwb,
                    Ly.cln[0], Ly.cln[1], D, a, dlo, sp ? sp->nemit : 0);
        FA_TRY(check_launch(ctx, "dwconv_ln"));
      } else {
        {
          ProfScope ps(ctx, "dwconv_gen");
          const dim3 grid(mx[3], n, cdiv(D / 4, 64));
          if (glu32)
            FA_LAUNCH(ps, dwconv_gen_kernel<float>, grid, dim3(64), 0, ctx->stream, (const float *)g32, slots, use_slots, cco, s3, o.conv_causal, Ly.dww, Ly.dwb, D, a, dlo,
                      y32);
          else
            FA_LAUNCH(ps, dwconv_gen_kernel<_Float16>, grid, dim3(64), 0, ctx->stream, (const _Float16 *)gg, slots, use_slots, cco, s3, o.conv_causal, Ly.dww, Ly.dwb, D, a,
                      dlo, y32);
          FA_TRY(check_launch(ctx, "dwconv_gen"));
        }
        if (y32) FA_TRY(ln_into(y32, Ly.cln[0], Ly.cln[1], a, dlo, true, "conv_ln_silu"));
        if (sp) {
          ProfScope ps(ctx, "stream_conv_cache");
          if (glu32)
            FA_LAUNCH(ps, stream_conv_cache_kernel<float>, dim3(8, n), dim3(256), 0, ctx->stream, slots, cco, (const float *)g32, D, sp->nemit, M / n);
          else
            FA_LAUNCH(ps, stream_conv_cache_kernel<_Float16>, dim3(8, n), dim3(256), 0, ctx->stream, slots, cco, (const _Float16 *)gg, D, sp->nemit, M / n);
          FA_TRY(check_launch(ctx, "stream_conv_cache"));
        }
      }
    }
    FA_TRY(gemm(a, dlo, D, Ly.pw2, x, nullptr, D, 0, FA_ACT_NONE, x, 0, dlo ? "pw2_x" : "pw2"));
    // FF2 + norm_out
    if (fold_ln)  // norm_ff2 folded into FF2 W1
      lnf = {Ly.ln[3][0], Ly.ln[3][1], hl != nullptr};
    else
      FA_TRY(ln(3, Ly, hl ? "ln_ff2_x" : "ln_ff2"));
    FA_TRY(gemm(h, hl, D, Ly.ff2w1, u, ul, c.DFF, 1, FA_ACT_SILU, nullptr, 0, hl ? "ff2_w1_x" : (ul ? "ff2_w1_u" : "ff2_w1")));
    FA_TRY(gemm(u, ul, c.DFF, Ly.ff2w2, x, nullptr, D, 0, FA_ACT_NONE, x, 0, ul ? "ff2_w2_x" : "ff2_w2"));
    if (fuse_ln && li + 1 < layers) {
      const auto &Ln = e->L[li + 1];
      _Float16 *nlo = (Ln.exact & FA_EXACT_LN_OUT) ? hlo : nullptr;
      const char *lab = nlo ? "ln_out_ff1_x" : "ln_out_ff1";
      ProfScope ps(ctx, lab);
      const dim3 grid(cdiv(M, 4));
      switch (D / 256) {
        case 1: FA_LAUNCH(ps, enc_ln2_kernel<1>, grid, dim3(256), 0, ctx->stream, x, Ly.ln[4][0], Ly.ln[4][1], Ln.ln[0][0], Ln.ln[0][1], h, nlo, M, 1e-5f); break;
        case 2: FA_LAUNCH(ps, enc_ln2_kernel<2>, grid, dim3(256), 0, ctx->stream, x, Ly.ln[4][0], Ly.ln[4][1], Ln.ln[0][0], Ln.ln[0][1], h, nlo, M, 1e-5f); break;
        case 4: FA_LAUNCH(ps, enc_ln2_kernel<4>, grid, dim3(256), 0, ctx->stream, x, Ly.ln[4][0], Ly.ln[4][1], Ln.ln[0][0], Ln.ln[0][1], h, nlo, M, 1e-5f); break;
        case 8: FA_LAUNCH(ps, enc_ln2_kernel<8>, grid, dim3(256), 0, ctx->stream, x, Ly.ln[4][0], Ly.ln[4][1], Ln.ln[0][0], Ln.ln[0][1], h, nlo, M, 1e-5f); break;
        default: return set_err(ctx, FA_E_UNSUPPORTED, "fused LayerNorm: D = %d", D);
      }
      FA_TRY(check_launch(ctx, lab));
    } else if (D == 1024) {
      ProfScope ps(ctx, "ln_out");
      FA_LAUNCH(ps, enc_ln_f32_kernel<4>, dim3(cdiv(M, 4)), dim3(256), 0, ctx->stream, x, Ly.ln[4][0], Ly.ln[4][1], M, 1e-5f);
      FA_TRY(check_launch(ctx, "ln_out"));
    } else {
      FA_TRY(layernorm_launch(ctx, x, Ly.ln[4][0], Ly.ln[4][1], x, 0, M, D, D, D, 1e-5f, "ln_out"));
    }
  }
  if (layout == 1) {
    ProfScope ps(ctx, "zero_pad");
    FA_LAUNCH(ps, zero_pad_rows_kernel, dim3(mx[3], n), dim3(256), 0, ctx->stream, x, D, s3, mx[3]);
    FA_TRY(check_launch(ctx, "zero_pad"));
  }
  return FA_OK;
}

}  // namespace fa

using namespace fa;

// Writes the feature-stream descriptor the front end reads (a kernel rather
// than a copy: its argument bytes are taken at launch, so the host array can
// change right after, and no memset / copy node ever sits in a graph).
__global__ void set_mel_src_kernel(MelSrc v, MelSrc *dst) {
  if (threadIdx.x == 0) dst->ptr = v.ptr, dst->ttot = v.ttot;
  if (threadIdx.x < kMaxWin) dst->start[threadIdx.x] = v.start[threadIdx.x];
}

// The forward over one batch of windows, from raw device pointers.  mel is
// either time-major rows [R0, melBins] (stream false) or the channel-major
// feature stream [melBins, mel_cols] whose windows start at columns starts[]
// (stream true).  xout: the [M, D] f32 result goes there; null: it stays in
// the workspace's xw (valid until the next forward in this workspace) and
// *xres names it.
int fa::encoder_forward_dev(fa_ctx *ctx, fa_encoder *e, const float *mel, int mel_rows, long mel_cols, bool stream, const int32_t *starts,
                        const int32_t *lens, int n, int layout, int layers_run, float *xout, const float **xres, int *M_out, const char *who) {
  if (!e || e->ctx != ctx) return set_err(ctx, FA_E_INVALID, "%s: encoder belongs to another context", who);
  if (n <= 0) return set_err(ctx, FA_E_INVALID, "%s: no windows", who);
  // At most 32 windows per batch: the largest batch validated on the GPU.  A
  // 64-window batch inside a one-hour windowed transcription once faulted the
  // GPU with no cause shown yet, so larger batches are refused here rather
  // than only by the Python pipeline.
#ifndef FA_ENC_MAX_WINDOWS  // raised only by the launch-audit build (tests/audit), never shipped
#define FA_ENC_MAX_WINDOWS 32
#endif
  constexpr int kMaxEncWin = FA_ENC_MAX_WINDOWS;
  static_assert(kMaxEncWin <= kMaxWin, "window tables");
  if (n > kMaxEncWin) return set_err(ctx, FA_E_UNSUPPORTED, "%s: %d windows in one batch (max %d)", who, n, kMaxEncWin);
  if (layout != 0 && layout != 1) return set_err(ctx, FA_E_INVALID, "%s: layout %d", who, layout);
  const fa_encoder_cfg &c = e->cfg;
  const int D = c.D, MB = c.melBins;
  if (!stream && mel_cols != MB) return set_err(ctx, FA_E_INVALID, "%s: mel must be f32 [rows, %d]", who, MB);
  if (stream && mel_rows != MB) return set_err(ctx, FA_E_INVALID, "%s: features must be f32 [%d, T]", who, MB);
  PassGeom g;
  FA_TRY(pass_geometry(ctx, e, lens, n, layout, e->opts.sub_pad_t, e->opts.sub_pad_b, &g));
  MelSrc src{};
  if (stream) {
    src.ttot = mel_cols;
    for (int i = 0; i < n; i++) {
      if (starts[i] < 0 || (long)starts[i] + lens[i] > mel_cols)
        return set_err(ctx, FA_E_INVALID, "%s: window %d [%d, +%d) outside the %ld-frame stream", who, i, starts[i], lens[i], mel_cols);
      src.start[i] = starts[i];
    }
  } else if (mel_rows < g.R[0]) {
    return set_err(ctx, FA_E_INVALID, "%s: mel has %d rows, windows need %d", who, mel_rows, g.R[0]);
  }
  const int M = g.M;
  if (M_out) *M_out = M;
  const int layers = layers_run < 0 ? c.layers : std::min(layers_run, c.layers);
  FA_TRY(pass_workspace(ctx, e, g, layers, false));
  const char *ge = getenv("FA_GRAPH");
  const bool use_graph = !ctx->prof_on && !(ge && ge[0] == '0');
  if (stream) {
    FA_TRY(grow(e, &e->W().msrc, &e->W().cap_msrc, sizeof(MelSrc)));
    g.mel_src = (const MelSrc *)e->W().msrc;
  }
  if (use_graph && !stream) FA_TRY(grow(e, &e->W().melw, &e->W().cap_melw, (size_t)g.R[0] * MB * 4));
  if (use_graph || !xout) FA_TRY(grow(e, &e->W().xw, &e->W().cap_xw, (size_t)M * D * 4));
  float *const x = xout ? xout : (float *)e->W().xw;
  if (xres) *xres = (const float *)e->W().xw;
  auto set_src = [&]() -> int {
    src.ptr = mel;
    ProfScope ps(ctx, "enc_src");
    FA_LAUNCH(ps, set_mel_src_kernel, dim3(1), dim3(64), 0, ctx->stream, src, (MelSrc *)e->W().msrc);
    return check_launch(ctx, "enc_src");
  };
  if (!use_graph) {  // profiling (its events are per launch) or FA_GRAPH=0
    if (stream) FA_TRY(set_src());
    return pass_launch(ctx, e, g, mel, x, layers, nullptr);
  }
  // The whole forward is a fixed kernel sequence for a given signature: it is
  // captured once into a hipGraph and replayed (one submission instead of
  // ~700 launches).  The graph reads its input from a fixed place (melw, or
  // the stream descriptor msrc for the channel-major form) and writes xw
  // (fixed per workspace generation), so the key holds no caller pointer and
  // no window start: a caller that keeps earlier outputs alive, or moves to
  // another stream or other starts, still replays the same graph.
  std::vector<int64_t> key = {(int64_t)e->ws_gen, layers, n, layout, stream ? 1 : 0};
  key.insert(key.end(), lens, lens + n);
  FA_TRY(encoder_graph_run(
      ctx, e, key,
      [&]() { return pass_launch(ctx, e, g, stream ? nullptr : (const float *)e->W().melw, (float *)e->W().xw, layers, nullptr); },
      [&]() { return stream ? set_src() : copy_f4(ctx, mel, e->W().melw, (size_t)g.R[0] * MB * 4, "enc_in"); }));
  if (xout) FA_TRY(copy_f4(ctx, e->W().xw, xout, (size_t)M * D * 4, "enc_out"));
  return FA_OK;
}

// Shared body of fa_encoder_forward (mel: time-major rows) and
// fa_encoder_forward_stream (mel: channel-major stream [melBins, T],
// starts: the windows' first columns): the output tensor around
// encoder_forward_dev.
static int encoder_forward_impl(fa_ctx *ctx, fa_encoder *e, fa_tensor mel, const int32_t *starts, long, const int32_t *lens, int n,
                                int layout, int layers_run, fa_tensor *out, const char *who) {
  if (!e || e->ctx != ctx) return set_err(ctx, FA_E_INVALID, "%s: encoder belongs to another context", who);
  if (n <= 0) return set_err(ctx, FA_E_INVALID, "%s: no windows", who);
  TensorRec *rm;
  FA_TRY(need(ctx, mel, &rm, who));
  if (rm->kind != S_F32) return set_err(ctx, FA_E_INVALID, "%s: %s must be f32", who, starts ? "features" : "mel");
  PassGeom g;
  FA_TRY(pass_geometry(ctx, e, lens, n, layout == 1 ? 1 : 0, e->opts.sub_pad_t, e->opts.sub_pad_b, &g));
  fa_tensor ox;
  TensorRec *rx;
  FA_TRY(new_tensor(ctx, g.M, e->cfg.D, S_F32, (size_t)g.M * e->cfg.D * 4, &ox, &rx));
  TensorGuard og(ctx, ox);  // released unless the forward is queued
  rm = get(ctx, mel);
  FA_TRY(encoder_forward_dev(ctx, e, (const float *)rm->ptr, rm->rows, rm->cols, starts != nullptr, starts, lens, n, layout, layers_run,
                             (float *)rx->ptr, nullptr, nullptr, who));
  *out = og.release();
  return FA_OK;
}

extern "C" {

int fa_encoder_tsub(int T) { return stride2_len(stride2_len(stride2_len(T))); }
int fa_encoder_tsub_of(const fa_encoder *enc, int T) { return enc ? enc_tsub(enc->opts, T) : -1; }

int fa_quantize_weights(int format, const float *w, int K, int N, void *q_out, void *scales_out) {
  if (!w || !q_out || !scales_out || K <= 0 || N <= 0) return FA_E_INVALID;
  std::vector<float> bt((size_t)N * K);
  for (int k = 0; k < K; k++)
    for (int n = 0; n < N; n++) bt[(size_t)n * K + k] = w[(size_t)k * N + n];
  if (format == 1) {
    quantize_int8_km(bt.data(), N, K, (int8_t *)q_out, (float *)scales_out);
    return FA_OK;
  }
  if (format == 2) {
    quantize_int4_km(bt.data(), N, K, (uint8_t *)q_out, (uint16_t *)scales_out);
    return FA_OK;
  }
  return FA_E_INVALID;
}

void fa_encoder_destroy(fa_encoder *enc) {
  if (!enc) return;
  (void)hipDeviceSynchronize();  // the context stream and the lane streams
  for (void *p : enc->allocs) (void)hipFree(p);
  for (auto &w : enc->ws) encoder_ws_free(w);
  stream_lanes_free(enc);
  for (int l = 0; l < fa_encoder::kLanes; l++) {
    if (enc->lane_done[l]) (void)hipEventDestroy(enc->lane_done[l]);
    if (enc->lane_stream[l]) (void)hipStreamDestroy(enc->lane_stream[l]);
  }
  if (enc->lanes_in) (void)hipEventDestroy(enc->lanes_in);
  delete enc;
}

int fa_encoder_set_exact(fa_encoder *enc, int first_layer, int last_layer, unsigned mask) {
  if (!enc) return FA_E_INVALID;
  const int nl = (int)enc->L.size();
  if (first_layer < 0 || last_layer >= nl || first_layer > last_layer) return set_err(enc->ctx, FA_E_INVALID, "setExact: layers [%d, %d] of %d", first_layer, last_layer, nl);
  if (mask & ~31u) return set_err(enc->ctx, FA_E_INVALID, "setExact: unknown bits 0x%x", mask);
  if ((mask & FA_EXACT_LN_OUT) && (enc->cfg.D % 256 || enc->cfg.D > 2048))
    return set_err(enc->ctx, FA_E_UNSUPPORTED, "setExact: exact LayerNorm output needs D a multiple of 256 (<= 2048)");
  for (int l = first_layer; l <= last_layer; l++) enc->L[l].exact = mask;
  enc->ws_gen++;  // captured forwards bake the masks in
  return FA_OK;
}

int fa_encoder_get_exact(const fa_encoder *enc, int layer) {
  if (!enc || layer < 0 || layer >= (int)enc->L.size()) return -1;
  return (int)enc->L[layer].exact;
}

int fa_encoder_load(fa_ctx *ctx, const fa_encoder_cfg *cfg, int n, const char *const *names, const float *const *data, const int64_t *counts,
                    int format, int max_T, fa_encoder **out) {
  return fa_encoder_load_opts(ctx, cfg, nullptr, n, names, data, counts, format, max_T, out);
}

int fa_encoder_load_opts(fa_ctx *ctx, const fa_encoder_cfg *cfg, const fa_encoder_opts *opts, int n, const char *const *names,
                         const float *const *data, const int64_t *counts, int format, int max_T, fa_encoder **out) {
  if (!ctx || !cfg || !out) return FA_E_INVALID;
  *out = nullptr;
  const fa_encoder_cfg c = *cfg;
  const fa_encoder_opts o = opts ? *opts : fa_encoder_opts{1, 1, 1, 1, 0, 0, 0, 0};
  if (o.sub_pad_t < 0 || o.sub_pad_b < 0 || o.sub_pad_l < 0 || o.sub_pad_r < 0 || o.sub_pad_t > 2 || o.sub_pad_l > 2 || o.sub_pad_b > 2 || o.sub_pad_r > 2)
    return set_err(ctx, FA_E_UNSUPPORTED, "encoder: subsampling pads t%d b%d l%d r%d (0..2 supported)", o.sub_pad_t, o.sub_pad_b, o.sub_pad_l, o.sub_pad_r);
  if (o.att_chunk < 0 || o.att_left < 0 || o.att_right < 0) return set_err(ctx, FA_E_INVALID, "encoder: negative attention chunk / context");
  if (c.HD != 128 || c.H * c.HD != c.D) return set_err(ctx, FA_E_UNSUPPORTED, "encoder: needs HD=128 and H*HD=D (got H=%d HD=%d D=%d)", c.H, c.HD, c.D);
  {
    int F = c.melBins;
    for (int i = 0; i < 3; i++) F = stride2_out(F, o.sub_pad_l, o.sub_pad_r);
    if (c.D % 64 || c.DFF % 64 || c.Csub % 64 || F != c.Fsub || (c.Csub * c.Fsub) % 32 || c.melBins + o.sub_pad_l + o.sub_pad_r > 4096)
      return set_err(ctx, FA_E_UNSUPPORTED, "encoder: D, DFF, Csub must be multiples of 64 and melBins must subsample to Fsub (%d bins -> %d, Fsub %d)",
                     c.melBins, F, c.Fsub);
  }
  if (c.Csub != 64 && c.Csub != 128 && c.Csub != 256 && c.Csub != 512) return set_err(ctx, FA_E_UNSUPPORTED, "encoder: Csub must be 64, 128, 256 or 512");
  if (c.dwK != 9) return set_err(ctx, FA_E_UNSUPPORTED, "encoder: depthwise kernel %d (9 supported)", c.dwK);
  if (max_T <= 0 || max_T > 1024) return set_err(ctx, FA_E_INVALID, "encoder: max_T %d outside 1..1024", max_T);
  if (format < FA_W_F16 || format > FA_W_INT4) return set_err(ctx, FA_E_INVALID, "encoder: weight format %d", format);
  std::unordered_map<std::string, std::pair<const float *, int64_t>> man;
  for (int i = 0; i < n; i++) man[names[i]] = {data[i], counts[i]};
  auto get = [&](const std::string &k, int64_t cnt, bool optional, const float **p) -> int {
    auto it = man.find(k);
    if (it == man.end()) {
      if (optional) {
        *p = nullptr;
        return FA_OK;
      }
      return set_err(ctx, FA_E_INVALID, "encoder load: missing tensor %s", k.c_str());
    }
    if (it->second.second != cnt) return set_err(ctx, FA_E_INVALID, "encoder load: %s has %lld values, expected %lld", k.c_str(), (long long)it->second.second, (long long)cnt);
    *p = it->second.first;
    return FA_OK;
  };
  fa_encoder *e = new fa_encoder();
  e->ctx = ctx;
  e->cfg = c;
  e->opts = o;
  e->format = format;
  e->maxT = max_T;
  if (const char *vf = getenv("FA_VT_FUSE")) e->vt_fuse = vf[0] != '0';
  if (const char *cl = getenv("FA_C01_LDS")) e->c01_lds = cl[0] != '0';
  if (const char *nl = getenv("FA_ENC_LANES")) e->nlanes = std::max(1, std::min(fa_encoder::kLanes, atoi(nl)));
  auto fail = [&](int st) {
    fa_encoder_destroy(e);
    return st;
  };
  const int D = c.D, DFF = c.DFF, C = c.Csub, F = c.Fsub;
  const double INV = 1.0 / std::sqrt((double)c.HD);
  // ── front end ──
  const float *p;
  int st;
  if ((st = get("c0w", (int64_t)C * 9, false, &p))) return fail(st);
  e->c0w = dupload(e, p, (size_t)C * 9);
  if ((st = get("c0b", C, false, &p))) return fail(st);
  e->c0b = dupload(e, p, C);
  for (int i : {1, 3}) {
    const float *w, *b;
    if ((st = get("c" + std::to_string(i) + "w", (int64_t)C * 9, false, &w))) return fail(st);
    if ((st = get("c" + std::to_string(i) + "b", C, false, &b))) return fail(st);
    std::vector<float> wt((size_t)9 * C);
    for (int ch = 0; ch < C; ch++)
      for (int k = 0; k < 9; k++) wt[(size_t)k * C + ch] = w[ch * 9 + k];
    float *dw = dupload(e, wt.data(), wt.size()), *db = dupload(e, b, C);
    if (i == 1) {
      e->c1w = dw;
      e->c1b = db;
    } else {
      e->c3w = dw;
      e->c3b = db;
    }
  }
  {
    // pointwise convs and the linear stay f16 in every format (the quantised
    // formats cover the conformer layers' linears)
    const int saved = e->format;
    e->format = FA_W_F16;
    for (int i : {2, 4}) {
      const float *w, *b;
      if ((st = get("c" + std::to_string(i) + "w", (int64_t)C * C, false, &w))) return fail(st);
      if ((st = get("c" + std::to_string(i) + "b", C, false, &b))) return fail(st);
      // [cout][cin] is already Bt; each input channel's row appears twice
      // (hi and lo halves of the activation pairs)
      std::vector<float> bt((size_t)C * 2 * C), bias(b, b + C), fold(C, 1.f);
      for (int co = 0; co < C; co++)
        for (int ci = 0; ci < C; ci++) bt[(size_t)co * 2 * C + 2 * ci] = bt[(size_t)co * 2 * C + 2 * ci + 1] = w[(size_t)co * C + ci];
      if ((st = build_lin(e, i == 2 ? e->c2 : e->c4, bt, C, 2 * C, fold, &bias, "pw conv"))) return fail(st);
    }
    const float *w, *b;
    if ((st = get("linw", (int64_t)C * F * D, false, &w))) return fail(st);
    if ((st = get("linb", D, false, &b))) return fail(st);
    // rows permuted from the reference's c*F+f to the channels-last f*C+c,
    // each duplicated for the hi/lo activation pairs: k' = 2*(f*C+c) + {0,1}
    std::vector<float> bt((size_t)D * 2 * C * F);
    for (int nn = 0; nn < D; nn++)
      for (int f = 0; f < F; f++)
        for (int ch = 0; ch < C; ch++) {
          const size_t k = (size_t)nn * 2 * C * F + 2 * (f * C + ch);
          bt[k] = bt[k + 1] = w[(size_t)(ch * F + f) * D + nn];
        }
    std::vector<float> bias(b, b + D), fold(D, 1.f);
    if ((st = build_lin(e, e->lin, bt, D, 2 * C * F, fold, &bias, "linw"))) return fail(st);
    e->format = saved;
  }
  // positional table pe(maxT) (raw-encoder.js:163-174), f32 on the device
  const int PR = 2 * max_T - 1;
  std::vector<float> pe((size_t)PR * D);
  {
    const double lg = std::log(10000.0) / D;
    for (int pi = 0; pi < PR; pi++) {
      const double pos = max_T - 1 - pi;
      for (int i = 0; i < D; i += 2) {
        const double dv = std::exp(i * -lg);
        pe[(size_t)pi * D + i] = (float)std::sin(pos * dv);
        pe[(size_t)pi * D + i + 1] = (float)std::cos(pos * dv);
      }
    }
  }
  float *pe_d = (float *)dev_alloc(ctx, pe.size() * 4);
  if (!pe_d) return fail(FA_E_OOM);
  (void)hipMemcpy(pe_d, pe.data(), pe.size() * 4, hipMemcpyHostToDevice);
  float *ptmp = (float *)dev_alloc(ctx, pe.size() * 4);
  if (!ptmp) {
    (void)hipFree(pe_d);
    return fail(FA_E_OOM);
  }
  // ── layers ──
  e->L.resize(c.layers);
  static const char *lnk[5] = {"lnff1", "lnatt", "lnconv", "lnff2", "lnout"};
  for (int li = 0; li < c.layers; li++) {
    auto g = [&](const char *s) { return "L" + std::to_string(li) + "_" + s; };
    auto &Ly = e->L[li];
    for (int j = 0; j < 5; j++) {
      const float *gw, *gb;
      if ((st = get(g(lnk[j]) + "_w", D, false, &gw)) || (st = get(g(lnk[j]) + "_b", D, false, &gb))) return fail(st);
      Ly.ln[j][0] = dupload(e, gw, D);
      Ly.ln[j][1] = dupload(e, gb, D);
    }
    {  // conv-module LayerNorm (streaming models; raw-encoder.js:361-364), when present
      const float *bw, *bb;
      if ((st = get(g("bnw"), D, true, &bw)) || (st = get(g("bnb"), D, true, &bb))) return fail(st);
      if ((bw == nullptr) != (bb == nullptr)) return fail(set_err(ctx, FA_E_INVALID, "encoder load: layer %d has only one of bnw / bnb", li));
      if (bw) {
        if (D % 256 || D > 2048) return fail(set_err(ctx, FA_E_UNSUPPORTED, "encoder load: conv-module LayerNorm needs D a multiple of 256 (<= 2048)"));
        Ly.cln[0] = dupload(e, bw, D);
        Ly.cln[1] = dupload(e, bb, D);
      }
    }
    auto kn_to_bt = [](const float *w, int K, int N) {
      std::vector<float> bt((size_t)N * K);
      for (int k = 0; k < K; k++)
        for (int nn = 0; nn < N; nn++) bt[(size_t)nn * K + k] = w[(size_t)k * N + nn];
      return bt;
    };
    auto optvec = [&](const char *k, int cnt, std::vector<float> &dst) -> int {
      const float *b;
      int s = get(g(k), cnt, true, &b);
      if (s) return s;
      if (b) dst.assign(b, b + cnt);
      return FA_OK;
    };
    // feed-forwards (W2 and b2 carry the macaron 0.5, raw-encoder.js:129-131)
    for (int ffi = 0; ffi < 2; ffi++) {
      const char *w1n = ffi ? "ff2w1" : "ff1w1", *w2n = ffi ? "ff2w2" : "ff1w2", *b1n = ffi ? "ff2b1" : "ff1b1", *b2n = ffi ? "ff2b2" : "ff1b2";
      const float *w1, *w2;
      if ((st = get(g(w1n), (int64_t)D * DFF, false, &w1)) || (st = get(g(w2n), (int64_t)DFF * D, false, &w2))) return fail(st);
      std::vector<float> b1, b2;
      if ((st = optvec(b1n, DFF, b1)) || (st = optvec(b2n, D, b2))) return fail(st);
      Lin &L1 = ffi ? Ly.ff2w1 : Ly.ff1w1, &L2 = ffi ? Ly.ff2w2 : Ly.ff1w2;
      if ((st = build_lin(e, L1, kn_to_bt(w1, D, DFF), DFF, D, std::vector<float>(DFF, 1.f), b1.empty() ? nullptr : &b1, w1n))) return fail(st);
      if ((st = build_lin(e, L2, kn_to_bt(w2, DFF, D), D, DFF, std::vector<float>(D, 0.5f), b2.empty() ? nullptr : &b2, w2n))) return fail(st);
    }
    // fused q|k|v, q (and its bias) carrying 1/sqrt(HD) (raw-encoder.js:133,138)
    {
      const float *wq, *wk, *wv;
      if ((st = get(g("q"), (int64_t)D * D, false, &wq)) || (st = get(g("k"), (int64_t)D * D, false, &wk)) || (st = get(g("v"), (int64_t)D * D, false, &wv)))
        return fail(st);
      std::vector<float> bt((size_t)3 * D * D), fold(3 * D, 1.f);
      const float *ws[3] = {wq, wk, wv};
      for (int part = 0; part < 3; part++)
        for (int k = 0; k < D; k++)
          for (int nn = 0; nn < D; nn++) bt[(size_t)(part * D + nn) * D + k] = ws[part][(size_t)k * D + nn];
      for (int nn = 0; nn < D; nn++) fold[nn] = (float)INV;
      std::vector<float> bq, bk, bv;
      if ((st = optvec("qb", D, bq)) || (st = optvec("kb", D, bk)) || (st = optvec("vb", D, bv))) return fail(st);
      std::vector<float> bias;
      if (!bq.empty() || !bk.empty() || !bv.empty()) {
        bias.assign(3 * D, 0.f);
        for (int nn = 0; nn < D; nn++) {
          if (!bq.empty()) bias[nn] = bq[nn];
          if (!bk.empty()) bias[D + nn] = bk[nn];
          if (!bv.empty()) bias[2 * D + nn] = bv[nn];
        }
      }
      if ((st = build_lin(e, Ly.qkv, bt, 3 * D, D, fold, bias.empty() ? nullptr : &bias, "qkv"))) return fail(st);
    }
    {
      const float *wo;
      if ((st = get(g("out"), (int64_t)D * D, false, &wo))) return fail(st);
      std::vector<float> bo;
      if ((st = optvec("outb", D, bo))) return fail(st);
      if ((st = build_lin(e, Ly.out, kn_to_bt(wo, D, D), D, D, std::vector<float>(D, 1.f), bo.empty() ? nullptr : &bo, "out"))) return fail(st);
    }
    // pos_bias_u/v · 1/sqrt(HD) (raw-encoder.js:124-125)
    {
      const float *pu, *pv;
      if ((st = get(g("pbu"), D, false, &pu)) || (st = get(g("pbv"), D, false, &pv))) return fail(st);
      std::vector<float> a(D), b(D);
      for (int i = 0; i < D; i++) {
        a[i] = (float)((double)pu[i] * INV);
        b[i] = (float)((double)pv[i] * INV);
      }
      Ly.pbu = dupload(e, a.data(), D);
      Ly.pbv = dupload(e, b.data(), D);
    }
    // conv module: pw1 columns permuted for the GLU epilogue (value c at
    // 16(c/8) + 4((c%8)/2) + c%2, gate c+D two columns later)
    {
      const float *w1, *w2, *dw, *dwb;
      if ((st = get(g("pw1"), (int64_t)2 * D * D, false, &w1)) || (st = get(g("pw2"), (int64_t)D * D, false, &w2)) ||
          (st = get(g("dw"), (int64_t)D * 9, false, &dw)) || (st = get(g("dwb"), D, false, &dwb)))
        return fail(st);
      std::vector<float> b1, b2;
      if ((st = optvec("pw1b", 2 * D, b1)) || (st = optvec("pw2b", D, b2))) return fail(st);
      std::vector<float> bt((size_t)2 * D * D), bp;
      if (!b1.empty()) bp.assign(2 * D, 0.f);
      for (int ch = 0; ch < D; ch++) {
        const int jv = 16 * (ch / 8) + 4 * ((ch % 8) / 2) + ch % 2, jg = jv + 2;
        std::memcpy(&bt[(size_t)jv * D], w1 + (size_t)ch * D, D * 4);
        std::memcpy(&bt[(size_t)jg * D], w1 + (size_t)(ch + D) * D, D * 4);
        if (!b1.empty()) {
          bp[jv] = b1[ch];
          bp[jg] = b1[ch + D];
        }
      }
      if ((st = build_lin(e, Ly.pw1, bt, 2 * D, D, std::vector<float>(2 * D, 1.f), bp.empty() ? nullptr : &bp, "pw1"))) return fail(st);
      std::vector<float> bt2(w2, w2 + (size_t)D * D);
      if ((st = build_lin(e, Ly.pw2, bt2, D, D, std::vector<float>(D, 1.f), b2.empty() ? nullptr : &b2, "pw2"))) return fail(st);
      std::vector<float> wt((size_t)9 * D);
      for (int ch = 0; ch < D; ch++)
        for (int k = 0; k < 9; k++) wt[(size_t)k * D + ch] = dw[ch * 9 + k];
      Ly.dww = dupload(e, wt.data(), wt.size());
      Ly.dwb = dupload(e, dwb, D);
    }
    // projected positional table P = pe · Wpos, cached for every T <= maxT
    // (the reference caches it per (layer, Tsub), raw-encoder.js:305-321)
    {
      const float *wp;
      if ((st = get(g("pos"), (int64_t)D * D, false, &wp))) return fail(st);
      std::vector<float> bt = kn_to_bt(wp, D, D);
      roundtrip_format(format, bt, D, D);
      std::vector<uint16_t> h((size_t)D * D);
      for (size_t i = 0; i < h.size(); i++) h[i] = h_f32_to_f16(bt[i]);
      void *wpd = dev_alloc(ctx, h.size() * 2);
      if (!wpd) return fail(FA_E_OOM);
      (void)hipMemcpy(wpd, h.data(), h.size() * 2, hipMemcpyHostToDevice);
      Ly.P = (_Float16 *)dev_alloc(ctx, (size_t)PR * D * 2);
      if (!Ly.P) return fail(FA_E_OOM);
      e->allocs.push_back(Ly.P);
      GemmArgs pa;
      pa.A = pe_d; pa.lda = D; pa.akind = A_F32;
      pa.B = wpd; pa.bkind = B_F16;
      pa.C = ptmp; pa.ldc = D;
      pa.M = PR; pa.N = D; pa.K = D;
      st = gemm_mfma(ctx, pa, "pos_table");
      if (!st) {
        hipLaunchKernelGGL(f32_to_f16_kernel, dim3(1024), dim3(256), 0, ctx->stream, ptmp, Ly.P, (long)PR * D);
        st = check_launch(ctx, "pos_table_f16");
      }
      (void)hipStreamSynchronize(ctx->stream);
      (void)hipFree(wpd);
      if (st) {
        (void)hipFree(pe_d);
        (void)hipFree(ptmp);
        return fail(st);
      }
    }
    for (auto &ln : Ly.ln)
      if (!ln[0] || !ln[1]) return fail(set_err(ctx, FA_E_OOM, "encoder load: layer %d", li));
  }
  (void)hipFree(pe_d);
  (void)hipFree(ptmp);
  if (!e->c0w || !e->c0b || !e->c1w || !e->c1b || !e->c3w || !e->c3b) return fail(set_err(ctx, FA_E_OOM, "encoder load: front end"));
  {  // default operand precision, every weight format (see fa_encoder_set_exact)
    const int nl = (int)e->L.size();
    int tail = format == FA_W_F16 ? kExactTail : kExactTailQuant;
    if (const char *et = getenv("FA_EXACT_TAIL")) tail = std::max(0, atoi(et));  // schedule sweeps
    for (int li = 0; li < nl; li++) {
      unsigned m = li >= nl - tail ? (format == FA_W_F16 ? kTailExact : kTailExactQuant) : kCheapExact;
      if (c.D % 256 || c.D > 2048) m &= ~(unsigned)FA_EXACT_LN_OUT;
      e->L[li].exact = m;
    }
  }
  *out = e;
  return FA_OK;
}

int fa_encoder_forward(fa_ctx *ctx, fa_encoder *e, fa_tensor mel, const int32_t *lens, int n, int layout, int layers_run, fa_tensor *out) {
  return encoder_forward_impl(ctx, e, mel, nullptr, 0, lens, n, layout, layers_run, out, "encoderForward");
}

int fa_encoder_forward_stream(fa_ctx *ctx, fa_encoder *e, fa_tensor feats, const int32_t *starts, const int32_t *lens, int n, int layout,
                              int layers_run, fa_tensor *out) {
  if (!starts) return set_err(ctx, FA_E_INVALID, "encoderForwardStream: no window starts");
  return encoder_forward_impl(ctx, e, feats, starts, 0, lens, n, layout, layers_run, out, "encoderForwardStream");
}

// Several batches of one feature stream, each exactly as fa_encoder_forward_stream
// computes it, with consecutive batches on two workspace lanes that run on
// streams of their own: while one batch's kernel tails and end-of-kernel
// write-backs drain, the other batch's kernels fill the idle CUs (measured
// two 16-window batches in 13.4 ms against 2 x 7.5 ms).  The lanes
// start after the work already queued on the context stream, and the context
// stream waits for both before anything queued after this call.
int fa_encoder_forward_stream_batches(fa_ctx *ctx, fa_encoder *e, fa_tensor feats, int nb, const int32_t *starts, const int32_t *lens,
                                      const int32_t *counts, int layout, int layers_run, fa_tensor *outs) {
  const char *who = "encoderForwardStreamBatches";
  if (!e || e->ctx != ctx) return set_err(ctx, FA_E_INVALID, "%s: encoder belongs to another context", who);
  if (nb <= 0 || !starts || !lens || !counts || !outs) return set_err(ctx, FA_E_INVALID, "%s: no batches", who);
  for (int b = 0; b < nb; b++) outs[b] = 0;
  for (int b = 0; b < nb; b++)
    if (counts[b] <= 0) return set_err(ctx, FA_E_INVALID, "%s: batch %d has %d windows", who, b, counts[b]);
  if (nb == 1) return encoder_forward_impl(ctx, e, feats, starts, 0, lens, counts[0], layout, layers_run, outs, who);
  for (int l = 0; l < e->nlanes; l++) {
    if (!e->lane_stream[l]) FA_HIP(ctx, hipStreamCreateWithFlags(&e->lane_stream[l], hipStreamNonBlocking));
    if (!e->lane_done[l]) FA_HIP(ctx, hipEventCreateWithFlags(&e->lane_done[l], hipEventDisableTiming));
  }
  if (!e->lanes_in) FA_HIP(ctx, hipEventCreateWithFlags(&e->lanes_in, hipEventDisableTiming));
  FA_HIP(ctx, hipEventRecord(e->lanes_in, ctx->stream));
  const hipStream_t home = ctx->stream;
  int st = FA_OK;
  bool used[fa_encoder::kLanes] = {};
  long off = 0;
  for (int b = 0; b < nb && st == FA_OK; b++) {
    const int l = b % e->nlanes;
    if (!used[l]) {
      st = hipStreamWaitEvent(e->lane_stream[l], e->lanes_in, 0) == hipSuccess ? FA_OK : set_err(ctx, FA_E_DEVICE, "%s: stream wait", who);
      used[l] = true;
    }
    if (st != FA_OK) break;
    // the batch's launches (and the tensors' pool bookkeeping) go to the lane's stream
    ctx->stream = e->lane_stream[l];
    e->lane = l;
    st = encoder_forward_impl(ctx, e, feats, starts + off, 0, lens + off, counts[b], layout, layers_run, &outs[b], who);
    e->lane = 0;
    ctx->stream = home;
    off += counts[b];
  }
  for (int l = 0; l < e->nlanes; l++)
    if (used[l]) {
      (void)hipEventRecord(e->lane_done[l], e->lane_stream[l]);
      (void)hipStreamWaitEvent(home, e->lane_done[l], 0);
    }
  if (st != FA_OK)  // no partial result: the batches already encoded are released
    for (int b = 0; b < nb; b++)
      if (outs[b]) {
        (void)fa_free_tensor(ctx, outs[b]);
        outs[b] = 0;
      }
  return st;
}

}  // extern "C"
