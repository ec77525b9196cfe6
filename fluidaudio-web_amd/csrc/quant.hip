// Skinny weight-only quantised GEMMs (M <= 64): y[M,N] = a[M,K] · dequant(W).
//
// These are HBM-bound: every weight byte is read once and the arithmetic is
// tiny, so the kernel is organised around the weight stream.  A block (4
// waves) owns 16 output columns; the K range is split across its waves and
// each wave streams 64-k chunks of its 16 weight rows (K-major storage: a
// column's weights are contiguous), dequantises them in registers and feeds a
// v_mfma_f32_16x16x32_f16 whose A fragments are the activations read straight
// from global as f16 (rows >= M are zero).  MFMA keeps the M=16 case off the VALU; for M=1/4 the
// unused MFMA rows are free next to the memory time.  Partial tiles are
// summed through LDS, then scale/bias/act are applied.
//
// Formats:
//   1  int8 per-output-column (quantize-parakeet-encoder.py:31-36), K-major
//      [N][K]; products exact in f16, scale applied to the f32 sum as the
//      reference's int8 kernels do (gemm.js:704-706, lib.rs:158);
//   2  int4 symmetric group-32, [N][K/32][16 B] (MatMulNBits layout,
//      lib.rs:164-203, zero point 8), f16 scales [N][K/32];
//   3  ONNX MatMulNBits (asymmetric): f32 scales [N][nblk], packed int4 zero
//      points [N][zpb] (gemm.js:893-919).
// For int4 each weight is dequantised ((q-zp)·s) and rounded to f16 before
// the MFMA.
#include "fa_internal.h"
#include "fa_device.h"
#include "ops.h"

namespace fa {

struct GemvArgs {
  const float *A;
  int M, K, N;
  const void *W;
  const void *scales;
  const uint8_t *zp;
  int zpb;
  float *Y;
  const float *bias;
  int act;
};

// Workgroup = NWB x KS waves: NWB column groups of 16 output columns, each
// K range split over KS waves (partial sums reduced through LDS).  The
// activations (M <= 16 rows) are staged once per workgroup in LDS as f16
// ([16][K + 8]), so every MFMA A fragment is one
// ds_read_b128.  Lane (g, c16) of a wave streams 64 contiguous weight bytes
// of its column per chunk together with the other three lanes of the
// column: int8 16 B = 16 k (chunk = 64 k), int4 16 B = 32 k, one group-32
// block with one scale (chunk = 128 k).  The k order inside a chunk is
// permuted identically for weights and activations (lane g's k values feed
// MFMA k slots g*8 .. g*8 + 7 of successive MFMAs).  Chunks go in groups of
// CB whose loads are all issued before the group's first MFMA (the first
// group's while the activations are staged).  Dequantisation is exact and
// the same as the GEMM route's (i8x8_to_h8, i4x8_to_h8: (q - 8)·s rounded
// once to f16); the int8 column scale is applied to the f32 sum.
template <int FMT, int NWB, int KS>
__device__ __forceinline__ void gemv_tile(const GemvArgs &p, int n0, _Float16 *sA) {
  constexpr int CB = FMT == 1 ? 16 : 8;   // chunks per load group
  constexpr int CK = FMT == 1 ? 64 : 128;  // k per chunk
  constexpr int NM = FMT == 1 ? 2 : 4;     // MFMAs per chunk
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, wc = wave % NWB, wk = wave / NWB;
  const int c16 = lane & 15, g = lane >> 4;
  const int K = p.K, KP = K + 8, nch = K / CK, nblk = K >> 5;
  const int cb = wk * nch / KS, ce = (wk + 1) * nch / KS;  // this wave's chunks
  const int n = min(n0 + wc * 16 + c16, p.N - 1);
  const uint8_t *Wc = reinterpret_cast<const uint8_t *>(p.W) + (size_t)n * (FMT == 1 ? K : K >> 1) + g * 16;
  const _Float16 *S4 = reinterpret_cast<const _Float16 *>(p.scales) + (size_t)n * nblk + g;
  uint4 w[CB];
  _Float16 s4[CB];
  auto load = [&](int c0) {
#pragma unroll
    for (int i = 0; i < CB; i++) {
      const int ch = min(c0 + i, ce - 1);  // past the range: a repeat, never used
      w[i] = *reinterpret_cast<const uint4 *>(Wc + ch * 64);
      if constexpr (FMT == 2) s4[i] = S4[ch * 4];
    }
  };
  if (cb < ce) load(cb);  // the first group's weights stream while the activations are staged
  // f32 [M][K] -> f16 rows of [16][KP]; rows >= M stay unwritten: they only
  // feed MFMA output rows >= M, which are never stored
  for (int idx = tid; idx < p.M * (K / 4); idx += 64 * NWB * KS) {
    const int r = idx / (K / 4), c = (idx - r * (K / 4)) * 4;
    const float4 v = *reinterpret_cast<const float4 *>(p.A + (size_t)r * K + c);
    *reinterpret_cast<h4 *>(sA + r * KP + c) = h4{(_Float16)v.x, (_Float16)v.y, (_Float16)v.z, (_Float16)v.w};
  }
  __syncthreads();
  f4 acc = f4{0.f, 0.f, 0.f, 0.f};
  const _Float16 *arow = sA + c16 * KP + g * (CK / 4);
  for (int c0 = cb; c0 < ce; c0 += CB) {
    if (c0 > cb) load(c0);
#pragma unroll
    for (int i = 0; i < CB; i++) {
      const int ch = c0 + i;
      if (ch < ce) {
        const uint32_t u[4] = {w[i].x, w[i].y, w[i].z, w[i].w};
#pragma unroll
        for (int j = 0; j < NM; j++) {
          const h8 b = FMT == 1 ? i8x8_to_h8(uint2{u[2 * j], u[2 * j + 1]}) : i4x8_to_h8(u[j], s4[i]);
          const h8 a = *reinterpret_cast<const h8 *>(arow + ch * CK + j * 8);
          acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, acc, 0, 0, 0);
        }
      }
    }
  }
  if constexpr (KS > 1) {  // partial sums of the K splits -> wave row wk = 0
    f4 *part = reinterpret_cast<f4 *>(sA + 16 * KP);
    if (wk > 0) part[((wk - 1) * NWB + wc) * 64 + lane] = acc;
    __syncthreads();
    if (wk > 0) return;
#pragma unroll
    for (int k = 1; k < KS; k++) {
      const f4 o = part[((k - 1) * NWB + wc) * 64 + lane];
      acc[0] += o[0]; acc[1] += o[1]; acc[2] += o[2]; acc[3] += o[3];
    }
  }
  const int col = n0 + wc * 16 + c16;
  if (col >= p.N) return;
  const float cs = FMT == 1 ? reinterpret_cast<const float *>(p.scales)[col] : 1.f;
  const float bv = p.bias ? p.bias[col] : 0.f;
#pragma unroll
  for (int r = 0; r < 4; r++) {
    const int m = g * 4 + r;
    if (m < p.M) p.Y[(size_t)m * p.N + col] = act_apply(acc[r] * cs + bv, p.act);
  }
}

// one product: 16 columns per workgroup, K split over 4 waves (N / 16
// workgroups fill the chip for the encoder's widths)
template <int FMT>
__global__ __launch_bounds__(256) void gemv_mfma_kernel(GemvArgs p) {
  extern __shared__ __attribute__((aligned(16))) _Float16 gemv_sA[];
  gemv_tile<FMT, 1, 4>(p, blockIdx.x * 16, gemv_sA);
}

constexpr int kGemvWaves = 8;  // batched: 128 columns per workgroup, whole K per wave
// Many independent products of one shape in one launch (blockIdx.y = item):
// the weight streams of all items are in flight together, so the launch runs
// at the HBM rate instead of one small matrix's latency.
constexpr int kGemvBatchItems = 48;
struct GemvItem {
  const float *A;
  const void *W;
  const void *scales;
  float *Y;
};
struct GemvBatch {
  GemvItem it[kGemvBatchItems];
};
template <int FMT>
__global__ __launch_bounds__(64 * kGemvWaves) void gemv_batch_kernel(GemvArgs base, GemvBatch b) {
  extern __shared__ __attribute__((aligned(16))) _Float16 gemv_sA[];
  const GemvItem &it = b.it[blockIdx.y];
  GemvArgs p = base;
  p.A = it.A;
  p.W = it.W;
  p.scales = it.scales;
  p.Y = it.Y;
  gemv_tile<FMT, kGemvWaves, 1>(p, blockIdx.x * 16 * kGemvWaves, gemv_sA);
}

// any-shape fallback: one thread per output, f32 math
__global__ void gemv_naive_kernel(GemvArgs p, int fmt) {
  const long idx = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= (long)p.M * p.N) return;
  const int m = (int)(idx / p.N), n = (int)(idx % p.N);
  const float *a = p.A + (size_t)m * p.K;
  float acc = 0.f;
  if (fmt == 1) {
    const int8_t *w = reinterpret_cast<const int8_t *>(p.W) + (size_t)n * p.K;
    for (int k = 0; k < p.K; k++) acc += a[k] * (float)w[k];
    acc *= reinterpret_cast<const float *>(p.scales)[n];
  } else {
    const int nblk = (p.K + 31) / 32;
    const uint8_t *w = reinterpret_cast<const uint8_t *>(p.W) + (size_t)n * nblk * 16;
    for (int k = 0; k < p.K; k++) {
      const int b = k >> 5, t = k & 31;
      const uint8_t byte = w[b * 16 + (t >> 1)];
      const float q = (float)((t & 1) ? (byte >> 4) : (byte & 0xf));
      float s, zp = 8.f;
      if (fmt == 2) {
        s = (float)reinterpret_cast<const _Float16 *>(p.scales)[(size_t)n * nblk + b];
      } else {
        s = reinterpret_cast<const float *>(p.scales)[(size_t)n * nblk + b];
        const uint8_t zb = p.zp[(size_t)n * p.zpb + (b >> 1)];
        zp = (float)((b & 1) ? (zb >> 4) : (zb & 0xf));
      }
      acc += a[k] * ((q - zp) * s);
    }
  }
  if (p.bias) acc += p.bias[n];
  p.Y[idx] = act_apply(acc, p.act);
}

static inline bool gemv_mfma_ok(int fmt, int M, int K) { return (fmt == 1 || fmt == 2) && M <= 64 && K % 128 == 0 && K <= 4096; }
static inline size_t gemv_lds(int K) { return (size_t)16 * (K + 8) * 2 + 3 * 64 * 16; }  // + the K-split partial sums
// the staged activations take up to 16 x 4104 halfs (131 KB) of dynamic LDS,
// beyond the default 64 KB launch limit: raise it once per process
static int gemv_prepare(fa_ctx *ctx) {
  static int st = -1;
  if (st < 0) {
    const int lim = 160 * 1024;
    st = (hipFuncSetAttribute((const void *)gemv_mfma_kernel<1>, hipFuncAttributeMaxDynamicSharedMemorySize, lim) == hipSuccess &&
          hipFuncSetAttribute((const void *)gemv_mfma_kernel<2>, hipFuncAttributeMaxDynamicSharedMemorySize, lim) == hipSuccess &&
          hipFuncSetAttribute((const void *)gemv_batch_kernel<1>, hipFuncAttributeMaxDynamicSharedMemorySize, lim) == hipSuccess &&
          hipFuncSetAttribute((const void *)gemv_batch_kernel<2>, hipFuncAttributeMaxDynamicSharedMemorySize, lim) == hipSuccess)
             ? 1
             : 0;
  }
  return st ? FA_OK : set_err(ctx, FA_E_DEVICE, "gemv: raising the dynamic LDS limit failed");
}

static int gemv_launch(fa_ctx *ctx, const GemvArgs &p, int fmt, const char *label) {
  if (p.M <= 0 || p.N <= 0) return FA_OK;
  if (gemv_mfma_ok(fmt, p.M, p.K)) {
    FA_TRY(gemv_prepare(ctx));
    // 16-row slabs (one launch for M <= 16)
    const dim3 grid(cdiv(p.N, 16));
    for (int m0 = 0; m0 < p.M; m0 += 16) {
      GemvArgs q = p;
      q.A = p.A + (size_t)m0 * p.K;
      q.Y = p.Y + (size_t)m0 * p.N;
      q.M = p.M - m0 < 16 ? p.M - m0 : 16;
      ProfScope ps(ctx, label, true);
      if (fmt == 1)
        FA_LAUNCH(ps, gemv_mfma_kernel<1>, grid, dim3(256), gemv_lds(p.K), ctx->stream, q);
      else
        FA_LAUNCH(ps, gemv_mfma_kernel<2>, grid, dim3(256), gemv_lds(p.K), ctx->stream, q);
      FA_TRY(check_launch(ctx, label));
    }
    return FA_OK;
  }
  ProfScope ps(ctx, label, true);
  FA_LAUNCH(ps, gemv_naive_kernel, dim3(cdiv((long)p.M * p.N, 256)), dim3(256), 0, ctx->stream, p, fmt);
  return check_launch(ctx, label);
}

int gemv_quant_launch(fa_ctx *ctx, const float *A, const void *W, const void *scales, int format, int M, int N, int K, float *Y, const float *bias,
                      int act, const char *label) {
  GemvArgs p{A, M, K, N, W, scales, nullptr, 0, Y, bias, act};
  if (format == 2 && K % 32 != 0) return set_err(ctx, FA_E_UNSUPPORTED, "%s: int4 group-32 needs K %% 32 == 0", label);
  return gemv_launch(ctx, p, format, label);
}


}  // namespace fa

using namespace fa;

extern "C" int fa_gemv_quant(fa_ctx *ctx, fa_tensor a, fa_tensor w, fa_tensor scales, int format, int N, int K, fa_tensor *out) {
  TensorRec *ra, *rw, *rs;
  FA_TRY(need(ctx, a, &ra, "gemvQuant a"));
  FA_TRY(need(ctx, w, &rw, "gemvQuant w"));
  FA_TRY(need(ctx, scales, &rs, "gemvQuant scales"));
  if (ra->kind != S_F32 || ra->cols != K) return set_err(ctx, FA_E_INVALID, "gemvQuant: a must be f32 [M,%d]", K);
  if (format != 1 && format != 2) return set_err(ctx, FA_E_INVALID, "gemvQuant: format %d", format);
  const size_t wbytes = format == 1 ? (size_t)N * K : (size_t)N * ((K + 31) / 32) * 16;
  if (rw->bytes < wbytes) return set_err(ctx, FA_E_INVALID, "gemvQuant: weight buffer has %zu bytes, need %zu", rw->bytes, wbytes);
  const int M = ra->rows;
  if (M > 64) return set_err(ctx, FA_E_UNSUPPORTED, "gemvQuant: M=%d > 64 (use the encoder GEMMs)", M);
  fa_tensor o;
  TensorRec *ro;
  FA_TRY(new_tensor(ctx, M, N, S_F32, (size_t)M * N * 4, &o, &ro));
  TensorGuard og(ctx, o);  // released unless the op completes
  ra = get(ctx, a); rw = get(ctx, w); rs = get(ctx, scales);
  FA_TRY(gemv_quant_launch(ctx, (const float *)ra->ptr, rw->ptr, rs->ptr, format, M, N, K, (float *)ro->ptr, nullptr, 0, format == 1 ? "gemv_int8" : "gemv_int4"));
  *out = og.release();
  return FA_OK;
}

extern "C" int fa_gemv_quant_batch(fa_ctx *ctx, int count, const fa_tensor *a, const fa_tensor *w, const fa_tensor *scales, int format, int N, int K,
                                   fa_tensor *out) {
  if (!ctx || !out || count <= 0 || !a || !w || !scales) return ctx ? set_err(ctx, FA_E_INVALID, "gemvQuantBatch: %d items", count) : FA_E_INVALID;
  if (format != 1 && format != 2) return set_err(ctx, FA_E_INVALID, "gemvQuantBatch: format %d", format);
  if (K % 128 != 0 || K > 4096 || N <= 0) return set_err(ctx, FA_E_UNSUPPORTED, "gemvQuantBatch: K=%d must be a multiple of 128, <= 4096", K);
  const size_t wbytes = format == 1 ? (size_t)N * K : (size_t)N * (K / 32) * 16;
  const size_t sbytes = format == 1 ? (size_t)N * 4 : (size_t)N * (K / 32) * 2;
  int M = -1;
  for (int i = 0; i < count; i++) {
    TensorRec *ra, *rw, *rs;
    FA_TRY(need(ctx, a[i], &ra, "gemvQuantBatch a"));
    FA_TRY(need(ctx, w[i], &rw, "gemvQuantBatch w"));
    FA_TRY(need(ctx, scales[i], &rs, "gemvQuantBatch scales"));
    if (ra->kind != S_F32 || ra->cols != K || (M >= 0 && ra->rows != M))
      return set_err(ctx, FA_E_INVALID, "gemvQuantBatch: item %d: a must be f32 [M,%d] with one M for all items", i, K);
    M = ra->rows;
    if (rw->bytes < wbytes || rs->bytes < sbytes) return set_err(ctx, FA_E_INVALID, "gemvQuantBatch: item %d: weight / scale buffer too small", i);
  }
  if (M < 1 || M > 16) return set_err(ctx, FA_E_UNSUPPORTED, "gemvQuantBatch: M=%d (1..16)", M);
  FA_TRY(gemv_prepare(ctx));
  fa_tensor o;
  TensorRec *ro;
  FA_TRY(new_tensor(ctx, count * M, N, S_F32, (size_t)count * M * N * 4, &o, &ro));
  TensorGuard og(ctx, o);  // released unless the op completes
  float *Y = (float *)ro->ptr;
  GemvArgs base{nullptr, M, K, N, nullptr, nullptr, nullptr, 0, nullptr, nullptr, 0};
  const char *label = format == 1 ? "gemv_batch_int8" : "gemv_batch_int4";
  for (int i0 = 0; i0 < count; i0 += kGemvBatchItems) {
    const int nb = std::min(kGemvBatchItems, count - i0);
    GemvBatch b{};
    for (int j = 0; j < nb; j++) {
      const int i = i0 + j;
      b.it[j] = {(const float *)get(ctx, a[i])->ptr, get(ctx, w[i])->ptr, get(ctx, scales[i])->ptr, Y + (size_t)i * M * N};
    }
    ProfScope ps(ctx, label);
    const dim3 grid(cdiv(N, 16 * kGemvWaves), nb);
    if (format == 1)
      FA_LAUNCH(ps, gemv_batch_kernel<1>, grid, dim3(64 * kGemvWaves), gemv_lds(K), ctx->stream, base, b);
    else
      FA_LAUNCH(ps, gemv_batch_kernel<2>, grid, dim3(64 * kGemvWaves), gemv_lds(K), ctx->stream, base, b);
    FA_TRY(check_launch(ctx, label));
  }
  *out = og.release();
  return FA_OK;
}
