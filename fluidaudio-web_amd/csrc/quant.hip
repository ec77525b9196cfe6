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

// 16 output columns per workgroup; wave w takes the 64-k chunks w, w+4, ...
// All of a lane's weight loads (16 k of its column per chunk) are issued
// before any MFMA so the workgroup's whole weight slice is in flight at once;
// the activations are read straight from global (L1/L2: every workgroup reads
// the same M x K block) as MFMA A fragments, rows >= M being register zeros.
template <int FMT>
__device__ __forceinline__ void gemv_dequant(const GemvArgs &p, int n, int kb, const uint4 &u8, const uint2 &u4, h8 &b0, h8 &b1) {
  if constexpr (FMT == 1) {
    const uint32_t w[4] = {u8.x, u8.y, u8.z, u8.w};
#pragma unroll
    for (int e = 0; e < 8; e++) {
      b0[e] = (_Float16)(float)(int8_t)((w[e >> 2] >> (8 * (e & 3))) & 0xff);
      b1[e] = (_Float16)(float)(int8_t)((w[2 + (e >> 2)] >> (8 * (e & 3))) & 0xff);
    }
  } else {
    const int blk = kb >> 5, nblk = p.K >> 5;
    float s, zp = 8.f;
    if constexpr (FMT == 2) {
      s = (float)reinterpret_cast<const _Float16 *>(p.scales)[(size_t)n * nblk + blk];
    } else {
      s = reinterpret_cast<const float *>(p.scales)[(size_t)n * nblk + blk];
      const uint8_t zb = p.zp[(size_t)n * p.zpb + (blk >> 1)];
      zp = (float)((blk & 1) ? (zb >> 4) : (zb & 0xf));
    }
#pragma unroll
    for (int e = 0; e < 8; e++) {
      b0[e] = (_Float16)(((float)((u4.x >> (4 * e)) & 0xf) - zp) * s);
      b1[e] = (_Float16)(((float)((u4.y >> (4 * e)) & 0xf) - zp) * s);
    }
  }
}

__device__ __forceinline__ h8 gemv_a8(const float *a) {
  const float4 x = reinterpret_cast<const float4 *>(a)[0], y = reinterpret_cast<const float4 *>(a)[1];
  return h8{(_Float16)x.x, (_Float16)x.y, (_Float16)x.z, (_Float16)x.w, (_Float16)y.x, (_Float16)y.y, (_Float16)y.z, (_Float16)y.w};
}

template <int FMT>
__global__ __launch_bounds__(256) void gemv_mfma_kernel(GemvArgs p) {
  constexpr int CB = 4;  // chunks per wave held in flight together
  __shared__ f4 sPart[4][64];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int n0 = blockIdx.x * 16;
  const int c16 = lane & 15, g = lane >> 4;
  const int n = min(n0 + c16, p.N - 1);
  const bool arow = c16 < p.M;
  const float *arow_p = p.A + (size_t)min(c16, p.M - 1) * p.K;
  f4 acc = f4{0.f, 0.f, 0.f, 0.f};
  const int nch = p.K / 64;
  for (int c0 = wave; c0 < nch; c0 += 4 * CB) {
    uint4 w8[CB];
    uint2 w4[CB];
#pragma unroll
    for (int i = 0; i < CB; i++) {
      const int ch = c0 + 4 * i;
      if (ch < nch) {
        const int kb = ch * 64 + g * 16;
        if constexpr (FMT == 1)
          w8[i] = *reinterpret_cast<const uint4 *>(reinterpret_cast<const int8_t *>(p.W) + (size_t)n * p.K + kb);
        else
          w4[i] = *reinterpret_cast<const uint2 *>(reinterpret_cast<const uint8_t *>(p.W) + (size_t)n * (p.K >> 1) + (kb >> 1));
      }
    }
#pragma unroll
    for (int i = 0; i < CB; i++) {
      const int ch = c0 + 4 * i;
      if (ch < nch) {
        const int kb = ch * 64 + g * 16;
        h8 b0, b1;
        gemv_dequant<FMT>(p, n, kb, w8[i], w4[i], b0, b1);
        h8 a0 = h8{0, 0, 0, 0, 0, 0, 0, 0}, a1 = a0;
        if (arow) {
          a0 = gemv_a8(arow_p + kb);
          a1 = gemv_a8(arow_p + kb + 8);
        }
        acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(a0, b0, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(a1, b1, acc, 0, 0, 0);
      }
    }
  }
  sPart[wave][lane] = acc;
  __syncthreads();
  if (wave != 0) return;
  f4 t = sPart[0][lane];
#pragma unroll
  for (int w = 1; w < 4; w++) {
    const f4 o = sPart[w][lane];
    t[0] += o[0]; t[1] += o[1]; t[2] += o[2]; t[3] += o[3];
  }
  const int col = n0 + c16;
  if (col >= p.N) return;
  const float cs = FMT == 1 ? reinterpret_cast<const float *>(p.scales)[col] : 1.f;
  const float bv = p.bias ? p.bias[col] : 0.f;
#pragma unroll
  for (int r = 0; r < 4; r++) {
    const int m = g * 4 + r;
    if (m < p.M) p.Y[(size_t)m * p.N + col] = act_apply(t[r] * cs + bv, p.act);
  }
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

static int gemv_launch(fa_ctx *ctx, const GemvArgs &p, int fmt, const char *label) {
  if (p.M <= 0 || p.N <= 0) return FA_OK;
  const bool single = !(p.M > 16 && p.M <= 64 && p.K % 64 == 0);
  ProfScope ps(ctx, label, single);
  if (p.M <= 16 && p.K % 64 == 0) {
    const size_t shm = 0;
    const dim3 grid(cdiv(p.N, 16));
    if (fmt == 1)
      FA_LAUNCH(ps, gemv_mfma_kernel<1>, grid, dim3(256), shm, ctx->stream, p);
    else if (fmt == 2)
      FA_LAUNCH(ps, gemv_mfma_kernel<2>, grid, dim3(256), shm, ctx->stream, p);
    else
      FA_LAUNCH(ps, gemv_mfma_kernel<3>, grid, dim3(256), shm, ctx->stream, p);
  } else if (p.M <= 64 && p.K % 64 == 0) {
    // M in (16, 64]: run 16-row slabs
    for (int m0 = 0; m0 < p.M; m0 += 16) {
      GemvArgs q = p;
      q.A = p.A + (size_t)m0 * p.K;
      q.Y = p.Y + (size_t)m0 * p.N;
      q.M = p.M - m0 < 16 ? p.M - m0 : 16;
      const size_t shm = 0;
      if (fmt == 1)
        hipLaunchKernelGGL(gemv_mfma_kernel<1>, dim3(cdiv(p.N, 16)), dim3(256), shm, ctx->stream, q);
      else if (fmt == 2)
        hipLaunchKernelGGL(gemv_mfma_kernel<2>, dim3(cdiv(p.N, 16)), dim3(256), shm, ctx->stream, q);
      else
        hipLaunchKernelGGL(gemv_mfma_kernel<3>, dim3(cdiv(p.N, 16)), dim3(256), shm, ctx->stream, q);
    }
  } else {
    FA_LAUNCH(ps, gemv_naive_kernel, dim3(cdiv((long)p.M * p.N, 256)), dim3(256), 0, ctx->stream, p, fmt);
  }
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
  ra = get(ctx, a); rw = get(ctx, w); rs = get(ctx, scales);
  FA_TRY(gemv_quant_launch(ctx, (const float *)ra->ptr, rw->ptr, rs->ptr, format, M, N, K, (float *)ro->ptr, nullptr, 0, format == 1 ? "gemv_int8" : "gemv_int4"));
  *out = o;
  return FA_OK;
}
