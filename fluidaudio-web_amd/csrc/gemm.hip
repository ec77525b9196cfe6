// GEMMs on gfx950 matrix cores.
//
//  gemm_mfma   C[M,N] = epi(A[M,K] · B[K,N]) with B stored K-major (Bᵀ [N][K])
//              as f16, int8 (per-column scale) or int4 group-32; A is f16 or
//              f32 (rounded to f16 on load, as the reference's f16-compute
//              kernel rounds A into workgroup memory, gemm.js:336-410).
//              v_mfma_f32_16x16x32_f16 tiles, f32 accumulation, LDS
//              double-buffering with register prefetch of the next K tile, and
//              weight dequant fused into the global->LDS staging.
//  gemm_f32    fp32 GEMM (v_mfma_f32_16x16x4_f32) for f32 B: the fp32 path.
//  gemm_naive  any-shape fallback (one thread per output).
//
// Epilogue order matches the reference kernels: × per-column scale (int8,
// gemm.js:704-706) → + bias → act → + residual (gemm.js:398-404).  The GLU
// epilogue pairs column 4g+x (value) with 4g+2+x (gate), x = 0, 1, and writes
// channel 2g+x = value·σ(gate) (gate clamped to ±30 as tensor-ops.js:18).
#include "gemm_impl.h"

#include <cstdio>
#include <cstdlib>

namespace fa {

// ── fp32 MFMA GEMM: B f32 row-major [K,N] ───────────────────────────────────
// 64x64 tile, 4 waves (2x2), BK 16, v_mfma_f32_16x16x4_f32.
__global__ __launch_bounds__(256) void gemm_f32_kernel(const float *__restrict__ A, const float *__restrict__ B, float *C, const float *bias,
                                                       const float *add, int M, int N, int K, int act) {
  constexpr int BM = 64, BN = 64, BK = 16;
  __shared__ float sA[BK][BM + 4];
  __shared__ float sB[BK][BN + 4];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, wm = wave >> 1, wn = wave & 1;
  const int nTN = (N + BN - 1) / BN, nTM = (M + BM - 1) / BM;
  const int tile = xcd_remap(blockIdx.x, nTM * nTN);
  const int m0 = (tile / nTN) * BM, n0 = (tile % nTN) * BN;
  f4 acc[2][2];
  for (int i = 0; i < 2; i++)
    for (int j = 0; j < 2; j++) acc[i][j] = f4{0.f, 0.f, 0.f, 0.f};
  for (int k0 = 0; k0 < K; k0 += BK) {
    {  // A tile [64 rows][16 k] -> sA[k][m]
      const int row = tid >> 2, kq = (tid & 3) * 4;
      const int gr = min(m0 + row, M - 1);
      float4 v = *reinterpret_cast<const float4 *>(A + (size_t)gr * K + k0 + kq);
      sA[kq + 0][row] = v.x; sA[kq + 1][row] = v.y; sA[kq + 2][row] = v.z; sA[kq + 3][row] = v.w;
    }
    {  // B tile [16 k][64 n]
      const int kr = tid >> 4, nq = (tid & 15) * 4;
      float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
      if (n0 + nq < N) v = *reinterpret_cast<const float4 *>(B + (size_t)(k0 + kr) * N + n0 + nq);
      sB[kr][nq + 0] = v.x; sB[kr][nq + 1] = v.y; sB[kr][nq + 2] = v.z; sB[kr][nq + 3] = v.w;
    }
    __syncthreads();
#pragma unroll
    for (int ks = 0; ks < BK; ks += 4) {
      float a0 = sA[ks + (lane >> 4)][wm * 32 + (lane & 15)];
      float a1 = sA[ks + (lane >> 4)][wm * 32 + 16 + (lane & 15)];
      float b0 = sB[ks + (lane >> 4)][wn * 32 + (lane & 15)];
      float b1 = sB[ks + (lane >> 4)][wn * 32 + 16 + (lane & 15)];
      acc[0][0] = __builtin_amdgcn_mfma_f32_16x16x4f32(a0, b0, acc[0][0], 0, 0, 0);
      acc[0][1] = __builtin_amdgcn_mfma_f32_16x16x4f32(a0, b1, acc[0][1], 0, 0, 0);
      acc[1][0] = __builtin_amdgcn_mfma_f32_16x16x4f32(a1, b0, acc[1][0], 0, 0, 0);
      acc[1][1] = __builtin_amdgcn_mfma_f32_16x16x4f32(a1, b1, acc[1][1], 0, 0, 0);
    }
    __syncthreads();
  }
  for (int i = 0; i < 2; i++)
    for (int j = 0; j < 2; j++) {
      const int col = n0 + wn * 32 + j * 16 + (lane & 15);
      for (int r = 0; r < 4; r++) {
        const int row = m0 + wm * 32 + i * 16 + (lane >> 4) * 4 + r;
        if (row >= M || col >= N) continue;
        float v = acc[i][j][r];
        if (bias) v += bias[col];
        v = act_apply(v, act);
        if (add) v += add[(size_t)row * N + col];
        C[(size_t)row * N + col] = v;
      }
    }
}

// ── any-shape fallback ──────────────────────────────────────────────────────
// b_kind 0: f32 row-major [K,N]; 1: f16 K-major (A rounded to f16, f32 sums).
__global__ void gemm_naive_kernel(const float *A, const void *B, int b_kind, float *C, const float *bias, const float *add, int M, int N, int K,
                                  int act) {
  const long idx = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= (long)M * N) return;
  const int row = (int)(idx / N), col = (int)(idx % N);
  float acc = 0.f;
  if (b_kind == 0) {
    const float *Bf = (const float *)B;
    for (int k = 0; k < K; k++) acc += A[(size_t)row * K + k] * Bf[(size_t)k * N + col];
  } else {
    const _Float16 *Bh = (const _Float16 *)B;
    for (int k = 0; k < K; k++) acc += (float)(_Float16)A[(size_t)row * K + k] * (float)Bh[(size_t)col * K + k];
  }
  if (bias) acc += bias[col];
  acc = act_apply(acc, act);
  if (add) acc += add[(size_t)row * N + col];
  C[(size_t)row * N + col] = acc;
}

int gemm_takes_direct(fa_ctx *ctx, const GemmArgs &p) {
  if (p.akind != A_F16 || epi_of(p) == EPI_GENERIC || pick_dma(ctx, p) < 0) return 0;
  if (p.bkind == B_F16) return 1;
  if (p.bkind == B_I8) return 1;
  if (p.bkind == B_I4) return !p.bzp && !p.bscale_f32;
  return 0;
}

int gemm_mfma(fa_ctx *ctx, const GemmArgs &p, const char *label) {
  if (p.vt && (epi_of(p) != EPI_F16 || !gemm_takes_direct(ctx, p)))
    return set_err(ctx, FA_E_UNSUPPORTED, "%s: transposed-V output needs the f16 epilogue of the direct-to-LDS route", label);
  if (p.M <= 0 || p.N <= 0) return FA_OK;
  if (p.K % 64 != 0) return set_err(ctx, FA_E_UNSUPPORTED, "%s: K=%d must be a multiple of 64", label, p.K);
  if (p.glu && p.N % 16 != 0) return set_err(ctx, FA_E_UNSUPPORTED, "%s: GLU epilogue needs N%%16==0", label);
  if ((p.Alo || p.Clo) && (p.akind != A_F16 || (p.Clo && !p.out_f16)))
    return set_err(ctx, FA_E_UNSUPPORTED, "%s: hi/lo planes are for f16 A with f16 output", label);
  if (p.Alo && !gemm_takes_direct(ctx, p))
    return set_err(ctx, FA_E_UNSUPPORTED, "%s: an exact lo plane needs the direct-to-LDS route (N %% 128, K %% 64, 16-byte alignment)", label);
  if (p.hilo && (p.glu || p.act != 0 || p.add || p.akind != A_F16 || p.bkind != B_F16))
    return set_err(ctx, FA_E_UNSUPPORTED, "%s: hi/lo epilogue is the f16 x f16 route's ReLU output only", label);
  if (p.akind == A_F16) {
    if (p.bkind == B_F16) return launch_kind<A_F16, B_F16>(ctx, p, label);
    if (p.bkind == B_I8) return gemm_launch_f16a_i8(ctx, p, label);
    return gemm_launch_f16a_i4(ctx, p, label);
  }
  if (p.bkind == B_F16) return launch_kind<A_F32, B_F16>(ctx, p, label);
  if (p.bkind == B_I8) return launch_kind<A_F32, B_I8>(ctx, p, label);
  return launch_kind<A_F32, B_I4>(ctx, p, label);
}

int gemm_f32(fa_ctx *ctx, const float *A, const float *B, float *C, const float *bias, const float *add, int M, int N, int K, int act,
             const char *label) {
  if (M <= 0 || N <= 0) return FA_OK;
  ProfScope ps(ctx, label);
  if (K % 16 == 0 && N % 4 == 0) {
    FA_LAUNCH(ps, gemm_f32_kernel, dim3(cdiv(M, 64) * cdiv(N, 64)), dim3(256), 0, ctx->stream, A, B, C, bias, add, M, N, K, act);
  } else {
    FA_LAUNCH(ps, gemm_naive_kernel, dim3(cdiv((long)M * N, 256)), dim3(256), 0, ctx->stream, A, (const void *)B, 0, C, bias, add, M, N,
                       K, act);
  }
  return check_launch(ctx, label);
}

int gemm_naive_f16(fa_ctx *ctx, const float *A, const void *Bkm, float *C, const float *bias, const float *add, int M, int N, int K, int act,
                   const char *label) {
  if (M <= 0 || N <= 0) return FA_OK;
  ProfScope ps(ctx, label);
  FA_LAUNCH(ps, gemm_naive_kernel, dim3(cdiv((long)M * N, 256)), dim3(256), 0, ctx->stream, A, Bkm, 1, C, bias, add, M, N, K, act);
  return check_launch(ctx, label);
}

}  // namespace fa
