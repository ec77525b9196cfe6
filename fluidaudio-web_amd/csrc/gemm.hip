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
// epilogue pairs column 16g+x (value) with 16g+8+x (gate) and writes channel
// 8g+x = value·σ(gate) (gate clamped to ±30 as tensor-ops.js:18).
#include "fa_internal.h"
#include "fa_device.h"
#include "gemm.h"

namespace fa {

// ── MFMA f16 GEMM ───────────────────────────────────────────────────────────
template <int AK>
__device__ __forceinline__ h8 load_a8(const GemmArgs &p, int row, int k) {
  if constexpr (AK == A_F16) {
    return *reinterpret_cast<const h8 *>(reinterpret_cast<const _Float16 *>(p.A) + (size_t)row * p.lda + k);
  } else {
    const float4 *src = reinterpret_cast<const float4 *>(reinterpret_cast<const float *>(p.A) + (size_t)row * p.lda + k);
    float4 x = src[0], y = src[1];
    h8 r;
    r[0] = (_Float16)x.x; r[1] = (_Float16)x.y; r[2] = (_Float16)x.z; r[3] = (_Float16)x.w;
    r[4] = (_Float16)y.x; r[5] = (_Float16)y.y; r[6] = (_Float16)y.z; r[7] = (_Float16)y.w;
    return r;
  }
}

template <int BKND>
__device__ __forceinline__ h8 load_b8(const GemmArgs &p, int n, int k) {
  if constexpr (BKND == B_F16) {
    return *reinterpret_cast<const h8 *>(reinterpret_cast<const _Float16 *>(p.B) + (size_t)n * p.K + k);
  } else if constexpr (BKND == B_I8) {
    uint2 u = *reinterpret_cast<const uint2 *>(reinterpret_cast<const int8_t *>(p.B) + (size_t)n * p.K + k);
    h8 r;
#pragma unroll
    for (int e = 0; e < 4; e++) {
      r[e] = (_Float16)(float)(int8_t)((u.x >> (8 * e)) & 0xff);
      r[4 + e] = (_Float16)(float)(int8_t)((u.y >> (8 * e)) & 0xff);
    }
    return r;
  } else {  // B_I4: [N][K/32][16 B], low nibble = even k
    const int nblk = p.K >> 5;
    const uint32_t u = *reinterpret_cast<const uint32_t *>(reinterpret_cast<const uint8_t *>(p.B) + (size_t)n * (p.K >> 1) + (k >> 1));
    const int blk = k >> 5;
    float s;
    if (p.bscale_f32)
      s = reinterpret_cast<const float *>(p.bscale)[(size_t)n * nblk + blk];
    else
      s = (float)reinterpret_cast<const _Float16 *>(p.bscale)[(size_t)n * nblk + blk];
    float zp = 8.f;
    if (p.bzp) {
      uint8_t zb = p.bzp[(size_t)n * p.zpb + (blk >> 1)];
      zp = (float)((blk & 1) ? (zb >> 4) : (zb & 0xf));
    }
    h8 r;
#pragma unroll
    for (int e = 0; e < 8; e++) r[e] = (_Float16)(((float)((u >> (4 * e)) & 0xf) - zp) * s);
    return r;
  }
}

template <int BM, int BN, int WM, int WN, int AK, int BKND>
__global__ __launch_bounds__(64 * WM * WN) void gemm_mfma_kernel(GemmArgs p) {
  constexpr int NT = 64 * WM * WN;
  constexpr int BK = 64, LS = BK + 8;  // LDS row stride in halfs (+8 breaks bank conflicts)
  constexpr int WTM = BM / WM, WTN = BN / WN;
  constexpr int TI = WTM / 16, TJ = WTN / 16;
  constexpr int CA = BM * 8 / NT, CB = BN * 8 / NT;
  static_assert(CA >= 1 && CB >= 1 && BM * 8 % NT == 0 && BN * 8 % NT == 0, "tile/thread mismatch");
  __shared__ __attribute__((aligned(16))) _Float16 sA[2][BM * LS];
  __shared__ __attribute__((aligned(16))) _Float16 sB[2][BN * LS];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;
  const int nTN = (p.N + BN - 1) / BN, nTM = (p.M + BM - 1) / BM;
  const int tile = xcd_remap(blockIdx.x, nTM * nTN);
  const int m0 = (tile / nTN) * BM, n0 = (tile % nTN) * BN;

  f4 acc[TI][TJ];
#pragma unroll
  for (int i = 0; i < TI; i++)
#pragma unroll
    for (int j = 0; j < TJ; j++) acc[i][j] = f4{0.f, 0.f, 0.f, 0.f};

  h8 ra[CA], rb[CB];
  auto gload = [&](int k0) {
#pragma unroll
    for (int c = 0; c < CA; c++) {
      const int idx = tid + c * NT, row = idx >> 3, kc = idx & 7;
      const int gr = min(m0 + row, p.M - 1);
      ra[c] = load_a8<AK>(p, gr, k0 + kc * 8);
    }
#pragma unroll
    for (int c = 0; c < CB; c++) {
      const int idx = tid + c * NT, row = idx >> 3, kc = idx & 7;
      const int gn = min(n0 + row, p.N - 1);
      rb[c] = load_b8<BKND>(p, gn, k0 + kc * 8);
    }
  };
  auto lstore = [&](int buf) {
#pragma unroll
    for (int c = 0; c < CA; c++) {
      const int idx = tid + c * NT, row = idx >> 3, kc = idx & 7;
      *reinterpret_cast<h8 *>(&sA[buf][row * LS + kc * 8]) = ra[c];
    }
#pragma unroll
    for (int c = 0; c < CB; c++) {
      const int idx = tid + c * NT, row = idx >> 3, kc = idx & 7;
      *reinterpret_cast<h8 *>(&sB[buf][row * LS + kc * 8]) = rb[c];
    }
  };

  const int nk = p.K / BK;
  gload(0);
  lstore(0);
  __syncthreads();
  const int arow = wm * WTM + (lane & 15), brow = wn * WTN + (lane & 15), kq = (lane >> 4) * 8;
  for (int kt = 0; kt < nk; kt++) {
    const int buf = kt & 1;
    if (kt + 1 < nk) gload((kt + 1) * BK);
#pragma unroll
    for (int s = 0; s < 2; s++) {
      h8 af[TI], bf[TJ];
#pragma unroll
      for (int i = 0; i < TI; i++) af[i] = *reinterpret_cast<const h8 *>(&sA[buf][(arow + i * 16) * LS + s * 32 + kq]);
#pragma unroll
      for (int j = 0; j < TJ; j++) bf[j] = *reinterpret_cast<const h8 *>(&sB[buf][(brow + j * 16) * LS + s * 32 + kq]);
#pragma unroll
      for (int i = 0; i < TI; i++)
#pragma unroll
        for (int j = 0; j < TJ; j++) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[i], bf[j], acc[i][j], 0, 0, 0);
    }
    if (kt + 1 < nk) lstore(buf ^ 1);
    __syncthreads();
  }

  // epilogue
  const int rbase = m0 + wm * WTM + (lane >> 4) * 4;
  const int cbase = n0 + wn * WTN;
#pragma unroll
  for (int j = 0; j < TJ; j++) {
    const int col = cbase + j * 16 + (lane & 15);
    const bool cok = col < p.N;
    const float cs = (p.colscale && cok) ? p.colscale[col] : 1.f;
    const float bv = (p.bias && cok) ? p.bias[col] : 0.f;
#pragma unroll
    for (int i = 0; i < TI; i++) {
#pragma unroll
      for (int r = 0; r < 4; r++) {
        const int row = rbase + i * 16 + r;
        float v = acc[i][j][r];
        if (p.colscale) v *= cs;
        v += bv;
        if (p.glu) {
          const float g = __shfl_xor(v, 8, 64);
          if ((lane & 8) == 0 && row < p.M && cok) {
            const int ch = ((cbase + j * 16) >> 1) + (lane & 7);
            const float o = v / (1.f + __expf(-fminf(fmaxf(g, -30.f), 30.f)));
            reinterpret_cast<_Float16 *>(p.C)[(size_t)row * p.ldc + ch] = (_Float16)o;
          }
          continue;
        }
        if (row >= p.M || !cok) continue;
        v = act_apply(v, p.act);
        if (p.add) v += p.add[(size_t)row * p.ldadd + col];
        if (p.out_f16)
          reinterpret_cast<_Float16 *>(p.C)[(size_t)row * p.ldc + col] = (_Float16)v;
        else
          reinterpret_cast<float *>(p.C)[(size_t)row * p.ldc + col] = v;
      }
    }
  }
}

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

// ── host dispatch ───────────────────────────────────────────────────────────
template <int BM, int BN, int WM, int WN, int AK, int BKND>
static int launch_cfg(fa_ctx *ctx, const GemmArgs &p, const char *label) {
  const unsigned tiles = cdiv(p.M, BM) * cdiv(p.N, BN);
  ProfScope ps(ctx, label);
  hipLaunchKernelGGL((gemm_mfma_kernel<BM, BN, WM, WN, AK, BKND>), dim3(tiles), dim3(64 * WM * WN), 0, ctx->stream, p);
  return check_launch(ctx, label);
}

template <int AK, int BKND>
static int launch_kind(fa_ctx *ctx, const GemmArgs &p, const char *label) {
  // Tile choice: keep >= ~1 tile per CU; wide tiles for big N.
  const long t128 = (long)cdiv(p.M, 128) * cdiv(p.N, 128);
  if (t128 >= ctx->num_cu) return launch_cfg<128, 128, 2, 2, AK, BKND>(ctx, p, label);
  return launch_cfg<64, 128, 2, 2, AK, BKND>(ctx, p, label);
}

int gemm_mfma(fa_ctx *ctx, const GemmArgs &p, const char *label) {
  if (p.M <= 0 || p.N <= 0) return FA_OK;
  if (p.K % 64 != 0) return set_err(ctx, FA_E_UNSUPPORTED, "%s: K=%d must be a multiple of 64", label, p.K);
  if (p.glu && (p.N % 16 != 0 || !p.out_f16)) return set_err(ctx, FA_E_UNSUPPORTED, "%s: GLU epilogue needs N%%16==0 and f16 out", label);
  if (p.akind == A_F16) {
    if (p.bkind == B_F16) return launch_kind<A_F16, B_F16>(ctx, p, label);
    if (p.bkind == B_I8) return launch_kind<A_F16, B_I8>(ctx, p, label);
    return launch_kind<A_F16, B_I4>(ctx, p, label);
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
    hipLaunchKernelGGL(gemm_f32_kernel, dim3(cdiv(M, 64) * cdiv(N, 64)), dim3(256), 0, ctx->stream, A, B, C, bias, add, M, N, K, act);
  } else {
    hipLaunchKernelGGL(gemm_naive_kernel, dim3(cdiv((long)M * N, 256)), dim3(256), 0, ctx->stream, A, (const void *)B, 0, C, bias, add, M, N,
                       K, act);
  }
  return check_launch(ctx, label);
}

int gemm_naive_f16(fa_ctx *ctx, const float *A, const void *Bkm, float *C, const float *bias, const float *add, int M, int N, int K, int act,
                   const char *label) {
  if (M <= 0 || N <= 0) return FA_OK;
  ProfScope ps(ctx, label);
  hipLaunchKernelGGL(gemm_naive_kernel, dim3(cdiv((long)M * N, 256)), dim3(256), 0, ctx->stream, A, Bkm, 1, C, bias, add, M, N, K, act);
  return check_launch(ctx, label);
}

}  // namespace fa
