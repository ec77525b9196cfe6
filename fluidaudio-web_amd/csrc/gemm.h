// GEMM launch interface shared by the C-ABI ops and the fused encoder.
#pragma once
#include <stdint.h>

struct fa_ctx;

namespace fa {

enum AKind : int { A_F16 = 0, A_F32 = 1 };
enum BKind : int { B_F16 = 0, B_I8 = 1, B_I4 = 2 };

// split-K factor of the skinny route for N <= kSkinnySplitMaxN, and its workspace for N
// columns (two 16-row tiles at most: 64 lanes x 16 bytes per tile)
constexpr int kSkinnySplit = 4, kSkinnySplitMaxN = 2048;
inline size_t skinny_split_bytes(int N) { return (size_t)kSkinnySplit * (N / 16) * 2 * 64 * 16; }

struct GemmArgs {
  const void *A = nullptr;  // [M, lda] row-major, f16 or f32
  const void *Alo = nullptr;  // optional f16 plane [M, lda]: A = A + Alo exactly (f16 x f16 route only)
  int lda = 0;
  int akind = A_F16;
  const void *B = nullptr;  // K-major: f16 [N][K] | int8 [N][K] | int4 [N][K/32][16 B]
  int bkind = B_F16;
  const void *bscale = nullptr;  // int4 scales [N][K/32]: f16 bits, or f32 when bscale_f32
  int bscale_f32 = 0;
  const uint8_t *bzp = nullptr;  // int4 zero points, packed [N][zpb] (null: 8)
  int zpb = 0;
  void *C = nullptr;  // [M, ldc], f32 or f16 (out_f16)
  void *Clo = nullptr;  // EPI f16 outputs only: also write lo = f16(v - f16(v)) here ([M, ldc])
  int ldc = 0;
  int out_f16 = 0;
  const float *colscale = nullptr;  // int8 per-output-column scale
  // the skinny route (<= 32 rows: K split over waves, so its sums are ordered
  // differently from the tiled kernels'); set by the streaming passes only, so
  // an offline batch's frames do not depend on how many windows it holds
  int allow_skinny = 0;
  // skinny route only: A = LayerNorm(ln_x) computed in the GEMM (f32 rows
  // [M, K], gamma / beta [K], K = 1024), the LayerNorm kernel's arithmetic;
  // ln_lo: also its exact lo plane (A ignored)
  const float *ln_x = nullptr, *ln_g = nullptr, *ln_b = nullptr;
  float ln_eps = 0.f;
  int ln_lo = 0;
  // skinny route only: workspace for split-K partial tiles (N <= 2048: the K
  // range is split over kSkinnySplit workgroups per 16 columns, whose partial
  // tiles a second kernel adds in split order before the epilogue); null: one
  // workgroup per 16 columns
  float *skp = nullptr;
  size_t skp_bytes = 0;
  const float *bias = nullptr;      // [N]
  const float *add = nullptr;       // f32 residual [M, ldadd]; may alias C
  int ldadd = 0;
  int act = 0;
  int glu = 0;   // GLU-pair epilogue (see gemm.hip), out [M, N/2] f16
  int hilo = 0;  // ReLU then an exact f16 pair per value: out [M, 2N] f16, (hi, lo) at columns 2n, 2n+1
  // f16 epilogue only: columns >= vcol0 go transposed to vt[vrow[row] + (col - vcol0) * vtp]
  // instead of C (rows with vrow < 0 are dropped); the direct-to-LDS route only
  _Float16 *vt = nullptr;
  const int *vrow = nullptr;
  int vcol0 = 0, vtp = 0;
  int M = 0, N = 0, K = 0;
};

// 1 when gemm_mfma runs p on the direct-to-LDS route (the one that honours vt)
int gemm_takes_direct(fa_ctx *ctx, const GemmArgs &p);

int gemm_mfma(fa_ctx *ctx, const GemmArgs &p, const char *label);
int gemm_f32(fa_ctx *ctx, const float *A, const float *B, float *C, const float *bias, const float *add, int M, int N, int K, int act,
             const char *label);
int gemm_naive_f16(fa_ctx *ctx, const float *A, const void *Bkm, float *C, const float *bias, const float *add, int M, int N, int K, int act,
                   const char *label);

}  // namespace fa
