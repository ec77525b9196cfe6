// GEMM kernel templates and their launch dispatch, shared by the translation
// units that instantiate them (gemm.hip: f16 and f32 weights; gemm_q8.hip /
// gemm_q4.hip: int8 and int4 weights, split so the instantiations compile in
// parallel).  See gemm.hip for the design.
#pragma once
#include "fa_internal.h"
#include "fa_device.h"
#include "gemm.h"

#include <cstdio>
#include <cstdlib>

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

// Epilogue variants, fixed at compile time so the per-element code is short and
// the accumulators stay in registers (a runtime activation switch per element
// pushed large tiles' accumulators to scratch).
enum Epi : int { EPI_F32 = 0, EPI_F16 = 1, EPI_F16_SILU = 2, EPI_F16_RELU = 3, EPI_GLU = 4, EPI_GENERIC = 5, EPI_HILO_RELU = 6 };

// Epilogue results: computed in f32, then rounded to f16.  The empty asm pins
// the f32 value in a register; without it the compiler may fuse the preceding
// scale-and-bias fma with the conversion into one f16-rounding v_fma_mix on
// some code paths and not others, and two kernels of the same math would
// disagree in the last f16 bit.
__device__ __forceinline__ _Float16 to_f16(float t) {
  asm("" : "+v"(t));
  return (_Float16)t;
}

__device__ __forceinline__ float sigmoid_mul(float v, float g) { return __fdividef(v, 1.f + __expf(-fminf(fmaxf(g, -30.f), 30.f))); }

// Epilogue of the register-staged kernel, through LDS (free after the main loop): each wave writes
// 16-row strips of its accumulators, then reads them back row-contiguous so
// every global access is a 16-byte vector and each row segment is written
// by consecutive lanes (the MFMA layout itself gives 2-4 byte scattered stores).
// `lds` holds 16 * (WTN + 4) floats per wave; (r0, c0) is the wave tile's origin.
template <int WTM, int WTN, int TI, int TJ, int EPI>
__device__ __forceinline__ void epilogue(const GemmArgs &p, f4 (&acc)[TI][TJ], float *lds, int r0, int c0, int wave, int lane) {
  constexpr int SS = WTN + 4;  // strip row stride (floats)
  float *strip = lds + wave * 16 * SS;
  constexpr int OCOLS = EPI == EPI_GLU ? WTN / 2 : WTN;  // output columns of this wave's strip
  constexpr int LPR = OCOLS / 4;                         // lanes per output row (4 values each)
  constexpr int RPP = 64 / LPR;                          // rows per pass
  static_assert(LPR >= 1 && LPR <= 64, "epilogue lane mapping");
  const int lc = (lane % LPR) * 4, lr = lane / LPR;
  // per-lane column constants (fixed across strips)
  float cs[4] = {1.f, 1.f, 1.f, 1.f}, bv[4] = {0.f, 0.f, 0.f, 0.f}, gcs[4] = {1.f, 1.f, 1.f, 1.f}, gbv[4] = {0.f, 0.f, 0.f, 0.f};
  int vcol[4], gcol[4];
#pragma unroll
  for (int e = 0; e < 4; e++) {
    if constexpr (EPI == EPI_GLU) {
      const int ch = lc + e;  // output channel within the strip
      vcol[e] = (ch >> 3) * 16 + ((ch & 7) >> 1) * 4 + (ch & 1);
      gcol[e] = vcol[e] + 2;
    } else {
      vcol[e] = lc + e;
      gcol[e] = vcol[e];
    }
    const int gv = c0 + vcol[e], gg = c0 + gcol[e];
    if (p.colscale) {
      cs[e] = gv < p.N ? p.colscale[gv] : 1.f;
      gcs[e] = gg < p.N ? p.colscale[gg] : 1.f;
    }
    if (p.bias) {
      bv[e] = gv < p.N ? p.bias[gv] : 0.f;
      gbv[e] = gg < p.N ? p.bias[gg] : 0.f;
    }
  }
#pragma unroll
  for (int i = 0; i < TI; i++) {
#pragma unroll
    for (int j = 0; j < TJ; j++)
#pragma unroll
      for (int r = 0; r < 4; r++) strip[((lane >> 4) * 4 + r) * SS + j * 16 + (lane & 15)] = acc[i][j][r];
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): strip written (global stores stay in flight)
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int pr = 0; pr < 16; pr += RPP) {
      const int rr = pr + lr;
      const int row = r0 + i * 16 + rr;
      if (lr < RPP && rr < 16 && row < p.M) {
        float v[4];
#pragma unroll
        for (int e = 0; e < 4; e++) v[e] = strip[rr * SS + vcol[e]] * cs[e] + bv[e];
        if constexpr (EPI == EPI_GLU) {
          const int ocol = (c0 >> 1) + lc;
          if (ocol + 3 < (p.N >> 1) && !p.out_f16) {
            float4 o;
            o.x = sigmoid_mul(v[0], strip[rr * SS + gcol[0]] * gcs[0] + gbv[0]);
            o.y = sigmoid_mul(v[1], strip[rr * SS + gcol[1]] * gcs[1] + gbv[1]);
            o.z = sigmoid_mul(v[2], strip[rr * SS + gcol[2]] * gcs[2] + gbv[2]);
            o.w = sigmoid_mul(v[3], strip[rr * SS + gcol[3]] * gcs[3] + gbv[3]);
            *reinterpret_cast<float4 *>(reinterpret_cast<float *>(p.C) + (size_t)row * p.ldc + ocol) = o;
          } else if (ocol + 3 < (p.N >> 1)) {
            h4 o;
#pragma unroll
            for (int e = 0; e < 4; e++) {
              const float t = sigmoid_mul(v[e], strip[rr * SS + gcol[e]] * gcs[e] + gbv[e]);
              o[e] = to_f16(t);
              v[e] = t - (float)o[e];
            }
            *reinterpret_cast<h4 *>(reinterpret_cast<_Float16 *>(p.C) + (size_t)row * p.ldc + ocol) = o;
            if (p.Clo) *reinterpret_cast<h4 *>(reinterpret_cast<_Float16 *>(p.Clo) + (size_t)row * p.ldc + ocol) = h4{(_Float16)v[0], (_Float16)v[1], (_Float16)v[2], (_Float16)v[3]};
          }
        } else {
          const int col = c0 + lc;
          if (col + 3 < p.N) {
            if constexpr (EPI == EPI_F32) {
              float4 o = make_float4(v[0], v[1], v[2], v[3]);
              if (p.add) {
                const float4 ad = *reinterpret_cast<const float4 *>(p.add + (size_t)row * p.ldadd + col);
                o.x += ad.x; o.y += ad.y; o.z += ad.z; o.w += ad.w;
              }
              *reinterpret_cast<float4 *>(reinterpret_cast<float *>(p.C) + (size_t)row * p.ldc + col) = o;
            } else if constexpr (EPI == EPI_HILO_RELU) {
              // v = hi + lo exactly (hi = f16(v), lo = f16(v - hi)) for a consumer
              // GEMM that reads both halves against duplicated weight rows
              h8 o;
#pragma unroll
              for (int e = 0; e < 4; e++) {
                const float t = fmaxf(v[e], 0.f);
                const _Float16 hi = to_f16(t);
                o[2 * e] = hi;
                o[2 * e + 1] = (_Float16)(t - (float)hi);
              }
              *reinterpret_cast<h8 *>(reinterpret_cast<_Float16 *>(p.C) + (size_t)row * p.ldc + 2 * col) = o;
            } else if constexpr (EPI == EPI_GENERIC) {
#pragma unroll
              for (int e = 0; e < 4; e++) {
                float o = act_apply(v[e], p.act);
                if (p.add) o += p.add[(size_t)row * p.ldadd + col + e];
                if (p.out_f16)
                  reinterpret_cast<_Float16 *>(p.C)[(size_t)row * p.ldc + col + e] = to_f16(o);
                else
                  reinterpret_cast<float *>(p.C)[(size_t)row * p.ldc + col + e] = o;
              }
            } else {
              h4 o, ol;
#pragma unroll
              for (int e = 0; e < 4; e++) {
                float t = v[e];
                if constexpr (EPI == EPI_F16_SILU) t = sigmoid_mul(t, t);
                if constexpr (EPI == EPI_F16_RELU) t = fmaxf(t, 0.f);
                o[e] = to_f16(t);
                ol[e] = (_Float16)(t - (float)o[e]);
              }
              *reinterpret_cast<h4 *>(reinterpret_cast<_Float16 *>(p.C) + (size_t)row * p.ldc + col) = o;
              if (p.Clo) *reinterpret_cast<h4 *>(reinterpret_cast<_Float16 *>(p.Clo) + (size_t)row * p.ldc + col) = ol;
            }
          } else {
            // ragged right edge (N not a multiple of 4 within this tile)
#pragma unroll
            for (int e = 0; e < 4; e++) {
              if (col + e >= p.N) break;
              float o = v[e];
              if constexpr (EPI == EPI_GENERIC) o = act_apply(o, p.act);
              if constexpr (EPI == EPI_F16_SILU) o = sigmoid_mul(o, o);
              if constexpr (EPI == EPI_F16_RELU) o = fmaxf(o, 0.f);
              if constexpr (EPI == EPI_F32 || EPI == EPI_GENERIC)
                if (p.add) o += p.add[(size_t)row * p.ldadd + col + e];
              if constexpr (EPI == EPI_HILO_RELU) {
                o = fmaxf(o, 0.f);
                const _Float16 hi = to_f16(o);
                reinterpret_cast<_Float16 *>(p.C)[(size_t)row * p.ldc + 2 * (col + e)] = hi;
                reinterpret_cast<_Float16 *>(p.C)[(size_t)row * p.ldc + 2 * (col + e) + 1] = (_Float16)(o - (float)hi);
              } else if (EPI == EPI_F32 || (EPI == EPI_GENERIC && !p.out_f16))
                reinterpret_cast<float *>(p.C)[(size_t)row * p.ldc + col + e] = o;
              else
                reinterpret_cast<_Float16 *>(p.C)[(size_t)row * p.ldc + col + e] = to_f16(o);
            }
          }
        }
      }
    }
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): strip reads done before the next strip overwrites it
    __builtin_amdgcn_wave_barrier();
  }
}

template <int BM, int BN, int WM, int WN, int AK, int BKND, int EPI>
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
    h8 af[2][TI], bf[2][TJ];
#pragma unroll
    for (int i = 0; i < TI; i++) af[0][i] = *reinterpret_cast<const h8 *>(&sA[buf][(arow + i * 16) * LS + kq]);
#pragma unroll
    for (int j = 0; j < TJ; j++) bf[0][j] = *reinterpret_cast<const h8 *>(&sB[buf][(brow + j * 16) * LS + kq]);
#pragma unroll
    for (int i = 0; i < TI; i++) af[1][i] = *reinterpret_cast<const h8 *>(&sA[buf][(arow + i * 16) * LS + 32 + kq]);
#pragma unroll
    for (int j = 0; j < TJ; j++) bf[1][j] = *reinterpret_cast<const h8 *>(&sB[buf][(brow + j * 16) * LS + 32 + kq]);
#pragma unroll
    for (int s = 0; s < 2; s++)
#pragma unroll
      for (int i = 0; i < TI; i++)
#pragma unroll
        for (int j = 0; j < TJ; j++) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[s][i], bf[s][j], acc[i][j], 0, 0, 0);
    if (kt + 1 < nk) lstore(buf ^ 1);
    __syncthreads();
  }

  epilogue<WTM, WTN, TI, TJ, EPI>(p, acc, reinterpret_cast<float *>(&sA[0][0]), m0 + wm * WTM, n0 + wn * WTN, wave, lane);
}

// Epilogue of the direct-to-LDS kernel, which runs its MFMAs with the operands
// swapped (C^T tiles): acc[i][j] holds row r0 + 16i + (lane & 15), columns
// c0 + 16j + 4(lane >> 4) + {0..3}.  Each lane owns four consecutive columns of
// one row and stores them straight from registers (16-byte f32 / 8-byte f16
// vectors): no LDS round trip, and nothing waits for the stores.  GLU weight
// columns are interleaved so the four columns are (value c, value c+1, gate c,
// gate c+1) of two consecutive output channels.
template <int TI, int TJ, int EPI>
__device__ __forceinline__ void epilogue_direct(const GemmArgs &p, f4 (&acc)[TI][TJ], int r0, int c0, int lane) {
  const int cl = 4 * (lane >> 4);
  const bool scaled = p.colscale != nullptr;  // int8 column scales, per-column folds
  f4 bv[TJ], cs[TJ];
#pragma unroll
  for (int j = 0; j < TJ; j++) {
    const int col = c0 + 16 * j + cl;
#pragma unroll
    for (int e = 0; e < 4; e++) {
      bv[j][e] = p.bias ? p.bias[col + e] : 0.f;
      cs[j][e] = scaled ? p.colscale[col + e] : 1.f;
    }
  }
  if (scaled) {  // acc * s + b in one rounding, as the register-staged route computes it
#pragma unroll
    for (int i = 0; i < TI; i++)
#pragma unroll
      for (int j = 0; j < TJ; j++)
#pragma unroll
        for (int e = 0; e < 4; e++) acc[i][j][e] = __builtin_fmaf(acc[i][j][e], cs[j][e], bv[j][e]);
  }
#pragma unroll
  for (int i = 0; i < TI; i++) {
    const int row = r0 + 16 * i + (lane & 15);
    if (row >= p.M) continue;
    int vr = -1;  // transposed-V destination of this row
    if constexpr (EPI == EPI_F16)
      if (p.vt) vr = p.vrow[row];
#pragma unroll
    for (int j = 0; j < TJ; j++) {
      const int col = c0 + 16 * j + cl;
      f4 v = scaled ? acc[i][j] : acc[i][j] + bv[j];
      if constexpr (EPI == EPI_F16) {
        if (p.vt && col >= p.vcol0) {  // 16 lanes = 16 consecutive keys: 32-byte runs per column
          if (vr >= 0) {
            _Float16 *dst = p.vt + vr + (size_t)(col - p.vcol0) * p.vtp;
#pragma unroll
            for (int e = 0; e < 4; e++) dst[(size_t)e * p.vtp] = to_f16(v[e]);
          }
          continue;
        }
      }
      if constexpr (EPI == EPI_F32) {
        if (p.add) v += *reinterpret_cast<const f4 *>(p.add + (size_t)row * p.ldadd + col);
        *reinterpret_cast<f4 *>(reinterpret_cast<float *>(p.C) + (size_t)row * p.ldc + col) = v;
      } else if constexpr (EPI == EPI_GLU) {
        const float t0 = sigmoid_mul(v[0], v[2]), t1 = sigmoid_mul(v[1], v[3]);
        const size_t o = (size_t)row * p.ldc + (col >> 1);
        if (!p.out_f16) {
          *reinterpret_cast<float2 *>(reinterpret_cast<float *>(p.C) + o) = make_float2(t0, t1);
        } else {
          const h2 h = h2{to_f16(t0), to_f16(t1)};
          *reinterpret_cast<h2 *>(reinterpret_cast<_Float16 *>(p.C) + o) = h;
          if (p.Clo) *reinterpret_cast<h2 *>(reinterpret_cast<_Float16 *>(p.Clo) + o) = h2{(_Float16)(t0 - (float)h[0]), (_Float16)(t1 - (float)h[1])};
        }
      } else if constexpr (EPI == EPI_HILO_RELU) {
        h8 o;
#pragma unroll
        for (int e = 0; e < 4; e++) {
          const float t = fmaxf(v[e], 0.f);
          const _Float16 hi = to_f16(t);
          o[2 * e] = hi;
          o[2 * e + 1] = (_Float16)(t - (float)hi);
        }
        *reinterpret_cast<h8 *>(reinterpret_cast<_Float16 *>(p.C) + (size_t)row * p.ldc + 2 * col) = o;
      } else if constexpr (EPI == EPI_GENERIC) {  // the ComputeContext's act-then-add, f32 or f16 out
        f4 t;
#pragma unroll
        for (int e = 0; e < 4; e++) t[e] = act_apply(v[e], p.act);
        if (p.add) t += *reinterpret_cast<const f4 *>(p.add + (size_t)row * p.ldadd + col);
        if (p.out_f16)
          *reinterpret_cast<h4 *>(reinterpret_cast<_Float16 *>(p.C) + (size_t)row * p.ldc + col) = h4{to_f16(t[0]), to_f16(t[1]), to_f16(t[2]), to_f16(t[3])};
        else
          *reinterpret_cast<f4 *>(reinterpret_cast<float *>(p.C) + (size_t)row * p.ldc + col) = t;
      } else {
        h4 o, ol;
#pragma unroll
        for (int e = 0; e < 4; e++) {
          float t = v[e];
          if constexpr (EPI == EPI_F16_SILU) t = sigmoid_mul(t, t);
          if constexpr (EPI == EPI_F16_RELU) t = fmaxf(t, 0.f);
          o[e] = to_f16(t);
          ol[e] = (_Float16)(t - (float)o[e]);
        }
        *reinterpret_cast<h4 *>(reinterpret_cast<_Float16 *>(p.C) + (size_t)row * p.ldc + col) = o;
        if (p.Clo) *reinterpret_cast<h4 *>(reinterpret_cast<_Float16 *>(p.Clo) + (size_t)row * p.ldc + col) = ol;
      }
    }
  }
}

// ── direct-to-LDS multi-stage GEMM (A f16, B f16 / int8 / int4 K-major) ────
// The encoder's hot path.  Each K tile (64 halfs = 128 B per row) of the
// stacked A|B panel is copied global->LDS by global_load_lds_dwordx4 (no VGPR
// staging), S tiles in flight in one LDS buffer.  Within a 128-byte
// row the 16-byte chunk c of row r lives in slot c ^ (r & 7), so the eight
// rows one ds_read_b128 phase touches hit distinct banks and each 8-lane group
// of a copy still reads one contiguous 128-byte row segment.  8-wave
// configurations run two waves per SIMD so one wave's MFMAs cover the other's
// LDS reads and barrier waits.
//
// The copies are issued from inline asm and their completion is tracked with
// explicit vmcnt waits: the compiler cannot tell the stages apart and would
// otherwise wait for every copy in flight before each LDS read.
// M0 is never a register-allocation candidate; the compiler only writes it
// immediately before its own M0-reading instructions, so setting it inside the
// asm statement is safe (clang still warns about clobbering a reserved register).
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void dma16(const void *g, uint32_t lds_addr) {
  asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(g), "s"(lds_addr) : "memory", "m0");
}
#pragma clang diagnostic pop
template <int N>
__device__ __forceinline__ void wait_vmcnt() {  // gfx9 s_waitcnt: vmcnt [3:0]+[15:14], expcnt 7, lgkmcnt 15 = no wait
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// LO = 1: A arrives as two f16 planes (A = hi + lo exactly); both are staged
// and each B fragment feeds two MFMAs, so the product carries f32-accurate A.
// BQ = 1: B is int8 K-major (per-column scale in the epilogue); its K tile is
// 64 bytes per row (16-byte chunk c at slot c ^ ((row >> 1) & 3)) and each
// fragment is widened to f16 exactly after the LDS read.
// BQ = 2: B is symmetric int4 group-32 ([N][K/32][16 B], f16 scales [N][K/32]);
// its K tile is 32 bytes per row (chunk c at slot c ^ ((row >> 2) & 1)), the
// two block scales of a row's K tile are one 4-byte load made a K tile ahead.
// WW = 1 (with BQ): the quantised K tile of B is widened to f16 once per
// workgroup, one tile ahead, into one of two f16 tiles laid out like the f16
// route's B tile; the fragment reads and MFMAs are then the f16 route's. B
// copies run one K tile ahead of A copies (copy group g holds A tile g and B
// tile g + 1), so the wait that makes A tile kt resident also makes B tile
// kt + 1 resident for its widening during step kt.
template <int BM, int BN, int WM, int WN, int S, int EPI, int LO = 0, int BQ = 0, int WW = 0>
__global__ __launch_bounds__(64 * WM * WN) __attribute__((amdgpu_waves_per_eu(WM * WN / 4, WM * WN / 4))) void gemm_dma_kernel(GemmArgs p) {
  constexpr int B8 = BQ == 1, B4 = BQ == 2;
  static_assert(!WW || BQ, "workgroup widening is for quantised B");
  constexpr int NW = WM * WN, BK = 64, RB = 128, RBB = B8 ? 64 : (B4 ? 32 : 128);
  static_assert(!B4 || S % 2 == 0, "int4 scale double-buffering follows the stage parity");
  constexpr int WTM = BM / WM, WTN = BN / WN, TI = WTM / 16, TJ = WTN / 16;
  constexpr int AR = BM * (1 + LO);                   // staged A rows: hi (and lo) planes
  constexpr int SA = AR * RB, STG = AR * RB + BN * RBB;
  constexpr int ITA = AR / 8, IT = ITA + BN * RBB / 1024;  // 1 KB copies per stage (A: 8 rows each; B: 8 or 16 rows)
  constexpr int IW = (IT + NW - 1) / NW, IMIN = IT / NW;  // per wave: at most / at least
  static_assert(BM % 16 == 0 && BN % 16 == 0 && NW % 4 == 0 && (BN * RBB) % 1024 == 0, "tile shape");
  static_assert(S >= 2 && S <= 4, "LDS stages");
  constexpr int WT = WW ? BN * RB : 0;  // one widened f16 B tile
  constexpr int SMEM = S * STG + 2 * WT;
  static_assert(SMEM <= 160 * 1024, "LDS");
  __shared__ __attribute__((aligned(1024))) char smem[SMEM];
  uint32_t sadr[4];
  {
    const uint32_t s0 = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(__attribute__((address_space(3))) char *)smem);
#pragma unroll
    for (int i = 0; i < 4; i++) sadr[i] = s0 + i * STG;
  }
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / WN, wn = wave % WN;
  const int nTN = p.N / BN, nTM = (p.M + BM - 1) / BM;
  // XCD-contiguous tile runs (xcd_remap), ordered in groups of 8 M-rows with N
  // outer inside a group: one XCD's run covers ~8 A panels x (run/8) B panels,
  // so its L2 holds both operands instead of streaming every B panel.
  const int tile = xcd_remap(blockIdx.x, nTM * nTN);
  constexpr int GM = 8;
  const int grp = tile / (GM * nTN), gm = min(GM, nTM - grp * GM), gi = tile - grp * GM * nTN;
  const int m0 = (grp * GM + gi % gm) * BM, n0 = (gi / gm) * BN;
  const _Float16 *A = reinterpret_cast<const _Float16 *>(p.A), *B = reinterpret_cast<const _Float16 *>(p.B);

  // copy i of this wave: an A copy moves rows [ins*8, ins*8+8) of the stacked
  // A (hi | lo) tile, a B copy 8 (f16) or 16 (int8) rows of the B tile
  const void *src[IW];
#pragma unroll
  for (int i = 0; i < IW; i++) {
    const int ins = wave + i * NW;
    if (ins < ITA) {
      const int r = ins * 8 + (lane >> 3), ch = (lane & 7) ^ (r & 7);
      if (r < BM)
        src[i] = A + (size_t)min(m0 + r, p.M - 1) * p.lda + ch * 8;  // rows past M repeat the last row; never stored
      else
        src[i] = reinterpret_cast<const _Float16 *>(p.Alo) + (size_t)min(m0 + r - BM, p.M - 1) * p.lda + ch * 8;
    } else if constexpr (B8) {
      const int r = (ins - ITA) * 16 + (lane >> 2), ch = (lane & 3) ^ ((r >> 1) & 3);
      src[i] = reinterpret_cast<const int8_t *>(p.B) + (size_t)(n0 + r) * p.K + ch * 16;
    } else if constexpr (B4) {
      const int r = (ins - ITA) * 32 + (lane >> 1), ch = (lane & 1) ^ ((r >> 2) & 1);
      src[i] = reinterpret_cast<const uint8_t *>(p.B) + (size_t)(n0 + r) * (p.K >> 1) + ch * 16;
    } else {
      const int r = (ins - ITA) * 8 + (lane >> 3), ch = (lane & 7) ^ (r & 7);
      src[i] = B + (size_t)(n0 + r) * p.K + ch * 8;
    }
  }
  // bonly: copy only B's K tile at k0 (the tile ahead of the first group)
  auto issue = [&](int sidx, int k0, bool bonly = false) {
    // WW: B runs one tile ahead; the last group re-copies the last tile (never
    // widened) so every group holds the same copies and the vmcnt waits hold
    const int kb = (WW && !bonly) ? min(k0 + BK, p.K - BK) : k0;
#pragma unroll
    for (int i = 0; i < IW; i++) {
      const int ins = wave + i * NW;
      if ((IT % NW == 0 || ins < IT) && (!bonly || ins >= ITA)) {
        const size_t koff = (ins < ITA || !BQ) ? (size_t)k0 * 2 : (B8 ? (size_t)kb : (size_t)(kb >> 1));  // bytes
        dma16(reinterpret_cast<const char *>(src[i]) + koff, sadr[sidx] + ins * 1024);
      }
    }
  };

  f4 acc[TI][TJ];
#pragma unroll
  for (int i = 0; i < TI; i++)
#pragma unroll
    for (int j = 0; j < TJ; j++) acc[i][j] = f4{0.f, 0.f, 0.f, 0.f};

  const int nk = p.K / BK;

  const int q = lane >> 4, sw = lane & 7;  // fragment rows are 16-aligned + (lane & 15)
  const int abase = (wm * WTM + (lane & 15)) * RB, bbase = SA + (wn * WTN + (lane & 15)) * RBB;
  const int sw8 = ((lane & 15) >> 1) & 3;  // int8 B rows: (row >> 1) & 3
  const int sw4 = ((lane & 15) >> 2) & 1;  // int4 B rows: (row >> 2) & 1
  h8 af[2][TI], bf[2][TJ], al[2][LO ? TI : 1];
  // int4 B: raw fragments (4 bytes + block scale) are kept as read and
  // widened right before their MFMAs, so the LDS read of the next half-step
  // is not waited for before this half-step's MFMAs issue (measured: int4
  // encoder 10.10 -> 9.57 ms; int8, whose widening is cheaper, was 1 % slower
  // this way and widens at the read)
  uint2 bq[2][B4 ? TJ : 1];
  _Float16 bs[2][B4 ? TJ : 1];
  // int4 block scales of the K tile being read, two sets by tile parity
  uint32_t scs[2][B4 ? TJ : 1];
  auto ldscale = [&](int set, int kt) {
    if constexpr (B4) {
      const int nblk = p.K >> 5;
#pragma unroll
      for (int j = 0; j < TJ; j++)
        scs[set][j] = *reinterpret_cast<const uint32_t *>(reinterpret_cast<const _Float16 *>(p.bscale) +
                                                          (size_t)(n0 + wn * WTN + j * 16 + (lane & 15)) * nblk + 2 * kt);
    }
  };
  // WW: tile kt's widened B lives in f16 tile kt & 1 (wpar)
  auto rdfrag = [&](int sidx, int ks, int slot, int set, int wpar = 0) {
    const char *base = smem + sidx * STG;
    const int so = ((ks * 4 + q) ^ sw) * 16;
#pragma unroll
    for (int i = 0; i < TI; i++) af[slot][i] = *reinterpret_cast<const h8 *>(base + abase + i * 16 * RB + so);
    if constexpr (LO) {
#pragma unroll
      for (int i = 0; i < TI; i++) al[slot][i] = *reinterpret_cast<const h8 *>(base + BM * RB + abase + i * 16 * RB + so);
    }
    if constexpr (WW) {
      const char *wb = smem + S * STG + wpar * WT + (wn * WTN + (lane & 15)) * RB + so;
#pragma unroll
      for (int j = 0; j < TJ; j++) bf[slot][j] = *reinterpret_cast<const h8 *>(wb + j * 16 * RB);
    } else if constexpr (B8) {
      // k = ks*32 + q*8: 16-byte chunk 2*ks + q/2, half q & 1
      const int so8 = ((((ks * 2 + (q >> 1)) ^ sw8) * 16) + (q & 1) * 8);
#pragma unroll
      for (int j = 0; j < TJ; j++) bf[slot][j] = i8x8_to_h8(*reinterpret_cast<const uint2 *>(base + bbase + j * 16 * RBB + so8));
    } else if constexpr (B4) {
      // k = ks*32 + q*8: 16-byte chunk ks (block ks of the tile), 4 bytes at q*4
      const int so4 = ((ks ^ sw4) * 16) + q * 4;
#pragma unroll
      for (int j = 0; j < TJ; j++) {
        const uint32_t sw2 = scs[set][j];
        bs[slot][j] = __builtin_bit_cast(_Float16, (uint16_t)(ks ? (sw2 >> 16) : (sw2 & 0xffffu)));
        bq[slot][j].x = *reinterpret_cast<const uint32_t *>(base + bbase + j * 16 * RBB + so4);
      }
    } else {
#pragma unroll
      for (int j = 0; j < TJ; j++) bf[slot][j] = *reinterpret_cast<const h8 *>(base + bbase + j * 16 * RB + so);
    }
  };
  // WW widening: unit u of a tile is 16 B-tile bytes of row u >> 2 (int8: raw
  // 16-byte chunk u & 3; int4: half u & 1 of raw chunk (u >> 1) & 1, one
  // group-32 block), written as two 16-byte f16 chunks of the f16 layout
  constexpr int NT = 64 * NW, NU = BN * 4, UPT = (NU + NT - 1) / NT;
  uint32_t wsc[2][WW && B4 ? UPT : 1];  // int4 block scales of the units, by tile parity
  auto ldwscale = [&](int set, int kt) {
    if constexpr (WW && B4) {
      const int nblk = p.K >> 5;
#pragma unroll
      for (int i = 0; i < UPT; i++) {
        const int u = tid + i * NT;
        if (NU % NT == 0 || u < NU)
          wsc[set][i] = *(reinterpret_cast<const uint16_t *>(p.bscale) + (size_t)(n0 + (u >> 2)) * nblk + 2 * kt + ((u >> 1) & 1));
      }
    }
  };
  auto widen = [&](int sidx, int kt, int set) {
    if constexpr (WW) {
      const char *raw = smem + sidx * STG + SA;
      char *dst = smem + S * STG + (kt & 1) * WT;
#pragma unroll
      for (int i = 0; i < UPT; i++) {
        const int u = tid + i * NT;
        if (NU % NT == 0 || u < NU) {
          const int r = u >> 2;
          h8 lo, hi;
          int c0;
          if constexpr (B8) {
            const int c = u & 3;
            const uint4 v = *reinterpret_cast<const uint4 *>(raw + r * 64 + ((c ^ ((r >> 1) & 3)) * 16));
            lo = i8x8_to_h8(uint2{v.x, v.y});
            hi = i8x8_to_h8(uint2{v.z, v.w});
            c0 = 2 * c;
          } else {
            const int ch = (u >> 1) & 1, half = u & 1;
            const uint2 v = *reinterpret_cast<const uint2 *>(raw + r * 32 + ((ch ^ ((r >> 2) & 1)) * 16) + half * 8);
            const _Float16 sc = __builtin_bit_cast(_Float16, (uint16_t)wsc[set][i]);
            lo = i4x8_to_h8(v.x, sc);
            hi = i4x8_to_h8(v.y, sc);
            c0 = ch * 4 + half * 2;
          }
          *reinterpret_cast<h8 *>(dst + r * RB + ((c0 ^ (r & 7)) * 16)) = lo;
          *reinterpret_cast<h8 *>(dst + r * RB + (((c0 + 1) ^ (r & 7)) * 16)) = hi;
        }
      }
    }
  };
  auto mma = [&](int slot) {
    if constexpr (B4 && !WW) {
#pragma unroll
      for (int j = 0; j < TJ; j++) bf[slot][j] = i4x8_to_h8(bq[slot][j].x, bs[slot][j]);
    }
#pragma unroll
    for (int i = 0; i < TI; i++)
#pragma unroll
      for (int j = 0; j < TJ; j++) {
        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(bf[slot][j], af[slot][i], acc[i][j], 0, 0, 0);  // C^T tile
        if constexpr (LO) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(bf[slot][j], al[slot][i], acc[i][j], 0, 0, 0);
      }
  };
  // K tile kt is in LDS once at most (S-2) later tiles are still in flight
  // (copies complete in issue order), for every wave: then barrier.
  auto ready = [&](int kt) {
    if (kt + S - 2 < nk)
      wait_vmcnt<(S - 2) * IMIN>();
    else
      wait_vmcnt<0>();
    __syncthreads();
  };

  if constexpr (WW) {
    // B tile 0 ahead of the first group, into the last stage (refilled by the
    // first step's copies, after the barrier that follows its widening)
    ldwscale(0, 0);
    if (1 < nk) ldwscale(1, 1);
    issue(S - 1, 0, true);
  }
#pragma unroll
  for (int s = 0; s < S - 1; s++)
    if (s < nk) issue(s, s * BK);

  if constexpr (!WW) ldscale(0, 0);
  ready(0);
  if constexpr (WW) {
    widen(S - 1, 0, 0);
    __syncthreads();
  }
  rdfrag(0, 0, 0, 0, 0);
  for (int kt0 = 0; kt0 < nk; kt0 += S) {
#pragma unroll
    for (int u = 0; u < S; u++) {
      const int kt = kt0 + u;
      if (kt < nk) {
        // refill the stage every wave finished reading before the last barrier
        if (kt + S - 1 < nk) issue((u + S - 1) % S, (kt + S - 1) * BK);
        if constexpr (WW) {
          rdfrag(u, 1, 1, 0, kt & 1);
          // B tile kt + 1 (resident in stage u since the last barrier) into the
          // f16 tile that tile kt - 1's reads, finished before that barrier, used
          if (kt + 1 < nk) widen(u, kt + 1, (u + 1) & 1);
          if (kt + 2 < nk) ldwscale(u & 1, kt + 2);  // int4: S is even, so u & 1 is kt's parity
        } else {
          if (kt + 1 < nk) ldscale((u + 1) & 1, kt + 1);  // int4: next tile's scales (S is even)
          rdfrag(u, 1, 1, u & 1);
        }
        mma(0);
        mma(1);  // placed before the wait so its MFMAs overlap the barrier
        if (kt + 1 < nk) {
          ready(kt + 1);
          rdfrag((u + 1) % S, 0, 0, (u + 1) & 1, (kt + 1) & 1);
        }
      }
    }
  }
  epilogue_direct<TI, TJ, EPI>(p, acc, m0 + wm * WTM, n0 + wn * WTN, lane);
}

// ── host dispatch ───────────────────────────────────────────────────────────
template <int BM, int BN, int WM, int WN, int AK, int BKND, int EPI>
static int launch_cfg(fa_ctx *ctx, const GemmArgs &p, const char *label) {
  const unsigned tiles = cdiv(p.M, BM) * cdiv(p.N, BN);
  ProfScope ps(ctx, label);
  FA_LAUNCH(ps, (gemm_mfma_kernel<BM, BN, WM, WN, AK, BKND, EPI>), dim3(tiles), dim3(64 * WM * WN), 0, ctx->stream, p);
  return check_launch(ctx, label);
}

static int epi_of(const GemmArgs &p) {
  if (p.glu) return EPI_GLU;
  if (p.hilo) return EPI_HILO_RELU;
  if (!p.out_f16) return (p.act == 0) ? EPI_F32 : EPI_GENERIC;
  if (p.add) return EPI_GENERIC;
  if (p.act == 0) return EPI_F16;
  if (p.act == 4) return EPI_F16_SILU;
  if (p.act == 3) return EPI_F16_RELU;
  return EPI_GENERIC;
}

// Tile configurations (BM x BN, 2x2 waves of (BM/2)x(BN/2)).  `slots` is how
// many workgroups fit on a CU (LDS-limited); rate1/rate2 are measured
// per-CU throughputs on MI355X (tile-area·K per µs, K=1024, f16) with one
// workgroup per CU and with every slot busy.  Bigger wave tiles read less
// LDS per MFMA; smaller tiles quantise better over 256 CUs.
struct TileCfg {
  int bm, bn, slots;
  float rate1, rate2;
};
static const TileCfg kTiles[] = {
    {256, 256, 1, 1285.f, 1285.f}, {192, 256, 1, 1199.f, 1199.f}, {256, 192, 1, 1228.f, 1228.f}, {192, 192, 1, 1072.f, 1072.f},
    {256, 128, 1, 1062.f, 1062.f}, {128, 256, 1, 1137.f, 1137.f}, {192, 128, 1, 1007.f, 1007.f}, {128, 128, 2, 1170.f, 1638.f},
    {192, 64, 2, 962.f, 1117.f},   {64, 128, 2, 700.f, 1024.f}};

static int pick_tile(fa_ctx *ctx, int M, int N) {
  // FA_GEMM_TILE=BMxBN pins one configuration (tuning sweeps).
  if (const char *e = getenv("FA_GEMM_TILE")) {
    int bm = 0, bn = 0;
    if (sscanf(e, "%dx%d", &bm, &bn) == 2)
      for (int i = 0; i < (int)(sizeof kTiles / sizeof kTiles[0]); i++)
        if (kTiles[i].bm == bm && kTiles[i].bn == bn) return i;
  }
  int best = 0;
  double bestc = 1e300;
  for (int i = 0; i < (int)(sizeof kTiles / sizeof kTiles[0]); i++) {
    const TileCfg &t = kTiles[i];
    const long tiles = (long)cdiv(M, t.bm) * cdiv(N, t.bn);
    const double area = (double)t.bm * t.bn;
    double c;
    if (tiles <= ctx->num_cu) {
      c = area / t.rate1;
    } else {
      const long rounds = (tiles + (long)t.slots * ctx->num_cu - 1) / ((long)t.slots * ctx->num_cu);
      c = rounds * area * t.slots / t.rate2;
    }
    if (c < bestc * 0.999) {
      bestc = c;
      best = i;
    }
  }
  return best;
}

// Direct-to-LDS configurations for f16 x f16: BM x BN, waves, stages, and the
// measured time of one full round (every CU busy with one tile, K = 1024) on
// MI355X at M = 3008; a launch costs ceil(tiles / CUs) rounds, scaled by K.
struct DmaCfg {
  int bm, bn;
  float us_round;
};
static const DmaCfg kDma[] = {{192, 256, 30.0f}, {192, 128, 18.3f}, {128, 128, 12.6f}, {96, 128, 11.7f}, {192, 192, 25.1f}};
// with a lo plane (two MFMAs per B fragment), same K = 1024 round timing
static const DmaCfg kDmaLo[] = {{192, 256, 51.0f}, {192, 128, 27.7f}, {96, 256, 27.0f}, {128, 128, 17.9f}, {96, 128, 16.5f}, {192, 192, 40.7f}};

static int pick_dma(fa_ctx *ctx, const GemmArgs &p) {
  // 16-byte operand copies; vector epilogue stores (up to 16 bytes at a multiple-of-4 column)
  if (p.K % 64 || p.lda % 8 || ((uintptr_t)p.A & 15) || ((uintptr_t)p.B & 15) || ((uintptr_t)p.Alo & 15)) return -1;
  if (p.ldc % 8 || p.ldadd % 4 || ((uintptr_t)p.C & 15) || ((uintptr_t)p.Clo & 15) || ((uintptr_t)p.add & 15)) return -1;
  const DmaCfg *tab = p.Alo ? kDmaLo : kDma;
  const int ntab = p.Alo ? (int)(sizeof kDmaLo / sizeof kDmaLo[0]) : (int)(sizeof kDma / sizeof kDma[0]);
  // FA_GEMM_DMA=0 turns the route off (not with a lo plane); 1..n pins
  // configuration 0..n-1 of the table in use when N fits it.
  if (const char *e = getenv("FA_GEMM_DMA")) {
    const int f = atoi(e);
    if (f == 0 && !p.Alo) return -1;
    if (f >= 1 && f <= ntab && p.N % tab[f - 1].bn == 0) return f - 1;
  }
  int best = -1;
  double bestc = 1e300;
  for (int i = 0; i < ntab; i++) {
    if (p.N % tab[i].bn) continue;
    const long tiles = (long)cdiv(p.M, tab[i].bm) * (p.N / tab[i].bn);
    const double c = (double)cdiv(tiles, ctx->num_cu) * tab[i].us_round;
    if (c < bestc * 0.999) {
      bestc = c;
      best = i;
    }
  }
  return best;
}

template <int BM, int BN, int WM, int WN, int S, int EPI, int LO = 0, int BQ = 0, int WW = 0>
static int launch_dma(fa_ctx *ctx, const GemmArgs &p, const char *label) {
  const unsigned tiles = cdiv(p.M, BM) * (p.N / BN);
  ProfScope ps(ctx, label);
  FA_LAUNCH(ps, (gemm_dma_kernel<BM, BN, WM, WN, S, EPI, LO, BQ, WW>), dim3(tiles), dim3(64 * WM * WN), 0, ctx->stream, p);
  return check_launch(ctx, label);
}

// Skinny route (M <= 16 TI rows, f16 A with an optional exact lo plane, f16
// B): the streaming passes' GEMMs, whose few rows leave a tiled kernel with a
// handful of workgroups streaming the whole weight matrix.  Workgroup = 16
// output columns x KS waves, wave w summing the K slice [w K/KS, (w+1) K/KS)
// with its B (16 columns) and A fragments loaded straight from global, G
// 32-deep steps of loads in flight; the slices' partial tiles are added
// through LDS in wave order and wave 0 runs the direct epilogue.
// SPLIT > 1: workgroup (x, y) sums the y-th of SPLIT K ranges and stores its
// raw tile in p.skp for gemm_skinny_split_sum_kernel (no epilogue here).
template <int TI, int KS, int EPI, int LO, int SPLIT = 1>
__global__ __launch_bounds__(64 * KS) void gemm_skinny_kernel(GemmArgs p) {
  constexpr int G = 8;
  __shared__ f4 part[KS > 1 ? KS - 1 : 1][TI][64];
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int c16 = lane & 15, g = lane >> 4;
  const int n0 = blockIdx.x * 16;
  const int ks = p.K / (KS * SPLIT), kb = blockIdx.y * (p.K / SPLIT) + wave * ks, nst = ks / 32;
  const _Float16 *B = reinterpret_cast<const _Float16 *>(p.B) + (size_t)(n0 + c16) * p.K + kb + g * 8;
  const _Float16 *A[TI], *Al[TI];
#pragma unroll
  for (int i = 0; i < TI; i++) {
    const size_t ro = (size_t)min(16 * i + c16, p.M - 1) * p.lda + kb + g * 8;
    A[i] = reinterpret_cast<const _Float16 *>(p.A) + ro;
    Al[i] = LO ? reinterpret_cast<const _Float16 *>(p.Alo) + ro : nullptr;
  }
  f4 acc[TI][1];
#pragma unroll
  for (int i = 0; i < TI; i++) acc[i][0] = f4{0.f, 0.f, 0.f, 0.f};
  for (int s0 = 0; s0 < nst; s0 += G) {
    h8 bf[G], af[G][TI], al[G][LO ? TI : 1];
#pragma unroll
    for (int u = 0; u < G; u++) {
      const int st = min(s0 + u, nst - 1) * 32;  // past the slice: a repeat, never used
      bf[u] = *reinterpret_cast<const h8 *>(B + st);
#pragma unroll
      for (int i = 0; i < TI; i++) {
        af[u][i] = *reinterpret_cast<const h8 *>(A[i] + st);
        if constexpr (LO) al[u][i] = *reinterpret_cast<const h8 *>(Al[i] + st);
      }
    }
#pragma unroll
    for (int u = 0; u < G; u++) {
      if (s0 + u < nst) {
#pragma unroll
        for (int i = 0; i < TI; i++) {
          acc[i][0] = __builtin_amdgcn_mfma_f32_16x16x32_f16(bf[u], af[u][i], acc[i][0], 0, 0, 0);  // C^T tile
          if constexpr (LO) acc[i][0] = __builtin_amdgcn_mfma_f32_16x16x32_f16(bf[u], al[u][i], acc[i][0], 0, 0, 0);
        }
      }
    }
  }
  if constexpr (KS > 1) {
    if (wave > 0)
#pragma unroll
      for (int i = 0; i < TI; i++) part[wave - 1][i][lane] = acc[i][0];
    __syncthreads();
    if (wave > 0) return;
#pragma unroll
    for (int w = 0; w < KS - 1; w++)
#pragma unroll
      for (int i = 0; i < TI; i++) acc[i][0] += part[w][i][lane];
  }
  if constexpr (SPLIT > 1) {
    f4 *dst = reinterpret_cast<f4 *>(p.skp) + (size_t)(blockIdx.y * gridDim.x + blockIdx.x) * TI * 64 + lane;
#pragma unroll
    for (int i = 0; i < TI; i++) dst[i * 64] = acc[i][0];
    return;
  }
  epilogue_direct<TI, 1, EPI>(p, acc, 0, n0, lane);
}

// The split-K skinny route's second launch: one wave per 16 columns adds the
// SPLIT partial tiles in split order, then runs the direct epilogue.
template <int TI, int SPLIT, int EPI>
__global__ __launch_bounds__(64) void gemm_skinny_split_sum_kernel(GemmArgs p) {
  const int lane = threadIdx.x;
  const f4 *src = reinterpret_cast<const f4 *>(p.skp) + (size_t)blockIdx.x * TI * 64 + lane;
  const size_t stride = (size_t)gridDim.x * TI * 64;  // one split's tiles
  f4 part[SPLIT][TI];
#pragma unroll
  for (int sp = 0; sp < SPLIT; sp++)
#pragma unroll
    for (int i = 0; i < TI; i++) part[sp][i] = src[sp * stride + i * 64];
  f4 acc[TI][1];
#pragma unroll
  for (int i = 0; i < TI; i++) {
    acc[i][0] = part[0][i];
#pragma unroll
    for (int sp = 1; sp < SPLIT; sp++) acc[i][0] += part[sp][i];
  }
  epilogue_direct<TI, 1, EPI>(p, acc, 0, blockIdx.x * 16, lane);
}

// The skinny route with the LayerNorm of its A rows folded in (stream
// passes: the norm_att / norm_conv / norm_ff2 launches disappear).  The
// workgroup first computes each row's mean and 1/std exactly as
// enc_ln_kernel does (one wave per row, float4 per lane at lane + 64 t, the
// same sums), then every A fragment is built from the f32 rows with the
// LayerNorm kernel's expression f16((x - mean) * inv * gamma + beta) (+ its
// exact lo plane).  K = 1024.
__device__ __forceinline__ float ln_affine(float x, float mean, float inv, float g, float b) { return (x - mean) * inv * g + b; }

template <int TI, int KS, int EPI, int LO>
__global__ __launch_bounds__(64 * KS) void gemm_skinny_ln_kernel(GemmArgs p) {
  constexpr int G = 4, D = 1024;
  __shared__ f4 part[KS > 1 ? KS - 1 : 1][TI][64];
  __shared__ float stat[2][32];
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int c16 = lane & 15, g = lane >> 4;
  for (int r = wave; r < p.M; r += KS) {  // row statistics
    const float4 *xr = reinterpret_cast<const float4 *>(p.ln_x + (size_t)r * D);
    float4 v[4];
#pragma unroll
    for (int t = 0; t < 4; t++) v[t] = xr[lane + 64 * t];
    float s = 0.f;
#pragma unroll
    for (int t = 0; t < 4; t++) s += v[t].x + v[t].y + v[t].z + v[t].w;
    const float mean = wave_sum(s) * (1.f / D);
    float q = 0.f;
#pragma unroll
    for (int t = 0; t < 4; t++) {
      const float a = v[t].x - mean, b = v[t].y - mean, c = v[t].z - mean, d = v[t].w - mean;
      q += a * a + b * b + c * c + d * d;
    }
    const float inv = rsqrtf(wave_sum(q) * (1.f / D) + p.ln_eps);
    if (lane == 0) {
      stat[0][r] = mean;
      stat[1][r] = inv;
    }
  }
  __syncthreads();
  const int n0 = blockIdx.x * 16;
  const int ks = p.K / KS, kb = wave * ks, nst = ks / 32;
  const _Float16 *B = reinterpret_cast<const _Float16 *>(p.B) + (size_t)(n0 + c16) * p.K + kb + g * 8;
  const float *X[TI];
  float mean[TI], inv[TI];
#pragma unroll
  for (int i = 0; i < TI; i++) {
    const int r = min(16 * i + c16, p.M - 1);
    X[i] = p.ln_x + (size_t)r * p.K + kb + g * 8;
    mean[i] = stat[0][r];
    inv[i] = stat[1][r];
  }
  const float *Gm = p.ln_g + kb + g * 8, *Bt = p.ln_b + kb + g * 8;
  f4 acc[TI][1];
#pragma unroll
  for (int i = 0; i < TI; i++) acc[i][0] = f4{0.f, 0.f, 0.f, 0.f};
  for (int s0 = 0; s0 < nst; s0 += G) {
    h8 bf[G];
    float4 xv[G][TI][2], gv[G][2], bv[G][2];
#pragma unroll
    for (int u = 0; u < G; u++) {
      const int st = min(s0 + u, nst - 1) * 32;  // past the slice: a repeat, never used
      bf[u] = *reinterpret_cast<const h8 *>(B + st);
#pragma unroll
      for (int e = 0; e < 2; e++) {
        gv[u][e] = reinterpret_cast<const float4 *>(Gm + st)[e];
        bv[u][e] = reinterpret_cast<const float4 *>(Bt + st)[e];
#pragma unroll
        for (int i = 0; i < TI; i++) xv[u][i][e] = reinterpret_cast<const float4 *>(X[i] + st)[e];
      }
    }
#pragma unroll
    for (int u = 0; u < G; u++) {
      if (s0 + u < nst) {
        const float gg[8] = {gv[u][0].x, gv[u][0].y, gv[u][0].z, gv[u][0].w, gv[u][1].x, gv[u][1].y, gv[u][1].z, gv[u][1].w};
        const float bb[8] = {bv[u][0].x, bv[u][0].y, bv[u][0].z, bv[u][0].w, bv[u][1].x, bv[u][1].y, bv[u][1].z, bv[u][1].w};
#pragma unroll
        for (int i = 0; i < TI; i++) {
          const float xx[8] = {xv[u][i][0].x, xv[u][i][0].y, xv[u][i][0].z, xv[u][i][0].w, xv[u][i][1].x, xv[u][i][1].y, xv[u][i][1].z, xv[u][i][1].w};
          h8 hi, lo;
#pragma unroll
          for (int e = 0; e < 8; e++) {
            const float o = ln_affine(xx[e], mean[i], inv[i], gg[e], bb[e]);  // enc_ln_kernel's expression
            hi[e] = (_Float16)o;
            lo[e] = (_Float16)(o - (float)hi[e]);
          }
          acc[i][0] = __builtin_amdgcn_mfma_f32_16x16x32_f16(bf[u], hi, acc[i][0], 0, 0, 0);  // C^T tile
          if constexpr (LO) acc[i][0] = __builtin_amdgcn_mfma_f32_16x16x32_f16(bf[u], lo, acc[i][0], 0, 0, 0);
        }
      }
    }
  }
  if constexpr (KS > 1) {
    if (wave > 0)
#pragma unroll
      for (int i = 0; i < TI; i++) part[wave - 1][i][lane] = acc[i][0];
    __syncthreads();
    if (wave > 0) return;
#pragma unroll
    for (int w = 0; w < KS - 1; w++)
#pragma unroll
      for (int i = 0; i < TI; i++) acc[i][0] += part[w][i][lane];
  }
  epilogue_direct<TI, 1, EPI>(p, acc, 0, n0, lane);
}

// K split per workgroup: 8 waves up to N = 2048, 4 above (16 measured slower
// at N = 1024: 8.8 against 6.0 us for the 1024 x 1024 two-plane product).
static inline int skinny_ks(int N) { return N <= 2048 ? 8 : 4; }

template <int EPI>
static int launch_skinny(fa_ctx *ctx, const GemmArgs &p, const char *label) {
  const int ks = skinny_ks(p.N);
  const int ti = p.M <= 16 ? 1 : 2;
  const char *se = getenv("FA_SKINNY_SPLIT");  // 0: one workgroup per 16 columns everywhere (read per call)
  const bool split_on = !(se && se[0] == '0');
  // N <= 2048 gives one workgroup per 16 columns only N / 16 <= 128 of the
  // chip's CUs: with two row tiles (17..32 rows, a batched stream pass) its K
  // range is split over kSkinnySplit workgroups instead.  Up to 16 rows the
  // second launch costs more than the extra CUs give (a single stream's pass),
  // and such passes keep the sums of one workgroup per 16 columns.
  const bool split = split_on && ti == 2 && !p.ln_x && p.skp && p.N <= kSkinnySplitMaxN && p.K % (32 * ks * kSkinnySplit) == 0 &&
                     p.skp_bytes >= skinny_split_bytes(p.N);
  ProfScope ps(ctx, label, !split);
  const dim3 grid(p.N / 16);
  if (p.ln_x) {  // A = LayerNorm(ln_x), built in the kernel
#define FA_SKL(TI, KS)                                                                                   \
  do {                                                                                                  \
    if (p.ln_lo)                                                                                        \
      FA_LAUNCH(ps, (gemm_skinny_ln_kernel<TI, KS, EPI, 1>), grid, dim3(64 * KS), 0, ctx->stream, p);  \
    else                                                                                                \
      FA_LAUNCH(ps, (gemm_skinny_ln_kernel<TI, KS, EPI, 0>), grid, dim3(64 * KS), 0, ctx->stream, p);  \
  } while (0)
    if (ti == 1) {
      if (ks == 4) FA_SKL(1, 4);
      else FA_SKL(1, 8);
    } else {
      if (ks == 4) FA_SKL(2, 4);
      else FA_SKL(2, 8);
    }
#undef FA_SKL
    return check_launch(ctx, label);
  }
#define FA_SK(TI, KS)                                                                                                        \
  do {                                                                                                                       \
    if (split) {                                                                                                             \
      const dim3 g2(p.N / 16, kSkinnySplit);                                                                                 \
      if (p.Alo)                                                                                                             \
        hipLaunchKernelGGL((gemm_skinny_kernel<TI, KS, EPI, 1, kSkinnySplit>), g2, dim3(64 * KS), 0, ctx->stream, p);       \
      else                                                                                                                   \
        hipLaunchKernelGGL((gemm_skinny_kernel<TI, KS, EPI, 0, kSkinnySplit>), g2, dim3(64 * KS), 0, ctx->stream, p);       \
      hipLaunchKernelGGL((gemm_skinny_split_sum_kernel<TI, kSkinnySplit, EPI>), grid, dim3(64), 0, ctx->stream, p);         \
    } else if (p.Alo) {                                                                                                      \
      FA_LAUNCH(ps, (gemm_skinny_kernel<TI, KS, EPI, 1>), grid, dim3(64 * KS), 0, ctx->stream, p);                         \
    } else {                                                                                                                 \
      FA_LAUNCH(ps, (gemm_skinny_kernel<TI, KS, EPI, 0>), grid, dim3(64 * KS), 0, ctx->stream, p);                         \
    }                                                                                                                        \
  } while (0)
  if (ti == 1) {
    if (ks == 4) FA_SK(1, 4);
    else FA_SK(1, 8);
  } else {
    if (ks == 4) FA_SK(2, 4);
    else FA_SK(2, 8);
  }
#undef FA_SK
  return check_launch(ctx, label);
}

// The skinny route takes f16 x f16 products of at most 32 rows with K a
// multiple of 32 x its K split, N a multiple of 16, 16-byte aligned operands.
static inline bool takes_skinny(const GemmArgs &p) {
  const char *e = getenv("FA_GEMM_SKINNY");
  if (e && e[0] == '0') return false;
  const int ks = skinny_ks(p.N);
  if (p.ln_x && (p.K != 1024 || p.Alo || ((uintptr_t)p.ln_x & 15) || ((uintptr_t)p.ln_g & 15) || ((uintptr_t)p.ln_b & 15))) return false;
  return p.allow_skinny && p.M <= 32 && p.akind == A_F16 && p.bkind == B_F16 && !p.vt && epi_of(p) != EPI_GENERIC && p.N % 16 == 0 && p.K % (32 * ks) == 0 &&
         p.lda % 8 == 0 && p.ldc % 8 == 0 && !((uintptr_t)p.A & 15) && !((uintptr_t)p.Alo & 15) && !((uintptr_t)p.B & 15) && !((uintptr_t)p.C & 15) &&
         !((uintptr_t)p.Clo & 15) && !((uintptr_t)p.add & 15) && p.ldadd % 4 == 0;
}

template <int AK, int BKND, int EPI>
static int launch_tile(fa_ctx *ctx, const GemmArgs &p, const char *label) {
  if constexpr (AK == A_F16 && BKND == B_F16 && EPI != EPI_GENERIC)
    if (takes_skinny(p)) return launch_skinny<EPI>(ctx, p, label);
  if (p.ln_x) return set_err(ctx, FA_E_UNSUPPORTED, "%s: a LayerNorm-folded A needs the skinny route (<= 32 rows, K = 1024)", label);
  if constexpr (AK == A_F16 && BKND == B_F16 && EPI != EPI_GENERIC) {
    if (p.Alo) {
      switch (pick_dma(ctx, p)) {
        case 0: return launch_dma<192, 256, 2, 4, 2, EPI, 1>(ctx, p, label);
        case 1: return launch_dma<192, 128, 4, 2, 2, EPI, 1>(ctx, p, label);
        case 2: return launch_dma<96, 256, 2, 4, 2, EPI, 1>(ctx, p, label);
        case 3: return launch_dma<128, 128, 2, 4, 3, EPI, 1>(ctx, p, label);
        case 4: return launch_dma<96, 128, 2, 4, 3, EPI, 1>(ctx, p, label);
        case 5: return launch_dma<192, 192, 2, 4, 2, EPI, 1>(ctx, p, label);
        default: return set_err(ctx, FA_E_UNSUPPORTED, "%s: lo plane needs N %% 128 == 0, K %% 64 == 0 and 16-byte aligned operands", label);
      }
    }
  }
  if constexpr (AK == A_F16 && BKND == B_F16) {  // also the ComputeContext's generic (act-then-add) epilogue
    switch (pick_dma(ctx, p)) {
      case 0: return launch_dma<192, 256, 2, 4, 2, EPI>(ctx, p, label);
      case 1: return launch_dma<192, 128, 4, 2, 3, EPI>(ctx, p, label);
      case 2: return launch_dma<128, 128, 2, 4, 4, EPI>(ctx, p, label);
      case 3: return launch_dma<96, 128, 2, 4, 4, EPI>(ctx, p, label);
      case 4: return launch_dma<192, 192, 2, 4, 3, EPI>(ctx, p, label);  // 48 KB stages: three fit
      default: break;
    }
  }
  if constexpr (AK == A_F16 && BKND == B_I8 && EPI != EPI_GENERIC) {
    if (p.Alo) switch (pick_dma(ctx, p)) {  // exact A planes against int8 weights
        case 0: return launch_dma<192, 256, 2, 4, 2, EPI, 1, 1>(ctx, p, label);
        case 1: return launch_dma<192, 128, 4, 2, 2, EPI, 1, 1>(ctx, p, label);
        case 2: return launch_dma<96, 256, 2, 4, 2, EPI, 1, 1>(ctx, p, label);
        case 3: return launch_dma<128, 128, 2, 4, 3, EPI, 1, 1>(ctx, p, label);
        case 4: return launch_dma<96, 128, 2, 4, 3, EPI, 1, 1>(ctx, p, label);
        case 5: return launch_dma<192, 192, 2, 4, 2, EPI, 1, 1>(ctx, p, label);
        default: return set_err(ctx, FA_E_UNSUPPORTED, "%s: lo plane needs N %% 128 == 0, K %% 64 == 0 and 16-byte aligned operands", label);
      }
    switch (pick_dma(ctx, p)) {  // int8 weights: same tile table, half the B bytes
        case 0: return launch_dma<192, 256, 2, 4, 2, EPI, 0, 1>(ctx, p, label);
        case 1: return launch_dma<192, 128, 2, 4, 3, EPI, 0, 1>(ctx, p, label);
        case 2: return launch_dma<128, 128, 2, 4, 4, EPI, 0, 1>(ctx, p, label);
        case 3: return launch_dma<96, 128, 2, 4, 4, EPI, 0, 1>(ctx, p, label);
        case 4: return launch_dma<192, 192, 2, 4, 3, EPI, 0, 1>(ctx, p, label);
        default: break;
      }
  }
  if constexpr (AK == A_F16 && BKND == B_I4 && EPI != EPI_GENERIC) {
    // symmetric group-32 with f16 scales (the encoder's int4 format): same tile
    // table, even stage counts (the scale sets alternate with the stages)
    // Nibble tiles are widened once per workgroup (WW) wherever the two f16
    // B tiles fit beside the stages: measured on MI355X at M = 192..3008, FF W2
    // 58.7 -> 51.0 us, FF W1 36.0 -> 32.3, q|k|v 29.2 -> 27.3, two-plane FF W2
    // 85.2 -> 72.5 (same bits). int8 stays per wave: its widening is cheaper
    // than the extra LDS write and read (FF W2 37.2 -> 42.1 us with WW).
    if (p.Alo && !p.bzp && !p.bscale_f32) switch (pick_dma(ctx, p)) {  // exact A planes (even stage counts)
        case 0: return launch_dma<192, 256, 2, 4, 2, EPI, 1, 2>(ctx, p, label);  // 176 KB with WW
        case 1: return launch_dma<192, 128, 4, 2, 2, EPI, 1, 2, 1>(ctx, p, label);
        case 2: return launch_dma<96, 256, 2, 4, 2, EPI, 1, 2, 1>(ctx, p, label);
        case 3: return launch_dma<128, 128, 2, 4, 2, EPI, 1, 2, 1>(ctx, p, label);
        case 4: return launch_dma<96, 128, 2, 4, 4, EPI, 1, 2, 1>(ctx, p, label);
        case 5: return launch_dma<192, 192, 2, 4, 2, EPI, 1, 2, 1>(ctx, p, label);
        default: return set_err(ctx, FA_E_UNSUPPORTED, "%s: lo plane needs N %% 128 == 0, K %% 64 == 0 and 16-byte aligned operands", label);
      }
    if (!p.Alo && !p.bzp && !p.bscale_f32) switch (pick_dma(ctx, p)) {
        case 0: return launch_dma<192, 256, 2, 4, 2, EPI, 0, 2, 1>(ctx, p, label);
        case 1: return launch_dma<192, 128, 2, 4, 2, EPI, 0, 2, 1>(ctx, p, label);
        case 2: return launch_dma<128, 128, 2, 4, 2, EPI, 0, 2, 1>(ctx, p, label);
        case 3: return launch_dma<96, 128, 2, 4, 2, EPI, 0, 2, 1>(ctx, p, label);
        case 4: return launch_dma<192, 192, 2, 4, 2, EPI, 0, 2, 1>(ctx, p, label);
        default: break;
      }
  }
  if (p.Alo) return set_err(ctx, FA_E_UNSUPPORTED, "%s: lo plane needs the f16 x f16 route", label);
  if constexpr (AK == A_F32 || EPI == EPI_GENERIC) {  // ComputeContext path: mid-size tiles
    const long t128 = (long)cdiv(p.M, 128) * cdiv(p.N, 128);
    if (t128 >= ctx->num_cu) return launch_cfg<128, 128, 2, 2, AK, BKND, EPI>(ctx, p, label);
    return launch_cfg<64, 128, 2, 2, AK, BKND, EPI>(ctx, p, label);
  } else {
    switch (pick_tile(ctx, p.M, p.N)) {
      case 0: return launch_cfg<256, 256, 2, 2, AK, BKND, EPI>(ctx, p, label);
      case 1: return launch_cfg<192, 256, 2, 2, AK, BKND, EPI>(ctx, p, label);
      case 2: return launch_cfg<256, 192, 2, 2, AK, BKND, EPI>(ctx, p, label);
      case 3: return launch_cfg<192, 192, 2, 2, AK, BKND, EPI>(ctx, p, label);
      case 4: return launch_cfg<256, 128, 2, 2, AK, BKND, EPI>(ctx, p, label);
      case 5: return launch_cfg<128, 256, 2, 2, AK, BKND, EPI>(ctx, p, label);
      case 6: return launch_cfg<192, 128, 2, 2, AK, BKND, EPI>(ctx, p, label);
      case 7: return launch_cfg<128, 128, 2, 2, AK, BKND, EPI>(ctx, p, label);
      case 8: return launch_cfg<192, 64, 2, 2, AK, BKND, EPI>(ctx, p, label);
      default: return launch_cfg<64, 128, 2, 2, AK, BKND, EPI>(ctx, p, label);
    }
  }
}

template <int AK, int BKND>
static int launch_kind(fa_ctx *ctx, const GemmArgs &p, const char *label) {
  switch (epi_of(p)) {
    case EPI_F32: return launch_tile<AK, BKND, EPI_F32>(ctx, p, label);
    case EPI_F16: return launch_tile<AK, BKND, EPI_F16>(ctx, p, label);
    case EPI_F16_SILU: return launch_tile<AK, BKND, EPI_F16_SILU>(ctx, p, label);
    case EPI_F16_RELU: return launch_tile<AK, BKND, EPI_F16_RELU>(ctx, p, label);
    case EPI_GLU: return launch_tile<AK, BKND, EPI_GLU>(ctx, p, label);
    case EPI_HILO_RELU: return launch_tile<AK, BKND, EPI_HILO_RELU>(ctx, p, label);
    default: return launch_tile<AK, BKND, EPI_GENERIC>(ctx, p, label);
  }
}

// Entry points of the quantised-weight translation units (A f16).
int gemm_launch_f16a_i8(fa_ctx *ctx, const GemmArgs &p, const char *label);
int gemm_launch_f16a_i4(fa_ctx *ctx, const GemmArgs &p, const char *label);

}  // namespace fa
