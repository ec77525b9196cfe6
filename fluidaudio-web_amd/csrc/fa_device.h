// Device-side helpers shared by the kernel translation units (gfx950, wave64).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace fa {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef float f4 __attribute__((ext_vector_type(4)));

// Fused activations, codes of src/gpu/kernels/actf.js:24; formulas of actf.js:5-22.
__device__ __forceinline__ float act_apply(float x, int a) {
  switch (a) {
    case 1: {
      float t = 0.7978845608028654f * (x + 0.044715f * x * x * x);
      t = fminf(fmaxf(t, -20.f), 20.f);
      return 0.5f * x * (1.f + tanhf(t));
    }
    case 2: return tanhf(fminf(fmaxf(x, -20.f), 20.f));
    case 3: return fmaxf(x, 0.f);
    case 4: return x / (1.f + __expf(-fminf(fmaxf(x, -30.f), 30.f)));
    case 5: {
      float z = x * 0.70710678118654752f;
      float t = 1.f / (1.f + 0.3275911f * fabsf(z));
      float y = 1.f - (((((1.061405429f * t - 1.453152027f) * t) + 1.421413741f) * t - 0.284496736f) * t + 0.254829592f) * t * __expf(-z * z);
      return 0.5f * x * (1.f + (z >= 0.f ? y : -y));
    }
    default: return x;
  }
}

__device__ __forceinline__ float silu_f(float x) { return x / (1.f + __expf(-fminf(fmaxf(x, -30.f), 30.f))); }

// Cross-lane reductions with DPP (VALU-latency lane swaps) instead of
// ds_bpermute round trips.  gfx9 DPP controls: quad_perm [1,0,3,2] = 0xB1,
// quad_perm [2,3,0,1] = 0x4E, row_half_mirror = 0x141 (lane i <-> 7-i within
// 8), row_mirror = 0x140 (lane i <-> 15-i within 16).  After the four steps
// every lane of a 16-lane row holds the row's reduction.
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ float row16_sum(float v) {
  v += dpp_f<0xB1>(v);
  v += dpp_f<0x4E>(v);
  v += dpp_f<0x141>(v);
  v += dpp_f<0x140>(v);
  return v;
}
__device__ __forceinline__ float row16_max(float v) {
  v = fmaxf(v, dpp_f<0xB1>(v));
  v = fmaxf(v, dpp_f<0x4E>(v));
  v = fmaxf(v, dpp_f<0x141>(v));
  v = fmaxf(v, dpp_f<0x140>(v));
  return v;
}
// Whole-wavefront reductions: rows by DPP, then the four row results read
// out of lanes 0, 16, 32, 48 (the result is wave-uniform).
__device__ __forceinline__ float wave_sum(float v) {
  v = row16_sum(v);
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 0)) +
         __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 16)) +
         __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 32)) +
         __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 48));
}
__device__ __forceinline__ float wave_max(float v) {
  v = row16_max(v);
  const float a = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 0));
  const float b = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 16));
  const float c = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 32));
  const float d = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 48));
  return fmaxf(fmaxf(a, b), fmaxf(c, d));
}

// Map a linear block id onto tiles so each of the 8 XCDs (which receive block
// ids round-robin) works on one contiguous run of tiles: neighbours share A
// or B panels in that XCD's L2.  Bijective for any tile count.
__device__ __forceinline__ int xcd_remap(int bid, int n) {
  const int q = n >> 3, r = n & 7;
  const int x = bid & 7, local = bid >> 3;
  const int base = x < r ? x * (q + 1) : r * (q + 1) + (x - r) * q;
  return base + local;
}

// int8 weights -> f16 pairs, exactly: with x = w ^ 0x80808080 each byte is
// b + 128, and the f16 with bits 0x64XX is 1024 + XX, so two byte_perms and a
// packed f16 subtract of 1152 give b for four bytes.
__device__ __forceinline__ h8 i8x8_to_h8(uint2 w) {
  const uint32_t x0 = w.x ^ 0x80808080u, x1 = w.y ^ 0x80808080u;
  const h2 off = h2{(_Float16)1152.f, (_Float16)1152.f};
  const h2 a = __builtin_bit_cast(h2, __builtin_amdgcn_perm(0x64646464u, x0, 0x04010400u)) - off;
  const h2 b = __builtin_bit_cast(h2, __builtin_amdgcn_perm(0x64646464u, x0, 0x04030402u)) - off;
  const h2 c = __builtin_bit_cast(h2, __builtin_amdgcn_perm(0x64646464u, x1, 0x04010400u)) - off;
  const h2 d = __builtin_bit_cast(h2, __builtin_amdgcn_perm(0x64646464u, x1, 0x04030402u)) - off;
  return h8{a[0], a[1], b[0], b[1], c[0], c[1], d[0], d[1]};
}

// 8 int4 weights (low nibble = even k) of one group-32 block -> f16
// (q - 8) * s, rounded once: nibbles are placed under an 0x64 high byte
// (f16 1024 + q), 1032 is subtracted exactly and the packed f16 multiply by
// the block scale rounds the exact product -- the value the register-staged
// route computes in f32 and rounds.
__device__ __forceinline__ h8 i4x8_to_h8(uint32_t u, _Float16 s) {
  const uint32_t lo = u & 0x0F0F0F0Fu, hi = (u >> 4) & 0x0F0F0F0Fu;
  const h2 off = h2{(_Float16)1032.f, (_Float16)1032.f}, sc = h2{s, s};
  const h2 a = (__builtin_bit_cast(h2, __builtin_amdgcn_perm(hi, lo, 0x0C040C00u) | 0x64006400u) - off) * sc;
  const h2 b = (__builtin_bit_cast(h2, __builtin_amdgcn_perm(hi, lo, 0x0C050C01u) | 0x64006400u) - off) * sc;
  const h2 c = (__builtin_bit_cast(h2, __builtin_amdgcn_perm(hi, lo, 0x0C060C02u) | 0x64006400u) - off) * sc;
  const h2 d = (__builtin_bit_cast(h2, __builtin_amdgcn_perm(hi, lo, 0x0C070C03u) | 0x64006400u) - off) * sc;
  return h8{a[0], a[1], b[0], b[1], c[0], c[1], d[0], d[1]};
}

}  // namespace fa
