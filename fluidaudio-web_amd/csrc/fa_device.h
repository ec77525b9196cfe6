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

}  // namespace fa
