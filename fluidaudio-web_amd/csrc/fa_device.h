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

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
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
