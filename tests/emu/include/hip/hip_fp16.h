// Stand-in for <hip/hip_fp16.h> in the CPU build of kernel sources
// (tests/emu): __half as the compiler's _Float16, converted with
// round-to-nearest-even like the device conversions.
#pragma once
typedef _Float16 __half;
inline __half __float2half_rn(float f) { return (__half)f; }
inline __half __float2half(float f) { return (__half)f; }
inline float __half2float(__half h) { return (float)h; }
inline unsigned short __half_as_ushort(__half h) {
  unsigned short u;
  __builtin_memcpy(&u, &h, 2);
  return u;
}
inline __half __ushort_as_half(unsigned short u) {
  __half h;
  __builtin_memcpy(&h, &u, 2);
  return h;
}
