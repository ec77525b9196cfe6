// Stand-in for <hip/hip_ext.h> in the CPU build of kernel sources
// (tests/emu): an extended launch records its two events around the launch.
#pragma once
#include "hip_runtime.h"
#define hipExtLaunchKernelGGL(k, g, b, shm, s, e0, e1, flags, ...)        \
  do {                                                                    \
    if (e0) (void)hipEventRecord((e0), (s));                              \
    ::emu::launch((s), k, dim3(g), dim3(b), (size_t)(shm), ##__VA_ARGS__); \
    if (e1) (void)hipEventRecord((e1), (s));                              \
  } while (0)
