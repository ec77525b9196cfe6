// CPU execution of the library's kernel sources (test infrastructure).
//
// This header stands in for <hip/hip_runtime.h> when a .hip source is
// compiled as host C++ (tests/emu/build_emu.py): kernels become ordinary
// functions, and a launch runs every workgroup on the CPU, one workgroup at a
// time, each thread a fiber (emu_rt.cpp).  __syncthreads and the wave
// operations the kernels use (ballot, shfl_xor, readfirstlane) block their
// fiber until the threads (or the wave's lanes) that take part have arrived.
// __shared__ arrays become static storage: one workgroup runs at a time, so
// they are the workgroup's LDS.  Device memory is host memory from malloc,
// sized as asked, so AddressSanitizer sees every out-of-bounds access a
// kernel makes.  The HIP API calls are synchronous.
#pragma once
#include <cmath>
#include <cstddef>
#include <cstdint>
#include <cstdlib>
#include <cstring>
#include <functional>
#include <type_traits>
#include <utility>

// ── qualifiers ──
#define __global__
#define __device__
#define __host__
#define __shared__ static
#define __constant__ static
#define __forceinline__ inline __attribute__((always_inline))
#define __launch_bounds__(...)
#define __align__(n) __attribute__((aligned(n)))
#define HIP_SYMBOL(x) ((const void *)&(x))

struct dim3 {
  unsigned x = 1, y = 1, z = 1;
  constexpr dim3(unsigned a = 1, unsigned b = 1, unsigned c = 1) : x(a), y(b), z(c) {}
};

// ── vector types (HIP's layouts: 8- and 16-byte aligned structs) ──
struct alignas(8) float2 {
  float x, y;
};
struct alignas(16) float4 {
  float x, y, z, w;
};
struct alignas(8) uint2 {
  unsigned x, y;
};
struct alignas(16) uint4 {
  unsigned x, y, z, w;
};
struct alignas(8) int2 {
  int x, y;
};
struct alignas(16) int4 {
  int x, y, z, w;
};
inline float4 make_float4(float x, float y, float z, float w) { return float4{x, y, z, w}; }
inline float2 make_float2(float x, float y) { return float2{x, y}; }

// ── runtime types ──
typedef enum hipError_t {
  hipSuccess = 0,
  hipErrorInvalidValue = 1,
  hipErrorOutOfMemory = 2,
  hipErrorInvalidDevice = 101,
  hipErrorInvalidHandle = 400,
  hipErrorNotReady = 600,
  hipErrorLaunchFailure = 719,
} hipError_t;
typedef enum hipMemcpyKind {
  hipMemcpyHostToHost = 0,
  hipMemcpyHostToDevice = 1,
  hipMemcpyDeviceToHost = 2,
  hipMemcpyDeviceToDevice = 3,
  hipMemcpyDefault = 4,
} hipMemcpyKind;
struct ihipStream_t;
struct ihipEvent_t;
struct ihipGraph_t;
struct ihipGraphExec_t;
typedef ihipStream_t *hipStream_t;
typedef ihipEvent_t *hipEvent_t;
typedef ihipGraph_t *hipGraph_t;
typedef ihipGraphExec_t *hipGraphExec_t;
typedef enum hipStreamCaptureMode {
  hipStreamCaptureModeGlobal = 0,
  hipStreamCaptureModeThreadLocal = 1,
  hipStreamCaptureModeRelaxed = 2,
} hipStreamCaptureMode;
typedef enum hipFuncAttribute {
  hipFuncAttributeMaxDynamicSharedMemorySize = 8,
} hipFuncAttribute;
#define hipStreamNonBlocking 0x01
#define hipEventDisableTiming 0x02
#define hipHostMallocDefault 0x0
struct hipDeviceProp_t {
  char name[256];
  char gcnArchName[256];
  int multiProcessorCount;
  size_t totalGlobalMem;
  int warpSize;
  int maxThreadsPerBlock;
  size_t sharedMemPerBlock;
};

extern "C" {
hipError_t hipGetDeviceCount(int *n);
hipError_t hipSetDevice(int d);
hipError_t hipGetDeviceProperties(hipDeviceProp_t *p, int d);
hipError_t hipDeviceSynchronize(void);
hipError_t hipMalloc(void **p, size_t n);
hipError_t hipFree(void *p);
hipError_t hipHostMalloc(void **p, size_t n, unsigned int flags);
hipError_t hipHostFree(void *p);
hipError_t hipMemcpy(void *dst, const void *src, size_t n, hipMemcpyKind k);
hipError_t hipMemcpyAsync(void *dst, const void *src, size_t n, hipMemcpyKind k, hipStream_t s);
hipError_t hipMemsetAsync(void *dst, int v, size_t n, hipStream_t s);
hipError_t hipStreamCreateWithFlags(hipStream_t *s, unsigned int flags);
hipError_t hipStreamDestroy(hipStream_t s);
hipError_t hipStreamSynchronize(hipStream_t s);
hipError_t hipStreamWaitEvent(hipStream_t s, hipEvent_t e, unsigned int flags);
hipError_t hipEventCreate(hipEvent_t *e);
hipError_t hipEventCreateWithFlags(hipEvent_t *e, unsigned flags);
hipError_t hipEventDestroy(hipEvent_t e);
hipError_t hipEventRecord(hipEvent_t e, hipStream_t s);
hipError_t hipEventSynchronize(hipEvent_t e);
hipError_t hipEventElapsedTime(float *ms, hipEvent_t a, hipEvent_t b);
hipError_t hipGetSymbolAddress(void **dev, const void *sym);
hipError_t hipFuncSetAttribute(const void *f, hipFuncAttribute a, int v);
hipError_t hipStreamBeginCapture(hipStream_t s, hipStreamCaptureMode m);
hipError_t hipStreamEndCapture(hipStream_t s, hipGraph_t *g);
hipError_t hipGraphInstantiateWithFlags(hipGraphExec_t *x, hipGraph_t g, unsigned long long flags);
hipError_t hipGraphLaunch(hipGraphExec_t x, hipStream_t s);
hipError_t hipGraphDestroy(hipGraph_t g);
hipError_t hipGraphExecDestroy(hipGraphExec_t x);
hipError_t hipGetLastError(void);
const char *hipGetErrorString(hipError_t e);
}  // extern "C"

// ── execution of a launch (emu_rt.cpp) ──
namespace emu {
struct Thread {
  dim3 tid;
  int lane, wave;
};
extern dim3 g_block_idx, g_block_dim, g_grid_dim;
Thread &self();
void run_grid(dim3 grid, dim3 block, const std::function<void()> &body);
void barrier();
uint64_t wave_exchange_u64(uint64_t v, int src_lane_xor, bool ballot);
uint64_t wave_readlane(uint64_t v, int lane);
uint32_t wave_dpp(uint32_t v, int ctrl);
void wave_sync();
// 16x16 MFMA with kb values of A and B per lane (K = 4 kb): lane l holds
// A[l % 16][kb (l / 16) + j] and B[kb (l / 16) + j][l % 16], and receives
// D[4 (l / 16) + r][l % 16]
void wave_mfma_16x16(const float *a, const float *b, int kb, const float *c4, float *d4);
void *dyn_lds();
void check_uniform(uint64_t v, const char *what);
void dma16(const void *g, uint32_t lds_addr);
uint32_t lds_base_hi();
void report(const char *what);

void set_dyn_lds(size_t bytes);
// a stream under capture records its operations (replayed by hipGraphLaunch)
bool capturing(hipStream_t s);
void record(hipStream_t s, std::function<void()> op);
template <class K, class... A>
void launch(hipStream_t s, K k, dim3 g, dim3 b, size_t shm, A &&...a) {
  // arguments are copied when the launch is made, as a kernel's by-value
  // parameters are (a captured launch replays these copies)
  std::function<void()> op = [k, g, b, shm, args = std::tuple<std::decay_t<A>...>(std::forward<A>(a)...)]() mutable {
    set_dyn_lds(shm);
    run_grid(g, b, [&]() { std::apply([&](auto &...x) { k(x...); }, args); });
  };
  if (capturing(s))
    record(s, std::move(op));
  else
    op();
}
}  // namespace emu

#define hipLaunchKernelGGL(k, g, b, shm, s, ...) ::emu::launch((s), k, dim3(g), dim3(b), (size_t)(shm), ##__VA_ARGS__)

// ── built-in variables ──
#define threadIdx (::emu::self().tid)
#define blockIdx (::emu::g_block_idx)
#define blockDim (::emu::g_block_dim)
#define gridDim (::emu::g_grid_dim)

// ── device functions ──
inline void __syncthreads() { ::emu::barrier(); }
inline unsigned long long __ballot(int pred) { return ::emu::wave_exchange_u64(pred ? 1 : 0, 0, true); }
inline int __popcll(unsigned long long v) { return __builtin_popcountll(v); }
inline int __shfl_xor(int v, int m) { return (int)(uint32_t)::emu::wave_exchange_u64((uint32_t)v, m, false); }
inline unsigned __shfl_xor(unsigned v, int m) { return (unsigned)::emu::wave_exchange_u64(v, m, false); }
inline float __shfl_xor(float v, int m) {
  uint32_t u;
  std::memcpy(&u, &v, 4);
  u = (uint32_t)::emu::wave_exchange_u64(u, m, false);
  std::memcpy(&v, &u, 4);
  return v;
}
inline double __shfl_xor(double v, int m) {
  uint64_t u;
  std::memcpy(&u, &v, 8);
  u = ::emu::wave_exchange_u64(u, m, false);
  std::memcpy(&v, &u, 8);
  return v;
}
inline float __uint_as_float(unsigned u) {
  float f;
  std::memcpy(&f, &u, 4);
  return f;
}
inline unsigned __float_as_uint(float f) {
  unsigned u;
  std::memcpy(&u, &f, 4);
  return u;
}
template <class T>
inline T emu_readfirstlane(T v) {  // the kernels apply it to values every lane holds alike: checked
  ::emu::check_uniform((uint64_t)v, "readfirstlane of a value that differs between lanes");
  return v;
}
#define __builtin_amdgcn_readfirstlane(x) emu_readfirstlane(x)
#define __builtin_amdgcn_s_waitcnt(x) ((void)(x))
// raw buffer loads: reads past the resource's size return 0 (the hardware's
// range check), reported as a finding
struct emu_rsrc {
  const char *base;
  int bytes;
};
#define __amdgpu_buffer_rsrc_t emu_rsrc
inline emu_rsrc emu_make_rsrc(void *p, int stride, int bytes, int flags) {
  (void)stride;
  (void)flags;
  return emu_rsrc{(const char *)p, bytes};
}
#define __builtin_amdgcn_make_buffer_rsrc(p, s, n, f) emu_make_rsrc((p), (s), (n), (f))
inline uint32_t emu_buffer_load_b32(emu_rsrc r, int voff, int soff, int aux) {
  (void)aux;
  const long o = (long)voff + soff;
  if (o < 0 || o + 4 > r.bytes) {
    ::emu::report("raw buffer load outside its resource (returns 0 on the GPU)");
    return 0;
  }
  uint32_t v;
  std::memcpy(&v, r.base + o, 4);
  return v;
}
#define __builtin_amdgcn_raw_buffer_load_b32(r, v, s, a) emu_buffer_load_b32((r), (v), (s), (a))

// cross-lane: readlane, DPP lane swaps (quad_perm, row_mirror,
// row_half_mirror), wave barriers, and the 16x16x32 f16 MFMA (operands
// exchanged across the wave, products summed in k order in f32, as one
// instruction on the device; the device's internal summation may round
// differently)
template <class T>
inline T emu_readlane(T v, int lane) {
  return (T)::emu::wave_readlane((uint64_t)(uint32_t)v, lane);
}
#define __builtin_amdgcn_readlane(v, l) emu_readlane((v), (l))
inline int emu_update_dpp(int old, int src, int ctrl, int row_mask, int bank_mask, bool bound_ctrl) {
  (void)old;
  (void)row_mask;
  (void)bank_mask;
  (void)bound_ctrl;
  return (int)::emu::wave_dpp((uint32_t)src, ctrl);
}
#define __builtin_amdgcn_update_dpp(o, s, c, rm, bm, bc) emu_update_dpp((o), (s), (c), (rm), (bm), (bc))
#define __builtin_amdgcn_wave_barrier() ::emu::wave_sync()
#define __builtin_amdgcn_sched_barrier(x) ((void)(x))
#define __builtin_amdgcn_ballot_w64(p) __ballot(p)
#define __builtin_amdgcn_exp2f(x) exp2f(x)
// v_perm_b32: byte i of the result is byte sel_i of {src0 : src1} (src1 the
// low bytes); selectors 0x0c / >= 0x0d give 0x00 / 0xff
inline uint32_t emu_perm(uint32_t s0, uint32_t s1, uint32_t sel) {
  const uint64_t both = ((uint64_t)s0 << 32) | s1;
  uint32_t r = 0;
  for (int i = 0; i < 4; i++) {
    const uint32_t b = (sel >> (8 * i)) & 0xff;
    uint32_t v;
    if (b < 8) v = (uint32_t)(both >> (8 * b)) & 0xff;
    else if (b == 0x0c) v = 0x00;
    else v = 0xff;
    r |= v << (8 * i);
  }
  return r;
}
#define __builtin_amdgcn_perm(a, b, s) emu_perm((a), (b), (s))
typedef _Float16 emu_h8 __attribute__((ext_vector_type(8)));
typedef float emu_f4 __attribute__((ext_vector_type(4)));
inline emu_f4 emu_mfma_16x16x32_f16(emu_h8 a, emu_h8 b, emu_f4 c, int cbsz, int abid, int blgp) {
  (void)cbsz;
  (void)abid;
  (void)blgp;
  float af[8], bf[8], cin[4] = {c[0], c[1], c[2], c[3]}, d[4];
  for (int j = 0; j < 8; j++) {
    af[j] = (float)a[j];
    bf[j] = (float)b[j];
  }
  ::emu::wave_mfma_16x16(af, bf, 8, cin, d);
  return emu_f4{d[0], d[1], d[2], d[3]};
}
#define __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, x, y, z) emu_mfma_16x16x32_f16((a), (b), (c), (x), (y), (z))
inline emu_f4 emu_mfma_16x16x4_f32(float a, float b, emu_f4 c, int cbsz, int abid, int blgp) {
  (void)cbsz;
  (void)abid;
  (void)blgp;
  float cin[4] = {c[0], c[1], c[2], c[3]}, d[4];
  ::emu::wave_mfma_16x16(&a, &b, 1, cin, d);
  return emu_f4{d[0], d[1], d[2], d[3]};
}
#define __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, x, y, z) emu_mfma_16x16x4_f32((a), (b), (c), (x), (y), (z))
inline float __expf(float x) { return expf(x); }
inline float __fdividef(float a, float b) { return a / b; }
inline float rsqrtf(float x) { return 1.0f / sqrtf(x); }

inline int min(int a, int b) { return a < b ? a : b; }
inline int max(int a, int b) { return a > b ? a : b; }
inline long min(long a, long b) { return a < b ? a : b; }
inline long max(long a, long b) { return a > b ? a : b; }
inline unsigned min(unsigned a, unsigned b) { return a < b ? a : b; }
inline unsigned max(unsigned a, unsigned b) { return a > b ? a : b; }
