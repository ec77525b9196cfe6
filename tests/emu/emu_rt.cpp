// CPU execution of kernel sources: the fiber scheduler behind
// tests/emu/include/hip/hip_runtime.h, and a synchronous host-memory HIP API.
//
// A launch runs its workgroups one after another.  Each thread of a workgroup
// is a fiber with its own stack; the scheduler resumes ready fibers in thread
// order.  A fiber that reaches __syncthreads or a wave operation parks; when
// every live thread of the workgroup is at the barrier (or every live lane of
// a wave at the same wave operation) they are released together, so a
// kernel's LDS hand-offs happen in an order its barriers allow.  A workgroup
// whose live threads all wait but can never be released (a barrier or wave
// operation under divergent control flow) is reported and the process aborts.
//
// Device allocations are malloc'd at their exact size and filled with 0xff
// bytes (NaN as f32), so kernels reading memory nobody wrote show up in
// results, and AddressSanitizer reports any access outside an allocation or
// outside a __shared__ array.
#include <hip/hip_runtime.h>

#include <sys/mman.h>

#include <chrono>
#include <cstdio>
#include <map>
#include <mutex>
#include <string>
#include <vector>

#if defined(__has_feature)
#if __has_feature(address_sanitizer)
#define EMU_ASAN 1
#endif
#endif
#ifdef EMU_ASAN
extern "C" void __sanitizer_start_switch_fiber(void **fake_stack_save, const void *bottom, size_t size);
extern "C" void __sanitizer_finish_switch_fiber(void *fake_stack_save, const void **bottom_old, size_t *size_old);
extern "C" void __asan_unpoison_memory_region(void const volatile *addr, size_t size);
#endif

// x86-64 context switch: saves the callee-saved registers on the current
// stack, stores the stack pointer in *save, switches to `to` and restores.
extern "C" void emu_swap(void **save, void *to);
asm(R"(
.text
.globl emu_swap
.type emu_swap,@function
emu_swap:
  pushq %rbp
  pushq %rbx
  pushq %r12
  pushq %r13
  pushq %r14
  pushq %r15
  movq %rsp, (%rdi)
  movq %rsi, %rsp
  popq %r15
  popq %r14
  popq %r13
  popq %r12
  popq %rbx
  popq %rbp
  ret
.size emu_swap, .-emu_swap
)");

namespace emu {

dim3 g_block_idx, g_block_dim, g_grid_dim;

namespace {
enum State { READY, AT_BARRIER, AT_WAVE, DONE };
enum WaveOp { W_BALLOT, W_SHFL, W_UNIFORM, W_READLANE, W_DPP, W_SYNC, W_MFMA };
constexpr size_t kStack = 128 * 1024;

struct Fiber {
  Thread t;
  State st = READY;
  void *sp = nullptr;
  char *stack = nullptr;
  WaveOp op = W_SHFL;
  uint64_t val = 0, res = 0;
  int arg = 0;
  const char *what = nullptr;
  float a[8], b[8];  // MFMA operands
  float c[4], d[4];
};

std::vector<Fiber> g_f;
int g_cur = -1;
void *g_sched_sp = nullptr;
const std::function<void()> *g_body = nullptr;
std::mutex g_launch_mu;
std::map<std::string, size_t> g_findings;
std::mutex g_find_mu;
#ifdef EMU_ASAN
void *g_sched_fake = nullptr;
const void *g_sched_bottom = nullptr;
size_t g_sched_size = 0;
#endif

void to_sched() {  // from a fiber
  Fiber &f = g_f[g_cur];
#ifdef EMU_ASAN
  void *fake = nullptr;
  __sanitizer_start_switch_fiber(f.st == DONE ? nullptr : &fake, g_sched_bottom, g_sched_size);
#endif
  emu_swap(&f.sp, g_sched_sp);
#ifdef EMU_ASAN
  __sanitizer_finish_switch_fiber(fake, &g_sched_bottom, &g_sched_size);
#endif
}

void trampoline() {
#ifdef EMU_ASAN
  __sanitizer_finish_switch_fiber(nullptr, &g_sched_bottom, &g_sched_size);
#endif
  (*g_body)();
  g_f[g_cur].st = DONE;
  to_sched();
  std::abort();  // a finished fiber is never resumed
}

void resume(int i) {  // from the scheduler
  g_cur = i;
#ifdef EMU_ASAN
  __sanitizer_start_switch_fiber(&g_sched_fake, g_f[i].stack, kStack);
#endif
  emu_swap(&g_sched_sp, g_f[i].sp);
#ifdef EMU_ASAN
  __sanitizer_finish_switch_fiber(g_sched_fake, nullptr, nullptr);
#endif
}

void start(Fiber &f) {
  if (!f.stack) {
    f.stack = (char *)mmap(nullptr, kStack, PROT_READ | PROT_WRITE, MAP_PRIVATE | MAP_ANONYMOUS | MAP_NORESERVE, -1, 0);
    if (f.stack == MAP_FAILED) {
      std::fprintf(stderr, "emu: cannot map a fiber stack\n");
      std::abort();
    }
  }
#ifdef EMU_ASAN
  // a finished fiber's last switch never returns, so the redzones of that
  // frame are still marked in the shadow of its stack: clear them for reuse
  __asan_unpoison_memory_region(f.stack, kStack);
#endif
  // initial frame: six callee-saved registers, then the return address
  // (trampoline); the top is 16-byte aligned, so trampoline starts with the
  // stack alignment of a called function
  uintptr_t top = ((uintptr_t)f.stack + kStack) & ~(uintptr_t)15;
  uint64_t *sp = (uint64_t *)(top - 64);
  for (int i = 0; i < 6; i++) sp[i] = 0;
  sp[6] = (uint64_t)(uintptr_t)&trampoline;
  sp[7] = 0;
  f.sp = sp;
  f.st = READY;
}

bool release_waves(int nthreads) {
  bool any = false;
  const int nw = (nthreads + 63) / 64;
  for (int w = 0; w < nw; w++) {
    const int l0 = w * 64, l1 = std::min(nthreads, l0 + 64);
    int live = 0, waiting = 0;
    for (int i = l0; i < l1; i++) {
      if (g_f[i].st == DONE) continue;
      live++;
      if (g_f[i].st == AT_WAVE) waiting++;
    }
    if (!live || waiting != live) continue;
    int first = l0;
    while (first < l1 && g_f[first].st != AT_WAVE) first++;
    const WaveOp op = g_f[first].op;
    uint64_t bits = 0;
    for (int i = l0; i < l1; i++)
      if (g_f[i].st == AT_WAVE && g_f[i].op != op) report("lanes of one wave at different wave operations");
    if (op == W_BALLOT)
      for (int i = l0; i < l1; i++)
        if (g_f[i].st == AT_WAVE && g_f[i].val) bits |= 1ull << (i - l0);
    if (op == W_MFMA) {  // D = C + A B: A[m][k] from lane m + 16 (k / kb), B[k][n] from lane n + 16 (k / kb)
      for (int i = l0; i < l1; i++)
        if (g_f[i].st != AT_WAVE) report("MFMA with lanes of the wave absent");
      for (int i = l0; i < l1; i++) {
        Fiber &f = g_f[i];
        if (f.st != AT_WAVE) continue;
        const int li = i - l0, n = li & 15, kb = f.arg;
        for (int r = 0; r < 4; r++) {
          const int m = 4 * (li >> 4) + r;
          float acc = 0.f;
          for (int k = 0; k < 4 * kb; k++) {
            const int la = l0 + m + 16 * (k / kb), lb = l0 + n + 16 * (k / kb);
            if (la < l1 && lb < l1) acc += g_f[la].a[k % kb] * g_f[lb].b[k % kb];
          }
          f.d[r] = f.c[r] + acc;
        }
      }
      for (int i = l0; i < l1; i++)
        if (g_f[i].st == AT_WAVE) g_f[i].st = READY;
      any = true;
      continue;
    }
    for (int i = l0; i < l1; i++) {
      Fiber &f = g_f[i];
      if (f.st != AT_WAVE) continue;
      if (op == W_SYNC) {
        f.res = 0;
      } else if (op == W_READLANE) {
        const int j = l0 + (f.arg & 63);
        f.res = (j < l1 && g_f[j].st == AT_WAVE) ? g_f[j].val : f.val;
      } else if (op == W_DPP) {
        const int li = i - l0, c = f.arg;
        int src = -1;
        if (c >= 0 && c <= 0xff) src = (li & ~3) | ((c >> (2 * (li & 3))) & 3);  // quad_perm
        else if (c == 0x140) src = (li & ~15) | (15 - (li & 15));              // row_mirror
        else if (c == 0x141) src = (li & ~7) | (7 - (li & 7));                 // row_half_mirror
        else report("DPP control the CPU build does not know");
        const int j = l0 + src;
        f.res = (src >= 0 && j < l1 && g_f[j].st == AT_WAVE) ? g_f[j].val : 0;
      } else if (op == W_BALLOT) {
        f.res = bits;
      } else if (op == W_SHFL) {
        const int j = l0 + ((i - l0) ^ f.arg);
        f.res = (j < l1 && g_f[j].st == AT_WAVE) ? g_f[j].val : f.val;  // an absent source lane: the lane's own value
      } else {
        for (int j = l0; j < l1; j++)
          if (g_f[j].st == AT_WAVE && g_f[j].val != f.val) {
            report(f.what);
            break;
          }
        f.res = f.val;
      }
    }
    for (int i = l0; i < l1; i++)
      if (g_f[i].st == AT_WAVE) g_f[i].st = READY;
    any = true;
  }
  return any;
}

void run_block(int nthreads) {
  for (int i = 0; i < nthreads; i++) start(g_f[i]);
  for (;;) {
    bool ran = false;
    for (int i = 0; i < nthreads; i++)
      if (g_f[i].st == READY) {
        resume(i);
        ran = true;
      }
    int live = 0, at_bar = 0;
    for (int i = 0; i < nthreads; i++) {
      if (g_f[i].st == DONE) continue;
      live++;
      if (g_f[i].st == AT_BARRIER) at_bar++;
    }
    if (!live) return;
    if (release_waves(nthreads)) continue;
    if (at_bar == live) {
      for (int i = 0; i < nthreads; i++)
        if (g_f[i].st == AT_BARRIER) g_f[i].st = READY;
      continue;
    }
    if (!ran) {
      std::fprintf(stderr, "emu: workgroup (%u,%u,%u) cannot proceed: %d live threads, %d at a barrier, the rest at wave operations "
                   "that part of their wave never reaches\n", g_block_idx.x, g_block_idx.y, g_block_idx.z, live, at_bar);
      std::abort();
    }
  }
}
}  // namespace

Thread &self() { return g_f[g_cur].t; }

void run_grid(dim3 grid, dim3 block, const std::function<void()> &body) {
  std::lock_guard<std::mutex> lk(g_launch_mu);
  const int nt = (int)(block.x * block.y * block.z);
  if (nt <= 0 || nt > 1024) {
    std::fprintf(stderr, "emu: block of %d threads\n", nt);
    std::abort();
  }
  if ((int)g_f.size() < nt) g_f.resize(nt);
  for (int i = 0; i < nt; i++) {
    g_f[i].t.tid = dim3(i % block.x, (i / block.x) % block.y, i / (block.x * block.y));
    g_f[i].t.lane = i & 63;
    g_f[i].t.wave = i >> 6;
  }
  g_grid_dim = grid;
  g_block_dim = block;
  g_body = &body;
  for (unsigned z = 0; z < grid.z; z++)
    for (unsigned y = 0; y < grid.y; y++)
      for (unsigned x = 0; x < grid.x; x++) {
        g_block_idx = dim3(x, y, z);
        run_block(nt);
      }
  g_body = nullptr;
  g_cur = -1;
}

void barrier() {
  g_f[g_cur].st = AT_BARRIER;
  to_sched();
}

uint64_t wave_exchange_u64(uint64_t v, int arg, bool ballot) {
  Fiber &f = g_f[g_cur];
  f.st = AT_WAVE;
  f.op = ballot ? W_BALLOT : W_SHFL;
  f.val = v;
  f.arg = arg;
  to_sched();
  return g_f[g_cur].res;
}

static uint64_t collective(WaveOp op, uint64_t v, int arg) {
  Fiber &f = g_f[g_cur];
  f.st = AT_WAVE;
  f.op = op;
  f.val = v;
  f.arg = arg;
  to_sched();
  return g_f[g_cur].res;
}
uint64_t wave_readlane(uint64_t v, int lane) { return collective(W_READLANE, v, lane); }
uint32_t wave_dpp(uint32_t v, int ctrl) { return (uint32_t)collective(W_DPP, v, ctrl); }
void wave_sync() { (void)collective(W_SYNC, 0, 0); }
void wave_mfma_16x16(const float *a, const float *b, int kb, const float *c4, float *d4) {
  Fiber &f = g_f[g_cur];
  std::memcpy(f.a, a, 4 * kb);
  std::memcpy(f.b, b, 4 * kb);
  std::memcpy(f.c, c4, 16);
  (void)collective(W_MFMA, 0, kb);
  std::memcpy(d4, g_f[g_cur].d, 16);
}

// dynamic LDS (extern __shared__): one buffer per launch, of the launch's size
static void *g_dyn = nullptr;
void set_dyn_lds(size_t bytes) {
  std::free(g_dyn);
  const size_t n = (bytes + 15) & ~(size_t)15;
  g_dyn = std::aligned_alloc(16, n ? n : 16);
  std::memset(g_dyn, 0xff, n ? n : 16);
}
void *dyn_lds() { return g_dyn; }

void check_uniform(uint64_t v, const char *what) {
  Fiber &f = g_f[g_cur];
  f.st = AT_WAVE;
  f.op = W_UNIFORM;
  f.val = v;
  f.what = what;
  to_sched();
}

// global_load_lds_dwordx4: each lane copies 16 bytes from its address to LDS
// at M0 + lane * 16.  LDS addresses are the low 32 bits of a __shared__
// array's host address; the high bits are those of this library's static data.
static char g_anchor;
uint32_t lds_base_hi() { return (uint32_t)((uintptr_t)&g_anchor >> 32); }
void dma16(const void *g, uint32_t lds_addr) {
  char *dst = (char *)(((uintptr_t)lds_base_hi() << 32) | lds_addr) + self().lane * 16;
  const long dist = (long)((uintptr_t)dst - (uintptr_t)&g_anchor);
  if (dist < -(64L << 20) || dist > (64L << 20)) {
    std::fprintf(stderr, "emu: LDS address 0x%x does not map to this library's static data\n", lds_addr);
    std::abort();
  }
  std::memcpy(dst, g, 16);
}

void report(const char *what) {
  std::lock_guard<std::mutex> lk(g_find_mu);
  g_findings[what]++;
}

}  // namespace emu

// ── synchronous HIP API on host memory ──
struct ihipStream_t {
  int flags;
  bool capturing = false;
  std::vector<std::function<void()>> ops;
};
struct ihipGraph_t {
  std::vector<std::function<void()>> ops;
};
struct ihipGraphExec_t {
  std::vector<std::function<void()>> ops;
};
namespace emu {
bool capturing(hipStream_t s) { return s && s->capturing; }
void record(hipStream_t s, std::function<void()> op) { s->ops.push_back(std::move(op)); }
}  // namespace emu
struct ihipEvent_t {
  std::chrono::steady_clock::time_point t;
  bool recorded = false;
};
static hipError_t g_last = hipSuccess;

hipError_t hipGetDeviceCount(int *n) {
  *n = 1;
  return hipSuccess;
}
hipError_t hipSetDevice(int d) { return d == 0 ? hipSuccess : hipErrorInvalidDevice; }
hipError_t hipGetDeviceProperties(hipDeviceProp_t *p, int d) {
  if (d != 0) return hipErrorInvalidDevice;
  std::memset(p, 0, sizeof *p);
  std::snprintf(p->name, sizeof p->name, "CPU execution of kernel sources");
  std::snprintf(p->gcnArchName, sizeof p->gcnArchName, "gfx950:sramecc+:xnack-");
  p->multiProcessorCount = 256;
  p->totalGlobalMem = 288ull << 30;
  p->warpSize = 64;
  p->maxThreadsPerBlock = 1024;
  p->sharedMemPerBlock = 160 * 1024;
  return hipSuccess;
}
hipError_t hipDeviceSynchronize(void) { return hipSuccess; }
hipError_t hipMalloc(void **p, size_t n) {
  *p = std::malloc(n ? n : 1);
  if (!*p) return hipErrorOutOfMemory;
  std::memset(*p, 0xff, n);
  return hipSuccess;
}
hipError_t hipFree(void *p) {
  std::free(p);
  return hipSuccess;
}
hipError_t hipHostMalloc(void **p, size_t n, unsigned int) {
  *p = std::calloc(1, n ? n : 1);
  return *p ? hipSuccess : hipErrorOutOfMemory;
}
hipError_t hipHostFree(void *p) {
  std::free(p);
  return hipSuccess;
}
hipError_t hipMemcpy(void *dst, const void *src, size_t n, hipMemcpyKind) {
  if (n) std::memmove(dst, src, n);
  return hipSuccess;
}
hipError_t hipMemcpyAsync(void *dst, const void *src, size_t n, hipMemcpyKind k, hipStream_t s) {
  if (emu::capturing(s)) {
    emu::record(s, [=]() { (void)hipMemcpy(dst, src, n, k); });
    return hipSuccess;
  }
  return hipMemcpy(dst, src, n, k);
}
hipError_t hipMemsetAsync(void *dst, int v, size_t n, hipStream_t s) {
  if (emu::capturing(s)) {
    emu::report("hipMemsetAsync recorded into a captured graph");
    emu::record(s, [=]() { std::memset(dst, v, n); });
    return hipSuccess;
  }
  if (n) std::memset(dst, v, n);
  return hipSuccess;
}
hipError_t hipFuncSetAttribute(const void *, hipFuncAttribute, int) { return hipSuccess; }
hipError_t hipStreamBeginCapture(hipStream_t s, hipStreamCaptureMode) {
  if (!s || s->capturing) return hipErrorInvalidValue;
  s->capturing = true;
  s->ops.clear();
  return hipSuccess;
}
hipError_t hipStreamEndCapture(hipStream_t s, hipGraph_t *g) {
  if (!s || !s->capturing) return hipErrorInvalidValue;
  s->capturing = false;
  *g = new ihipGraph_t{std::move(s->ops)};
  s->ops.clear();
  return hipSuccess;
}
hipError_t hipGraphInstantiateWithFlags(hipGraphExec_t *x, hipGraph_t g, unsigned long long) {
  *x = new ihipGraphExec_t{g->ops};
  return hipSuccess;
}
hipError_t hipGraphLaunch(hipGraphExec_t x, hipStream_t s) {
  if (emu::capturing(s)) return hipErrorInvalidValue;
  for (auto &op : x->ops) op();
  return hipSuccess;
}
hipError_t hipGraphDestroy(hipGraph_t g) {
  delete g;
  return hipSuccess;
}
hipError_t hipGraphExecDestroy(hipGraphExec_t x) {
  delete x;
  return hipSuccess;
}
hipError_t hipStreamCreateWithFlags(hipStream_t *s, unsigned int flags) {
  *s = new ihipStream_t{(int)flags};
  return hipSuccess;
}
hipError_t hipStreamDestroy(hipStream_t s) {
  delete s;
  return hipSuccess;
}
hipError_t hipStreamSynchronize(hipStream_t) { return hipSuccess; }
hipError_t hipStreamWaitEvent(hipStream_t, hipEvent_t, unsigned int) { return hipSuccess; }
hipError_t hipEventCreate(hipEvent_t *e) {
  *e = new ihipEvent_t();
  return hipSuccess;
}
hipError_t hipEventCreateWithFlags(hipEvent_t *e, unsigned) { return hipEventCreate(e); }
hipError_t hipEventDestroy(hipEvent_t e) {
  delete e;
  return hipSuccess;
}
hipError_t hipEventRecord(hipEvent_t e, hipStream_t s) {
  if (emu::capturing(s)) return hipSuccess;
  e->t = std::chrono::steady_clock::now();
  e->recorded = true;
  return hipSuccess;
}
hipError_t hipEventSynchronize(hipEvent_t) { return hipSuccess; }
hipError_t hipEventElapsedTime(float *ms, hipEvent_t a, hipEvent_t b) {
  if (!a->recorded || !b->recorded) return hipErrorNotReady;
  *ms = std::chrono::duration<float, std::milli>(b->t - a->t).count();
  return hipSuccess;
}
hipError_t hipGetSymbolAddress(void **dev, const void *sym) {  // a __device__ array is host static data here
  *dev = const_cast<void *>(sym);
  return sym ? hipSuccess : hipErrorInvalidValue;
}
hipError_t hipGetLastError(void) {
  hipError_t e = g_last;
  g_last = hipSuccess;
  return e;
}
const char *hipGetErrorString(hipError_t e) { return e == hipSuccess ? "no error" : "emulation error"; }

// Findings that are not faults on the GPU (reads past a buffer resource,
// non-uniform readfirstlane operands, lanes at different wave operations):
// "what count" per line into buf; returns the number of kinds.
extern "C" int emu_findings(char *buf, int cap) {
  std::lock_guard<std::mutex> lk(emu::g_find_mu);
  std::string s;
  for (const auto &f : emu::g_findings) s += f.first + " " + std::to_string(f.second) + "\n";
  if (buf && cap > 0) std::snprintf(buf, cap, "%s", s.c_str());
  return (int)emu::g_findings.size();
}
