// Launch audit: a host-only stand-in for the HIP runtime entry points that
// libfa_hip.so calls, linked with the library's own objects into a test build
// (tests/audit/build_audit.py) so that the library's host code -- window
// planning, workspace sizing, graph capture and replay, pools, profiler,
// stream lanes -- runs on a machine without a GPU.  Kernels are not executed.
// Every call is checked instead:
//   * device memory comes from one reserved address range and is never
//     reused, so a pointer into a freed block is always recognised;
//   * each kernel launch's arguments are read with the kernel's own argument
//     layout (offsets, sizes and kinds from the code object's metadata, passed
//     in as a table), and every 8-byte word of an argument that falls inside
//     the device range must lie inside a live allocation -- at launch, and
//     again at every replay of a captured graph;
//   * block sizes are checked against the kernel's maximum flat workgroup
//     size and its static LDS against the CU's 160 KB, grid dims against the
//     hardware limits;
//   * streams, events, graphs and graph executables are checked for use after
//     destruction, events for elapsed-time queries before being recorded, and
//     graph launches for executables destroyed or never instantiated;
//   * ordering between streams: every stream, event and the host thread keep
//     a vector clock (stream order, event record / wait, stream / event /
//     device synchronisation, synchronous copies on the null stream, hipFree
//     as a device synchronisation), and every byte range a kernel (from its
//     extent model), copy or fill touches is checked against the earlier
//     accesses to the same block: a write and another access to overlapping
//     bytes from two streams with no happens-before path between them is a
//     race.  All library streams are non-blocking, so the null stream is
//     ordered with none of them.
// Violations are collected and read back with audit_report().  The contents
// of device memory are whatever the host wrote (kernels never run), so a
// readback sees zeros or uploaded data.
#define __HIP_PLATFORM_AMD__ 1
#include <hip/hip_runtime_api.h>
#include <sys/mman.h>
#include <cxxabi.h>
#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <cstdint>
#include <map>
#include <mutex>
#include <string>
#include <vector>
#include <fstream>
#include <sstream>

namespace {

std::mutex &mu() { static std::mutex *m = new std::mutex(); return *m; }
#define g_mu mu()
std::vector<std::string> &viol() { static auto *v = new std::vector<std::string>(); return *v; }
#define g_viol viol()
size_t g_launches = 0, g_replays = 0, g_replayed_launches = 0, g_allocs = 0;
// failure injection (tests of error paths): the allocation / launch after this
// many more successful ones fails once (-1: off)
long g_fail_alloc_after = -1, g_fail_launch_after = -1;

void violation(const std::string &s) {
  if (g_viol.size() < 1000) g_viol.push_back(s);
}

// ── device memory: one reserved range, bump allocation, never reused ──
constexpr size_t kReserve = 1ull << 40;  // 1 TB of address space, committed on touch
char *g_base = nullptr;
size_t g_top = 0;
struct Block {
  size_t size;
  bool live;
  std::string what;
};
std::map<uintptr_t, Block> &blocks() { static auto *m = new std::map<uintptr_t, Block>(); return *m; }  // start -> block
#define g_blocks blocks()

void heap_init() {
  if (g_base) return;
  void *p = mmap(nullptr, kReserve, PROT_READ | PROT_WRITE, MAP_PRIVATE | MAP_ANONYMOUS | MAP_NORESERVE, -1, 0);
  if (p == MAP_FAILED) {
    std::fprintf(stderr, "launch audit: cannot reserve the device range\n");
    std::abort();
  }
  g_base = (char *)p;
}
bool in_range(uintptr_t v) { return g_base && v >= (uintptr_t)g_base && v < (uintptr_t)g_base + g_top; }
// the block holding address v (live or freed), or null
const std::pair<const uintptr_t, Block> *block_of(uintptr_t v) {
  auto it = g_blocks.upper_bound(v);
  if (it == g_blocks.begin()) return nullptr;
  --it;
  if (v < it->first + it->second.size) return &*it;
  return nullptr;
}
void *dev_alloc(size_t n, const char *what) {
  heap_init();
  const size_t a = (g_top + 4095) & ~(size_t)4095;  // page-aligned: every block starts on its own page
  if (a + n + 4096 > kReserve) return nullptr;
  g_top = a + (n ? n : 1) + 4096;                   // one guard page between blocks
  g_blocks[(uintptr_t)g_base + a] = Block{n ? n : 1, true, what};
  g_allocs++;
  return g_base + a;
}

// ── kernels: names from registration, argument layouts from the table ──
struct Arg {
  int offset, size;
  bool pointer;  // global_buffer
  bool hidden;
};
struct KernelInfo {
  std::string name, pretty;
  std::vector<Arg> args;
  int max_threads = 1024, lds = 0, scratch = 0;
  bool known = false;
};
std::map<const void *, KernelInfo> &kernels() { static auto *m = new std::map<const void *, KernelInfo>(); return *m; }  // host stub -> info
#define g_kernels kernels()
std::map<std::string, KernelInfo> &table() { static auto *m = new std::map<std::string, KernelInfo>(); return *m; }  // mangled name -> layout
#define g_table table()
bool g_table_loaded = false;
std::map<const void *, std::pair<size_t, void *>> &vars() { static auto *m = new std::map<const void *, std::pair<size_t, void *>>(); return *m; }  // host shadow -> (size, device copy)
#define g_vars vars()

void load_table() {
  if (g_table_loaded) return;
  g_table_loaded = true;
  const char *path = std::getenv("FA_AUDIT_KERNARGS");
  if (!path) {
    violation("FA_AUDIT_KERNARGS is not set: kernel argument layouts unknown");
    return;
  }
  std::ifstream f(path);
  // line: name max_threads lds scratch nargs (offset size kind)...
  std::string line;
  while (std::getline(f, line)) {
    std::istringstream is(line);
    KernelInfo k;
    int na = 0;
    is >> k.name >> k.max_threads >> k.lds >> k.scratch >> na;
    for (int i = 0; i < na; i++) {
      Arg a;
      std::string kind;
      is >> a.offset >> a.size >> kind;
      a.pointer = kind == "global_buffer";
      a.hidden = kind.rfind("hidden_", 0) == 0;
      k.args.push_back(a);
    }
    k.known = true;
    g_table[k.name] = k;
  }
}

std::string demangle(const char *m) {
  int st = 0;
  char *d = abi::__cxa_demangle(m, nullptr, nullptr, &st);
  std::string s = (st == 0 && d) ? d : m;
  std::free(d);
  return s;
}

// ── opaque handles: never freed, so use after destruction is recognised ──
enum Kind { K_STREAM = 1, K_EVENT, K_GRAPH, K_EXEC };
struct Launch {
  const KernelInfo *k;
  std::vector<std::vector<char>> args;
  dim3 grid, block;
};
struct Op {  // a captured operation
  int type;  // 0 kernel, 1 memcpy, 2 memset
  Launch l;
  const void *p0 = nullptr, *p1 = nullptr;
  size_t bytes = 0;
};
using VClock = std::vector<uint64_t>;
struct Handle {
  int kind;
  int sid = 0;  // streams: index of the stream's clock (0 = the null stream)
  bool blocking = false;  // streams created without hipStreamNonBlocking
  VClock vc;    // events: the recording stream's clock at the record
  bool live = true;
  bool recorded = false;   // events
  bool capturing = false;  // streams
  std::vector<Op> ops;     // streams under capture, graphs, executables
};
std::vector<Handle *> &handles() { static auto *v = new std::vector<Handle *>(); return *v; }
#define g_handles handles()
std::vector<VClock> &stream_clocks() { static auto *v = new std::vector<VClock>(1); return *v; }  // [sid]
std::vector<char> &stream_blocking() { static auto *v = new std::vector<char>(1, 0); return *v; }  // [sid]
Handle *new_handle(int kind) {
  Handle *h = new Handle();
  h->kind = kind;
  if (kind == K_STREAM) {
    h->sid = (int)stream_clocks().size();
    stream_clocks().emplace_back();
    stream_blocking().push_back(0);
  }
  g_handles.push_back(h);
  return h;
}
bool check_handle(const void *p, int kind, const char *api, bool null_ok) {
  if (!p) {
    if (!null_ok) violation(std::string(api) + ": null handle");
    return null_ok;
  }
  const Handle *h = (const Handle *)p;
  bool found = false;
  for (Handle *x : g_handles)
    if (x == h) found = true;
  if (!found || h->kind != kind) {
    violation(std::string(api) + ": not a handle of the right kind");
    return false;
  }
  if (!h->live) {
    violation(std::string(api) + ": handle used after destruction");
    return false;
  }
  return true;
}

// check one device address used by an operation
void check_addr(uintptr_t v, const std::string &who, bool must) {
  if (!v) return;
  if (!in_range(v)) {
    if (must) violation(who + ": pointer outside device memory");
    return;
  }
  const auto *b = block_of(v);
  if (!b) {
    violation(who + ": pointer into a guard page (past the end of a block)");
    return;
  }
  if (!b->second.live) violation(who + ": pointer into a freed block (" + b->second.what + ")");
}
void check_span(const void *p, size_t n, const std::string &who) {
  const uintptr_t v = (uintptr_t)p;
  if (!in_range(v) || !n) return;
  const auto *b = block_of(v);
  if (!b) {
    violation(who + ": span starts outside any block");
    return;
  }
  if (!b->second.live) violation(who + ": span in a freed block (" + b->second.what + ")");
  if (v + n > b->first + b->second.size) violation(who + ": span of " + std::to_string(n) + " bytes runs past the end of its block");
}

// Pointer arguments must point into live blocks.  By-value aggregates are
// scanned word by word only for kernels without an extent model: a struct's
// padding is not initialised, so a word that joins an int field to padding
// holding half of an old pointer can read as an address; a kernel with a
// model has the fields it uses checked by the model instead.
void check_launch_args(const Launch &l, const char *when, bool scan_aggregates) {
  const KernelInfo &k = *l.k;
  const std::string who = std::string(when) + " " + k.pretty;
  for (size_t i = 0; i < l.args.size(); i++) {
    const std::vector<char> &a = l.args[i];
    const Arg &m = k.args[i];
    if (!m.pointer && !scan_aggregates && a.size() > 8) continue;
    for (size_t o = 0; o + 8 <= a.size(); o += 8) {
      uint64_t v;
      std::memcpy(&v, a.data() + o, 8);
      check_addr(v, who + " arg " + std::to_string(i), m.pointer && o == 0);
    }
  }
}

// ── ordering between streams: vector clocks and per-block access lists ──
VClock g_host;  // what the host thread has waited for
void vc_join(VClock &a, const VClock &b) {
  if (a.size() < b.size()) a.resize(b.size(), 0);
  for (size_t i = 0; i < b.size(); i++)
    if (b[i] > a[i]) a[i] = b[i];
}
bool vc_covers(const VClock &v, int sid, uint64_t clk) { return (size_t)sid < v.size() && v[sid] >= clk; }
int stream_sid(hipStream_t s) { return s ? ((Handle *)s)->sid : 0; }
// One operation queued on a stream: it follows everything the host has waited
// for and everything earlier on its stream; the null stream and the blocking
// streams also wait for each other's earlier work.  Returns the stream's clock.
VClock &begin_op(int sid) {
  VClock &v = stream_clocks()[sid];
  vc_join(v, g_host);
  if (sid == 0) {
    for (size_t i = 1; i < stream_clocks().size(); i++)
      if (stream_blocking()[i]) vc_join(v, stream_clocks()[i]);
  } else if (stream_blocking()[sid]) {
    vc_join(v, stream_clocks()[0]);
  }
  if (v.size() <= (size_t)sid) v.resize(sid + 1, 0);
  v[sid]++;
  return v;
}
struct Acc {
  uintptr_t lo, hi;
  bool write;
  int sid;
  uint64_t clk;
  std::string who;
};
std::map<uintptr_t, std::vector<Acc>> &accesses() { static auto *m = new std::map<uintptr_t, std::vector<Acc>>(); return *m; }  // block start -> list
size_t g_race_checks = 0;
std::map<std::string, size_t> &races() { static auto *m = new std::map<std::string, size_t>(); return *m; }
void access(int sid, uintptr_t p, size_t n, bool write, const std::string &who) {
  if (!n || !in_range(p)) return;
  const auto *b = block_of(p);
  if (!b || !b->second.live) return;  // reported by the range checks
  const uintptr_t lo = p, hi = std::min<uintptr_t>(p + n, b->first + b->second.size);
  const VClock &v = stream_clocks()[sid];
  const uint64_t clk = v[sid];
  std::vector<Acc> &list = accesses()[b->first];
  g_race_checks++;
  size_t keep = 0;
  for (size_t i = 0; i < list.size(); i++) {
    Acc &e = list[i];
    const bool ordered = vc_covers(v, e.sid, e.clk);
    if (e.lo < hi && lo < e.hi && (e.write || write) && !ordered) {
      const std::string key = who + (write ? " writes" : " reads") + " / " + e.who + (e.write ? " writes" : " reads");
      if (races()[key]++ == 0)
        violation("race: " + who + (write ? " writes " : " reads ") + std::to_string(hi - lo) + " bytes of a block (" + b->second.what +
                  ") on stream " + std::to_string(sid) + " with no ordering after " + e.who + (e.write ? " (write)" : " (read)") + " on stream " +
                  std::to_string(e.sid));
    }
    // an access the host has waited for precedes every later operation; one
    // covered by this access and ordered before it is shadowed by it
    const bool drop = vc_covers(g_host, e.sid, e.clk) || (lo <= e.lo && e.hi <= hi && ordered && (write || !e.write));
    if (!drop) list[keep++] = std::move(e);
  }
  list.resize(keep);
  list.push_back(Acc{lo, hi, write, sid, clk, who});
}
void host_join_all() {
  for (const VClock &v : stream_clocks()) vc_join(g_host, v);
}

// ── per-kernel extents (extents.cpp): every range a kernel reads or writes
// must lie inside one live block ──
}  // namespace
namespace audit_ext {
struct Span {
  uintptr_t p;
  size_t bytes;
  bool write;
  std::string what;
};
int extents(const std::string &mangled, const std::string &pretty, const std::vector<std::vector<char>> &a, unsigned gx, unsigned gy, unsigned gz,
            unsigned threads, std::vector<Span> &o, std::string &note);
extern bool g_dry;
}  // namespace audit_ext
namespace {
std::map<std::string, size_t> &unmodelled() { static auto *m = new std::map<std::string, size_t>(); return *m; }
size_t g_extent_checks = 0;
// returns whether the kernel has an extent model
bool check_extents(const Launch &l, const char *when, int sid) {
  const KernelInfo &k = *l.k;
  std::vector<audit_ext::Span> sp;
  std::string note;
  if (!audit_ext::extents(k.name, k.pretty, l.args, l.grid.x, l.grid.y, l.grid.z, l.block.x * l.block.y * l.block.z, sp, note)) {
    unmodelled()[k.pretty]++;
    return false;
  }
  const std::string who = std::string(when) + " " + k.pretty;
  if (!note.empty()) violation(who + ": " + note);
  for (const auto &s : sp) {
    g_extent_checks++;
    const std::string w = who + " " + (s.write ? "writes " : "reads ") + s.what;
    if (!in_range(s.p)) {
      violation(w + ": range starts outside device memory");
      continue;
    }
    check_span((const void *)s.p, s.bytes, w);
    access(sid, s.p, s.bytes, s.write, k.pretty + " (" + s.what + ")");
  }
  return true;
}

void check_geometry(const KernelInfo &k, dim3 g, dim3 b, size_t shm) {
  const unsigned nt = b.x * b.y * b.z;
  if (!nt || !g.x || !g.y || !g.z) violation(k.pretty + ": empty grid or block");
  if ((int)nt > k.max_threads) violation(k.pretty + ": " + std::to_string(nt) + " threads per block, kernel allows " + std::to_string(k.max_threads));
  if (g.y > 65535 || g.z > 65535) violation(k.pretty + ": grid y/z above 65535");
  if ((size_t)k.lds + shm > 160 * 1024) violation(k.pretty + ": LDS " + std::to_string(k.lds + shm) + " bytes");
}

struct CallCfg {
  dim3 g, b;
  size_t shm;
  hipStream_t s;
};
thread_local std::vector<CallCfg> t_cfg;
hipError_t g_last = hipSuccess;

Handle *capturing_stream(hipStream_t s) {
  Handle *h = (Handle *)s;
  if (h && h->capturing) return h;
  return nullptr;
}

hipError_t do_launch(const void *f, dim3 g, dim3 b, void **args, size_t shm, hipStream_t s) {
  std::lock_guard<std::mutex> lk(g_mu);
  load_table();
  if (!check_handle(s, K_STREAM, "launch", true)) return hipErrorInvalidHandle;
  auto it = g_kernels.find(f);
  if (it == g_kernels.end()) {
    violation("launch of an unregistered kernel");
    return hipErrorInvalidDeviceFunction;
  }
  KernelInfo &k = it->second;
  if (g_fail_launch_after >= 0 && g_fail_launch_after-- == 0) {
    g_last = hipErrorLaunchFailure;
    return hipErrorLaunchFailure;
  }
  if (!k.known) {
    violation(k.pretty + ": no argument layout in the table");
    return hipSuccess;
  }
  Launch l{&k, {}, g, b};
  int vis = 0;
  for (const Arg &a : k.args)
    if (!a.hidden) vis++;
  for (int i = 0; i < vis; i++) {
    const Arg &a = k.args[i];
    std::vector<char> v(a.size);
    std::memcpy(v.data(), args[i], a.size);
    l.args.push_back(std::move(v));
  }
  g_launches++;
  static FILE *logf = std::getenv("FA_AUDIT_LOG") ? std::fopen(std::getenv("FA_AUDIT_LOG"), "w") : nullptr;
  if (logf) std::fprintf(logf, "%s %u %u %u %u\n", k.pretty.c_str(), g.x, g.y, g.z, b.x * b.y * b.z);
  check_geometry(k, g, b, shm);
  Handle *cs = capturing_stream(s);
  if (!cs) {  // a captured launch runs (and is checked) at each replay
    const int sid = stream_sid(s);
    begin_op(sid);
    check_launch_args(l, "launch", !check_extents(l, "launch", sid));
  } else {  // captured: checked at each replay; here only the pointer arguments
    std::vector<audit_ext::Span> sp;
    std::string note;
    audit_ext::g_dry = true;
    const bool has_model = audit_ext::extents(k.name, k.pretty, l.args, g.x, g.y, g.z, b.x * b.y * b.z, sp, note) != 0;
    audit_ext::g_dry = false;
    check_launch_args(l, "launch", !has_model);
  }
  if (cs) cs->ops.push_back(Op{0, l});
  return hipSuccess;
}

}  // namespace

extern "C" {

// ── registration ──
void **__hipRegisterFatBinary(const void *) {
  static void *mod = nullptr;
  return &mod;
}
void __hipUnregisterFatBinary(void **) {}
void __hipRegisterFunction(void **, const void *host, char *, const char *dev, unsigned int, void *, void *, void *, void *, int *) {
  std::lock_guard<std::mutex> lk(g_mu);
  load_table();
  KernelInfo k;
  auto t = g_table.find(dev);
  if (t != g_table.end()) k = t->second;
  k.name = dev;
  k.pretty = demangle(dev);
  g_kernels[host] = k;
}
void __hipRegisterVar(void **, void *var, char *, char *, int, size_t size, int, int) {
  std::lock_guard<std::mutex> lk(g_mu);
  g_vars[var] = {size, dev_alloc(size, "__device__ variable")};
}
hipError_t __hipPushCallConfiguration(dim3 g, dim3 b, size_t shm, hipStream_t s) {
  t_cfg.push_back({g, b, shm, s});
  return hipSuccess;
}
hipError_t __hipPopCallConfiguration(dim3 *g, dim3 *b, size_t *shm, hipStream_t *s) {
  if (t_cfg.empty()) return hipErrorInvalidConfiguration;
  CallCfg c = t_cfg.back();
  t_cfg.pop_back();
  *g = c.g;
  *b = c.b;
  *shm = c.shm;
  *s = c.s;
  return hipSuccess;
}

// ── launches ──
hipError_t hipLaunchKernel(const void *f, dim3 g, dim3 b, void **args, size_t shm, hipStream_t s) { return do_launch(f, g, b, args, shm, s); }
hipError_t hipExtLaunchKernel(const void *f, dim3 g, dim3 b, void **args, size_t shm, hipStream_t s, hipEvent_t e0, hipEvent_t e1, int) {
  {
    std::lock_guard<std::mutex> lk(g_mu);
    if (!check_handle(e0, K_EVENT, "hipExtLaunchKernel start event", true) || !check_handle(e1, K_EVENT, "hipExtLaunchKernel stop event", true))
      return hipErrorInvalidHandle;
    if (e0) ((Handle *)e0)->recorded = true;
    if (e1) ((Handle *)e1)->recorded = true;
    if (e0 && check_handle(s, K_STREAM, "hipExtLaunchKernel", true) && !capturing_stream(s)) ((Handle *)e0)->vc = begin_op(stream_sid(s));
  }
  const hipError_t r = do_launch(f, g, b, args, shm, s);
  if (e1) {
    std::lock_guard<std::mutex> lk(g_mu);
    if (check_handle(s, K_STREAM, "hipExtLaunchKernel", true) && !capturing_stream(s)) ((Handle *)e1)->vc = stream_clocks()[stream_sid(s)];
  }
  return r;
}
hipError_t hipFuncSetAttribute(const void *, hipFuncAttribute, int) { return hipSuccess; }
hipError_t hipGetLastError(void) {
  hipError_t e = g_last;
  g_last = hipSuccess;
  return e;
}
const char *hipGetErrorString(hipError_t e) { return e == hipSuccess ? "no error" : "audit error"; }

// ── device ──
hipError_t hipGetDeviceCount(int *n) {
  *n = 1;
  return hipSuccess;
}
hipError_t hipSetDevice(int d) { return d == 0 ? hipSuccess : hipErrorInvalidDevice; }
hipError_t hipGetDevicePropertiesR0600(hipDeviceProp_tR0600 *p, int d) {
  if (d != 0) return hipErrorInvalidDevice;
  std::memset(p, 0, sizeof *p);
  std::snprintf(p->name, sizeof p->name, "launch audit (gfx950 geometry)");
  std::snprintf(p->gcnArchName, sizeof p->gcnArchName, "gfx950:sramecc+:xnack-");
  p->multiProcessorCount = 256;
  p->totalGlobalMem = 288ull << 30;
  p->warpSize = 64;
  p->maxThreadsPerBlock = 1024;
  p->sharedMemPerBlock = 160 * 1024;
  p->clockRate = 2400000;
  p->major = 9;
  p->minor = 5;
  return hipSuccess;
}
hipError_t hipDeviceSynchronize(void) {
  std::lock_guard<std::mutex> lk(g_mu);
  host_join_all();
  return hipSuccess;
}
hipError_t hipGetSymbolAddress(void **dev, const void *sym) {
  std::lock_guard<std::mutex> lk(g_mu);
  auto it = g_vars.find(sym);
  if (it == g_vars.end()) {
    violation("hipGetSymbolAddress of an unregistered symbol");
    return hipErrorInvalidSymbol;
  }
  *dev = it->second.second;
  return hipSuccess;
}

// ── memory ──
hipError_t hipMalloc(void **p, size_t n) {
  std::lock_guard<std::mutex> lk(g_mu);
  if (g_fail_alloc_after >= 0 && g_fail_alloc_after-- == 0) {
    *p = nullptr;
    return hipErrorOutOfMemory;
  }
  *p = dev_alloc(n, "hipMalloc");
  return *p ? hipSuccess : hipErrorOutOfMemory;
}
hipError_t hipFree(void *p) {
  std::lock_guard<std::mutex> lk(g_mu);
  if (!p) return hipSuccess;
  auto it = g_blocks.find((uintptr_t)p);
  if (it == g_blocks.end()) {
    violation("hipFree of a pointer that is not a block start");
    return hipErrorInvalidValue;
  }
  if (!it->second.live) {
    violation("hipFree of a block freed before");
    return hipErrorInvalidValue;
  }
  it->second.live = false;
  host_join_all();  // hipFree waits for the device
  accesses().erase(it->first);
  madvise(p, it->second.size, MADV_DONTNEED);  // hand the pages back; the addresses stay reserved
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
static hipError_t copy(void *dst, const void *src, size_t n, hipStream_t s, const char *api, bool sync) {
  std::lock_guard<std::mutex> lk(g_mu);
  if (!check_handle(s, K_STREAM, api, true)) return hipErrorInvalidHandle;
  check_span(dst, n, std::string(api) + " destination");
  check_span(src, n, std::string(api) + " source");
  if (!capturing_stream(s)) {
    const int sid = stream_sid(s);
    begin_op(sid);
    access(sid, (uintptr_t)src, n, false, std::string(api) + " source");
    access(sid, (uintptr_t)dst, n, true, std::string(api) + " destination");
    if (sync) vc_join(g_host, stream_clocks()[sid]);  // returns when the copy is done
  }
  if (Handle *cs = capturing_stream(s)) {
    Op o;
    o.type = 1;
    o.p0 = dst;
    o.p1 = src;
    o.bytes = n;
    cs->ops.push_back(o);
  }
  if (n) std::memmove(dst, src, n);
  return hipSuccess;
}
hipError_t hipMemcpy(void *dst, const void *src, size_t n, hipMemcpyKind) { return copy(dst, src, n, nullptr, "hipMemcpy", true); }
hipError_t hipMemcpyAsync(void *dst, const void *src, size_t n, hipMemcpyKind, hipStream_t s) { return copy(dst, src, n, s, "hipMemcpyAsync", false); }
hipError_t hipMemsetAsync(void *dst, int v, size_t n, hipStream_t s) {
  std::lock_guard<std::mutex> lk(g_mu);
  if (!check_handle(s, K_STREAM, "hipMemsetAsync", true)) return hipErrorInvalidHandle;
  check_span(dst, n, "hipMemsetAsync");
  if (!capturing_stream(s)) {
    const int sid = stream_sid(s);
    begin_op(sid);
    access(sid, (uintptr_t)dst, n, true, "hipMemsetAsync");
  }
  if (Handle *cs = capturing_stream(s)) {
    violation("hipMemsetAsync recorded into a captured graph");
    Op o;
    o.type = 2;
    o.p0 = dst;
    o.bytes = n;
    cs->ops.push_back(o);
  }
  if (n) std::memset(dst, v, n);
  return hipSuccess;
}

// ── streams and events ──
hipError_t hipStreamCreateWithFlags(hipStream_t *s, unsigned int flags) {
  std::lock_guard<std::mutex> lk(g_mu);
  Handle *h = new_handle(K_STREAM);
  h->blocking = !(flags & hipStreamNonBlocking);
  stream_blocking()[h->sid] = h->blocking;
  *s = (hipStream_t)h;
  return hipSuccess;
}
hipError_t hipStreamDestroy(hipStream_t s) {
  std::lock_guard<std::mutex> lk(g_mu);
  if (!check_handle(s, K_STREAM, "hipStreamDestroy", false)) return hipErrorInvalidHandle;
  ((Handle *)s)->live = false;
  return hipSuccess;
}
hipError_t hipStreamSynchronize(hipStream_t s) {
  std::lock_guard<std::mutex> lk(g_mu);
  if (!check_handle(s, K_STREAM, "hipStreamSynchronize", true)) return hipErrorInvalidHandle;
  vc_join(g_host, stream_clocks()[stream_sid(s)]);
  return hipSuccess;
}
hipError_t hipStreamWaitEvent(hipStream_t s, hipEvent_t e, unsigned int) {
  std::lock_guard<std::mutex> lk(g_mu);
  if (!check_handle(s, K_STREAM, "hipStreamWaitEvent", true) || !check_handle(e, K_EVENT, "hipStreamWaitEvent", false)) return hipErrorInvalidHandle;
  if (capturing_stream(s)) violation("hipStreamWaitEvent on a capturing stream (not modelled)");
  else vc_join(stream_clocks()[stream_sid(s)], ((Handle *)e)->vc);
  return hipSuccess;
}
hipError_t hipEventCreate(hipEvent_t *e) {
  std::lock_guard<std::mutex> lk(g_mu);
  *e = (hipEvent_t)new_handle(K_EVENT);
  return hipSuccess;
}
hipError_t hipEventCreateWithFlags(hipEvent_t *e, unsigned) { return hipEventCreate(e); }
hipError_t hipEventDestroy(hipEvent_t e) {
  std::lock_guard<std::mutex> lk(g_mu);
  if (!check_handle(e, K_EVENT, "hipEventDestroy", false)) return hipErrorInvalidHandle;
  ((Handle *)e)->live = false;
  return hipSuccess;
}
hipError_t hipEventRecord(hipEvent_t e, hipStream_t s) {
  std::lock_guard<std::mutex> lk(g_mu);
  if (!check_handle(e, K_EVENT, "hipEventRecord", false) || !check_handle(s, K_STREAM, "hipEventRecord", true)) return hipErrorInvalidHandle;
  ((Handle *)e)->recorded = true;
  if (capturing_stream(s)) violation("hipEventRecord on a capturing stream (not modelled)");
  else {
    VClock &v = stream_clocks()[stream_sid(s)];
    vc_join(v, g_host);
    ((Handle *)e)->vc = v;
  }
  return hipSuccess;
}
hipError_t hipEventSynchronize(hipEvent_t e) {
  std::lock_guard<std::mutex> lk(g_mu);
  if (!check_handle(e, K_EVENT, "hipEventSynchronize", false)) return hipErrorInvalidHandle;
  vc_join(g_host, ((Handle *)e)->vc);
  return hipSuccess;
}
hipError_t hipEventElapsedTime(float *ms, hipEvent_t a, hipEvent_t b) {
  std::lock_guard<std::mutex> lk(g_mu);
  *ms = 0.f;
  if (!check_handle(a, K_EVENT, "hipEventElapsedTime", false) || !check_handle(b, K_EVENT, "hipEventElapsedTime", false)) return hipErrorInvalidHandle;
  if (!((Handle *)a)->recorded || !((Handle *)b)->recorded) return hipErrorNotReady;  // legal: reported, not a violation
  return hipSuccess;
}

// ── graphs ──
hipError_t hipStreamBeginCapture(hipStream_t s, hipStreamCaptureMode) {
  std::lock_guard<std::mutex> lk(g_mu);
  if (!check_handle(s, K_STREAM, "hipStreamBeginCapture", false)) return hipErrorInvalidHandle;
  Handle *h = (Handle *)s;
  if (h->capturing) violation("hipStreamBeginCapture on a stream already capturing");
  h->capturing = true;
  h->ops.clear();
  return hipSuccess;
}
hipError_t hipStreamEndCapture(hipStream_t s, hipGraph_t *g) {
  std::lock_guard<std::mutex> lk(g_mu);
  if (!check_handle(s, K_STREAM, "hipStreamEndCapture", false)) return hipErrorInvalidHandle;
  Handle *h = (Handle *)s;
  if (!h->capturing) violation("hipStreamEndCapture without a capture");
  h->capturing = false;
  Handle *gr = new_handle(K_GRAPH);
  gr->ops.swap(h->ops);
  *g = (hipGraph_t)gr;
  return hipSuccess;
}
hipError_t hipGraphInstantiateWithFlags(hipGraphExec_t *x, hipGraph_t g, unsigned long long) {
  std::lock_guard<std::mutex> lk(g_mu);
  if (!check_handle(g, K_GRAPH, "hipGraphInstantiate", false)) return hipErrorInvalidHandle;
  Handle *e = new_handle(K_EXEC);
  e->ops = ((Handle *)g)->ops;
  *x = (hipGraphExec_t)e;
  return hipSuccess;
}
hipError_t hipGraphDestroy(hipGraph_t g) {
  std::lock_guard<std::mutex> lk(g_mu);
  if (!check_handle(g, K_GRAPH, "hipGraphDestroy", false)) return hipErrorInvalidHandle;
  ((Handle *)g)->live = false;
  ((Handle *)g)->ops.clear();
  return hipSuccess;
}
hipError_t hipGraphExecDestroy(hipGraphExec_t x) {
  std::lock_guard<std::mutex> lk(g_mu);
  if (!check_handle(x, K_EXEC, "hipGraphExecDestroy", false)) return hipErrorInvalidHandle;
  ((Handle *)x)->live = false;
  return hipSuccess;
}
hipError_t hipGraphLaunch(hipGraphExec_t x, hipStream_t s) {
  std::lock_guard<std::mutex> lk(g_mu);
  if (!check_handle(x, K_EXEC, "hipGraphLaunch", false) || !check_handle(s, K_STREAM, "hipGraphLaunch", true)) return hipErrorInvalidHandle;
  g_replays++;
  if (capturing_stream(s)) violation("hipGraphLaunch into a capturing stream");
  const int sid = stream_sid(s);
  for (const Op &o : ((Handle *)x)->ops) {  // nodes captured from one stream run in order
    begin_op(sid);
    if (o.type == 0) {
      g_replayed_launches++;
      check_launch_args(o.l, "graph replay", !check_extents(o.l, "graph replay", sid));
    } else {
      check_span(o.p0, o.bytes, "graph replay copy/set destination");
      if (o.type == 1) check_span(o.p1, o.bytes, "graph replay copy source");
      if (o.type == 1) access(sid, (uintptr_t)o.p1, o.bytes, false, "graph replay copy source");
      access(sid, (uintptr_t)o.p0, o.bytes, true, "graph replay copy/set destination");
    }
  }
  return hipSuccess;
}

// ── report ──
// Writes the violations (one per line) into buf; returns their count.
int audit_report(char *buf, int cap, unsigned long long *counts) {
  std::lock_guard<std::mutex> lk(g_mu);
  std::string s;
  for (const std::string &v : g_viol) s += v + "\n";
  if (buf && cap > 0) std::snprintf(buf, cap, "%s", s.c_str());
  if (counts) {
    counts[0] = g_launches;
    counts[1] = g_replays;
    counts[2] = g_replayed_launches;
    counts[3] = g_allocs;
  }
  return (int)g_viol.size();
}
// Kernels launched without an extent model ("name count" per line) and the
// number of ranges checked.
int audit_extent_report(char *buf, int cap, unsigned long long *checks) {
  std::lock_guard<std::mutex> lk(g_mu);
  std::string s;
  for (const auto &u : unmodelled()) s += u.first + " " + std::to_string(u.second) + "\n";
  if (buf && cap > 0) std::snprintf(buf, cap, "%s", s.c_str());
  if (checks) *checks = g_extent_checks;
  return (int)unmodelled().size();
}
// Accesses checked for ordering, and the races found ("access / earlier
// access count" per line).
int audit_race_report(char *buf, int cap, unsigned long long *checks) {
  std::lock_guard<std::mutex> lk(g_mu);
  std::string s;
  for (const auto &r : races()) s += r.first + " " + std::to_string(r.second) + "\n";
  if (buf && cap > 0) std::snprintf(buf, cap, "%s", s.c_str());
  if (checks) *checks = g_race_checks;
  return (int)races().size();
}
void audit_fail_alloc(long after) {
  std::lock_guard<std::mutex> lk(g_mu);
  g_fail_alloc_after = after;
}
void audit_fail_launch(long after) {
  std::lock_guard<std::mutex> lk(g_mu);
  g_fail_launch_after = after;
}
void audit_clear(void) {
  std::lock_guard<std::mutex> lk(g_mu);
  g_viol.clear();
  races().clear();
}

}  // extern "C"

namespace {
// Hosts that cannot call audit_report (the N-API addon under Node): with
// FA_AUDIT_REPORT set, the counts, the violations, the kernels without an
// extent model and the races are written to that file at process exit, one
// "key value" line each for the counts.
struct ExitReport {
  ~ExitReport() {
    const char *path = std::getenv("FA_AUDIT_REPORT");
    if (!path) return;
    std::lock_guard<std::mutex> lk(g_mu);
    std::ofstream f(path);
    f << "launches " << g_launches << "\nreplays " << g_replays << "\nallocations " << g_allocs << "\nextent_checks " << g_extent_checks
      << "\norder_checks " << g_race_checks << "\n";
    for (const std::string &v : g_viol) f << "violation " << v << "\n";
    for (const auto &u : unmodelled()) f << "unmodelled " << u.first << "\n";
    for (const auto &r : races()) f << "race " << r.first << "\n";
  }
} g_exit_report;
}  // namespace
