// Internal declarations shared by the runtime and the kernel translation units.
#pragma once
#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <hip/hip_ext.h>

#include <cstdint>
#include <cstdio>
#include <string>
#include <unordered_map>
#include <vector>

#include "../../include/fa_hip.h"

namespace fa {

enum StoreKind : int {
  S_F32 = 0,   // row-major f32 [rows, cols]
  S_F16KM = 1, // f16 weight, stored K-major: element (k, n) of a [K=rows, N=cols] matrix at n*K + k
  S_BYTES = 2, // raw bytes (int8/int4 payloads), `bytes` long
  S_F16RM = 3, // f16 row-major activations [rows, cols] (allocF16)
};

struct TensorRec {
  void *ptr = nullptr;
  size_t bytes = 0;  // allocation size (pool key)
  int rows = 0, cols = 0;
  int kind = S_F32;
  uint32_t gen = 1;
  bool live = false;
  bool view = false;       // rowsView alias: never pooled
  bool pooled = false;     // storage returns to the pool on free/arena pop
  uint64_t arena = 0;      // owning arena id (0 = persistent / none)
  void *aux = nullptr;     // derived cache (e.g. repacked int8 weights), freed with the tensor
  size_t aux_bytes = 0;
};

struct Arena {
  uint64_t id;
  std::vector<uint32_t> slots;
};

struct ProfRec {
  char label[48];
  hipEvent_t a, b;
};

struct Staged {
  void *host = nullptr;  // pinned
  size_t bytes = 0;
  int kind = S_F32;
  int rows = 0, cols = 0;
  hipEvent_t ev = nullptr;
  bool consumed = false;
};

}  // namespace fa

struct fa_ctx {
  int device = 0;
  hipStream_t stream = nullptr;
  std::string err;
  std::vector<fa::TensorRec> recs;
  std::vector<uint32_t> free_slots;
  std::unordered_map<size_t, std::vector<void *>> pool;
  size_t pooled_bytes = 0;
  uint64_t created = 0, created_bytes = 0, reused = 0;
  std::vector<fa::Arena> arenas;
  uint64_t next_arena = 1;
  bool batch_open = false;
  // profiler
  bool prof_on = false;
  int prof_max = 0;
  std::vector<fa::ProfRec> prof;
  std::vector<hipEvent_t> prof_free_events;
  std::string prof_filter;  // label prefix; empty = all launches
  // staged reads
  std::vector<fa::Staged> staged;
  std::vector<uint32_t> staged_gen;
  int num_cu = 256;
  // log-mel front end: constant tables (window, twiddles, filterbank) for
  // mel_tab_mels bins, and per-(window, bin) statistics scratch
  void *mel_tab = nullptr;
  int mel_tab_mels = 0;
  void *mel_scratch = nullptr;
  size_t mel_scratch_bytes = 0;
};

namespace fa {

// ── status helpers ────────────────────────────────────────────────────────
int set_err(fa_ctx *ctx, int code, const char *fmt, ...);
#define FA_TRY(expr)                  \
  do {                                \
    int _st = (expr);                 \
    if (_st != FA_OK) return _st;     \
  } while (0)
#define FA_HIP(ctx, expr)                                                                                   \
  do {                                                                                                      \
    hipError_t _e = (expr);                                                                                 \
    if (_e != hipSuccess) return ::fa::set_err((ctx), FA_E_DEVICE, "%s: %s", #expr, hipGetErrorString(_e)); \
  } while (0)

// ── tensor access ─────────────────────────────────────────────────────────
TensorRec *get(fa_ctx *ctx, fa_tensor t);  // nullptr (error set) when stale
int need(fa_ctx *ctx, fa_tensor t, TensorRec **out, const char *what);
int opt(fa_ctx *ctx, fa_tensor t, TensorRec **out, const char *what);  // t == 0 -> *out = nullptr
int new_tensor(fa_ctx *ctx, int rows, int cols, int kind, size_t bytes, fa_tensor *out, TensorRec **rec = nullptr);
int new_persistent(fa_ctx *ctx, int rows, int cols, int kind, size_t bytes, fa_tensor *out, TensorRec **rec = nullptr);
void *dev_alloc(fa_ctx *ctx, size_t bytes);  // raw hipMalloc, nullptr on failure (error set)

// A freshly allocated output tensor, freed when the scope ends unless
// release() handed it to the caller: an op that fails after allocating its
// output leaves nothing behind.
struct TensorGuard {
  fa_ctx *ctx;
  fa_tensor t;
  TensorGuard(fa_ctx *c, fa_tensor x) : ctx(c), t(x) {}
  TensorGuard(const TensorGuard &) = delete;
  TensorGuard &operator=(const TensorGuard &) = delete;
  ~TensorGuard() {
    if (t) (void)fa_free_tensor(ctx, t);
  }
  fa_tensor release() {
    const fa_tensor r = t;
    t = 0;
    return r;
  }
};

// ── launch bracketing for the profiler ────────────────────────────────────
// A ProfScope opened around a launch claims a (start, stop) event pair when a
// profile is open for its label.  FA_LAUNCH hands the pair to
// hipExtLaunchKernelGGL, which stamps them at the kernel's own start and end
// (no marker packets between dispatches); a scope that covers several
// launches or copies (ext = false) records the events on the stream instead.
struct ProfScope {
  fa_ctx *ctx;
  int idx;
  bool ext;
  hipEvent_t a = nullptr, b = nullptr;
  ProfScope(fa_ctx *c, const char *label, bool ext_launch = true);
  ~ProfScope();
};
#define FA_LAUNCH(ps, kernel, grid, block, shm, stream, ...)                                           \
  do {                                                                                                 \
    if ((ps).a)                                                                                        \
      hipExtLaunchKernelGGL(kernel, grid, block, shm, stream, (ps).a, (ps).b, 0, __VA_ARGS__);         \
    else                                                                                               \
      hipLaunchKernelGGL(kernel, grid, block, shm, stream, __VA_ARGS__);                               \
  } while (0)
int check_launch(fa_ctx *ctx, const char *what);

// Looks up the allocation-free mel path's static device array for ctx->device
// (once per device; mel.hip).  Called by fa_ctx_create with the device current.
int mel_static_init(fa_ctx *ctx);
void mel_static_release(fa_ctx *ctx);  // fa_ctx_destroy: gives up the static scratch
// Log-mel internals shared with the windowed-transcription runner (mel.hip).
int tdt_decode_dev(fa_tdt *d, const float *fr, long rows, const int32_t *lens, int n, int cap, int32_t *ids, int32_t *frame_idx, int32_t *counts);
int mel_prepare(fa_ctx *ctx, int n, int n_mels, int normalize);
int mel_windows_dev(fa_ctx *ctx, const float *pcm, long nsamp, const int32_t *starts, const int32_t *lens, int n, int n_mels, double log_guard,
                    int normalize, float *y, long *total);

inline unsigned cdiv(long a, long b) { return (unsigned)((a + b - 1) / b); }

}  // namespace fa
