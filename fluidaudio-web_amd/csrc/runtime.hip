// Context, tensor handles, exact-size buffer pool with arena scopes, readback,
// batching and the event profiler.
//
// Semantics follow the reference's WebGPU backend:
//  - pool: exact-size free lists, `put` never frees (src/gpu/buffer-pool.js:21-47);
//    on one in-order HIP stream a recycled buffer is only written by work
//    queued after every earlier reader, so reuse is ordered-safe;
//  - arenas: allocations land in the newest open scope, scopes may close out of
//    order, pin() exempts or promotes to the parent (buffer-pool.js:49-126);
//  - no open arena -> a persistent allocation that never draws from the pool
//    (buffer-pool.js:53-61);
//  - batches are non-reentrant (src/gpu/scheduler.js:17-31);
//  - staged reads are single-use (compute.js:1112-1128).
#include <cstdarg>
#include <cstring>
#include <algorithm>

#include "fa_internal.h"

namespace fa {

int set_err(fa_ctx *ctx, int code, const char *fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  if (ctx) ctx->err = buf;
  return code;
}

static inline uint32_t slot_of(fa_tensor t) { return (uint32_t)(t & 0xffffffffu) - 1u; }
static inline uint32_t gen_of(fa_tensor t) { return (uint32_t)(t >> 32); }

TensorRec *get(fa_ctx *ctx, fa_tensor t) {
  if (t == 0) {
    set_err(ctx, FA_E_INVALID, "null tensor handle");
    return nullptr;
  }
  uint32_t s = slot_of(t);
  if (s >= ctx->recs.size() || !ctx->recs[s].live || ctx->recs[s].gen != gen_of(t)) {
    set_err(ctx, FA_E_INVALID, "stale tensor handle (released by popArena/freeTensor)");
    return nullptr;
  }
  return &ctx->recs[s];
}

int need(fa_ctx *ctx, fa_tensor t, TensorRec **out, const char *what) {
  if (t == 0) return set_err(ctx, FA_E_INVALID, "%s: missing tensor", what);
  TensorRec *r = get(ctx, t);
  if (!r) return set_err(ctx, FA_E_INVALID, "%s: stale tensor handle", what);
  *out = r;
  return FA_OK;
}

int opt(fa_ctx *ctx, fa_tensor t, TensorRec **out, const char *what) {
  if (t == 0) {
    *out = nullptr;
    return FA_OK;
  }
  return need(ctx, t, out, what);
}

void *dev_alloc(fa_ctx *ctx, size_t bytes) {
  void *p = nullptr;
  hipError_t e = hipMalloc(&p, bytes < 256 ? 256 : bytes);
  if (e != hipSuccess) {
    (void)hipGetLastError();
    set_err(ctx, FA_E_OOM, "hipMalloc(%zu): %s", bytes, hipGetErrorString(e));
    return nullptr;
  }
  ctx->created++;
  ctx->created_bytes += bytes;
  return p;
}

static uint32_t take_slot(fa_ctx *ctx) {
  if (!ctx->free_slots.empty()) {
    uint32_t s = ctx->free_slots.back();
    ctx->free_slots.pop_back();
    return s;
  }
  ctx->recs.emplace_back();
  return (uint32_t)ctx->recs.size() - 1;
}

static fa_tensor handle_of(fa_ctx *ctx, uint32_t s) { return ((uint64_t)ctx->recs[s].gen << 32) | (uint64_t)(s + 1); }

static void release_slot(fa_ctx *ctx, uint32_t s) {
  TensorRec &r = ctx->recs[s];
  if (r.aux) {
    (void)hipFree(r.aux);
    r.aux = nullptr;
  }
  r.live = false;
  r.gen++;
  r.ptr = nullptr;
  ctx->free_slots.push_back(s);
}

static void pool_put(fa_ctx *ctx, void *p, size_t bytes) {
  ctx->pool[bytes].push_back(p);
  ctx->pooled_bytes += bytes;
}

static void *pool_get(fa_ctx *ctx, size_t bytes) {
  auto it = ctx->pool.find(bytes);
  if (it != ctx->pool.end() && !it->second.empty()) {
    void *p = it->second.back();
    it->second.pop_back();
    ctx->pooled_bytes -= bytes;
    ctx->reused++;
    return p;
  }
  return dev_alloc(ctx, bytes);
}

int new_persistent(fa_ctx *ctx, int rows, int cols, int kind, size_t bytes, fa_tensor *out, TensorRec **rec) {
  if (rows < 0 || cols < 0) return set_err(ctx, FA_E_INVALID, "negative shape [%d,%d]", rows, cols);
  void *p = dev_alloc(ctx, bytes);
  if (!p) return FA_E_OOM;
  uint32_t s = take_slot(ctx);
  TensorRec &r = ctx->recs[s];
  uint32_t g = r.gen;
  r = TensorRec();
  r.gen = g;
  r.ptr = p;
  r.bytes = bytes;
  r.rows = rows;
  r.cols = cols;
  r.kind = kind;
  r.live = true;
  r.pooled = false;
  *out = handle_of(ctx, s);
  if (rec) *rec = &r;
  return FA_OK;
}

// alloc(): pooled + arena-tracked when an arena is open, else persistent.
int new_tensor(fa_ctx *ctx, int rows, int cols, int kind, size_t bytes, fa_tensor *out, TensorRec **rec) {
  if (rows < 0 || cols < 0) return set_err(ctx, FA_E_INVALID, "negative shape [%d,%d]", rows, cols);
  if (ctx->arenas.empty()) return new_persistent(ctx, rows, cols, kind, bytes, out, rec);
  bytes = bytes < 256 ? 256 : ((bytes + 255) & ~(size_t)255);
  void *p = pool_get(ctx, bytes);
  if (!p) return FA_E_OOM;
  uint32_t s = take_slot(ctx);
  TensorRec &r = ctx->recs[s];
  uint32_t g = r.gen;
  r = TensorRec();
  r.gen = g;
  r.ptr = p;
  r.bytes = bytes;
  r.rows = rows;
  r.cols = cols;
  r.kind = kind;
  r.live = true;
  r.pooled = true;
  r.arena = ctx->arenas.back().id;
  ctx->arenas.back().slots.push_back(s);
  *out = handle_of(ctx, s);
  if (rec) *rec = &r;
  return FA_OK;
}

// ── profiler ──────────────────────────────────────────────────────────────
static hipEvent_t take_event(fa_ctx *ctx) {
  if (!ctx->prof_free_events.empty()) {
    hipEvent_t e = ctx->prof_free_events.back();
    ctx->prof_free_events.pop_back();
    return e;
  }
  hipEvent_t e = nullptr;
  if (hipEventCreate(&e) != hipSuccess) return nullptr;
  return e;
}

// Profile filter: comma-separated entries, each an exact label or, ending in
// '*', a label prefix.
static bool prof_match(const std::string &filter, const char *label) {
  size_t i = 0;
  while (i <= filter.size()) {
    size_t j = filter.find(',', i);
    if (j == std::string::npos) j = filter.size();
    if (j > i) {
      const bool prefix = filter[j - 1] == '*';
      const size_t len = j - i - (prefix ? 1 : 0);
      if (prefix ? std::strncmp(label, filter.c_str() + i, len) == 0 : (std::strlen(label) == len && std::strncmp(label, filter.c_str() + i, len) == 0))
        return true;
    }
    i = j + 1;
  }
  return false;
}

ProfScope::ProfScope(fa_ctx *c, const char *label, bool ext_launch) : ctx(c), idx(-1), ext(ext_launch) {
  if (!ctx->prof_on || (int)ctx->prof.size() >= ctx->prof_max) return;
  if (!ctx->prof_filter.empty() && !prof_match(ctx->prof_filter, label)) return;
  ProfRec r;
  std::snprintf(r.label, sizeof r.label, "%s", label);
  r.a = take_event(ctx);
  r.b = take_event(ctx);
  if (!r.a || !r.b) return;
  if (!ext) (void)hipEventRecord(r.a, ctx->stream);
  ctx->prof.push_back(r);
  idx = (int)ctx->prof.size() - 1;
  if (ext) {
    a = r.a;
    b = r.b;
  }
}
ProfScope::~ProfScope() {
  if (idx >= 0 && !ext) (void)hipEventRecord(ctx->prof[idx].b, ctx->stream);
}

int check_launch(fa_ctx *ctx, const char *what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return set_err(ctx, FA_E_DEVICE, "%s launch: %s", what, hipGetErrorString(e));
  return FA_OK;
}

}  // namespace fa

using namespace fa;

extern "C" {

const char *fa_version(void) { return "fa_hip 0.1 gfx950"; }

int fa_ctx_create(int device, fa_ctx **out) {
  if (!out) return FA_E_INVALID;
  *out = nullptr;
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess || n <= 0) {
    (void)hipGetLastError();
    return FA_E_DEVICE;
  }
  if (device < 0 || device >= n) return FA_E_INVALID;
  if (hipSetDevice(device) != hipSuccess) return FA_E_DEVICE;
  hipDeviceProp_t prop;
  if (hipGetDeviceProperties(&prop, device) != hipSuccess) return FA_E_DEVICE;
  if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0) return FA_E_UNSUPPORTED;
  fa_ctx *ctx = new fa_ctx();
  ctx->device = device;
  ctx->num_cu = prop.multiProcessorCount;
  if (hipStreamCreateWithFlags(&ctx->stream, hipStreamNonBlocking) != hipSuccess) {
    delete ctx;
    return FA_E_DEVICE;
  }
  if (const int st = fa::mel_static_init(ctx)) {
    (void)hipStreamDestroy(ctx->stream);
    delete ctx;
    return st;
  }
  *out = ctx;
  return FA_OK;
}

void fa_ctx_destroy(fa_ctx *ctx) {
  if (!ctx) return;
  (void)hipSetDevice(ctx->device);
  (void)hipStreamSynchronize(ctx->stream);
  mel_static_release(ctx);
  for (auto &r : ctx->recs) {
    if (!r.live) continue;
    if (!r.view && r.ptr) (void)hipFree(r.ptr);
    if (r.aux) (void)hipFree(r.aux);
  }
  for (auto &kv : ctx->pool)
    for (void *p : kv.second) (void)hipFree(p);
  if (ctx->mel_tab) (void)hipFree(ctx->mel_tab);
  if (ctx->mel_scratch) (void)hipFree(ctx->mel_scratch);
  for (auto &p : ctx->prof) {
    (void)hipEventDestroy(p.a);
    (void)hipEventDestroy(p.b);
  }
  for (auto e : ctx->prof_free_events) (void)hipEventDestroy(e);
  for (auto &s : ctx->staged) {
    if (s.host) (void)hipHostFree(s.host);
    if (s.ev) (void)hipEventDestroy(s.ev);
  }
  (void)hipStreamDestroy(ctx->stream);
  delete ctx;
}

const char *fa_last_error(const fa_ctx *ctx) { return ctx ? ctx->err.c_str() : "null context"; }

int fa_sync(fa_ctx *ctx) {
  FA_HIP(ctx, hipStreamSynchronize(ctx->stream));
  return FA_OK;
}

// ── uploads / allocation ─────────────────────────────────────────────────
int fa_upload(fa_ctx *ctx, const float *data, int rows, int cols, fa_tensor *out) {
  size_t n = (size_t)rows * cols;
  TensorRec *r;
  FA_TRY(new_persistent(ctx, rows, cols, S_F32, n * 4, out, &r));
  if (n) FA_HIP(ctx, hipMemcpyAsync(r->ptr, data, n * 4, hipMemcpyHostToDevice, ctx->stream));
  FA_HIP(ctx, hipStreamSynchronize(ctx->stream));  // `data` may be reused by the caller right away
  return FA_OK;
}

// f16 weights are stored K-major (transposed) so the GEMM's B operand is read
// like its A operand: 8 consecutive k per lane, 16-byte loads.  The context
// owns this format, as GpuContext owns its tile-major one (compute.js:224-243).
int fa_upload_f16(fa_ctx *ctx, const float *data, int rows, int cols, fa_tensor *out) {
  size_t n = (size_t)rows * cols;
  std::vector<__half> h(n);
  for (int k = 0; k < rows; k++)
    for (int j = 0; j < cols; j++) h[(size_t)j * rows + k] = __float2half_rn(data[(size_t)k * cols + j]);
  TensorRec *r;
  FA_TRY(new_persistent(ctx, rows, cols, S_F16KM, n * 2, out, &r));
  if (n) FA_HIP(ctx, hipMemcpyAsync(r->ptr, h.data(), n * 2, hipMemcpyHostToDevice, ctx->stream));
  FA_HIP(ctx, hipStreamSynchronize(ctx->stream));
  return FA_OK;
}

int fa_upload_f16_rows(fa_ctx *ctx, const float *data, int rows, int cols, fa_tensor *out) {
  const size_t n = (size_t)rows * cols;
  std::vector<__half> h(n);
  for (size_t i = 0; i < n; i++) h[i] = __float2half_rn(data[i]);
  TensorRec *r;
  FA_TRY(new_tensor(ctx, rows, cols, S_F16RM, n * 2, out, &r));
  if (n) FA_HIP(ctx, hipMemcpyAsync(r->ptr, h.data(), n * 2, hipMemcpyHostToDevice, ctx->stream));
  FA_HIP(ctx, hipStreamSynchronize(ctx->stream));
  return FA_OK;
}

int fa_alloc(fa_ctx *ctx, int rows, int cols, fa_tensor *out) {
  return new_tensor(ctx, rows, cols, S_F32, (size_t)rows * cols * 4, out);
}

int fa_alloc_f16(fa_ctx *ctx, int rows, int cols, fa_tensor *out) {
  return new_tensor(ctx, rows, cols, S_F16RM, (size_t)rows * cols * 2, out);
}

int fa_upload_bytes(fa_ctx *ctx, const void *data, size_t nbytes, fa_tensor *out) {
  TensorRec *r;
  FA_TRY(new_persistent(ctx, 1, (int)std::min<size_t>(nbytes, 0x7fffffff), S_BYTES, nbytes, out, &r));
  if (nbytes) FA_HIP(ctx, hipMemcpyAsync(r->ptr, data, nbytes, hipMemcpyHostToDevice, ctx->stream));
  FA_HIP(ctx, hipStreamSynchronize(ctx->stream));
  return FA_OK;
}

int fa_tensor_info(fa_ctx *ctx, fa_tensor t, int *rows, int *cols, int *dtype) {
  TensorRec *r;
  FA_TRY(need(ctx, t, &r, "tensorInfo"));
  if (rows) *rows = r->rows;
  if (cols) *cols = r->cols;
  if (dtype) *dtype = r->kind == S_F32 ? FA_F32 : (r->kind == S_BYTES ? FA_BYTES : FA_F16);
  return FA_OK;
}

// freeTensor: f16 tensors and views are ignored (compute.js:1016-1020).
int fa_free_tensor(fa_ctx *ctx, fa_tensor t) {
  if (t == 0) return FA_OK;
  TensorRec *r = get(ctx, t);
  if (!r) return FA_E_INVALID;
  if (r->view || r->kind == S_F16KM || r->kind == S_F16RM) return FA_OK;
  uint32_t s = slot_of(t);
  if (r->arena) {
    for (auto &a : ctx->arenas)
      if (a.id == r->arena) {
        auto it = std::find(a.slots.begin(), a.slots.end(), s);
        if (it != a.slots.end()) a.slots.erase(it);
      }
  }
  pool_put(ctx, r->ptr, r->bytes);  // persistent storage joins the pool too (compute.js:1012-1020)
  release_slot(ctx, s);
  return FA_OK;
}

int fa_push_arena(fa_ctx *ctx, fa_arena *out) {
  Arena a;
  a.id = ctx->next_arena++;
  ctx->arenas.push_back(a);
  if (out) *out = a.id;
  return FA_OK;
}

int fa_pop_arena(fa_ctx *ctx, fa_arena handle) {
  if (ctx->arenas.empty()) return FA_OK;
  size_t i = ctx->arenas.size();
  if (handle == 0) {
    i = ctx->arenas.size() - 1;
  } else {
    for (size_t j = 0; j < ctx->arenas.size(); j++)
      if (ctx->arenas[j].id == handle) i = j;
    if (i == ctx->arenas.size()) return FA_OK;  // already closed: no-op like indexOf < 0
  }
  Arena a = ctx->arenas[i];
  ctx->arenas.erase(ctx->arenas.begin() + i);
  for (uint32_t s : a.slots) {
    TensorRec &r = ctx->recs[s];
    if (!r.live || r.arena != a.id) continue;
    pool_put(ctx, r.ptr, r.bytes);
    release_slot(ctx, s);
  }
  return FA_OK;
}

int fa_pin(fa_ctx *ctx, fa_tensor t, int to_parent) {
  TensorRec *r;
  FA_TRY(need(ctx, t, &r, "pin"));
  uint32_t s = slot_of(t);
  for (int ai = (int)ctx->arenas.size() - 1; ai >= 0; ai--) {
    Arena &a = ctx->arenas[ai];
    auto it = std::find(a.slots.begin(), a.slots.end(), s);
    if (it == a.slots.end()) continue;
    a.slots.erase(it);
    if (to_parent && ai > 0) {
      ctx->arenas[ai - 1].slots.push_back(s);
      r->arena = ctx->arenas[ai - 1].id;
    } else {
      r->arena = 0;  // persistent
    }
    return FA_OK;
  }
  return FA_OK;
}

int fa_trim_pool(fa_ctx *ctx, size_t budget) {
  if (ctx->pooled_bytes <= budget) return FA_OK;
  FA_HIP(ctx, hipStreamSynchronize(ctx->stream));
  std::vector<size_t> keys;
  for (auto &kv : ctx->pool) keys.push_back(kv.first);
  std::sort(keys.begin(), keys.end(), std::greater<size_t>());
  for (size_t k : keys) {
    auto &lst = ctx->pool[k];
    while (!lst.empty() && ctx->pooled_bytes > budget) {
      (void)hipFree(lst.back());
      lst.pop_back();
      ctx->pooled_bytes -= k;
    }
    if (lst.empty()) ctx->pool.erase(k);
    if (ctx->pooled_bytes <= budget) break;
  }
  return FA_OK;
}

int fa_pool_info(fa_ctx *ctx, size_t *pooled_bytes, uint64_t *created, uint64_t *created_bytes, uint64_t *reused) {
  if (pooled_bytes) *pooled_bytes = ctx->pooled_bytes;
  if (created) *created = ctx->created;
  if (created_bytes) *created_bytes = ctx->created_bytes;
  if (reused) *reused = ctx->reused;
  return FA_OK;
}

// ── readback ─────────────────────────────────────────────────────────────
static void host_from_device(const TensorRec *r, const void *src, float *out) {
  size_t n = (size_t)r->rows * r->cols;
  if (r->kind == S_F32) {
    std::memcpy(out, src, n * 4);
  } else if (r->kind == S_F16RM) {
    const __half *h = (const __half *)src;
    for (size_t i = 0; i < n; i++) out[i] = __half2float(h[i]);
  } else if (r->kind == S_F16KM) {  // back to [K,N] row-major
    const __half *h = (const __half *)src;
    for (int k = 0; k < r->rows; k++)
      for (int j = 0; j < r->cols; j++) out[(size_t)k * r->cols + j] = __half2float(h[(size_t)j * r->rows + k]);
  }
}

static size_t payload_bytes(const TensorRec *r) {
  size_t n = (size_t)r->rows * r->cols;
  return r->kind == S_F32 ? n * 4 : (r->kind == S_BYTES ? (size_t)r->cols : n * 2);
}

int fa_download(fa_ctx *ctx, fa_tensor t, float *out) {
  TensorRec *r;
  FA_TRY(need(ctx, t, &r, "download"));
  if (r->kind == S_BYTES) return set_err(ctx, FA_E_INVALID, "download: byte tensor");
  size_t nb = payload_bytes(r);
  if (r->kind == S_F32) {
    if (nb) FA_HIP(ctx, hipMemcpyAsync(out, r->ptr, nb, hipMemcpyDeviceToHost, ctx->stream));
    FA_HIP(ctx, hipStreamSynchronize(ctx->stream));
    return FA_OK;
  }
  std::vector<uint8_t> tmp(nb);
  if (nb) FA_HIP(ctx, hipMemcpyAsync(tmp.data(), r->ptr, nb, hipMemcpyDeviceToHost, ctx->stream));
  FA_HIP(ctx, hipStreamSynchronize(ctx->stream));
  host_from_device(r, tmp.data(), out);
  return FA_OK;
}

int fa_stage_download(fa_ctx *ctx, fa_tensor t, fa_staged *out) {
  TensorRec *r;
  FA_TRY(need(ctx, t, &r, "stageDownload"));
  if (r->kind == S_BYTES) return set_err(ctx, FA_E_INVALID, "stageDownload: byte tensor");
  Staged s;
  s.bytes = payload_bytes(r);
  s.kind = r->kind;
  s.rows = r->rows;
  s.cols = r->cols;
  FA_HIP(ctx, hipHostMalloc(&s.host, s.bytes ? s.bytes : 4, hipHostMallocDefault));
  FA_HIP(ctx, hipEventCreateWithFlags(&s.ev, hipEventDisableTiming));
  if (s.bytes) FA_HIP(ctx, hipMemcpyAsync(s.host, r->ptr, s.bytes, hipMemcpyDeviceToHost, ctx->stream));
  FA_HIP(ctx, hipEventRecord(s.ev, ctx->stream));
  uint32_t idx = (uint32_t)ctx->staged.size();
  for (uint32_t i = 0; i < ctx->staged.size(); i++)
    if (ctx->staged[i].host == nullptr && ctx->staged[i].ev == nullptr) {
      idx = i;
      break;
    }
  if (idx == ctx->staged.size()) {
    ctx->staged.push_back(s);
    ctx->staged_gen.push_back(1);
  } else {
    ctx->staged[idx] = s;
  }
  *out = ((uint64_t)ctx->staged_gen[idx] << 32) | (idx + 1);
  return FA_OK;
}

int fa_staged_read(fa_ctx *ctx, fa_staged h, float *out) {
  uint32_t idx = (uint32_t)(h & 0xffffffffu) - 1u, g = (uint32_t)(h >> 32);
  if (h == 0 || idx >= ctx->staged.size() || ctx->staged_gen[idx] != g)
    return set_err(ctx, FA_E_STATE, "StagedRead.read(): already consumed (single-use)");
  Staged &s = ctx->staged[idx];
  FA_HIP(ctx, hipEventSynchronize(s.ev));
  TensorRec tmp;
  tmp.rows = s.rows;
  tmp.cols = s.cols;
  tmp.kind = s.kind;
  host_from_device(&tmp, s.host, out);
  (void)hipHostFree(s.host);
  (void)hipEventDestroy(s.ev);
  s.host = nullptr;
  s.ev = nullptr;
  ctx->staged_gen[idx]++;
  return FA_OK;
}

int fa_rows_view(fa_ctx *ctx, fa_tensor t, int rows, fa_tensor *out) {
  TensorRec *r;
  FA_TRY(need(ctx, t, &r, "rowsView"));
  if (rows < 0 || rows > r->rows) return set_err(ctx, FA_E_INVALID, "rowsView: %d rows of a %d-row tensor", rows, r->rows);
  if (r->kind == S_F16KM) return set_err(ctx, FA_E_UNSUPPORTED, "rowsView of a K-major f16 weight");
  TensorRec copy = *r;
  uint32_t s = take_slot(ctx);
  TensorRec &v = ctx->recs[s];
  uint32_t g = v.gen;
  v = copy;
  v.gen = g;
  v.rows = rows;
  v.view = true;
  v.pooled = false;
  v.arena = 0;
  v.aux = nullptr;
  v.live = true;
  *out = handle_of(ctx, s);
  return FA_OK;
}

// ── batching: ops are always queued on the stream in order; a batch marks a
// recording scope and enforces the reference's non-reentrancy. ─────────────
int fa_begin_batch(fa_ctx *ctx) {
  if (ctx->batch_open) return set_err(ctx, FA_E_STATE, "beginBatch: a batch is already open");
  ctx->batch_open = true;
  return FA_OK;
}
int fa_end_batch(fa_ctx *ctx) {
  if (!ctx->batch_open) return set_err(ctx, FA_E_STATE, "endBatch without beginBatch");
  ctx->batch_open = false;
  return FA_OK;
}
int fa_batch_open(fa_ctx *ctx) { return ctx->batch_open ? 1 : 0; }

// ── profiler ──────────────────────────────────────────────────────────────
int fa_profile_start(fa_ctx *ctx, int max_ops) {
  for (auto &p : ctx->prof) {
    ctx->prof_free_events.push_back(p.a);
    ctx->prof_free_events.push_back(p.b);
  }
  ctx->prof.clear();
  ctx->prof_max = max_ops > 0 ? max_ops : 4096;
  ctx->prof.reserve(ctx->prof_max);
  ctx->prof_on = true;
  return FA_OK;
}

int fa_profile_only(fa_ctx *ctx, const char *prefix) {
  ctx->prof_filter = prefix ? prefix : "";
  return FA_OK;
}

int fa_profile_end(fa_ctx *ctx, int cap, char (*labels)[48], float *ms, int *count) {
  ctx->prof_on = false;
  FA_HIP(ctx, hipStreamSynchronize(ctx->stream));
  int n = (int)ctx->prof.size();
  for (int i = 0; i < n && i < cap; i++) {
    float t = 0;
    (void)hipEventElapsedTime(&t, ctx->prof[i].a, ctx->prof[i].b);
    if (ms) ms[i] = t;
    if (labels) std::snprintf(labels[i], 48, "%s", ctx->prof[i].label);
  }
  if (count) *count = n;
  for (auto &p : ctx->prof) {
    ctx->prof_free_events.push_back(p.a);
    ctx->prof_free_events.push_back(p.b);
  }
  ctx->prof.clear();
  return FA_OK;
}

}  // extern "C"
