// Streaming FastConformer encode on the fused encoder: per-chunk passes that
// continue from device-resident caches.
//
// Function (src/engines/asr-parakeet/streaming-encoder.js): a stream computes
// the offline chunked-causal encoder's frames (attention limited to
// [chunk start - left, chunk end + right], causal depthwise conv) while mel
// frames arrive; frames of a chunk become final once the chunk (plus, with
// right context, a provisional lookahead that is recomputed next pass) has
// been seen.
//
// Design here: a pass is one run of the fused encoder's kernel sequence over
// the pass's mel rows (pass_launch in encoder.hip, one window) with
//  - the subsampling padded in time only at the stream's edges (top pad on
//    the first pass, bottom pad at the flush) and fed the 14 mel rows of
//    look-back its first output needs;
//  - attention over [the layer's cached keys ; the pass's keys] with the chunk
//    mask expressed relative to the pass start (passes start on chunk
//    boundaries) and the positional term read from the encoder's load-time
//    table;
//  - the causal depthwise conv reading its k-1 frames of history from a cache.
// The caches live on the device and are double-buffered: a pass reads one
// set and writes the next (K / V of the last `left` emitted frames per layer
// in f16, the depthwise conv's k-1 input rows per layer in f32), so nothing
// is copied back to the host but the emitted frames.
//
// Several streams of one encoder (fa_stream_push_many) whose next passes have
// the same shape (rows, pads, cached keys) run as ONE batched pass: window w
// of the pass is stream w, its caches named by tables (KvSlots, CcSlots),
// so the weights are read once for all of them (a pass over a few frames is
// bound by reading the ~1.2 GB of f16 weights).  Passes run on the encoder's
// stream lanes (a HIP stream, workspace and staging buffers each); groups of
// different shapes run on different lanes at once.  Steady-state passes (full
// key caches, no pads) are replayed from captured hipGraphs keyed by their
// shape and cache table.
#include <algorithm>
#include <cstring>
#include <map>
#include <tuple>
#include <vector>

#include "fa_internal.h"
#include "encoder_impl.h"

using namespace fa;

struct fa_stream {
  fa_ctx *ctx = nullptr;
  fa_encoder *enc = nullptr;
  int C = 0, left = 0, right = 0, B = 0, max_chunk = 64;
  int dMax = 0, Pn = 0;
  int subT = 0;        // emitted frames so far
  bool flushed = false;
  std::vector<float> fifo;  // mel frames [frames][melBins], fifo[0] = global frame fifo_start
  long fifo_start = 0;
  _Float16 *kc[2] = {nullptr, nullptr}, *vc[2] = {nullptr, nullptr};  // [layers][left][D]
  float *cc[2] = {nullptr, nullptr};                                  // [layers][8][D]
  int cur = 0, Lc = 0;
  // a pass failed after it had started changing this stream's caches: its
  // state is unknown, so later pushes are refused
  bool failed = false;
};

// One lane of stream passes: HIP stream, workspace, the pass's mel rows and
// output frames, the device cache table, captured passes.
struct StreamLane {
  EncWs ws;
  hipStream_t hs = nullptr;
  hipEvent_t done = nullptr, in = nullptr;
  float *mel_dev = nullptr, *x_dev = nullptr;
  size_t mel_cap = 0, x_cap = 0;
  uint64_t buf_gen = 0;  // moves when mel_dev / x_dev are reallocated
  std::vector<EncWs::Captured> graphs;
  uint64_t graph_clock = 0;
  // pinned host staging of a pass's mel rows, two buffers used in turn (a
  // buffer is rewritten only after its previous copy has completed)
  float *stage[2] = {nullptr, nullptr};
  size_t stage_cap[2] = {0, 0};
  hipEvent_t staged[2] = {nullptr, nullptr};
  int next_stage = 0;
};

namespace {

constexpr int kLookback = 14;  // mel rows before 8*subT the next pass's first frame reads (three k=3 stride-2 convs)
constexpr int kKT = 9;

// The emitted frames of every window of a batched pass: rows [w nq, w nq +
// nemit) of x to window w's output tensor.
struct OutRows {
  float *dst[kMaxStreamGroup];
};
__global__ __launch_bounds__(256) void stream_out_kernel(const float4 *__restrict__ x, int nq, int nemit, int D4, OutRows o) {
  const int w = blockIdx.y;
  const long n4 = (long)nemit * D4;
  const float4 *src = x + (size_t)w * nq * D4;
  float4 *dst = reinterpret_cast<float4 *>(o.dst[w]);
  for (long i = (long)blockIdx.x * 256 + threadIdx.x; i < n4; i += (long)gridDim.x * 256) dst[i] = src[i];
}

int lane_grow(fa_ctx *ctx, StreamLane *L, void **buf, size_t *cap, size_t need) {
  if (need <= *cap) return FA_OK;
  if (*buf) {
    (void)hipStreamSynchronize(L->hs);
    (void)hipFree(*buf);
    *buf = nullptr;
  }
  *buf = dev_alloc(ctx, need);
  if (!*buf) return FA_E_OOM;
  *cap = need;
  L->buf_gen++;
  return FA_OK;
}

int get_lane(fa_ctx *ctx, fa_encoder *e, int l, StreamLane **out) {
  if (!e->slane[l]) {
    StreamLane *L = new StreamLane();
    e->slane[l] = L;
    if (hipStreamCreateWithFlags(&L->hs, hipStreamNonBlocking) != hipSuccess || hipEventCreateWithFlags(&L->done, hipEventDisableTiming) != hipSuccess ||
        hipEventCreateWithFlags(&L->in, hipEventDisableTiming) != hipSuccess || hipEventCreateWithFlags(&L->staged[0], hipEventDisableTiming) != hipSuccess ||
        hipEventCreateWithFlags(&L->staged[1], hipEventDisableTiming) != hipSuccess)
      return set_err(ctx, FA_E_DEVICE, "encodeStreamPush: creating a stream lane failed");
  }
  *out = e->slane[l];
  return FA_OK;
}

// While a pass is queued, the context's launches go to the lane's HIP stream
// and the encoder's workspace is the lane's.
struct PassScope {
  fa_ctx *c;
  fa_encoder *e;
  hipStream_t s0;
  EncWs *w0;
  PassScope(fa_ctx *ctx, fa_encoder *enc, StreamLane *L) : c(ctx), e(enc), s0(ctx->stream), w0(enc->ws_ovr) {
    c->stream = L->hs;
    e->ws_ovr = &L->ws;
  }
  ~PassScope() {
    c->stream = s0;
    e->ws_ovr = w0;
  }
};

// The shape of a stream's next pass: m mel rows at the FIFO head, pads,
// nComp frames computed, the first nemit emitted.
struct PassPlan {
  int m = 0, pt = 0, pb = 0, nComp = 0, nemit = 0;
};

// The next chunk pass the buffered frames allow (false: none yet).
bool next_pass(const fa_stream *st, PassPlan *p) {
  const int MB = st->enc->cfg.melBins;
  const int M = (int)(st->fifo.size() / MB);
  // frames a pass can finish: the first pass reads 8*nComp - 7 rows (top
  // padded), later passes 8*nComp + 7 (14 rows of look-back); nComp
  // includes the provisional lookahead B, and n is a whole number of chunks
  int n = st->subT == 0 ? (M + 7) / 8 - st->B : (M - 7 >= 0 ? (M - 7) / 8 : -1) - st->B;
  n = std::min(n, st->max_chunk);
  n -= ((n % st->C) + st->C) % st->C;
  // the next pass reads kLookback mel rows before 8 * subT, so the first pass
  // emits at least two frames (matters for one-frame chunks only; frames do not
  // depend on where passes split the stream)
  if (n < (st->subT == 0 ? std::max(st->C, 2) : st->C)) return false;
  p->nComp = n + st->B;
  p->nemit = n;
  p->m = st->subT == 0 ? 8 * p->nComp - 7 : 8 * p->nComp + 7;
  p->pt = st->subT == 0 ? st->enc->opts.sub_pad_t : 0;
  p->pb = 0;
  return true;
}

// After a chunk pass: drop the FIFO rows the next pass no longer reads.
void advance_fifo(fa_stream *st, int nemit) {
  const int MB = st->enc->cfg.melBins;
  st->subT += nemit;
  const long keep_from = 8L * st->subT - kLookback;
  const long drop = keep_from - st->fifo_start;  // >= 0: subT >= 2 after the first pass
  st->fifo.erase(st->fifo.begin(), st->fifo.begin() + (size_t)drop * MB);
  st->fifo_start = keep_from;
}

// One pass of n streams with the same plan and the same cached-key count, on
// lane L: window w = sts[w]; its emitted frames are appended to outs[w].
// The stream state (cache half, cached-key count, FIFO, emitted frames) moves
// only once the pass is queued, all of it together: a failure before that
// (sizes, allocations) leaves every stream as it was, so the same push can be
// repeated; a failure while the pass is being queued marks the streams failed.
// advance: drop the FIFO rows the next pass no longer reads (false: a flush).
int run_group(fa_ctx *ctx, fa_encoder *e, StreamLane *L, fa_stream *const *sts, int n, const PassPlan &pl, std::vector<fa_tensor> *const *outs,
              bool advance) {
  PassScope scope(ctx, e, L);
  const fa_encoder_cfg &c = e->cfg;
  const int MB = c.melBins, D = c.D, m = pl.m, nComp = pl.nComp, nemit = pl.nemit;
  fa_stream *s0 = sts[0];
  if (n < 1 || n > kMaxStreamGroup) return set_err(ctx, FA_E_INVALID, "stream pass: %d streams in one pass", n);
  if (D % 4) return set_err(ctx, FA_E_UNSUPPORTED, "stream pass: D %d not a multiple of 4", D);
  std::vector<int32_t> lens(n, m);
  PassGeom g;
  FA_TRY(pass_geometry(ctx, e, lens.data(), n, 0, pl.pt, pl.pb, &g));
  if (g.M != n * nComp) return set_err(ctx, FA_E_STATE, "stream pass: %d mel rows give %d frames, expected %d", m, g.M / n, nComp);
  if (s0->Lc + nComp > 256) return set_err(ctx, FA_E_UNSUPPORTED, "stream pass: %d cached + %d new keys (at most 256)", s0->Lc, nComp);
  FA_TRY(pass_workspace(ctx, e, g, c.layers, true));
  // the windows' output tensors first: nothing is queued and no state moves
  // unless all of them exist
  OutRows orows{};
  std::vector<fa_tensor> mine;
  for (int w = 0; w < n; w++) {
    fa_tensor o;
    TensorRec *ro;
    const int st = new_tensor(ctx, nemit, D, S_F32, (size_t)nemit * D * 4, &o, &ro);
    if (st != FA_OK) {
      for (fa_tensor t : mine) (void)fa_free_tensor(ctx, t);
      return st;
    }
    orows.dst[w] = (float *)ro->ptr;
    mine.push_back(o);
  }
  auto give_back = [&]() {
    for (fa_tensor t : mine) (void)fa_free_tensor(ctx, t);
    return FA_OK;
  };
  // from the first queued operation on, a failure leaves the caches unknown
  auto fail = [&](int st) {
    for (int w = 0; w < n; w++) sts[w]->failed = true;
    give_back();
    return st;
  };
  {
    int st = lane_grow(ctx, L, (void **)&L->mel_dev, &L->mel_cap, (size_t)n * m * MB * 4);
    if (st == FA_OK) st = lane_grow(ctx, L, (void **)&L->x_dev, &L->x_cap, (size_t)n * nComp * D * 4);
    if (st != FA_OK) {
      give_back();
      return st;
    }
  }
  {  // the windows' mel rows, copied from the FIFOs into pinned staging, then to the device
    const int b = L->next_stage;
    L->next_stage ^= 1;
    const size_t bytes = (size_t)n * m * MB * 4;
    if (hipEventSynchronize(L->staged[b]) != hipSuccess) {  // this buffer's previous copy (two passes back) is done
      give_back();
      return set_err(ctx, FA_E_DEVICE, "stream pass: staging wait");
    }
    if (bytes > L->stage_cap[b]) {
      if (L->stage[b]) (void)hipHostFree(L->stage[b]);
      L->stage[b] = nullptr;
      L->stage_cap[b] = 0;
      if (hipHostMalloc((void **)&L->stage[b], bytes, hipHostMallocDefault) != hipSuccess) {
        L->stage[b] = nullptr;
        give_back();
        return set_err(ctx, FA_E_OOM, "stream pass: pinned staging of %zu bytes", bytes);
      }
      L->stage_cap[b] = bytes;
    }
    for (int w = 0; w < n; w++) std::memcpy(L->stage[b] + (size_t)w * m * MB, sts[w]->fifo.data(), (size_t)m * MB * 4);
    if (hipMemcpyAsync(L->mel_dev, L->stage[b], bytes, hipMemcpyHostToDevice, L->hs) != hipSuccess ||
        hipEventRecord(L->staged[b], L->hs) != hipSuccess)
      return fail(set_err(ctx, FA_E_DEVICE, "stream pass: mel upload"));
  }
  KvSlots kv{};
  CcSlots cc{};
  for (int w = 0; w < n; w++) {
    fa_stream *st = sts[w];
    kv.kc_in[w] = st->kc[st->cur];
    kv.vc_in[w] = st->vc[st->cur];
    kv.kc_out[w] = st->kc[st->cur ^ 1];
    kv.vc_out[w] = st->vc[st->cur ^ 1];
    cc.cc_in[w] = st->cc[st->cur];
    cc.cc_out[w] = st->cc[st->cur ^ 1];
  }
  StreamPass sp;
  sp.Lc = s0->Lc;
  sp.nemit = nemit;
  sp.keep = std::min(s0->left, s0->Lc + nemit);
  sp.chunk = s0->C;
  sp.left = s0->left;
  sp.right = s0->right;
  sp.kv = kv;
  sp.cc = cc;
  sp.Pn = s0->Pn;
  sp.dMax = s0->dMax;
  sp.kv_ld = s0->left;
  auto launch = [&]() { return pass_launch(ctx, e, g, L->mel_dev, L->x_dev, c.layers, &sp); };
  const char *ge = getenv("FA_GRAPH");
  const bool steady = s0->Lc == s0->left && pl.pb == 0 && pl.pt == 0;
  if (steady && !ctx->prof_on && !(ge && ge[0] == '0')) {
    // the cache tables are baked into the launches, so every pointer in them
    // is part of the key (a new stream may get a freed stream's address for
    // one cache and not for another); a stable set of streams alternates
    // between two captured passes (the caches' double buffers)
    std::vector<int64_t> key = {(int64_t)e->ws_gen, (int64_t)L->buf_gen, n, m, nComp, nemit};
    for (int w = 0; w < n; w++)
      for (const void *p : {(const void *)kv.kc_in[w], (const void *)kv.vc_in[w], (const void *)kv.kc_out[w], (const void *)kv.vc_out[w],
                            (const void *)cc.cc_in[w], (const void *)cc.cc_out[w]})
        key.push_back((int64_t)(uintptr_t)p);
    EncWs::Captured *hit = nullptr;
    for (auto &gr : L->graphs)
      if (gr.key == key) hit = &gr;
    if (!hit) {
      if (hipStreamBeginCapture(ctx->stream, hipStreamCaptureModeThreadLocal) != hipSuccess)
        return fail(set_err(ctx, FA_E_DEVICE, "stream pass: graph capture"));
      const int rc = launch();
      hipGraph_t graph = nullptr;
      const hipError_t ce = hipStreamEndCapture(ctx->stream, &graph);
      if (rc != FA_OK) {
        if (graph) (void)hipGraphDestroy(graph);
        return fail(rc);
      }
      if (ce != hipSuccess) return fail(set_err(ctx, FA_E_DEVICE, "stream pass: graph capture: %s", hipGetErrorString(ce)));
      hipGraphExec_t exec = nullptr;
      const hipError_t ie = hipGraphInstantiateWithFlags(&exec, graph, 0);
      (void)hipGraphDestroy(graph);
      if (ie != hipSuccess) return fail(set_err(ctx, FA_E_DEVICE, "stream pass: graph instantiate: %s", hipGetErrorString(ie)));
      if (L->graphs.size() >= 16) {  // two per stable set of streams and chunk shape
        size_t lru = 0;
        for (size_t i = 1; i < L->graphs.size(); i++)
          if (L->graphs[i].used < L->graphs[lru].used) lru = i;
        (void)hipStreamSynchronize(ctx->stream);
        (void)hipGraphExecDestroy(L->graphs[lru].exec);
        L->graphs.erase(L->graphs.begin() + lru);
      }
      L->graphs.push_back({key, exec, 0});
      hit = &L->graphs.back();
    }
    hit->used = ++L->graph_clock;
    if (hipGraphLaunch(hit->exec, ctx->stream) != hipSuccess) return fail(set_err(ctx, FA_E_DEVICE, "stream pass: graph launch"));
  } else {
    const int rc = launch();
    if (rc != FA_OK) return fail(rc);
  }
  {
    ProfScope ps(ctx, "stream_out");
    const long n4 = (long)nemit * (D / 4);
    FA_LAUNCH(ps, stream_out_kernel, dim3((unsigned)std::max<long>(1, std::min<long>(cdiv(n4, 256), 64)), n), dim3(256), 0, ctx->stream,
              (const float4 *)L->x_dev, nComp, nemit, D / 4, orows);
    const int rc = check_launch(ctx, "stream_out");
    if (rc != FA_OK) return fail(rc);
  }
  // the pass is queued: every window's caches moved to the other buffer half,
  // its FIFO moves past the rows this pass consumed, the frames are its own
  for (int w = 0; w < n; w++) {
    sts[w]->cur ^= 1;
    sts[w]->Lc = sp.keep;
    if (advance) advance_fifo(sts[w], nemit);
    outs[w]->push_back(mine[w]);
  }
  return FA_OK;
}

int emit(fa_stream *st, std::vector<fa_tensor> &outs, fa_tensor *out) {
  *out = 0;
  if (outs.empty()) return FA_OK;
  if (outs.size() == 1) {
    *out = outs[0];
    return FA_OK;
  }
  const int rc = fa_concat_rows(st->ctx, outs.data(), (int)outs.size(), out);
  for (fa_tensor t : outs) (void)fa_free_tensor(st->ctx, t);
  return rc;
}

// Queue rounds of passes until no stream has a pass ready: in each round the
// streams with a ready pass are grouped by (plan, cached keys), each group is
// one batched pass, groups go round-robin to the lanes; a round starts after
// the previous one (a stream's passes follow each other through its caches).
// Lanes start after the work queued on the context stream, and the context
// stream waits for every lane used.
int run_rounds(fa_ctx *ctx, fa_encoder *e, std::vector<fa_stream *> &sts, std::vector<std::vector<fa_tensor>> &frames, const PassPlan *flush) {
  const int nl = std::max(1, e->nlanes);
  StreamLane *L0;
  FA_TRY(get_lane(ctx, e, 0, &L0));
  FA_HIP(ctx, hipEventRecord(L0->in, ctx->stream));
  std::vector<bool> used(nl, false);
  int rc = FA_OK;
  for (int round = 0; rc == FA_OK; round++) {
    // (plan, Lc) -> member indices
    std::map<std::tuple<int, int, int, int, int, int>, std::vector<int>> groups;
    for (int i = 0; i < (int)sts.size(); i++) {
      PassPlan p;
      if (flush) {
        if (round > 0) continue;
        p = *flush;
      } else if (!next_pass(sts[i], &p)) {
        continue;
      }
      groups[std::make_tuple(p.m, p.pt, p.pb, p.nComp, p.nemit, sts[i]->Lc)].push_back(i);
    }
    if (groups.empty()) break;
    std::vector<bool> wait_prev(nl, round > 0);
    int k = 0;
    for (auto &kv : groups) {
      const auto &key = kv.first;
      PassPlan p;
      p.m = std::get<0>(key);
      p.pt = std::get<1>(key);
      p.pb = std::get<2>(key);
      p.nComp = std::get<3>(key);
      p.nemit = std::get<4>(key);
      const std::vector<int> &mem = kv.second;
      for (size_t b0 = 0; b0 < mem.size() && rc == FA_OK; b0 += kMaxStreamGroup, k++) {
        const int nb = (int)std::min<size_t>(kMaxStreamGroup, mem.size() - b0);
        const int l = k % nl;
        StreamLane *L;
        if ((rc = get_lane(ctx, e, l, &L)) != FA_OK) break;
        if (!used[l]) {
          if (hipStreamWaitEvent(L->hs, L0->in, 0) != hipSuccess) rc = set_err(ctx, FA_E_DEVICE, "stream pass: lane wait");
          used[l] = true;
        }
        if (wait_prev[l]) {  // after every lane's previous round
          for (int j = 0; j < nl; j++)
            if (e->slane[j] && j != l) (void)hipStreamWaitEvent(L->hs, e->slane[j]->done, 0);
          wait_prev[l] = false;
        }
        if (rc != FA_OK) break;
        std::vector<fa_stream *> g(nb);
        std::vector<std::vector<fa_tensor> *> o(nb);
        for (int w = 0; w < nb; w++) {
          g[w] = sts[mem[b0 + w]];
          o[w] = &frames[mem[b0 + w]];
        }
        rc = run_group(ctx, e, L, g.data(), nb, p, o.data(), !flush);
      }
      if (rc != FA_OK) break;
    }
    for (int l = 0; l < nl; l++)
      if (used[l]) (void)hipEventRecord(e->slane[l]->done, e->slane[l]->hs);
    if (flush) break;
  }
  for (int l = 0; l < nl; l++)
    if (used[l]) (void)hipStreamWaitEvent(ctx->stream, e->slane[l]->done, 0);
  return rc;
}

}  // namespace

void fa::stream_lanes_free(fa_encoder *e) {
  for (auto &L : e->slane) {
    if (!L) continue;
    if (L->hs) (void)hipStreamSynchronize(L->hs);
    for (auto &g : L->graphs)
      if (g.exec) (void)hipGraphExecDestroy(g.exec);
    encoder_ws_free(L->ws);
    for (void *p : {(void *)L->mel_dev, (void *)L->x_dev})
      if (p) (void)hipFree(p);
    for (int b = 0; b < 2; b++) {
      if (L->stage[b]) (void)hipHostFree(L->stage[b]);
      if (L->staged[b]) (void)hipEventDestroy(L->staged[b]);
    }
    if (L->done) (void)hipEventDestroy(L->done);
    if (L->in) (void)hipEventDestroy(L->in);
    if (L->hs) (void)hipStreamDestroy(L->hs);
    delete L;
    L = nullptr;
  }
}

extern "C" {

int fa_stream_create(fa_ctx *ctx, fa_encoder *enc, int lookahead_chunks, int max_chunk, fa_stream **out) {
  if (!ctx || !out) return FA_E_INVALID;
  *out = nullptr;
  if (!enc || enc->ctx != ctx) return set_err(ctx, FA_E_INVALID, "createEncodeStream: encoder belongs to another context");
  const fa_encoder_opts &o = enc->opts;
  if (o.att_chunk <= 0 || !o.conv_causal) return set_err(ctx, FA_E_INVALID, "createEncodeStream: needs a streaming model (attention chunk + causal conv)");
  if (o.sub_pad_t != 2) return set_err(ctx, FA_E_UNSUPPORTED, "createEncodeStream: the subsampling continuation needs a top pad of 2");
  if (o.att_right > 0 && lookahead_chunks < 1) return set_err(ctx, FA_E_INVALID, "createEncodeStream: right context needs lookahead_chunks >= 1");
  if (lookahead_chunks < 0 || max_chunk < o.att_chunk || max_chunk > 128) return set_err(ctx, FA_E_INVALID, "createEncodeStream: lookahead %d / max_chunk %d", lookahead_chunks, max_chunk);
  fa_stream *st = new fa_stream();
  st->ctx = ctx;
  st->enc = enc;
  st->C = o.att_chunk;
  st->left = o.att_left;
  st->right = o.att_right;
  st->B = o.att_right > 0 ? lookahead_chunks * o.att_chunk : 0;
  st->max_chunk = max_chunk;
  st->dMax = st->left + st->C - 1;
  st->Pn = st->dMax + st->C - 1 + st->right + 1;  // distances dMax .. -(C-1+right)
  if (enc->maxT - 1 < st->dMax || enc->maxT - 1 < st->C - 1 + st->right) {
    delete st;
    return set_err(ctx, FA_E_INVALID, "createEncodeStream: the encoder's max_T %d must exceed left + chunk (%d)", enc->maxT, st->dMax + 1);
  }
  const int L = enc->cfg.layers, D = enc->cfg.D;
  const size_t kv = (size_t)L * std::max(1, st->left) * D * 2, cb = (size_t)L * (kKT - 1) * D * 4;
  for (int i = 0; i < 2; i++) {
    st->kc[i] = (_Float16 *)dev_alloc(ctx, kv);
    st->vc[i] = (_Float16 *)dev_alloc(ctx, kv);
    st->cc[i] = (float *)dev_alloc(ctx, cb);
    if (!st->kc[i] || !st->vc[i] || !st->cc[i]) {
      fa_stream_destroy(st);
      return FA_E_OOM;
    }
  }
  // the first pass sees a zero depthwise-conv history (the offline causal pad)
  if (hipMemsetAsync(st->cc[0], 0, cb, ctx->stream) != hipSuccess) {
    fa_stream_destroy(st);
    return set_err(ctx, FA_E_DEVICE, "createEncodeStream: clearing the conv cache failed");
  }
  *out = st;
  return FA_OK;
}

int fa_stream_push(fa_stream *st, const float *mel, int count, fa_tensor *out) {
  if (!st || !out) return FA_E_INVALID;
  return fa_stream_push_many(1, &st, &mel, &count, out);
}

int fa_stream_push_many(int n, fa_stream *const *sts, const float *const *mels, const int *counts, fa_tensor *outs) {
  if (n <= 0 || !sts || !mels || !counts || !outs) return FA_E_INVALID;
  for (int i = 0; i < n; i++) {
    if (!sts[i]) return FA_E_INVALID;
    outs[i] = 0;
  }
  fa_ctx *ctx = sts[0]->ctx;
  fa_encoder *e = sts[0]->enc;
  for (int i = 0; i < n; i++) {
    fa_stream *st = sts[i];
    if (st->ctx != ctx || st->enc != e) return set_err(ctx, FA_E_INVALID, "encodeStreamPush: streams of different encoders in one call");
    for (int j = 0; j < i; j++)
      if (sts[j] == st) return set_err(ctx, FA_E_INVALID, "encodeStreamPush: stream %d repeats stream %d in one call", i, j);
    if (st->flushed) return set_err(ctx, FA_E_STATE, "encodeStreamPush: stream already flushed; create a new stream");
    if (st->failed) return set_err(ctx, FA_E_STATE, "encodeStreamPush: a pass of this stream failed earlier; create a new stream");
    if (counts[i] < 0 || (counts[i] > 0 && !mels[i])) return set_err(ctx, FA_E_INVALID, "encodeStreamPush: %d frames", counts[i]);
  }
  const int MB = e->cfg.melBins;
  std::vector<fa_stream *> v(sts, sts + n);
  for (int i = 0; i < n; i++) {  // mel-major [melBins][count] -> frame-major FIFO rows
    fa_stream *st = sts[i];
    const size_t old = st->fifo.size() / MB;
    const int count = counts[i];
    st->fifo.resize((old + count) * MB);
    for (int t = 0; t < count; t++)
      for (int ch = 0; ch < MB; ch++) st->fifo[(old + t) * MB + ch] = mels[i][(size_t)ch * count + t];
  }
  std::vector<std::vector<fa_tensor>> frames(n);
  // the FIFO rows stay appended on failure: a stream whose passes did not
  // start can be pushed to again; one whose passes ran in this call lost their
  // frames with the error and is marked failed
  int rc = run_rounds(ctx, e, v, frames, nullptr);
  std::vector<bool> moved(n);
  for (int i = 0; i < n; i++) moved[i] = !frames[i].empty();
  for (int i = 0; i < n; i++) {
    if (rc == FA_OK)
      rc = emit(sts[i], frames[i], &outs[i]);
    else
      for (fa_tensor t : frames[i]) (void)fa_free_tensor(ctx, t);
  }
  if (rc != FA_OK)
    for (int i = 0; i < n; i++) {
      if (moved[i]) sts[i]->failed = true;
      if (outs[i]) {
        (void)fa_free_tensor(ctx, outs[i]);
        outs[i] = 0;
      }
    }
  return rc;
}

int fa_stream_flush(fa_stream *st, fa_tensor *out) {
  if (!st || !out) return FA_E_INVALID;
  fa_ctx *ctx = st->ctx;
  *out = 0;
  if (st->flushed) return set_err(ctx, FA_E_STATE, "encodeStreamFlush: stream already flushed");
  if (st->failed) return set_err(ctx, FA_E_STATE, "encodeStreamFlush: a pass of this stream failed earlier");
  st->flushed = true;
  const int MB = st->enc->cfg.melBins;
  const int M = (int)(st->fifo.size() / MB);
  if (M == 0) return FA_OK;
  // the tail: top pad only if nothing was emitted yet, bottom pad (the signal end)
  const int pt = st->subT == 0 ? st->enc->opts.sub_pad_t : 0, pb = st->enc->opts.sub_pad_b;
  int T = M;
  for (int i = 0; i < 3; i++) {
    const int q = T + pt + pb - 3;
    T = q < 0 ? 0 : q / 2 + 1;
  }
  if (T <= 0) return FA_OK;
  if (T > st->enc->maxT) return set_err(ctx, FA_E_UNSUPPORTED, "encodeStreamFlush: %d tail frames > max_T", T);
  PassPlan p;
  p.m = M;
  p.pt = pt;
  p.pb = pb;
  p.nComp = T;
  p.nemit = T;
  std::vector<fa_stream *> v{st};
  std::vector<std::vector<fa_tensor>> frames(1);
  const int rc = run_rounds(ctx, st->enc, v, frames, &p);
  if (rc != FA_OK) {
    for (fa_tensor t : frames[0]) (void)fa_free_tensor(ctx, t);
    return rc;
  }
  st->fifo.clear();
  return emit(st, frames[0], out);
}

void fa_stream_destroy(fa_stream *st) {
  if (!st) return;
  (void)hipStreamSynchronize(st->ctx->stream);  // the context stream waits for every pass of the stream's pushes
  for (int i = 0; i < 2; i++)
    for (void *p : {(void *)st->kc[i], (void *)st->vc[i], (void *)st->cc[i]})
      if (p) (void)hipFree(p);
  delete st;
}

}  // extern "C"
