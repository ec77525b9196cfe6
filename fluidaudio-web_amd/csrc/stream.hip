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
// is copied back to the host but the emitted frames.  Steady-state passes
// (full key cache, same chunk size) repeat one of two kernel sequences and
// are replayed from captured hipGraphs.
#include <algorithm>
#include <cstring>
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
  float *mel_dev = nullptr, *x_dev = nullptr;
  size_t mel_cap = 0, x_cap = 0;
  uint64_t buf_gen = 0;  // moves when mel_dev / x_dev are reallocated
  std::vector<EncWs::Captured> graphs;
  uint64_t graph_clock = 0;
  // Each stream's passes run on a HIP stream of its own with a workspace of
  // its own, so several streams' passes (fa_stream_push_many) are in flight
  // together.  A push starts after the work queued on the context stream
  // (event `in`) and the context stream waits for it (event `done`), so its
  // frames are ordinary context tensors.
  EncWs ws;
  hipStream_t hs = nullptr;
  hipEvent_t in = nullptr, done = nullptr;
};

namespace {

constexpr int kLookback = 14;  // mel rows before 8*subT the next pass's first frame reads (three k=3 stride-2 convs)
constexpr int kKT = 9;

int grow_buf(fa_stream *st, void **buf, size_t *cap, size_t need) {
  if (need <= *cap) return FA_OK;
  if (*buf) {
    (void)hipStreamSynchronize(st->ctx->stream);
    (void)hipFree(*buf);
    *buf = nullptr;
  }
  *buf = dev_alloc(st->ctx, need);
  if (!*buf) return FA_E_OOM;
  *cap = need;
  st->buf_gen++;
  return FA_OK;
}

// While a pass is queued, the context's launches go to the stream's HIP stream
// and the encoder's workspace is the stream's.
struct PassScope {
  fa_ctx *c;
  fa_encoder *e;
  hipStream_t s0;
  EncWs *w0;
  explicit PassScope(fa_stream *st) : c(st->ctx), e(st->enc), s0(st->ctx->stream), w0(st->enc->ws_ovr) {
    c->stream = st->hs;
    e->ws_ovr = &st->ws;
  }
  ~PassScope() {
    c->stream = s0;
    e->ws_ovr = w0;
  }
};

// One pass over m mel rows at the FIFO head: nComp frames computed, the first
// nemit emitted (appended to `outs` as a [nemit, D] tensor) and cached.
int run_pass(fa_stream *st, int m, int pt, int pb, int nComp, int nemit, std::vector<fa_tensor> &outs) {
  PassScope scope(st);
  fa_ctx *ctx = st->ctx;
  fa_encoder *e = st->enc;
  const fa_encoder_cfg &c = e->cfg;
  const int MB = c.melBins, D = c.D;
  const int32_t len = m;
  PassGeom g;
  FA_TRY(pass_geometry(ctx, e, &len, 1, 0, pt, pb, &g));
  if (g.M != nComp) return set_err(ctx, FA_E_STATE, "stream pass: %d mel rows give %d frames, expected %d", m, g.M, nComp);
  if (st->Lc + nComp > 256) return set_err(ctx, FA_E_UNSUPPORTED, "stream pass: %d cached + %d new keys (at most 256)", st->Lc, nComp);
  FA_TRY(pass_workspace(ctx, e, g, c.layers, true));
  FA_TRY(grow_buf(st, (void **)&st->mel_dev, &st->mel_cap, (size_t)m * MB * 4));
  FA_TRY(grow_buf(st, (void **)&st->x_dev, &st->x_cap, (size_t)nComp * D * 4));
  FA_HIP(ctx, hipMemcpyAsync(st->mel_dev, st->fifo.data(), (size_t)m * MB * 4, hipMemcpyHostToDevice, ctx->stream));
  FA_HIP(ctx, hipStreamSynchronize(ctx->stream));  // the FIFO is edited once this pass is queued
  StreamPass sp;
  sp.Lc = st->Lc;
  sp.nemit = nemit;
  sp.keep = std::min(st->left, st->Lc + nemit);
  sp.chunk = st->C;
  sp.left = st->left;
  sp.right = st->right;
  sp.kc_in = st->kc[st->cur];
  sp.vc_in = st->vc[st->cur];
  sp.kc_out = st->kc[st->cur ^ 1];
  sp.vc_out = st->vc[st->cur ^ 1];
  sp.cc_in = st->cc[st->cur];
  sp.cc_out = st->cc[st->cur ^ 1];
  sp.Pn = st->Pn;
  sp.dMax = st->dMax;
  sp.kv_ld = st->left;
  auto launch = [&]() { return pass_launch(ctx, e, g, st->mel_dev, st->x_dev, c.layers, &sp); };
  const char *ge = getenv("FA_GRAPH");
  const bool steady = st->Lc == st->left && pb == 0 && pt == 0;
  if (steady && !ctx->prof_on && !(ge && ge[0] == '0')) {
    std::vector<int64_t> key = {(int64_t)e->ws_gen, (int64_t)st->buf_gen, m, nComp, nemit, st->cur};
    EncWs::Captured *hit = nullptr;
    for (auto &gr : st->graphs)
      if (gr.key == key) hit = &gr;
    if (!hit) {
      FA_HIP(ctx, hipStreamBeginCapture(ctx->stream, hipStreamCaptureModeThreadLocal));
      const int rc = launch();
      hipGraph_t graph = nullptr;
      const hipError_t ce = hipStreamEndCapture(ctx->stream, &graph);
      if (rc != FA_OK) {
        if (graph) (void)hipGraphDestroy(graph);
        return rc;
      }
      if (ce != hipSuccess) return set_err(ctx, FA_E_DEVICE, "stream pass: graph capture: %s", hipGetErrorString(ce));
      hipGraphExec_t exec = nullptr;
      const hipError_t ie = hipGraphInstantiateWithFlags(&exec, graph, 0);
      (void)hipGraphDestroy(graph);
      if (ie != hipSuccess) return set_err(ctx, FA_E_DEVICE, "stream pass: graph instantiate: %s", hipGetErrorString(ie));
      if (st->graphs.size() >= 4) {  // a stream repeats at most a few signatures
        size_t lru = 0;
        for (size_t i = 1; i < st->graphs.size(); i++)
          if (st->graphs[i].used < st->graphs[lru].used) lru = i;
        (void)hipStreamSynchronize(ctx->stream);
        (void)hipGraphExecDestroy(st->graphs[lru].exec);
        st->graphs.erase(st->graphs.begin() + lru);
      }
      st->graphs.push_back({key, exec, 0});
      hit = &st->graphs.back();
    }
    hit->used = ++st->graph_clock;
    FA_HIP(ctx, hipGraphLaunch(hit->exec, ctx->stream));
  } else {
    FA_TRY(launch());
  }
  st->cur ^= 1;
  st->Lc = sp.keep;
  fa_tensor o;
  TensorRec *ro;
  FA_TRY(new_tensor(ctx, nemit, D, S_F32, (size_t)nemit * D * 4, &o, &ro));
  FA_TRY(encoder_copy_f4(ctx, st->x_dev, ro->ptr, (size_t)nemit * D * 4, "stream_out"));
  outs.push_back(o);
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


// The passes a push of `count` mel-major frames makes ready, queued on the
// stream's HIP stream; their frames are appended to outs.
int push_passes(fa_stream *st, const float *mel, int count, std::vector<fa_tensor> &outs) {
  const int MB = st->enc->cfg.melBins;
  // mel-major [melBins][count] -> frame-major FIFO rows
  const size_t old = st->fifo.size() / MB;
  st->fifo.resize((old + count) * MB);
  for (int t = 0; t < count; t++)
    for (int ch = 0; ch < MB; ch++) st->fifo[(old + t) * MB + ch] = mel[(size_t)ch * count + t];
  for (;;) {
    const int M = (int)(st->fifo.size() / MB);
    // frames a pass can finish: the first pass reads 8*nComp - 7 rows (top
    // padded), later passes 8*nComp + 7 (14 rows of look-back); nComp
    // includes the provisional lookahead B, and n is a whole number of chunks
    int n = st->subT == 0 ? (M + 7) / 8 - st->B : (M - 7 >= 0 ? (M - 7) / 8 : -1) - st->B;
    n = std::min(n, st->max_chunk);
    n -= ((n % st->C) + st->C) % st->C;
    if (n < st->C) break;
    const int nComp = n + st->B;
    const int m = st->subT == 0 ? 8 * nComp - 7 : 8 * nComp + 7;
    const int pt = st->subT == 0 ? st->enc->opts.sub_pad_t : 0;
    FA_TRY(run_pass(st, m, pt, 0, nComp, n, outs));
    // keep the look-back of the next pass's first frame
    st->subT += n;
    const long keep_from = 8L * st->subT - kLookback;
    const long drop = keep_from - st->fifo_start;
    st->fifo.erase(st->fifo.begin(), st->fifo.begin() + (size_t)drop * MB);
    st->fifo_start = keep_from;
  }
  return FA_OK;
}

}  // namespace

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
  if (hipStreamCreateWithFlags(&st->hs, hipStreamNonBlocking) != hipSuccess || hipEventCreateWithFlags(&st->in, hipEventDisableTiming) != hipSuccess ||
      hipEventCreateWithFlags(&st->done, hipEventDisableTiming) != hipSuccess) {
    fa_stream_destroy(st);
    return set_err(ctx, FA_E_DEVICE, "createEncodeStream: creating the stream's HIP stream failed");
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
  for (int i = 0; i < n; i++) {
    fa_stream *st = sts[i];
    if (st->ctx != ctx) return set_err(ctx, FA_E_INVALID, "encodeStreamPush: streams of different contexts in one call");
    for (int j = 0; j < i; j++)
      if (sts[j] == st) return set_err(ctx, FA_E_INVALID, "encodeStreamPush: stream %d repeats stream %d in one call", i, j);
    if (st->flushed) return set_err(ctx, FA_E_STATE, "encodeStreamPush: stream already flushed; create a new stream");
    if (counts[i] < 0 || (counts[i] > 0 && !mels[i])) return set_err(ctx, FA_E_INVALID, "encodeStreamPush: %d frames", counts[i]);
  }
  // every stream's passes start after the work already queued on the context stream
  FA_HIP(ctx, hipEventRecord(sts[0]->in, ctx->stream));
  for (int i = 0; i < n; i++) FA_HIP(ctx, hipStreamWaitEvent(sts[i]->hs, sts[0]->in, 0));
  std::vector<std::vector<fa_tensor>> frames(n);
  int rc = FA_OK;
  for (int i = 0; i < n && rc == FA_OK; i++) rc = push_passes(sts[i], mels[i], counts[i], frames[i]);
  // the context stream waits for every stream (also after an error, so later work stays ordered)
  for (int i = 0; i < n; i++) {
    (void)hipEventRecord(sts[i]->done, sts[i]->hs);
    (void)hipStreamWaitEvent(ctx->stream, sts[i]->done, 0);
  }
  for (int i = 0; i < n; i++) {
    if (rc == FA_OK)
      rc = emit(sts[i], frames[i], &outs[i]);
    else
      for (fa_tensor t : frames[i]) (void)fa_free_tensor(ctx, t);
  }
  if (rc != FA_OK)
    for (int i = 0; i < n; i++)
      if (outs[i]) {
        (void)fa_free_tensor(ctx, outs[i]);
        outs[i] = 0;
      }
  return rc;
}

int fa_stream_flush(fa_stream *st, fa_tensor *out) {
  if (!st || !out) return FA_E_INVALID;
  fa_ctx *ctx = st->ctx;
  *out = 0;
  if (st->flushed) return set_err(ctx, FA_E_STATE, "encodeStreamFlush: stream already flushed");
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
  std::vector<fa_tensor> outs;
  FA_HIP(ctx, hipEventRecord(st->in, ctx->stream));
  FA_HIP(ctx, hipStreamWaitEvent(st->hs, st->in, 0));
  const int rc = run_pass(st, M, pt, pb, T, T, outs);
  (void)hipEventRecord(st->done, st->hs);
  (void)hipStreamWaitEvent(ctx->stream, st->done, 0);
  if (rc != FA_OK) {
    for (fa_tensor t : outs) (void)fa_free_tensor(ctx, t);
    return rc;
  }
  st->fifo.clear();
  return emit(st, outs, out);
}

void fa_stream_destroy(fa_stream *st) {
  if (!st) return;
  (void)hipStreamSynchronize(st->ctx->stream);
  if (st->hs) (void)hipStreamSynchronize(st->hs);
  encoder_ws_free(st->ws);
  for (auto &g : st->graphs)
    if (g.exec) (void)hipGraphExecDestroy(g.exec);
  for (int i = 0; i < 2; i++)
    for (void *p : {(void *)st->kc[i], (void *)st->vc[i], (void *)st->cc[i]})
      if (p) (void)hipFree(p);
  if (st->mel_dev) (void)hipFree(st->mel_dev);
  if (st->x_dev) (void)hipFree(st->x_dev);
  if (st->in) (void)hipEventDestroy(st->in);
  if (st->done) (void)hipEventDestroy(st->done);
  if (st->hs) (void)hipStreamDestroy(st->hs);
  delete st;
}

}  // extern "C"
