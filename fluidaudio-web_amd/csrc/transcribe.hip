// Windowed transcription's device stages as one pipelined call
// (src/engines/asr-parakeet/pipeline.js:32-143): for every group of windows of
// a resident PCM stream, log-mel -> encoder forward -> joint projection ->
// greedy TDT decode.  The reference overlaps its stages across CPU and GPU
// (mel and the WASM decode on the CPU while the GPU encodes the next group);
// here every stage is on the GPU, and the overlap is between HIP streams:
// group g+1's mel, encoder and projection are queued on an encoder lane
// before group g's decode runs on the context stream, so the encoder's GEMMs
// fill the chip while the decode's short dependent steps (and its host
// round trips every 16 steps) run.  Buffers are per group parity and owned by
// the call; nothing comes from the context's tensor pool, whose reuse is
// ordered only on one stream.
#include <algorithm>
#include <vector>

#include "fa_internal.h"
#include "encoder_impl.h"
#include "gemm.h"

using namespace fa;

namespace {

constexpr int kHopSamples = 160;  // mel hop (mel.hip)
constexpr int kJoint = 640;       // projected frame width the decoder reads
constexpr int kMaxGroup = 32;     // windows per encoder batch

struct Events {
  std::vector<hipEvent_t> all;
  hipEvent_t make(fa_ctx *ctx) {
    hipEvent_t e = nullptr;
    if (hipEventCreateWithFlags(&e, hipEventDisableTiming) != hipSuccess) {
      set_err(ctx, FA_E_DEVICE, "transcribeGroups: event creation failed");
      return nullptr;
    }
    all.push_back(e);
    return e;
  }
  ~Events() {
    for (hipEvent_t e : all) (void)hipEventDestroy(e);
  }
};

struct Buffers {
  std::vector<void *> all;
  void *make(fa_ctx *ctx, size_t bytes) {
    void *p = dev_alloc(ctx, std::max<size_t>(bytes, 256));
    if (p) all.push_back(p);
    return p;
  }
  ~Buffers() {
    for (void *p : all) (void)hipFree(p);
  }
};

}  // namespace

extern "C" int fa_transcribe_groups(fa_ctx *ctx, fa_encoder *e, fa_tdt *dec, fa_tensor pcm, int n_groups, const int32_t *counts,
                                    const int32_t *starts, const int32_t *lens, fa_tensor projW, fa_tensor projB, int n_mels, double log_guard,
                                    int normalize, int cap, int32_t *ids, int32_t *frame_idx, int32_t *n_out, int32_t *tsub) {
  const char *who = "transcribeGroups";
  if (!ctx) return FA_E_INVALID;
  if (!e || e->ctx != ctx) return set_err(ctx, FA_E_INVALID, "%s: encoder belongs to another context", who);
  if (!dec) return set_err(ctx, FA_E_INVALID, "%s: no decoder", who);
  if (n_groups <= 0 || !counts || !starts || !lens || !ids || !frame_idx || !n_out || !tsub || cap <= 0)
    return set_err(ctx, FA_E_INVALID, "%s: empty plan or null output", who);
  if (n_mels != e->cfg.melBins) return set_err(ctx, FA_E_INVALID, "%s: %d mel bins, the encoder takes %d", who, n_mels, e->cfg.melBins);
  TensorRec *rp, *rw, *rb;
  FA_TRY(need(ctx, pcm, &rp, who));
  FA_TRY(need(ctx, projW, &rw, who));
  FA_TRY(opt(ctx, projB, &rb, who));
  if (rp->kind != S_F32) return set_err(ctx, FA_E_INVALID, "%s: PCM must be an f32 tensor", who);
  if (rw->kind != S_F32 || rw->rows != e->cfg.D || rw->cols != kJoint)
    return set_err(ctx, FA_E_INVALID, "%s: projection must be f32 [%d, %d]", who, e->cfg.D, kJoint);
  if (rb && (rb->kind != S_F32 || rb->rows * rb->cols != kJoint)) return set_err(ctx, FA_E_INVALID, "%s: projection bias must be f32 [%d]", who, kJoint);
  const long nsamp = (long)rp->rows * rp->cols;
  const float *pcm_d = (const float *)rp->ptr, *W = (const float *)rw->ptr, *B = rb ? (const float *)rb->ptr : nullptr;

  // plan: per group its window range, mel columns and encoder rows
  std::vector<long> first(n_groups + 1, 0);
  std::vector<int> T, Tsub;
  size_t feat_max = 0, rows_max = 0;
  int win_max = 0;
  for (int g = 0; g < n_groups; g++) {
    if (counts[g] < 1 || counts[g] > kMaxGroup) return set_err(ctx, FA_E_INVALID, "%s: group %d has %d windows (1..%d)", who, g, counts[g], kMaxGroup);
    first[g + 1] = first[g] + counts[g];
    long cols = 0, rows = 0;
    for (long w = first[g]; w < first[g + 1]; w++) {
      if (lens[w] < 0 || starts[w] < 0 || (long)starts[w] + lens[w] > nsamp)
        return set_err(ctx, FA_E_INVALID, "%s: window %ld [%d, +%d) outside the %ld-sample stream", who, w, starts[w], lens[w], nsamp);
      const int t = lens[w] / kHopSamples;
      if (t <= 0) return set_err(ctx, FA_E_INVALID, "%s: window %ld has no mel frame (drop it before the call)", who, w);
      T.push_back(t);
      Tsub.push_back(fa_encoder_tsub_of(e, t));
      cols += t;
      rows += Tsub.back();
    }
    feat_max = std::max(feat_max, (size_t)cols);
    rows_max = std::max(rows_max, (size_t)rows);
    win_max = std::max(win_max, counts[g]);
  }
  for (size_t w = 0; w < Tsub.size(); w++) tsub[w] = Tsub[w];

  const int nl = std::max(1, std::min(e->nlanes, (int)fa_encoder::kLanes));
  for (int l = 0; l < nl; l++)
    if (!e->lane_stream[l]) FA_HIP(ctx, hipStreamCreateWithFlags(&e->lane_stream[l], hipStreamNonBlocking));
  // tables and statistics scratch sized once, before any lane runs
  FA_TRY(mel_prepare(ctx, win_max, n_mels, normalize));
  Buffers buf;
  Events ev;
  float *feats[2], *proj[2];
  for (int b = 0; b < 2; b++) {
    feats[b] = (float *)buf.make(ctx, feat_max * n_mels * 4);
    proj[b] = (float *)buf.make(ctx, rows_max * kJoint * 4);
    if (!feats[b] || !proj[b]) return FA_E_OOM;
  }
  hipEvent_t ev_in = ev.make(ctx), ev_mel = ev.make(ctx), ev_grp[2] = {ev.make(ctx), ev.make(ctx)}, ev_dec[2] = {ev.make(ctx), ev.make(ctx)};
  for (hipEvent_t x : ev.all)
    if (!x) return FA_E_DEVICE;
  const hipStream_t home = ctx->stream;
  FA_HIP(ctx, hipEventRecord(ev_in, home));
  std::vector<bool> lane_used(nl, false);

  // group g's mel, encoder and projection on lane g % nl
  auto enqueue = [&](int g) -> int {
    const int l = g % nl, b = g & 1;
    const hipStream_t ls = e->lane_stream[l];
    if (!lane_used[l]) {
      FA_HIP(ctx, hipStreamWaitEvent(ls, ev_in, 0));
      lane_used[l] = true;
    }
    if (g > 0) FA_HIP(ctx, hipStreamWaitEvent(ls, ev_mel, 0));     // one mel at a time: the statistics scratch is shared
    if (g > 1) FA_HIP(ctx, hipStreamWaitEvent(ls, ev_dec[b], 0));  // group g-2 decoded: its feature and frame buffers are free
    ctx->stream = ls;
    e->lane = l;
    const long w0 = first[g];
    const int n = counts[g];
    long total = 0;
    int rc = mel_windows_dev(ctx, pcm_d, nsamp, starts + w0, lens + w0, n, n_mels, log_guard, normalize, feats[b], &total);
    if (rc == FA_OK && hipEventRecord(ev_mel, ls) != hipSuccess) rc = set_err(ctx, FA_E_DEVICE, "%s: event record", who);
    std::vector<int32_t> col(n);
    for (int i = 0, c = 0; i < n; i++) {
      col[i] = c;
      c += T[w0 + i];
    }
    const float *x = nullptr;
    int M = 0;
    if (rc == FA_OK)
      rc = encoder_forward_dev(ctx, e, feats[b], n_mels, total, true, col.data(), T.data() + w0, n, 0, -1, nullptr, &x, &M, who);
    if (rc == FA_OK) rc = gemm_f32(ctx, x, W, proj[b], B, nullptr, M, kJoint, e->cfg.D, 0, "transcribe_proj");
    if (rc == FA_OK && hipEventRecord(ev_grp[b], ls) != hipSuccess) rc = set_err(ctx, FA_E_DEVICE, "%s: event record", who);
    e->lane = 0;
    ctx->stream = home;
    return rc;
  };

  int rc = enqueue(0);
  for (int g = 0; g < n_groups && rc == FA_OK; g++) {
    if (g + 1 < n_groups) rc = enqueue(g + 1);  // the next group's stages run while this one decodes
    if (rc != FA_OK) break;
    const int b = g & 1;
    if (hipStreamWaitEvent(home, ev_grp[b], 0) != hipSuccess) {
      rc = set_err(ctx, FA_E_DEVICE, "%s: stream wait", who);
      break;
    }
    const long w0 = first[g];
    rc = tdt_decode_dev(dec, proj[b], (long)rows_max, Tsub.data() + w0, counts[g], cap, ids + w0 * cap, frame_idx + w0 * cap, n_out + w0);
    if (rc == FA_OK && hipEventRecord(ev_dec[b], home) != hipSuccess) rc = set_err(ctx, FA_E_DEVICE, "%s: event record", who);
  }
  // the lanes' queued work ends before the buffers go (also on an error path)
  for (int l = 0; l < nl; l++)
    if (lane_used[l]) (void)hipStreamSynchronize(e->lane_stream[l]);
  (void)hipStreamSynchronize(home);
  return rc;
}
