// The fused encoder's internal state, shared by encoder.hip (load, offline
// forward) and stream.hip (chunk-by-chunk streaming passes).
#pragma once
#include <cstdint>
#include <functional>
#include <vector>

#include "fa_internal.h"
#include "attention.h"
#include "gemm.h"

namespace fa {

typedef WinTable WinStage;

// A linear's device weights in one of the three storage formats.
struct Lin {
  void *w = nullptr;          // f16 [N][K] | int8 [N][K] | int4 [N][K/32][16 B]
  void *scales = nullptr;     // int4: f16 bits [N][K/32]
  float *colscale = nullptr;  // int8: s[n]·fold[n]; int4: fold[n] (null when all 1)
  float *bias = nullptr;      // [N] (folded), or null
  int bkind = B_F16;
  int N = 0, K = 0;
};

// One workspace lane of the fused encoder: grow-only device buffers and the
// forwards captured on them.
struct EncWs {
  // captured forwards (hipGraph), keyed by everything baked into the launch
  // arguments; ws_gen moves whenever a workspace buffer or a precision mask
  // changes (the encoder's ws_gen), so stale graphs never match again
  struct Captured {
    std::vector<int64_t> key;
    hipGraphExec_t exec = nullptr;
    uint64_t used = 0;
  };
  std::vector<Captured> graphs;
  uint64_t graph_clock = 0;
  // workspace (grow-only)
  void *hlo = nullptr, *ulo = nullptr, *alo = nullptr, *g32 = nullptr, *vt = nullptr, *vrow = nullptr, *s2 = nullptr, *s2p = nullptr, *s3 = nullptr, *s3p = nullptr, *h = nullptr, *u = nullptr, *a = nullptr, *g = nullptr;
  size_t cap_hlo = 0, cap_ulo = 0, cap_alo = 0, cap_g32 = 0, cap_vt = 0, cap_vrow = 0, cap_s2 = 0, cap_s2p = 0, cap_s3 = 0, cap_s3p = 0, cap_m = 0, cap_u = 0;
  // graph-mode input and residual-stream buffers: a captured forward reads the
  // mel rows from melw and works on xw, so its launches never name the
  // caller's (pool-recycled) tensors; copies in and out run outside the graph
  void *melw = nullptr, *xw = nullptr;
  size_t cap_melw = 0, cap_xw = 0;
  // device MelSrc of the channel-major forward (fa_encoder_forward_stream)
  void *msrc = nullptr;
  size_t cap_msrc = 0;
  void *dw32 = nullptr;  // f32 depthwise output ahead of the conv-module LayerNorm
  size_t cap_dw32 = 0;
  void *wdq = nullptr;  // quantised formats, batches of >= kDequantRows rows: one layer's linears widened to f16
  size_t cap_wdq = 0;
  void *skp = nullptr;  // stream passes: the skinny GEMMs' split-K partial tiles
  size_t cap_skp = 0;
};

}  // namespace fa

struct fa_encoder {
  fa_ctx *ctx = nullptr;
  fa_encoder_cfg cfg{};
  fa_encoder_opts opts{1, 1, 1, 1, 0, 0, 0, 0};
  int format = FA_W_F16;
  int maxT = 0;
  std::vector<void *> allocs;
  // front end
  float *c0w = nullptr, *c0b = nullptr, *c1w = nullptr, *c1b = nullptr, *c3w = nullptr, *c3b = nullptr;
  fa::Lin c2, c4, lin;
  struct Layer {
    float *ln[5][2];
    fa::Lin ff1w1, ff1w2, qkv, out, pw1, pw2, ff2w1, ff2w2;
    float *pbu = nullptr, *pbv = nullptr, *dww = nullptr, *dwb = nullptr;
    _Float16 *P = nullptr;  // [2*maxT-1, D]
    float *cln[2] = {nullptr, nullptr};  // conv-module LayerNorm of the depthwise output (streaming models), or none
    unsigned exact = 0;     // FA_EXACT_* operands carried as exact f16 hi/lo pairs
  };
  std::vector<Layer> L;
  uint64_t ws_gen = 0;
  bool vt_fuse = true;  // q|k|v epilogue writes the transposed V (FA_VT_FUSE=0 at load: v_transpose_kernel)
  bool c01_lds = true;  // front end stages mel rows in LDS (FA_C01_LDS=0 at load: per-tap global loads)
  // Workspace lanes: a forward works in ws[lane] on that lane's stream.  Lane
  // 0 runs on the context stream; fa_encoder_forward_stream_batches puts
  // consecutive batches on two lanes with streams of their own, so one batch's
  // kernel tails and end-of-kernel write-backs overlap the other's work.
  static constexpr int kLanes = 4;  // capacity; nlanes in use (FA_ENC_LANES at load, default 2)
  int nlanes = 2;
  fa::EncWs ws[kLanes];
  int lane = 0;
  hipStream_t lane_stream[kLanes] = {};
  hipEvent_t lane_done[kLanes] = {}, lanes_in = nullptr;
  // a stream pass works in its stream lane's workspace (stream.hip)
  fa::EncWs *ws_ovr = nullptr;
  struct StreamLane *slane[kLanes] = {};
  fa::EncWs &W() { return ws_ovr ? *ws_ovr : ws[lane]; }
};

namespace fa {

// Where the channel-major feature stream [melBins, ttot] lives and where each
// window starts in it (column).  Kept in device memory so that a captured
// forward reads it at replay time: a new stream or new window starts need no
// recapture, only a refresh of these bytes before the launch.
struct MelSrc {
  const float *ptr;
  long ttot;
  int start[kMaxWin];
};

// One pass of the encoder over a batch of windows: stage tables for the four
// time resolutions (mel, after each stride-2 conv), frequency bins per stage,
// and the time pads of this pass (offline: the model's; a streaming pass pads
// only at the stream's edges).
struct PassGeom {
  int n = 0, layout = 0, pt = 0, pb = 0;
  WinStage s[4];
  int mx[4] = {0, 0, 0, 0}, R[4] = {0, 0, 0, 0}, F[4] = {0, 0, 0, 0};
  int M = 0;
  // set: the front end reads the channel-major feature stream this device
  // descriptor names (MelSrc) instead of time-major rows at s[0].off
  const MelSrc *mel_src = nullptr;
};

// The caches of the streams in one batched stream pass, window w = stream w:
// its layer-0 K / V caches ([layers][left][D] f16) and depthwise-conv cache
// ([layers][8][D] f32), the set the pass reads and the set it writes.  Passed
// by value to the kernels that use them (a table in device memory cost each
// of those kernels a dependent pointer load), so a captured pass is keyed by
// the table.
constexpr int kMaxStreamGroup = 16;
struct KvSlots {
  const _Float16 *kc_in[kMaxStreamGroup], *vc_in[kMaxStreamGroup];
  _Float16 *kc_out[kMaxStreamGroup], *vc_out[kMaxStreamGroup];
};
struct CcSlots {
  const float *cc_in[kMaxStreamGroup];
  float *cc_out[kMaxStreamGroup];
};

// A streaming chunk pass over g.n streams (windows of nq = g.M / g.n frames
// each): the frames of a window attend to `Lc` cached keys of its stream's
// earlier passes followed by their own; the first `nemit` frames are emitted,
// and their keys / depthwise inputs become the next pass's caches.
struct StreamPass {
  int Lc = 0, nemit = 0, keep = 0;
  int chunk = 0, left = 0, right = 0;
  KvSlots kv{};  // one entry per window
  CcSlots cc{};
  // positional term: distance dMax - r at row r of the layer's table (the
  // offline table's rows maxT-1-dMax ..), Pn = dMax - dMin + 1 rows
  int Pn = 0, dMax = 0;
  int kv_ld = 0;  // rows per layer slice of the K/V caches (= left)
};

int pass_geometry(fa_ctx *ctx, const fa_encoder *e, const int32_t *lens, int n, int layout, int pt, int pb, PassGeom *g);
int pass_workspace(fa_ctx *ctx, fa_encoder *e, const PassGeom &g, int layers, bool stream);
int pass_launch(fa_ctx *ctx, fa_encoder *e, const PassGeom &g, const float *mel, float *x, int layers, const StreamPass *sp);
// One batched forward from raw device pointers (encoder.hip): the feature
// stream [melBins, mel_cols] (stream) or time-major mel rows; the result goes
// to xout, or stays in the current workspace's xw (xout null, *xres names it).
int encoder_forward_dev(fa_ctx *ctx, fa_encoder *e, const float *mel, int mel_rows, long mel_cols, bool stream, const int32_t *starts,
                        const int32_t *lens, int n, int layout, int layers_run, float *xout, const float **xres, int *M_out, const char *who);
int encoder_grow(fa_encoder *e, void **buf, size_t *cap, size_t need);
// frees a workspace's buffers and captured forwards (the device must be idle for them)
void encoder_ws_free(EncWs &w);
// the stream lanes of an encoder (stream.hip), at encoder destruction
void stream_lanes_free(fa_encoder *e);
int encoder_copy_f4(fa_ctx *ctx, const void *src, void *dst, size_t bytes, const char *label);
int encoder_graph_run(fa_ctx *ctx, fa_encoder *e, const std::vector<int64_t> &key, const std::function<int()> &launch,
                      const std::function<int()> &pre);

}  // namespace fa
