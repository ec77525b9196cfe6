// Per-kernel extent models for the launch audit (launch_audit.cpp): for each
// kernel of the windowed-transcription path, the byte range of every buffer
// it reads or writes, computed from its launch arguments the way the kernel
// indexes them (the grid / guard logic of each kernel restated on the host).
// The audit checks every range against the allocation it starts in, at launch
// and at every graph replay.  Two kernels whose outputs later launches index
// by (the feature-stream descriptor, the transposed-V row map) are also
// executed here, so the ranges that depend on them use the values a GPU run
// would hold.
//
// Compiled with ROCm's clang++ as host code (the product's GemmArgs /
// AttnArgs / WinTable come from its own headers, so layouts cannot drift).
#include <cstdint>
#include <cstring>
#include <string>
#include <vector>
#include <algorithm>
#include <cstdio>

#include "../../fluidaudio-web_amd/csrc/attention.h"
#include "../../fluidaudio-web_amd/csrc/gemm.h"

namespace audit_ext {

struct Span {
  uintptr_t p;
  size_t bytes;
  bool write;
  std::string what;
};

// mirrors of by-value argument structs defined in .hip sources (their sizes
// are checked against the code objects' argument sizes before use)
struct MelSrcM {
  const float *ptr;
  long ttot;
  int start[fa::kMaxWin];
};
struct TdtWinM {
  int t, T, emitted, n_out, emit, off, last, cur;
};
struct TdtStateM {
  TdtWinM *win;
  float *h, *c, *pp, *j, *z, *pv;
  int *pi;
  float *dv;
  int *di, *ids, *frs, *alive;
};
// streaming passes: per-window cache pointers (encoder_impl.h KvSlots /
// CcSlots) and output rows (stream.hip OutRows), kMaxStreamGroup = 16 windows
constexpr int kSG = 16;
struct KvSlotsM {
  const _Float16 *kc_in[kSG], *vc_in[kSG];
  _Float16 *kc_out[kSG], *vc_out[kSG];
};
struct CcSlotsM {
  const float *cc_in[kSG];
  float *cc_out[kSG];
};
struct OutRowsM {
  float *dst[kSG];
};
constexpr int kTH = 640, kTV = 8193, kTL = 8198, kTNB = (kTL + 63) / 64, kTLP = kTNB * 64;
constexpr int kBins = 257, kHop = 160;

// transposed-V row maps written by the front end's depthwise kernel:
// vrow buffer start -> (entries written, largest value)
struct VrowShadow {
  uintptr_t base = 0;
  long entries = 0;
};
static VrowShadow g_vrow;

template <typename T>
static T arg(const std::vector<std::vector<char>> &a, size_t i) {
  T v{};
  if (i < a.size()) std::memcpy(&v, a[i].data(), std::min(sizeof(T), a[i].size()));
  return v;
}
static bool size_is(const std::vector<std::vector<char>> &a, size_t i, size_t n) { return i < a.size() && a[i].size() == n; }

// template arguments of a demangled "name<a, b, ...>(...)"
static std::vector<long> targs(const std::string &pretty) {
  std::vector<long> v;
  const size_t lt = pretty.find('<'), gt = pretty.find('>');
  if (lt == std::string::npos || gt == std::string::npos) return v;
  std::string s = pretty.substr(lt + 1, gt - lt - 1);
  size_t p = 0;
  while (p < s.size()) {
    size_t q = s.find(',', p);
    if (q == std::string::npos) q = s.size();
    v.push_back(std::strtol(s.c_str() + p, nullptr, 10));
    p = q + 1;
  }
  return v;
}
// the first integer template argument in a mangled name after `key` ("...ILi4E...")
static long mangled_int(const std::string &m, const std::string &key) {
  const size_t k = m.find(key);
  if (k == std::string::npos) return -1;
  const size_t i = m.find("ILi", k);
  if (i == std::string::npos) return -1;
  return std::strtol(m.c_str() + i + 3, nullptr, 10);
}

static void rd(std::vector<Span> &o, const void *p, size_t bytes, const char *what) {
  if (p && bytes) o.push_back({(uintptr_t)p, bytes, false, what});
}
static void wr(std::vector<Span> &o, const void *p, size_t bytes, const char *what) {
  if (p && bytes) o.push_back({(uintptr_t)p, bytes, true, what});
}
// elements [lo, hi) of an array of `elt`-byte elements at p
static void rng(std::vector<Span> &o, const void *p, long lo, long hi, size_t elt, bool w, const char *what) {
  if (!p || hi <= lo) return;
  o.push_back({(uintptr_t)p + (uintptr_t)lo * elt, (size_t)(hi - lo) * elt, w, what});
}

// GemmArgs extents for the tiled routes (rows past M are clamped on load and
// never stored).  C / add element types follow the epilogue.
static void gemm_spans(const fa::GemmArgs &p, int epi, std::vector<Span> &o, std::string &note) {
  using namespace fa;
  const long M = p.M, N = p.N, K = p.K;
  if (M <= 0 || N <= 0) return;
  const size_t ae = p.akind == A_F32 ? 4 : 2;
  rng(o, p.A, 0, (M - 1) * p.lda + K, ae, false, "A");
  rng(o, p.Alo, 0, (M - 1) * p.lda + K, 2, false, "Alo");
  if (p.bkind == B_F16) rd(o, p.B, (size_t)N * K * 2, "B f16");
  if (p.bkind == B_I8) rd(o, p.B, (size_t)N * K, "B int8");
  if (p.bkind == B_I4) {
    rd(o, p.B, (size_t)N * K / 2, "B int4");
    rd(o, p.bscale, (size_t)N * (K / 32) * (p.bscale_f32 ? 4 : 2), "B scales");
    if (p.bzp) rd(o, p.bzp, (size_t)N * p.zpb, "B zero points");
  }
  rd(o, p.colscale, (size_t)N * 4, "colscale");
  rd(o, p.bias, (size_t)N * 4, "bias");
  if (p.add) rng(o, p.add, 0, (M - 1) * p.ldadd + N, 4, false, "add");
  // 0 F32, 1 F16, 2 F16_SILU, 3 F16_RELU, 4 GLU, 5 HILO_RELU, 6 GENERIC (gemm_impl.h)
  long cols = N;
  size_t ce = 4;
  if (epi == 1 || epi == 2 || epi == 3) ce = 2;
  if (epi == 4) {
    cols = N / 2;
    ce = p.out_f16 ? 2 : 4;
  }
  if (epi == 5) {
    cols = 2 * N;
    ce = 2;
  }
  if (epi == 6) ce = p.out_f16 ? 2 : 4;
  long ccols = cols;
  if (p.vt && epi == 1) ccols = std::min<long>(cols, p.vcol0);  // columns >= vcol0 go to vt
  rng(o, p.C, 0, (M - 1) * p.ldc + ccols, ce, true, "C");
  if (p.Clo) rng(o, p.Clo, 0, (M - 1) * p.ldc + ccols, 2, true, "Clo");
  if (p.vt && epi == 1) {
    rd(o, p.vrow, (size_t)M * 4, "vrow");
    if (g_vrow.base != (uintptr_t)p.vrow) {
      note = "vt written through a row map no depthwise launch wrote";
      return;
    }
    long mx = -1;
    const int *vr = p.vrow;
    for (long r = 0; r < M; r++) mx = std::max<long>(mx, vr[r]);
    if (mx >= 0) rng(o, p.vt, 0, mx + (N - p.vcol0 - 1) * (long)p.vtp + 1, 2, true, "vt");
  }
}

// Returns 1 and fills `o` when the kernel has a model; 0 otherwise.
// `note` receives a geometry complaint (a grid that does not cover the work).
int extents(const std::string &mangled, const std::string &pretty, const std::vector<std::vector<char>> &a, unsigned gx, unsigned gy, unsigned gz,
            unsigned threads, std::vector<Span> &o, std::string &note) {
  using namespace fa;
  auto has = [&](const char *s) { return mangled.find(s) != std::string::npos; };
  if (has("mel_frames_kernel")) {
    if (!size_is(a, 2, sizeof(WinTable))) return 0;
    const float *pcm = arg<const float *>(a, 0);
    const WinTable src = arg<WinTable>(a, 2), dst = arg<WinTable>(a, 3);
    const int nm = arg<int>(a, 7);
    const long total = arg<long>(a, 9);
    float *out = arg<float *>(a, 10);
    if ((int)gy != src.n) note = "mel_frames: grid.y != windows";
    rd(o, arg<const void *>(a, 4), 512 * 8 + 2 * 128 * 8 + 2 * 256 * 8, "mel tables");  // MelTab
    rd(o, arg<const void *>(a, 5), (size_t)nm * kBins * 4, "filterbank");
    rd(o, arg<const void *>(a, 6), (size_t)nm * 2 * 4, "bounds");
    for (int w = 0; w < src.n; w++) {
      const int T = src.len[w] / kHop;
      if (T > (int)gx) note = "mel_frames: grid.x below a window's frames";
      rng(o, pcm, src.off[w], (long)src.off[w] + src.len[w], 4, false, "pcm window");
      if (T > 0) rng(o, out, dst.off[w], (long)(nm - 1) * total + dst.off[w] + T, 4, true, "mel out");
    }
    return 1;
  }
  if (has("mel_stats_kernel") || has("mel_norm_kernel")) {
    const bool stats = has("mel_stats_kernel");
    if (!size_is(a, 1, sizeof(WinTable))) return 0;
    float *x = arg<float *>(a, 0);
    const WinTable dst = arg<WinTable>(a, 1);
    const int nm = arg<int>(a, 2);
    const long total = arg<long>(a, 3);
    double *st = arg<double *>(a, 4);
    const int nw = stats ? (int)gy : (int)gz;
    if (nw > dst.n) note = "mel stats/norm: grid covers more windows than the table";
    for (int w = 0; w < std::min(nw, dst.n); w++) {
      if (dst.len[w] > 0) rng(o, x, dst.off[w], (long)(nm - 1) * total + dst.off[w] + dst.len[w], 4, !stats, "mel rows");
      rng(o, st, 2L * w * nm, 2L * (w + 1) * nm, 8, stats, "mel stats");
      if (!stats && (long)gx * 256 < dst.len[w]) note = "mel_norm: grid.x below a window's frames";
    }
    return 1;
  }
  if (has("set_mel_src_kernel")) {
    if (!size_is(a, 0, sizeof(MelSrcM))) {
      note = "MelSrc layout differs from its mirror";
      return 0;
    }
    const MelSrcM v = arg<MelSrcM>(a, 0);
    MelSrcM *d = arg<MelSrcM *>(a, 1);
    wr(o, d, sizeof(MelSrcM), "MelSrc");
    if (d) std::memcpy(d, &v, sizeof v);  // executed: the front end indexes through it
    return 1;
  }
  if (has("sub_c01_kernel")) {
    const long cpl = mangled_int(mangled, "sub_c01_kernel");
    if (cpl <= 0 || !size_is(a, 2, sizeof(WinTable))) return 0;
    const int C = 64 * (int)cpl;
    const float *mel = arg<const float *>(a, 0);
    const int MB = arg<int>(a, 1);
    const WinTable s0 = arg<WinTable>(a, 2), s2 = arg<WinTable>(a, 5);
    const int F2 = arg<int>(a, 6);
    rd(o, arg<const void *>(a, 7), (size_t)C * 9 * 4, "c0 w");
    rd(o, arg<const void *>(a, 8), (size_t)C * 4, "c0 b");
    rd(o, arg<const void *>(a, 9), (size_t)C * 9 * 4, "c1 w");
    rd(o, arg<const void *>(a, 10), (size_t)C * 4, "c1 b");
    _Float16 *y = arg<_Float16 *>(a, 11);
    const MelSrcM *src = arg<const MelSrcM *>(a, 14);
    if (src) rd(o, src, sizeof(MelSrcM), "MelSrc");
    const int nw = (int)gy;
    if (nw > s0.n) note = "sub_c01: grid covers more windows than the table";
    for (int w = 0; w < std::min(nw, s0.n); w++) {
      const int T0 = s0.len[w];
      if (T0 > 0) {
        if (src)
          rng(o, src->ptr, src->start[w], src->start[w] + (long)(MB - 1) * src->ttot + T0, 4, false, "mel stream window");
        else
          rng(o, mel, (long)s0.off[w] * MB, (long)(s0.off[w] + T0) * MB, 4, false, "mel rows");
      }
      if ((long)gx * 4 < s2.len[w]) note = "sub_c01: grid.x below a window's rows";
      rng(o, y, (long)s2.off[w] * F2 * 2 * C, (long)(s2.off[w] + s2.len[w]) * F2 * 2 * C, 2, true, "c01 out");
    }
    return 1;
  }
  if (has("sub_dw_kernel")) {
    const long cpl = mangled_int(mangled, "sub_dw_kernel");
    if (cpl <= 0 || !size_is(a, 1, sizeof(WinTable))) return 0;
    const int C = 64 * (int)cpl;
    const float *x = arg<const float *>(a, 0);
    const WinTable in = arg<WinTable>(a, 1), out = arg<WinTable>(a, 3);
    const int Fin = arg<int>(a, 2), Fout = arg<int>(a, 4);
    rd(o, arg<const void *>(a, 5), (size_t)9 * C * 4, "dw w");
    rd(o, arg<const void *>(a, 6), (size_t)C * 4, "dw b");
    _Float16 *y = arg<_Float16 *>(a, 7);
    int *vrow = arg<int *>(a, 8);
    const int vstride = arg<int>(a, 9), vpad = arg<int>(a, 10);
    const int nw = (int)gy;
    if (nw > in.n || nw > out.n) note = "sub_dw: grid covers more windows than the tables";
    long vmax = 0;
    for (int w = 0; w < std::min(nw, out.n); w++) {
      rng(o, x, (long)in.off[w] * Fin * C, (long)(in.off[w] + in.len[w]) * Fin * C, 4, false, "dw in");
      rng(o, y, (long)out.off[w] * Fout * 2 * C, (long)(out.off[w] + out.len[w]) * Fout * 2 * C, 2, true, "dw out");
      if ((long)gx * 4 < out.len[w]) note = "sub_dw: grid.x below a window's rows";
      if (vrow) {
        const int nv = std::min<long>((long)gx * 4, std::max(out.len[w], vpad));
        rng(o, vrow, out.off[w], (long)out.off[w] + nv, 4, true, "vrow");
        vmax = std::max<long>(vmax, (long)out.off[w] + nv);
      }
    }
    if (vrow) {  // executed: the q|k|v epilogue scatters V through it
      g_vrow.base = (uintptr_t)vrow;
      g_vrow.entries = vmax;
      for (int w = 0; w < std::min(nw, out.n); w++) {
        const int nv = std::min<long>((long)gx * 4, std::max(out.len[w], vpad));
        for (int t = 0; t < nv; t++) vrow[out.off[w] + t] = t < out.len[w] ? w * vstride + t : -1;
      }
    }
    return 1;
  }
  if (has("enc_ln_kernel") || has("enc_ln2_kernel") || has("enc_ln_f32_kernel")) {
    const bool two = has("enc_ln2_kernel"), f32 = has("enc_ln_f32_kernel");
    const long V = mangled_int(mangled, two ? "enc_ln2_kernel" : (f32 ? "enc_ln_f32_kernel" : "enc_ln_kernel"));
    if (V <= 0) return 0;
    const long D = 256 * V;
    const float *x = arg<const float *>(a, 0);
    int rows;
    if (f32) {
      rows = arg<int>(a, 3);
      rd(o, arg<const void *>(a, 1), D * 4, "gamma");
      rd(o, arg<const void *>(a, 2), D * 4, "beta");
      rng(o, x, 0, rows * D, 4, true, "ln rows");
    } else if (two) {
      rows = arg<int>(a, 7);
      for (int i = 1; i <= 4; i++) rd(o, arg<const void *>(a, i), D * 4, "ln params");
      rng(o, x, 0, rows * D, 4, true, "ln rows");
      rng(o, arg<const void *>(a, 5), 0, rows * D, 2, true, "ln out");
      rng(o, arg<const void *>(a, 6), 0, rows * D, 2, true, "ln out lo");
    } else {
      rows = arg<int>(a, 5);
      rd(o, arg<const void *>(a, 1), D * 4, "gamma");
      rd(o, arg<const void *>(a, 2), D * 4, "beta");
      rng(o, x, 0, rows * D, 4, false, "ln rows");
      rng(o, arg<const void *>(a, 3), 0, rows * D, 2, true, "ln out");
      rng(o, arg<const void *>(a, 4), 0, rows * D, 2, true, "ln out lo");
    }
    if ((long)gx * 4 < rows || threads != 256) note = "LayerNorm: grid below its rows";
    return 1;
  }
  if (has("dwconv_silu_kernel")) {
    // dwconv_silu_kernel<KT, TT, CPT, TI>(x, y, ylo, wt, b, D, st)
    const size_t xe = has("ILi9ELi16ELi4EfE") || mangled.find("EfEEv") != std::string::npos ? 4 : 2;
    if (!size_is(a, 6, sizeof(WinTable))) return 0;
    const int D = arg<int>(a, 5);
    const WinTable st = arg<WinTable>(a, 6);
    rd(o, arg<const void *>(a, 3), (size_t)9 * D * 4, "dw taps");
    rd(o, arg<const void *>(a, 4), (size_t)D * 4, "dw bias");
    const int nw = (int)gy;
    if (nw > st.n) note = "dwconv: grid covers more windows than the table";
    for (int w = 0; w < std::min(nw, st.n); w++) {
      rng(o, arg<const void *>(a, 0), (long)st.off[w] * D, (long)(st.off[w] + st.len[w]) * D, xe, false, "dw in");
      rng(o, arg<const void *>(a, 1), (long)st.off[w] * D, (long)(st.off[w] + st.len[w]) * D, 2, true, "dw out");
      rng(o, arg<const void *>(a, 2), (long)st.off[w] * D, (long)(st.off[w] + st.len[w]) * D, 2, true, "dw out lo");
      if ((long)gx * 16 < st.len[w]) note = "dwconv: grid.x below a window's frames";
    }
    return 1;
  }
  if (has("relpos_attn_t_kernel")) {
    if (!size_is(a, 0, sizeof(AttnArgs))) return 0;
    const AttnArgs t = arg<AttnArgs>(a, 0);
    const _Float16 *vt = arg<const _Float16 *>(a, 1);
    const int Tp = arg<int>(a, 2);
    const long HW = (long)t.H * t.HD;
    rd(o, t.pbu, HW * 4, "pos bias u");
    rd(o, t.pbv, HW * 4, "pos bias v");
    rng(o, t.pos, 0, (long)(t.prows - 1) * t.ldp + HW, 2, false, "pos table");
    const int nw = (int)gz;
    if (nw > t.win.n) note = "attention: grid covers more windows than the table";
    for (int w = 0; w < std::min(nw, t.win.n); w++) {
      const long off = t.win.off[w], T = t.win.len[w];
      if (T <= 0) continue;
      rng(o, t.q, off * t.ldq, (off + T - 1) * t.ldq + HW, 2, false, "q");
      rng(o, t.k, off * t.ldk, (off + T - 1) * t.ldk + HW, 2, false, "k");
      rng(o, t.out, off * t.ldo, (off + T - 1) * t.ldo + HW, 2, true, "attention out");
      rng(o, t.out_lo, off * t.ldo, (off + T - 1) * t.ldo + HW, 2, true, "attention out lo");
      // K blocks of 32 keys read from Vt: columns up to the window's rounded length
      if ((T + 31) / 32 * 32 > Tp) note = "attention: a window's key blocks run past Tp";
      rng(o, vt, (long)w * HW * Tp, (long)(w + 1) * HW * Tp, 2, false, "vt");
      if ((long)gx * 96 < T) note = "attention: grid.x below a window's queries";
      if (T - 1 > t.pcenter || t.pcenter + T - 1 >= t.prows) note = "attention: window longer than the positional table";
    }
    return 1;
  }
  if (has("gemm_dma_kernel") || has("gemm_mfma_kernel")) {
    if (!size_is(a, 0, sizeof(GemmArgs))) return 0;
    const GemmArgs p = arg<GemmArgs>(a, 0);
    const std::vector<long> ta = targs(pretty);
    // gemm_dma_kernel<BM, BN, WM, WN, S, EPI, LO, BQ, WW>, gemm_mfma_kernel<BM, BN, WM, WN, AK, BKND, EPI>
    const bool dma = has("gemm_dma_kernel");
    if (ta.size() < 7) return 0;
    const long BM = ta[0], BN = ta[1], epi = dma ? ta[5] : ta[6];
    const long tiles = (p.M + BM - 1) / BM * ((p.N + BN - 1) / BN);
    if ((long)gx * gy * gz < tiles) note = "GEMM: grid below its tiles";
    if (dma && (p.N % BN || p.K % 64)) note = "GEMM: N or K not a whole number of tiles";
    gemm_spans(p, (int)epi, o, note);
    return 1;
  }
  if (has("gemm_skinny_kernel") || has("gemm_skinny_split_sum_kernel") || has("gemm_skinny_ln_kernel")) {
    if (!size_is(a, 0, sizeof(GemmArgs))) return 0;
    const GemmArgs p = arg<GemmArgs>(a, 0);
    const std::vector<long> ta = targs(pretty);
    // gemm_skinny_kernel<TI, KS, EPI, LO, SPLIT>, gemm_skinny_split_sum_kernel<TI, SPLIT, EPI>, gemm_skinny_ln_kernel<TI, KS, EPI, LO>
    if (ta.size() < 3) return 0;
    const bool sum = has("gemm_skinny_split_sum_kernel"), ln = has("gemm_skinny_ln_kernel");
    const long TI = ta[0], epi = ta[2], split = sum ? ta[1] : (!ln && ta.size() >= 5 ? ta[4] : 1);
    if (16 * TI < p.M) note = "skinny GEMM: row tiles below M";
    if ((long)gx * 16 != p.N) note = "skinny GEMM: grid.x * 16 != N";
    if (ln) {
      if (p.M > 32) note = "skinny LayerNorm GEMM: more rows than its statistics slots";
      rng(o, p.ln_x, 0, (long)p.M * p.K, 4, false, "LayerNorm rows");
      rd(o, p.ln_g, (size_t)p.K * 4, "LayerNorm gamma");
      rd(o, p.ln_b, (size_t)p.K * 4, "LayerNorm beta");
    }
    const size_t tiles = (size_t)split * gx * TI * 64 * 16;  // bytes of the split partial tiles
    if (sum || split > 1) {
      if (tiles > p.skp_bytes) note = "skinny split: partial tiles past the workspace";
      if (sum) rd(o, p.skp, tiles, "split partials");
      else wr(o, p.skp, tiles, "split partials");
    }
    if (sum) {  // the epilogue only
      GemmArgs q = p;
      q.A = q.Alo = nullptr;
      q.B = nullptr;
      gemm_spans(q, (int)epi, o, note);
    } else if (split > 1) {  // operands only, no epilogue
      GemmArgs q = p;
      q.C = q.Clo = nullptr;
      q.add = nullptr;
      q.bias = nullptr;
      q.colscale = nullptr;
      gemm_spans(q, (int)epi, o, note);
    } else {
      gemm_spans(p, (int)epi, o, note);
    }
    return 1;
  }
  if (has("stream_attn_kernel")) {
    if (!size_is(a, 2, sizeof(KvSlotsM))) return 0;
    const _Float16 *u = arg<const _Float16 *>(a, 0);
    const int ldu = arg<int>(a, 1), Lc = arg<int>(a, 4), nq = arg<int>(a, 5), D = arg<int>(a, 6), Pn = arg<int>(a, 8), nemit = arg<int>(a, 17),
              keep = arg<int>(a, 18);
    const KvSlotsM kv = arg<KvSlotsM>(a, 2);
    const size_t kvo = arg<size_t>(a, 3);
    const int H = (int)gy, n = (int)gz;
    if (Lc + nq > 256) note = "stream attention: more keys than its 256 LDS rows";
    if (H * 128 != D) note = "stream attention: heads x 128 != D";
    if (n > kSG) note = "stream attention: more windows than cache slots";
    if ((long)gx * 4 < nq) note = "stream attention: grid.x below the queries";
    rng(o, arg<const void *>(a, 7), 0, (long)Pn * D, 2, false, "positional rows");
    rd(o, arg<const void *>(a, 10), (size_t)D * 4, "pos bias u");
    rd(o, arg<const void *>(a, 11), (size_t)D * 4, "pos bias v");
    for (int w = 0; w < std::min(n, kSG); w++) {
      rng(o, u, (long)w * nq * ldu, (long)w * nq * ldu + (long)(nq - 1) * ldu + 3 * D, 2, false, "q|k|v rows");
      rng(o, kv.kc_in[w], kvo, kvo + (size_t)Lc * D, 2, false, "cached keys");
      rng(o, kv.vc_in[w], kvo, kvo + (size_t)Lc * D, 2, false, "cached values");
      if (keep > 0 && kv.kc_out[w]) {
        if (Lc + nemit - keep < 0 || Lc + nemit > Lc + nq) note = "stream attention: kept rows outside the keys";
        rng(o, kv.kc_out[w], kvo, kvo + (size_t)keep * D, 2, true, "next keys");
        rng(o, kv.vc_out[w], kvo, kvo + (size_t)keep * D, 2, true, "next values");
      }
      rng(o, arg<const void *>(a, 15), (long)w * nq * D, (long)(w + 1) * nq * D, 2, true, "attention out");
      rng(o, arg<const void *>(a, 16), (long)w * nq * D, (long)(w + 1) * nq * D, 2, true, "attention out lo");
    }
    return 1;
  }
  if (has("dwconv_ln_kernel")) {
    if (!size_is(a, 1, sizeof(CcSlotsM)) || !size_is(a, 4, sizeof(WinTable))) return 0;
    const size_t xe = has("dwconv_ln_kernelIfE") ? 4 : 2;
    const CcSlotsM cc = arg<CcSlotsM>(a, 1);
    const int use = arg<int>(a, 2), D = arg<int>(a, 10), nemit = arg<int>(a, 13);
    const size_t cco = arg<size_t>(a, 3);
    const WinTable st = arg<WinTable>(a, 4);
    rd(o, arg<const void *>(a, 6), (size_t)9 * D * 4, "dw taps");
    for (int i = 7; i <= 9; i++) rd(o, arg<const void *>(a, i), (size_t)D * 4, "dw bias / LayerNorm");
    const int nw = (int)gy;
    if (nw > st.n) note = "dwconv_ln: grid covers more windows than the table";
    if ((int)threads * 4 < D) note = "dwconv_ln: block below D / 4 threads";
    for (int w = 0; w < std::min(nw, st.n); w++) {
      rng(o, arg<const void *>(a, 0), (long)st.off[w] * D, (long)(st.off[w] + st.len[w]) * D, xe, false, "dw in");
      rng(o, arg<const void *>(a, 11), (long)st.off[w] * D, (long)(st.off[w] + st.len[w]) * D, 2, true, "dw out");
      rng(o, arg<const void *>(a, 12), (long)st.off[w] * D, (long)(st.off[w] + st.len[w]) * D, 2, true, "dw out lo");
      if ((int)gx < st.len[w]) note = "dwconv_ln: grid.x below a window's frames";
      if (use && w < kSG) {
        rng(o, cc.cc_in[w], cco, cco + (size_t)8 * D, 4, false, "conv cache");
        rng(o, cc.cc_out[w], cco, cco + (size_t)8 * D, 4, true, "next conv cache");
        if (nemit > st.len[w]) note = "dwconv_ln: emitted rows past the window";
      }
    }
    return 1;
  }
  if (has("stream_out_kernel")) {
    if (!size_is(a, 4, sizeof(OutRowsM))) return 0;
    const int nq = arg<int>(a, 1), nemit = arg<int>(a, 2), D4 = arg<int>(a, 3);
    const OutRowsM r = arg<OutRowsM>(a, 4);
    for (int w = 0; w < std::min<int>((int)gy, kSG); w++) {
      rng(o, arg<const void *>(a, 0), (long)w * nq * D4, (long)w * nq * D4 + (long)nemit * D4, 16, false, "pass rows");
      rng(o, r.dst[w], 0, (long)nemit * D4, 16, true, "stream output");
    }
    if (nemit > nq) note = "stream_out: more emitted rows than the pass has";
    return 1;
  }
  if (has("f32_to_f16_kernel")) {
    const long n = arg<long>(a, 2);
    rng(o, arg<const void *>(a, 0), 0, n, 4, false, "f32 in");
    rng(o, arg<const void *>(a, 1), 0, n, 2, true, "f16 out");
    return 1;
  }
  if (has("gemm_f32_kernel")) {
    const float *A = arg<const float *>(a, 0), *B = arg<const float *>(a, 1);
    float *Cp = arg<float *>(a, 2);
    const float *bias = arg<const float *>(a, 3), *add = arg<const float *>(a, 4);
    const long M = arg<int>(a, 5), N = arg<int>(a, 6), K = arg<int>(a, 7);
    rng(o, A, 0, M * K, 4, false, "A");
    rng(o, B, 0, K * N, 4, false, "B");
    rng(o, Cp, 0, M * N, 4, true, "C");
    rd(o, bias, N * 4, "bias");
    rng(o, add, 0, M * N, 4, false, "add");
    if ((long)gx < ((M + 63) / 64) * ((N + 63) / 64)) note = "gemm_f32: grid below its tiles";
    return 1;
  }
  if (has("copy_f4_kernel")) {
    const long n4 = arg<long>(a, 2);
    rng(o, arg<const void *>(a, 0), 0, n4, 16, false, "copy src");
    rng(o, arg<const void *>(a, 1), 0, n4, 16, true, "copy dst");
    return 1;
  }
  // ── TDT decoder: window state as uploaded by the host (t = 0, T = lens) ──
  auto tdt_state = [&](size_t i, int n) {
    const TdtStateM s = arg<TdtStateM>(a, i);
    rd(o, s.win, (size_t)n * sizeof(TdtWinM), "tdt windows");
    rd(o, s.h, (size_t)n * 4 * kTH * 4, "tdt h");
    rd(o, s.c, (size_t)n * 4 * kTH * 4, "tdt c");
    rd(o, s.pp, (size_t)n * kTH * 4, "tdt pp");
    rd(o, s.j, (size_t)n * kTH * 4, "tdt j");
    rd(o, s.z, (size_t)n * 32 * kTH * 4, "tdt z");
    rd(o, s.pv, (size_t)n * kTNB * 4, "tdt pv");
    rd(o, s.pi, (size_t)n * kTNB * 4, "tdt pi");
    rd(o, s.dv, (size_t)n * 4, "tdt dv");
    rd(o, s.di, (size_t)n * 4, "tdt di");
    rd(o, s.alive, (size_t)n * 4, "tdt alive");
    return s;
  };
  if (has("tdt_joint_kernel")) {
    if (!size_is(a, 5, sizeof(TdtStateM))) return 0;
    const int ldw = arg<int>(a, 1), ncols = arg<int>(a, 2), n = arg<int>(a, 6);
    rd(o, arg<const void *>(a, 0), (size_t)kTH * ldw * 4, "joint W");
    rd(o, arg<const void *>(a, 3), (size_t)ncols * 4, "joint bias");
    rd(o, arg<const void *>(a, 4), (size_t)n * kTH * 4, "joint x");
    if (ldw < (int)gx * 64) note = "tdt_joint: slabs past the padded row";
    if (n > 64 || (long)gy * 8 < n) note = "tdt_joint: windows not covered";
    tdt_state(5, n);
    return 1;
  }
  if (has("tdt_update_kernel")) {
    if (!size_is(a, 0, sizeof(TdtStateM))) return 0;
    const int cap = arg<int>(a, 1), n = (int)gx;
    const TdtStateM s = tdt_state(0, n);
    wr(o, s.ids, (size_t)n * cap * 4, "tdt ids");
    wr(o, s.frs, (size_t)n * cap * 4, "tdt frames");
    return 1;
  }
  if (has("tdt_z_kernel")) {
    if (!size_is(a, 4, sizeof(TdtStateM))) return 0;
    const int n = arg<int>(a, 5);
    rd(o, arg<const void *>(a, 0), (size_t)4 * kTH * kTH * 4, "lstm W");
    rd(o, arg<const void *>(a, 1), (size_t)4 * kTH * kTH * 4, "lstm R");
    const TdtStateM s = tdt_state(4, n);
    const float *embed = arg<const float *>(a, 2);
    for (int w = 0; w < n && s.win; w++) {
      const int last = s.win[w].last;
      if (last < 0 || last >= kTV) note = "tdt_z: embedding row outside the table";
      rng(o, embed, (long)last * kTH, (long)(last + 1) * kTH, 4, false, "embed row");
    }
    if (gx != 4 * kTH / 64 * 8) note = "tdt_z: grid.x";
    return 1;
  }
  if (has("tdt_gates_kernel")) {
    if (!size_is(a, 2, sizeof(TdtStateM))) return 0;
    const int n = (int)gy;
    rd(o, arg<const void *>(a, 0), (size_t)8 * kTH * 4, "lstm bias");
    tdt_state(2, n);
    return 1;
  }
  if (has("tdt_proj_kernel")) {
    if (!size_is(a, 4, sizeof(TdtStateM))) return 0;
    const int n = arg<int>(a, 5);
    rd(o, arg<const void *>(a, 0), (size_t)kTH * kTH * 4, "pred W");
    rd(o, arg<const void *>(a, 1), (size_t)kTH * 4, "pred bias");
    rd(o, arg<const void *>(a, 2), (size_t)n * 4 * kTH * 4, "pred h");
    const TdtStateM s = tdt_state(4, n);
    const float *fr = arg<const float *>(a, 3);
    for (int w = 0; w < n && s.win; w++)
      if (s.win[w].T > 0) rng(o, fr, (long)s.win[w].off * kTH, (long)(s.win[w].off + s.win[w].T) * kTH, 4, false, "frames");
    if (gx * 64 != kTH) note = "tdt_proj: grid.x";
    return 1;
  }
  return 0;
}

}  // namespace audit_ext
