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
// a dry call (whether a kernel has a model, asked while a graph is being
// captured) computes the ranges but executes nothing
bool g_dry = false;

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
// ── ComputeContext op kernels (ops.hip, ops_aux.hip, quant.hip fallbacks,
// gemm.hip's any-shape GEMM): grid-stride loops over their outputs, inputs
// indexed as each kernel does ──
struct GemvArgsM {
  const float *A;
  int M, K, N;
  const void *W, *scales;
  const uint8_t *zp;
  int zpb;
  float *Y;
  const float *bias;
  int act;
};
struct GemvItemM {
  const float *A;
  const void *W, *scales;
  float *Y;
};
constexpr int kGemvItems = 48, kGemvWavesM = 8;

// quantised weights of one product ([N] rows of K, fmt 1 int8 + f32 column
// scales, 2 int4 group-32 + f16 scales, 3 int4 + f32 scales + zero points)
static void gemv_spans(const GemvArgsM &p, int fmt, std::vector<Span> &o) {
  const long nblk = (p.K + 31) / 32;
  rng(o, p.A, 0, (long)p.M * p.K, 4, false, "gemv A");
  if (fmt == 1) {
    rng(o, p.W, 0, (long)p.N * p.K, 1, false, "gemv W int8");
    rng(o, p.scales, 0, p.N, 4, false, "gemv scales");
  } else {
    rng(o, p.W, 0, (long)p.N * nblk * 16, 1, false, "gemv W int4");
    rng(o, p.scales, 0, (long)p.N * nblk, fmt == 2 ? 2 : 4, false, "gemv scales");
    if (fmt == 3) rng(o, p.zp, 0, (long)(p.N - 1) * p.zpb + (nblk - 1) / 2 + 1, 1, false, "gemv zero points");
  }
  rng(o, p.Y, 0, (long)p.M * p.N, 4, true, "gemv Y");
  rng(o, p.bias, 0, p.N, 4, false, "gemv bias");
}

static int op_extents(const std::string &mangled, const std::vector<std::vector<char>> &a, unsigned gx, unsigned gy, unsigned gz, unsigned threads,
                      std::vector<Span> &o, std::string &note) {
  (void)gz;
  // the identifier as mangled (its length, then the name), so "transpose_kernel"
  // does not match "v_transpose_kernel"
  auto has = [&](const char *s) { return mangled.find(std::to_string(std::strlen(s)) + s) != std::string::npos; };
  auto P = [&](size_t i) { return arg<const void *>(a, i); };
  auto I = [&](size_t i) { return (long)arg<int>(a, i); };
  if (has("layernorm_kernel")) {
    const long rows = I(4), cols = I(5), ldx = I(6), ldy = I(7);
    const size_t ye = mangled.find("layernorm_kernelIfE") != std::string::npos ? 4 : 2;
    if (rows > 0) {
      rng(o, P(0), 0, (rows - 1) * ldx + cols, 4, false, "layernorm x");
      rng(o, P(3), 0, (rows - 1) * ldy + cols, ye, true, "layernorm y");
    }
    rng(o, P(1), 0, cols, 4, false, "gamma");
    rng(o, P(2), 0, cols, 4, false, "beta");
    if ((long)gx * 4 < rows) note = "layernorm: grid below its rows";
    return 1;
  }
  if (has("softmax_kernel")) {
    const long rows = I(2), cols = I(3);
    rng(o, P(0), 0, rows * cols, 4, false, "softmax x");
    rng(o, P(1), 0, rows * cols, 4, true, "softmax y");
    if ((long)gx * 4 < rows) note = "softmax: grid below its rows";
    return 1;
  }
  if (has("ewise_kernel")) {
    const long n = arg<long>(a, 3), cols = I(4);
    const int bcast = arg<int>(a, 5);
    rng(o, P(0), 0, n, 4, false, "ewise a");
    rng(o, P(1), 0, bcast ? std::min(n, cols) : n, 4, false, "ewise b");
    rng(o, P(2), 0, n, 4, true, "ewise c");
    return 1;
  }
  if (has("unary_kernel") || has("leaky_relu_kernel")) {
    const long n = arg<long>(a, 2);
    rng(o, P(0), 0, n, 4, false, "unary x");
    rng(o, P(1), 0, n, 4, true, "unary y");
    return 1;
  }
  if (has("glu_kernel")) {
    const long C = I(2), T = I(3);
    rng(o, P(0), 0, 2 * C * T, 4, false, "glu x");
    rng(o, P(1), 0, C * T, 4, true, "glu y");
    return 1;
  }
  if (has("transpose_kernel")) {
    const long R = I(2), C = I(3);
    rng(o, P(0), 0, R * C, 4, false, "transpose x");
    rng(o, P(1), 0, R * C, 4, true, "transpose y");
    if ((long)gx * 32 < C || (long)gy * 32 < R) note = "transpose: grid below the matrix";
    return 1;
  }
  if (has("slice_cols_kernel") || has("set_cols_kernel")) {
    const bool set = has("set_cols_kernel");
    const long rows = I(2), C = I(3), c0 = I(4), W = I(5);
    if (rows > 0 && W > 0) {
      rng(o, P(set ? 0 : 1), 0, rows * W, 4, !set, set ? "setCols src" : "sliceCols y");
      rng(o, P(set ? 1 : 0), c0, (rows - 1) * C + c0 + W, 4, set, set ? "setCols dst" : "sliceCols x");
    }
    if (c0 < 0 || c0 + W > C) note = "slice/set cols: columns outside the row";
    return 1;
  }
  if (has("sub_reshape_kernel")) {
    const long n = I(2) * I(3) * I(4);
    rng(o, P(0), 0, n, 4, false, "subReshape x");
    rng(o, P(1), 0, n, 4, true, "subReshape y");
    return 1;
  }
  if (has("row_bias_act_kernel")) {
    const long rows = I(3), cols = I(4);
    rng(o, P(0), 0, rows * cols, 4, false, "rowBiasAct x");
    rng(o, P(1), 0, rows, 4, false, "rowBiasAct bias");
    rng(o, P(2), 0, rows * cols, 4, true, "rowBiasAct y");
    return 1;
  }
  if (has("chan_bias_act_kernel")) {
    const long cols = I(2), n = arg<long>(a, 3);
    rng(o, P(0), 0, n, 4, true, "chanBiasAct y");
    if (cols > 0) rng(o, P(1), 0, (n + cols - 1) / cols, 4, false, "chanBiasAct bias");
    return 1;
  }
  if (has("round_f16_kernel")) {
    const long n = arg<long>(a, 2);
    rng(o, P(0), 0, n, 4, false, "round x");
    rng(o, P(1), 0, n, 2, true, "round y");
    if (n % 4) note = "round_f16: n not a multiple of 4";
    return 1;
  }
  if (has("conv1d_kernel")) {
    const long cout = I(4), cin = I(5), L = I(6), Lout = I(7), K = I(8), groups = I(12);
    if (groups <= 0 || cin % groups || cout % groups) note = "conv1d: groups";
    rng(o, P(0), 0, cin * L, 4, false, "conv1d x");
    rng(o, P(1), 0, cout * (groups > 0 ? cin / groups : 0) * K, 4, false, "conv1d w");
    rng(o, P(2), 0, cout, 4, false, "conv1d bias");
    rng(o, P(3), 0, cout * Lout, 4, true, "conv1d y");
    return 1;
  }
  if (has("conv2d_kernel")) {
    const long cout = I(4), cin = I(5), H = I(6), Wd = I(7), Ho = I(8), Wo = I(9), kh = I(10), kw = I(11), groups = I(16);
    if (groups <= 0 || cin % groups || cout % groups) note = "conv2d: groups";
    rng(o, P(0), 0, cin * H * Wd, 4, false, "conv2d x");
    rng(o, P(1), 0, cout * (groups > 0 ? cin / groups : 0) * kh * kw, 4, false, "conv2d w");
    rng(o, P(2), 0, cout, 4, false, "conv2d bias");
    rng(o, P(3), 0, cout * Ho * Wo, 4, true, "conv2d y");
    return 1;
  }
  if (has("conv_transpose1d_kernel")) {
    const long Cin = I(4), L = I(5), Cout = I(6), k = I(7), Lout = I(8), groups = I(12);
    if (groups <= 0 || Cin % groups || Cout % groups) note = "convTranspose1d: groups";
    rng(o, P(0), 0, Cin * L, 4, false, "convT x");
    rng(o, P(1), 0, Cin * (groups > 0 ? Cout / groups : 0) * k, 4, false, "convT w");
    rng(o, P(2), 0, Cout, 4, false, "convT bias");
    rng(o, P(3), 0, Cout * Lout, 4, true, "convT y");
    return 1;
  }
  if (has("im2col_kernel")) {
    const long Cin = I(2), L = I(3), k = I(4), Lout = I(5);
    rng(o, P(0), 0, Cin * L, 4, false, "im2col x");
    rng(o, P(1), 0, Cin * k * Lout, 4, true, "im2col y");
    return 1;
  }
  if (has("bmm_qk_kernel")) {
    const long T = I(4), Tb = I(5), H = I(6), HD = I(7), W = I(8), shared = I(9);
    rng(o, P(0), 0, W * T * H * HD, 4, false, "bmmQK q");
    rng(o, P(1), 0, (shared ? Tb : W * Tb) * H * HD, 4, false, "bmmQK b");
    rng(o, P(2), 0, H * HD, 4, false, "bmmQK q bias");
    rng(o, P(3), 0, W * H * T * Tb, 4, true, "bmmQK out");
    return 1;
  }
  if (has("bmm_pv_kernel")) {
    const long Tq = I(3), Tk = I(4), H = I(5), HD = I(6), W = I(7);
    rng(o, P(0), 0, W * H * Tq * Tk, 4, false, "bmmPV p");
    rng(o, P(1), 0, W * Tk * H * HD, 4, false, "bmmPV v");
    rng(o, P(2), 0, W * Tq * H * HD, 4, true, "bmmPV out");
    return 1;
  }
  if (has("relshift_stream_kernel")) {
    const long total = arg<long>(a, 2), Lk = I(4), Pw = I(5);
    rng(o, P(1), 0, total, 4, true, "relShiftStream y");
    if (Lk > 0 && total > 0) rng(o, P(0), 0, ((total - 1) / Lk + 1) * Pw, 4, false, "relShiftStream x");
    return 1;
  }
  if (has("relshift_kernel")) {
    const long t = I(2), H = I(3);
    rng(o, P(1), 0, H * t * t, 4, true, "relShift y");
    if (t > 0 && H > 0) {
      // x[(h t + f / 2t) p + (f mod 2t) - 1] grows with f over the columns it
      // reads (f mod 2t != 0): the largest is at the last such f
      const long p = 2 * t - 1, twoT = 2 * t;
      long f = t + (t - 1) * p + (t - 1);
      if (f % twoT == 0) f--;
      rng(o, P(0), 0, ((H - 1) * t + f / twoT) * p + (f % twoT - 1) + 1, 4, false, "relShift x");
    }
    return 1;
  }
  if (has("repack_i8_kernel")) {
    const long K = I(2), N = I(3);
    rng(o, P(0), 0, K * N, 1, false, "repack src");
    rng(o, P(1), 0, K * N, 1, true, "repack dst");
    if ((long)gx * 64 < N || (long)gy * 64 < K) note = "repack_i8: grid below the matrix";
    return 1;
  }
  if (has("dequant_i8_kernel")) {
    const long K = I(3), N = I(4);
    rng(o, P(0), 0, K * N, 1, false, "dequant q");
    rng(o, P(1), 0, N, 4, false, "dequant scales");
    rng(o, P(2), 0, K * N, 4, true, "dequant w");
    return 1;
  }
  if (has("dequant_i4_kernel")) {
    const long K = I(3), N = I(4), nblk = (K + 31) / 32;
    rng(o, P(0), 0, N * nblk * 16, 1, false, "dequant q4");
    rng(o, P(1), 0, N * nblk, 2, false, "dequant scales");
    rng(o, P(2), 0, K * N, 4, true, "dequant w");
    return 1;
  }
  if (has("f16_to_f32_rows_kernel")) {
    const long n = I(2) * I(3);
    rng(o, P(0), 0, n, 2, false, "f16 src");
    rng(o, P(1), 0, n, 4, true, "f32 dst");
    return 1;
  }
  if (has("nbits_dequant_f32_kernel")) {
    const long zpb = I(3), K = I(4), N = I(5), nblk = (K + 31) / 32;
    rng(o, P(0), 0, N * nblk * 16, 1, false, "nbits q");
    rng(o, P(1), 0, N * nblk, 4, false, "nbits scales");
    if (N > 0) rng(o, P(2), 0, (N - 1) * zpb + (nblk - 1) / 2 + 1, 1, false, "nbits zero points");
    rng(o, P(6), 0, K * N, 4, true, "nbits w");
    return 1;
  }
  if (has("snake_kernel")) {
    const long C = I(3), L = I(4);
    rng(o, P(0), 0, C * L, 4, false, "snake x");
    rng(o, P(1), 0, C, 4, false, "snake alpha");
    rng(o, P(2), 0, C * L, 4, true, "snake y");
    return 1;
  }
  if (has("adain_kernel")) {
    const long L = I(4), rows = gx;
    rng(o, P(0), 0, rows * L, 4, false, "adain x");
    rng(o, P(1), 0, rows, 4, false, "adain scale");
    rng(o, P(2), 0, rows, 4, false, "adain shift");
    rng(o, P(3), 0, rows * L, 4, true, "adain y");
    return 1;
  }
  if (has("gather_cols_kernel")) {
    const uint32_t *idx = arg<const uint32_t *>(a, 1);
    const long C = I(3), T = I(4), outCols = I(5);
    rng(o, idx, 0, outCols, 4, false, "gather indices");
    rng(o, P(2), 0, C * outCols, 4, true, "gather y");
    long mx = -1;  // the indices as uploaded (the host writes them)
    for (long f = 0; f < outCols && idx; f++) mx = std::max<long>(mx, idx[f]);
    if (mx >= T) note = "gatherCols: an index outside the row";
    if (C > 0 && mx >= 0) rng(o, P(0), 0, (C - 1) * T + mx + 1, 4, false, "gather x");
    return 1;
  }
  if (has("lstm_kernel")) {
    const long seq = I(5), inp = I(6), hid = I(7), dirs = gx;
    rng(o, P(0), 0, seq * inp, 4, false, "lstm x");
    rng(o, P(1), 0, dirs * 4 * hid * inp, 4, false, "lstm w");
    rng(o, P(2), 0, dirs * 4 * hid * hid, 4, false, "lstm r");
    rng(o, P(3), 0, dirs * 8 * hid, 4, false, "lstm b");
    rng(o, P(4), 0, seq * 2 * hid, 4, true, "lstm out");
    if (dirs > 2 || (long)threads < 4 * hid) note = "lstm: block below its gate rows or more than 2 directions";
    return 1;
  }
  if (has("jbatch_kernel")) {
    const long base = I(3), B = I(4), hid = I(5);
    rng(o, P(0), base * hid, (base + B) * hid, 4, false, "jbatch enc");
    rng(o, P(1), 0, hid, 4, false, "jbatch pred");
    rng(o, P(2), 0, B * hid, 4, true, "jbatch y");
    return 1;
  }
  if (has("argmax_rows_kernel")) {
    const long logits = I(3), rows = gx;
    rng(o, P(0), 0, rows * logits, 4, false, "argmax x");
    rng(o, P(1), 0, rows * 4, 4, true, "argmax res");
    return 1;
  }
  if (has("joint_argmax_kernel")) {
    const long frame = I(5), hidden = I(6), logits = I(8), rows = gx;
    rng(o, P(0), frame * hidden, (frame + rows) * hidden, 4, false, "jointArgmax enc");
    rng(o, P(1), 0, hidden, 4, false, "jointArgmax pred");
    rng(o, P(2), 0, hidden * logits, 4, false, "jointArgmax outW");
    rng(o, P(3), 0, logits, 4, false, "jointArgmax outB");
    rng(o, P(4), 0, rows * 4, 4, true, "jointArgmax res");
    return 1;
  }
  if (has("gemm_naive_kernel")) {
    const int bk = arg<int>(a, 2);
    const long M = I(6), N = I(7), K = I(8);
    rng(o, P(0), 0, M * K, 4, false, "naive A");
    rng(o, P(1), 0, K * N, bk ? 2 : 4, false, "naive B");
    rng(o, P(3), 0, M * N, 4, true, "naive C");
    rng(o, P(4), 0, N, 4, false, "naive bias");
    rng(o, P(5), 0, M * N, 4, false, "naive add");
    if ((long)gx * threads < M * N) note = "gemm_naive: grid below its outputs";
    return 1;
  }
  if (has("gemv_naive_kernel") || has("gemv_mfma_kernel")) {
    if (!size_is(a, 0, sizeof(GemvArgsM))) {
      note = "GemvArgs layout differs from its mirror";
      return 0;
    }
    const GemvArgsM p = arg<GemvArgsM>(a, 0);
    const bool naive = has("gemv_naive_kernel");
    const int fmt = naive ? arg<int>(a, 1) : (mangled.find("gemv_mfma_kernelILi1E") != std::string::npos ? 1 : 2);
    gemv_spans(p, fmt, o);
    if (naive && (long)gx * threads < (long)p.M * p.N) note = "gemv_naive: grid below its outputs";
    if (!naive && (p.M > 16 || (long)gx * 16 < p.N || p.K % 128)) note = "gemv_mfma: more than 16 rows, grid below N, or K not a multiple of 128";
    return 1;
  }
  if (has("gemv_batch_kernel")) {
    if (!size_is(a, 0, sizeof(GemvArgsM)) || !size_is(a, 1, sizeof(GemvItemM) * kGemvItems)) {
      note = "GemvArgs / GemvBatch layout differs from its mirror";
      return 0;
    }
    const GemvArgsM base = arg<GemvArgsM>(a, 0);
    std::vector<GemvItemM> it(kGemvItems);
    std::memcpy(it.data(), a[1].data(), sizeof(GemvItemM) * kGemvItems);
    const int fmt = mangled.find("gemv_batch_kernelILi1E") != std::string::npos ? 1 : 2;
    for (unsigned y = 0; y < gy && y < (unsigned)kGemvItems; y++) {
      GemvArgsM p = base;
      p.A = it[y].A;
      p.W = it[y].W;
      p.scales = it[y].scales;
      p.Y = it[y].Y;
      gemv_spans(p, fmt, o);
    }
    if (gy > (unsigned)kGemvItems || base.M > 16 || (long)gx * 16 * kGemvWavesM < base.N) note = "gemv_batch: items, rows or grid out of range";
    return 1;
  }
  return 0;
}

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
    if (d && !g_dry) std::memcpy(d, &v, sizeof v);  // executed: the front end indexes through it
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
    if (vrow && !g_dry) {  // executed: the q|k|v epilogue scatters V through it
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
  if (has("dwconv_gen_kernel")) {
    if (!size_is(a, 1, sizeof(CcSlotsM)) || !size_is(a, 4, sizeof(WinTable))) return 0;
    const size_t xe = has("dwconv_gen_kernelIfE") ? 4 : 2;
    const CcSlotsM cc = arg<CcSlotsM>(a, 1);
    const int use = arg<int>(a, 2), D = arg<int>(a, 8);
    const size_t cco = arg<size_t>(a, 3);
    const WinTable st = arg<WinTable>(a, 4);
    const void *y32 = arg<const void *>(a, 11);
    rd(o, arg<const void *>(a, 6), (size_t)9 * D * 4, "dw taps");
    rd(o, arg<const void *>(a, 7), (size_t)D * 4, "dw bias");
    const int nw = (int)gy;
    if (nw > st.n) note = "dwconv_gen: grid covers more windows than the table";
    if ((long)gz * 64 * 4 < D || D % 4) note = "dwconv_gen: grid.z below D / 4 lanes, or D not a multiple of 4";
    for (int w = 0; w < std::min(nw, st.n); w++) {
      const long lo = (long)st.off[w] * D, hi = (long)(st.off[w] + st.len[w]) * D;
      rng(o, arg<const void *>(a, 0), lo, hi, xe, false, "dw in");
      if (y32) {
        rng(o, y32, lo, hi, 4, true, "dw out f32");
      } else {
        rng(o, arg<const void *>(a, 9), lo, hi, 2, true, "dw out");
        rng(o, arg<const void *>(a, 10), lo, hi, 2, true, "dw out lo");
      }
      if ((int)gx < st.len[w]) note = "dwconv_gen: grid.x below a window's frames";
      if (use && w < kSG) rng(o, cc.cc_in[w], cco, cco + (size_t)8 * D, 4, false, "conv cache");
    }
    return 1;
  }
  if (has("stream_conv_cache_kernel")) {
    if (!size_is(a, 0, sizeof(CcSlotsM))) return 0;
    const size_t xe = has("stream_conv_cache_kernelIfE") ? 4 : 2;
    const CcSlotsM cc = arg<CcSlotsM>(a, 0);
    const size_t cco = arg<size_t>(a, 1);
    const long D = arg<int>(a, 3), nemit = arg<int>(a, 4), nq = arg<int>(a, 5);
    if (gx != 8) note = "stream_conv_cache: grid.x is not the cache's 8 rows";
    for (unsigned w = 0; w < gy && w < (unsigned)kSG; w++) {
      rng(o, cc.cc_out[w], cco, cco + 8 * D, 4, true, "next conv cache");
      if (nemit < 8) rng(o, cc.cc_in[w], cco + nemit * D, cco + 8 * D, 4, false, "conv cache");
      if (nemit > 0) rng(o, arg<const void *>(a, 2), ((long)w * nq + std::max(0L, nemit - 8)) * D, ((long)w * nq + nemit) * D, xe, false, "GLU rows");
      if (nemit > nq) note = "stream_conv_cache: emitted rows past the pass";
    }
    if (gy > (unsigned)kSG) note = "stream_conv_cache: more windows than cache slots";
    return 1;
  }
  if (has("zero_pad_rows_kernel")) {
    if (!size_is(a, 2, sizeof(WinTable))) return 0;
    float *x = arg<float *>(a, 0);
    const long D = arg<int>(a, 1), Tpad = arg<int>(a, 3);
    const WinTable st = arg<WinTable>(a, 2);
    if ((int)gy > st.n) note = "zero_pad_rows: grid covers more windows than the table";
    for (int w = 0; w < std::min((int)gy, st.n); w++) {
      const long end = std::min<long>(Tpad, gx);
      if (end > st.len[w]) rng(o, x, (st.off[w] + (long)st.len[w]) * D, (st.off[w] + end) * D, 4, true, "pad rows");
    }
    return 1;
  }
  if (has("v_transpose_kernel")) {
    if (!size_is(a, 2, sizeof(WinTable))) return 0;
    const long ldv = arg<int>(a, 1), H = arg<int>(a, 3), Tp = arg<int>(a, 4), HD = 128;
    const WinTable win = arg<WinTable>(a, 2);
    if ((long)gx * 64 < Tp || (long)gy != H) note = "v_transpose: grid below the keys or heads";
    if ((int)gz > win.n) note = "v_transpose: grid covers more windows than the table";
    for (int w = 0; w < std::min((int)gz, win.n); w++) {
      if (win.len[w] > Tp) note = "v_transpose: a window longer than Tp";
      if (win.len[w] > 0) rng(o, arg<const void *>(a, 0), win.off[w] * ldv, (win.off[w] + (long)win.len[w] - 1) * ldv + H * HD, 2, false, "v rows");
      rng(o, arg<const void *>(a, 5), (long)w * H * HD * Tp, (long)(w + 1) * H * HD * Tp, 2, true, "vt");
    }
    return 1;
  }
  if (has("relpos_attn_kernel")) {
    if (!size_is(a, 0, sizeof(AttnArgs))) return 0;
    const AttnArgs t = arg<AttnArgs>(a, 0);
    const size_t e = mangled.find("relpos_attn_kernelIffE") != std::string::npos ? 4 : 2;
    const long HW = (long)t.H * t.HD;
    rd(o, t.pbu, HW * 4, "pos bias u");
    rd(o, t.pbv, HW * 4, "pos bias v");
    rng(o, t.pos, 0, (long)(t.prows - 1) * t.ldp + HW, e, false, "pos table");
    const int nw = (int)gz;
    if (nw > t.win.n) note = "attention: grid covers more windows than the table";
    for (int w = 0; w < std::min(nw, t.win.n); w++) {
      const long off = t.win.off[w], T = t.win.len[w];
      if (T <= 0) continue;
      rng(o, t.q, off * t.ldq, (off + T - 1) * t.ldq + HW, e, false, "q");
      rng(o, t.k, off * t.ldk, (off + T - 1) * t.ldk + HW, e, false, "k");
      rng(o, t.v, off * t.ldv, (off + T - 1) * t.ldv + HW, e, false, "v");
      rng(o, t.out, off * t.ldo, (off + T - 1) * t.ldo + HW, e, true, "attention out");
      rng(o, t.out_lo, off * t.ldo, (off + T - 1) * t.ldo + HW, 2, true, "attention out lo");
      if ((long)gx * 64 < T) note = "attention: grid.x below a window's queries";
      if (T - 1 > t.pcenter || t.pcenter + T - 1 >= t.prows) note = "attention: window longer than the positional table";
    }
    return 1;
  }
  if (has("pack_windows_kernel")) {
    if (!size_is(a, 3, sizeof(WinTable))) return 0;
    const long Ttot = arg<long>(a, 1), MB = arg<int>(a, 2), Tpad = arg<int>(a, 5);
    const WinTable dst = arg<WinTable>(a, 3), src = arg<WinTable>(a, 4);
    if ((long)gy * 64 < MB || (int)gz > dst.n) note = "pack_windows: grid below the channels or above the windows";
    for (int w = 0; w < std::min((int)gz, dst.n); w++) {
      const long len = dst.len[w], rows = Tpad > 0 ? Tpad : len, start = src.off[w];
      if ((long)gx * 64 < rows) note = "pack_windows: grid.x below a window's rows";
      const long tin = std::min(len, Ttot - start);  // frames read: t < len and start + t < Ttot
      if (tin > 0 && MB > 0) rng(o, arg<const void *>(a, 0), start, (MB - 1) * Ttot + start + tin, 4, false, "feature stream");
      if (rows > 0 && MB > 0) rng(o, arg<const void *>(a, 6), dst.off[w] * MB, (dst.off[w] + rows) * MB, 4, true, "packed rows");
    }
    return 1;
  }
  if (has("row_map_kernel")) {
    const long rows = arg<int>(a, 1);
    rng(o, arg<const void *>(a, 2), 0, rows, 4, true, "row map");
    if ((long)gx * threads < rows) note = "row_map: grid below its rows";
    return 1;
  }
  if (has("wdq_kernel")) {
    struct WdqListM {
      const uint8_t *w[8];
      const _Float16 *s[8];
      _Float16 *out[8];
      long chunks[8];
      int n, i4;
    };
    if (!size_is(a, 0, sizeof(WdqListM))) {
      note = "WdqList layout differs from its mirror";
      return 0;
    }
    const WdqListM L = arg<WdqListM>(a, 0);
    if ((int)gy > L.n || L.n > 8) note = "wdq: grid covers more items than the list";
    for (int i = 0; i < std::min<int>((int)gy, 8); i++) {
      const long n8 = L.chunks[i];
      if ((long)gx * 256 * 4 < n8) note = "wdq: grid below an item's chunks";
      if (L.i4) {
        rng(o, L.w[i], 0, n8, 4, false, "int4 words");
        rng(o, L.s[i], 0, (n8 + 3) / 4, 2, false, "int4 scales");
      } else {
        rng(o, L.w[i], 0, n8, 8, false, "int8 bytes");
      }
      rng(o, L.out[i], 0, n8, 16, true, "widened f16");
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
  // ── TDT decoder: window state as uploaded by the host (t = 0, T = lens);
  // `w` names the fields the kernel writes (the others are read) ──
  enum { W_WIN = 1, W_HC = 2, W_PPJ = 4, W_Z = 8, W_P = 16, W_ALIVE = 32 };
  auto tdt_state = [&](size_t i, int n, int w) {
    const TdtStateM s = arg<TdtStateM>(a, i);
    auto f = [&](const void *p, size_t bytes, int bit, const char *what) { (w & bit ? wr : rd)(o, p, bytes, what); };
    f(s.win, (size_t)n * sizeof(TdtWinM), W_WIN, "tdt windows");
    f(s.h, (size_t)n * 4 * kTH * 4, W_HC, "tdt h");
    f(s.c, (size_t)n * 4 * kTH * 4, W_HC, "tdt c");
    f(s.pp, (size_t)n * kTH * 4, W_PPJ, "tdt pp");
    f(s.j, (size_t)n * kTH * 4, W_PPJ, "tdt j");
    f(s.z, (size_t)n * 32 * kTH * 4, W_Z, "tdt z");
    f(s.pv, (size_t)n * kTNB * 4, W_P, "tdt pv");
    f(s.pi, (size_t)n * kTNB * 4, W_P, "tdt pi");
    f(s.dv, (size_t)n * 4, W_P, "tdt dv");
    f(s.di, (size_t)n * 4, W_P, "tdt di");
    f(s.alive, (size_t)n * 4, W_ALIVE, "tdt alive");
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
    tdt_state(5, n, W_P);
    return 1;
  }
  if (has("tdt_update_kernel")) {
    if (!size_is(a, 0, sizeof(TdtStateM))) return 0;
    const int cap = arg<int>(a, 1), n = (int)gx;
    const TdtStateM s = tdt_state(0, n, W_WIN | W_ALIVE);
    wr(o, s.ids, (size_t)n * cap * 4, "tdt ids");
    wr(o, s.frs, (size_t)n * cap * 4, "tdt frames");
    return 1;
  }
  if (has("tdt_z_kernel")) {
    if (!size_is(a, 4, sizeof(TdtStateM))) return 0;
    const int n = arg<int>(a, 5);
    rd(o, arg<const void *>(a, 0), (size_t)4 * kTH * kTH * 4, "lstm W");
    rd(o, arg<const void *>(a, 1), (size_t)4 * kTH * kTH * 4, "lstm R");
    const TdtStateM s = tdt_state(4, n, W_Z);
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
    tdt_state(2, n, W_HC);
    return 1;
  }
  if (has("tdt_proj_kernel")) {
    if (!size_is(a, 4, sizeof(TdtStateM))) return 0;
    const int n = arg<int>(a, 5);
    rd(o, arg<const void *>(a, 0), (size_t)kTH * kTH * 4, "pred W");
    rd(o, arg<const void *>(a, 1), (size_t)kTH * 4, "pred bias");
    rd(o, arg<const void *>(a, 2), (size_t)n * 4 * kTH * 4, "pred h");
    const TdtStateM s = tdt_state(4, n, W_PPJ);
    const float *fr = arg<const float *>(a, 3);
    for (int w = 0; w < n && s.win; w++)
      if (s.win[w].T > 0) rng(o, fr, (long)s.win[w].off * kTH, (long)(s.win[w].off + s.win[w].T) * kTH, 4, false, "frames");
    if (gx * 64 != kTH) note = "tdt_proj: grid.x";
    return 1;
  }
  return op_extents(mangled, a, gx, gy, gz, threads, o, note);
}

}  // namespace audit_ext
