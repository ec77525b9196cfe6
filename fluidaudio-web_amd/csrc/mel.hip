// Log-mel front end on the GPU: PCM windows -> the encoder's feature stream.
//
// Restates the reference's JS preprocessor (JsPreprocessor,
// src/engines/asr-nemotron/nemotron-mel.js:451-603) with Parakeet's settings
// (src/engines/asr-parakeet/parakeet-mel.js:8-22: log guard 2^-24, per-feature
// normalisation), applied per window slice as the pipeline does
// (src/engines/asr-parakeet/mel-scheduler.js:8-21).  The reference computes the
// STFT in f64 (JS doubles) and rounds the power spectrum, the log-mel and the
// features to f32; gfx950 runs f64 at the f32 VALU rate, so the kernels keep
// the same f64 arithmetic, operation by operation (this file is compiled with
// -ffp-contract=off: no multiply-add is fused), and the constants (Hann window,
// twiddles, filterbank) are computed on the host in f64 exactly as the
// reference computes them.
//
//   mel_frames_kernel   one wave per frame: pre-emphasis + Hann window, the
//                       reference's radix-2 256-point complex FFT in LDS
//                       (bit reversal, explicit length-2/4/8 stages, table
//                       twiddles), real-spectrum reconstruction, power (f32),
//                       sparse filterbank sums (f64), log -> raw log-mel (f32)
//   mel_stats_kernel    per (window, bin): mean and 1/(std + 1e-5), summed over
//                       the frames in order (one thread per bin) from LDS tiles
//   mel_norm_kernel     (raw - mean) * inv, in place
#include <algorithm>
#include <cmath>
#include <cstring>
#include <mutex>
#include <vector>

#include "fa_internal.h"
#include "attention.h"

namespace fa {

constexpr int kNfft = 512, kWin = 400, kHop = 160, kBins = 257, kMaxMels = 128;

// Device constant tables, one allocation: doubles, then the filterbank, then bounds.
struct MelTab {
  double hann[kNfft];
  double c256[128], s256[128];  // twiddles of the 256-point FFT
  double c512[256], s512[256];  // twiddles of the 512-point real spectrum
};
constexpr size_t kTabFb = sizeof(MelTab);

// Slaney mel scale (nemotron-mel.js:57-69).
static double hz2mel(double f) {
  const double f_sp = 200.0 / 3, min_log_mel = 1000.0 / f_sp, step = std::log(6.4) / 27.0;
  return f >= 1000.0 ? min_log_mel + std::log(f / 1000.0) / step : f / f_sp;
}
static double mel2hz(double m) {
  const double f_sp = 200.0 / 3, min_log_mel = 1000.0 / f_sp, step = std::log(6.4) / 27.0;
  return m >= min_log_mel ? 1000.0 * std::exp(step * (m - min_log_mel)) : m * f_sp;
}

// Host tables: Hann window (nemotron-mel.js:141-151), twiddles (:163-176),
// slaney filterbank (:80-118) and its nonzero bin ranges (:401-419).
static void build_tables(int nmels, MelTab &t, std::vector<float> &fb, std::vector<int> &bounds) {
  for (int i = 0; i < kNfft; i++) t.hann[i] = 0;
  for (int n = 0; n < kWin; n++) t.hann[56 + n] = 0.5 * (1 - std::cos((2 * M_PI * n) / (kWin - 1)));
  for (int i = 0; i < 128; i++) {
    const double a = (-2 * M_PI * i) / 256;
    t.c256[i] = std::cos(a);
    t.s256[i] = std::sin(a);
  }
  for (int i = 0; i < 256; i++) {
    const double a = (-2 * M_PI * i) / 512;
    t.c512[i] = std::cos(a);
    t.s512[i] = std::sin(a);
  }
  double freqs[kBins];
  for (int i = 0; i < kBins; i++) freqs[i] = (8000.0 * i) / (kBins - 1);
  const double m0 = hz2mel(0.0), m1 = hz2mel(8000.0);
  std::vector<double> fp(nmels + 2), fd(nmels + 1);
  for (int i = 0; i < nmels + 2; i++) fp[i] = mel2hz(m0 + ((m1 - m0) * i) / (nmels + 1));
  for (int i = 0; i < nmels + 1; i++) fd[i] = fp[i + 1] - fp[i];
  fb.assign((size_t)nmels * kBins, 0.f);
  bounds.assign(2 * nmels, 0);
  for (int m = 0; m < nmels; m++) {
    const double enorm = 2.0 / (fp[m + 2] - fp[m]);
    int lo = -1, hi = -1;
    for (int k = 0; k < kBins; k++) {
      const double down = (freqs[k] - fp[m]) / fd[m], up = (fp[m + 2] - freqs[k]) / fd[m + 1];
      const float v = (float)(std::max(0.0, std::min(down, up)) * enorm);
      fb[(size_t)m * kBins + k] = v;
      if (v > 0) {
        if (lo < 0) lo = k;
        hi = k;
      }
    }
    if (lo < 0) {
      lo = 0;
      hi = -1;
    }
    bounds[2 * m] = lo;
    bounds[2 * m + 1] = hi + 1;
  }
}

// One butterfly of the reference's transform: t = w * x[q]; x[q] = x[p] - t; x[p] += t.
__device__ __forceinline__ void bfly(double *re, double *im, int p, int q, double tr, double ti) {
  const double rp = re[p], ip = im[p];
  re[q] = rp - tr;
  im[q] = ip - ti;
  re[p] = rp + tr;
  im[p] = ip + ti;
}

// Block = one wave = one frame.  grid = (frames of the longest window, windows).
// pcm: the resident sample stream; src.off/len: window start / length in samples;
// dst.off: the window's first output column; out: [nmels][total] f32.
__global__ __launch_bounds__(64) void mel_frames_kernel(const float *__restrict__ pcm, long nsamp, WinTable src, WinTable dst, const MelTab *__restrict__ tab,
                                                        const float *__restrict__ fb, const int *__restrict__ bounds, int nmels, double guard,
                                                        long total, float *__restrict__ out) {
  __shared__ double re[256], im[256];
  __shared__ float pw[kBins];
  const int w = blockIdx.y, t = blockIdx.x, lane = threadIdx.x;
  const int n = src.len[w];
  if (t >= n / kHop) return;
  const float *a = pcm + src.off[w];
  // pre-emphasis (first sample of the window kept), zero padding of 256 on
  // each side, Hann window; even samples -> re, odd -> im, bit-reversed
#pragma unroll
  for (int e = 0; e < 4; e++) {
    const int k = lane + 64 * e;  // complex index 0..255
    double v[2];
#pragma unroll
    for (int h = 0; h < 2; h++) {
      const int i = 2 * k + h;                 // frame sample 0..511
      const long j = (long)t * kHop + i - 256;  // window sample
      double x = 0;
      if (j == 0)
        x = a[0];
      else if (j > 0 && j < n)
        x = (float)((double)a[j] - 0.97 * (double)a[j - 1]);
      v[h] = x * tab->hann[i];
    }
    const int br = __builtin_bitreverse32((unsigned)k) >> 24;
    re[br] = v[0];
    im[br] = v[1];
  }
  __syncthreads();
  // length-2 and length-4 stages: twiddles (1, 0) and (0, -1)
#pragma unroll
  for (int e = 0; e < 2; e++) {
    const int p = 2 * (lane + 64 * e);
    bfly(re, im, p, p + 1, re[p + 1], im[p + 1]);
  }
  __syncthreads();
#pragma unroll
  for (int e = 0; e < 2; e++) {
    const int b = lane + 64 * e, i = (b >> 1) * 4, k = b & 1, p = i + k, q = p + 2;
    if (k == 0)
      bfly(re, im, p, q, re[q], im[q]);
    else
      bfly(re, im, p, q, im[q], -re[q]);
  }
  __syncthreads();
  // length-8 stage with the reference's constants (+-SQRT1_2, -SQRT1_2)
  {
    constexpr double r2 = 0.70710678118654757;
#pragma unroll
    for (int e = 0; e < 2; e++) {
      const int b = lane + 64 * e, i = (b >> 2) * 8, k = b & 3, p = i + k, q = p + 4;
      const double xr = re[q], xi = im[q];
      double tr, ti;
      if (k == 0) {
        tr = xr;
        ti = xi;
      } else if (k == 2) {
        tr = xi;
        ti = -xr;
      } else {
        const double wc = k == 1 ? r2 : -r2, ws = -r2;
        tr = xr * wc - xi * ws;
        ti = xr * ws + xi * wc;
      }
      bfly(re, im, p, q, tr, ti);
    }
  }
  __syncthreads();
  for (int len = 16; len <= 256; len <<= 1) {
    const int half = len >> 1, step = 256 / len;
#pragma unroll
    for (int e = 0; e < 2; e++) {
      const int b = lane + 64 * e, i = (b / half) * len, k = b % half, p = i + k, q = p + half;
      const double wc = tab->c256[k * step], ws = tab->s256[k * step];
      const double xr = re[q], xi = im[q];
      bfly(re, im, p, q, xr * wc - xi * ws, xr * ws + xi * wc);
    }
    __syncthreads();
  }
  // real-spectrum reconstruction -> power (f32), nemotron-mel.js:503-537
  if (lane == 0) {
    const double z0r = re[0], z0i = im[0];
    pw[0] = (float)((z0r + z0i) * (z0r + z0i));
    pw[256] = (float)((z0r - z0i) * (z0r - z0i));
    pw[128] = (float)(re[128] * re[128] + im[128] * im[128]);
  }
#pragma unroll
  for (int e = 0; e < 2; e++) {
    const int k = lane + 64 * e;
    if (k >= 1 && k < 128) {
      const double rk = re[k], ik = im[k], rnk = re[256 - k], ink = im[256 - k];
      const double xer = 0.5 * (rk + rnk), xei = 0.5 * (ik - ink), xor_ = 0.5 * (ik + ink), xoi = -0.5 * (rk - rnk);
      const double wc = tab->c512[k], ws = tab->s512[k];
      const double tr = xor_ * wc - xoi * ws, ti = xor_ * ws + xoi * wc;
      const double xkr = xer + tr, xki = xei + ti, xnr = xer - tr, xni = xei - ti;
      pw[k] = (float)(xkr * xkr + xki * xki);
      pw[256 - k] = (float)(xnr * xnr + xni * xni);
    }
  }
  __syncthreads();
  // filterbank over each filter's nonzero bins, in bin order; log -> f32
  for (int m = lane; m < nmels; m += 64) {
    const int lo = bounds[2 * m], hi = bounds[2 * m + 1];
    const float *f = fb + (size_t)m * kBins;
    double v = 0;
    for (int k = lo; k < hi; k++) v += (double)pw[k] * (double)f[k];
    out[(size_t)m * total + dst.off[w] + t] = (float)log(v + guard);
  }
}

// Workgroup = (16 bins, window).  The sums run over the window's frames in
// frame order in f64, one thread per bin, as the reference does; the frames
// are staged through LDS 256 at a time with coalesced loads (rows padded to
// 257 floats so the 16 summing threads hit distinct banks).
constexpr int kStatRows = 16, kStatT = 256;
__global__ __launch_bounds__(256) void mel_stats_kernel(const float *__restrict__ x, WinTable dst, int nmels, long total, double *__restrict__ stats) {
  __shared__ float tile[kStatRows][kStatT + 1];
  const int w = blockIdx.y, m0 = blockIdx.x * kStatRows, tid = threadIdx.x, T = dst.len[w];
  const int rows = min(kStatRows, nmels - m0);
  const float *base = x + (size_t)m0 * total + dst.off[w];
  double mean = 0, acc = 0;
  for (int pass = 0; pass < 2; pass++) {
    acc = 0;
    for (int t0 = 0; t0 < T; t0 += kStatT) {
      const int n = min(kStatT, T - t0);
      if (tid < n)
        for (int r = 0; r < rows; r++) tile[r][tid] = base[(size_t)r * total + t0 + tid];
      __syncthreads();
      if (tid < rows) {
        if (pass == 0)
          for (int t = 0; t < n; t++) acc += tile[tid][t];
        else
          for (int t = 0; t < n; t++) {
            const double d = tile[tid][t] - mean;
            acc += d * d;
          }
      }
      __syncthreads();
    }
    if (pass == 0) mean = acc / T;
  }
  if (tid < rows) {
    const int id = w * nmels + m0 + tid;
    stats[2 * id] = mean;
    stats[2 * id + 1] = T > 1 ? 1.0 / (sqrt(acc / (T - 1)) + 1e-5) : 0.0;
  }
}

// grid = (column blocks of the longest window, bins, windows)
__global__ __launch_bounds__(256) void mel_norm_kernel(float *__restrict__ x, WinTable dst, int nmels, long total, const double *__restrict__ stats) {
  const int w = blockIdx.z, m = blockIdx.y, t = blockIdx.x * 256 + threadIdx.x;
  if (t >= dst.len[w]) return;
  const double mean = stats[2 * (w * nmels + m)], inv = stats[2 * (w * nmels + m) + 1];
  float *r = x + (size_t)m * total + dst.off[w] + t;
  *r = (float)((*r - mean) * inv);
}

static int ensure_tables(fa_ctx *ctx, int nmels) {
  if (ctx->mel_tab && ctx->mel_tab_mels == nmels) return FA_OK;
  MelTab t;
  std::vector<float> fb;
  std::vector<int> bounds;
  build_tables(nmels, t, fb, bounds);
  const size_t bytes = kTabFb + fb.size() * 4 + bounds.size() * 4;
  if (ctx->mel_tab) {
    FA_HIP(ctx, hipStreamSynchronize(ctx->stream));  // in-flight kernels may still read the old tables
    (void)hipFree(ctx->mel_tab);
    ctx->mel_tab = nullptr;
  }
  void *p = dev_alloc(ctx, bytes);
  if (!p) return FA_E_OOM;
  ctx->mel_tab = p;
  ctx->mel_tab_mels = nmels;
  std::vector<char> host(bytes);
  std::memcpy(host.data(), &t, kTabFb);
  std::memcpy(host.data() + kTabFb, fb.data(), fb.size() * 4);
  std::memcpy(host.data() + kTabFb + fb.size() * 4, bounds.data(), bounds.size() * 4);
  FA_HIP(ctx, hipMemcpy(p, host.data(), bytes, hipMemcpyHostToDevice));
  return FA_OK;
}

// Launch the three stages for n windows; tab / fb / bounds are the constant
// tables for n_mels, stats holds 2 doubles per (window, bin) for up to kMaxWin
// windows (every slot the normalisation reads is written by mel_stats first).
static int mel_launch(fa_ctx *ctx, const float *pcm, long nsamp, const int32_t *starts, const int32_t *lens, int n, int n_mels, double log_guard,
                      int normalize, long total, float *y, const MelTab *tab, const float *fb, const int *bounds, double *stats) {
  long acc = 0;
  for (int w0 = 0; w0 < n; w0 += kMaxWin) {
    WinTable src{}, dst{};
    src.n = dst.n = std::min(kMaxWin, n - w0);
    int wmx = 0;
    for (int i = 0; i < src.n; i++) {
      src.off[i] = starts[w0 + i];
      src.len[i] = lens[w0 + i];
      dst.off[i] = (int)acc;
      dst.len[i] = lens[w0 + i] / kHop;
      acc += dst.len[i];
      wmx = std::max(wmx, dst.len[i]);
    }
    if (wmx == 0) continue;
    {
      ProfScope ps(ctx, "mel_frames");
      FA_LAUNCH(ps, mel_frames_kernel, dim3(wmx, src.n), dim3(64), 0, ctx->stream, pcm, nsamp, src, dst, tab, fb, bounds, n_mels, log_guard, total, y);
      FA_TRY(check_launch(ctx, "mel_frames"));
    }
    if (normalize) {
      {
        ProfScope ps(ctx, "mel_stats");
        FA_LAUNCH(ps, mel_stats_kernel, dim3(cdiv(n_mels, kStatRows), dst.n), dim3(256), 0, ctx->stream, (const float *)y, dst, n_mels, total, stats);
        FA_TRY(check_launch(ctx, "mel_stats"));
      }
      ProfScope ps(ctx, "mel_norm");
      FA_LAUNCH(ps, mel_norm_kernel, dim3(cdiv(wmx, 256), n_mels, dst.n), dim3(256), 0, ctx->stream, y, dst, n_mels, total, (const double *)stats);
      FA_TRY(check_launch(ctx, "mel_norm"));
    }
  }
  return FA_OK;
}

// Window / bin / size checks shared by both entry points; returns the output
// column count in *total.
static int mel_check(fa_ctx *ctx, long nsamp, const int32_t *starts, const int32_t *lens, int n, int n_mels, double log_guard, long *total) {
  if (n <= 0) return set_err(ctx, FA_E_INVALID, "melWindows: no windows");
  if (!starts || !lens) return set_err(ctx, FA_E_INVALID, "melWindows: null window arrays");
  if (n_mels < 1 || n_mels > kMaxMels) return set_err(ctx, FA_E_INVALID, "melWindows: %d mel bins (1..%d)", n_mels, kMaxMels);
  if (!(log_guard >= 0)) return set_err(ctx, FA_E_INVALID, "melWindows: log guard must be >= 0");
  long t = 0;
  for (int i = 0; i < n; i++) {
    if (lens[i] < 0 || starts[i] < 0 || (long)starts[i] + lens[i] > nsamp)
      return set_err(ctx, FA_E_INVALID, "melWindows: window %d [%d, +%d) outside the %ld-sample stream", i, starts[i], lens[i], nsamp);
    t += lens[i] / kHop;
  }
  if (t > 0x7fffffff / kMaxMels) return set_err(ctx, FA_E_INVALID, "melWindows: %ld frames in one call", t);
  *total = t;
  return FA_OK;
}

// ── allocation-free variant: one static device array per GPU ─────────────────
// Layout: the constant tables sized for kMaxMels bins (MelTab, filterbank,
// bounds), then the statistics of kMaxWin windows x kMaxMels bins.
constexpr size_t kStaticTabBytes = (kTabFb + (size_t)kMaxMels * kBins * 4 + 2 * kMaxMels * 4 + 255) / 256 * 256;
constexpr size_t kStaticStatBytes = (size_t)kMaxWin * kMaxMels * 2 * sizeof(double);
constexpr size_t kScratchBytes = kStaticTabBytes + kStaticStatBytes;
static_assert(kScratchBytes == 273920, "static scratch size (documented in fa_hip.h)");
static __device__ __align__(256) char scratch[kScratchBytes];

// Per device: the array's device address (from hipGetSymbolAddress with that
// device current; the array's host-side name is not a device address), the
// bin count its tables currently hold, and the context that uses it: one
// context per device at a time, so every use is ordered on that context's
// stream (calls from a second context are refused until the first is
// destroyed).
constexpr int kMaxDevices = 64;
struct StaticScratch {
  char *ptr = nullptr;
  int tab_mels = 0;
  const fa_ctx *owner = nullptr;
};
static StaticScratch g_static[kMaxDevices];
static std::mutex g_static_mu;

static int upload_static_tables(fa_ctx *ctx, StaticScratch &ss, int nmels) {
  MelTab t;
  std::vector<float> fb;
  std::vector<int> bounds;
  build_tables(nmels, t, fb, bounds);
  std::vector<char> host(kTabFb + fb.size() * 4 + bounds.size() * 4);
  std::memcpy(host.data(), &t, kTabFb);
  std::memcpy(host.data() + kTabFb, fb.data(), fb.size() * 4);
  std::memcpy(host.data() + kTabFb + fb.size() * 4, bounds.data(), bounds.size() * 4);
  // earlier calls (all on this context's stream) may still read the tables being replaced
  FA_HIP(ctx, hipStreamSynchronize(ctx->stream));
  FA_HIP(ctx, hipMemcpy(ss.ptr, host.data(), host.size(), hipMemcpyHostToDevice));
  ss.tab_mels = nmels;
  return FA_OK;
}

// Called by fa_ctx_create with ctx->device current: looks the array up once
// per device and fills its tables for 128 bins (Parakeet's front end).
int mel_static_init(fa_ctx *ctx) {
  if (ctx->device < 0 || ctx->device >= kMaxDevices) return set_err(ctx, FA_E_UNSUPPORTED, "device %d beyond %d", ctx->device, kMaxDevices);
  std::lock_guard<std::mutex> lk(g_static_mu);
  StaticScratch &ss = g_static[ctx->device];
  if (!ss.ptr) {
    void *p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) return set_err(ctx, FA_E_DEVICE, "hipGetSymbolAddress(mel scratch): %s", hipGetErrorString(e));
    ss.ptr = (char *)p;
    FA_TRY(upload_static_tables(ctx, ss, kMaxMels));
  }
  return FA_OK;
}

// fa_ctx_destroy: the context gives up the static scratch of its device.
void mel_static_release(fa_ctx *ctx) {
  if (ctx->device < 0 || ctx->device >= kMaxDevices) return;
  std::lock_guard<std::mutex> lk(g_static_mu);
  if (g_static[ctx->device].owner == ctx) g_static[ctx->device].owner = nullptr;
}

// The constant tables for n_mels bins and the statistics scratch for n
// windows (growing either waits for the context stream), so that later
// calls for at most n windows allocate nothing.
int mel_prepare(fa_ctx *ctx, int n, int n_mels, int normalize) {
  FA_TRY(ensure_tables(ctx, n_mels));
  const size_t sbytes = (size_t)std::min(std::max(n, 1), kMaxWin) * n_mels * 2 * sizeof(double);
  if (normalize && ctx->mel_scratch_bytes < sbytes) {
    if (ctx->mel_scratch) {
      FA_HIP(ctx, hipStreamSynchronize(ctx->stream));
      (void)hipFree(ctx->mel_scratch);
      ctx->mel_scratch = nullptr;
      ctx->mel_scratch_bytes = 0;
    }
    if (!(ctx->mel_scratch = dev_alloc(ctx, sbytes))) return FA_E_OOM;
    ctx->mel_scratch_bytes = sbytes;
  }
  return FA_OK;
}

// The log-mel features of n windows of a resident PCM stream into y
// [n_mels, *total] on the context stream (after mel_prepare for n windows).
int mel_windows_dev(fa_ctx *ctx, const float *pcm, long nsamp, const int32_t *starts, const int32_t *lens, int n, int n_mels, double log_guard,
                    int normalize, float *y, long *total) {
  FA_TRY(mel_check(ctx, nsamp, starts, lens, n, n_mels, log_guard, total));
  FA_TRY(mel_prepare(ctx, n, n_mels, normalize));
  if (*total == 0) return FA_OK;
  const MelTab *tab = (const MelTab *)ctx->mel_tab;
  const float *fb = (const float *)((const char *)ctx->mel_tab + kTabFb);
  const int *bounds = (const int *)((const char *)ctx->mel_tab + kTabFb + (size_t)n_mels * kBins * 4);
  return mel_launch(ctx, pcm, nsamp, starts, lens, n, n_mels, log_guard, normalize, *total, y, tab, fb, bounds, (double *)ctx->mel_scratch);
}

}  // namespace fa

using namespace fa;

extern "C" {

int fa_mel_windows(fa_ctx *ctx, fa_tensor pcm, const int32_t *starts, const int32_t *lens, int n, int n_mels, double log_guard, int normalize,
                   fa_tensor *out) {
  TensorRec *rp;
  FA_TRY(need(ctx, pcm, &rp, "melWindows"));
  if (rp->kind != S_F32) return set_err(ctx, FA_E_INVALID, "melWindows: PCM must be an f32 tensor");
  const long nsamp = (long)rp->rows * rp->cols;
  long total = 0;
  FA_TRY(mel_check(ctx, nsamp, starts, lens, n, n_mels, log_guard, &total));
  FA_TRY(mel_prepare(ctx, n, n_mels, normalize));
  fa_tensor o;
  TensorRec *ro;
  FA_TRY(new_tensor(ctx, n_mels, (int)total, S_F32, (size_t)n_mels * total * 4, &o, &ro));
  TensorGuard og(ctx, o);  // released unless the op completes
  rp = get(ctx, pcm);
  if (total > 0) FA_TRY(mel_windows_dev(ctx, (const float *)rp->ptr, nsamp, starts, lens, n, n_mels, log_guard, normalize, (float *)ro->ptr, &total));
  *out = og.release();
  return FA_OK;
}

int fa_mel_windows_static(fa_ctx *ctx, const float *pcm, int64_t nsamp, const int32_t *starts, const int32_t *lens, int n, int n_mels,
                          double log_guard, int normalize, float *out, int64_t out_cols) {
  if (!ctx) return FA_E_INVALID;
  if (!pcm || !out) return set_err(ctx, FA_E_INVALID, "melWindowsStatic: null device pointer");
  if (n > kMaxWin) return set_err(ctx, FA_E_UNSUPPORTED, "melWindowsStatic: %d windows in one call (the static scratch holds %d)", n, kMaxWin);
  long total = 0;
  FA_TRY(mel_check(ctx, (long)nsamp, starts, lens, n, n_mels, log_guard, &total));
  if (total != out_cols) return set_err(ctx, FA_E_INVALID, "melWindowsStatic: the windows give %ld frames, out has %lld columns", total, (long long)out_cols);
  if (ctx->device < 0 || ctx->device >= kMaxDevices) return set_err(ctx, FA_E_STATE, "melWindowsStatic: device %d", ctx->device);
  // held from the owner / table check through the launch
  std::lock_guard<std::mutex> lk(g_static_mu);
  StaticScratch &ss = g_static[ctx->device];
  if (!ss.ptr) return set_err(ctx, FA_E_STATE, "melWindowsStatic: static scratch not set up for device %d", ctx->device);
  if (ss.owner && ss.owner != ctx)
    return set_err(ctx, FA_E_STATE, "melWindowsStatic: another context on device %d uses the static scratch (one context per device)", ctx->device);
  ss.owner = ctx;
  if (ss.tab_mels != n_mels) FA_TRY(upload_static_tables(ctx, ss, n_mels));  // another bin count: synchronous (not capturable)
  if (total == 0) return FA_OK;
  const MelTab *tab = (const MelTab *)ss.ptr;
  const float *fb = (const float *)(ss.ptr + kTabFb);
  const int *bounds = (const int *)(ss.ptr + kTabFb + (size_t)n_mels * kBins * 4);
  double *stats = (double *)(ss.ptr + kStaticTabBytes);
  return mel_launch(ctx, pcm, (long)nsamp, starts, lens, n, n_mels, log_guard, normalize, total, out, tab, fb, bounds, stats);
}

}  // extern "C"
