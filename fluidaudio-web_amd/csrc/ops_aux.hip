// The remaining required members of the reference's backend contract
// (src/gpu/compute.d.ts:174-234): the TTS-side ops (lstm, snake, adain,
// convTranspose1d, im2col, gatherCols, leakyRelu) and the TDT decoder-side
// fusions (jbatch, argmaxRows, jointArgmax).  None is on the encoder's hot
// path; each is a plain, correct kernel with the arithmetic of the reference's
// CPU backend (src/gpu/wasm-context.js), which computes in JS doubles and
// stores f32: accumulations here run in f64 in the reference's order where it
// decides results (argmax indices), and this file is compiled with
// -ffp-contract=off so no multiply-add is fused.
#include <algorithm>
#include <vector>

#include "fa_internal.h"
#include "fa_device.h"

namespace fa {

static inline unsigned grid_of(long n) {
  const long b = (n + 255) / 256;
  return (unsigned)std::max(1L, std::min(b, 65535L * 4));
}

// leakyRelu (wasm-context.js:406-413): v > 0 ? v : slope * v, slope a JS double.
__global__ void leaky_relu_kernel(const float *x, float *y, long n, double slope) {
  for (long i = (long)blockIdx.x * 256 + threadIdx.x; i < n; i += (long)gridDim.x * 256) {
    const float v = x[i];
    y[i] = v > 0.f ? v : (float)(slope * (double)v);
  }
}

// snake (wasm-context.js:414-427): x + sin(a x)^2 / (a + 1e-9), a per row.
__global__ void snake_kernel(const float *x, const float *alpha, float *y, int C, int L) {
  const long n = (long)C * L;
  for (long i = (long)blockIdx.x * 256 + threadIdx.x; i < n; i += (long)gridDim.x * 256) {
    const double a = alpha[i / L], v = x[i];
    const double inv = 1.0 / (a + 1e-9), s = sin(a * v);
    y[i] = (float)(v + inv * s * s);
  }
}

// adain (wasm-context.js:344-362): per row, mean and variance over the row in
// f64, then (x - mean) * rsqrt(var + eps) * scale[row] + shift[row].
// One 256-thread block per row; partial sums in f64, combined in LDS.
__global__ __launch_bounds__(256) void adain_kernel(const float *x, const float *scale, const float *shift, float *y, int L, double eps) {
  __shared__ double red[256];
  const int r = blockIdx.x, t = threadIdx.x;
  const float *xr = x + (size_t)r * L;
  double s = 0;
  for (int j = t; j < L; j += 256) s += xr[j];
  red[t] = s;
  __syncthreads();
  for (int w = 128; w > 0; w >>= 1) {
    if (t < w) red[t] += red[t + w];
    __syncthreads();
  }
  const double mean = red[0] / L;
  __syncthreads();
  double v = 0;
  for (int j = t; j < L; j += 256) {
    const double d = xr[j] - mean;
    v += d * d;
  }
  red[t] = v;
  __syncthreads();
  for (int w = 128; w > 0; w >>= 1) {
    if (t < w) red[t] += red[t + w];
    __syncthreads();
  }
  const double inv = 1.0 / sqrt(red[0] / L + eps), sc = scale[r], sh = shift[r];
  for (int j = t; j < L; j += 256) y[(size_t)r * L + j] = (float)((xr[j] - mean) * inv * sc + sh);
}

// im2col (wasm-context.js:271-285): x [Cin, L] -> [Cin*k, Lout], zero padding.
__global__ void im2col_kernel(const float *x, float *y, int Cin, int L, int k, int Lout, int stride, int pad, int dilation) {
  const long n = (long)Cin * k * Lout;
  for (long i = (long)blockIdx.x * 256 + threadIdx.x; i < n; i += (long)gridDim.x * 256) {
    const int lo = (int)(i % Lout);
    const long rk = i / Lout;
    const int kk = (int)(rk % k), ci = (int)(rk / k);
    const int li = lo * stride + kk * dilation - pad;
    y[i] = (li >= 0 && li < L) ? x[(size_t)ci * L + li] : 0.f;
  }
}

// convTranspose1d (wasm-context.js:686-741): x [Cin, L], w [Cin][Cout/g][k];
// out[co, lo] = bias + Σ_{ci in group, kk} x[ci, li] w[ci, co, kk] over
// lo + pad - kk*dilation = li*stride; accumulated in f64, act applied once.
__global__ void conv_transpose1d_kernel(const float *x, const float *w, const float *bias, float *y, int Cin, int L, int Cout, int k, int Lout,
                                        int stride, int pad, int dilation, int groups, int act) {
  const long n = (long)Cout * Lout;
  const int cinG = Cin / groups, coutG = Cout / groups;
  for (long i = (long)blockIdx.x * 256 + threadIdx.x; i < n; i += (long)gridDim.x * 256) {
    const int lo = (int)(i % Lout), co = (int)(i / Lout);
    const int g = co / coutG, coInG = co - g * coutG;
    double acc = bias ? bias[co] : 0.0;
    for (int ci = 0; ci < cinG; ci++) {
      const int rc = g * cinG + ci;
      for (int kk = 0; kk < k; kk++) {
        const int num = lo + pad - kk * dilation;
        if (num < 0 || num % stride) continue;
        const int li = num / stride;
        if (li < L) acc += (double)x[(size_t)rc * L + li] * (double)w[((size_t)rc * coutG + coInG) * k + kk];
      }
    }
    y[i] = act_apply((float)acc, act);
  }
}

// gatherCols (wasm-context.js:453-460): out[r, f] = x[r, idx[f]].
__global__ void gather_cols_kernel(const float *x, const uint32_t *idx, float *y, int C, int T, int outCols) {
  const long n = (long)C * outCols;
  for (long i = (long)blockIdx.x * 256 + threadIdx.x; i < n; i += (long)gridDim.x * 256) {
    const int f = (int)(i % outCols), r = (int)(i / outCols);
    y[i] = x[(size_t)r * T + idx[f]];
  }
}

// Bidirectional LSTM, batch 1 (wasm-context.js:742-776; ONNX gate order
// i, o, f, c).  w [2][4H][inp], r [2][4H][H], b [2][8H] (Wb then Rb).  One
// block per direction, one thread per gate row (4H <= 1024): every step the
// gate pre-activations (f64, bias first, then W·x, then R·h, each in k order)
// go to LDS, then the first H threads update the cell.  c and h are kept as
// f32, as the reference stores them in Float32Arrays.
__global__ __launch_bounds__(1024) void lstm_kernel(const float *x, const float *w, const float *r, const float *b, float *out, int seq, int inp,
                                                    int hid) {
  extern __shared__ double sm[];
  double *gate = sm;                        // [4H]
  float *h = reinterpret_cast<float *>(sm + 4 * hid);  // [H]
  float *c = h + hid;                       // [H]
  const int dir = blockIdx.x, g = threadIdx.x;
  const float *wd = w + (size_t)dir * 4 * hid * inp, *rd = r + (size_t)dir * 4 * hid * hid, *bd = b + (size_t)dir * 8 * hid;
  if (g < hid) {
    h[g] = 0.f;
    c[g] = 0.f;
  }
  __syncthreads();
  for (int s = 0; s < seq; s++) {
    const int t = dir ? seq - 1 - s : s;
    if (g < 4 * hid) {
      double acc = (double)bd[g] + (double)bd[4 * hid + g];
      const float *wr = wd + (size_t)g * inp, *xt = x + (size_t)t * inp;
      for (int kk = 0; kk < inp; kk++) acc += (double)wr[kk] * (double)xt[kk];
      const float *rr = rd + (size_t)g * hid;
      for (int kk = 0; kk < hid; kk++) acc += (double)rr[kk] * (double)h[kk];
      gate[g] = acc;
    }
    __syncthreads();
    if (g < hid) {
      const double it = 1.0 / (1.0 + exp(-gate[g])), ot = 1.0 / (1.0 + exp(-gate[hid + g]));
      const double ft = 1.0 / (1.0 + exp(-gate[2 * hid + g])), ct = tanh(gate[3 * hid + g]);
      const float cn = (float)(ft * (double)c[g] + it * ct);
      const float hn = (float)(ot * tanh((double)cn));
      c[g] = cn;
      h[g] = hn;  // read by the next step only, after the barrier below
      out[((size_t)t * 2 + dir) * hid + g] = hn;
    }
    __syncthreads();
  }
}

// jbatch (wasm-context.js:564-572): out[i, k] = relu(encProj[base+i, k] + predProj[k]).
__global__ void jbatch_kernel(const float *enc, const float *pred, float *y, int base, int B, int hid) {
  const long n = (long)B * hid;
  for (long i = (long)blockIdx.x * 256 + threadIdx.x; i < n; i += (long)gridDim.x * 256) {
    const int k = (int)(i % hid), r = (int)(i / hid);
    const float v = enc[((size_t)base + r) * hid + k] + pred[k];
    y[i] = v > 0.f ? v : 0.f;
  }
}

// Token / duration argmax of a row of logits (first maximum wins, as the
// reference's strict > scan from start values 0 / -1e30).  Each thread scans
// its columns n = t, t + blockDim, ... in order; the block then reduces,
// preferring the lower index on equal values, which gives the sequential
// scan's answer.
struct ArgBest {
  double bv = -1e30, bdv = -1e30;
  int bt = 0x7fffffff, bd = 0x7fffffff;
  __device__ void see(double v, int n, int vocab) {
    if (n < vocab) {
      if (v > bv) { bv = v; bt = n; }
    } else if (v > bdv) { bdv = v; bd = n - vocab; }
  }
  __device__ void merge(double ov, int ot, double odv, int od) {
    if (ov > bv || (ov == bv && ot < bt)) { bv = ov; bt = ot; }
    if (odv > bdv || (odv == bdv && od < bd)) { bdv = odv; bd = od; }
  }
};

// blockDim.x a multiple of 64, at most 1024; thread 0 writes res[0..3].
__device__ void block_argmax(ArgBest b, float *res) {
  __shared__ double sv[16], sdv[16];
  __shared__ int st[16], sd[16];
  for (int off = 32; off > 0; off >>= 1)
    b.merge(__shfl_xor(b.bv, off), __shfl_xor(b.bt, off), __shfl_xor(b.bdv, off), __shfl_xor(b.bd, off));
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
  if (lane == 0) {
    sv[wave] = b.bv; st[wave] = b.bt; sdv[wave] = b.bdv; sd[wave] = b.bd;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < nw; w++) b.merge(sv[w], st[w], sdv[w], sd[w]);
    res[0] = (float)(b.bt == 0x7fffffff ? 0 : b.bt);
    res[1] = (float)b.bv;
    res[2] = (float)(b.bd == 0x7fffffff ? 0 : b.bd);
    res[3] = (float)b.bdv;
  }
}

// argmaxRows (wasm-context.js:573-598): x [B, logits] -> [B, 4]; one block per row.
__global__ __launch_bounds__(256) void argmax_rows_kernel(const float *x, float *res, int vocab, int logits) {
  const int r = blockIdx.x;
  ArgBest b;
  for (int n = threadIdx.x; n < logits; n += blockDim.x) b.see(x[(size_t)r * logits + n], n, vocab);
  block_argmax(b, res + (size_t)r * 4);
}

// jointArgmax (wasm-context.js:599-633): for frame+w, j = relu(encProj + pred)
// (f32), logits s[n] = outB[n] + Σ_k j[k] outW[k, n] summed in f64 in k order
// (each product of two f32 values is exact in f64, so every partial sum is
// the reference's), then the row argmax.  One 256-thread block per frame.
__global__ __launch_bounds__(256) void joint_argmax_kernel(const float *enc, const float *pred, const float *outW, const float *outB, float *res,
                                                           int frame, int hidden, int vocab, int logits) {
  extern __shared__ float jv[];  // [hidden]
  const int w = blockIdx.x, t = threadIdx.x;
  for (int k = t; k < hidden; k += 256) {
    const float v = enc[((size_t)frame + w) * hidden + k] + pred[k];
    jv[k] = v > 0.f ? v : 0.f;
  }
  __syncthreads();
  ArgBest b;
  for (int n = t; n < logits; n += 256) {
    double acc = outB[n];
    for (int k = 0; k < hidden; k++) acc += (double)jv[k] * (double)outW[(size_t)k * logits + n];
    b.see(acc, n, vocab);
  }
  block_argmax(b, res + (size_t)w * 4);
}

}  // namespace fa

using namespace fa;

#define F32P(r) reinterpret_cast<float *>((r)->ptr)
#define CF32P(r) reinterpret_cast<const float *>((r) ? (r)->ptr : nullptr)

static int need32(fa_ctx *ctx, fa_tensor t, TensorRec **r, const char *what) {
  FA_TRY(need(ctx, t, r, what));
  if ((*r)->kind != S_F32) return set_err(ctx, FA_E_INVALID, "%s: expected an f32 tensor", what);
  return FA_OK;
}

static int out32(fa_ctx *ctx, int rows, int cols, fa_tensor *o, TensorRec **ro) {
  return new_tensor(ctx, rows, cols, S_F32, (size_t)rows * cols * 4, o, ro);
}

extern "C" {

int fa_leaky_relu(fa_ctx *ctx, fa_tensor x, double slope, fa_tensor *out) {
  TensorRec *rx, *ro;
  FA_TRY(need32(ctx, x, &rx, "leakyRelu"));
  fa_tensor o;
  FA_TRY(out32(ctx, rx->rows, rx->cols, &o, &ro));
  TensorGuard og(ctx, o);  // released unless the op completes
  rx = get(ctx, x);
  const long n = (long)rx->rows * rx->cols;
  ProfScope ps(ctx, "leakyRelu");
  if (n) FA_LAUNCH(ps, leaky_relu_kernel, dim3(grid_of(n)), dim3(256), 0, ctx->stream, F32P(rx), F32P(ro), n, slope);
  FA_TRY(check_launch(ctx, "leakyRelu"));
  *out = og.release();
  return FA_OK;
}

int fa_snake(fa_ctx *ctx, fa_tensor x, fa_tensor alpha, fa_tensor *out) {
  TensorRec *rx, *ra, *ro;
  FA_TRY(need32(ctx, x, &rx, "snake"));
  FA_TRY(need32(ctx, alpha, &ra, "snake alpha"));
  if ((long)ra->rows * ra->cols < rx->rows) return set_err(ctx, FA_E_INVALID, "snake: alpha has %d values, x has %d rows", ra->rows * ra->cols, rx->rows);
  fa_tensor o;
  FA_TRY(out32(ctx, rx->rows, rx->cols, &o, &ro));
  TensorGuard og(ctx, o);  // released unless the op completes
  rx = get(ctx, x); ra = get(ctx, alpha);
  const long n = (long)rx->rows * rx->cols;
  ProfScope ps(ctx, "snake");
  if (n) FA_LAUNCH(ps, snake_kernel, dim3(grid_of(n)), dim3(256), 0, ctx->stream, F32P(rx), F32P(ra), F32P(ro), rx->rows, rx->cols);
  FA_TRY(check_launch(ctx, "snake"));
  *out = og.release();
  return FA_OK;
}

int fa_adain(fa_ctx *ctx, fa_tensor x, fa_tensor scale, fa_tensor shift, double eps, fa_tensor *out) {
  TensorRec *rx, *rs, *rh, *ro;
  FA_TRY(need32(ctx, x, &rx, "adain"));
  FA_TRY(need32(ctx, scale, &rs, "adain scale"));
  FA_TRY(need32(ctx, shift, &rh, "adain shift"));
  if ((long)rs->rows * rs->cols < rx->rows || (long)rh->rows * rh->cols < rx->rows) return set_err(ctx, FA_E_INVALID, "adain: scale/shift shorter than %d rows", rx->rows);
  if (rx->cols <= 0) return set_err(ctx, FA_E_INVALID, "adain: empty rows");
  fa_tensor o;
  FA_TRY(out32(ctx, rx->rows, rx->cols, &o, &ro));
  TensorGuard og(ctx, o);  // released unless the op completes
  rx = get(ctx, x); rs = get(ctx, scale); rh = get(ctx, shift);
  ProfScope ps(ctx, "adain");
  if (rx->rows) FA_LAUNCH(ps, adain_kernel, dim3(rx->rows), dim3(256), 0, ctx->stream, F32P(rx), F32P(rs), F32P(rh), F32P(ro), rx->cols, eps);
  FA_TRY(check_launch(ctx, "adain"));
  *out = og.release();
  return FA_OK;
}

int fa_im2col(fa_ctx *ctx, fa_tensor x, int k, int stride, int pad, int dilation, fa_tensor *out) {
  TensorRec *rx, *ro;
  FA_TRY(need32(ctx, x, &rx, "im2col"));
  if (k <= 0 || stride <= 0 || pad < 0 || dilation <= 0) return set_err(ctx, FA_E_INVALID, "im2col: bad geometry");
  const int Cin = rx->rows, L = rx->cols;
  const int Lout = (L + 2 * pad - dilation * (k - 1) - 1) / stride + 1;
  if (Lout <= 0) return set_err(ctx, FA_E_INVALID, "im2col: empty output");
  fa_tensor o;
  FA_TRY(out32(ctx, Cin * k, Lout, &o, &ro));
  TensorGuard og(ctx, o);  // released unless the op completes
  rx = get(ctx, x);
  const long n = (long)Cin * k * Lout;
  ProfScope ps(ctx, "im2col");
  FA_LAUNCH(ps, im2col_kernel, dim3(grid_of(n)), dim3(256), 0, ctx->stream, F32P(rx), F32P(ro), Cin, L, k, Lout, stride, pad, dilation);
  FA_TRY(check_launch(ctx, "im2col"));
  *out = og.release();
  return FA_OK;
}

int fa_conv_transpose1d(fa_ctx *ctx, fa_tensor x, fa_tensor w, int cout, int k, fa_tensor bias, int stride, int pad, int dilation, int groups,
                        int output_padding, int act, fa_tensor *out) {
  TensorRec *rx, *rw, *rb, *ro;
  FA_TRY(need32(ctx, x, &rx, "convTranspose1d"));
  FA_TRY(need32(ctx, w, &rw, "convTranspose1d w"));
  FA_TRY(opt(ctx, bias, &rb, "convTranspose1d bias"));
  const int Cin = rx->rows, L = rx->cols;
  if (groups <= 0 || Cin % groups || cout % groups || k <= 0 || stride <= 0 || dilation <= 0 || pad < 0 || output_padding < 0 || act < 0 || act > 5)
    return set_err(ctx, FA_E_INVALID, "convTranspose1d: bad geometry (cin %d, cout %d, groups %d)", Cin, cout, groups);
  if ((long)rw->rows * rw->cols < (long)Cin * (cout / groups) * k) return set_err(ctx, FA_E_INVALID, "convTranspose1d: weight too small");
  if (rb && (long)rb->rows * rb->cols < cout) return set_err(ctx, FA_E_INVALID, "convTranspose1d: bias shorter than %d", cout);
  const int Lout = (L - 1) * stride - 2 * pad + dilation * (k - 1) + output_padding + 1;
  if (Lout <= 0) return set_err(ctx, FA_E_INVALID, "convTranspose1d: empty output");
  fa_tensor o;
  FA_TRY(out32(ctx, cout, Lout, &o, &ro));
  TensorGuard og(ctx, o);  // released unless the op completes
  rx = get(ctx, x); rw = get(ctx, w); rb = bias ? get(ctx, bias) : nullptr;
  ProfScope ps(ctx, "convTranspose1d");
  FA_LAUNCH(ps, conv_transpose1d_kernel, dim3(grid_of((long)cout * Lout)), dim3(256), 0, ctx->stream, F32P(rx), F32P(rw), CF32P(rb), F32P(ro), Cin, L,
            cout, k, Lout, stride, pad, dilation, groups, act);
  FA_TRY(check_launch(ctx, "convTranspose1d"));
  *out = og.release();
  return FA_OK;
}

int fa_gather_cols(fa_ctx *ctx, fa_tensor x, const uint32_t *idx, int n_idx, fa_tensor *out) {
  TensorRec *rx, *ro, *ri;
  FA_TRY(need32(ctx, x, &rx, "gatherCols"));
  if (n_idx <= 0 || !idx) return set_err(ctx, FA_E_INVALID, "gatherCols: empty index map");
  for (int f = 0; f < n_idx; f++)
    if (idx[f] >= (uint32_t)rx->cols) return set_err(ctx, FA_E_INVALID, "gatherCols: index %u at %d outside %d columns", idx[f], f, rx->cols);
  fa_tensor o, ti;
  FA_TRY(out32(ctx, rx->rows, n_idx, &o, &ro));
  TensorGuard og(ctx, o);  // released unless the op completes
  FA_TRY(new_tensor(ctx, 1, n_idx, S_BYTES, (size_t)n_idx * 4, &ti, &ri));
  FA_HIP(ctx, hipMemcpyAsync(ri->ptr, idx, (size_t)n_idx * 4, hipMemcpyHostToDevice, ctx->stream));
  FA_HIP(ctx, hipStreamSynchronize(ctx->stream));  // the host index array may go away when this call returns
  rx = get(ctx, x); ro = get(ctx, o); ri = get(ctx, ti);
  const long n = (long)rx->rows * n_idx;
  ProfScope ps(ctx, "gatherCols");
  if (n) FA_LAUNCH(ps, gather_cols_kernel, dim3(grid_of(n)), dim3(256), 0, ctx->stream, F32P(rx), (const uint32_t *)ri->ptr, F32P(ro), rx->rows, rx->cols, n_idx);
  FA_TRY(check_launch(ctx, "gatherCols"));
  FA_TRY(fa_free_tensor(ctx, ti));  // pooled storage: later allocations follow on the same stream
  *out = og.release();
  return FA_OK;
}

int fa_lstm(fa_ctx *ctx, fa_tensor x, fa_tensor w, fa_tensor r, fa_tensor b, int hid, fa_tensor *out) {
  TensorRec *rx, *rw, *rr, *rb, *ro;
  FA_TRY(need32(ctx, x, &rx, "lstm"));
  FA_TRY(need32(ctx, w, &rw, "lstm W"));
  FA_TRY(need32(ctx, r, &rr, "lstm R"));
  FA_TRY(need32(ctx, b, &rb, "lstm B"));
  const int seq = rx->rows, inp = rx->cols;
  if (hid <= 0 || hid > 256) return set_err(ctx, FA_E_UNSUPPORTED, "lstm: hidden size %d (1..256)", hid);
  if ((long)rw->rows * rw->cols < 8L * hid * inp || (long)rr->rows * rr->cols < 8L * hid * hid || (long)rb->rows * rb->cols < 16L * hid)
    return set_err(ctx, FA_E_INVALID, "lstm: W/R/B smaller than [2,4H,%d] / [2,4H,H] / [2,8H]", inp);
  fa_tensor o;
  FA_TRY(out32(ctx, seq, 2 * hid, &o, &ro));
  TensorGuard og(ctx, o);  // released unless the op completes
  rx = get(ctx, x); rw = get(ctx, w); rr = get(ctx, r); rb = get(ctx, b);
  const size_t smem = (size_t)4 * hid * 8 + (size_t)2 * hid * 4;
  ProfScope ps(ctx, "lstm");
  if (seq) FA_LAUNCH(ps, lstm_kernel, dim3(2), dim3(std::max(64, (4 * hid + 63) / 64 * 64)), smem, ctx->stream, F32P(rx), F32P(rw), F32P(rr), F32P(rb), F32P(ro),
                     seq, inp, hid);
  FA_TRY(check_launch(ctx, "lstm"));
  *out = og.release();
  return FA_OK;
}

int fa_jbatch(fa_ctx *ctx, fa_tensor enc, int base, int B, fa_tensor pred, int hid, fa_tensor *out) {
  TensorRec *re, *rp, *ro;
  FA_TRY(need32(ctx, enc, &re, "jbatch"));
  FA_TRY(need32(ctx, pred, &rp, "jbatch predProj"));
  if (base < 0 || B <= 0 || hid <= 0 || (long)(base + B) * hid > (long)re->rows * re->cols || (long)rp->rows * rp->cols < hid)
    return set_err(ctx, FA_E_INVALID, "jbatch: rows [%d, %d) x %d outside the inputs", base, base + B, hid);
  fa_tensor o;
  FA_TRY(out32(ctx, B, hid, &o, &ro));
  TensorGuard og(ctx, o);  // released unless the op completes
  re = get(ctx, enc); rp = get(ctx, pred);
  ProfScope ps(ctx, "jbatch");
  FA_LAUNCH(ps, jbatch_kernel, dim3(grid_of((long)B * hid)), dim3(256), 0, ctx->stream, F32P(re), F32P(rp), F32P(ro), base, B, hid);
  FA_TRY(check_launch(ctx, "jbatch"));
  *out = og.release();
  return FA_OK;
}

int fa_argmax_rows(fa_ctx *ctx, fa_tensor x, int B, int vocab, int logits, fa_tensor *out) {
  TensorRec *rx, *ro;
  FA_TRY(need32(ctx, x, &rx, "argmaxRows"));
  if (B <= 0 || logits <= 0 || vocab < 0 || vocab > logits || (long)B * logits > (long)rx->rows * rx->cols)
    return set_err(ctx, FA_E_INVALID, "argmaxRows: %d rows of %d logits (vocab %d) outside the input", B, logits, vocab);
  fa_tensor o;
  FA_TRY(out32(ctx, B, 4, &o, &ro));
  TensorGuard og(ctx, o);  // released unless the op completes
  rx = get(ctx, x);
  ProfScope ps(ctx, "argmaxRows");
  FA_LAUNCH(ps, argmax_rows_kernel, dim3(B), dim3(256), 0, ctx->stream, F32P(rx), F32P(ro), vocab, logits);
  FA_TRY(check_launch(ctx, "argmaxRows"));
  *out = og.release();
  return FA_OK;
}

int fa_joint_argmax(fa_ctx *ctx, fa_tensor enc, int frame, int count, fa_tensor pred, fa_tensor outW, fa_tensor outB, int hidden, int vocab, int logits,
                    fa_tensor *out) {
  TensorRec *re, *rp, *rw, *rb, *ro;
  FA_TRY(need32(ctx, enc, &re, "jointArgmax"));
  FA_TRY(need32(ctx, pred, &rp, "jointArgmax predProj"));
  FA_TRY(need32(ctx, outW, &rw, "jointArgmax outW"));
  FA_TRY(need32(ctx, outB, &rb, "jointArgmax outB"));
  if (frame < 0 || count <= 0 || hidden <= 0 || logits <= 0 || vocab < 0 || vocab > logits || hidden > 16384 ||
      (long)(frame + count) * hidden > (long)re->rows * re->cols || (long)rp->rows * rp->cols < hidden ||
      (long)rw->rows * rw->cols < (long)hidden * logits || (long)rb->rows * rb->cols < logits)
    return set_err(ctx, FA_E_INVALID, "jointArgmax: frames [%d, %d), hidden %d, logits %d outside the inputs", frame, frame + count, hidden, logits);
  fa_tensor o;
  FA_TRY(out32(ctx, count, 4, &o, &ro));
  TensorGuard og(ctx, o);  // released unless the op completes
  re = get(ctx, enc); rp = get(ctx, pred); rw = get(ctx, outW); rb = get(ctx, outB);
  const size_t smem = (size_t)hidden * 4;
  ProfScope ps(ctx, "jointArgmax");
  FA_LAUNCH(ps, joint_argmax_kernel, dim3(count), dim3(256), smem, ctx->stream, F32P(re), F32P(rp), F32P(rw), F32P(rb), F32P(ro), frame, hidden, vocab,
            logits);
  FA_TRY(check_launch(ctx, "jointArgmax"));
  *out = og.release();
  return FA_OK;
}

}  // extern "C"
