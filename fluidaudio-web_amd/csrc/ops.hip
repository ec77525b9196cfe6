// ComputeContext ops (src/gpu/compute.d.ts:155-228) on fp32 tensors: the
// encoder's op subset, each a gfx950 kernel.  Bandwidth kernels use one wave
// per row with wave-shuffle reductions (the reference uses a 64-lane
// workgroup-memory tree, normalization.js:29-58, and one thread per softmax
// row, normalization.js:61-77).
#include <cstring>
#include <vector>

#include "fa_internal.h"
#include "fa_device.h"
#include "gemm.h"
#include "attention.h"
#include "ops.h"

namespace fa {

// ── row layernorm: f32 in, f32 or f16 out; one wave per row ───────────────
template <typename TO>
__global__ __launch_bounds__(256) void layernorm_kernel(const float *x, const float *__restrict__ gamma, const float *__restrict__ beta,
                                                        TO *y, int rows, int cols, int ldx, int ldy,
                                                        float eps) {
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (row >= rows) return;
  const float *xr = x + (size_t)row * ldx;
  TO *yr = y + (size_t)row * ldy;
  if (cols == 1024) {  // the encoder width: 16 values per lane held in registers
    float4 v[4];
    float s = 0.f;
#pragma unroll
    for (int t = 0; t < 4; t++) {
      v[t] = reinterpret_cast<const float4 *>(xr)[lane + 64 * t];
      s += v[t].x + v[t].y + v[t].z + v[t].w;
    }
    const float mean = wave_sum(s) * (1.f / 1024.f);
    float q = 0.f;
#pragma unroll
    for (int t = 0; t < 4; t++) {
      float a = v[t].x - mean, b = v[t].y - mean, c = v[t].z - mean, d = v[t].w - mean;
      q += a * a + b * b + c * c + d * d;
    }
    const float inv = rsqrtf(wave_sum(q) * (1.f / 1024.f) + eps);
#pragma unroll
    for (int t = 0; t < 4; t++) {
      const int c0 = (lane + 64 * t) * 4;
      const float4 gm = reinterpret_cast<const float4 *>(gamma)[lane + 64 * t];
      const float4 bt = reinterpret_cast<const float4 *>(beta)[lane + 64 * t];
      yr[c0 + 0] = (TO)((v[t].x - mean) * inv * gm.x + bt.x);
      yr[c0 + 1] = (TO)((v[t].y - mean) * inv * gm.y + bt.y);
      yr[c0 + 2] = (TO)((v[t].z - mean) * inv * gm.z + bt.z);
      yr[c0 + 3] = (TO)((v[t].w - mean) * inv * gm.w + bt.w);
    }
    return;
  }
  float s = 0.f;
  for (int j = lane; j < cols; j += 64) s += xr[j];
  const float mean = wave_sum(s) / cols;
  float q = 0.f;
  for (int j = lane; j < cols; j += 64) {
    const float d = xr[j] - mean;
    q += d * d;
  }
  const float inv = rsqrtf(wave_sum(q) / cols + eps);
  for (int j = lane; j < cols; j += 64) yr[j] = (TO)((xr[j] - mean) * inv * gamma[j] + beta[j]);
}

int layernorm_launch(fa_ctx *ctx, const float *x, const float *g, const float *b, void *y, int out_f16, int rows, int cols, int ldx, int ldy,
                     float eps, const char *label) {
  if (rows <= 0) return FA_OK;
  ProfScope ps(ctx, label);
  if (out_f16)
    FA_LAUNCH(ps, layernorm_kernel<_Float16>, dim3(cdiv(rows, 4)), dim3(256), 0, ctx->stream, x, g, b, (_Float16 *)y, rows, cols, ldx, ldy, eps);
  else
    FA_LAUNCH(ps, layernorm_kernel<float>, dim3(cdiv(rows, 4)), dim3(256), 0, ctx->stream, x, g, b, (float *)y, rows, cols, ldx, ldy, eps);
  return check_launch(ctx, label);
}

// ── softmax: one wave per row ─────────────────────────────────────────────
__global__ __launch_bounds__(256) void softmax_kernel(const float *__restrict__ x, float *__restrict__ y, int rows, int cols) {
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (row >= rows) return;
  const float *xr = x + (size_t)row * cols;
  float *yr = y + (size_t)row * cols;
  float mx = -INFINITY;
  for (int j = lane; j < cols; j += 64) mx = fmaxf(mx, xr[j]);
  mx = wave_max(mx);
  float s = 0.f;
  for (int j = lane; j < cols; j += 64) s += __expf(xr[j] - mx);
  const float inv = 1.f / wave_sum(s);
  for (int j = lane; j < cols; j += 64) yr[j] = __expf(xr[j] - mx) * inv;
}

// ── elementwise ───────────────────────────────────────────────────────────
__global__ void ewise_kernel(const float *a, const float *b, float *c, long n, int cols, int bcast, int op) {
  for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (long)gridDim.x * blockDim.x) {
    const float bv = bcast ? b[i % cols] : b[i];
    c[i] = op ? a[i] * bv : a[i] + bv;
  }
}
__global__ void unary_kernel(const float *x, float *y, long n, int kind, float s) {
  for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (long)gridDim.x * blockDim.x) {
    const float v = x[i];
    y[i] = kind == 0 ? v * s : (kind == 1 ? silu_f(v) : fmaxf(v, 0.f));
  }
}
__global__ void glu_kernel(const float *x, float *y, int C, int T) {
  const long n = (long)C * T;
  for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (long)gridDim.x * blockDim.x) {
    const long c = i / T, t = i % T;
    const float a = x[c * T + t], b = x[(c + C) * T + t];
    y[i] = a * (1.f / (1.f + __expf(-fminf(fmaxf(b, -30.f), 30.f))));
  }
}
__global__ void transpose_kernel(const float *x, float *y, int R, int C) {
  __shared__ float tile[32][33];
  const int bx = blockIdx.x * 32, by = blockIdx.y * 32;
  const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;  // 256 threads: 32 x 8
  for (int k = ty; k < 32; k += 8) {
    const int r = by + k, c = bx + tx;
    if (r < R && c < C) tile[k][tx] = x[(size_t)r * C + c];
  }
  __syncthreads();
  for (int k = ty; k < 32; k += 8) {
    const int c = bx + k, r = by + tx;
    if (r < R && c < C) y[(size_t)c * R + r] = tile[tx][k];
  }
}
__global__ void slice_cols_kernel(const float *x, float *y, int rows, int C, int col0, int W) {
  const long n = (long)rows * W;
  for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (long)gridDim.x * blockDim.x) {
    const long r = i / W, j = i % W;
    y[i] = x[r * C + col0 + j];
  }
}
__global__ void set_cols_kernel(const float *src, float *dst, int rows, int C, int col0, int W) {
  const long n = (long)rows * W;
  for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (long)gridDim.x * blockDim.x) {
    const long r = i / W, j = i % W;
    dst[r * C + col0 + j] = src[i];
  }
}
__global__ void sub_reshape_kernel(const float *x, float *y, int C, int Tsub, int F) {
  const long CF = (long)C * F, n = (long)Tsub * CF;
  for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (long)gridDim.x * blockDim.x) {
    const long ho = i / CF, rem = i % CF, c = rem / F, wo = rem % F;
    y[i] = x[c * ((long)Tsub * F) + ho * F + wo];
  }
}
__global__ void row_bias_act_kernel(const float *x, const float *b, float *y, int rows, int cols, int act) {
  const long n = (long)rows * cols;
  for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (long)gridDim.x * blockDim.x) y[i] = act_apply(x[i] + b[i / cols], act);
}

// ── convolutions (direct; the encoder's fused path has its own kernels) ────
__global__ void conv1d_kernel(const float *x, const float *w, const float *bias, float *y, int cout, int cin, int L, int Lout, int K, int stride,
                              int padl, int dil, int groups, int act) {
  const long n = (long)cout * Lout;
  for (long idx = (long)blockIdx.x * blockDim.x + threadIdx.x; idx < n; idx += (long)gridDim.x * blockDim.x) {
    const int co = (int)(idx / Lout), lo = (int)(idx % Lout);
    const int cinG = cin / groups, coutG = cout / groups, g = co / coutG;
    float acc = 0.f;
    for (int ci = 0; ci < cinG; ci++) {
      const float *xr = x + (size_t)(g * cinG + ci) * L;
      const float *wr = w + ((size_t)co * cinG + ci) * K;
      for (int k = 0; k < K; k++) {
        const int li = lo * stride + k * dil - padl;
        if (li >= 0 && li < L) acc += xr[li] * wr[k];
      }
    }
    if (bias) acc += bias[co];
    y[idx] = act_apply(acc, act);
  }
}
// f32 -> f16 (round to nearest even), 4 values per thread (n % 4 == 0)
__global__ void round_f16_kernel(const float *__restrict__ x, _Float16 *__restrict__ y, long n) {
  for (long i = ((long)blockIdx.x * blockDim.x + threadIdx.x) * 4; i < n; i += (long)gridDim.x * blockDim.x * 4) {
    const float4 v = *reinterpret_cast<const float4 *>(x + i);
    *reinterpret_cast<h4 *>(y + i) = h4{(_Float16)v.x, (_Float16)v.y, (_Float16)v.z, (_Float16)v.w};
  }
}
// y[r][c] = act(y[r][c] + bias[r]) over rows of `cols` values (bias may be null)
__global__ void chan_bias_act_kernel(float *__restrict__ y, const float *__restrict__ bias, int cols, long n, int act) {
  for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (long)gridDim.x * blockDim.x) {
    float v = y[i];
    if (bias) v += bias[i / cols];
    y[i] = act_apply(v, act);
  }
}
__global__ void conv2d_kernel(const float *x, const float *w, const float *bias, float *y, int cout, int cin, int H, int Wd, int Ho, int Wo, int kh,
                              int kw, int sh, int sw, int pt, int pl, int groups, int act) {
  const long n = (long)cout * Ho * Wo;
  for (long idx = (long)blockIdx.x * blockDim.x + threadIdx.x; idx < n; idx += (long)gridDim.x * blockDim.x) {
    const int co = (int)(idx / ((long)Ho * Wo));
    const int rem = (int)(idx % ((long)Ho * Wo)), ho = rem / Wo, wo = rem % Wo;
    const int cinG = cin / groups, coutG = cout / groups, g = co / coutG;
    float acc = bias ? bias[co] : 0.f;
    for (int ci = 0; ci < cinG; ci++) {
      const float *xc = x + (size_t)(g * cinG + ci) * H * Wd;
      const float *wc = w + ((size_t)co * cinG + ci) * kh * kw;
      for (int a = 0; a < kh; a++) {
        const int hi = ho * sh + a - pt;
        if (hi < 0 || hi >= H) continue;
        for (int b = 0; b < kw; b++) {
          const int wi = wo * sw + b - pl;
          if (wi < 0 || wi >= Wd) continue;
          acc += xc[(size_t)hi * Wd + wi] * wc[a * kw + b];
        }
      }
    }
    y[idx] = act_apply(acc, act);
  }
}

// ── attention building blocks (fp32; the fused kernel is attention.hip) ────
__global__ void bmm_qk_kernel(const float *q, const float *b, const float *qb, float *out, int T, int Tb, int H, int HD, int W, int bShared) {
  const long n = (long)W * H * T * Tb;
  const int stride = H * HD;
  for (long idx = (long)blockIdx.x * blockDim.x + threadIdx.x; idx < n; idx += (long)gridDim.x * blockDim.x) {
    const int j = (int)(idx % Tb);
    const long r = idx / Tb;
    const int i = (int)(r % T), wh = (int)(r / T), h = wh % H, w = wh / H;
    const float *qr = q + ((size_t)w * T + i) * stride + h * HD;
    const float *br = b + (size_t)(bShared ? j : w * Tb + j) * stride + h * HD;
    float acc = 0.f;
    for (int d = 0; d < HD; d++) acc += (qr[d] + (qb ? qb[h * HD + d] : 0.f)) * br[d];
    out[idx] = acc;
  }
}
__global__ void bmm_pv_kernel(const float *p, const float *v, float *out, int Tq, int Tk, int H, int HD, int W) {
  const int stride = H * HD;
  const long n = (long)W * Tq * stride;
  for (long idx = (long)blockIdx.x * blockDim.x + threadIdx.x; idx < n; idx += (long)gridDim.x * blockDim.x) {
    const int c = (int)(idx % stride);
    const long r = idx / stride;
    const int i = (int)(r % Tq), w = (int)(r / Tq), h = c / HD;
    const float *pr = p + (((size_t)w * H + h) * Tq + i) * Tk;
    float acc = 0.f;
    for (int j = 0; j < Tk; j++) acc += pr[j] * v[((size_t)w * Tk + j) * stride + c];
    out[idx] = acc;
  }
}
// NeMo rel_shift closed form (attention.js:283-286): y[i,j] = xp[f], f = t + i(2t-1) + j
// over the left-padded [t, 2t] view (column 0 = 0).
__global__ void relshift_kernel(const float *x, float *y, int t, int H) {
  const long n = (long)H * t * t;
  const long p = 2L * t - 1, twoT = 2L * t;
  for (long idx = (long)blockIdx.x * blockDim.x + threadIdx.x; idx < n; idx += (long)gridDim.x * blockDim.x) {
    const long j = idx % t, hi = idx / t, i = hi % t, h = hi / t;
    const long f = t + i * p + j, col = f % twoT;
    y[idx] = col == 0 ? 0.f : x[(h * t + f / twoT) * p + (col - 1)];
  }
}

// Streaming rel_shift + chunked-causal mask (compute.js:689-703,
// wasm-context.js:509-524): n new queries at absolute positions q = subT + i
// against Lk keys at k = subT - Lc + j; x holds each query's bd term over a
// truncated positional table whose column pi is relative distance dMax - pi.
// y = x[row, clamp(dMax - (q - k), 0, P - 1)], or -1e4 when k lies outside
// the query's chunk window [cs - left, cs + C - 1 + right], cs = C * (q / C).
__global__ void relshift_stream_kernel(const float *x, float *y, long total, int n, int Lk, int P, int dMax, int Lc, int subT, int C, int left,
                                       int right) {
  for (long idx = (long)blockIdx.x * blockDim.x + threadIdx.x; idx < total; idx += (long)gridDim.x * blockDim.x) {
    const long r = idx / Lk;
    const int j = (int)(idx - r * Lk), i = (int)(r % n);
    const int q = subT + i, cs = C * (q / C), k = subT - Lc + j;
    float v = -10000.0f;
    if (k >= cs - left && k <= cs + C - 1 + right) {
      const int d = min(P - 1, max(0, dMax - (q - k)));
      v = x[r * P + d];
    }
    y[idx] = v;
  }
}

// ── quantised-weight helpers ──────────────────────────────────────────────
__global__ void repack_i8_kernel(const int8_t *src, int8_t *dst, int K, int N) {  // [K][N] -> [N][K]
  __shared__ int8_t tile[64][65];
  const int bk = blockIdx.y * 64, bn = blockIdx.x * 64;
  for (int e = threadIdx.x; e < 64 * 64; e += blockDim.x) {
    const int r = e / 64, c = e % 64;
    if (bk + r < K && bn + c < N) tile[r][c] = src[(size_t)(bk + r) * N + bn + c];
  }
  __syncthreads();
  for (int e = threadIdx.x; e < 64 * 64; e += blockDim.x) {
    const int r = e / 64, c = e % 64;  // r: n, c: k
    if (bn + r < N && bk + c < K) dst[(size_t)(bn + r) * K + bk + c] = tile[c][r];
  }
}
__global__ void dequant_i8_kernel(const int8_t *q, const float *s, float *w, int K, int N) {
  const long n = (long)K * N;
  for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (long)gridDim.x * blockDim.x) w[i] = (float)q[i] * s[i % N];
}
__global__ void dequant_i4_kernel(const uint8_t *bq, const _Float16 *s, float *w, int K, int N) {
  const long n = (long)K * N;
  const int nblk = (K + 31) / 32;
  for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (long)gridDim.x * blockDim.x) {
    const int k = (int)(i / N), c = (int)(i % N);
    const int b = k >> 5, t = k & 31;
    const uint8_t byte = bq[((size_t)c * nblk + b) * 16 + (t >> 1)];
    const int nib = (t & 1) ? (byte >> 4) : (byte & 0xf);
    w[i] = (float)(nib - 8) * (float)s[(size_t)c * nblk + b];
  }
}

// f16 tensor -> f32 row-major [rows, cols]: row-major (allocF16) or K-major
// (uploadF16: element (r, c) at c * rows + r).
__global__ void f16_to_f32_rows_kernel(const _Float16 *src, float *dst, int rows, int cols, int kmajor) {
  const long n = (long)rows * cols;
  for (long i = (long)blockIdx.x * 256 + threadIdx.x; i < n; i += (long)gridDim.x * 256) {
    const int r = (int)(i / cols), c = (int)(i % cols);
    dst[i] = (float)src[kmajor ? (size_t)c * rows + r : (size_t)i];
  }
}

// ONNX MatMulNBits weights (bits 4, block 32; gemm.js:893-919) -> f32 [K, N]:
// (q - zp) * s exactly as the reference kernel dequantises in f32.
__global__ void nbits_dequant_f32_kernel(const uint8_t *bq, const float *scales, const uint8_t *zp, int zpb, int K, int N, float *w) {
  const long n_el = (long)K * N;
  const int nblk = (K + 31) / 32;
  for (long i = (long)blockIdx.x * 256 + threadIdx.x; i < n_el; i += (long)gridDim.x * 256) {
    const int k = (int)(i / N), n = (int)(i % N), b = k >> 5, t = k & 31;
    const uint8_t byte = bq[((size_t)n * nblk + b) * 16 + (t >> 1)];
    const float q = (float)((t & 1) ? (byte >> 4) : (byte & 0xf));
    const uint8_t zb = zp[(size_t)n * zpb + (b >> 1)];
    const float z = (float)((b & 1) ? (zb >> 4) : (zb & 0xf));
    w[i] = (q - z) * scales[(size_t)n * nblk + b];
  }
}

static inline unsigned gs(long n) {
  long b = (n + 255) / 256;
  return (unsigned)(b < 1 ? 1 : (b > 65535 * 4 ? 65535 * 4 : b));
}

}  // namespace fa

using namespace fa;

// ── C ABI ──────────────────────────────────────────────────────────────────
#define F32(r) reinterpret_cast<float *>((r)->ptr)
#define CF32(r) reinterpret_cast<const float *>((r) ? (r)->ptr : nullptr)

static int need_f32(fa_ctx *ctx, TensorRec *r, const char *what) {
  if (r && r->kind != S_F32) return set_err(ctx, FA_E_INVALID, "%s: expected an f32 tensor", what);
  return FA_OK;
}

// An f32 view of an operand for the ops whose kernels read f32: f16 tensors
// (uploadF16 / allocF16, the reference's f16-storage tensors) are widened
// into a pooled temporary (*tmp, freed by the caller after its launch).
static int as_f32(fa_ctx *ctx, fa_tensor t, fa_tensor *use, fa_tensor *tmp, const char *what) {
  TensorRec *r;
  *tmp = 0;
  *use = t;
  FA_TRY(need(ctx, t, &r, what));
  if (r->kind == S_F32) return FA_OK;
  if (r->kind != S_F16KM && r->kind != S_F16RM) return set_err(ctx, FA_E_INVALID, "%s: expected an f32 or f16 tensor", what);
  TensorRec *ro;
  FA_TRY(new_tensor(ctx, r->rows, r->cols, S_F32, (size_t)r->rows * r->cols * 4, tmp, &ro));
  r = get(ctx, t);
  const long n = (long)r->rows * r->cols;
  if (n) hipLaunchKernelGGL(f16_to_f32_rows_kernel, dim3(gs(n)), dim3(256), 0, ctx->stream, (const _Float16 *)r->ptr, F32(ro), r->rows, r->cols,
                           r->kind == S_F16KM ? 1 : 0);
  FA_TRY(check_launch(ctx, what));
  *use = *tmp;
  return FA_OK;
}

extern "C" {

static int matmul_impl(fa_ctx *ctx, fa_tensor a, fa_tensor b, fa_tensor bias, int act, fa_tensor add, fa_tensor *out);
int fa_matmul(fa_ctx *ctx, fa_tensor a, fa_tensor b, fa_tensor bias, int act, fa_tensor add, fa_tensor *out) {
  TensorRec *ra;
  FA_TRY(need(ctx, a, &ra, "matmul"));
  if (ra->kind != S_F16KM) return matmul_impl(ctx, a, b, bias, act, add, out);
  // A uploaded as an f16 weight (matmulF16 with f16 a, compute.d.ts:164):
  // widened to f32 rows, then the route of its B
  fa_tensor a32, tmp;
  FA_TRY(as_f32(ctx, a, &a32, &tmp, "matmul A"));
  const int st = matmul_impl(ctx, a32, b, bias, act, add, out);
  (void)fa_free_tensor(ctx, tmp);
  return st;
}

static int matmul_impl(fa_ctx *ctx, fa_tensor a, fa_tensor b, fa_tensor bias, int act, fa_tensor add, fa_tensor *out) {
  TensorRec *ra, *rb, *rbias, *radd;
  FA_TRY(need(ctx, a, &ra, "matmul"));
  FA_TRY(need(ctx, b, &rb, "matmul"));
  FA_TRY(opt(ctx, bias, &rbias, "matmul bias"));
  FA_TRY(opt(ctx, add, &radd, "matmul add"));
  if (ra->kind != S_F32 && ra->kind != S_F16RM) return set_err(ctx, FA_E_INVALID, "matmul: A must be an f32 or row-major f16 tensor");
  const int M = ra->rows, K = ra->cols, N = rb->cols;
  if (rb->rows != K) return set_err(ctx, FA_E_INVALID, "matmul: A [%d,%d] @ B [%d,%d]", M, K, rb->rows, rb->cols);
  if (rbias && rbias->rows * rbias->cols != N) return set_err(ctx, FA_E_INVALID, "matmul: bias has %d elements, N=%d", rbias->rows * rbias->cols, N);
  if (radd && (radd->rows != M || radd->cols != N)) return set_err(ctx, FA_E_INVALID, "matmul: add [%d,%d] != [%d,%d]", radd->rows, radd->cols, M, N);
  if (act < 0 || act > 5) return set_err(ctx, FA_E_INVALID, "matmul: act code %d", act);
  fa_tensor o;
  TensorRec *ro;
  FA_TRY(new_tensor(ctx, M, N, S_F32, (size_t)M * N * 4, &o, &ro));
  TensorGuard og(ctx, o);  // released unless the op completes
  ra = get(ctx, a); rb = get(ctx, b); rbias = bias ? get(ctx, bias) : nullptr; radd = add ? get(ctx, add) : nullptr;  // recs may move
  if (ra->kind == S_F16RM && (rb->kind != S_F16KM || K % 64)) return set_err(ctx, FA_E_UNSUPPORTED, "matmul: f16 A needs an f16 B and K %% 64 == 0");
  if (rb->kind == S_F16KM) {
    if (K % 64 == 0) {
      // f32 A on the f16 route is rounded to f16 (compute.js:413-416): for
      // more than a few rows it is rounded once into a scratch tensor, so the
      // product runs on the direct-to-LDS kernels (same values and K order as
      // the register-staged kernel, which rounds inside its loads)
      fa_tensor a16 = 0;
      TensorRec *r16 = nullptr;
      if (ra->kind == S_F32 && M >= 256) {
        FA_TRY(new_tensor(ctx, M, K, S_F16RM, (size_t)M * K * 2, &a16, &r16));
        ra = get(ctx, a); rb = get(ctx, b); rbias = bias ? get(ctx, bias) : nullptr; radd = add ? get(ctx, add) : nullptr; ro = get(ctx, og.t);
        ProfScope ps(ctx, "matmul_a16");
        const long n = (long)M * K;
        FA_LAUNCH(ps, round_f16_kernel, dim3((unsigned)std::min<long>(cdiv(n / 4, 256), 4096)), dim3(256), 0, ctx->stream, F32(ra),
                  (_Float16 *)r16->ptr, n);
        FA_TRY(check_launch(ctx, "matmul_a16"));
      }
      TensorGuard g16(ctx, a16);  // pool-ordered: released after the product is queued
      GemmArgs p;
      p.A = r16 ? r16->ptr : ra->ptr; p.lda = K; p.akind = (r16 || ra->kind == S_F16RM) ? A_F16 : A_F32;
      p.B = rb->ptr; p.bkind = B_F16;
      p.C = ro->ptr; p.ldc = N;
      p.bias = CF32(rbias); p.add = CF32(radd); p.ldadd = N; p.act = act;
      p.M = M; p.N = N; p.K = K;
      FA_TRY(gemm_mfma(ctx, p, "matmul_f16"));
    } else {
      FA_TRY(gemm_naive_f16(ctx, F32(ra), rb->ptr, F32(ro), CF32(rbias), CF32(radd), M, N, K, act, "matmul_f16_naive"));
    }
  } else if (rb->kind == S_F32) {
    FA_TRY(gemm_f32(ctx, F32(ra), F32(rb), F32(ro), CF32(rbias), CF32(radd), M, N, K, act, "matmul_f32"));
  } else {
    return set_err(ctx, FA_E_INVALID, "matmul: B must be an f32 or f16 tensor");
  }
  *out = og.release();
  return FA_OK;
}

int fa_matmul_pair(fa_ctx *ctx, fa_tensor a_hi, fa_tensor a_lo, fa_tensor b, fa_tensor bias, fa_tensor add, fa_tensor *out) {
  TensorRec *rh, *rl, *rb, *rbias, *radd;
  FA_TRY(need(ctx, a_hi, &rh, "matmulPair"));
  FA_TRY(need(ctx, a_lo, &rl, "matmulPair lo"));
  FA_TRY(need(ctx, b, &rb, "matmulPair"));
  FA_TRY(opt(ctx, bias, &rbias, "matmulPair bias"));
  FA_TRY(opt(ctx, add, &radd, "matmulPair add"));
  if (rh->kind != S_F16RM || rl->kind != S_F16RM || rh->rows != rl->rows || rh->cols != rl->cols)
    return set_err(ctx, FA_E_INVALID, "matmulPair: A hi and lo must be row-major f16 tensors of one shape");
  if (rb->kind != S_F16KM) return set_err(ctx, FA_E_INVALID, "matmulPair: B must be an f16 weight tensor (uploadF16)");
  const int M = rh->rows, K = rh->cols, N = rb->cols;
  if (rb->rows != K) return set_err(ctx, FA_E_INVALID, "matmulPair: A [%d,%d] @ B [%d,%d]", M, K, rb->rows, rb->cols);
  if (rbias && rbias->rows * rbias->cols != N) return set_err(ctx, FA_E_INVALID, "matmulPair: bias has %d elements, N=%d", rbias->rows * rbias->cols, N);
  if (radd && (radd->rows != M || radd->cols != N)) return set_err(ctx, FA_E_INVALID, "matmulPair: add [%d,%d] != [%d,%d]", radd->rows, radd->cols, M, N);
  fa_tensor o;
  TensorRec *ro;
  FA_TRY(new_tensor(ctx, M, N, S_F32, (size_t)M * N * 4, &o, &ro));
  TensorGuard og(ctx, o);  // released unless the op completes
  rh = get(ctx, a_hi); rl = get(ctx, a_lo); rb = get(ctx, b); rbias = bias ? get(ctx, bias) : nullptr; radd = add ? get(ctx, add) : nullptr;
  GemmArgs p;
  p.A = rh->ptr; p.Alo = rl->ptr; p.lda = K; p.akind = A_F16;
  p.B = rb->ptr; p.bkind = B_F16;
  p.C = ro->ptr; p.ldc = N;
  p.bias = CF32(rbias); p.add = CF32(radd); p.ldadd = N;
  p.M = M; p.N = N; p.K = K;
  FA_TRY(gemm_mfma(ctx, p, "matmul_pair"));
  *out = og.release();
  return FA_OK;
}

int fa_matmul_int8(fa_ctx *ctx, fa_tensor a, fa_tensor wq, fa_tensor scale, int N, int K, fa_tensor bias, int act, fa_tensor *out) {
  TensorRec *ra, *rw, *rs, *rbias;
  FA_TRY(need(ctx, a, &ra, "matmulInt8"));
  FA_TRY(need(ctx, wq, &rw, "matmulInt8 wq"));
  FA_TRY(need(ctx, scale, &rs, "matmulInt8 scale"));
  FA_TRY(opt(ctx, bias, &rbias, "matmulInt8 bias"));
  FA_TRY(need_f32(ctx, ra, "matmulInt8 A"));
  if (ra->cols != K) return set_err(ctx, FA_E_INVALID, "matmulInt8: A has %d cols, K=%d", ra->cols, K);
  if (rw->kind != S_BYTES || rw->bytes < (size_t)K * N) return set_err(ctx, FA_E_INVALID, "matmulInt8: wq must hold K*N int8 bytes");
  const int M = ra->rows;
  // Repack once into the K-major layout the GEMM streams (cached on the tensor).
  if (!rw->aux) {
    void *p = dev_alloc(ctx, (size_t)K * N);
    if (!p) return FA_E_OOM;
    rw = get(ctx, wq);
    rw->aux = p;
    rw->aux_bytes = (size_t)K * N;
    ProfScope ps(ctx, "repack_i8");
    FA_LAUNCH(ps, repack_i8_kernel, dim3(cdiv(N, 64), cdiv(K, 64)), dim3(256), 0, ctx->stream, (const int8_t *)rw->ptr, (int8_t *)p, K, N);
    FA_TRY(check_launch(ctx, "repack_i8"));
  }
  fa_tensor o;
  TensorRec *ro;
  FA_TRY(new_tensor(ctx, M, N, S_F32, (size_t)M * N * 4, &o, &ro));
  TensorGuard og(ctx, o);  // released unless the op completes
  ra = get(ctx, a); rw = get(ctx, wq); rs = get(ctx, scale); rbias = bias ? get(ctx, bias) : nullptr;
  if (M <= 64 || K % 64 != 0) {
    FA_TRY(gemv_quant_launch(ctx, F32(ra), rw->aux, F32(rs), 1, M, N, K, F32(ro), CF32(rbias), act, "matmulInt8_gemv"));
  } else {
    GemmArgs p;
    p.A = ra->ptr; p.lda = K; p.akind = A_F32;
    p.B = rw->aux; p.bkind = B_I8;
    p.colscale = F32(rs);
    p.C = ro->ptr; p.ldc = N;
    p.bias = CF32(rbias); p.act = act;
    p.M = M; p.N = N; p.K = K;
    FA_TRY(gemm_mfma(ctx, p, "matmulInt8"));
  }
  *out = og.release();
  return FA_OK;
}

int fa_matmul_nbits(fa_ctx *ctx, fa_tensor a, fa_tensor bq, fa_tensor scales, fa_tensor zp, int N, int block_size, fa_tensor *out) {
  TensorRec *ra, *rq, *rs, *rz;
  FA_TRY(need(ctx, a, &ra, "matmulNBits"));
  FA_TRY(need(ctx, bq, &rq, "matmulNBits bq"));
  FA_TRY(need(ctx, scales, &rs, "matmulNBits scales"));
  FA_TRY(need(ctx, zp, &rz, "matmulNBits zp"));
  FA_TRY(need_f32(ctx, ra, "matmulNBits A"));
  if (block_size != 32) return set_err(ctx, FA_E_UNSUPPORTED, "matmulNBits: block_size %d (32 supported)", block_size);
  const int M = ra->rows, K = ra->cols;
  const int nblk = (K + 31) / 32, zpb = (nblk + 1) / 2;
  if (rq->bytes < (size_t)N * nblk * 16) return set_err(ctx, FA_E_INVALID, "matmulNBits: bq too small");
  fa_tensor o;
  TensorRec *ro;
  FA_TRY(new_tensor(ctx, M, N, S_F32, (size_t)M * N * 4, &o, &ro));
  TensorGuard og(ctx, o);  // released unless the op completes
  if ((long)rs->rows * rs->cols < (long)N * nblk || rz->bytes < (size_t)N * zpb) return set_err(ctx, FA_E_INVALID, "matmulNBits: scales / zero points too small");
  // The reference's kernel dequantises in f32 (arbitrary f32 block scales and
  // zero points): the weights are expanded to f32 [K, N] once per call and
  // multiplied on the fp32 MFMA route, so results carry f32 accuracy.  (The
  // encoder's own int4 format runs fused in its f16 GEMMs instead.)
  fa_tensor tw;
  TensorRec *rw;
  FA_TRY(new_tensor(ctx, K, N, S_F32, (size_t)K * N * 4, &tw, &rw));
  TensorGuard tg(ctx, tw);  // the f32 weights live for this call only
  ra = get(ctx, a); rq = get(ctx, bq); rs = get(ctx, scales); rz = get(ctx, zp); ro = get(ctx, o);
  {
    ProfScope ps(ctx, "matmulNBits_dequant");
    FA_LAUNCH(ps, nbits_dequant_f32_kernel, dim3(gs((long)K * N)), dim3(256), 0, ctx->stream, (const uint8_t *)rq->ptr, F32(rs), (const uint8_t *)rz->ptr,
              zpb, K, N, F32(rw));
    FA_TRY(check_launch(ctx, "matmulNBits_dequant"));
  }
  FA_TRY(gemm_f32(ctx, F32(ra), F32(rw), F32(ro), nullptr, nullptr, M, N, K, 0, "matmulNBits"));
  *out = og.release();
  return FA_OK;
}

int fa_layernorm(fa_ctx *ctx, fa_tensor x, fa_tensor gamma, fa_tensor beta, float eps, fa_tensor *out) {
  TensorRec *rx, *rg, *rb;
  FA_TRY(need(ctx, x, &rx, "layernorm"));
  FA_TRY(need(ctx, gamma, &rg, "layernorm gamma"));
  FA_TRY(need(ctx, beta, &rb, "layernorm beta"));
  FA_TRY(need_f32(ctx, rx, "layernorm x"));
  const int R = rx->rows, Cc = rx->cols;
  if (rg->rows * rg->cols < Cc || rb->rows * rb->cols < Cc) return set_err(ctx, FA_E_INVALID, "layernorm: gamma/beta shorter than %d", Cc);
  fa_tensor o;
  TensorRec *ro;
  FA_TRY(new_tensor(ctx, R, Cc, S_F32, (size_t)R * Cc * 4, &o, &ro));
  TensorGuard og(ctx, o);  // released unless the op completes
  rx = get(ctx, x); rg = get(ctx, gamma); rb = get(ctx, beta);
  FA_TRY(layernorm_launch(ctx, F32(rx), F32(rg), F32(rb), ro->ptr, 0, R, Cc, Cc, Cc, eps, "layernorm"));
  *out = og.release();
  return FA_OK;
}

int fa_softmax(fa_ctx *ctx, fa_tensor x, fa_tensor *out) {
  TensorRec *rx;
  FA_TRY(need(ctx, x, &rx, "softmax"));
  FA_TRY(need_f32(ctx, rx, "softmax"));
  const int R = rx->rows, Cc = rx->cols;
  fa_tensor o;
  TensorRec *ro;
  FA_TRY(new_tensor(ctx, R, Cc, S_F32, (size_t)R * Cc * 4, &o, &ro));
  TensorGuard og(ctx, o);  // released unless the op completes
  rx = get(ctx, x);
  ProfScope ps(ctx, "softmax");
  if (R) FA_LAUNCH(ps, softmax_kernel, dim3(cdiv(R, 4)), dim3(256), 0, ctx->stream, F32(rx), F32(ro), R, Cc);
  FA_TRY(check_launch(ctx, "softmax"));
  *out = og.release();
  return FA_OK;
}

static int unary(fa_ctx *ctx, fa_tensor x, int kind, float s, fa_tensor *out, const char *name) {
  TensorRec *rx;
  FA_TRY(need(ctx, x, &rx, name));
  FA_TRY(need_f32(ctx, rx, name));
  fa_tensor o;
  TensorRec *ro;
  const long n = (long)rx->rows * rx->cols;
  FA_TRY(new_tensor(ctx, rx->rows, rx->cols, S_F32, (size_t)n * 4, &o, &ro));
  TensorGuard og(ctx, o);  // released unless the op completes
  rx = get(ctx, x);
  ProfScope ps(ctx, name);
  if (n) FA_LAUNCH(ps, unary_kernel, dim3(gs(n)), dim3(256), 0, ctx->stream, F32(rx), F32(ro), n, kind, s);
  FA_TRY(check_launch(ctx, name));
  *out = og.release();
  return FA_OK;
}
int fa_scale(fa_ctx *ctx, fa_tensor x, float s, fa_tensor *out) { return unary(ctx, x, 0, s, out, "scale"); }
int fa_silu(fa_ctx *ctx, fa_tensor x, fa_tensor *out) { return unary(ctx, x, 1, 0.f, out, "silu"); }
int fa_relu(fa_ctx *ctx, fa_tensor x, fa_tensor *out) { return unary(ctx, x, 2, 0.f, out, "relu"); }

int fa_ewise(fa_ctx *ctx, fa_tensor a, fa_tensor b, int op, fa_tensor *out) {
  TensorRec *ra, *rb;
  FA_TRY(need(ctx, a, &ra, "ewise"));
  FA_TRY(need(ctx, b, &rb, "ewise"));
  FA_TRY(need_f32(ctx, ra, "ewise a"));
  FA_TRY(need_f32(ctx, rb, "ewise b"));
  const int bcast = rb->rows == 1;
  if (!bcast && (rb->rows != ra->rows || rb->cols != ra->cols)) return set_err(ctx, FA_E_INVALID, "ewise: shapes [%d,%d] vs [%d,%d]", ra->rows, ra->cols, rb->rows, rb->cols);
  if (bcast && rb->cols != ra->cols) return set_err(ctx, FA_E_INVALID, "ewise: broadcast row has %d cols, need %d", rb->cols, ra->cols);
  const long n = (long)ra->rows * ra->cols;
  fa_tensor o;
  TensorRec *ro;
  FA_TRY(new_tensor(ctx, ra->rows, ra->cols, S_F32, (size_t)n * 4, &o, &ro));
  TensorGuard og(ctx, o);  // released unless the op completes
  ra = get(ctx, a); rb = get(ctx, b);
  ProfScope ps(ctx, "ewise");
  if (n) FA_LAUNCH(ps, ewise_kernel, dim3(gs(n)), dim3(256), 0, ctx->stream, F32(ra), F32(rb), F32(ro), n, ra->cols, bcast, op ? 1 : 0);
  FA_TRY(check_launch(ctx, "ewise"));
  *out = og.release();
  return FA_OK;
}

int fa_glu(fa_ctx *ctx, fa_tensor x, fa_tensor *out) {
  TensorRec *rx;
  FA_TRY(need(ctx, x, &rx, "glu"));
  FA_TRY(need_f32(ctx, rx, "glu"));
  if (rx->rows % 2) return set_err(ctx, FA_E_INVALID, "glu: odd channel count %d", rx->rows);
  const int C = rx->rows / 2, T = rx->cols;
  fa_tensor o;
  TensorRec *ro;
  FA_TRY(new_tensor(ctx, C, T, S_F32, (size_t)C * T * 4, &o, &ro));
  TensorGuard og(ctx, o);  // released unless the op completes
  rx = get(ctx, x);
  ProfScope ps(ctx, "glu");
  if ((long)C * T) FA_LAUNCH(ps, glu_kernel, dim3(gs((long)C * T)), dim3(256), 0, ctx->stream, F32(rx), F32(ro), C, T);
  FA_TRY(check_launch(ctx, "glu"));
  *out = og.release();
  return FA_OK;
}

int fa_transpose(fa_ctx *ctx, fa_tensor x, fa_tensor *out) {
  TensorRec *rx;
  FA_TRY(need(ctx, x, &rx, "transpose"));
  FA_TRY(need_f32(ctx, rx, "transpose"));
  const int R = rx->rows, Cc = rx->cols;
  fa_tensor o;
  TensorRec *ro;
  FA_TRY(new_tensor(ctx, Cc, R, S_F32, (size_t)R * Cc * 4, &o, &ro));
  TensorGuard og(ctx, o);  // released unless the op completes
  rx = get(ctx, x);
  ProfScope ps(ctx, "transpose");
  if ((long)R * Cc) FA_LAUNCH(ps, transpose_kernel, dim3(cdiv(Cc, 32), cdiv(R, 32)), dim3(256), 0, ctx->stream, F32(rx), F32(ro), R, Cc);
  FA_TRY(check_launch(ctx, "transpose"));
  *out = og.release();
  return FA_OK;
}

int fa_slice_cols(fa_ctx *ctx, fa_tensor x, int col0, int width, fa_tensor *out) {
  TensorRec *rx;
  FA_TRY(need(ctx, x, &rx, "sliceCols"));
  FA_TRY(need_f32(ctx, rx, "sliceCols"));
  if (col0 < 0 || width < 0 || col0 + width > rx->cols) return set_err(ctx, FA_E_INVALID, "sliceCols: [%d,%d) of %d cols", col0, col0 + width, rx->cols);
  fa_tensor o;
  TensorRec *ro;
  FA_TRY(new_tensor(ctx, rx->rows, width, S_F32, (size_t)rx->rows * width * 4, &o, &ro));
  TensorGuard og(ctx, o);  // released unless the op completes
  rx = get(ctx, x);
  const long n = (long)rx->rows * width;
  ProfScope ps(ctx, "sliceCols");
  if (n) FA_LAUNCH(ps, slice_cols_kernel, dim3(gs(n)), dim3(256), 0, ctx->stream, F32(rx), F32(ro), rx->rows, rx->cols, col0, width);
  FA_TRY(check_launch(ctx, "sliceCols"));
  *out = og.release();
  return FA_OK;
}

int fa_set_cols(fa_ctx *ctx, fa_tensor dst, fa_tensor src, int col0) {
  TensorRec *rd, *rs;
  FA_TRY(need(ctx, dst, &rd, "setCols"));
  FA_TRY(need(ctx, src, &rs, "setCols"));
  FA_TRY(need_f32(ctx, rd, "setCols"));
  FA_TRY(need_f32(ctx, rs, "setCols"));
  if (rs->rows != rd->rows || col0 < 0 || col0 + rs->cols > rd->cols) return set_err(ctx, FA_E_INVALID, "setCols: src [%d,%d] at col %d of [%d,%d]", rs->rows, rs->cols, col0, rd->rows, rd->cols);
  const long n = (long)rs->rows * rs->cols;
  ProfScope ps(ctx, "setCols");
  if (n) FA_LAUNCH(ps, set_cols_kernel, dim3(gs(n)), dim3(256), 0, ctx->stream, F32(rs), F32(rd), rs->rows, rd->cols, col0, rs->cols);
  return check_launch(ctx, "setCols");
}

int fa_slice_rows(fa_ctx *ctx, fa_tensor x, int row0, int count, fa_tensor *out) {
  TensorRec *rx;
  FA_TRY(need(ctx, x, &rx, "sliceRows"));
  FA_TRY(need_f32(ctx, rx, "sliceRows"));
  if (row0 < 0 || count < 0 || row0 + count > rx->rows) return set_err(ctx, FA_E_INVALID, "sliceRows: [%d,%d) of %d rows", row0, row0 + count, rx->rows);
  fa_tensor o;
  TensorRec *ro;
  FA_TRY(new_tensor(ctx, count, rx->cols, S_F32, (size_t)count * rx->cols * 4, &o, &ro));
  TensorGuard og(ctx, o);  // released unless the op completes
  rx = get(ctx, x);
  if (count) FA_HIP(ctx, hipMemcpyAsync(ro->ptr, F32(rx) + (size_t)row0 * rx->cols, (size_t)count * rx->cols * 4, hipMemcpyDeviceToDevice, ctx->stream));
  *out = og.release();
  return FA_OK;
}

int fa_copy_rows(fa_ctx *ctx, fa_tensor dst, fa_tensor src, int row_offset) {
  TensorRec *rd, *rs;
  FA_TRY(need(ctx, dst, &rd, "copyRows"));
  FA_TRY(need(ctx, src, &rs, "copyRows"));
  FA_TRY(need_f32(ctx, rd, "copyRows dst"));
  FA_TRY(need_f32(ctx, rs, "copyRows src"));
  if (rs->cols != rd->cols || row_offset < 0 || row_offset + rs->rows > rd->rows) return set_err(ctx, FA_E_INVALID, "copyRows: out of range");
  const size_t nb = (size_t)rs->rows * rs->cols * 4;
  if (nb) FA_HIP(ctx, hipMemcpyAsync(F32(rd) + (size_t)row_offset * rd->cols, rs->ptr, nb, hipMemcpyDeviceToDevice, ctx->stream));
  return FA_OK;
}

int fa_concat_rows(fa_ctx *ctx, const fa_tensor *ts, int n, fa_tensor *out) {
  if (n <= 0) return set_err(ctx, FA_E_INVALID, "concatRows: no tensors");
  int rows = 0, cols = -1;
  for (int i = 0; i < n; i++) {
    TensorRec *r;
    FA_TRY(need(ctx, ts[i], &r, "concatRows"));
    FA_TRY(need_f32(ctx, r, "concatRows"));
    if (cols >= 0 && r->cols != cols) return set_err(ctx, FA_E_INVALID, "concatRows: column mismatch");
    cols = r->cols;
    rows += r->rows;
  }
  fa_tensor o;
  TensorRec *ro;
  FA_TRY(new_tensor(ctx, rows, cols, S_F32, (size_t)rows * cols * 4, &o, &ro));
  TensorGuard og(ctx, o);  // released unless the op completes
  size_t off = 0;
  for (int i = 0; i < n; i++) {
    TensorRec *r = get(ctx, ts[i]);
    ro = get(ctx, o);
    const size_t nb = (size_t)r->rows * r->cols * 4;
    if (nb) FA_HIP(ctx, hipMemcpyAsync((char *)ro->ptr + off, r->ptr, nb, hipMemcpyDeviceToDevice, ctx->stream));
    off += nb;
  }
  *out = og.release();
  return FA_OK;
}

int fa_sub_reshape(fa_ctx *ctx, fa_tensor x, int C, int Tsub, int F, fa_tensor *out) {
  TensorRec *rx;
  FA_TRY(need(ctx, x, &rx, "subReshape"));
  FA_TRY(need_f32(ctx, rx, "subReshape"));
  if ((long)rx->rows * rx->cols != (long)C * Tsub * F) return set_err(ctx, FA_E_INVALID, "subReshape: %d elements != C*Tsub*F", rx->rows * rx->cols);
  fa_tensor o;
  TensorRec *ro;
  FA_TRY(new_tensor(ctx, Tsub, C * F, S_F32, (size_t)Tsub * C * F * 4, &o, &ro));
  TensorGuard og(ctx, o);  // released unless the op completes
  rx = get(ctx, x);
  const long n = (long)Tsub * C * F;
  ProfScope ps(ctx, "subReshape");
  if (n) FA_LAUNCH(ps, sub_reshape_kernel, dim3(gs(n)), dim3(256), 0, ctx->stream, F32(rx), F32(ro), C, Tsub, F);
  FA_TRY(check_launch(ctx, "subReshape"));
  *out = og.release();
  return FA_OK;
}

int fa_row_bias_act(fa_ctx *ctx, fa_tensor x, fa_tensor bias, int act, fa_tensor *out) {
  TensorRec *rx, *rb;
  FA_TRY(need(ctx, x, &rx, "rowBiasAct"));
  FA_TRY(need(ctx, bias, &rb, "rowBiasAct bias"));
  if (rb->rows * rb->cols < rx->rows) return set_err(ctx, FA_E_INVALID, "rowBiasAct: bias shorter than rows");
  fa_tensor o;
  TensorRec *ro;
  const long n = (long)rx->rows * rx->cols;
  FA_TRY(new_tensor(ctx, rx->rows, rx->cols, S_F32, (size_t)n * 4, &o, &ro));
  TensorGuard og(ctx, o);  // released unless the op completes
  rx = get(ctx, x); rb = get(ctx, bias);
  ProfScope ps(ctx, "rowBiasAct");
  if (n) FA_LAUNCH(ps, row_bias_act_kernel, dim3(gs(n)), dim3(256), 0, ctx->stream, F32(rx), F32(rb), F32(ro), rx->rows, rx->cols, act);
  FA_TRY(check_launch(ctx, "rowBiasAct"));
  *out = og.release();
  return FA_OK;
}

static int conv1d_impl(fa_ctx *ctx, fa_tensor x, fa_tensor w, int cout, int k, fa_tensor bias, int stride, int pad_left, int pad_right, int dilation,
                       int groups, int act, fa_tensor *out);
int fa_conv1d(fa_ctx *ctx, fa_tensor x, fa_tensor w, int cout, int k, fa_tensor bias, int stride, int pad_left, int pad_right, int dilation,
              int groups, int act, fa_tensor *out) {
  // f16-storage operands (conv1dFastF16 with uploadF16 tensors) are widened to f32
  fa_tensor x32, w32, tx, tw;
  FA_TRY(as_f32(ctx, x, &x32, &tx, "conv1d x"));
  int st = as_f32(ctx, w, &w32, &tw, "conv1d w");
  if (!st) st = conv1d_impl(ctx, x32, w32, cout, k, bias, stride, pad_left, pad_right, dilation, groups, act, out);
  if (tx) (void)fa_free_tensor(ctx, tx);
  if (tw) (void)fa_free_tensor(ctx, tw);
  return st;
}

static int conv1d_impl(fa_ctx *ctx, fa_tensor x, fa_tensor w, int cout, int k, fa_tensor bias, int stride, int pad_left, int pad_right, int dilation,
                       int groups, int act, fa_tensor *out) {
  TensorRec *rx, *rw, *rb;
  FA_TRY(need(ctx, x, &rx, "conv1d"));
  FA_TRY(need(ctx, w, &rw, "conv1d w"));
  FA_TRY(opt(ctx, bias, &rb, "conv1d bias"));
  FA_TRY(need_f32(ctx, rx, "conv1d x"));
  FA_TRY(need_f32(ctx, rw, "conv1d w"));
  const int Cin = rx->rows, L = rx->cols;
  if (groups <= 0 || Cin % groups || cout % groups || stride <= 0 || dilation <= 0 || k <= 0)
    return set_err(ctx, FA_E_INVALID, "conv1d: bad geometry (cin %d, cout %d, groups %d)", Cin, cout, groups);
  if ((long)rw->rows * rw->cols < (long)cout * (Cin / groups) * k) return set_err(ctx, FA_E_INVALID, "conv1d: weight too small");
  const int Lout = (L + pad_left + pad_right - dilation * (k - 1) - 1) / stride + 1;
  if (Lout <= 0) return set_err(ctx, FA_E_INVALID, "conv1d: empty output");
  fa_tensor o;
  TensorRec *ro;
  FA_TRY(new_tensor(ctx, cout, Lout, S_F32, (size_t)cout * Lout * 4, &o, &ro));
  TensorGuard og(ctx, o);  // released unless the op completes
  rx = get(ctx, x); rw = get(ctx, w); rb = bias ? get(ctx, bias) : nullptr;
  ProfScope ps(ctx, "conv1d");
  FA_LAUNCH(ps, conv1d_kernel, dim3(gs((long)cout * Lout)), dim3(256), 0, ctx->stream, F32(rx), F32(rw), CF32(rb), F32(ro), cout, Cin, L, Lout,
                     k, stride, pad_left, dilation, groups, act);
  FA_TRY(check_launch(ctx, "conv1d"));
  *out = og.release();
  return FA_OK;
}

int fa_conv2d(fa_ctx *ctx, fa_tensor x, fa_tensor w, int cout, int cin, int h, int wd, int kh, int kw, fa_tensor bias, int sh, int sw, int pt,
              int pb, int pl, int pr, int groups, int act, fa_tensor *out) {
  TensorRec *rx, *rw, *rb;
  FA_TRY(need(ctx, x, &rx, "conv2d"));
  FA_TRY(need(ctx, w, &rw, "conv2d w"));
  FA_TRY(opt(ctx, bias, &rb, "conv2d bias"));
  FA_TRY(need_f32(ctx, rx, "conv2d x"));
  if ((long)rx->rows * rx->cols != (long)cin * h * wd) return set_err(ctx, FA_E_INVALID, "conv2d: x has %ld elements, cin*h*w=%ld", (long)rx->rows * rx->cols, (long)cin * h * wd);
  if (groups <= 0 || cin % groups || cout % groups) return set_err(ctx, FA_E_INVALID, "conv2d: bad groups");
  const int Ho = (h + pt + pb - kh) / sh + 1, Wo = (wd + pl + pr - kw) / sw + 1;
  if (Ho <= 0 || Wo <= 0) return set_err(ctx, FA_E_INVALID, "conv2d: empty output");
  fa_tensor o;
  TensorRec *ro;
  FA_TRY(new_tensor(ctx, cout, Ho * Wo, S_F32, (size_t)cout * Ho * Wo * 4, &o, &ro));
  TensorGuard og(ctx, o);  // released unless the op completes
  rx = get(ctx, x); rw = get(ctx, w); rb = bias ? get(ctx, bias) : nullptr;
  if (kh == 1 && kw == 1 && sh == 1 && sw == 1 && groups == 1 && pt == 0 && pb == 0 && pl == 0 && pr == 0 && cin % 16 == 0 && (Ho * Wo) % 4 == 0) {
    // a pointwise conv is the product W [cout, cin] x X [cin, H*W] (channel-major
    // x is row-major X): the f32 GEMM, then the per-channel bias and activation
    FA_TRY(gemm_f32(ctx, F32(rw), F32(rx), F32(ro), nullptr, nullptr, cout, Ho * Wo, cin, 0, "conv2d_pw"));
    if (rb || act) {
      ProfScope ps(ctx, "conv2d_pw_bias");
      const long n = (long)cout * Ho * Wo;
      FA_LAUNCH(ps, chan_bias_act_kernel, dim3((unsigned)std::min<long>(cdiv(n, 256), 8192)), dim3(256), 0, ctx->stream, F32(ro), CF32(rb), Ho * Wo,
                n, act);
      FA_TRY(check_launch(ctx, "conv2d_pw_bias"));
    }
    *out = og.release();
    return FA_OK;
  }
  ProfScope ps(ctx, "conv2d");
  FA_LAUNCH(ps, conv2d_kernel, dim3(gs((long)cout * Ho * Wo)), dim3(256), 0, ctx->stream, F32(rx), F32(rw), CF32(rb), F32(ro), cout, cin, h, wd,
                     Ho, Wo, kh, kw, sh, sw, pt, pl, groups, act);
  FA_TRY(check_launch(ctx, "conv2d"));
  *out = og.release();
  return FA_OK;
}

int fa_bmm_qk(fa_ctx *ctx, fa_tensor q, fa_tensor b, fa_tensor qb, int H, int HD, int W, int b_shared, fa_tensor *out) {
  TensorRec *rq, *rb, *rqb;
  FA_TRY(need(ctx, q, &rq, "bmmQK"));
  FA_TRY(need(ctx, b, &rb, "bmmQK b"));
  FA_TRY(opt(ctx, qb, &rqb, "bmmQK qb"));
  if (W <= 0 || rq->rows % W || (!b_shared && rb->rows % W) || rq->cols != H * HD || rb->cols != H * HD)
    return set_err(ctx, FA_E_INVALID, "bmmQK: shapes");
  const int T = rq->rows / W, Tb = b_shared ? rb->rows : rb->rows / W;
  fa_tensor o;
  TensorRec *ro;
  FA_TRY(new_tensor(ctx, W * H * T, Tb, S_F32, (size_t)W * H * T * Tb * 4, &o, &ro));
  TensorGuard og(ctx, o);  // released unless the op completes
  rq = get(ctx, q); rb = get(ctx, b); rqb = qb ? get(ctx, qb) : nullptr;
  ProfScope ps(ctx, "bmmQK");
  FA_LAUNCH(ps, bmm_qk_kernel, dim3(gs((long)W * H * T * Tb)), dim3(256), 0, ctx->stream, F32(rq), F32(rb), CF32(rqb), F32(ro), T, Tb, H, HD, W,
                     b_shared);
  FA_TRY(check_launch(ctx, "bmmQK"));
  *out = og.release();
  return FA_OK;
}

int fa_bmm_pv(fa_ctx *ctx, fa_tensor p, fa_tensor v, int H, int HD, int W, fa_tensor *out) {
  TensorRec *rp, *rv;
  FA_TRY(need(ctx, p, &rp, "bmmPV"));
  FA_TRY(need(ctx, v, &rv, "bmmPV v"));
  if (W <= 0 || rv->rows % W || rp->rows % (W * H) || rv->cols != H * HD) return set_err(ctx, FA_E_INVALID, "bmmPV: shapes");
  const int Tk = rv->rows / W, Tq = rp->rows / (W * H);
  if (rp->cols != Tk) return set_err(ctx, FA_E_INVALID, "bmmPV: probs have %d cols, Tk=%d", rp->cols, Tk);
  fa_tensor o;
  TensorRec *ro;
  FA_TRY(new_tensor(ctx, W * Tq, H * HD, S_F32, (size_t)W * Tq * H * HD * 4, &o, &ro));
  TensorGuard og(ctx, o);  // released unless the op completes
  rp = get(ctx, p); rv = get(ctx, v);
  ProfScope ps(ctx, "bmmPV");
  FA_LAUNCH(ps, bmm_pv_kernel, dim3(gs((long)W * Tq * H * HD)), dim3(256), 0, ctx->stream, F32(rp), F32(rv), F32(ro), Tq, Tk, H, HD, W);
  FA_TRY(check_launch(ctx, "bmmPV"));
  *out = og.release();
  return FA_OK;
}

int fa_rel_shift_b(fa_ctx *ctx, fa_tensor x, int H, fa_tensor *out) {
  TensorRec *rx;
  FA_TRY(need(ctx, x, &rx, "relShiftB"));
  if (H <= 0 || rx->rows % H) return set_err(ctx, FA_E_INVALID, "relShiftB: rows %d not divisible by H=%d", rx->rows, H);
  const int t = rx->rows / H;
  if (rx->cols != 2 * t - 1) return set_err(ctx, FA_E_INVALID, "relShiftB: expected %d cols, got %d", 2 * t - 1, rx->cols);
  fa_tensor o;
  TensorRec *ro;
  FA_TRY(new_tensor(ctx, H * t, t, S_F32, (size_t)H * t * t * 4, &o, &ro));
  TensorGuard og(ctx, o);  // released unless the op completes
  rx = get(ctx, x);
  ProfScope ps(ctx, "relShiftB");
  if ((long)H * t * t) FA_LAUNCH(ps, relshift_kernel, dim3(gs((long)H * t * t)), dim3(256), 0, ctx->stream, F32(rx), F32(ro), t, H);
  FA_TRY(check_launch(ctx, "relShiftB"));
  *out = og.release();
  return FA_OK;
}

int fa_rel_shift(fa_ctx *ctx, fa_tensor x, fa_tensor *out) { return fa_rel_shift_b(ctx, x, 1, out); }

int fa_rel_shift_stream(fa_ctx *ctx, fa_tensor x, int H, int n, int Lk, int dMax, int Lc, int subT, int C, int left, int right, fa_tensor *out) {
  TensorRec *rx;
  FA_TRY(need(ctx, x, &rx, "relShiftStream"));
  if (rx->kind != S_F32) return set_err(ctx, FA_E_INVALID, "relShiftStream: x must be f32");
  if (H <= 0 || n <= 0 || (long)H * n != rx->rows) return set_err(ctx, FA_E_INVALID, "relShiftStream: x has %d rows, H*n = %d*%d", rx->rows, H, n);
  if (Lk < 0 || C <= 0 || subT < 0 || left < 0 || right < 0 || rx->cols <= 0)
    return set_err(ctx, FA_E_INVALID, "relShiftStream: Lk %d, C %d, subT %d, left %d, right %d", Lk, C, subT, left, right);
  fa_tensor o;
  TensorRec *ro;
  const long total = (long)H * n * Lk;
  FA_TRY(new_tensor(ctx, H * n, Lk, S_F32, (size_t)total * 4, &o, &ro));
  TensorGuard og(ctx, o);  // released unless the op completes
  rx = get(ctx, x);
  ProfScope ps(ctx, "relShiftStream");
  if (total)
    FA_LAUNCH(ps, relshift_stream_kernel, dim3(gs(total)), dim3(256), 0, ctx->stream, F32(rx), F32(ro), total, n, Lk, rx->cols, dMax, Lc, subT, C,
              left, right);
  FA_TRY(check_launch(ctx, "relShiftStream"));
  *out = og.release();
  return FA_OK;
}

int fa_attn_fused(fa_ctx *ctx, fa_tensor q, fa_tensor k, fa_tensor v, fa_tensor pos, fa_tensor pbu, fa_tensor pbv, int H, int HD, int W, fa_tensor *out) {
  TensorRec *rq, *rk, *rv, *rp, *ru, *rw;
  FA_TRY(need(ctx, q, &rq, "attnFused q"));
  FA_TRY(need(ctx, k, &rk, "attnFused k"));
  FA_TRY(need(ctx, v, &rv, "attnFused v"));
  FA_TRY(need(ctx, pos, &rp, "attnFused pos"));
  FA_TRY(need(ctx, pbu, &ru, "attnFused pbu"));
  FA_TRY(need(ctx, pbv, &rw, "attnFused pbv"));
  if (W <= 0 || rq->rows % W || rq->cols != H * HD || rk->rows != rq->rows || rv->rows != rq->rows) return set_err(ctx, FA_E_INVALID, "attnFused: shapes");
  const int T = rq->rows / W;
  if (rp->rows != 2 * T - 1 || rp->cols != H * HD) return set_err(ctx, FA_E_INVALID, "attnFused: pos must be [2T-1, H*HD]");
  if (HD != 128) return set_err(ctx, FA_E_UNSUPPORTED, "attnFused: HD %d", HD);
  if (T > 1024) return set_err(ctx, FA_E_UNSUPPORTED, "attnFused: T %d > 1024", T);
  fa_tensor o;
  TensorRec *ro;
  FA_TRY(new_tensor(ctx, rq->rows, H * HD, S_F32, (size_t)rq->rows * H * HD * 4, &o, &ro));
  TensorGuard og(ctx, o);  // released unless the op completes
  rq = get(ctx, q); rk = get(ctx, k); rv = get(ctx, v); rp = get(ctx, pos); ru = get(ctx, pbu); rw = get(ctx, pbv);
  AttnArgs a;
  a.q = rq->ptr; a.k = rk->ptr; a.v = rv->ptr;
  a.ldq = a.ldk = a.ldv = H * HD;
  a.pos = rp->ptr; a.ldp = H * HD; a.prows = 2 * T - 1; a.pcenter = T - 1;
  a.pbu = F32(ru); a.pbv = F32(rw);
  a.out = ro->ptr; a.ldo = H * HD;
  a.H = H; a.HD = HD;
  for (int w0 = 0; w0 < W; w0 += kMaxWin) {  // windows in launches of at most kMaxWin
    a.win.n = W - w0 < kMaxWin ? W - w0 : kMaxWin;
    for (int i = 0; i < a.win.n; i++) {
      a.win.off[i] = (w0 + i) * T;
      a.win.len[i] = T;
    }
    FA_TRY(relpos_attention(ctx, a, 1, 1, T, "attnFused"));
  }
  *out = og.release();
  return FA_OK;
}

int fa_dequant_int8(fa_ctx *ctx, fa_tensor wq, fa_tensor scale, int K, int N, fa_tensor *out) {
  TensorRec *rw, *rs;
  FA_TRY(need(ctx, wq, &rw, "dequantInt8"));
  FA_TRY(need(ctx, scale, &rs, "dequantInt8 scale"));
  if (rw->bytes < (size_t)K * N || (long)rs->rows * rs->cols < N) return set_err(ctx, FA_E_INVALID, "dequantInt8: sizes");
  fa_tensor o;
  TensorRec *ro;
  FA_TRY(new_tensor(ctx, K, N, S_F32, (size_t)K * N * 4, &o, &ro));
  TensorGuard og(ctx, o);  // released unless the op completes
  rw = get(ctx, wq); rs = get(ctx, scale);
  ProfScope ps(ctx, "dequantInt8");
  FA_LAUNCH(ps, dequant_i8_kernel, dim3(gs((long)K * N)), dim3(256), 0, ctx->stream, (const int8_t *)rw->ptr, F32(rs), F32(ro), K, N);
  FA_TRY(check_launch(ctx, "dequantInt8"));
  *out = og.release();
  return FA_OK;
}

int fa_dequant_int4(fa_ctx *ctx, fa_tensor bq, fa_tensor scales_f16, int K, int N, fa_tensor *out) {
  TensorRec *rq, *rs;
  FA_TRY(need(ctx, bq, &rq, "dequantInt4"));
  FA_TRY(need(ctx, scales_f16, &rs, "dequantInt4 scales"));
  const int nblk = (K + 31) / 32;
  if (rq->bytes < (size_t)N * nblk * 16 || rs->bytes < (size_t)N * nblk * 2) return set_err(ctx, FA_E_INVALID, "dequantInt4: sizes");
  fa_tensor o;
  TensorRec *ro;
  FA_TRY(new_tensor(ctx, K, N, S_F32, (size_t)K * N * 4, &o, &ro));
  TensorGuard og(ctx, o);  // released unless the op completes
  rq = get(ctx, bq); rs = get(ctx, scales_f16);
  ProfScope ps(ctx, "dequantInt4");
  FA_LAUNCH(ps, dequant_i4_kernel, dim3(gs((long)K * N)), dim3(256), 0, ctx->stream, (const uint8_t *)rq->ptr, (const _Float16 *)rs->ptr, F32(ro), K, N);
  FA_TRY(check_launch(ctx, "dequantInt4"));
  *out = og.release();
  return FA_OK;
}

}  // extern "C"
