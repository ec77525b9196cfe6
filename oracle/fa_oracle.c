/*
 * fa_oracle.c — CPU restatement of fluidaudio-web's CPU (WASM) math for the
 * Parakeet FastConformer encoder path.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the parity checker and the reported
 * CPU baseline; nothing in the product library links or calls it.  Only
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it.
 *
 * Every function restates one reference routine and cites it.  Citations are
 * relative to the reference checkout (FluidInference/fluidaudio-web):
 *   lib.rs   = rust/wasm-kernels/src/lib.rs          (the wasm32+simd128 kernels)
 *   wctx     = src/gpu/wasm-context.js                (the WasmContext backend)
 *   enc      = src/engines/asr-parakeet/raw-encoder.js
 *   quant.py = scripts/quantize-parakeet-encoder.py
 *
 * Arithmetic follows the reference exactly where it is specified:
 *  - matmul_f32 accumulates in f32, i-k-j order, c = c + a*b with no fused
 *    multiply-add (lib.rs:59-94).  Built with -ffp-contract=off; the 4-wide SSE
 *    loop gives the same bits as the scalar loop (each lane is independent).
 *  - bias/activation, layernorm, softmax, glu, conv2d, bmmQK/bmmPV are plain JS
 *    over Float32Array, i.e. double arithmetic stored back to f32 (wctx).
 *  - depthwise conv1d is the Rust f32 loop (lib.rs:99-138).
 *  - int8 / int4 GEMMs accumulate in f32 (lib.rs:143-203).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#include <immintrin.h>
#ifdef _OPENMP
#include <omp.h>
#endif

enum { ACT_NONE = 0, ACT_GELU = 1, ACT_TANH = 2, ACT_RELU = 3, ACT_SILU = 4, ACT_GELU_ERF = 5 };

static int g_threads = 1;

/* Number of OpenMP threads the parallel loops use (1 = the reference's
 * single-threaded WASM context).  Row-parallel loops never change results. */
void or_set_threads(int n) { g_threads = n < 1 ? 1 : n; }
int or_get_threads(void) { return g_threads; }

/* ── activations: wctx:12-38 (JS doubles) ─────────────────────────────────── */
static double gelu_tanh(double x) {
  double t = 0.7978845608028654 * (x + 0.044715 * x * x * x);
  if (t < -20) t = -20;
  if (t > 20) t = 20;
  return 0.5 * x * (1 + tanh(t));
}
static double erf_a(double x) {
  double t = 1 / (1 + 0.3275911 * fabs(x));
  double y = 1 - ((((1.061405429 * t - 1.453152027) * t + 1.421413741) * t - 0.284496736) * t + 0.254829592) * t * exp(-x * x);
  return x >= 0 ? y : -y;
}
static double silu1(double x) {
  double c = x < -30 ? -30 : (x > 30 ? 30 : x);
  return x / (1 + exp(-c));
}
double or_act(double v, int act) {
  switch (act) {
    case ACT_GELU: return gelu_tanh(v);
    case ACT_TANH: return tanh(v);
    case ACT_RELU: return v > 0 ? v : 0;
    case ACT_SILU: return silu1(v);
    case ACT_GELU_ERF: return 0.5 * v * (1 + erf_a(v * 0.70710678118654752));
    default: return v;
  }
}

/* ── f32 GEMM: lib.rs:59-94 (matmul_f32) ─────────────────────────────────────
 * C[M,N] = A[M,K] @ B[K,N]; per row: zero, then for each k: c += a_ik * b_k. */
void or_matmul_f32(const float *a, const float *b, float *c, int m, int k, int n) {
  const int n4 = n & ~3;
#pragma omp parallel for num_threads(g_threads) schedule(static)
  for (int i = 0; i < m; i++) {
    float *crow = c + (size_t)i * n;
    memset(crow, 0, sizeof(float) * (size_t)n);
    const float *arow = a + (size_t)i * k;
    for (int kk = 0; kk < k; kk++) {
      const float aik = arow[kk];
      const __m128 av = _mm_set1_ps(aik);
      const float *brow = b + (size_t)kk * n;
      int j = 0;
      for (; j < n4; j += 4) {
        __m128 bv = _mm_loadu_ps(brow + j);
        __m128 cv = _mm_loadu_ps(crow + j);
        _mm_storeu_ps(crow + j, _mm_add_ps(cv, _mm_mul_ps(av, bv)));
      }
      for (; j < n; j++) crow[j] += aik * brow[j];
    }
  }
}

/* wctx:290-297 — per-column bias + act in doubles, stored to f32. */
void or_bias_act_cols(float *out, int m, int n, const float *bias, int act) {
  if (!bias && act == ACT_NONE) return;
#pragma omp parallel for num_threads(g_threads) schedule(static)
  for (int i = 0; i < m; i++)
    for (int j = 0; j < n; j++) {
      double v = (double)out[(size_t)i * n + j] + (bias ? (double)bias[j] : 0.0);
      out[(size_t)i * n + j] = (float)or_act(v, act);
    }
}

/* wctx:298-305 — per-row bias + act. */
void or_bias_act_rows(float *out, int r, int c, const float *bias, int act) {
  if (!bias && act == ACT_NONE) return;
  for (int i = 0; i < r; i++)
    for (int j = 0; j < c; j++) {
      double v = (double)out[(size_t)i * c + j] + (bias ? (double)bias[i] : 0.0);
      out[(size_t)i * c + j] = (float)or_act(v, act);
    }
}

/* wctx:135-156 — WasmContext.matmul: bare GEMM, then bias/act, then add. */
void or_matmul(const float *a, const float *b, float *c, int m, int k, int n, const float *bias, int act, const float *add) {
  or_matmul_f32(a, b, c, m, k, n);
  or_bias_act_cols(c, m, n, bias, act);
  if (add) {
    size_t tot = (size_t)m * n;
    for (size_t i = 0; i < tot; i++) c[i] = (float)((double)c[i] + (double)add[i]);
  }
}

/* lib.rs:143-162 — int8 GEMM, wq row-major [k*N+n] int8, scale per column.
 * acc (f32) += a * q; y = acc * scale.  Bias/act as wctx:171-189. */
void or_matmul_int8(const float *a, const int8_t *wq, const float *scale, float *y, int m, int n, int k, const float *bias, int act) {
#pragma omp parallel for num_threads(g_threads) schedule(static)
  for (int i = 0; i < m; i++) {
    const float *arow = a + (size_t)i * k;
    for (int j = 0; j < n; j++) {
      float acc = 0.0f;
      for (int kk = 0; kk < k; kk++) acc += arow[kk] * (float)wq[(size_t)kk * n + j];
      y[(size_t)i * n + j] = acc * scale[j];
    }
  }
  or_bias_act_cols(y, m, n, bias, act);
}

/* lib.rs:169-203 — int4 MatMulNBits: bq [N][nblk][16 B], low nibble = even k;
 * zero-points packed int4 [N][zpb], even block = low nibble; f32 scales [N][nblk].
 * acc (f32) += a * ((q - zp) * scale). */
void or_matmul_nbits(const float *a, const uint8_t *bq, const float *scales, const uint8_t *zp, float *y, int m, int n, int k, int nblk, int zpb, int blocksize) {
#pragma omp parallel for num_threads(g_threads) schedule(static)
  for (int j = 0; j < n; j++) {
    const uint8_t *bq_row = bq + (size_t)j * nblk * 16;
    const uint8_t *zp_row = zp + (size_t)j * zpb;
    const float *sc_row = scales + (size_t)j * nblk;
    for (int i = 0; i < m; i++) {
      const float *arow = a + (size_t)i * k;
      float acc = 0.0f;
      for (int blk = 0; blk < nblk; blk++) {
        const float s = sc_row[blk];
        const uint8_t zb = zp_row[blk / 2];
        const float zpv = (float)((blk & 1) == 0 ? (zb & 0x0f) : (zb >> 4));
        const uint8_t *bb = bq_row + (size_t)blk * 16;
        for (int t = 0; t < blocksize; t++) {
          int kk = blk * blocksize + t;
          if (kk >= k) break;
          uint8_t byte = bb[t / 2];
          float q = (float)((t & 1) == 0 ? (byte & 0x0f) : (byte >> 4));
          acc += arow[kk] * ((q - zpv) * s);
        }
      }
      y[(size_t)i * n + j] = acc;
    }
  }
}

/* wctx:308-326 — row layernorm, JS doubles. */
void or_layernorm(const float *x, const float *gamma, const float *beta, float *out, int r, int c, double eps) {
#pragma omp parallel for num_threads(g_threads) schedule(static)
  for (int i = 0; i < r; i++) {
    const float *xr = x + (size_t)i * c;
    double mean = 0;
    for (int j = 0; j < c; j++) mean += xr[j];
    mean /= c;
    double v = 0;
    for (int j = 0; j < c; j++) {
      double d = xr[j] - mean;
      v += d * d;
    }
    v /= c;
    double inv = 1 / sqrt(v + eps);
    for (int j = 0; j < c; j++) out[(size_t)i * c + j] = (float)((xr[j] - mean) * inv * gamma[j] + beta[j]);
  }
}

/* wctx:327-343 — row softmax: e stored to f32 first, then divided by the
 * double sum of the unrounded exponentials. */
void or_softmax(const float *x, float *out, int r, int c) {
#pragma omp parallel for num_threads(g_threads) schedule(static)
  for (int i = 0; i < r; i++) {
    const float *xr = x + (size_t)i * c;
    float *o = out + (size_t)i * c;
    double mx = -INFINITY;
    for (int j = 0; j < c; j++) mx = xr[j] > mx ? xr[j] : mx;
    double s = 0;
    for (int j = 0; j < c; j++) {
      double e = exp(xr[j] - mx);
      o[j] = (float)e;
      s += e;
    }
    for (int j = 0; j < c; j++) o[j] = (float)((double)o[j] / s);
  }
}

/* wctx:428-434 — GLU over channel rows [2C,T] -> [C,T] (no clamp on CPU). */
void or_glu(const float *x, float *out, int c2, int t) {
  int c = c2 / 2;
  for (int ch = 0; ch < c; ch++)
    for (int j = 0; j < t; j++) {
      double a = x[(size_t)ch * t + j], b = x[(size_t)(ch + c) * t + j];
      out[(size_t)ch * t + j] = (float)(a * (1 / (1 + exp(-b))));
    }
}

/* wctx:396-400 */
void or_silu(const float *x, float *out, size_t n) {
  for (size_t i = 0; i < n; i++) out[i] = (float)silu1(x[i]);
}

/* wctx:435-441 */
void or_transpose(const float *x, float *out, int r, int c) {
  for (int i = 0; i < r; i++)
    for (int j = 0; j < c; j++) out[(size_t)j * r + i] = x[(size_t)i * c + j];
}

/* wctx:632-685 — direct conv2d (batch 1), x [Cin, H*W], w [Cout,Cin/g,kh,kw];
 * double accumulator seeded with the bias. */
void or_conv2d(const float *x, const float *w, const float *bias, float *out, int cout, int cin, int h, int wd, int kh, int kw, int sh, int sw,
               int pt, int pb, int pl, int pr, int groups, int act) {
  const int ho_n = (h + pt + pb - kh) / sh + 1, wo_n = (wd + pl + pr - kw) / sw + 1;
  const int cing = cin / groups, coutg = cout / groups;
#pragma omp parallel for num_threads(g_threads) schedule(static)
  for (int co = 0; co < cout; co++) {
    const int g = co / coutg;
    for (int ho = 0; ho < ho_n; ho++)
      for (int wo = 0; wo < wo_n; wo++) {
        double acc = bias ? (double)bias[co] : 0.0;
        for (int ci = 0; ci < cing; ci++) {
          const int rc = g * cing + ci;
          for (int a = 0; a < kh; a++) {
            const int hi = ho * sh + a - pt;
            if (hi < 0 || hi >= h) continue;
            for (int bb = 0; bb < kw; bb++) {
              const int wi = wo * sw + bb - pl;
              if (wi < 0 || wi >= wd) continue;
              acc += (double)x[(size_t)rc * h * wd + (size_t)hi * wd + wi] * (double)w[(((size_t)co * cing + ci) * kh + a) * kw + bb];
            }
          }
        }
        out[(size_t)co * ho_n * wo_n + (size_t)ho * wo_n + wo] = (float)or_act(acc, act);
      }
  }
}

/* lib.rs:99-138 (conv1d_f32, used by wctx:251-263 for groups>1) + wctx:298-305
 * bias/act.  f32 accumulation, zero weights skipped. */
void or_conv1d_grouped(const float *x, const float *w, const float *bias, float *y, int cout, int cin, int l, int k, int stride, int pad_left,
                       int pad_right, int dilation, int groups, int act) {
  const int lout = (l + pad_left + pad_right - dilation * (k - 1) - 1) / stride + 1;
  const int cin_g = cin / groups, cout_g = cout / groups;
#pragma omp parallel for num_threads(g_threads) schedule(static)
  for (int co = 0; co < cout; co++) {
    const int g = co / cout_g;
    float *yrow = y + (size_t)co * lout;
    for (int t = 0; t < lout; t++) yrow[t] = 0.0f;
    for (int cig = 0; cig < cin_g; cig++) {
      const int ci = g * cin_g + cig;
      const float *xrow = x + (size_t)ci * l;
      const size_t wbase = ((size_t)co * cin_g + cig) * k;
      for (int kk = 0; kk < k; kk++) {
        const float wv = w[wbase + kk];
        if (wv == 0.0f) continue;
        const int off = kk * dilation;
        for (int t = 0; t < lout; t++) {
          const int src = t * stride + off;
          if (src >= pad_left) {
            const int xi = src - pad_left;
            if (xi < l) yrow[t] += xrow[xi] * wv;
          }
        }
      }
    }
  }
  or_bias_act_rows(y, cout, lout, bias, act);
}

/* wctx:552-563 — subsampling reshape [C, Tsub*F] -> [Tsub, C*F]. */
void or_subreshape(const float *x, float *out, int c, int tsub, int f) {
  const int cf = c * f;
  for (int idx = 0; idx < tsub * cf; idx++) {
    int ho = idx / cf, rem = idx % cf, ch = rem / f, wo = rem % f;
    out[idx] = x[(size_t)ch * (tsub * f) + (size_t)ho * f + wo];
  }
}

/* wctx:462-482 — batched (q + qb) · bᵀ over heads; b shared across windows
 * when b_shared (the positional table).  Double accumulation. */
void or_bmm_qk(const float *q, int q_rows, const float *b, int b_rows, const float *qb, float *out, int H, int HD, int W, int b_shared) {
  const int T = q_rows / W, Tb = b_shared ? b_rows : b_rows / W, stride = H * HD;
#pragma omp parallel for collapse(2) num_threads(g_threads) schedule(static)
  for (int w = 0; w < W; w++)
    for (int h = 0; h < H; h++) {
      const int ho = h * HD;
      for (int i = 0; i < T; i++) {
        const size_t qBase = ((size_t)w * T + i) * stride + ho, oBase = (((size_t)w * H + h) * T + i) * Tb;
        for (int j = 0; j < Tb; j++) {
          const size_t bBase = (size_t)(b_shared ? j : w * Tb + j) * stride + ho;
          double acc = 0;
          for (int d = 0; d < HD; d++) acc += ((double)q[qBase + d] + (qb ? (double)qb[ho + d] : 0.0)) * (double)b[bBase + d];
          out[oBase + j] = (float)acc;
        }
      }
    }
}

/* wctx:484-500 — batched probs · V; p [W*H*Tq, Tk], v [W*Tk, H*HD]. */
void or_bmm_pv(const float *p, int p_rows, const float *v, int v_rows, float *out, int H, int HD, int W) {
  const int Tk = v_rows / W, Tq = p_rows / (W * H), stride = H * HD;
#pragma omp parallel for collapse(2) num_threads(g_threads) schedule(static)
  for (int w = 0; w < W; w++)
    for (int i = 0; i < Tq; i++)
      for (int c = 0; c < stride; c++) {
        const int h = c / HD;
        const size_t pBase = (((size_t)w * H + h) * Tq + i) * Tk;
        double acc = 0;
        for (int j = 0; j < Tk; j++) acc += (double)p[pBase + j] * (double)v[((size_t)w * Tk + j) * stride + c];
        out[((size_t)w * Tq + i) * stride + c] = (float)acc;
      }
}

/* wctx:525-538 — batched NeMo rel_shift [H*t, 2t-1] -> [H*t, t]. */
void or_relshift_b(const float *x, float *out, int rows, int H) {
  const int t = rows / H, p = 2 * t - 1, twoT = 2 * t;
  for (int h = 0; h < H; h++)
    for (int i = 0; i < t; i++)
      for (int j = 0; j < t; j++) {
        const long f = (long)t + (long)i * p + j, col = f % twoT;
        out[((size_t)h * t + i) * t + j] = col == 0 ? 0.0f : x[((size_t)h * t + f / twoT) * p + (col - 1)];
      }
}

/* wctx:509-524 — streaming rel_shift + chunked-causal mask: x [H*n, P] -> [H*n, Lk]. */
void or_relshift_stream(const float *x, float *out, int H, int n, int Lk, int P, int dMax, int Lc, int subT, int C, int left, int right) {
  for (int r = 0; r < H * n; r++) {
    const int i = r % n, q = subT + i, cs = C * (int)floor((double)q / C);
    for (int j = 0; j < Lk; j++) {
      const int k = subT - Lc + j;
      int d = dMax - (q - k);
      if (d < 0) d = 0;
      if (d > P - 1) d = P - 1;
      out[(size_t)r * Lk + j] = (k < cs - left || k > cs + C - 1 + right) ? -10000.0f : x[(size_t)r * P + d];
    }
  }
}

/* enc:163-174 — sinusoidal table over 2T-1 relative positions T-1 .. -(T-1). */
void or_pos_encoding(int T, int D, float *pe) {
  const double lg = log(10000.0) / D;
  for (int pi = 0; pi < 2 * T - 1; pi++) {
    const double pos = T - 1 - pi;
    for (int i = 0; i < D; i += 2) {
      const double dv = exp(i * -lg);
      pe[(size_t)pi * D + i] = (float)sin(pos * dv);
      pe[(size_t)pi * D + i + 1] = (float)cos(pos * dv);
    }
  }
}

/* quant.py:31-36 — per-output-column symmetric int8 of w [K,N] ([in,out]).
 * s = f32(max|w|)/127 in f32 (s == 0 -> 1); q = clip(rint(w/s), -127, 127). */
void or_quantize_int8_cols(const float *w, int K, int N, int8_t *q, float *scale) {
  for (int n = 0; n < N; n++) {
    float mx = 0.0f;
    for (int k = 0; k < K; k++) {
      float a = fabsf(w[(size_t)k * N + n]);
      mx = a > mx ? a : mx;
    }
    float s = mx / 127.0f;
    if (s == 0.0f) s = 1.0f;
    scale[n] = s;
  }
  for (int k = 0; k < K; k++)
    for (int n = 0; n < N; n++) {
      float r = rintf(w[(size_t)k * N + n] / scale[n]);
      r = r < -127.0f ? -127.0f : (r > 127.0f ? 127.0f : r);
      q[(size_t)k * N + n] = (int8_t)r;
    }
}

/* Dequant of the int8 format (enc:68-70: out = q * sc[col]). */
void or_dequant_int8_cols(const int8_t *q, const float *scale, int K, int N, float *w) {
  for (int k = 0; k < K; k++)
    for (int n = 0; n < N; n++) w[(size_t)k * N + n] = (float)q[(size_t)k * N + n] * scale[n];
}

/* f16 helpers (round-to-nearest-even), used for the int4 scale format. */
static uint16_t f32_to_f16_bits(float f) {
  uint32_t x;
  memcpy(&x, &f, 4);
  uint32_t sign = (x >> 16) & 0x8000u, ax = x & 0x7fffffffu;
  if (ax >= 0x7f800000u) return (uint16_t)(sign | (ax > 0x7f800000u ? 0x7e00u : 0x7c00u));
  if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); /* >= 65520 rounds to inf */
  if (ax < 0x38800000u) {                                    /* subnormal / zero in f16 */
    if (ax < 0x33000000u) return (uint16_t)sign;             /* < 2^-25: rounds to 0 */
    uint32_t mant = (ax & 0x7fffffu) | 0x800000u;
    int e = (int)(ax >> 23);
    int shift = 126 - e; /* value in units of 2^-24 (f16 subnormal step) = mant >> (126 - e) */
    uint32_t q = mant >> shift, rem = mant & ((1u << shift) - 1u), half = 1u << (shift - 1);
    if (rem > half || (rem == half && (q & 1u))) q++;
    return (uint16_t)(sign | q);
  }
  uint32_t e = ((ax >> 23) - 112u) << 10, m = ax & 0x7fffffu;
  uint32_t h = e | (m >> 13);
  uint32_t rem = m & 0x1fffu;
  if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
  return (uint16_t)(sign | h);
}
static float f16_bits_to_f32(uint16_t h) {
  uint32_t s = (uint32_t)(h & 0x8000u) << 16, e = (h >> 10) & 0x1fu, m = h & 0x3ffu, x;
  if (e == 0) {
    float v = ldexpf((float)m, -24);
    return s ? -v : v;
  } else if (e == 31) {
    x = s | 0x7f800000u | (m << 13);
  } else {
    x = s | ((e + 112u) << 23) | (m << 13);
  }
  float f;
  memcpy(&f, &x, 4);
  return f;
}
uint16_t or_f32_to_f16(float f) { return f32_to_f16_bits(f); }
float or_f16_to_f32(uint16_t h) { return f16_bits_to_f32(h); }

/* Symmetric int4 group-32 with f16 scales, stored in the MatMulNBits layout of
 * lib.rs:164-203 with every zero-point = 8.  w is [K,N] ([in,out]); for output
 * column n and block b: s = f16(max|w| / 7) (0 -> 1), q = clip(rint(w / s),
 * -8, 7), nibble = q + 8, low nibble = even k.  K % 32 may be non-zero (the
 * last block is partial, its padding nibbles encode q = 0).  zp is written as
 * the packed [N][ceil(nblk/2)] int4 array (all 8s) so the reference kernel can
 * consume it unchanged; scales_f32 receives the f16 scales widened to f32. */
void or_quantize_int4_g32(const float *w, int K, int N, uint8_t *bq, uint16_t *scales_f16, float *scales_f32, uint8_t *zp) {
  const int nblk = (K + 31) / 32, zpb = (nblk + 1) / 2;
  for (int n = 0; n < N; n++) {
    for (int b = 0; b < nblk; b++) {
      float mx = 0.0f;
      for (int t = 0; t < 32 && b * 32 + t < K; t++) {
        float a = fabsf(w[(size_t)(b * 32 + t) * N + n]);
        mx = a > mx ? a : mx;
      }
      uint16_t sh = f32_to_f16_bits(mx / 7.0f);
      float s = f16_bits_to_f32(sh);
      if (s == 0.0f) {
        sh = 0x3c00u;
        s = 1.0f;
      }
      scales_f16[(size_t)n * nblk + b] = sh;
      if (scales_f32) scales_f32[(size_t)n * nblk + b] = s;
      uint8_t *blk = bq + ((size_t)n * nblk + b) * 16;
      memset(blk, 0x88, 16);
      for (int t = 0; t < 32 && b * 32 + t < K; t++) {
        float r = rintf(w[(size_t)(b * 32 + t) * N + n] / s);
        r = r < -8.0f ? -8.0f : (r > 7.0f ? 7.0f : r);
        uint8_t nib = (uint8_t)((int)r + 8);
        if (t & 1)
          blk[t / 2] = (uint8_t)((blk[t / 2] & 0x0f) | (nib << 4));
        else
          blk[t / 2] = (uint8_t)((blk[t / 2] & 0xf0) | nib);
      }
    }
    if (zp) memset(zp + (size_t)n * zpb, 0x88, (size_t)zpb);
  }
}

/* Dequant of the int4 group-32 format to [K,N] f32: w = (nib - 8) * s. */
void or_dequant_int4_g32(const uint8_t *bq, const uint16_t *scales_f16, int K, int N, float *w) {
  const int nblk = (K + 31) / 32;
  for (int n = 0; n < N; n++)
    for (int k = 0; k < K; k++) {
      int b = k / 32, t = k % 32;
      uint8_t byte = bq[((size_t)n * nblk + b) * 16 + t / 2];
      int nib = (t & 1) ? (byte >> 4) : (byte & 0x0f);
      w[(size_t)k * N + n] = (float)(nib - 8) * f16_bits_to_f32(scales_f16[(size_t)n * nblk + b]);
    }
}

/* ════════════════════════════════════════════════════════════════════════════
 * The encoder forward: enc:39-161 (load-time folds) + enc:177-222 (preEncode)
 * + enc:235-386 (parakeetEncodeBatch), composed from the ops above exactly as
 * the reference composes ComputeContext calls on the WASM backend.
 *
 * Weights arrive as one flat f32 array plus an offset table.  Table order:
 *   global: c0w c0b c1w c1b c2w c2b c3w c3b c4w c4b linw linb         (12)
 *   per layer (OR_LAYER_KEYS entries, in this order):
 *     lnff1_w lnff1_b ff1w1 ff1w2 ff1b1 ff1b2 lnatt_w lnatt_b q k v pos out
 *     qb kb vb outb pbu pbv lnconv_w lnconv_b pw1 pw1b dw dwb pw2 pw2b
 *     lnff2_w lnff2_b ff2w1 ff2w2 ff2b1 ff2b2 lnout_w lnout_b
 * An offset of -1 marks an absent optional tensor (biases).  Shapes are the
 * manifest's: matrices [in,out], pw1 [2D,D], pw2 [D,D], dw [D,1,K].
 * ════════════════════════════════════════════════════════════════════════════ */
#define OR_GLOBAL_KEYS 12
#define OR_LAYER_KEYS 35
enum {
  L_LNFF1_W, L_LNFF1_B, L_FF1W1, L_FF1W2, L_FF1B1, L_FF1B2, L_LNATT_W, L_LNATT_B, L_Q, L_K, L_V, L_POS, L_OUT, L_QB, L_KB, L_VB, L_OUTB,
  L_PBU, L_PBV, L_LNCONV_W, L_LNCONV_B, L_PW1, L_PW1B, L_DW, L_DWB, L_PW2, L_PW2B, L_LNFF2_W, L_LNFF2_B, L_FF2W1, L_FF2W2, L_FF2B1,
  L_FF2B2, L_LNOUT_W, L_LNOUT_B
};

typedef struct {
  int D, DFF, H, HD, layers, dwK, Csub, Fsub, melBins;
} or_cfg;

int or_layer_keys(void) { return OR_LAYER_KEYS; }
int or_global_keys(void) { return OR_GLOBAL_KEYS; }

static float *dup_scaled(const float *src, size_t n, double s) {
  float *o = (float *)malloc(n * sizeof(float));
  for (size_t i = 0; i < n; i++) o[i] = (float)((double)src[i] * s); /* enc:77-81 */
  return o;
}
static float *pw_transpose(const float *w, int cout, int cin) { /* enc:115-120 */
  float *t = (float *)malloc((size_t)cin * cout * sizeof(float));
  for (int co = 0; co < cout; co++)
    for (int ci = 0; ci < cin; ci++) t[(size_t)ci * cout + co] = w[(size_t)co * cin + ci];
  return t;
}

/* preEncode (enc:177-222) for one window: mel [melBins, T] channel-major ->
 * x [Tsub, D].  Returns Tsub; out must hold Tsub*D floats. */
int or_pre_encode(const or_cfg *cfg, const float *wflat, const int64_t *off, const float *mel, int T, float *out) {
  const int Csub = cfg->Csub, mb = cfg->melBins;
  float *x0 = (float *)malloc((size_t)T * mb * sizeof(float));
  for (int t = 0; t < T; t++)
    for (int c = 0; c < mb; c++) x0[(size_t)t * mb + c] = mel[(size_t)c * T + t];
  /* [cout, cin, k, stride, groups, act, isStride2] — enc:187-193 */
  static const int conv[5][7] = {
      {0, 1, 3, 2, 1, ACT_RELU, 1}, {0, 0, 3, 2, -1, ACT_NONE, 1}, {0, 0, 1, 1, 1, ACT_RELU, 0}, {0, 0, 3, 2, -1, ACT_NONE, 1}, {0, 0, 1, 1, 1, ACT_RELU, 0}};
  float *s = x0;
  int Hh = T, Wd = mb, cin = 1;
  for (int i = 0; i < 5; i++) {
    const int k = conv[i][2], st = conv[i][3], groups = conv[i][4] < 0 ? Csub : 1, act = conv[i][5], s2 = conv[i][6];
    const int p = s2 ? 1 : 0;
    const int Ho = (Hh + 2 * p - k) / st + 1, Wo = (Wd + 2 * p - k) / st + 1;
    float *y = (float *)malloc((size_t)Csub * Ho * Wo * sizeof(float));
    or_conv2d(s, wflat + off[2 * i], wflat + off[2 * i + 1], y, Csub, cin, Hh, Wd, k, k, st, st, p, p, p, p, groups, act);
    free(s);
    s = y;
    Hh = Ho;
    Wd = Wo;
    cin = Csub;
  }
  const int Tsub = Hh, F = Wd;
  float *flat = (float *)malloc((size_t)Tsub * Csub * F * sizeof(float));
  or_subreshape(s, flat, Csub, Tsub, F);
  free(s);
  or_matmul(flat, wflat + off[10], out, Tsub, Csub * F, cfg->D, wflat + off[11], ACT_NONE, NULL);
  free(flat);
  return Tsub;
}

static const float *W_(const float *wflat, const int64_t *loff, int key) { return loff[key] < 0 ? NULL : wflat + loff[key]; }

/* Macaron feed-forward ff() (enc:284): x += 0.5·W2·silu(W1·LN(x) + b1) + 0.5·b2,
 * the 0.5 folded into W2/b2 at load (enc:129-131,154-156).  which = 0 for FF1,
 * 1 for FF2. */
static void or_ff(const or_cfg *cfg, const float *wflat, const int64_t *loff, float *x, int M, int which, float *h, float *u, float *t2) {
  const int D = cfg->D, DFF = cfg->DFF;
  const int lw = which == 0 ? L_LNFF1_W : L_LNFF2_W;
  const int w1 = which == 0 ? L_FF1W1 : L_FF2W1, w2 = which == 0 ? L_FF1W2 : L_FF2W2;
  const int b1 = which == 0 ? L_FF1B1 : L_FF2B1, b2 = which == 0 ? L_FF1B2 : L_FF2B2;
  float *w2s = dup_scaled(W_(wflat, loff, w2), (size_t)DFF * D, 0.5);
  float *b2s = W_(wflat, loff, b2) ? dup_scaled(W_(wflat, loff, b2), D, 0.5) : NULL;
  or_layernorm(x, W_(wflat, loff, lw), W_(wflat, loff, lw + 1), h, M, D, 1e-5);
  or_matmul(h, W_(wflat, loff, w1), u, M, D, DFF, W_(wflat, loff, b1), ACT_SILU, NULL);
  or_matmul(u, w2s, t2, M, DFF, D, b2s, ACT_NONE, x);
  memcpy(x, t2, (size_t)M * D * sizeof(float));
  free(w2s);
  free(b2s);
}

/* Rel-pos multi-head self-attention block (enc:301-345) on x [W*T, D], in place:
 * x += out(softmax(relpos scores)·V).  q weights/bias and pos_bias_u/v carry the
 * 1/sqrt(HD) fold (enc:124-125,133,138).  pe is the [2T-1, D] sinusoid table. */
static void or_attention(const or_cfg *cfg, const float *wflat, const int64_t *loff, float *x, int W, int T, const float *pe, float *h, float *t2) {
  const int D = cfg->D, H = cfg->H, HD = cfg->HD, M = W * T;
  const double INV = 1.0 / sqrt((double)HD);
  const size_t MD = (size_t)M * D;
  float *qs = dup_scaled(W_(wflat, loff, L_Q), (size_t)D * D, INV);
  float *qbs = W_(wflat, loff, L_QB) ? dup_scaled(W_(wflat, loff, L_QB), D, INV) : NULL;
  float *pbu = dup_scaled(W_(wflat, loff, L_PBU), (size_t)H * HD, INV);
  float *pbv = dup_scaled(W_(wflat, loff, L_PBV), (size_t)H * HD, INV);
  float *q = (float *)malloc(MD * sizeof(float)), *k = (float *)malloc(MD * sizeof(float)), *v = (float *)malloc(MD * sizeof(float));
  or_layernorm(x, W_(wflat, loff, L_LNATT_W), W_(wflat, loff, L_LNATT_B), h, M, D, 1e-5);
  or_matmul(h, qs, q, M, D, D, qbs, ACT_NONE, NULL);
  or_matmul(h, W_(wflat, loff, L_K), k, M, D, D, W_(wflat, loff, L_KB), ACT_NONE, NULL);
  or_matmul(h, W_(wflat, loff, L_V), v, M, D, D, W_(wflat, loff, L_VB), ACT_NONE, NULL);
  const int P = 2 * T - 1;
  float *p = (float *)malloc((size_t)P * D * sizeof(float));
  or_matmul(pe, W_(wflat, loff, L_POS), p, P, D, D, NULL, ACT_NONE, NULL);
  const size_t SR = (size_t)W * H * T;
  float *ac = (float *)malloc(SR * T * sizeof(float));
  float *bdr = (float *)malloc(SR * P * sizeof(float));
  float *bd = (float *)malloc(SR * T * sizeof(float));
  or_bmm_qk(q, M, k, M, pbu, ac, H, HD, W, 0);  /* ac = (q+u)·kᵀ */
  or_bmm_qk(q, M, p, P, pbv, bdr, H, HD, W, 1); /* (q+v)·pᵀ, [W*H*T, 2T-1] */
  or_relshift_b(bdr, bd, (int)SR, W * H);
  for (size_t i = 0; i < SR * T; i++) ac[i] = (float)((double)ac[i] + (double)bd[i]);
  or_softmax(ac, bd, (int)SR, T);
  or_bmm_pv(bd, (int)SR, v, M, h, H, HD, W);
  or_matmul(h, W_(wflat, loff, L_OUT), t2, M, D, D, W_(wflat, loff, L_OUTB), ACT_NONE, x);
  memcpy(x, t2, MD * sizeof(float));
  free(qs); free(qbs); free(pbu); free(pbv); free(q); free(k); free(v); free(p); free(ac); free(bdr); free(bd);
}

/* Conv module (enc:348-369), Parakeet form (BatchNorm folded into dw, SiLU
 * fused): x += pw2(silu(dwconv_k(glu(pw1(LN(x)))))), depthwise per window. */
static void or_conv_module(const or_cfg *cfg, const float *wflat, const int64_t *loff, float *x, int W, int T, float *h, float *u, float *t2) {
  const int D = cfg->D, K = cfg->dwK, M = W * T;
  const size_t MD = (size_t)M * D;
  float *pw1T = pw_transpose(W_(wflat, loff, L_PW1), 2 * D, D);
  float *pw2T = pw_transpose(W_(wflat, loff, L_PW2), D, D);
  or_layernorm(x, W_(wflat, loff, L_LNCONV_W), W_(wflat, loff, L_LNCONV_B), h, M, D, 1e-5);
  or_matmul(h, pw1T, u, M, D, 2 * D, W_(wflat, loff, L_PW1B), ACT_NONE, NULL); /* [M, 2D] */
  float *pre1t = (float *)malloc((size_t)2 * D * M * sizeof(float));
  or_transpose(u, pre1t, M, 2 * D); /* [2D, M] */
  float *glu = (float *)malloc(MD * sizeof(float));
  or_glu(pre1t, glu, 2 * D, M); /* [D, M] */
  float *dwo = (float *)malloc(MD * sizeof(float));
  float *sl = (float *)malloc((size_t)D * T * sizeof(float)), *so = (float *)malloc((size_t)D * T * sizeof(float));
  const int padL = (K - 1) >> 1, padR = (K - 1) >> 1; /* enc:279-280 (non-causal) */
  for (int wi = 0; wi < W; wi++) { /* sliceCols -> conv1d -> setCols (enc:352-359) */
    for (int c = 0; c < D; c++) memcpy(sl + (size_t)c * T, glu + (size_t)c * M + (size_t)wi * T, T * sizeof(float));
    or_conv1d_grouped(sl, W_(wflat, loff, L_DW), W_(wflat, loff, L_DWB), so, D, D, T, K, 1, padL, padR, 1, D, ACT_SILU);
    for (int c = 0; c < D; c++) memcpy(dwo + (size_t)c * M + (size_t)wi * T, so + (size_t)c * T, T * sizeof(float));
  }
  or_transpose(dwo, h, D, M); /* [M, D] */
  or_matmul(h, pw2T, t2, M, D, D, W_(wflat, loff, L_PW2B), ACT_NONE, x);
  memcpy(x, t2, MD * sizeof(float));
  free(pw1T); free(pw2T); free(pre1t); free(glu); free(dwo); free(sl); free(so);
}

/* One conformer block on x [W*T, D], in place: enc:300-371 for one layer L. */
void or_layer(const or_cfg *cfg, const float *wflat, const int64_t *loff, float *x, int W, int T, const float *pe) {
  const int D = cfg->D, M = W * T;
  const size_t MD = (size_t)M * D;
  const int U = cfg->DFF > 2 * D ? cfg->DFF : 2 * D;
  float *h = (float *)malloc(MD * sizeof(float)), *u = (float *)malloc((size_t)M * U * sizeof(float)), *t2 = (float *)malloc(MD * sizeof(float));
  or_ff(cfg, wflat, loff, x, M, 0, h, u, t2);
  or_attention(cfg, wflat, loff, x, W, T, pe, h, t2);
  or_conv_module(cfg, wflat, loff, x, W, T, h, u, t2);
  or_ff(cfg, wflat, loff, x, M, 1, h, u, t2);
  or_layernorm(x, W_(wflat, loff, L_LNOUT_W), W_(wflat, loff, L_LNOUT_B), t2, M, D, 1e-5);
  memcpy(x, t2, MD * sizeof(float));
  free(h);
  free(u);
  free(t2);
}

/* parakeetEncodeBatch (enc:235-386): W windows of equal length T (mel frames),
 * mels [W][melBins*T] channel-major; out [W*Tsub, D].  Runs `layers` layers
 * (<= cfg->layers; the full stack when equal).  Returns Tsub, or -1 when the
 * windows' subsampled lengths differ (the reference throws, enc:241). */
int or_encode_batch(const or_cfg *cfg, const float *wflat, const int64_t *off, const float *mels, int W, int T, int layers, float *out) {
  const int D = cfg->D;
  int Tsub = -1;
  for (int w = 0; w < W; w++) {
    const int ts = or_pre_encode(cfg, wflat, off, mels + (size_t)w * cfg->melBins * T, T, out + (size_t)w * (Tsub < 0 ? 0 : Tsub) * D);
    if (Tsub >= 0 && ts != Tsub) return -1;
    Tsub = ts;
  }
  float *pe = (float *)malloc((size_t)(2 * Tsub - 1) * D * sizeof(float));
  or_pos_encoding(Tsub, D, pe);
  for (int L = 0; L < layers; L++) or_layer(cfg, wflat, off + OR_GLOBAL_KEYS + (size_t)L * OR_LAYER_KEYS, out, W, Tsub, pe);
  free(pe);
  return Tsub;
}

/* Output length of the 3-stage stride-2 front end (enc:217-218 with pad 1,1). */
int or_tsub(int T) {
  for (int i = 0; i < 3; i++) T = (T + 2 - 3) / 2 + 1;
  return T;
}

/* ── log-mel front end ──────────────────────────────────────────────────────
 * JsPreprocessor (src/engines/asr-nemotron/nemotron-mel.js) with Parakeet's
 * settings (src/engines/asr-parakeet/parakeet-mel.js:8-22: log guard 2^-24,
 * per-feature normalisation).  JS doubles throughout; the arrays the reference
 * keeps in Float32Array (pre-emphasised samples, power spectrum, raw log-mel,
 * features, filterbank) are rounded to f32 where it stores them.  Built with
 * -ffp-contract=off: every a*b+c is a separate multiply and add, as in JS. */
#define MEL_NFFT 512
#define MEL_WIN 400
#define MEL_HOP 160
#define MEL_NBINS 257

static double mel_hz_to_mel(double f) { /* nemotron-mel.js:63-65 */
  const double f_sp = 200.0 / 3, min_log_hz = 1000.0, min_log_mel = min_log_hz / f_sp, log_step = log(6.4) / 27.0;
  return f >= min_log_hz ? min_log_mel + log(f / min_log_hz) / log_step : f / f_sp;
}
static double mel_mel_to_hz(double m) { /* nemotron-mel.js:67-69 */
  const double f_sp = 200.0 / 3, min_log_hz = 1000.0, min_log_mel = min_log_hz / f_sp, log_step = log(6.4) / 27.0;
  return m >= min_log_mel ? min_log_hz * exp(log_step * (m - min_log_mel)) : m * f_sp;
}

/* Slaney-normalised triangular filterbank [nmels][257], f32 (nemotron-mel.js:80-118). */
void or_mel_filterbank(int nmels, float *fb) {
  double freqs[MEL_NBINS];
  for (int i = 0; i < MEL_NBINS; i++) freqs[i] = (8000.0 * i) / (MEL_NBINS - 1);
  const double mmin = mel_hz_to_mel(0.0), mmax = mel_hz_to_mel(8000.0);
  const int np = nmels + 2;
  double *fpts = (double *)malloc(sizeof(double) * np), *fdiff = (double *)malloc(sizeof(double) * (np - 1));
  for (int i = 0; i < np; i++) fpts[i] = mel_mel_to_hz(mmin + ((mmax - mmin) * i) / (np - 1));
  for (int i = 0; i < np - 1; i++) fdiff[i] = fpts[i + 1] - fpts[i];
  for (int m = 0; m < nmels; m++) {
    const double enorm = 2.0 / (fpts[m + 2] - fpts[m]);
    for (int k = 0; k < MEL_NBINS; k++) {
      const double down = (freqs[k] - fpts[m]) / fdiff[m], up = (fpts[m + 2] - freqs[k]) / fdiff[m + 1];
      const double v = down < up ? down : up;
      fb[m * MEL_NBINS + k] = (float)((v > 0 ? v : 0) * enorm);
    }
  }
  free(fpts);
  free(fdiff);
}

/* Symmetric 400-point Hann window zero-padded to 512 (nemotron-mel.js:141-151). */
void or_mel_hann(double *w) {
  for (int i = 0; i < MEL_NFFT; i++) w[i] = 0;
  for (int n = 0; n < MEL_WIN; n++) w[56 + n] = 0.5 * (1 - cos((2 * M_PI * n) / (MEL_WIN - 1)));
}

/* cos/sin of -2*pi*i/n, i < n/2 (nemotron-mel.js:163-176). */
void or_mel_twiddles(int n, double *c, double *s) {
  for (int i = 0; i < n / 2; i++) {
    const double a = (-2 * M_PI * i) / n;
    c[i] = cos(a);
    s[i] = sin(a);
  }
}

/* In-place radix-2 DIT FFT with the reference's stage structure: bit
 * reversal, explicit stages of length 2, 4 and 8 (constants (1,0), (0,-1),
 * (+-SQRT1_2, -SQRT1_2)), then table twiddles (nemotron-mel.js:199-330). */
static void mel_fft(double *re, double *im, int n, const double *tc, const double *ts) {
  int bits = 0;
  while ((1 << bits) < n) bits++;
  for (int i = 0; i < n; i++) {
    int x = i, r = 0;
    for (int b = 0; b < bits; b++) {
      r = (r << 1) | (x & 1);
      x >>= 1;
    }
    if (i < r) {
      double t = re[i]; re[i] = re[r]; re[r] = t;
      t = im[i]; im[i] = im[r]; im[r] = t;
    }
  }
#define BFLY(p, q, tr, ti) do { re[q] = re[p] - (tr); im[q] = im[p] - (ti); re[p] += (tr); im[p] += (ti); } while (0)
  for (int i = 0; i < n; i += 2) { const double tr = re[i + 1], ti = im[i + 1]; BFLY(i, i + 1, tr, ti); }
  for (int i = 0; i < n; i += 4) {
    { const double tr = re[i + 2], ti = im[i + 2]; BFLY(i, i + 2, tr, ti); }
    { const double tr = im[i + 3], ti = -re[i + 3]; BFLY(i + 1, i + 3, tr, ti); }
  }
  const double r2 = 0.70710678118654757; /* Math.SQRT1_2 */
  for (int i = 0; i < n; i += 8) {
    { const double tr = re[i + 4], ti = im[i + 4]; BFLY(i, i + 4, tr, ti); }
    { const double wc = r2, ws = -r2; const int q = i + 5;
      const double tr = re[q] * wc - im[q] * ws, ti = re[q] * ws + im[q] * wc; BFLY(i + 1, q, tr, ti); }
    { const double tr = im[i + 6], ti = -re[i + 6]; BFLY(i + 2, i + 6, tr, ti); }
    { const double wc = -r2, ws = -r2; const int q = i + 7;
      const double tr = re[q] * wc - im[q] * ws, ti = re[q] * ws + im[q] * wc; BFLY(i + 3, q, tr, ti); }
  }
  for (int len = 16; len <= n; len <<= 1) {
    const int half = len >> 1, step = n / len;
    for (int i = 0; i < n; i += len)
      for (int k = 0; k < half; k++) {
        const double wc = tc[k * step], ws = ts[k * step];
        const int p = i + k, q = p + half;
        const double tr = re[q] * wc - im[q] * ws, ti = re[q] * ws + im[q] * wc;
        BFLY(p, q, tr, ti);
      }
  }
#undef BFLY
}

/* Power spectrum (257 bins, f32) of one windowed 512-sample frame `x` (f64):
 * one 256-point complex FFT of the even/odd samples, then the real-spectrum
 * reconstruction (nemotron-mel.js:503-537). */
void or_mel_power(const double *x, float *power) {
  double re[256], im[256], c256[128], s256[128], c512[256], s512[256];
  or_mel_twiddles(256, c256, s256);
  or_mel_twiddles(512, c512, s512);
  for (int k = 0; k < 256; k++) {
    re[k] = x[2 * k];
    im[k] = x[2 * k + 1];
  }
  mel_fft(re, im, 256, c256, s256);
  const double z0r = re[0], z0i = im[0];
  power[0] = (float)((z0r + z0i) * (z0r + z0i));
  power[256] = (float)((z0r - z0i) * (z0r - z0i));
  for (int k = 1; k < 128; k++) {
    const double rk = re[k], ik = im[k], rnk = re[256 - k], ink = im[256 - k];
    const double xer = 0.5 * (rk + rnk), xei = 0.5 * (ik - ink), xor_ = 0.5 * (ik + ink), xoi = -0.5 * (rk - rnk);
    const double wc = c512[k], ws = s512[k];
    const double tr = xor_ * wc - xoi * ws, ti = xor_ * ws + xoi * wc;
    const double xkr = xer + tr, xki = xei + ti, xnr = xer - tr, xni = xei - ti;
    power[k] = (float)(xkr * xkr + xki * xki);
    power[256 - k] = (float)(xnr * xnr + xni * xni);
  }
  power[128] = (float)(re[128] * re[128] + im[128] * im[128]);
}

/* Log-mel features of one mono 16 kHz window (computeRawMel
 * nemotron-mel.js:451-557, then normalizeFeatures :569-603 when `normalize`).
 * out: [nmels][floor(n/160)] f32.  Returns floor(n/160). */
int or_mel(const float *audio, long n, int nmels, double log_guard, int normalize, float *out) {
  const long T = n / MEL_HOP;
  if (n <= 0 || T == 0) return 0;
  const long plen = n + MEL_NFFT;
  double *padded = (double *)calloc(plen, sizeof(double));
  padded[256] = audio[0];
  for (long i = 1; i < n; i++) padded[256 + i] = (float)((double)audio[i] - 0.97 * (double)audio[i - 1]);
  double win[MEL_NFFT], x[MEL_NFFT];
  or_mel_hann(win);
  float *fb = (float *)malloc(sizeof(float) * nmels * MEL_NBINS);
  or_mel_filterbank(nmels, fb);
  int *lo = (int *)malloc(sizeof(int) * nmels), *hi = (int *)malloc(sizeof(int) * nmels);
  for (int m = 0; m < nmels; m++) { /* fbBounds, nemotron-mel.js:401-419 */
    int s = -1, e = -1;
    for (int k = 0; k < MEL_NBINS; k++)
      if (fb[m * MEL_NBINS + k] > 0) {
        if (s < 0) s = k;
        e = k;
      }
    if (s < 0) { s = 0; e = -1; }
    lo[m] = s;
    hi[m] = e + 1;
  }
  float power[MEL_NBINS];
  for (long t = 0; t < T; t++) {
    for (int i = 0; i < MEL_NFFT; i++) x[i] = padded[t * MEL_HOP + i] * win[i];
    or_mel_power(x, power);
    for (int m = 0; m < nmels; m++) {
      double v = 0;
      for (int k = lo[m]; k < hi[m]; k++) v += (double)power[k] * (double)fb[m * MEL_NBINS + k];
      out[m * T + t] = (float)log(v + log_guard);
    }
  }
  if (normalize)
    for (int m = 0; m < nmels; m++) {
      float *r = out + m * T;
      double sum = 0;
      for (long t = 0; t < T; t++) sum += r[t];
      const double mean = sum / T;
      double var = 0;
      for (long t = 0; t < T; t++) {
        const double d = r[t] - mean;
        var += d * d;
      }
      const double inv = T > 1 ? 1.0 / (sqrt(var / (T - 1)) + 1e-5) : 0;
      for (long t = 0; t < T; t++) r[t] = (float)((r[t] - mean) * inv);
    }
  free(padded);
  free(fb);
  free(lo);
  free(hi);
  return (int)T;
}

/* ── greedy TDT decoder ─────────────────────────────────────────────────────
 * rust/parakeet-decoder/src/lib.rs `decode_proj` (:285-318) and its helpers,
 * restated in f32 exactly as the wasm32 code computes them: the decoder's own
 * polynomial expf (:47-54) with its floorf / ldexpf (:55-62), sigmoid / tanhf
 * (:44, :63), 4-lane dot products summed lane by lane (:108-121), the ONNX
 * iofc LSTM step (:124-137), pred projection (:148-162) and the joint over
 * pre-projected frames (:164-217, :220-223).  Weights:
 *   embed [8193][640], lw/lr [2][2560][640] (gate rows i, o, f, c), lb [2][5120]
 *   (W bias then R bias), pred_w [640][640] (k-major), pred_b [640],
 *   out_w [640][8198] (row n = hidden unit), out_b [8198]. */
#define TDT_HID 640
#define TDT_VOCAB 8193
#define TDT_LOGITS 8198
#define TDT_BLANK 8192
#define TDT_MAX_SYMBOLS 10

static float tdt_floorf(float x) {
  const float i = (float)(int)x;
  return i > x ? i - 1.0f : i;
}
static float tdt_ldexpf(float x, int e) {
  float r = x;
  int n = e;
  while (n > 30) { r *= 1073741824.0f; n -= 30; }
  while (n < -30) { r *= 9.313225746154785e-10f; n += 30; }
  union { uint32_t u; float f; } b;
  b.u = (uint32_t)(127 + n) << 23;
  return r * b.f;
}
float or_tdt_expf(float x) {
  const float xc = x > 30.0f ? 30.0f : (x < -30.0f ? -30.0f : x);
  const float t = xc * 1.4426950408889634f;
  const float fl = tdt_floorf(t);
  const float frac = t - fl;
  const float p = 1.0f + frac * (0.6931472f + frac * (0.2402265f + frac * (0.0555041f + frac * 0.0096181f)));
  return tdt_ldexpf(p, (int)fl);
}
static float tdt_sigmoid(float x) { return 1.0f / (1.0f + or_tdt_expf(-x)); }
static float tdt_tanhf(float x) {
  const float e = or_tdt_expf(2.0f * x);
  return (e - 1.0f) / (e + 1.0f);
}
static float tdt_dotv(const float *a, const float *b, int n) {
  float acc[4] = {0, 0, 0, 0};
  int i = 0;
  for (; i + 4 <= n; i += 4)
    for (int l = 0; l < 4; l++) acc[l] = acc[l] + a[i + l] * b[i + l];
  float s = acc[0] + acc[1] + acc[2] + acc[3];
  for (; i < n; i++) s += a[i] * b[i];
  return s;
}

typedef struct {
  const float *embed, *lw[2], *lr[2], *lb[2], *pred_w, *pred_b, *out_w, *out_b;
  float h[2][TDT_HID], c[2][TDT_HID], nh[2][TDT_HID], nc[2][TDT_HID], predproj[TDT_HID], j[TDT_HID], out[TDT_LOGITS];
} tdt_state;

static void tdt_lstm_step(tdt_state *s, int layer, const float *x) {
  const float *w = s->lw[layer], *r = s->lr[layer], *b = s->lb[layer];
  const float *hp = s->h[layer];
  const int H = TDT_HID;
  for (int g = 0; g < H; g++) {
    const int wi = g * H, wo = (H + g) * H, wf = (2 * H + g) * H, wc = (3 * H + g) * H;
    const float zi = b[g] + b[4 * H + g] + tdt_dotv(w + wi, x, H) + tdt_dotv(r + wi, hp, H);
    const float zo = b[H + g] + b[5 * H + g] + tdt_dotv(w + wo, x, H) + tdt_dotv(r + wo, hp, H);
    const float zf = b[2 * H + g] + b[6 * H + g] + tdt_dotv(w + wf, x, H) + tdt_dotv(r + wf, hp, H);
    const float zc = b[3 * H + g] + b[7 * H + g] + tdt_dotv(w + wc, x, H) + tdt_dotv(r + wc, hp, H);
    const float cc = tdt_sigmoid(zf) * s->c[layer][g] + tdt_sigmoid(zi) * tdt_tanhf(zc);
    s->nc[layer][g] = cc;
    s->nh[layer][g] = tdt_sigmoid(zo) * tdt_tanhf(cc);
  }
}
/* predict(token) (:140-145) + compute_predproj (:148-162) */
static void tdt_predict(tdt_state *s, int token) {
  tdt_lstm_step(s, 0, s->embed + (size_t)token * TDT_HID);
  tdt_lstm_step(s, 1, s->nh[0]);
  for (int n = 0; n < TDT_HID; n++) s->predproj[n] = s->pred_b[n];
  for (int k = 0; k < TDT_HID; k++) {
    const float d = s->nh[1][k];
    const float *row = s->pred_w + (size_t)k * TDT_HID;
    for (int n = 0; n < TDT_HID; n++) s->predproj[n] = s->predproj[n] + d * row[n];
  }
}
/* joint_tail over a pre-projected frame (:164-217) */
static void tdt_joint(tdt_state *s, const float *frame) {
  for (int n = 0; n < TDT_HID; n++) {
    const float v = frame[n] + s->predproj[n];
    s->j[n] = v > 0.0f ? v : 0.0f;
  }
  for (int m = 0; m < TDT_LOGITS; m++) s->out[m] = s->out_b[m];
  for (int n = 0; n < TDT_HID; n++) {
    const float jn = s->j[n];
    if (jn == 0.0f) continue;
    const float *row = s->out_w + (size_t)n * TDT_LOGITS;
    for (int m = 0; m < TDT_LOGITS; m++) s->out[m] = s->out[m] + jn * row[m];
  }
}

/* decode_proj: greedy TDT over T pre-projected frames [T][640]; returns the
 * token count, writes ids and their frame indices (at most cap). */
int or_tdt_decode_proj(const float *embed, const float *l0w, const float *l0r, const float *l0b, const float *l1w, const float *l1r,
                       const float *l1b, const float *pred_w, const float *pred_b, const float *out_w, const float *out_b, const float *frames,
                       int T, int32_t *ids, int32_t *fr, int cap) {
  tdt_state *s = (tdt_state *)calloc(1, sizeof(tdt_state));
  s->embed = embed;
  s->lw[0] = l0w; s->lr[0] = l0r; s->lb[0] = l0b;
  s->lw[1] = l1w; s->lr[1] = l1r; s->lb[1] = l1b;
  s->pred_w = pred_w; s->pred_b = pred_b; s->out_w = out_w; s->out_b = out_b;
  int n_out = 0, emitted = 0, t = 0;
  tdt_predict(s, TDT_BLANK);
  while (t < T) {
    tdt_joint(s, frames + (size_t)t * TDT_HID);
    int max_id = 0, step = 0;
    float max_v = -INFINITY, dv = -INFINITY;
    for (int i = 0; i < TDT_VOCAB; i++)
      if (s->out[i] > max_v) { max_v = s->out[i]; max_id = i; }
    for (int i = TDT_VOCAB; i < TDT_LOGITS; i++)
      if (s->out[i] > dv) { dv = s->out[i]; step = i - TDT_VOCAB; }
    if (max_id != TDT_BLANK) {
      memcpy(s->h, s->nh, sizeof s->h); /* commit_state (:146) */
      memcpy(s->c, s->nc, sizeof s->c);
      if (n_out < cap) { ids[n_out] = max_id; fr[n_out] = t; }
      n_out++;
      emitted++;
      tdt_predict(s, max_id);
    }
    if (step > 0) { t += step; emitted = 0; }
    else if (max_id == TDT_BLANK || emitted >= TDT_MAX_SYMBOLS) { t += 1; emitted = 0; }
  }
  free(s);
  return n_out;
}

/* Pieces for the pins: one LSTM step of `layer` from (h, c) with input x ->
 * (nh, nc), and the joint logits of one frame with a given pred projection. */
void or_tdt_lstm(const float *w, const float *r, const float *b, const float *x, const float *h, const float *c, float *nh, float *nc) {
  tdt_state *s = (tdt_state *)calloc(1, sizeof(tdt_state));
  s->lw[0] = w; s->lr[0] = r; s->lb[0] = b;
  memcpy(s->h[0], h, sizeof(float) * TDT_HID);
  memcpy(s->c[0], c, sizeof(float) * TDT_HID);
  tdt_lstm_step(s, 0, x);
  memcpy(nh, s->nh[0], sizeof(float) * TDT_HID);
  memcpy(nc, s->nc[0], sizeof(float) * TDT_HID);
  free(s);
}
void or_tdt_joint(const float *out_w, const float *out_b, const float *frame, const float *predproj, float *logits) {
  tdt_state *s = (tdt_state *)calloc(1, sizeof(tdt_state));
  s->out_w = out_w; s->out_b = out_b;
  memcpy(s->predproj, predproj, sizeof(float) * TDT_HID);
  tdt_joint(s, frame);
  memcpy(logits, s->out, sizeof(float) * TDT_LOGITS);
  free(s);
}
