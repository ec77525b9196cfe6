/*
 * fa_napi.c — thin N-API addon over the C ABI (include/fa_hip.h) for a
 * JavaScript/TypeScript host on Node.  Each export forwards its arguments to
 * one fa_* entry point: contexts and encoders are napi externals, tensor /
 * arena / staged handles are BigInt (0n = none), host arrays are TypedArrays.
 * A non-OK status throws an Error carrying fa_last_error(), as the
 * reference's GpuContext throws on misuse.  hip-context.js builds the
 * ComputeContext class (src/gpu/compute.d.ts) on top of these functions.
 */
#define NAPI_VERSION 8
#include <node_api.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "../../include/fa_hip.h"

#define NA(call)                                                     \
  do {                                                               \
    if ((call) != napi_ok) {                                         \
      napi_throw_error(env, NULL, "fa_hip addon: N-API call failed"); \
      return NULL;                                                   \
    }                                                                \
  } while (0)
#define MAXA 20

static napi_value throw_status(napi_env env, fa_ctx *ctx, int st) {
  const char *m = ctx ? fa_last_error(ctx) : "";
  char buf[600];
  snprintf(buf, sizeof buf, "%s (fa status %d)", (m && *m) ? m : "fa_hip call failed", st);
  napi_throw_error(env, NULL, buf);
  return NULL;
}

static int args(napi_env env, napi_callback_info info, size_t want, napi_value *v) {
  size_t n = MAXA;
  if (napi_get_cb_info(env, info, &n, v, NULL, NULL) != napi_ok) return 0;
  if (n < want) {
    napi_throw_type_error(env, NULL, "fa_hip addon: too few arguments");
    return 0;
  }
  return 1;
}
static void *ext(napi_env env, napi_value v) {
  void *p = NULL;
  napi_get_value_external(env, v, &p);
  return p;
}
static uint64_t big(napi_env env, napi_value v) {
  uint64_t x = 0;
  bool lossless;
  napi_valuetype t;
  napi_typeof(env, v, &t);
  if (t == napi_bigint)
    napi_get_value_bigint_uint64(env, v, &x, &lossless);
  else if (t == napi_number) {
    int64_t i = 0;
    napi_get_value_int64(env, v, &i);
    x = (uint64_t)i;
  }
  return x;
}
static int32_t i32(napi_env env, napi_value v) {
  int32_t x = 0;
  napi_get_value_int32(env, v, &x);
  return x;
}
static double f64(napi_env env, napi_value v) {
  double x = 0;
  napi_get_value_double(env, v, &x);
  return x;
}
static napi_value mkbig(napi_env env, uint64_t x) {
  napi_value r;
  napi_create_bigint_uint64(env, x, &r);
  return r;
}
static size_t typed_el(napi_typedarray_type t) {
  switch (t) {
    case napi_float32_array: case napi_int32_array: case napi_uint32_array: return 4;
    case napi_uint16_array: case napi_int16_array: return 2;
    case napi_float64_array: case napi_bigint64_array: case napi_biguint64_array: return 8;
    default: return 1;
  }
}
static void *typed(napi_env env, napi_value v, size_t *len_bytes) {
  napi_typedarray_type t;
  size_t len, off;
  void *data;
  napi_value ab;
  if (napi_get_typedarray_info(env, v, &t, &len, &data, &ab, &off) != napi_ok) return NULL;
  if (len_bytes) *len_bytes = len * typed_el(t);
  return data;
}

/* A TypedArray of exactly the expected element type (NULL otherwise): the
 * C ABI reinterprets the bytes, so an Int32Array passed where floats are
 * expected must be refused, not reinterpreted. */
static void *typed_as(napi_env env, napi_value v, napi_typedarray_type want, size_t *len_bytes) {
  napi_typedarray_type t;
  size_t len, off;
  void *data;
  napi_value ab;
  if (napi_get_typedarray_info(env, v, &t, &len, &data, &ab, &off) != napi_ok || t != want) return NULL;
  if (len_bytes) *len_bytes = len * typed_el(t);
  return data;
}

/* ── lifecycle ──────────────────────────────────────────────────────────── */
static napi_value js_ctx_create(napi_env env, napi_callback_info info) {
  napi_value a[MAXA];
  if (!args(env, info, 1, a)) return NULL;
  fa_ctx *c = NULL;
  int st = fa_ctx_create(i32(env, a[0]), &c);
  if (st) return throw_status(env, NULL, st);
  napi_value r;
  NA(napi_create_external(env, c, NULL, NULL, &r));
  return r;
}
static napi_value js_ctx_destroy(napi_env env, napi_callback_info info) {
  napi_value a[MAXA];
  if (!args(env, info, 1, a)) return NULL;
  fa_ctx_destroy((fa_ctx *)ext(env, a[0]));
  return NULL;
}
static napi_value js_version(napi_env env, napi_callback_info info) {
  (void)info;
  napi_value r;
  NA(napi_create_string_utf8(env, fa_version(), NAPI_AUTO_LENGTH, &r));
  return r;
}
static napi_value js_sync(napi_env env, napi_callback_info info) {
  napi_value a[MAXA];
  if (!args(env, info, 1, a)) return NULL;
  fa_ctx *c = ext(env, a[0]);
  int st = fa_sync(c);
  return st ? throw_status(env, c, st) : NULL;
}

/* ── tensors ────────────────────────────────────────────────────────────── */
static napi_value up_common(napi_env env, napi_callback_info info, int f16) {
  napi_value a[MAXA];
  if (!args(env, info, 4, a)) return NULL;
  fa_ctx *c = ext(env, a[0]);
  size_t nb = 0;
  float *d = typed_as(env, a[1], napi_float32_array, &nb);
  int rows = i32(env, a[2]), cols = i32(env, a[3]);
  if (!d || nb < (size_t)rows * cols * 4) {
    napi_throw_range_error(env, NULL, "upload: Float32Array shorter than rows*cols");
    return NULL;
  }
  fa_tensor t = 0;
  int st = f16 ? fa_upload_f16(c, d, rows, cols, &t) : fa_upload(c, d, rows, cols, &t);
  return st ? throw_status(env, c, st) : mkbig(env, t);
}
static napi_value js_upload(napi_env env, napi_callback_info info) { return up_common(env, info, 0); }
static napi_value js_upload_f16(napi_env env, napi_callback_info info) { return up_common(env, info, 1); }
static napi_value js_alloc_common(napi_env env, napi_callback_info info, int f16) {
  napi_value a[MAXA];
  if (!args(env, info, 3, a)) return NULL;
  fa_ctx *c = ext(env, a[0]);
  fa_tensor t = 0;
  int st = f16 ? fa_alloc_f16(c, i32(env, a[1]), i32(env, a[2]), &t) : fa_alloc(c, i32(env, a[1]), i32(env, a[2]), &t);
  return st ? throw_status(env, c, st) : mkbig(env, t);
}
static napi_value js_alloc(napi_env env, napi_callback_info info) { return js_alloc_common(env, info, 0); }
static napi_value js_alloc_f16(napi_env env, napi_callback_info info) { return js_alloc_common(env, info, 1); }
static napi_value js_upload_bytes(napi_env env, napi_callback_info info) {
  napi_value a[MAXA];
  if (!args(env, info, 2, a)) return NULL;
  fa_ctx *c = ext(env, a[0]);
  size_t nb = 0;
  void *d = typed(env, a[1], &nb);
  fa_tensor t = 0;
  int st = fa_upload_bytes(c, d, nb, &t);
  return st ? throw_status(env, c, st) : mkbig(env, t);
}
static napi_value js_tensor_info(napi_env env, napi_callback_info info) {
  napi_value a[MAXA];
  if (!args(env, info, 2, a)) return NULL;
  fa_ctx *c = ext(env, a[0]);
  int r = 0, cc = 0, d = 0;
  int st = fa_tensor_info(c, big(env, a[1]), &r, &cc, &d);
  if (st) return throw_status(env, c, st);
  napi_value arr, x;
  NA(napi_create_array_with_length(env, 3, &arr));
  int vals[3] = {r, cc, d};
  for (int i = 0; i < 3; i++) {
    NA(napi_create_int32(env, vals[i], &x));
    NA(napi_set_element(env, arr, i, x));
  }
  return arr;
}
static napi_value js_download(napi_env env, napi_callback_info info) {
  napi_value a[MAXA];
  if (!args(env, info, 3, a)) return NULL;
  fa_ctx *c = ext(env, a[0]);
  int n = i32(env, a[2]);
  void *buf;
  napi_value ab, out;
  NA(napi_create_arraybuffer(env, (size_t)n * 4, &buf, &ab));
  int st = fa_download(c, big(env, a[1]), (float *)buf);
  if (st) return throw_status(env, c, st);
  NA(napi_create_typedarray(env, napi_float32_array, n, ab, 0, &out));
  return out;
}
static napi_value js_stage(napi_env env, napi_callback_info info) {
  napi_value a[MAXA];
  if (!args(env, info, 2, a)) return NULL;
  fa_ctx *c = ext(env, a[0]);
  fa_staged s = 0;
  int st = fa_stage_download(c, big(env, a[1]), &s);
  return st ? throw_status(env, c, st) : mkbig(env, s);
}
static napi_value js_staged_read(napi_env env, napi_callback_info info) {
  napi_value a[MAXA];
  if (!args(env, info, 3, a)) return NULL;
  fa_ctx *c = ext(env, a[0]);
  int n = i32(env, a[2]);
  void *buf;
  napi_value ab, out;
  NA(napi_create_arraybuffer(env, (size_t)n * 4, &buf, &ab));
  int st = fa_staged_read(c, big(env, a[1]), (float *)buf);
  if (st) return throw_status(env, c, st);
  NA(napi_create_typedarray(env, napi_float32_array, n, ab, 0, &out));
  return out;
}

/* handle-in / handle-out helpers for the many simple ops */
#define CTX fa_ctx *c = ext(env, a[0])
#define T(i) big(env, a[i])
#define I(i) i32(env, a[i])
#define RET_T(expr)                                      \
  do {                                                   \
    fa_tensor _o = 0;                                    \
    int _st = (expr);                                    \
    return _st ? throw_status(env, c, _st) : mkbig(env, _o); \
  } while (0)
#define RET_VOID(expr)                                   \
  do {                                                   \
    int _st = (expr);                                    \
    return _st ? throw_status(env, c, _st) : NULL;       \
  } while (0)
#define FN(name, nargs, body)                                      \
  static napi_value name(napi_env env, napi_callback_info info) { \
    napi_value a[MAXA];                                            \
    if (!args(env, info, nargs, a)) return NULL;                   \
    CTX;                                                           \
    body;                                                          \
  }

FN(js_free, 2, RET_VOID(fa_free_tensor(c, T(1))))
FN(js_pin, 3, RET_VOID(fa_pin(c, T(1), I(2))))
FN(js_push_arena, 1, RET_T(fa_push_arena(c, &_o)))
FN(js_pop_arena, 2, RET_VOID(fa_pop_arena(c, T(1))))
FN(js_trim_pool, 2, RET_VOID(fa_trim_pool(c, (size_t)f64(env, a[1]))))
FN(js_rows_view, 3, RET_T(fa_rows_view(c, T(1), I(2), &_o)))
FN(js_begin_batch, 1, RET_VOID(fa_begin_batch(c)))
FN(js_end_batch, 1, RET_VOID(fa_end_batch(c)))
FN(js_matmul, 6, RET_T(fa_matmul(c, T(1), T(2), T(3), I(4), T(5), &_o)))
FN(js_matmul_int8, 8, RET_T(fa_matmul_int8(c, T(1), T(2), T(3), I(4), I(5), T(6), I(7), &_o)))
FN(js_matmul_nbits, 7, RET_T(fa_matmul_nbits(c, T(1), T(2), T(3), T(4), I(5), I(6), &_o)))
FN(js_layernorm, 5, RET_T(fa_layernorm(c, T(1), T(2), T(3), (float)f64(env, a[4]), &_o)))
FN(js_softmax, 2, RET_T(fa_softmax(c, T(1), &_o)))
FN(js_conv1d, 12, RET_T(fa_conv1d(c, T(1), T(2), I(3), I(4), T(5), I(6), I(7), I(8), I(9), I(10), I(11), &_o)))
FN(js_conv2d, 18, RET_T(fa_conv2d(c, T(1), T(2), I(3), I(4), I(5), I(6), I(7), I(8), T(9), I(10), I(11), I(12), I(13), I(14), I(15), I(16), I(17), &_o)))
FN(js_bmm_qk, 8, RET_T(fa_bmm_qk(c, T(1), T(2), T(3), I(4), I(5), I(6), I(7), &_o)))
FN(js_bmm_pv, 6, RET_T(fa_bmm_pv(c, T(1), T(2), I(3), I(4), I(5), &_o)))
FN(js_rel_shift, 2, RET_T(fa_rel_shift(c, T(1), &_o)))
FN(js_rel_shift_b, 3, RET_T(fa_rel_shift_b(c, T(1), I(2), &_o)))
FN(js_rel_shift_stream, 11, RET_T(fa_rel_shift_stream(c, T(1), I(2), I(3), I(4), I(5), I(6), I(7), I(8), I(9), I(10), &_o)))
FN(js_attn_fused, 10, RET_T(fa_attn_fused(c, T(1), T(2), T(3), T(4), T(5), T(6), I(7), I(8), I(9), &_o)))
FN(js_ewise, 4, RET_T(fa_ewise(c, T(1), T(2), I(3), &_o)))
FN(js_scale, 3, RET_T(fa_scale(c, T(1), (float)f64(env, a[2]), &_o)))
FN(js_silu, 2, RET_T(fa_silu(c, T(1), &_o)))
FN(js_relu, 2, RET_T(fa_relu(c, T(1), &_o)))
FN(js_glu, 2, RET_T(fa_glu(c, T(1), &_o)))
FN(js_transpose, 2, RET_T(fa_transpose(c, T(1), &_o)))
FN(js_slice_cols, 4, RET_T(fa_slice_cols(c, T(1), I(2), I(3), &_o)))
FN(js_set_cols, 4, RET_VOID(fa_set_cols(c, T(1), T(2), I(3))))
FN(js_slice_rows, 4, RET_T(fa_slice_rows(c, T(1), I(2), I(3), &_o)))
FN(js_copy_rows, 4, RET_VOID(fa_copy_rows(c, T(1), T(2), I(3))))
FN(js_sub_reshape, 5, RET_T(fa_sub_reshape(c, T(1), I(2), I(3), I(4), &_o)))
FN(js_row_bias_act, 4, RET_T(fa_row_bias_act(c, T(1), T(2), I(3), &_o)))
FN(js_profile_start, 2, RET_VOID(fa_profile_start(c, I(1))))
/* the remaining required ComputeContext members (compute.d.ts:174-234) */
FN(js_leaky_relu, 3, RET_T(fa_leaky_relu(c, T(1), f64(env, a[2]), &_o)))
FN(js_snake, 3, RET_T(fa_snake(c, T(1), T(2), &_o)))
FN(js_adain, 5, RET_T(fa_adain(c, T(1), T(2), T(3), f64(env, a[4]), &_o)))
FN(js_im2col, 6, RET_T(fa_im2col(c, T(1), I(2), I(3), I(4), I(5), &_o)))
FN(js_conv_transpose1d, 12, RET_T(fa_conv_transpose1d(c, T(1), T(2), I(3), I(4), T(5), I(6), I(7), I(8), I(9), I(10), I(11), &_o)))
FN(js_lstm, 6, RET_T(fa_lstm(c, T(1), T(2), T(3), T(4), I(5), &_o)))
FN(js_jbatch, 6, RET_T(fa_jbatch(c, T(1), I(2), I(3), T(4), I(5), &_o)))
FN(js_argmax_rows, 5, RET_T(fa_argmax_rows(c, T(1), I(2), I(3), I(4), &_o)))
FN(js_joint_argmax, 10, RET_T(fa_joint_argmax(c, T(1), I(2), I(3), T(4), T(5), T(6), I(7), I(8), I(9), &_o)))

/* gatherCols(ctx, x, Uint32Array idx) */
static napi_value js_gather_cols(napi_env env, napi_callback_info info) {
  napi_value a[MAXA];
  if (!args(env, info, 3, a)) return NULL;
  CTX;
  size_t nb = 0;
  const uint32_t *idx = typed_as(env, a[2], napi_uint32_array, &nb);
  if (!idx) {
    napi_throw_type_error(env, NULL, "gatherCols: idxMap must be a Uint32Array");
    return NULL;
  }
  fa_tensor o = 0;
  int st = fa_gather_cols(c, T(1), idx, (int)(nb / 4), &o);
  return st ? throw_status(env, c, st) : mkbig(env, o);
}

static napi_value js_concat_rows(napi_env env, napi_callback_info info) {
  napi_value a[MAXA];
  if (!args(env, info, 2, a)) return NULL;
  CTX;
  uint32_t n = 0;
  NA(napi_get_array_length(env, a[1], &n));
  fa_tensor *hs = calloc(n ? n : 1, sizeof *hs);
  for (uint32_t i = 0; i < n; i++) {
    napi_value e;
    NA(napi_get_element(env, a[1], i, &e));
    hs[i] = big(env, e);
  }
  fa_tensor o = 0;
  int st = fa_concat_rows(c, hs, (int)n, &o);
  free(hs);
  return st ? throw_status(env, c, st) : mkbig(env, o);
}

static napi_value js_profile_end(napi_env env, napi_callback_info info) {
  napi_value a[MAXA];
  if (!args(env, info, 1, a)) return NULL;
  CTX;
  int cap = 65536, n = 0;
  char(*labels)[48] = malloc((size_t)cap * 48);
  float *ms = malloc((size_t)cap * sizeof(float));
  int st = fa_profile_end(c, cap, labels, ms, &n);
  if (st) {
    free(labels);
    free(ms);
    return throw_status(env, c, st);
  }
  napi_value arr;
  NA(napi_create_array_with_length(env, (size_t)(n < cap ? n : cap), &arr));
  for (int i = 0; i < n && i < cap; i++) {
    napi_value o, l, m;
    NA(napi_create_object(env, &o));
    NA(napi_create_string_utf8(env, labels[i], NAPI_AUTO_LENGTH, &l));
    NA(napi_create_double(env, ms[i], &m));
    NA(napi_set_named_property(env, o, "label", l));
    NA(napi_set_named_property(env, o, "ms", m));
    NA(napi_set_element(env, arr, (uint32_t)i, o));
  }
  free(labels);
  free(ms);
  return arr;
}

/* ── ragged windows + fused encoder ─────────────────────────────────────── */
static napi_value js_pack_windows(napi_env env, napi_callback_info info) {
  napi_value a[MAXA];
  if (!args(env, info, 5, a)) return NULL;
  CTX;
  size_t nb1 = 0, nb2 = 0;
  int32_t *starts = typed_as(env, a[2], napi_int32_array, &nb1), *lens = typed_as(env, a[3], napi_int32_array, &nb2);
  if (!starts || !lens || nb1 != nb2) {
    napi_throw_type_error(env, NULL, "packWindows: starts/lens must be Int32Arrays of one length");
    return NULL;
  }
  fa_tensor o = 0;
  int st = fa_pack_windows(c, T(1), starts, lens, (int)(nb2 / 4), I(4), &o);
  return st ? throw_status(env, c, st) : mkbig(env, o);
}

/* melWindows(ctx, pcm, starts: Int32Array, lens: Int32Array, nMels, logGuard, normalize) */
static napi_value js_mel_windows(napi_env env, napi_callback_info info) {
  napi_value a[MAXA];
  if (!args(env, info, 7, a)) return NULL;
  CTX;
  size_t nb1 = 0, nb2 = 0;
  int32_t *starts = typed_as(env, a[2], napi_int32_array, &nb1), *lens = typed_as(env, a[3], napi_int32_array, &nb2);
  if (!starts || !lens || nb1 != nb2) {
    napi_throw_type_error(env, NULL, "melWindows: starts/lens must be Int32Arrays of one length");
    return NULL;
  }
  double guard = 0;
  if (napi_get_value_double(env, a[5], &guard) != napi_ok) {
    napi_throw_type_error(env, NULL, "melWindows: logGuard must be a number");
    return NULL;
  }
  fa_tensor o = 0;
  int st = fa_mel_windows(c, T(1), starts, lens, (int)(nb2 / 4), I(4), guard, I(6), &o);
  return st ? throw_status(env, c, st) : mkbig(env, o);
}

/* tdtLoad(ctx, [Float32Array x 11] in the decoder manifest order) -> external */
static napi_value js_tdt_load(napi_env env, napi_callback_info info) {
  napi_value a[MAXA];
  if (!args(env, info, 2, a)) return NULL;
  CTX;
  /* element counts fa_tdt_load reads (the decoder manifest's shapes) */
  static const size_t want[11] = {8193u * 640, 2560u * 640, 2560u * 640, 5120, 2560u * 640, 2560u * 640, 5120, 640u * 640, 640, 640u * 8198, 8198};
  const float *w[11];
  for (uint32_t i = 0; i < 11; i++) {
    napi_value d;
    NA(napi_get_element(env, a[1], i, &d));
    size_t nb = 0;
    w[i] = typed_as(env, d, napi_float32_array, &nb);
    if (!w[i] || nb != want[i] * 4) {
      char m[160];
      snprintf(m, sizeof m, "tdtLoad: weight %u must be a Float32Array of %zu values", i, want[i]);
      napi_throw_type_error(env, NULL, m);
      return NULL;
    }
  }
  fa_tdt *dec = NULL;
  int st = fa_tdt_load(c, w, &dec);
  if (st) return throw_status(env, c, st);
  napi_value r;
  NA(napi_create_external(env, dec, NULL, NULL, &r));
  return r;
}

/* tdtDecode(ctx, dec, frames, Int32Array lens, cap, Int32Array ids, Int32Array frameIdx, Int32Array counts) */
static napi_value js_tdt_decode(napi_env env, napi_callback_info info) {
  napi_value a[MAXA];
  if (!args(env, info, 8, a)) return NULL;
  CTX;
  size_t nl = 0, ni = 0, nf = 0, nc = 0;
  int32_t *lens = typed_as(env, a[3], napi_int32_array, &nl), *ids = typed_as(env, a[5], napi_int32_array, &ni), *fr = typed_as(env, a[6], napi_int32_array, &nf),
          *cnt = typed_as(env, a[7], napi_int32_array, &nc);
  const int n = (int)(nl / 4), cap = I(4);
  if (!lens || !ids || !fr || !cnt || cap <= 0 || ni < (size_t)n * cap * 4 || nf < ni || nc < (size_t)n * 4) {
    napi_throw_type_error(env, NULL, "tdtDecode: lens / ids / frameIdx / counts must be Int32Arrays of n, n*cap, n*cap, n");
    return NULL;
  }
  int st = fa_tdt_decode((fa_tdt *)ext(env, a[1]), T(2), lens, n, cap, ids, fr, cnt);
  if (st) return throw_status(env, c, st);
  napi_value u;
  NA(napi_get_undefined(env, &u));
  return u;
}

static napi_value js_tdt_destroy(napi_env env, napi_callback_info info) {
  napi_value a[MAXA];
  if (!args(env, info, 1, a)) return NULL;
  fa_tdt_destroy((fa_tdt *)ext(env, a[0]));
  napi_value u;
  NA(napi_get_undefined(env, &u));
  return u;
}

static void enc_finalize(napi_env env, void *data, void *hint) {
  (void)env;
  (void)hint;
  (void)data; /* encoders are destroyed explicitly with encoderDestroy */
}

static napi_value js_encoder_load(napi_env env, napi_callback_info info) {
  /* (ctx, Int32Array cfg[9], names[], Float32Array[] data, format, maxT) */
  napi_value a[MAXA];
  if (!args(env, info, 6, a)) return NULL;
  CTX;
  size_t cfb = 0;
  int32_t *cf = typed_as(env, a[1], napi_int32_array, &cfb);
  if (!cf || cfb < 9 * 4) {
    napi_throw_type_error(env, NULL, "encoderLoad: cfg must be an Int32Array of 9 values");
    return NULL;
  }
  fa_encoder_cfg cfg = {cf[0], cf[1], cf[2], cf[3], cf[4], cf[5], cf[6], cf[7], cf[8]};
  uint32_t n = 0;
  NA(napi_get_array_length(env, a[2], &n));
  char **names = calloc(n, sizeof *names);
  const float **data = calloc(n, sizeof *data);
  int64_t *counts = calloc(n, sizeof *counts);
  for (uint32_t i = 0; i < n; i++) {
    napi_value s, d;
    size_t len = 0, nb = 0;
    NA(napi_get_element(env, a[2], i, &s));
    NA(napi_get_value_string_utf8(env, s, NULL, 0, &len));
    names[i] = malloc(len + 1);
    NA(napi_get_value_string_utf8(env, s, names[i], len + 1, &len));
    NA(napi_get_element(env, a[3], i, &d));
    data[i] = typed_as(env, d, napi_float32_array, &nb);
    counts[i] = (int64_t)(nb / 4);
    if (!data[i]) {
      for (uint32_t j = 0; j <= i; j++) free(names[j]);
      free(names);
      free(data);
      free(counts);
      napi_throw_type_error(env, NULL, "encoderLoad: every weight must be a Float32Array");
      return NULL;
    }
  }
  fa_encoder *e = NULL;
  int st = fa_encoder_load(c, &cfg, (int)n, (const char *const *)names, data, counts, I(4), I(5), &e);
  for (uint32_t i = 0; i < n; i++) free(names[i]);
  free(names);
  free(data);
  free(counts);
  if (st) return throw_status(env, c, st);
  napi_value r;
  NA(napi_create_external(env, e, enc_finalize, NULL, &r));
  return r;
}

static napi_value js_encoder_forward(napi_env env, napi_callback_info info) {
  /* (ctx, enc, mel, Int32Array lens, layout, layers) */
  napi_value a[MAXA];
  if (!args(env, info, 6, a)) return NULL;
  CTX;
  size_t nb = 0;
  int32_t *lens = typed_as(env, a[3], napi_int32_array, &nb);
  if (!lens) {
    napi_throw_type_error(env, NULL, "encoderForward: lens must be an Int32Array");
    return NULL;
  }
  fa_tensor o = 0;
  int st = fa_encoder_forward(c, ext(env, a[1]), T(2), lens, (int)(nb / 4), I(4), I(5), &o);
  return st ? throw_status(env, c, st) : mkbig(env, o);
}

static napi_value js_encoder_forward_stream(napi_env env, napi_callback_info info) {
  /* (ctx, enc, feats, Int32Array starts, Int32Array lens, layout, layers) */
  napi_value a[MAXA];
  if (!args(env, info, 7, a)) return NULL;
  CTX;
  size_t nb1 = 0, nb2 = 0;
  int32_t *starts = typed_as(env, a[3], napi_int32_array, &nb1), *lens = typed_as(env, a[4], napi_int32_array, &nb2);
  if (!starts || !lens || nb1 != nb2) {
    napi_throw_type_error(env, NULL, "encoderForwardStream: starts/lens must be Int32Arrays of one length");
    return NULL;
  }
  fa_tensor o = 0;
  int st = fa_encoder_forward_stream(c, ext(env, a[1]), T(2), starts, lens, (int)(nb2 / 4), I(5), I(6), &o);
  return st ? throw_status(env, c, st) : mkbig(env, o);
}

static napi_value js_encoder_forward_stream_batches(napi_env env, napi_callback_info info) {
  /* (ctx, enc, feats, Int32Array starts, Int32Array lens, Int32Array counts, layout, layers) -> [BigInt tensor per batch] */
  napi_value a[MAXA];
  if (!args(env, info, 8, a)) return NULL;
  CTX;
  size_t nb1 = 0, nb2 = 0, nb3 = 0;
  int32_t *starts = typed_as(env, a[3], napi_int32_array, &nb1), *lens = typed_as(env, a[4], napi_int32_array, &nb2);
  int32_t *counts = typed_as(env, a[5], napi_int32_array, &nb3);
  if (!starts || !lens || !counts || nb1 != nb2 || nb3 == 0) {
    napi_throw_type_error(env, NULL, "encoderForwardStreamBatches: starts/lens/counts must be Int32Arrays (starts, lens of one length)");
    return NULL;
  }
  const int nb = (int)(nb3 / 4);
  long total = 0;
  for (int b = 0; b < nb; b++) total += counts[b];
  if (total != (long)(nb2 / 4)) {
    napi_throw_type_error(env, NULL, "encoderForwardStreamBatches: counts must sum to the number of windows");
    return NULL;
  }
  fa_tensor *outs = (fa_tensor *)calloc((size_t)nb, sizeof(fa_tensor));
  if (!outs) {
    napi_throw_error(env, NULL, "encoderForwardStreamBatches: out of host memory");
    return NULL;
  }
  int st = fa_encoder_forward_stream_batches(c, ext(env, a[1]), T(2), nb, starts, lens, counts, I(6), I(7), outs);
  if (st) {
    free(outs);
    return throw_status(env, c, st);
  }
  napi_value arr;
  napi_status ok = napi_create_array_with_length(env, (size_t)nb, &arr);
  for (int b = 0; b < nb && ok == napi_ok; b++) ok = napi_set_element(env, arr, (uint32_t)b, mkbig(env, outs[b]));
  if (ok != napi_ok) {  /* no array reaches the caller: every batch's tensor is released here */
    for (int b = 0; b < nb; b++) (void)fa_free_tensor(c, outs[b]);
    free(outs);
    napi_throw_error(env, NULL, "encoderForwardStreamBatches: building the result array failed");
    return NULL;
  }
  free(outs);
  return arr;
}

static napi_value js_encoder_destroy(napi_env env, napi_callback_info info) {
  napi_value a[MAXA];
  if (!args(env, info, 1, a)) return NULL;
  fa_encoder_destroy(ext(env, a[0]));
  return NULL;
}

static napi_value js_encoder_tsub(napi_env env, napi_callback_info info) {
  napi_value a[MAXA], r;
  if (!args(env, info, 1, a)) return NULL;
  NA(napi_create_int32(env, fa_encoder_tsub(i32(env, a[0])), &r));
  return r;
}

#define EXPORT(js, fn) {js, NULL, fn, NULL, NULL, NULL, napi_default, NULL}

static napi_value init(napi_env env, napi_value exports) {
  napi_property_descriptor d[] = {
      EXPORT("ctxCreate", js_ctx_create), EXPORT("ctxDestroy", js_ctx_destroy), EXPORT("version", js_version), EXPORT("sync", js_sync),
      EXPORT("upload", js_upload), EXPORT("uploadF16", js_upload_f16), EXPORT("alloc", js_alloc), EXPORT("allocF16", js_alloc_f16),
      EXPORT("uploadBytes", js_upload_bytes), EXPORT("tensorInfo", js_tensor_info), EXPORT("download", js_download),
      EXPORT("stageDownload", js_stage), EXPORT("stagedRead", js_staged_read), EXPORT("freeTensor", js_free), EXPORT("pin", js_pin),
      EXPORT("pushArena", js_push_arena), EXPORT("popArena", js_pop_arena), EXPORT("trimPool", js_trim_pool), EXPORT("rowsView", js_rows_view),
      EXPORT("beginBatch", js_begin_batch), EXPORT("endBatch", js_end_batch), EXPORT("matmul", js_matmul), EXPORT("matmulInt8", js_matmul_int8),
      EXPORT("matmulNBits", js_matmul_nbits), EXPORT("layernorm", js_layernorm), EXPORT("softmax", js_softmax), EXPORT("conv1d", js_conv1d),
      EXPORT("conv2d", js_conv2d), EXPORT("bmmQK", js_bmm_qk), EXPORT("bmmPV", js_bmm_pv), EXPORT("relShift", js_rel_shift),
      EXPORT("relShiftB", js_rel_shift_b), EXPORT("relShiftStream", js_rel_shift_stream), EXPORT("attnFused", js_attn_fused), EXPORT("ewise", js_ewise), EXPORT("scale", js_scale),
      EXPORT("silu", js_silu), EXPORT("relu", js_relu), EXPORT("glu", js_glu), EXPORT("transpose", js_transpose),
      EXPORT("sliceCols", js_slice_cols), EXPORT("setCols", js_set_cols), EXPORT("sliceRows", js_slice_rows), EXPORT("copyRows", js_copy_rows),
      EXPORT("concatRows", js_concat_rows), EXPORT("subReshape", js_sub_reshape), EXPORT("rowBiasAct", js_row_bias_act),
      EXPORT("profileStart", js_profile_start), EXPORT("profileEnd", js_profile_end), EXPORT("packWindows", js_pack_windows), EXPORT("melWindows", js_mel_windows),
      EXPORT("encoderLoad", js_encoder_load), EXPORT("encoderForward", js_encoder_forward),
      EXPORT("encoderForwardStream", js_encoder_forward_stream), EXPORT("encoderForwardStreamBatches", js_encoder_forward_stream_batches),
      EXPORT("encoderDestroy", js_encoder_destroy),
      EXPORT("encoderTsub", js_encoder_tsub), EXPORT("tdtLoad", js_tdt_load), EXPORT("tdtDecode", js_tdt_decode), EXPORT("tdtDestroy", js_tdt_destroy),
      EXPORT("leakyRelu", js_leaky_relu), EXPORT("snake", js_snake), EXPORT("adain", js_adain), EXPORT("im2col", js_im2col),
      EXPORT("convTranspose1d", js_conv_transpose1d), EXPORT("gatherCols", js_gather_cols), EXPORT("lstm", js_lstm), EXPORT("jbatch", js_jbatch),
      EXPORT("argmaxRows", js_argmax_rows), EXPORT("jointArgmax", js_joint_argmax),
  };
  napi_define_properties(env, exports, sizeof d / sizeof d[0], d);
  return exports;
}

NAPI_MODULE(NODE_GYP_MODULE_NAME, init)
