/*
 * fa_hip.h — C ABI of the MI355X (gfx950) backend for fluidaudio-web's
 * Parakeet FastConformer encoder path.
 *
 * The ABI mirrors the reference's backend contract, `ComputeContext`
 * (src/gpu/compute.d.ts:106-255), restricted to the members the encoder uses,
 * plus one fused whole-encoder entry that replaces the op-by-op
 * `parakeetEncodeBatch` (src/engines/asr-parakeet/raw-encoder.js:235-386).
 * A host binds it through FFI (N-API addon, ctypes); nothing here exposes a
 * C++ or torch type.  Each declaration cites the reference member it replaces.
 *
 * Conventions
 *  - Every call returns FA_OK (0) or an error code; fa_last_error(ctx) then
 *    holds the message (the reference throws an Error with that text).
 *  - Tensors are opaque 64-bit handles (0 = none).  A tensor is a 2-D
 *    row-major matrix {rows, cols}; storage is device memory owned by the
 *    context.  Using a handle after its arena closed or after fa_free_tensor
 *    fails with FA_E_INVALID ("stale tensor handle") instead of touching
 *    recycled memory.
 *  - All work is ordered on the context's single HIP stream, so a later op
 *    always sees the results of earlier ones; only download/staged reads wait.
 *  - Calls are not thread-safe: one host thread drives one context, as one JS
 *    thread drives a GpuContext.
 */
#ifndef FA_HIP_H
#define FA_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct fa_ctx fa_ctx;
typedef struct fa_encoder fa_encoder;
typedef uint64_t fa_tensor; /* 0 = null */
typedef uint64_t fa_arena;  /* 0 = "the newest open arena" */
typedef uint64_t fa_staged;

enum fa_status {
  FA_OK = 0,
  FA_E_INVALID = 1,     /* bad argument, shape mismatch, stale handle */
  FA_E_STATE = 2,       /* misuse: nested batch, second staged read, ... */
  FA_E_DEVICE = 3,      /* HIP runtime error */
  FA_E_OOM = 4,         /* device allocation failed */
  FA_E_UNSUPPORTED = 5  /* shape/format the kernels do not cover */
};

/* Activation codes: src/gpu/kernels/actf.js:24 (ACT). */
enum fa_act { FA_ACT_NONE = 0, FA_ACT_GELU = 1, FA_ACT_TANH = 2, FA_ACT_RELU = 3, FA_ACT_SILU = 4, FA_ACT_GELU_ERF = 5 };

/* Tensor storage kinds reported by fa_tensor_info. */
enum fa_dtype { FA_F32 = 0, FA_F16 = 1, FA_BYTES = 2 };

/* ── lifecycle ───────────────────────────────────────────────────────────────
 * Replaces createContext / new GpuContext(device) (src/gpu/context.js:23-37,
 * src/gpu/compute.js:78) and destroy() (compute.d.ts:133). */
int fa_ctx_create(int device, fa_ctx **out);
void fa_ctx_destroy(fa_ctx *ctx);
const char *fa_last_error(const fa_ctx *ctx);
/* Library version string, e.g. "fa_hip 0.1 gfx950". */
const char *fa_version(void);
/* Wait for all queued work (no reference counterpart; hosts use it before timing). */
int fa_sync(fa_ctx *ctx);

/* ── tensors & memory: compute.d.ts:110-133 ─────────────────────────────────── */
int fa_upload(fa_ctx *ctx, const float *data, int rows, int cols, fa_tensor *out);     /* upload */
int fa_upload_f16(fa_ctx *ctx, const float *data, int rows, int cols, fa_tensor *out); /* uploadF16: f16 storage (RNE) */
int fa_alloc(fa_ctx *ctx, int rows, int cols, fa_tensor *out);                         /* alloc (uninitialised) */
int fa_alloc_f16(fa_ctx *ctx, int rows, int cols, fa_tensor *out);                     /* allocF16 */
/* Row-major f16 activations [rows, cols] (RNE), pool-owned like alloc.  No
 * counterpart in compute.d.ts: a host that keeps activations in f16 feeds them
 * to matmul's f16 x f16 route (A f16, B from uploadF16) with this. */
int fa_upload_f16_rows(fa_ctx *ctx, const float *data, int rows, int cols, fa_tensor *out);
int fa_upload_bytes(fa_ctx *ctx, const void *data, size_t nbytes, fa_tensor *out);     /* uploadBytes (int8/int4 payloads) */
int fa_free_tensor(fa_ctx *ctx, fa_tensor t);                                          /* freeTensor (f16/views ignored) */
int fa_pin(fa_ctx *ctx, fa_tensor t, int to_parent);                                   /* pin */
int fa_push_arena(fa_ctx *ctx, fa_arena *out);                                         /* pushArena */
int fa_pop_arena(fa_ctx *ctx, fa_arena handle);                                        /* popArena (0 = newest) */
int fa_trim_pool(fa_ctx *ctx, size_t budget_bytes);                                    /* trimPool */
int fa_tensor_info(fa_ctx *ctx, fa_tensor t, int *rows, int *cols, int *dtype);
/* Pool telemetry (poolInfo/memStats, compute.d.ts:252-254). */
int fa_pool_info(fa_ctx *ctx, size_t *pooled_bytes, uint64_t *created, uint64_t *created_bytes, uint64_t *reused);

/* ── readback: compute.d.ts:136-145 ─────────────────────────────────────────── */
int fa_download(fa_ctx *ctx, fa_tensor t, float *out);          /* download (rows*cols floats) */
int fa_stage_download(fa_ctx *ctx, fa_tensor t, fa_staged *out); /* stageDownload */
int fa_staged_read(fa_ctx *ctx, fa_staged s, float *out);        /* StagedRead.read (single-use) */
int fa_rows_view(fa_ctx *ctx, fa_tensor t, int rows, fa_tensor *out); /* rowsView */

/* ── batching: compute.d.ts:148-151 ─────────────────────────────────────────── */
int fa_begin_batch(fa_ctx *ctx); /* beginBatch (nesting is FA_E_STATE) */
int fa_end_batch(fa_ctx *ctx);   /* endBatch */
int fa_batch_open(fa_ctx *ctx);  /* 1 when a batch is open */

/* ── linear algebra: compute.d.ts:155-168 ───────────────────────────────────── */
/* matmul: C = act(A[M,K] @ B[K,N] + bias[1,N]) (+ add[M,N]).  B may be f32
 * (fp32 MFMA path) or f16 (A rounded to f16, f16 MFMA, f32 accumulate — the
 * reference's f16-compute route, compute.js:413-416). */
int fa_matmul(fa_ctx *ctx, fa_tensor a, fa_tensor b, fa_tensor bias, int act, fa_tensor add, fa_tensor *out);
/* matmulInt8: wq = int8 [K,N] row-major bytes (4 per u32, gemm.js:679-708),
 * scale [1,N] per output column; out = act(scale[n]·Σ a·q + bias). */
/* C = (A_hi + A_lo) · B (+ bias) (+ add), f32 out: A carried as two exact f16
 * planes (from fa_upload_f16_rows), B an f16 weight tensor; each B fragment
 * feeds two MFMAs.  No counterpart in compute.d.ts: the fused encoder's
 * two-plane operand route, exposed for hosts that need f32-accurate
 * activations against f16 weights.  Needs N % 128 == 0 and K % 64 == 0. */
int fa_matmul_pair(fa_ctx *ctx, fa_tensor a_hi, fa_tensor a_lo, fa_tensor b, fa_tensor bias, fa_tensor add, fa_tensor *out);
int fa_matmul_int8(fa_ctx *ctx, fa_tensor a, fa_tensor wq, fa_tensor scale, int N, int K, fa_tensor bias, int act, fa_tensor *out);
/* matmulNBits: ONNX MatMulNBits (bits=4): bq [N][nblk][16 B], scales f32
 * [N*nblk], zp packed int4 [N][ceil(nblk/2)] (gemm.js:893-919). */
int fa_matmul_nbits(fa_ctx *ctx, fa_tensor a, fa_tensor bq, fa_tensor scales, fa_tensor zp, int N, int block_size, fa_tensor *out);
int fa_layernorm(fa_ctx *ctx, fa_tensor x, fa_tensor gamma, fa_tensor beta, float eps, fa_tensor *out); /* layernorm */
int fa_softmax(fa_ctx *ctx, fa_tensor x, fa_tensor *out);                                               /* softmax */

/* ── convolution: compute.d.ts:172-179 ──────────────────────────────────────── */
/* conv1d: x [Cin, L], w = Cout*(Cin/groups)*K, out [Cout, Lout]. */
int fa_conv1d(fa_ctx *ctx, fa_tensor x, fa_tensor w, int cout, int k, fa_tensor bias, int stride, int pad_left, int pad_right, int dilation,
              int groups, int act, fa_tensor *out);
/* conv2d (batch 1): x [Cin, H*W], w [Cout, Cin/groups, kh, kw] flat, out [Cout, Ho*Wo]. */
int fa_conv2d(fa_ctx *ctx, fa_tensor x, fa_tensor w, int cout, int cin, int h, int wd, int kh, int kw, fa_tensor bias, int stride_h, int stride_w,
              int pad_top, int pad_bottom, int pad_left, int pad_right, int groups, int act, fa_tensor *out);

/* ── attention: compute.d.ts:191-197 ────────────────────────────────────────── */
int fa_bmm_qk(fa_ctx *ctx, fa_tensor q, fa_tensor b, fa_tensor qb, int H, int HD, int W, int b_shared, fa_tensor *out); /* bmmQK */
int fa_bmm_pv(fa_ctx *ctx, fa_tensor p, fa_tensor v, int H, int HD, int W, fa_tensor *out);                          /* bmmPV */
int fa_rel_shift(fa_ctx *ctx, fa_tensor x, fa_tensor *out);                                                           /* relShift */
int fa_rel_shift_b(fa_ctx *ctx, fa_tensor x, int H, fa_tensor *out);                                                  /* relShiftB */
/* relShiftStream (compute.js:689-703, wasm-context.js:509-524): x [H*n, P] -> [H*n, Lk],
 * y[h*n+i, j] = x[h*n+i, clamp(dMax - (q - k), 0, P-1)], q = subT + i, k = subT - Lc + j;
 * -1e4 where k is outside [C*floor(q/C) - left, C*floor(q/C) + C - 1 + right]. */
int fa_rel_shift_stream(fa_ctx *ctx, fa_tensor x, int H, int n, int Lk, int dMax, int Lc, int subT, int C, int left, int right, fa_tensor *out);
/* attnFused (compute.d.ts:248): fused rel-pos attention over W windows of T
 * rows; q/k/v [W*T, H*HD], pos [2T-1, H*HD], pbu/pbv [1, H*HD].  Unlike the
 * reference (T <= 256, compute.js:680) any T up to 1024 is accepted. */
int fa_attn_fused(fa_ctx *ctx, fa_tensor q, fa_tensor k, fa_tensor v, fa_tensor pos, fa_tensor pbu, fa_tensor pbv, int H, int HD, int W,
                  fa_tensor *out);

/* ── elementwise & data movement: compute.d.ts:202-228 ──────────────────────── */
int fa_ewise(fa_ctx *ctx, fa_tensor a, fa_tensor b, int op /*0 add, 1 mul*/, fa_tensor *out); /* ewise/add/mul (b [1,cols] broadcasts) */
int fa_scale(fa_ctx *ctx, fa_tensor x, float s, fa_tensor *out);
int fa_silu(fa_ctx *ctx, fa_tensor x, fa_tensor *out);
int fa_relu(fa_ctx *ctx, fa_tensor x, fa_tensor *out);
int fa_glu(fa_ctx *ctx, fa_tensor x, fa_tensor *out); /* [2C,T] -> [C,T], gate clamped to ±30 (tensor-ops.js:5-19) */
int fa_transpose(fa_ctx *ctx, fa_tensor x, fa_tensor *out);
int fa_slice_cols(fa_ctx *ctx, fa_tensor x, int col0, int width, fa_tensor *out);
int fa_set_cols(fa_ctx *ctx, fa_tensor dst, fa_tensor src, int col0);
int fa_slice_rows(fa_ctx *ctx, fa_tensor x, int row0, int count, fa_tensor *out);
int fa_copy_rows(fa_ctx *ctx, fa_tensor dst, fa_tensor src, int row_offset);
int fa_concat_rows(fa_ctx *ctx, const fa_tensor *ts, int n, fa_tensor *out);
int fa_sub_reshape(fa_ctx *ctx, fa_tensor x, int C, int Tsub, int F, fa_tensor *out); /* subReshape */
int fa_row_bias_act(fa_ctx *ctx, fa_tensor x, fa_tensor bias, int act, fa_tensor *out); /* rowBiasAct (compute.d.ts:249) */

/* ── the other required members: compute.d.ts:174-234, with the CPU backend's
 * arithmetic (src/gpu/wasm-context.js; JS doubles, f32 stores).  Not on the
 * encoder's path: plain kernels so the backend is a complete ComputeContext. */
int fa_leaky_relu(fa_ctx *ctx, fa_tensor x, double slope, fa_tensor *out);             /* leakyRelu (wasm-context.js:406-413) */
int fa_snake(fa_ctx *ctx, fa_tensor x, fa_tensor alpha, fa_tensor *out);              /* snake: x + sin^2(a x)/(a + 1e-9), a per row (:414-427) */
int fa_adain(fa_ctx *ctx, fa_tensor x, fa_tensor scale, fa_tensor shift, double eps, fa_tensor *out); /* adain: per-row instance norm + affine (:344-362) */
/* im2col: x [Cin, L] -> [Cin*k, Lout], Lout = (L + 2 pad - dilation (k-1) - 1)/stride + 1 (:271-285).
 * conv1dGemm / conv1dFast / conv1dFastF16 are compositions of im2col, matmul
 * and conv1d in the host layer, as in the CPU backend (:265-288). */
int fa_im2col(fa_ctx *ctx, fa_tensor x, int k, int stride, int pad, int dilation, fa_tensor *out);
/* convTranspose1d: x [Cin, L], w = Cin*(Cout/groups)*k, out [Cout, Lout],
 * Lout = (L-1) stride - 2 pad + dilation (k-1) + output_padding + 1 (:686-741). */
int fa_conv_transpose1d(fa_ctx *ctx, fa_tensor x, fa_tensor w, int cout, int k, fa_tensor bias, int stride, int pad, int dilation, int groups,
                        int output_padding, int act, fa_tensor *out);
/* gatherCols: out [C, n_idx], out[r, f] = x[r, idx[f]] (host index array; :453-460). */
int fa_gather_cols(fa_ctx *ctx, fa_tensor x, const uint32_t *idx, int n_idx, fa_tensor *out);
/* lstm: bidirectional, batch 1, ONNX gate order i,o,f,c; x [seq, inp],
 * w [2,4H,inp], r [2,4H,H], b [2,8H] -> [seq, 2H]; H <= 256 (:742-776). */
int fa_lstm(fa_ctx *ctx, fa_tensor x, fa_tensor w, fa_tensor r, fa_tensor b, int hid, fa_tensor *out);
/* jbatch: out [B, hid] = relu(enc[base+i, :] + pred) (:564-572). */
int fa_jbatch(fa_ctx *ctx, fa_tensor enc, int base, int B, fa_tensor pred, int hid, fa_tensor *out);
/* argmaxRows: x [B, logits] -> [B, 4] = (token index, token max, duration
 * index, duration max); tokens are columns < vocab, first maximum wins (:573-598). */
int fa_argmax_rows(fa_ctx *ctx, fa_tensor x, int B, int vocab, int logits, fa_tensor *out);
/* jointArgmax: for frames [frame, frame+count): relu(enc + pred) @ outW [hidden, logits]
 * + outB, then argmaxRows -> [count, 4] (:599-633). */
int fa_joint_argmax(fa_ctx *ctx, fa_tensor enc, int frame, int count, fa_tensor pred, fa_tensor outW, fa_tensor outB, int hidden, int vocab,
                    int logits, fa_tensor *out);

/* ── profiling: startProfile/endProfile (compute.d.ts:250-251) ──────────────────
 * While a profile is open every kernel launch is bracketed by HIP events on
 * the context stream.  fa_profile_end waits, then returns up to `cap` records
 * (label, milliseconds) and the number recorded in *count. */
int fa_profile_start(fa_ctx *ctx, int max_ops);
int fa_profile_end(fa_ctx *ctx, int cap, char (*labels)[48], float *ms, int *count);
/* Restrict the open profile to some launches: `filter` is a comma-separated
 * list of exact labels, an entry ending in '*' matching a label prefix
 * (NULL or "" = every launch).  Fewer bracketing events perturb the stream
 * less; this is how a benchmark times one kernel inside a full forward.  No
 * reference counterpart (an extension of startProfile). */
int fa_profile_only(fa_ctx *ctx, const char *filter);

/* ── weight-only quantised formats (no single reference function: the
 * quantiser is scripts/quantize-parakeet-encoder.py:31-36, the dequant
 * raw-encoder.js:64-75; int4 follows MatMulNBits, lib.rs:164-203) ─────────── */
/* Dequantise int8 per-column [K,N] (q·scale[n], exact in f32) into out [K,N] f32. */
int fa_dequant_int8(fa_ctx *ctx, fa_tensor wq, fa_tensor scale, int K, int N, fa_tensor *out);
/* Dequantise symmetric int4 group-32 (bq [N][K/32][16 B], f16 scale bits
 * [N][K/32] as bytes) into out [K,N] f32: (nibble-8)·scale. */
int fa_dequant_int4(fa_ctx *ctx, fa_tensor bq, fa_tensor scales_f16, int K, int N, fa_tensor *out);

/* Host-side quantiser used by fa_encoder_load (no device work, callable
 * without a GPU).  w is the reference's [K, N] ([in, out]) f32 matrix.
 *   format 1 (int8, quantize-parakeet-encoder.py:31-36): q_out int8 K-major
 *     [N][K]; scales_out f32 [N] = f32(max_k|w|)/127 (0 -> 1); q =
 *     clip(rint(w/s), -127, 127).
 *   format 2 (int4 symmetric group-32): q_out [N][ceil(K/32)][16 B], nibble =
 *     q + 8, low nibble = even k (MatMulNBits order, lib.rs:164-203);
 *     scales_out f16 bits [N][ceil(K/32)] = f16(max|w|/7) (0 -> 1.0);
 *     q = clip(rint(w/s), -8, 7); padding nibbles of a partial block encode 0.
 * No reference counterpart for format 2: the reference's int4 path is
 * asymmetric MatMulNBits with f32 scales. */
int fa_quantize_weights(int format, const float *w, int K, int N, void *q_out, void *scales_out);

/* Skinny weight-only GEMV (M <= 64): y [M,N] f32 = a[M,K] (f32) @ W, W int8
 * per-column (scale f32 [N]) or int4 group-32 (f16 scale bits).  format: 1 =
 * int8 ([N][K] K-major bytes), 2 = int4 (bq [N][K/32][16 B]).  The weight
 * layouts are the ones the fused encoder stores (see fa_encoder_load). */
int fa_gemv_quant(fa_ctx *ctx, fa_tensor a, fa_tensor w, fa_tensor scales, int format, int N, int K, fa_tensor *out);
/* `count` independent GEMVs of one shape in one launch per 48 items: item i
 * computes a[i] [M,K] @ W_i (format and layouts as fa_gemv_quant; one M in
 * 1..16 for all items, K a multiple of 128, <= 4096) into rows [i*M, (i+1)*M) of out
 * [count*M, N].  No reference counterpart (the reference issues one matmul
 * per weight, gemm.js:697-706 / 893-919): for callers with many weight
 * buffers ready at once (the q / k / v / FF linears of several streams or
 * layers' independent projections), whose weight streams then run at the
 * HBM rate together instead of one small matrix's launch latency each. */
int fa_gemv_quant_batch(fa_ctx *ctx, int count, const fa_tensor *a, const fa_tensor *w, const fa_tensor *scales, int format, int N, int K,
                        fa_tensor *out);

/* ── ragged window packing (the new batched-window path) ──────────────────────
 * Cuts n windows [start_i, start_i+len_i) out of a channel-major feature
 * stream feats [melBins, Ttotal] (the reference's mel layout,
 * raw-encoder.js:181-182 transposes it per window on the host) and packs
 * them time-major into out.
 *   layout 0 (packed):  out [Σ len_i, melBins], window i at row Σ_{j<i} len_j;
 *   layout 1 (padded):  out [n*Tmax, melBins], window i at row i*Tmax, rows
 *                       past len_i zero-filled; Tmax = max len_i.
 * Windows may overlap in the stream.  starts/lens are host arrays. */
int fa_pack_windows(fa_ctx *ctx, fa_tensor feats, const int32_t *starts, const int32_t *lens, int n, int layout, fa_tensor *out);

/* ── greedy TDT decoding (joint + prediction network + token loop) ───────────
 * Replaces the decoder the pipeline runs after each encoder batch:
 * rust/parakeet-decoder/src/lib.rs decode_proj (:285-318), reached through
 * src/engines/asr-parakeet/raw-decoder-wasm.js, and its WebGPU port
 * gpuDecodeBatch (src/engines/asr-parakeet/gpu-decoder.js:248-273).  Same
 * arithmetic as decode_proj (f32, its polynomial expf, lane-ordered dots), so
 * token ids and frames equal the reference's.
 * fa_tdt_load: w = 11 host f32 arrays in the reference's decoder manifest order
 *   embed [8193*640], l0_W [2560*640], l0_R [2560*640], l0_B [5120], l1_W, l1_R,
 *   l1_B, predW [640*640] (k-major), predB [640], outW [640*8198], outB [8198].
 * fa_tdt_decode: frames = f32 [rows, 640] pre-projected encoder frames (the
 *   joint's encoder projection applied, pipeline.js:57-61), window i = lens[i]
 *   rows after the previous windows' rows; writes up to cap token ids and their
 *   frame indices per window (ids / frame_idx are [n][cap]) and each window's
 *   token count (may exceed cap: the tokens past cap are dropped).  Synchronous. */
typedef struct fa_tdt fa_tdt;
int fa_tdt_load(fa_ctx *ctx, const float *const *w, fa_tdt **out);
void fa_tdt_destroy(fa_tdt *dec);
int fa_tdt_decode(fa_tdt *dec, fa_tensor frames, const int32_t *lens, int n, int cap, int32_t *ids, int32_t *frame_idx, int32_t *counts);
/* Windowed transcription's device stages, pipelined (replaces the group loop
 * of src/engines/asr-parakeet/pipeline.js:32-143 transcribeWindowed with the
 * GPU decoder): n_groups groups of windows of one resident f32 PCM tensor,
 * group g = the next counts[g] (1..32) windows of starts/lens (samples; every
 * window must hold at least one 160-sample mel hop).  Per group: log-mel
 * features (fa_mel_windows with n_mels = the encoder's bins, log_guard,
 * normalize), the encoder forward over the group read in place from them
 * (fa_encoder_forward_stream, packed layout), the joint projection
 * x @ projW (+ projB) (f32 [D, 640], [640]; fa_matmul's f32 route), and the
 * greedy TDT decode (fa_tdt_decode with capacity cap).  Group g+1's mel,
 * encoder and projection are queued on an encoder lane before group g
 * decodes on the context stream, so they overlap; the results equal the
 * stage-by-stage calls bit for bit.  Outputs per window w (in plan order):
 * ids / frame_idx [w * cap, +cap), n_out[w] (tokens emitted, may exceed cap),
 * tsub[w] (encoder frames).  Buffers are the call's own (two groups' worth);
 * the call returns when everything it queued has finished. */
int fa_transcribe_groups(fa_ctx *ctx, fa_encoder *enc, fa_tdt *dec, fa_tensor pcm, int n_groups, const int32_t *counts, const int32_t *starts,
                         const int32_t *lens, fa_tensor projW, fa_tensor projB, int n_mels, double log_guard, int normalize, int cap, int32_t *ids,
                         int32_t *frame_idx, int32_t *n_out, int32_t *tsub);

/* ── log-mel front end (PCM windows -> the feature stream above) ─────────────
 * Replaces ParakeetMel.process (src/engines/asr-parakeet/parakeet-mel.js:14-22)
 * applied to each window slice of the sample stream, as the pipeline's mel
 * scheduler does (src/engines/asr-parakeet/mel-scheduler.js:8-21); the
 * arithmetic is JsPreprocessor.computeRawMel + normalizeFeatures
 * (src/engines/asr-nemotron/nemotron-mel.js:451-603): pre-emphasis 0.97,
 * symmetric 400-point Hann window in a 512-point f64 FFT, hop 160, slaney
 * filterbank, log(mel + log_guard), then (normalize = 1) per-feature
 * mean / (std + 1e-5) over the window's frames.
 *   pcm:   f32 tensor holding the mono 16 kHz sample stream (any shape; read flat);
 *   window i = samples [starts[i], starts[i] + lens[i]) (may overlap);
 *   out:   f32 [n_mels, Σ floor(lens[i]/160)], window i's features at column
 *          Σ_{j<i} floor(lens[j]/160): the channel-major stream fa_pack_windows
 *          reads.  A window shorter than 160 samples contributes no column (the
 *          reference returns length 0 and the scheduler drops it).
 * n_mels 1..128 (Parakeet 128); log_guard 2^-24 (Parakeet) or 1e-10 with
 * normalize 0 (Nemotron's raw log-mel, its first floor(len/160) frames). */
int fa_mel_windows(fa_ctx *ctx, fa_tensor pcm, const int32_t *starts, const int32_t *lens, int n, int n_mels, double log_guard, int normalize,
                   fa_tensor *out);
/* fa_mel_windows for callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, hosts that forbid hipMalloc).  No
 * counterpart in the reference.  Same arguments and results as
 * fa_mel_windows, but the PCM (nsamp f32 samples) and the output
 * (f32 [n_mels][out_cols], out_cols = Σ floor(lens[i]/160)) are device
 * pointers the caller owns, and nothing is allocated: the constant tables and
 * the per-(window, bin) statistics live in one static device array of
 * 273,920 bytes per GPU (held until the process ends), set up by
 * fa_ctx_create.  Limits: n <= 64 windows per call (FA_E_UNSUPPORTED above),
 * n_mels <= 128.  The first call with an n_mels other than 128 on a device
 * uploads that bin count's tables with a synchronous copy (make it outside
 * graph capture).  Every call on a GPU shares the array, so it serves one
 * context per GPU at a time: the first context that calls it owns it until
 * that context is destroyed, and calls from another context on the same GPU
 * return FA_E_STATE; the owner's calls are ordered on its stream. */
int fa_mel_windows_static(fa_ctx *ctx, const float *pcm, int64_t nsamp, const int32_t *starts, const int32_t *lens, int n, int n_mels,
                          double log_guard, int normalize, float *out, int64_t out_cols);
/* Row -> window index map of a batch (the index map every window-aware kernel
 * uses), computed on the device and copied to host_map: entry r is the window
 * owning row r, or -1 for a padding row.  stage 0 = mel frames, 1..3 = after
 * each stride-2 subsampling conv (3 = encoder frames).  Call with host_map ==
 * NULL to get the row count in *rows first. */
int fa_window_row_map(fa_ctx *ctx, const int32_t *lens, int n, int layout, int stage, int32_t *host_map, int *rows);

/* ── fused encoder: loadParakeetEncoder + parakeetEncodeBatch
 * (raw-encoder.js:39-161, 235-386) ────────────────────────────────────────── */
typedef struct fa_encoder_cfg {
  int D, DFF, H, HD, layers, dwK, Csub, Fsub, melBins;
} fa_encoder_cfg;

/* Model options of the streaming FastConformer variants (EOU / Nemotron
 * configs, src/engines/asr-parakeet/raw-encoder.js:187-219,250-280,361-364):
 *   sub_pad_*    pads of the three stride-2 subsampling convs (Parakeet: 1,1,1,1;
 *                EOU: t2 b1 l2 r1); the frequency bins after the front end
 *                follow from melBins and the left/right pads;
 *   conv_causal  depthwise conv padded (K-1, 0) instead of ((K-1)/2, (K-1)/2);
 *   att_chunk    > 0: query i sees keys [cs - att_left, cs + att_chunk - 1 +
 *                att_right], cs = att_chunk * floor(i / att_chunk) (0 = all keys).
 * A layer whose manifest has "L<i>_bnw" / "L<i>_bnb" normalises the depthwise
 * output with that LayerNorm before its SiLU (raw-encoder.js:361-364). */
typedef struct fa_encoder_opts {
  int sub_pad_t, sub_pad_b, sub_pad_l, sub_pad_r;
  int conv_causal;
  int att_chunk, att_left, att_right;
} fa_encoder_opts;

/* Weight storage formats for the encoder's linears. */
enum fa_weight_format { FA_W_F16 = 0, FA_W_INT8 = 1, FA_W_INT4 = 2 };

/* Load weights given as manifest entries (name, f32 data, element count); the
 * names are the reference manifest's ("c0w", "linw", "L3_ff1w1", ...).  The
 * load-time folds of raw-encoder.js:124-156 (q·1/√HD, pos_bias·1/√HD, FF
 * linear2·0.5) are applied here.  `format` picks the storage of the layer
 * linears: f16, int8 per-output-channel (quantize-parakeet-encoder.py:31-36)
 * or int4 symmetric group-32 with f16 scales; dequant is fused into the GEMM
 * loads.  max_T bounds the subsampled window length (frames per window after
 * the 8x front end) the encoder will accept (<= 1024). */
int fa_encoder_load(fa_ctx *ctx, const fa_encoder_cfg *cfg, int n, const char *const *names, const float *const *data, const int64_t *counts,
                    int format, int max_T, fa_encoder **out);
/* fa_encoder_load with model options (NULL = the offline Parakeet defaults:
 * pads 1, symmetric depthwise conv, full attention).  The options shape every
 * forward of the encoder and the streams created on it. */
int fa_encoder_load_opts(fa_ctx *ctx, const fa_encoder_cfg *cfg, const fa_encoder_opts *opts, int n, const char *const *names,
                         const float *const *data, const int64_t *counts, int format, int max_T, fa_encoder **out);
void fa_encoder_destroy(fa_encoder *enc);

/* Operand precision per conformer layer.  The f16 route rounds five kinds of
 * GEMM/conv operands to f16; each bit below instead carries that operand as
 * an exact f16 pair (hi = f16(v), lo = f16(v - hi)) feeding two MFMAs per
 * weight fragment, or (FA_EXACT_GLU) keeps it f32.  No counterpart in the
 * reference (its f16 route keeps f16 partial sums, gemm.js:380-391); this is
 * how the f16 encoder holds the fp32 path's frame-wise decisions.  Every
 * weight format takes every mask.  Default: attention / GLU / depthwise
 * outputs exact in every layer; in the last 8 layers also the LayerNorm
 * outputs, and for int8 / int4 weights the FF hidden state too.
 * Layers [first, last] get `mask`. */
enum fa_exact_bits {
  FA_EXACT_LN_OUT = 1,    /* LayerNorm outputs -> FF W1, q|k|v, pw1 */
  FA_EXACT_FF_HIDDEN = 2, /* FF hidden (after SiLU) -> FF W2 */
  FA_EXACT_ATTN_OUT = 4,  /* attention output -> out-projection */
  FA_EXACT_GLU = 8,       /* GLU output -> depthwise conv (f32) */
  FA_EXACT_DW_OUT = 16    /* depthwise conv output -> pw2 */
};
int fa_encoder_set_exact(fa_encoder *enc, int first_layer, int last_layer, unsigned mask);
/* Current mask of one layer (or -1 for an invalid layer). */
int fa_encoder_get_exact(const fa_encoder *enc, int layer);

/* Encode a batch of windows.  mel: [Σ len_i, melBins] (layout 0) or
 * [n*Tmax, melBins] (layout 1) time-major f32 rows as fa_pack_windows makes
 * them; lens: host mel-frame lengths.  out receives [Σ Tsub_i, D] (layout 0)
 * or [n*TsubMax, D] (layout 1, rows past a window's Tsub are zero) f32
 * frames.  Each window's frames equal its standalone encode: attention keys,
 * the depthwise conv and the subsampling convs never cross window bounds.
 * 1 <= n <= 32 (FA_E_UNSUPPORTED above: the largest batch validated on the GPU).
 * layers_run < 0 runs all layers. */
int fa_encoder_forward(fa_ctx *ctx, fa_encoder *enc, fa_tensor mel, const int32_t *lens, int n, int layout, int layers_run, fa_tensor *out);
/* The same encode with the windows read in place from the channel-major
 * feature stream feats [melBins, T] (fa_mel_windows' output, the layout
 * fa_pack_windows reads): window i = columns [starts[i], starts[i]+lens[i]).
 * out equals fa_encoder_forward(fa_pack_windows(feats, starts, lens, layout))
 * bit for bit, with no packed copy made.  Replaces the per-window transpose
 * + encoder call of the reference's encode path (raw-encoder.js:181-182,
 * pipeline.js:74).  Windows may overlap; starts/lens are host arrays. */
int fa_encoder_forward_stream(fa_ctx *ctx, fa_encoder *enc, fa_tensor feats, const int32_t *starts, const int32_t *lens, int n, int layout,
                              int layers_run, fa_tensor *out);
/* nb batches of one feature stream: batch b = the next counts[b] windows of
 * starts/lens, outs[b] = fa_encoder_forward_stream of that batch, bit for bit.
 * Consecutive batches run on two workspace lanes with streams of their own,
 * so one batch's kernel tails and write-backs overlap the next batch's
 * kernels; the lanes start after the work queued on the context stream and
 * the context stream waits for both.  On failure every outs[b] is 0 (batches
 * already encoded are released).  Replaces the loop over window groups
 * of the reference's windowed transcription (pipeline.js:66-80). */
int fa_encoder_forward_stream_batches(fa_ctx *ctx, fa_encoder *enc, fa_tensor feats, int nb, const int32_t *starts, const int32_t *lens,
                                      const int32_t *counts, int layout, int layers_run, fa_tensor *outs);
/* Subsampled length of a window of T mel frames (raw-encoder.js:217-218). */
int fa_encoder_tsub(int T);
/* The same for this encoder's subsampling pads. */
int fa_encoder_tsub_of(const fa_encoder *enc, int T);

/* ── streaming encoder: createEncodeStream / encodeStreamPush /
 * encodeStreamFlush / disposeEncodeStream
 * (src/engines/asr-parakeet/streaming-encoder.js:33-182) ──────────────────
 * A stream runs chunk passes of the fused encoder with the K / V and
 * depthwise-conv caches kept on the device; its frames are those of the
 * offline chunked-causal encoder (fa_encoder_forward on the same encoder).
 * enc: loaded with att_chunk > 0, conv_causal and sub_pad_t 2 (the streaming
 * models), max_T > att_left + att_chunk.  lookahead_chunks: provisional
 * right-context chunks recomputed each pass (>= 1 when att_right > 0; error
 * against offline frames shrinks as it grows).  max_chunk: frames per pass
 * (att_chunk .. 128).
 * fa_stream_push: mel = host f32 [melBins][count] (mel-major); runs every pass
 * the buffered frames allow; *out = the new frames [n, D] (f32), or 0 when
 * none are final yet.  fa_stream_flush: encodes the tail with the bottom pad;
 * the stream accepts no push afterwards (FA_E_STATE). */
typedef struct fa_stream fa_stream;
int fa_stream_create(fa_ctx *ctx, fa_encoder *enc, int lookahead_chunks, int max_chunk, fa_stream **out);
int fa_stream_push(fa_stream *st, const float *mel, int count, fa_tensor *out);
/* Push to n distinct streams of one encoder in one call: stream i gets
 * mels[i] (counts[i] frames) and outs[i] as fa_stream_push would give it.
 * Streams whose next passes have the same shape run as one batched pass (up
 * to 16 streams, the weights read once for all); other groups run at the same
 * time on the encoder's stream lanes (HIP streams with workspaces of their
 * own).  The lanes start after the work queued on the context stream, and the
 * context stream waits for all of them.  Frames equal solo pushes bit for bit
 * while a batched pass has at most 16 rows; from 17 to 32 rows the K range of
 * the GEMMs is split over workgroups and summed in split order, and beyond 32
 * rows the tiled GEMMs sum in their order: within the encoder's tolerance and
 * deterministic for a given grouping, but a stream's bits then depend on
 * which other streams had a pass ready in the same call.  On failure every
 * outs[i] is 0 and the pushed frames stay queued in each stream: a failure
 * before a stream's pass was queued (sizes, allocations) leaves it as it was,
 * and its next push emits the frames of both pushes; a stream whose pass had
 * been queued in this call (its caches moved, its frames discarded with the
 * error) is marked failed, and every later push or flush of it returns
 * FA_E_STATE.  The reference serves one stream per encodeStreamPush
 * (streaming-encoder.js:182-297); this is that call for n streams at once. */
int fa_stream_push_many(int n, fa_stream *const *sts, const float *const *mels, const int *counts, fa_tensor *outs);
int fa_stream_flush(fa_stream *st, fa_tensor *out);
void fa_stream_destroy(fa_stream *st);

#ifdef __cplusplus
}
#endif
#endif /* FA_HIP_H */
