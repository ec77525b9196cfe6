// Ragged window packing on the GPU.
//
// The reference cuts fixed 15 s windows on the host and transposes each
// window's mel [melBins, T] to [T, melBins] before upload
// (src/engines/asr-parakeet/windowing.js:5-34, raw-encoder.js:181-182), and
// batches only equal-length windows (raw-encoder.js:241).  Here a whole
// feature stream stays resident and one kernel gathers any set of
// variable-length (possibly overlapping) windows into a time-major batch,
// either packed back to back or padded to the longest window.
#include <algorithm>
#include <vector>

#include "fa_internal.h"
#include "fa_device.h"
#include "attention.h"

namespace fa {

// Block = (64-frame tile, 64-channel tile, window).  The 16 loads of a
// thread (feats[c][start + t], coalesced along t) are all issued before the
// tile goes through LDS; the transposed rows leave as float4 stores of four
// channels (coalesced along c).
__global__ __launch_bounds__(256) void pack_windows_kernel(const float *__restrict__ feats, long Ttot, int MB, WinTable dst, WinTable src, int Tpad,
                                                           float *__restrict__ out) {
  __shared__ float tile[64][65];
  const int w = blockIdx.z, t0 = blockIdx.x * 64, c0 = blockIdx.y * 64;
  const int len = dst.len[w];
  const int rows = Tpad > 0 ? Tpad : len;  // padded batches also write zero rows
  if (t0 >= rows) return;
  const long start = src.off[w];
  const int tt = threadIdx.x & 63, cq = threadIdx.x >> 6;
  float v[16];
#pragma unroll
  for (int i = 0; i < 16; i++) {
    const int c = c0 + cq + 4 * i, t = t0 + tt;
    v[i] = (c < MB && t < len && start + t < Ttot) ? feats[(size_t)c * Ttot + start + t] : 0.f;
  }
#pragma unroll
  for (int i = 0; i < 16; i++) tile[cq + 4 * i][tt] = v[i];
  __syncthreads();
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const int e = threadIdx.x + 256 * i, r = e >> 4, c4 = (e & 15) * 4;  // frame t0 + r, channels c0 + c4 .. + 3
    const int c = c0 + c4, t = t0 + r;
    if (c < MB && t < rows)
      *reinterpret_cast<float4 *>(out + (size_t)(dst.off[w] + t) * MB + c) = make_float4(tile[c4][r], tile[c4 + 1][r], tile[c4 + 2][r], tile[c4 + 3][r]);
  }
}

__global__ void row_map_kernel(WinTable st, int rows, int32_t *map) {
  const int r = blockIdx.x * blockDim.x + threadIdx.x;
  if (r >= rows) return;
  int owner = -1;
  for (int w = 0; w < st.n; w++)
    if (r >= st.off[w] && r < st.off[w] + st.len[w]) owner = w;
  map[r] = owner;
}

static inline int s2len(int T) { return T <= 0 ? 0 : (T - 1) / 2 + 1; }

}  // namespace fa

using namespace fa;

extern "C" {

int fa_pack_windows(fa_ctx *ctx, fa_tensor feats, const int32_t *starts, const int32_t *lens, int n, int layout, fa_tensor *out) {
  TensorRec *rf;
  FA_TRY(need(ctx, feats, &rf, "packWindows"));
  if (rf->kind != S_F32) return set_err(ctx, FA_E_INVALID, "packWindows: features must be f32 [melBins, T]");
  if (rf->rows % 4) return set_err(ctx, FA_E_UNSUPPORTED, "packWindows: melBins %d must be a multiple of 4", rf->rows);
  if (n <= 0) return set_err(ctx, FA_E_INVALID, "packWindows: no windows");
  if (layout != 0 && layout != 1) return set_err(ctx, FA_E_INVALID, "packWindows: layout %d", layout);
  const int MB = rf->rows;
  const long Ttot = rf->cols;
  int mx = 0;
  long total = 0;
  for (int i = 0; i < n; i++) {
    if (lens[i] <= 0 || starts[i] < 0 || (long)starts[i] + lens[i] > Ttot)
      return set_err(ctx, FA_E_INVALID, "packWindows: window %d [%d, +%d) outside the %ld-frame stream", i, starts[i], lens[i], Ttot);
    mx = std::max(mx, lens[i]);
    total += lens[i];
  }
  const long rows = layout == 0 ? total : (long)n * mx;
  if (rows > 0x7fffffff) return set_err(ctx, FA_E_INVALID, "packWindows: batch too large");
  fa_tensor o;
  TensorRec *ro;
  FA_TRY(new_tensor(ctx, (int)rows, MB, S_F32, (size_t)rows * MB * 4, &o, &ro));
  TensorGuard og(ctx, o);  // released unless the op completes
  rf = get(ctx, feats);
  ProfScope ps(ctx, "pack_windows", n <= kMaxWin);
  for (int w0 = 0; w0 < n; w0 += kMaxWin) {
    WinTable dst{}, src{};
    dst.n = src.n = std::min(kMaxWin, n - w0);
    long acc = 0;
    for (int i = 0; i < w0; i++) acc += lens[i];
    for (int i = 0; i < dst.n; i++) {
      const int wi = w0 + i;
      dst.off[i] = layout == 0 ? (int)acc : wi * mx;
      dst.len[i] = lens[wi];
      src.off[i] = starts[wi];
      src.len[i] = lens[wi];
      acc += lens[wi];
    }
    FA_LAUNCH(ps, pack_windows_kernel, dim3(cdiv(mx, 64), cdiv(MB, 64), dst.n), dim3(256), 0, ctx->stream, (const float *)rf->ptr, Ttot, MB, dst, src,
                       layout == 1 ? mx : 0, (float *)ro->ptr);
    FA_TRY(check_launch(ctx, "pack_windows"));
  }
  *out = og.release();
  return FA_OK;
}

int fa_window_row_map(fa_ctx *ctx, const int32_t *lens, int n, int layout, int stage, int32_t *host_map, int *rows) {
  if (n <= 0 || n > kMaxWin) return set_err(ctx, FA_E_INVALID, "windowRowMap: %d windows (1..%d)", n, kMaxWin);
  if (stage < 0 || stage > 3 || (layout != 0 && layout != 1)) return set_err(ctx, FA_E_INVALID, "windowRowMap: stage/layout");
  WinTable st{};
  st.n = n;
  int mx = 0;
  for (int i = 0; i < n; i++) {
    int T = lens[i];
    for (int s = 0; s < stage; s++) T = s2len(T);
    st.len[i] = T;
    mx = std::max(mx, T);
  }
  int acc = 0;
  for (int i = 0; i < n; i++) {
    st.off[i] = layout == 0 ? acc : i * mx;
    acc += layout == 0 ? st.len[i] : mx;
  }
  if (rows) *rows = acc;
  if (!host_map) return FA_OK;
  int32_t *d = (int32_t *)dev_alloc(ctx, (size_t)acc * 4 + 4);
  if (!d) return FA_E_OOM;
  hipLaunchKernelGGL(row_map_kernel, dim3(cdiv(acc, 256)), dim3(256), 0, ctx->stream, st, acc, d);
  int st2 = check_launch(ctx, "windowRowMap");
  if (!st2 && acc) {
    hipError_t e = hipMemcpyAsync(host_map, d, (size_t)acc * 4, hipMemcpyDeviceToHost, ctx->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
    if (e != hipSuccess) st2 = set_err(ctx, FA_E_DEVICE, "windowRowMap: %s", hipGetErrorString(e));
  }
  (void)hipStreamSynchronize(ctx->stream);
  (void)hipFree(d);
  return st2;
}

}  // extern "C"
