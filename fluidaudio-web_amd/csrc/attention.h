// Fused rel-pos attention launch interface.
#pragma once
#include <stdint.h>

struct fa_ctx;

namespace fa {

// Per-launch window table, passed by value in the kernel arguments so no
// device-side table (and no host->device copy ordering) is involved.
constexpr int kMaxWin = 64;
struct WinTable {
  int n = 0;
  int off[kMaxWin];
  int len[kMaxWin];
};

struct AttnArgs {
  const void *q = nullptr, *k = nullptr, *v = nullptr;  // [rows, ld*] (head h at columns h*HD ..)
  int ldq = 0, ldk = 0, ldv = 0;
  const void *pos = nullptr;  // projected positional table [prows, ldp]
  int ldp = 0, prows = 0;
  int pcenter = 0;            // table row of relative position 0
  const float *pbu = nullptr, *pbv = nullptr;  // [H*HD], 1/sqrt(HD) folded
  void *out = nullptr;        // [rows, ldo]
  void *out_lo = nullptr;     // f16 route, optional: exact remainder plane f16(o - f16(o)), [rows, ldo]
  int ldo = 0;
  WinTable win;               // window row offsets / lengths (by value: no device table)
  int chunk = 0, left = 0, right = 0;  // chunk > 0: query i sees keys [cs - left, cs + chunk - 1 + right], cs = chunk * floor(i / chunk)
  int H = 0, HD = 0;
};

int relpos_attention(fa_ctx *ctx, const AttnArgs &a, int in_f32, int out_f32, int Tmax, const char *label);
// f16 q/k/v/pos/out (the fused encoder): transposes V into vt (capacity
// W * H * 128 * round_up(Tmax, 64) halfs), then the LDS-staged kernel.
// transpose = 0: vt already holds V (written by the q|k|v GEMM's epilogue)
int relpos_attention_f16(fa_ctx *ctx, const AttnArgs &a, int Tmax, _Float16 *vt, const char *label, bool transpose = true);

}  // namespace fa
