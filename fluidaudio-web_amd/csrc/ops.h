// Launch helpers shared between translation units.
#pragma once
#include <stdint.h>

struct fa_ctx;

namespace fa {

int layernorm_launch(fa_ctx *ctx, const float *x, const float *g, const float *b, void *y, int out_f16, int rows, int cols, int ldx, int ldy,
                     float eps, const char *label);
int gemv_quant_launch(fa_ctx *ctx, const float *A, const void *W, const void *scales, int format, int M, int N, int K, float *Y, const float *bias,
                      int act, const char *label);
}  // namespace fa
