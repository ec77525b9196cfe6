// A f16 x B int8 GEMM instantiations (kept apart from gemm.hip so
// the kernel templates of each weight format compile in parallel).
#include "gemm_impl.h"

namespace fa {

int gemm_launch_f16a_i8(fa_ctx *ctx, const GemmArgs &p, const char *label) { return launch_kind<A_F16, B_I8>(ctx, p, label); }

}  // namespace fa
