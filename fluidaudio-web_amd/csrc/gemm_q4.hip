// A f16 x B int4 group-32 GEMM instantiations (kept apart from gemm.hip so
// the kernel templates of each weight format compile in parallel).
#include "gemm_impl.h"

namespace fa {

int gemm_launch_f16a_i4(fa_ctx *ctx, const GemmArgs &p, const char *label) { return launch_kind<A_F16, B_I4>(ctx, p, label); }

}  // namespace fa
