// The one-row forward recurrence at four whole slices, gru_fwd_local_kernel<4,
// 1, false, 16, true> (H = 256; sixteen compute wavefronts, one batch row per
// workgroup), in a translation unit of its own: the build compiles this file
// with LLVM's iterative-minreg machine scheduler (-mllvm
// -amdgpu-sched-strategy=iterative-minreg), a per-translation-unit option.
// Measured on MI355X (same box, three alternating pairs, forward per launch):
// c2 409.7-411.4 vs 411.3-415.2 us, c5 (eight chunks) 3192.6-3193.9 vs
// 3221.5-3224.0 us.  Of the other strategies, max-ilp and iterative-ilp
// measured slower on this kernel, and the other recurrence kernels keep the
// default (the four-row kernels measured slower under every other one).
#include "rec_reg_kernels.h"

namespace rka {

const void* rec_fwd1_kernel() { return reinterpret_cast<const void*>(&gru_fwd_local_kernel<4, 1, false, 16, true>); }

}  // namespace rka
