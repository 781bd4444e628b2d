// The one-row backward recurrence's whole-slice instances at three and four
// slices, gru_bwd_local_kernel<S, 1, 16, 1, true> (H = 64 S = 192 or 256;
// sixteen wavefronts, one batch row per workgroup), in a translation unit of
// their own: the build compiles this file with LLVM's max-ilp machine
// scheduler (-mllvm -amdgpu-sched-strategy=max-ilp), a per-translation-unit
// option.  Measured on MI355X (same box, alternating pairs, backward per
// launch): c2 (H = 256) 402.0-406.6 vs 409.6-414.9 us, H = 192 367.3-371.1
// vs 373.1-375.4 us.  Where it measured no faster it is not used: two slices
// (H = 128: 365 vs 347 us), H = 160 (three slices, not whole: 384 vs 381
// us), c5 (four, not whole: no change); it also slows the four-row forward by
// 7 % (c4) and the one-row forward by ~3 us (c2).
#include "rec_reg_kernels.h"

namespace rka {

const void* rec_bwd1_kernel(int slices) {
    return slices == 3 ? reinterpret_cast<const void*>(&gru_bwd_local_kernel<3, 1, 16, 1, true>)
                       : reinterpret_cast<const void*>(&gru_bwd_local_kernel<4, 1, 16, 1, true>);
}

}  // namespace rka
