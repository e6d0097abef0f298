// fra_inst.hip -- the forward and backward kernel instances of one head_dim.
//
// Compiled once per entry of FRA_HEAD_DIMS (fra_fwd_types.h) with
// -DFRA_HEAD_DIM=<D>, so that the instances of different head dims build in
// parallel; the dispatch units (fra_fwd.hip, fra_bwd.hip) reach them through
// pick_d<D> and bwd_kernels_d<D>.
#include "fra_bwd_kernels.h"
#include "fra_fwd_kernels.h"

#ifndef FRA_HEAD_DIM
#error "compile with -DFRA_HEAD_DIM=<head_dim>"
#endif

namespace fra_internal {
template void pick_d<FRA_HEAD_DIM>(bool, int, bool, int, int, Choice &);
template BwdKernels bwd_kernels_d<FRA_HEAD_DIM>(int, bool);
}  // namespace fra_internal
