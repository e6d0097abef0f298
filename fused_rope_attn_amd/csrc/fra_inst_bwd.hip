// fra_inst_bwd.hip -- the backward kernel instances of one head_dim.
//
// Compiled once per entry of FRA_HEAD_DIMS (fra_fwd_types.h) with
// -DFRA_HEAD_DIM=<D>; the dispatch unit (fra_bwd.hip) reaches them through
// bwd_kernels_d<D>.
#include "fra_bwd_kernels.h"

#ifndef FRA_HEAD_DIM
#error "compile with -DFRA_HEAD_DIM=<head_dim>"
#endif

namespace fra_internal {
template BwdKernels bwd_kernels_d<FRA_HEAD_DIM>(int, bool);
}  // namespace fra_internal
