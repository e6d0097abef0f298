// fra_inst_fwd.hip -- the forward kernel instances of one head_dim.
//
// Compiled once per entry of FRA_HEAD_DIMS (fra_fwd_types.h) with
// -DFRA_HEAD_DIM=<D>, so that the instances of different head dims build in
// parallel; the dispatch unit (fra_fwd.hip) reaches them through pick_d<D>.
#include "fra_fwd_kernels.h"

#ifndef FRA_HEAD_DIM
#error "compile with -DFRA_HEAD_DIM=<head_dim>"
#endif

namespace fra_internal {
template void pick_d<FRA_HEAD_DIM>(bool, int, bool, int, int, Choice &);
}  // namespace fra_internal
