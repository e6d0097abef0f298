// fra_bwd_types.h -- backward types shared by the dispatch (fra_bwd.hip) and
// the per-head_dim kernel instances (fra_inst_bwd.hip).
#pragma once

#include <stdint.h>

#include "fra_fwd_types.h"

#pragma GCC visibility push(hidden)
namespace fra_internal {

// Kernel parameters, passed by value.  Strides are in elements.
struct BParams {
    const char *q, *k, *v, *cos, *sin, *out, *dout;
    const float *lse;
    const int32_t *cu;
    char *dq, *dk, *dv;
    float *dvec;  // [num_heads, total]: rowsum(dout * out)
    char *qr, *kr;  // longer segments: q_rot, k_rot ([total, num_heads, head_dim], storage dtype)
    int64_t sq_s, sq_h, sk_s, sk_h, sv_s, sv_h, so_s, so_h, sdo_s, sdo_h;
    int64_t sdq_s, sdq_h, sdk_s, sdk_h, sdv_s, sdv_h, sr_s;
    int32_t total, num_heads, num_seqs;
    int32_t blocks;    // row blocks per (segment, head) of the dq and dk/dv units
    float scale;       // softmax_scale
    float scale_log2;  // softmax_scale * log2(e)
};

typedef void (*BwdFn)(BParams);

struct BwdKernels {
    BwdFn dot, rotate, matrix;  // longer segments: Dvec, q_rot / k_rot, then dq and dk/dv units
    int nw;
    BwdFn window;       // every segment <= 64 tokens: the one-pass kernel, V staged
    BwdFn window_vreg;  // ... V in registers (four workgroups per CU where three fit otherwise)
    int per_cu, per_cu_vreg;
};

// Backward kernel instances of one head_dim (defined in fra_bwd_kernels.h,
// instantiated by fra_inst_bwd.hip for every entry of FRA_HEAD_DIMS).
template <int D> BwdKernels bwd_kernels_d(int qkv, bool full);
#define FRA_EXTERN_BWD_D(D) extern template BwdKernels bwd_kernels_d<D>(int, bool);
FRA_HEAD_DIMS(FRA_EXTERN_BWD_D)
#undef FRA_EXTERN_BWD_D

}  // namespace fra_internal
#pragma GCC visibility pop
