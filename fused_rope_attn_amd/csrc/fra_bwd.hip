// fra_bwd.hip -- backward dispatch and its part of the C ABI (include/fra.h).
// The kernels are in fra_bwd_kernels.h, compiled once per head_dim by
// fra_inst_bwd.hip; see there for the arithmetic.
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include <algorithm>

#include "fra.h"
#include "fra_device.h"
#include "fra_bwd_types.h"

namespace {

using namespace fra_internal;

bool bwd_pick(int d, int qkv, bool full, BwdKernels &k) {
    switch (d) {
#define FRA_BWD_CASE(D) \
    case D: k = bwd_kernels_d<D>(qkv, full); return true;
        FRA_HEAD_DIMS(FRA_BWD_CASE)
#undef FRA_BWD_CASE
        default: return false;
    }
}


bool aligned_to(const void *ptr, int bytes) { return ((uintptr_t)ptr % (uintptr_t)bytes) == 0; }

// Scratch of the longer-segment path: Dvec ([H, N] fp32, padded to 256
// bytes), then q_rot and k_rot ([N, H, D] in the storage dtype).  The
// one-pass window kernel needs none.
int64_t bwd_ws_dvec_bytes(const fra_bwd_args *a) { return ((int64_t)a->num_heads * a->total_seq * 4 + 255) / 256 * 256; }
int64_t bwd_ws_rot_bytes(const fra_bwd_args *a) { return (int64_t)a->total_seq * a->num_heads * a->head_dim * 2; }
int64_t bwd_ws_bytes(const fra_bwd_args *a) {
    return a->max_seqlen <= 64 ? 0 : bwd_ws_dvec_bytes(a) + 2 * bwd_ws_rot_bytes(a);
}

int bwd_check(const fra_bwd_args *a) {
    if (!a) return fra_fail(FRA_EINVAL, "args is NULL");
    if (a->flags != 0) return fra_fail(FRA_EINVAL, "flags must be 0, got %d", a->flags);
    if (a->num_heads <= 0) return fra_fail(FRA_EINVAL, "num_heads must be positive, got %d", a->num_heads);
    if (a->head_dim <= 0 || a->head_dim % 2 != 0)
        return fra_fail(FRA_EINVAL, "head_dim must be positive and even, got %d", a->head_dim);
    if (a->total_seq < 0) return fra_fail(FRA_EINVAL, "total_seq must be >= 0, got %d", a->total_seq);
    if (a->num_seqs < 1) return fra_fail(FRA_EINVAL, "num_seqs must be >= 1, got %d", a->num_seqs);
    if (a->max_seqlen < 1) return fra_fail(FRA_EINVAL, "max_seqlen must be >= 1, got %d", a->max_seqlen);
    if (a->qkv_dtype != FRA_DTYPE_BF16 && a->qkv_dtype != FRA_DTYPE_F16)
        return fra_fail(FRA_EINVAL, "qkv_dtype must be bf16 or f16, got %d", a->qkv_dtype);
    if (a->rope_dtype != FRA_DTYPE_F32 && a->rope_dtype != FRA_DTYPE_BF16 && a->rope_dtype != FRA_DTYPE_F16)
        return fra_fail(FRA_EINVAL, "rope_dtype must be f32, bf16 or f16, got %d", a->rope_dtype);
    const int d = a->head_dim;
    if (a->rope_width != d / 2 && a->rope_width != d)
        return fra_fail(FRA_EINVAL, "rope_width must be head_dim/2=%d or head_dim=%d, got %d", d / 2, d,
                        a->rope_width);
    if (!(a->softmax_scale > 0.f) || a->softmax_scale == __builtin_inff())
        return fra_fail(FRA_EINVAL, "softmax_scale must be finite and > 0, got %g", (double)a->softmax_scale);
    if (!a->q || !a->k || !a->v || !a->cos || !a->sin || !a->out || !a->dout || !a->lse || !a->cu_seqlens ||
        !a->dq || !a->dk || !a->dv)
        return fra_fail(FRA_EINVAL, "a tensor pointer is NULL");
    const int64_t st[19] = {a->q_stride_seq,    a->q_stride_head,  a->k_stride_seq,    a->k_stride_head,
                            a->v_stride_seq,    a->v_stride_head,  a->out_stride_seq,  a->out_stride_head,
                            a->dout_stride_seq, a->dout_stride_head, a->dq_stride_seq, a->dq_stride_head,
                            a->dk_stride_seq,   a->dk_stride_head, a->dv_stride_seq,   a->dv_stride_head,
                            a->rope_stride_seq, 0, 0};
    for (int i = 0; i < 17; ++i)
        if (st[i] < 0) return fra_fail(FRA_EINVAL, "strides must be >= 0");
    BwdKernels k;
    if (!bwd_pick(d, a->qkv_dtype, a->rope_width == d, k))
        return fra_fail(FRA_EUNSUPPORTED, "head_dim=%d has no compiled kernel (built:" FRA_HEAD_DIMS_STRING ")", d);
    if (a->rope_dtype != FRA_DTYPE_F32)
        return fra_fail(FRA_EUNSUPPORTED, "the backward takes float32 cos/sin tables, got %s",
                        a->rope_dtype == FRA_DTYPE_BF16 ? "bf16" : "f16");
    const void *t16[8] = {a->q, a->k, a->v, a->out, a->dout, a->dq, a->dk, a->dv};
    for (int i = 0; i < 8; ++i)
        if (!aligned_to(t16[i], 16))
            return fra_fail(FRA_EUNSUPPORTED, "q/k/v/out/dout/dq/dk/dv must be 16-byte aligned");
    for (int i = 0; i < 16; ++i)
        if (st[i] % 8)
            return fra_fail(FRA_EUNSUPPORTED,
                            "q/k/v/out/dout/dq/dk/dv strides must be multiples of 8 elements");
    if (!aligned_to(a->cos, 16) || !aligned_to(a->sin, 16) || a->rope_stride_seq % 4)
        return fra_fail(FRA_EUNSUPPORTED,
                        "cos/sin must be 16-byte aligned with a row stride that is a multiple of 4 elements");
    if (!aligned_to(a->lse, 4)) return fra_fail(FRA_EINVAL, "lse must be 4-byte aligned");
    return FRA_OK;
}

// Which backward kernels fra_bwd_varlen() launches for checked arguments.
// Window layers: the staged one-pass kernel, or its register-V instance where
// the fourth workgroup per CU makes the grid fit one round that three do
// not.  Longer segments: row dots, rotation, then the dq / dk,dv kernel.
struct BwdChoice {
    BwdKernels k;
    bool window, vreg;
    int64_t grid;  // workgroups of the main kernel
    int block;     // its threads per workgroup
};
int bwd_choose(const fra_bwd_args *a, BwdChoice &c) {
    const int d = a->head_dim;
    bwd_pick(d, a->qkv_dtype, a->rope_width == d, c.k);
    const int64_t sh = (int64_t)a->num_seqs * a->num_heads;
    c.window = a->max_seqlen <= 64;
    c.vreg = false;
    if (c.window) {
        const int64_t cus = device_cus();
        c.vreg = c.k.window_vreg && sh > cus * c.k.per_cu && sh <= cus * c.k.per_cu_vreg;
        c.grid = sh;
        c.block = 128;
    } else {
        const int rows_per_wg = 32 * c.k.nw;
        c.grid = 2 * sh * ((a->max_seqlen + rows_per_wg - 1) / rows_per_wg);
        c.block = 64 * c.k.nw;
    }
    if (c.grid > 0x7fffffff)
        return fra_fail(FRA_EUNSUPPORTED, "grid of %lld workgroups is too large", (long long)c.grid);
    return FRA_OK;
}

}  // namespace

extern "C" {

int fra_bwd_query_plan(const fra_bwd_args *args, fra_plan *out) {
    if (!out) return fra_fail(FRA_EINVAL, "plan is NULL");
    int rc = bwd_check(args);
    if (rc != FRA_OK) return rc;
    BwdChoice c;
    rc = bwd_choose(args, c);
    if (rc != FRA_OK) return rc;
    memset(out, 0, sizeof(*out));
    out->kernel = c.window ? FRA_KERNEL_WINDOW : FRA_KERNEL_LONG;
    out->grid = (int32_t)c.grid;
    out->block = c.block;
    out->block_q = c.window ? 64 : 32 * c.k.nw;
    out->block_kv = 64;
    snprintf(out->name, sizeof(out->name), "bwd_%s_d%d_%s", c.window ? (c.vreg ? "window_vreg" : "window") : "long",
             args->head_dim, args->qkv_dtype == FRA_DTYPE_BF16 ? "bf16" : "f16");
    return fra_fail(FRA_OK, "%s", "");
}

int fra_bwd_workspace_bytes(const fra_bwd_args *args, int64_t *bytes) {
    if (!bytes) return fra_fail(FRA_EINVAL, "bytes is NULL");
    *bytes = 0;
    const int rc = bwd_check(args);
    if (rc != FRA_OK) return rc;
    *bytes = bwd_ws_bytes(args);
    return fra_fail(FRA_OK, "%s", "");
}

int fra_bwd_varlen(const fra_bwd_args *a, void *stream) {
    int rc = bwd_check(a);
    if (rc != FRA_OK) return rc;
    if (a->total_seq == 0) return fra_fail(FRA_OK, "%s", "");
    if (bwd_ws_bytes(a) > 0 && (!a->workspace || a->workspace_bytes < bwd_ws_bytes(a) || !aligned_to(a->workspace, 16)))
        return fra_fail(FRA_EINVAL, "workspace must be 16-byte aligned and hold at least %lld bytes",
                        (long long)bwd_ws_bytes(a));
    const int d = a->head_dim;
    BwdChoice ch;
    rc = bwd_choose(a, ch);
    if (rc != FRA_OK) return rc;
    const BwdKernels &k = ch.k;

    BParams p;
    memset(&p, 0, sizeof(p));
    p.q = (const char *)a->q;
    p.k = (const char *)a->k;
    p.v = (const char *)a->v;
    p.cos = (const char *)a->cos;
    p.sin = (const char *)a->sin;
    p.out = (const char *)a->out;
    p.dout = (const char *)a->dout;
    p.lse = a->lse;
    p.cu = a->cu_seqlens;
    p.dq = (char *)a->dq;
    p.dk = (char *)a->dk;
    p.dv = (char *)a->dv;
    p.dvec = (float *)a->workspace;
    p.qr = (char *)a->workspace + bwd_ws_dvec_bytes(a);
    p.kr = p.qr + bwd_ws_rot_bytes(a);
    p.sq_s = a->q_stride_seq;
    p.sq_h = a->q_stride_head;
    p.sk_s = a->k_stride_seq;
    p.sk_h = a->k_stride_head;
    p.sv_s = a->v_stride_seq;
    p.sv_h = a->v_stride_head;
    p.so_s = a->out_stride_seq;
    p.so_h = a->out_stride_head;
    p.sdo_s = a->dout_stride_seq;
    p.sdo_h = a->dout_stride_head;
    p.sdq_s = a->dq_stride_seq;
    p.sdq_h = a->dq_stride_head;
    p.sdk_s = a->dk_stride_seq;
    p.sdk_h = a->dk_stride_head;
    p.sdv_s = a->dv_stride_seq;
    p.sdv_h = a->dv_stride_head;
    p.sr_s = a->rope_stride_seq;
    p.total = a->total_seq;
    p.num_heads = a->num_heads;
    p.num_seqs = a->num_seqs;
    p.scale = a->softmax_scale;
    p.scale_log2 = a->softmax_scale * kLog2e;

    const hipStream_t st = (hipStream_t)stream;
    const int64_t rows = (int64_t)a->total_seq * a->num_heads;
    const int64_t sh = (int64_t)a->num_seqs * a->num_heads;
    if (ch.window) {
        p.blocks = 1;
        hipLaunchKernelGGL(ch.vreg ? k.window_vreg : k.window, dim3((unsigned)sh), dim3(128), 0, st, p);
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess)
            return fra_fail(FRA_EHIP, "launch of the window backward kernel failed: %s", hipGetErrorString(e));
        return fra_fail(FRA_OK, "%s", "");
    }
    const int rows_per_wg = 32 * k.nw;
    const int64_t blocks = (a->max_seqlen + rows_per_wg - 1) / rows_per_wg;
    const int64_t grid_dot = (rows + 255) / 256, grid = ch.grid;
    if (grid_dot > 0x7fffffff)
        return fra_fail(FRA_EUNSUPPORTED, "grid of %lld workgroups is too large", (long long)grid_dot);
    p.blocks = (int32_t)blocks;
    const int64_t grid_rot = (rows * (d / 8) + 255) / 256;
    if (grid_rot > 0x7fffffff) return fra_fail(FRA_EUNSUPPORTED, "grid of %lld workgroups is too large", (long long)grid_rot);
    hipLaunchKernelGGL(k.dot, dim3((unsigned)grid_dot), dim3(256), 0, st, p);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fra_fail(FRA_EHIP, "launch of the backward row dot products failed: %s", hipGetErrorString(e));
    hipLaunchKernelGGL(k.rotate, dim3((unsigned)grid_rot), dim3(256), 0, st, p);
    e = hipGetLastError();
    if (e != hipSuccess) return fra_fail(FRA_EHIP, "launch of the backward rotation failed: %s", hipGetErrorString(e));
    hipLaunchKernelGGL(k.matrix, dim3((unsigned)grid), dim3(64 * k.nw), 0, st, p);
    e = hipGetLastError();
    if (e != hipSuccess) return fra_fail(FRA_EHIP, "launch of the dq / dk,dv kernel failed: %s", hipGetErrorString(e));
    return fra_fail(FRA_OK, "%s", "");
}

}  // extern "C"
