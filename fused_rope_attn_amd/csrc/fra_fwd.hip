// fra_fwd.hip -- forward dispatch and the C ABI of libfra.so (include/fra.h):
// argument checks, kernel choice, workspace sizing and launches.  The
// kernels themselves are in fra_fwd_kernels.h, compiled once per head_dim
// by fra_inst_fwd.hip.
#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <mutex>

#include "fra.h"
#include "fra_device.h"
#include "fra_fwd_types.h"

namespace {

using namespace fra_internal;

// ---- host-side dispatch ---------------------------------------------------------

thread_local char g_err[512] = "";

int fail(int code, const char *fmt, ...) __attribute__((format(printf, 2, 3)));
int fail(int code, const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
    return code;
}

// The long kernel's split last round.  Units (segment, head, query block)
// run one workgroup per CU; when the last round of workgroups leaves CUs
// idle, its units are split into up to kSplitMaxParts parts of their key
// range, at least kSplitMinBlocks key blocks each on the longest segment
// (shorter parts lose more to the partial writes and the merge launch than
// the shorter last round gains: measured 8 us slower at 4 and 8 key
// blocks per segment, 16 x 80 heads).  Each part
// writes its unnormalised rows, running max and row sum to the workspace;
// split_merge_kernel, the next launch on the stream, combines them.
//
// The grid has max_seqlen's query blocks for every (segment, head); in a
// layer of unequal segments the blocks past a shorter segment's end exit at
// once, so the rounds are counted from a bound on the blocks that hold
// queries: per head at most ceil(total / 256) + num_seqs.  Layers of equal
// segments (and single segments) meet the bound and plan as before; for the
// six unequal images of a ragged layer (10493 tokens, 16 heads) it is 752 of
// 1056 units, no split, and the call 2.6% faster than with the split that
// the full count asked for (its parts were mostly empty blocks).
struct SplitPlan {
    int64_t units;  // units split (the last round)
    int parts;      // parts per unit (1: no split)
    int64_t bytes;
};
SplitPlan split_plan(int64_t units, const fra_fwd_args *a) {
    SplitPlan sp = {0, 1, 0};
    const int64_t slots = device_cus();
    if (units <= 0) return sp;
    const int d = a->head_dim, max_seqlen = a->max_seqlen;
    const int64_t bound = (int64_t)a->num_heads * (((int64_t)a->total_seq + kLongBQ - 1) / kLongBQ + a->num_seqs);
    units = std::min(units, bound);
    const int64_t rounds = (units + slots - 1) / slots;
    const int64_t tail = units - (rounds - 1) * slots;
    int parts = (int)std::min<int64_t>(slots / tail, kSplitMaxParts);
    parts = std::min(parts, ((max_seqlen + kLongBKV - 1) / kLongBKV) / kSplitMinBlocks);
    if (parts < 2) return sp;
    sp.units = tail;
    sp.parts = parts;
    sp.bytes = split_workspace_bytes(tail, parts, d);
    return sp;
}

// Head dims with compiled kernels (FRA_HEAD_DIMS).
bool pick_kernel(int d, bool window, int hw, bool full, int qkv, int rd, Choice &c) {
    switch (d) {
#define FRA_PICK_CASE(D) \
    case D: pick_d<D>(window, hw, full, qkv, rd, c); return true;
        FRA_HEAD_DIMS(FRA_PICK_CASE)
#undef FRA_PICK_CASE
        default: return false;
    }
}

bool aligned(const void *ptr, int bytes) { return ((uintptr_t)ptr % (uintptr_t)bytes) == 0; }

// Bytes of the k_rot rows the long kernel's PRE variant reads (rounded up to
// 256 so the split scratch after them stays aligned).
int64_t krot_workspace_bytes(const fra_fwd_args *a) {
    return ((int64_t)a->total_seq * a->num_heads * a->head_dim * 2 + 255) / 256 * 256;
}

const char *dtype_name(int dt) {
    switch (dt) {
        case FRA_DTYPE_BF16: return "bf16";
        case FRA_DTYPE_F16: return "f16";
        case FRA_DTYPE_F32: return "f32";
        case kRopePos: return "pos";
        default: return "?";
    }
}

// allow_pre false: the rotated-K part of a workspace is not used (K is
// rotated in the long kernel); all of the workspace may hold split scratch.
// rope non-NULL: the position variant (fra_fwd_varlen_pos); the cos/sin
// fields of args are then ignored.
// rows non-NULL: the row-gather variant (fra_fwd_varlen_gather), window
// layers only.
int plan(const fra_fwd_args *a, Choice &c, KParams &kp, bool allow_pre = true,
         const fra_rope_positions *rope = nullptr, const int32_t *rows = nullptr) {
    if (!a) return fail(FRA_EINVAL, "args is NULL");
    if (a->flags != 0) return fail(FRA_EINVAL, "flags must be 0, got %d", a->flags);
    if (a->num_heads <= 0) return fail(FRA_EINVAL, "num_heads must be positive, got %d", a->num_heads);
    if (a->head_dim <= 0 || a->head_dim % 2 != 0)
        return fail(FRA_EINVAL, "head_dim must be positive and even, got %d", a->head_dim);
    if (a->total_seq < 0) return fail(FRA_EINVAL, "total_seq must be >= 0, got %d", a->total_seq);
    if (a->num_seqs < 1) return fail(FRA_EINVAL, "num_seqs must be >= 1, got %d", a->num_seqs);
    if (a->max_seqlen < 1) return fail(FRA_EINVAL, "max_seqlen must be >= 1, got %d", a->max_seqlen);
    if (a->qkv_dtype != FRA_DTYPE_BF16 && a->qkv_dtype != FRA_DTYPE_F16)
        return fail(FRA_EINVAL, "qkv_dtype must be bf16 or f16, got %d", a->qkv_dtype);
    const bool pos = rope != nullptr;
    const int d = a->head_dim;
    if (pos) {
        if (!rope->pos || !rope->inv_freq) return fail(FRA_EINVAL, "rope positions or inv_freq is NULL");
        if (d % 4) return fail(FRA_EINVAL, "head_dim must be a multiple of 4 for rope positions, got %d", d);
        if (!aligned(rope->pos, 8) || !aligned(rope->inv_freq, 4))
            return fail(FRA_EUNSUPPORTED, "rope positions must be 8-byte aligned and inv_freq 4-byte aligned");
    } else {
        if (a->rope_dtype != FRA_DTYPE_F32 && a->rope_dtype != FRA_DTYPE_BF16 && a->rope_dtype != FRA_DTYPE_F16)
            return fail(FRA_EINVAL, "rope_dtype must be f32, bf16 or f16, got %d", a->rope_dtype);
        if (a->rope_width != d / 2 && a->rope_width != d)
            return fail(FRA_EINVAL, "rope_width must be head_dim/2=%d or head_dim=%d, got %d", d / 2, d, a->rope_width);
    }
    const int rd = pos ? kRopePos : a->rope_dtype;
    const bool full = !pos && a->rope_width == d;
    const int64_t rope_stride = pos ? 0 : a->rope_stride_seq;
    if (!(a->softmax_scale > 0.f) || a->softmax_scale == __builtin_inff())
        return fail(FRA_EINVAL, "softmax_scale must be finite and > 0, got %g", (double)a->softmax_scale);
    if (!a->q || !a->k || !a->v || (!pos && (!a->cos || !a->sin)) || !a->out || !a->cu_seqlens)
        return fail(FRA_EINVAL, "a tensor pointer is NULL");
    const int64_t strides[9] = {a->q_stride_seq, a->q_stride_head, a->k_stride_seq, a->k_stride_head,
                                a->v_stride_seq, a->v_stride_head, a->out_stride_seq, a->out_stride_head,
                                rope_stride};
    for (int i = 0; i < 9; ++i)
        if (strides[i] < 0) return fail(FRA_EINVAL, "strides must be >= 0");

    // The window kernel addresses 64 rows of a tensor with 32-bit offsets.
    const int64_t max_row_bytes = 2 * std::max(std::max(a->q_stride_seq, a->k_stride_seq),
                                               std::max(a->v_stride_seq, a->out_stride_seq));
    const bool small_rows = 64 * max_row_bytes < ((int64_t)1 << 31) && 64 * 4 * rope_stride < ((int64_t)1 << 31);
    // (the gather variant addresses its rows with 64-bit offsets)
    const bool window = a->max_seqlen <= 64 && d <= kWindowMaxD && (small_rows || rows);
    if (rows && !window)
        return fail(FRA_EUNSUPPORTED,
                    "the row gather is for window layers: segments of at most 64 tokens at head_dim <= %d "
                    "(max_seqlen %d, head_dim %d)", kWindowMaxD, a->max_seqlen, d);
    if (rows && !aligned(rows, 4)) return fail(FRA_EINVAL, "row_index must be 4-byte aligned");
    memset(&c, 0, sizeof(c));
    if (!pick_kernel(d, window, kWinHeadsMax, full, a->qkv_dtype, rd, c))
        return fail(FRA_EUNSUPPORTED, "head_dim=%d has no compiled kernel (built:" FRA_HEAD_DIMS_STRING ")", d);
    if (pos && !window && !c.fn_pre)
        return fail(FRA_EUNSUPPORTED, "head_dim=%d has no long kernel for rope positions", d);
    if (!c.fn && !(pos && !window))
        return fail(FRA_EUNSUPPORTED,
                    "%s cos/sin of width %d (rows of %d bytes) cannot be staged by the long kernel, which "
                    "moves table rows in 16-byte chunks; pass float32 tables",
                    dtype_name(a->rope_dtype), a->rope_width, 2 * a->rope_width);
    if (!window) {
        // The long kernel moves K, V and table rows from HBM to LDS in 16-byte
        // chunks, addressing 64 rows of each with 32-bit offsets.
        if (!small_rows)
            return fail(FRA_EUNSUPPORTED, "64 rows of q/k/v/out/cos/sin must span less than 2 GiB");
        const int re = a->rope_dtype == FRA_DTYPE_F32 ? 4 : 2;
        if (!aligned(a->k, 16) || a->k_stride_seq % 8 || a->k_stride_head % 8)
            return fail(FRA_EUNSUPPORTED,
                        "k must be 16-byte aligned with strides that are multiples of 8 elements "
                        "(segments longer than 64 tokens)");
        if (!pos && (!aligned(a->cos, 16) || !aligned(a->sin, 16) || (a->rope_stride_seq * re) % 16))
            return fail(FRA_EUNSUPPORTED,
                        "cos/sin must be 16-byte aligned with a row stride that is a multiple of 16 bytes "
                        "(segments longer than 64 tokens)");
    }

    // Alignment: Q/K/out are read/written in 8-byte quads, V in 16-byte
    // chunks, fp32 tables in 16-byte quads and 16-bit tables in 8-byte quads.
    const int re = a->rope_dtype == FRA_DTYPE_F32 ? 4 : 2;
    if (!aligned(a->q, 8) || !aligned(a->k, 8) || !aligned(a->out, 8) || !aligned(a->v, 16) ||
        (!pos && (!aligned(a->cos, 4 * re) || !aligned(a->sin, 4 * re))))
        return fail(FRA_EUNSUPPORTED, "tensor base pointers are not aligned (q/k/out 8 B, v 16 B, cos/sin %d B)", 4 * re);
    if (a->q_stride_seq % 4 || a->q_stride_head % 4 || a->k_stride_seq % 4 || a->k_stride_head % 4 ||
        a->out_stride_seq % 4 || a->out_stride_head % 4 || a->v_stride_seq % 8 || a->v_stride_head % 8 ||
        rope_stride % 4)
        return fail(FRA_EUNSUPPORTED,
                    "strides must be multiples of 4 elements (q/k/out/cos/sin) and 8 elements (v)");

    kp.q = (const char *)a->q;
    kp.k = (const char *)a->k;
    kp.v = (const char *)a->v;
    kp.cos = (const char *)a->cos;
    kp.sin = (const char *)a->sin;
    kp.out = (char *)a->out;
    kp.cu = a->cu_seqlens;
    kp.sq_s = a->q_stride_seq;
    kp.sq_h = a->q_stride_head;
    kp.sk_s = a->k_stride_seq;
    kp.sk_h = a->k_stride_head;
    kp.sv_s = a->v_stride_seq;
    kp.sv_h = a->v_stride_head;
    kp.so_s = a->out_stride_seq;
    kp.so_h = a->out_stride_head;
    kp.sr_s = rope_stride;
    kp.pos = pos ? rope->pos : nullptr;
    kp.inv_freq = pos ? rope->inv_freq : nullptr;
    kp.rows = rows;
    kp.total = a->total_seq;
    kp.num_heads = a->num_heads;
    kp.num_seqs = a->num_seqs;
    kp.max_seqlen = a->max_seqlen;
    kp.scale_log2 = a->softmax_scale * kLog2e;
    kp.lse = a->lse;
    kp.krot = nullptr;
    if (a->lse && !aligned(a->lse, 4)) return fail(FRA_EINVAL, "lse must be 4-byte aligned");
    if (a->workspace && !aligned(a->workspace, 16)) return fail(FRA_EINVAL, "workspace must be 16-byte aligned");

    const int64_t sh = (int64_t)a->num_seqs * a->num_heads;
    int64_t grid;
    kp.tail_first = 0;
    kp.tail_split = 1;
    kp.ws = nullptr;
    kp.dense_heads = a->q_stride_head == d && a->k_stride_head == d && a->v_stride_head == d && a->out_stride_head == d;
    if (window) {
        // Heads per workgroup.  Two when that grid still runs in one round of
        // resident workgroups (shorter per-workgroup chains: measured 2.6%
        // faster at 144 windows x 16 heads, 4% at 16 windows), else four.
        // One head, its two query tiles on two wavefronts, when there are
        // no more (segment, head) pairs than CUs, where two-head workgroups
        // would leave CUs idle (16 windows x 16 heads: 13.5 against 14.5 us;
        // at 64 windows, four pairs a CU, the duplicated K staging made it
        // 6% slower than two heads).  FRA_WINDOW_HEADS=1, 2 or 4 forces a
        // form that has an instance (tests and tuning).
        int want = 0;
        if (const char *e = getenv("FRA_WINDOW_HEADS")) want = atoi(e);
        if (want != 1 && want != 2 && want != 4) want = 0;
        if (want != 4) {
            const int64_t g2 = (int64_t)a->num_seqs * ((a->num_heads + 1) / 2);
            Choice c2;
            memset(&c2, 0, sizeof(c2));
            pick_kernel(d, true, 2, full, a->qkv_dtype, rd, c2);
            if (c2.fn && (want == 2 || (want == 0 && g2 <= (int64_t)device_cus() * c2.per_cu))) c = c2;
        }
        if (want == 0 || want == 1) {
            Choice c1;
            memset(&c1, 0, sizeof(c1));
            pick_kernel(d, true, 1, full, a->qkv_dtype, rd, c1);
            if (c1.fn && (want == 1 || sh <= (int64_t)device_cus())) c = c1;
        }
        kp.qblocks = 1;
        grid = (int64_t)a->num_seqs * ((a->num_heads + c.heads - 1) / c.heads);
        c.kernel = FRA_KERNEL_WINDOW;
        c.block = 64 * (c.heads == 1 ? 2 : c.heads);
        c.block_q = 64;
        c.block_kv = 64;
        snprintf(c.name, sizeof(c.name), "window_d%d_%s_rope%s%s", d, dtype_name(a->qkv_dtype), dtype_name(rd),
                 rows ? "_gather" : "");
        if (rows) c.fn = c.fn_gather;
    } else {
        kp.qblocks = (a->max_seqlen + kLongBQ - 1) / kLongBQ;
        const int64_t units = sh * kp.qblocks;
        const SplitPlan sp = split_plan(units, a);
        kp.tail_first = (int32_t)std::min<int64_t>(units, 0x7fffffff);
        kp.tail_split = 1;
        // Workspace: [k_rot rows | split scratch].  With room for k_rot the
        // PRE variant runs (krot_kernel first); the rest, if enough, holds
        // the split scratch.  Without it (e.g. sized for the split alone)
        // the kernel stages raw K and rotates it per block.
        const int64_t kr_bytes = krot_workspace_bytes(a);
        int64_t ws_left = a->workspace_bytes;
        kp.ws = (char *)a->workspace;
        c.pre = 0;
        if (allow_pre && a->workspace && a->workspace_bytes >= kr_bytes && c.fn_pre) {
            c.pre = 1;
            c.fn = c.fn_pre;
            c.lds = c.lds_pre;
            kp.krot = (char *)a->workspace;
            kp.ws = (char *)a->workspace + kr_bytes;
            ws_left -= kr_bytes;
        }

        grid = units;
        if (sp.parts > 1 && ws_left >= sp.bytes) {
            kp.tail_first = (int32_t)(units - sp.units);
            kp.tail_split = sp.parts;
            grid = kp.tail_first + sp.units * sp.parts;
            c.split_units = (int)sp.units;
            c.split_parts = sp.parts;
        }
        c.kernel = FRA_KERNEL_LONG;
        c.block = kLongThreads;
        c.block_q = kLongBQ;
        c.block_kv = kLongBKV;
        snprintf(c.name, sizeof(c.name), "long_d%d_%s_rope%s", d, dtype_name(a->qkv_dtype), dtype_name(rd));
    }
    if (grid > 0x7fffffff) return fail(FRA_EUNSUPPORTED, "grid of %lld workgroups is too large", (long long)grid);
    c.grid = (int)grid;
    return FRA_OK;
}

}  // namespace

int fra_fail(int code, const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
    return code;
}

namespace {

// The launches of one planned forward call on `stream`.
int launch(const fra_fwd_args *args, const Choice &c, const KParams &kp, void *stream) {
    g_err[0] = 0;
    if (args->total_seq == 0) return FRA_OK;
    if (c.split_parts > 1 && !args->workspace)
        return fail(FRA_EINVAL, "workspace_bytes is set but workspace is NULL");
    if (c.pre) {
        const int64_t items = (int64_t)args->total_seq * args->num_heads * (args->head_dim / 8);
        const int64_t blocks = (items + 255) / 256;
        if (blocks > 0x7fffffff) return fail(FRA_EUNSUPPORTED, "grid of %lld workgroups is too large", (long long)blocks);
        hipLaunchKernelGGL(c.krot, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream, kp);
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return fail(FRA_EHIP, "launch of the K rotation of %s failed: %s", c.name, hipGetErrorString(e));
    }
    hipLaunchKernelGGL(c.fn, dim3(c.grid), dim3(c.block), 0, (hipStream_t)stream, kp);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(FRA_EHIP, "launch of %s failed: %s", c.name, hipGetErrorString(e));
    if (c.split_parts > 1) {
        hipLaunchKernelGGL(c.merge, dim3(c.split_units * split_merge_blocks(args->head_dim)), dim3(256), 0, (hipStream_t)stream, kp);
        e = hipGetLastError();
        if (e != hipSuccess) return fail(FRA_EHIP, "launch of the merge of %s failed: %s", c.name, hipGetErrorString(e));
    }
    return FRA_OK;
}

// ---- the allocation-free entry point (fra_fwd_varlen_static) ----------------------
//
// Device scratch of fra_fwd_varlen_static(): the partial rows of a split last
// round of the long kernel (per split unit and part, kLongBQ rows of
// split_row_floats(head_dim) floats).  The split never gives more (unit,
// part) pairs than the device has CUs, so with 256 CUs and head_dim <= 128
// the largest need is 256 x 256 x 132 x 4 B = 34.6 MB.  Every device the
// library runs on holds one copy until the process ends.  Nothing in it needs
// to start at zero: each part writes every row the merge reads.
constexpr int64_t kStaticScratchBytes = (int64_t)36 << 20;
static __device__ __align__(256) unsigned char scratch[kStaticScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void *g_scratch_ptr[kMaxDevices];  // device address of `scratch`, per device

// The current device's address of `scratch`, looked up once per device with
// that device current (the array's name is only a host-side handle).
int static_scratch(void **out) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return fail(FRA_EHIP, "hipGetDevice failed: %s", hipGetErrorString(e));
    if (dev < 0 || dev >= kMaxDevices) return fail(FRA_EUNSUPPORTED, "device %d is beyond the %d the library tracks", dev, kMaxDevices);
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void *p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p)
            return fail(FRA_EHIP, "hipGetSymbolAddress of the static scratch failed on device %d: %s", dev,
                        hipGetErrorString(e));
        g_scratch_ptr[dev] = p;
    }
    *out = g_scratch_ptr[dev];
    return FRA_OK;
}

}  // namespace

extern "C" {

int fra_fwd_varlen(const fra_fwd_args *args, void *stream) {
    Choice c;
    KParams kp;
    const int rc = plan(args, c, kp);
    if (rc != FRA_OK) return rc;
    return launch(args, c, kp, stream);
}

int fra_fwd_varlen_static(const fra_fwd_args *args, void *stream) {
    if (!args) return fail(FRA_EINVAL, "args is NULL");
    fra_fwd_args a = *args;
    a.workspace = nullptr;
    a.workspace_bytes = 0;
    Choice c;
    KParams kp;
    int rc = plan(&a, c, kp, false);
    if (rc != FRA_OK) return rc;
    if (c.kernel == FRA_KERNEL_LONG) {
        const SplitPlan sp = split_plan((int64_t)a.num_seqs * a.num_heads * kp.qblocks, &a);
        if (sp.parts > 1) {
            if (sp.bytes > kStaticScratchBytes)
                return fail(FRA_EUNSUPPORTED,
                            "this call needs %lld bytes of scratch, more than the %lld bytes of the library's "
                            "static scratch; use fra_fwd_varlen with a workspace",
                            (long long)sp.bytes, (long long)kStaticScratchBytes);
            rc = static_scratch(&a.workspace);
            if (rc != FRA_OK) return rc;
            a.workspace_bytes = sp.bytes;
            rc = plan(&a, c, kp, false);
            if (rc != FRA_OK) return rc;
        }
    }
    return launch(&a, c, kp, stream);
}

int fra_fwd_varlen_gather(const fra_fwd_args *args, const fra_rope_positions *rope, const int32_t *row_index,
                          void *stream) {
    if (!row_index) return fail(FRA_EINVAL, "row_index is NULL");
    Choice c;
    KParams kp;
    const int rc = plan(args, c, kp, true, rope, row_index);
    if (rc != FRA_OK) return rc;
    return launch(args, c, kp, stream);
}

int fra_fwd_varlen_pos(const fra_fwd_args *args, const fra_rope_positions *rope, void *stream) {
    if (!rope) return fail(FRA_EINVAL, "rope is NULL");
    Choice c;
    KParams kp;
    const int rc = plan(args, c, kp, true, rope);
    if (rc != FRA_OK) return rc;
    if (c.kernel == FRA_KERNEL_LONG && !c.pre)
        return fail(FRA_EUNSUPPORTED,
                    "rope positions on segments longer than 64 tokens need the rotated-K part of a workspace "
                    "(%lld bytes; fra_workspace_bytes_pos)", (long long)krot_workspace_bytes(args));
    return launch(args, c, kp, stream);
}

}  // extern "C"

namespace {

int workspace_bytes(const fra_fwd_args *args, const fra_rope_positions *rope, int64_t *bytes) {
    if (!bytes) return fail(FRA_EINVAL, "bytes is NULL");
    *bytes = 0;
    if (!args) return fail(FRA_EINVAL, "args is NULL");
    fra_fwd_args a = *args;
    a.workspace = nullptr;
    a.workspace_bytes = 0;
    Choice c;
    KParams kp;
    const int rc = plan(&a, c, kp, true, rope);
    if (rc != FRA_OK) return rc;
    if (c.kernel == FRA_KERNEL_LONG) {
        const SplitPlan sp = split_plan((int64_t)a.num_seqs * a.num_heads * kp.qblocks, &a);
        *bytes = krot_workspace_bytes(&a) + (sp.parts > 1 ? sp.bytes : 0);
    }
    g_err[0] = 0;
    return FRA_OK;
}

int query_plan(const fra_fwd_args *args, const fra_rope_positions *rope, fra_plan *out) {
    if (!out) return fail(FRA_EINVAL, "plan is NULL");
    Choice c;
    KParams kp;
    const int rc = plan(args, c, kp, true, rope);
    if (rc != FRA_OK) return rc;
    out->kernel = c.kernel;
    out->grid = c.grid;
    out->block = c.block;
    out->block_q = c.block_q;
    out->block_kv = c.block_kv;
    out->lds_bytes = c.lds;
    out->split_units = c.split_units;
    out->split_parts = c.split_parts;
    memcpy(out->name, c.name, sizeof(out->name));
    g_err[0] = 0;
    return FRA_OK;
}

}  // namespace

extern "C" {

int fra_workspace_bytes(const fra_fwd_args *args, int64_t *bytes) { return workspace_bytes(args, nullptr, bytes); }

int fra_workspace_bytes_pos(const fra_fwd_args *args, const fra_rope_positions *rope, int64_t *bytes) {
    if (!rope) return fail(FRA_EINVAL, "rope is NULL");
    return workspace_bytes(args, rope, bytes);
}

int fra_query_plan_pos(const fra_fwd_args *args, const fra_rope_positions *rope, fra_plan *plan) {
    if (!rope) return fail(FRA_EINVAL, "rope is NULL");
    return query_plan(args, rope, plan);
}

int fra_query_plan(const fra_fwd_args *args, fra_plan *out) { return query_plan(args, nullptr, out); }

int fra_supports_head_dim(int32_t head_dim) {
    Choice c;
    return pick_kernel(head_dim, true, kWinHeadsMax, false, FRA_DTYPE_BF16, FRA_DTYPE_F32, c) ? 1 : 0;
}

const char *fra_last_error(void) { return g_err; }

const char *fra_version(void) { return "fra 0.1.0 (gfx950)"; }

int32_t fra_abi_version(void) { return FRA_ABI_VERSION; }

int32_t fra_sizeof_args(void) { return (int32_t)sizeof(fra_fwd_args); }

int32_t fra_sizeof_plan(void) { return (int32_t)sizeof(fra_plan); }

int32_t fra_sizeof_bwd_args(void) { return (int32_t)sizeof(fra_bwd_args); }

}  // extern "C"
