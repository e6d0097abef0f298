// fra_fwd_types.h -- forward types and constants shared by the dispatch
// (fra_fwd.hip) and the per-head_dim kernel instances (fra_inst_fwd.hip, fra_inst_bwd.hip).
#pragma once

#include <stdint.h>

#include "fra.h"

// Head dims with compiled kernels.  fra_inst_fwd.hip and fra_inst_bwd.hip are compiled once per entry
// with -DFRA_HEAD_DIM=<D> (fused_rope_attn_amd/build.py reads this list);
// each must be a multiple of 8 so that both halves of a row start on an
// 8-byte boundary.  A build may pass its own list (-D'FRA_HEAD_DIMS(X)=...')
// to compile fewer instances.
#ifndef FRA_HEAD_DIMS
#define FRA_HEAD_DIMS(X) X(64) X(72) X(80) X(96) X(128)
#endif
#define FRA_HEAD_DIM_STR(D) " " #D
#define FRA_HEAD_DIMS_STRING FRA_HEAD_DIMS(FRA_HEAD_DIM_STR)  // " 64 72 ..." for messages

#pragma GCC visibility push(hidden)
namespace fra_internal {

// Kernel parameters, passed by value.  Strides are in elements.
// Kernel parameters, passed by value.  Strides are in elements.
struct KParams {
    const char *q, *k, *v, *cos, *sin;
    char *out;
    const int32_t *cu;
    int64_t sq_s, sq_h, sk_s, sk_h, sv_s, sv_h, so_s, so_h, sr_s;
    int32_t total, num_heads, num_seqs, max_seqlen;
    int32_t qblocks;      // long kernel: query blocks per (segment, head)
    // Long kernel, split last round: units (segment, head, query block) from
    // tail_first on are split into tail_split parts of their key range; the
    // parts' partial results go to ws.
    int32_t tail_first, tail_split;
    char *ws;
    int32_t dense_heads;  // window kernel: q, k, v and out have head stride == head_dim
    float scale_log2;     // softmax_scale * log2(e)
    float *lse;           // optional [num_heads, total] natural-log row sums (NULL: not written)
    char *krot;           // long kernel, PRE variant: k_rot rows [total, num_heads, head_dim] (workspace)
    // Rope from positions (fra_fwd_varlen_pos): (h, w) int32 per token and
    // head_dim/4 inverse frequencies; cos/sin are then unused.
    const int32_t *pos;
    const float *inv_freq;
    // Window kernel, gather variant (fra_fwd_varlen_gather): tensor row of
    // every slot of cu_seqlens' index space (NULL: the slot itself).
    const int32_t *rows;
};

// Internal rope "dtype" of the position variant: the kernels compute cos/sin
// from KParams::pos and ::inv_freq (table width head_dim / 2).
constexpr int kRopePos = 3;

typedef void (*KernelFn)(KParams);

constexpr int kWinHeadsMax = 4;  // window kernel: heads (wavefronts) per workgroup, at most
// The window kernel keeps the Q_rot and K_rot operands of 64 tokens in
// registers; above this head_dim the long kernel serves short segments too.
constexpr int kWindowMaxD = 96;

constexpr int kLongWaves = 8;
constexpr int kLongBQ = 32 * kLongWaves;  // query rows per workgroup
constexpr int kLongBKV = 64;              // key/value rows per stage
constexpr int kLongThreads = 64 * kLongWaves;

// Split last round of the long kernel (see split_plan in fra_fwd.hip).
// Workspace: per (split unit, part), kLongBQ rows of split_row_floats(D) floats:
// O (unnormalised, head_dim values), m (running max in scale*log2e units) and
// l (row sum of P).
constexpr int kSplitMaxParts = 8;
constexpr int kSplitMinBlocks = 8;  // key blocks per part, at least

__host__ __device__ constexpr int split_row_floats(int d) { return (d + 2 + 3) / 4 * 4; }  // 16-byte pitch

// Workgroups (of 256 threads, one per (row, 8 columns)) of the merge per unit.
__host__ __device__ constexpr int split_merge_blocks(int d) { return (kLongBQ * (d / 8) + 255) / 256; }

inline int64_t split_workspace_bytes(int64_t units, int parts, int d) {
    return units * parts * kLongBQ * (int64_t)split_row_floats(d) * 4;
}

struct Choice {
    KernelFn fn;
    KernelFn merge;   // split_merge_kernel of the long kernel's instance
    KernelFn fn_pre;  // long kernel, PRE variant (K rotated beforehand by krot)
    KernelFn krot;    // krot_kernel of the instance
    KernelFn fn_gather;  // window kernel: the row-gather instance
    int lds_pre;
    int pre;          // the plan uses fn_pre and krot
    int kernel, grid, block, block_q, block_kv, lds, split_units, split_parts;
    int heads;       // window kernel: heads (wavefronts) per workgroup
    int per_cu;      // window kernel: workgroups resident per CU
    char name[64];
};

// Kernel instances of one head_dim (defined in fra_fwd_kernels.h,
// instantiated by fra_inst_fwd.hip): fills c.fn (and the long kernel's merge,
// PRE and krot instances) for a window (hw heads per workgroup) or long
// layer; c.fn stays NULL when the combination has no kernel.
template <int D> void pick_d(bool window, int hw, bool full, int qkv, int rd, Choice &c);
#define FRA_EXTERN_PICK_D(D) extern template void pick_d<D>(bool, int, bool, int, int, Choice &);
FRA_HEAD_DIMS(FRA_EXTERN_PICK_D)
#undef FRA_EXTERN_PICK_D

}  // namespace fra_internal
#pragma GCC visibility pop
