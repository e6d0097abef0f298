/*
 * fra.h -- C ABI of the MI355X (gfx950) fused RoPE + varlen attention library
 * (libfra.so).
 *
 * The library replaces the device side of the reference's one hot path:
 *
 *   reference fused_attn.py:218-231  the launch of fused_attn_kernel[grid](...)
 *   reference fused_attn.py:235-423  the Triton kernel itself
 *
 * The Python entry point fused_rope_attention() of the reference
 * (fused_attn.py:139-232) is mirrored one level up, in
 * fused_rope_attn_amd/fused_attn.py, and calls fra_fwd_varlen() below.
 *
 * Conventions
 *   - Plain C: POD arguments, device pointers, element strides, int status.
 *   - No C++ exception crosses this boundary; every entry point returns a
 *     status code and leaves a message for fra_last_error().
 *   - All work is enqueued on the caller's HIP stream; nothing is
 *     synchronised, nothing is allocated, no global state is mutated, so the
 *     calls are reentrant and capturable into a HIP graph.  Device memory
 *     beyond the tensors (the long kernel's optional workspace) is passed in
 *     by the caller.
 *   - Tensors are [total_seq, num_heads, head_dim] with unit stride on
 *     head_dim; the two outer strides are free (packed qkv views work).
 */
#ifndef FRA_H
#define FRA_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define FRA_ABI_VERSION 3

/* Element types. */
enum fra_dtype {
    FRA_DTYPE_BF16 = 0,
    FRA_DTYPE_F16 = 1,
    FRA_DTYPE_F32 = 2
};

/* Status codes (0 = success, negative = failure). */
enum fra_status {
    FRA_OK = 0,
    FRA_EINVAL = -1,        /* invalid argument: null pointer, bad shape, enum or stride */
    FRA_EUNSUPPORTED = -2,  /* valid request this build does not implement (head_dim, alignment) */
    FRA_EHIP = -3           /* the HIP runtime reported an error at launch */
};

/* Kernel families chosen by the dispatcher. */
enum fra_kernel {
    FRA_KERNEL_NONE = 0,
    FRA_KERNEL_WINDOW = 1,  /* every segment <= 64 tokens: one (segment, head) per wavefront */
    FRA_KERNEL_LONG = 2     /* split-Q flash tiling over K/V blocks staged in LDS */
};

/*
 * Arguments of one forward call.  Mirrors the argument list of the
 * reference launch (fused_attn.py:219-231): the six tensors, cu_seqlens,
 * the strides, NUM_WINDOWS / NUM_HEADS / MAX_SEQLEN and HEAD_DIM, plus the
 * softmax scale that the reference hard-codes as 1/sqrt(head_dim)
 * (fused_attn.py:353-355) and the cos/sin width and dtypes it infers from
 * the tensors.
 */
typedef struct fra_fwd_args {
    const void *q;              /* [total_seq, num_heads, head_dim], qkv_dtype */
    const void *k;
    const void *v;
    const void *cos;            /* [total_seq, rope_width], rope_dtype */
    const void *sin;            /* same shape, dtype and strides as cos */
    void *out;                  /* [total_seq, num_heads, head_dim], qkv_dtype */
    const int32_t *cu_seqlens;  /* device, [num_seqs + 1], cumulative token offsets */
    int64_t q_stride_seq, q_stride_head;      /* in elements; head_dim stride is 1 */
    int64_t k_stride_seq, k_stride_head;
    int64_t v_stride_seq, v_stride_head;
    int64_t out_stride_seq, out_stride_head;
    int64_t rope_stride_seq;    /* in elements, shared by cos and sin */
    int32_t total_seq;          /* rows of q/k/v/out/cos/sin; segments are clamped to it */
    int32_t num_heads;
    int32_t head_dim;
    int32_t num_seqs;           /* number of segments = len(cu_seqlens) - 1 */
    int32_t max_seqlen;         /* >= 1 and >= every segment length */
    int32_t rope_width;         /* head_dim/2 (reference layout) or head_dim (HF cat(emb, emb)) */
    int32_t qkv_dtype;          /* FRA_DTYPE_BF16 or FRA_DTYPE_F16 */
    int32_t rope_dtype;         /* FRA_DTYPE_F32, FRA_DTYPE_BF16 or FRA_DTYPE_F16 */
    float softmax_scale;        /* > 0; the reference uses 1/sqrt(head_dim) */
    int32_t flags;              /* reserved, must be 0 */
    /*
     * Optional device workspace of the long kernel, 16-byte aligned (no
     * counterpart in the reference, whose launch takes no scratch memory).
     * Its first total_seq*num_heads*head_dim*2 bytes (rounded up to 256)
     * take K rotated once per call by a small kernel launched first on the
     * same stream, which the attention kernel then stages instead of
     * rotating every key block once per query block.  When the whole holds
     * what fra_workspace_bytes() reports, the rest also lets the units of a
     * partly filled last round of workgroups split along the key range,
     * with a second small kernel merging their parts.  Less than the rotated-K
     * part (NULL / 0 included): K is rotated in the kernel and nothing is
     * split.  Scratch only: no contents are expected before the call or
     * kept after it; calls that share a workspace must not overlap.
     */
    void *workspace;
    int64_t workspace_bytes;
    /*
     * Optional output (no counterpart in the reference, whose kernel keeps
     * the softmax statistics in registers): the natural-log row sums
     * lse[h * total_seq + t] = log(sum_j exp(softmax_scale * q_rot[t,h] .
     * k_rot[j,h])) over the keys j of t's segment, fp32, [num_heads,
     * total_seq] contiguous, 4-byte aligned.  fra_bwd_varlen() consumes it.
     * Entries of rows outside every segment are not written.  NULL: none.
     */
    float *lse;
} fra_fwd_args;

/* What fra_fwd_varlen() would launch for a set of arguments. */
typedef struct fra_plan {
    int32_t kernel;             /* enum fra_kernel */
    int32_t grid;               /* workgroups (1-D grid) */
    int32_t block;              /* threads per workgroup */
    int32_t block_q;            /* query rows per workgroup */
    int32_t block_kv;           /* key/value rows per LDS stage */
    int32_t lds_bytes;          /* static LDS per workgroup */
    int32_t split_units;        /* long kernel: units of the last round split along keys (0: none) */
    int32_t split_parts;        /* ... into this many parts each */
    char name[64];              /* kernel instance name */
} fra_plan;

/*
 * Fused split-half RoPE on Q and K + non-causal softmax attention over the
 * packed segments [cu_seqlens[i], cu_seqlens[i+1]).  Replaces
 * reference fused_attn.py:218-231 (+ the kernel at :235-423).
 *
 * Semantics (as the reference kernel): the rotation is computed in fp32 and
 * rounded to the input dtype (fused_attn.py:340-345, 385-390); logits are
 * scaled by softmax_scale*log2(e) and exponentiated with exp2 (:353-355,
 * :398-405); P is rounded to the value dtype before PV (:413); fp32
 * accumulation; the output is acc / rowsum rounded to the output dtype
 * (:417-423).  Empty segments are skipped (:295-296).  Rows outside every
 * segment are not written (:196).  Segment bounds are clamped to
 * [0, total_seq], so a malformed cu_seqlens never reads or writes outside
 * the tensors; a max_seqlen below the true maximum gives unspecified values
 * in the rows of the longer segments, never an out-of-bounds access.
 *
 * `stream` is a hipStream_t (NULL = the null stream).
 * Returns FRA_OK or a negative enum fra_status.
 */
int fra_fwd_varlen(const fra_fwd_args *args, void *stream);

/*
 * fra_fwd_varlen() for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  No counterpart in the reference.  Same arguments, semantics
 * and outputs as fra_fwd_varlen() with args->workspace ignored: K is rotated
 * inside the long kernel, and a split last round keeps its partial rows in a
 * static device array of the library (36 MiB per device, held until the
 * process ends; enough for any call on a device of up to 256 CUs at
 * head_dim <= 128), so nothing is allocated or freed.  A call that would
 * need more scratch than that returns FRA_EUNSUPPORTED.  Every call on one
 * device shares that array: calls that overlap on one device (other streams,
 * other threads) race and must be serialised by the caller.
 */
int fra_fwd_varlen_static(const fra_fwd_args *args, void *stream);

/* Fill *plan with the kernel choice for args without launching anything
 * (the split fields reflect args->workspace_bytes). */
int fra_query_plan(const fra_fwd_args *args, fra_plan *plan);

/*
 * RoPE positions instead of cos/sin tables (fra_fwd_varlen_pos).  For token t
 * with patch position (h, w) = (pos[2t], pos[2t + 1]) the kernels compute, in
 * fp32, the angles of the reference's table row t (compute_rope_2d,
 * fused_attn.py:78-116): column j < head_dim/4 is h * inv_freq[j], column
 * head_dim/4 + j is w * inv_freq[j] (one fp32 product each, as the
 * reference's outer product), and take their cosine and sine in registers.
 * The table of width head_dim/2 is never materialised.
 */
typedef struct fra_rope_positions {
    const int32_t *pos;         /* device, [total_seq, 2] contiguous int32 (h, w), rows in q/k order; 8-byte aligned */
    const float *inv_freq;      /* device, [head_dim / 4] fp32: 1 / theta^(2j / (head_dim / 2)) */
} fra_rope_positions;

/*
 * fra_fwd_varlen() with the rotation angles computed from positions
 * (fra_rope_positions) instead of read from cos/sin tables.  Replaces the
 * pair reference compute_rope_2d (fused_attn.py:33-136) + the table reads
 * of the kernel (fused_attn.py:325-329, 370-374); the table is never built
 * or read.  args->cos, args->sin, rope_width, rope_dtype and
 * rope_stride_seq are ignored (cos/sin may be NULL); head_dim must be a
 * multiple of 4.  Segments longer than 64 tokens need the rotated-K part of
 * a workspace (fra_workspace_bytes() of the same args): the long kernel
 * takes K rotated once per call; without it the call returns
 * FRA_EUNSUPPORTED.  Forward only (fra_bwd_varlen takes tables).
 */
int fra_fwd_varlen_pos(const fra_fwd_args *args, const fra_rope_positions *rope, void *stream);

/*
 * The window shuffle fused into the kernel's addressing: a window layer on
 * tensors kept in image order.  cu_seqlens describes the windows over the
 * slots 0 .. total_seq-1 of window order, as for fra_fwd_varlen(), and slot
 * i reads and writes row row_index[i] of q, k, v, out and of cos/sin (or
 * pos) -- the gather reference window_shuffle does before the encoder's
 * blocks (utils.py:105-126: row_index[i] = window_index[i / m^2] * m^2 +
 * i % m^2) and whose inverse window_unshuffle applies after them
 * (utils.py:129-153).  lse, when given, is indexed by tensor row.  Rows
 * that no segment's slot maps to are not written.  row_index is device
 * int32 [total_seq], 4-byte aligned; entries are clamped into [0, total_seq).
 * rope NULL: tables from args (as fra_fwd_varlen); else positions (as
 * fra_fwd_varlen_pos).  Window layers only (segments of at most 64 tokens,
 * head_dim <= 96); otherwise FRA_EUNSUPPORTED.  No counterpart in the
 * reference, which shuffles with two gathers around the encoder.
 */
int fra_fwd_varlen_gather(const fra_fwd_args *args, const fra_rope_positions *rope, const int32_t *row_index,
                          void *stream);

/* fra_workspace_bytes() and fra_query_plan() of a fra_fwd_varlen_pos() call
 * (no counterpart in the reference, which has no position variant). */
int fra_workspace_bytes_pos(const fra_fwd_args *args, const fra_rope_positions *rope, int64_t *bytes);
int fra_query_plan_pos(const fra_fwd_args *args, const fra_rope_positions *rope, fra_plan *plan);

/*
 * Workspace bytes the long kernel can use for these arguments (their
 * workspace fields are ignored): rotated K plus the split scratch when a
 * split applies; 0 for the window kernel.  No counterpart in
 * the reference (its Triton launch allocates nothing); callers that cannot
 * allocate simply pass no workspace and get the unsplit kernel.
 */
int fra_workspace_bytes(const fra_fwd_args *args, int64_t *bytes);

/*
 * Arguments of one backward call (no counterpart in the reference, which is
 * forward-only; this is the training side of the same op).  Given dout =
 * dL/dout of a forward call with the same q, k, v, cos, sin, cu_seqlens,
 * max_seqlen and softmax_scale, and that call's out and lse, it writes
 * dq, dk, dv = dL/dq, dL/dk, dL/dv.  cos and sin get no gradient.
 * Every [total_seq, num_heads, head_dim] tensor (q, k, v, out, dout, dq,
 * dk, dv) is 16-byte aligned with strides that are multiples of 8 elements;
 * cos/sin are aligned to 4 of their elements with a row stride that is a
 * multiple of 4 elements.  Rows outside every segment are not written.
 */
typedef struct fra_bwd_args {
    const void *q;
    const void *k;
    const void *v;
    const void *cos;
    const void *sin;
    const void *out;            /* the forward's output */
    const void *dout;           /* gradient of the output, qkv_dtype */
    const float *lse;           /* the forward's lse, [num_heads, total_seq] */
    const int32_t *cu_seqlens;
    void *dq;                   /* outputs, qkv_dtype */
    void *dk;
    void *dv;
    int64_t q_stride_seq, q_stride_head;
    int64_t k_stride_seq, k_stride_head;
    int64_t v_stride_seq, v_stride_head;
    int64_t out_stride_seq, out_stride_head;
    int64_t dout_stride_seq, dout_stride_head;
    int64_t dq_stride_seq, dq_stride_head;
    int64_t dk_stride_seq, dk_stride_head;
    int64_t dv_stride_seq, dv_stride_head;
    int64_t rope_stride_seq;
    int32_t total_seq;
    int32_t num_heads;
    int32_t head_dim;
    int32_t num_seqs;
    int32_t max_seqlen;
    int32_t rope_width;
    int32_t qkv_dtype;
    int32_t rope_dtype;
    float softmax_scale;
    int32_t flags;              /* reserved, must be 0 */
    /* Device scratch of at least fra_bwd_workspace_bytes() bytes, 16-byte
     * aligned: the per-row dot products of dout and out, and q and k rotated
     * once per call.  None (0 bytes) when max_seqlen <= 64. */
    void *workspace;
    int64_t workspace_bytes;
} fra_bwd_args;

/*
 * Gradients of fra_fwd_varlen() (see fra_bwd_args).  Three kernels on
 * `stream`: the row dot products of dout and out, then dq (one workgroup per
 * block of queries, looping over the keys of its segment) and dk, dv (one
 * workgroup per block of keys, looping over the queries).  No atomics: the
 * result is deterministic.  Returns FRA_OK or a negative enum fra_status.
 */
int fra_bwd_varlen(const fra_bwd_args *args, void *stream);

/* Workspace bytes fra_bwd_varlen() needs for these arguments. */
int fra_bwd_workspace_bytes(const fra_bwd_args *args, int64_t *bytes);

/* Fill *plan with the backward's main kernel for args without launching
 * anything: kernel FRA_KERNEL_WINDOW (one workgroup per (segment, head);
 * name "bwd_window_..." or, with V held in registers, "bwd_window_vreg_...")
 * or FRA_KERNEL_LONG ("bwd_long_...", the dq and dk/dv units); grid and
 * block of that kernel.  No counterpart in the reference (forward-only). */
int fra_bwd_query_plan(const fra_bwd_args *args, fra_plan *plan);

/* 1 if head_dim has a compiled kernel in this build, else 0. */
int fra_supports_head_dim(int32_t head_dim);

/* Message of the last failing call on this thread ("" if none). */
const char *fra_last_error(void);

/* Library version string. */
const char *fra_version(void);

/* FRA_ABI_VERSION of the built library. */
int32_t fra_abi_version(void);

/* sizeof(fra_fwd_args) / sizeof(fra_plan) / sizeof(fra_bwd_args) as
 * compiled, for FFI checks. */
int32_t fra_sizeof_args(void);
int32_t fra_sizeof_plan(void);
int32_t fra_sizeof_bwd_args(void);

#ifdef __cplusplus
}
#endif

#endif /* FRA_H */
