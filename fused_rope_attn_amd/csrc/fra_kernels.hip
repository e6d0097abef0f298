// fra_kernels.hip -- gfx950 kernels of the fused RoPE + varlen attention path.
//
// Two kernel families replace the reference's single Triton kernel
// (reference fused_attn.py:235-423):
//
//   window_kernel  every segment has <= 64 tokens (Qwen2.5-VL window layers).
//                  One wavefront owns one (segment, head): it loads Q and K
//                  rows straight into MFMA operand registers, rotates them in
//                  fp32 there, stages V transposed in LDS, and does one
//                  64x64 softmax -- no online rescaling is needed.
//   long_kernel    segments of any length (full-attention layers).  Split-Q
//                  flash tiling: a 4-wave workgroup owns 128 query rows of one
//                  (segment, head); K is rotated once per 64-row block while
//                  it is staged in LDS, V is staged transposed, and each wave
//                  runs an exp2 online softmax over its 32 rows.
//
// Matrix products use v_mfma_f32_32x32x16_{bf16,f16}.  Scores are computed
// transposed (S^T = K_rot Q_rot^T) so that the 32x32 accumulator layout puts
// one query per lane column: row max and row sum are in-lane reductions plus
// one exchange with lane^32, and P^T is already in the B-operand layout of the
// PV product O^T = V^T P^T.
//
// The contraction index of QK^T may be visited in any order as long as Q and
// K use the same one.  The window kernel feeds k-slot group g (lanes 32g..)
// of MFMA step t with {x0r[4i..4i+3], x1r[4i..4i+3]} for quad i = g*S + t, so
// each lane rotates only the quads it feeds (no redundant loads).  The long
// kernel keeps K_rot in LDS in natural order [x0r | x1r | 0-pad].
#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include <algorithm>

#include "fra.h"

namespace {

typedef uint32_t u32;
typedef uint16_t u16;
typedef __attribute__((__vector_size__(2 * sizeof(u32)))) u32 u32x2;
typedef __attribute__((__vector_size__(4 * sizeof(u32)))) u32 u32x4;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4;
typedef __attribute__((__vector_size__(16 * sizeof(float)))) float f32x16;
typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8;
typedef __attribute__((__vector_size__(2 * sizeof(__bf16)))) __bf16 bf16x2;
typedef __attribute__((__vector_size__(8 * sizeof(_Float16)))) _Float16 f16x8;
typedef __attribute__((__vector_size__(2 * sizeof(_Float16)))) _Float16 f16x2;

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kNegInf = -__builtin_inff();

// Kernel parameters, passed by value.  Strides are in elements.
struct KParams {
    const char *q, *k, *v, *cos, *sin;
    char *out;
    const int32_t *cu;
    int64_t sq_s, sq_h, sk_s, sk_h, sv_s, sv_h, so_s, so_h, sr_s;
    int32_t total, num_heads, num_seqs, max_seqlen;
    int32_t qblocks;      // long kernel: query blocks per (segment, head)
    float scale_log2;     // softmax_scale * log2(e)
};

// ---- element traits ---------------------------------------------------------

struct BF16 {
    static __device__ __forceinline__ float lo(u32 w) { return __builtin_bit_cast(float, w << 16); }
    static __device__ __forceinline__ float hi(u32 w) { return __builtin_bit_cast(float, w & 0xffff0000u); }
    static __device__ __forceinline__ u32 pack(float a, float b) {
        bf16x2 v = {(__bf16)a, (__bf16)b};  // v_cvt_pk_bf16_f32, round to nearest even
        return __builtin_bit_cast(u32, v);
    }
    static __device__ __forceinline__ f32x16 mma(u32x4 a, u32x4 b, f32x16 c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                      __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
    }
};

struct F16 {
    static __device__ __forceinline__ float lo(u32 w) {
        return (float)__builtin_bit_cast(_Float16, (u16)(w & 0xffffu));
    }
    static __device__ __forceinline__ float hi(u32 w) {
        return (float)__builtin_bit_cast(_Float16, (u16)(w >> 16));
    }
    static __device__ __forceinline__ u32 pack(float a, float b) {
        f16x2 v = {(_Float16)a, (_Float16)b};  // round to nearest even
        return __builtin_bit_cast(u32, v);
    }
    static __device__ __forceinline__ f32x16 mma(u32x4 a, u32x4 b, f32x16 c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                     __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
    }
};

// cos/sin table element types: a quad (4 consecutive entries) as fp32.
template <int RD> struct Rope;
template <> struct Rope<FRA_DTYPE_F32> {
    static constexpr int kBytes = 4;
    static __device__ __forceinline__ f32x4 quad(const char *p) { return *(const f32x4 *)p; }
};
template <> struct Rope<FRA_DTYPE_BF16> {
    static constexpr int kBytes = 2;
    static __device__ __forceinline__ f32x4 quad(const char *p) {
        u32x2 w = *(const u32x2 *)p;
        return f32x4{BF16::lo(w[0]), BF16::hi(w[0]), BF16::lo(w[1]), BF16::hi(w[1])};
    }
};
template <> struct Rope<FRA_DTYPE_F16> {
    static constexpr int kBytes = 2;
    static __device__ __forceinline__ f32x4 quad(const char *p) {
        u32x2 w = *(const u32x2 *)p;
        return f32x4{F16::lo(w[0]), F16::hi(w[0]), F16::lo(w[1]), F16::hi(w[1])};
    }
};

// ---- small helpers ------------------------------------------------------------

// Consecutive logical units on the same XCD.  Workgroup b is dispatched to
// XCD b % 8; this bijection on [0, n) gives XCD x the contiguous range of
// units [x*ceil, ...), so units that share cache lines (adjacent heads of a
// window, the query blocks of one head) share one L2.
__device__ __forceinline__ int xcd_remap(int b, int n) {
    constexpr int kXcd = 8;
    const int xcd = b % kXcd, local = b / kXcd;
    const int base = n / kXcd, rem = n % kXcd;
    return xcd < rem ? xcd * (base + 1) + local : rem * (base + 1) + (xcd - rem) * base + local;
}

// Value held by lane (lane ^ 32).
__device__ __forceinline__ float xchg32(float x) {
    const int lane = threadIdx.x & 63;
    return __builtin_bit_cast(float, __builtin_amdgcn_ds_bpermute((lane ^ 32) << 2, __builtin_bit_cast(int, x)));
}

// max(a, b, c) in one instruction (the compiler only forms v_max3_f32 under
// no-NaN assumptions, which the -inf masking rules out).
__device__ __forceinline__ float max3f(float a, float b, float c) {
    float d;
    asm("v_max3_f32 %0, %1, %2, %3" : "=v"(d) : "v"(a), "v"(b), "v"(c));
    return d;
}

// An opaque copy of v: index arithmetic derived from it is recomputed in each
// phase instead of being kept live (in registers) across the whole kernel.
__device__ __forceinline__ int fresh(int v) {
    asm volatile("" : "+v"(v));
    return v;
}

__device__ __forceinline__ u32 perm(u32 hi_src, u32 lo_src, u32 sel) {
    return __builtin_amdgcn_perm(hi_src, lo_src, sel);
}
constexpr u32 kSelLo = 0x05040100u;  // {lo16(lo_src), lo16(hi_src)}
constexpr u32 kSelHi = 0x07060302u;  // {hi16(lo_src), hi16(hi_src)}

// Split-half rotation of one quad pair, in fp32 with separately rounded
// products (reference fused_attn.py:340-345 and :385-390; the same order of
// roundings as the unfused torch path), packed to the storage dtype.
template <class E>
__device__ __forceinline__ void rotate_quad(u32x2 x0w, u32x2 x1w, f32x4 c0, f32x4 s0, f32x4 c1, f32x4 s1,
                                            u32x2 &r0w, u32x2 &r1w) {
#pragma clang fp contract(off)
    const float x0[4] = {E::lo(x0w[0]), E::hi(x0w[0]), E::lo(x0w[1]), E::hi(x0w[1])};
    const float x1[4] = {E::lo(x1w[0]), E::hi(x1w[0]), E::lo(x1w[1]), E::hi(x1w[1])};
    float r0[4], r1[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        r0[i] = x0[i] * c0[i] - x1[i] * s0[i];
        r1[i] = x0[i] * s1[i] + x1[i] * c1[i];
    }
    r0w = u32x2{E::pack(r0[0], r0[1]), E::pack(r0[2], r0[3])};
    r1w = u32x2{E::pack(r1[0], r1[1]), E::pack(r1[2], r1[3])};
}

// Loads quad i (entries 4i..4i+3) of both halves of one x row and of the
// matching cos/sin rows, and rotates it.  The loads are unconditional -- the
// caller passes pointers that are valid for every lane (rows clamped into the
// segment) -- so the load stream stays one straight-line block; `valid` false
// zeroes the result.  FULL selects tables of width D (second half used for
// x1', the HF layout) over width D/2 (the reference layout).
template <int D, class E, int RD, bool FULL>
__device__ __forceinline__ void load_rotate_quad(const char *xrow, const char *crow, const char *srow, int i,
                                                 bool valid, u32x2 &r0w, u32x2 &r1w) {
    constexpr int HALF = D / 2;
    constexpr int RB = Rope<RD>::kBytes;
    u32x2 x0 = *(const u32x2 *)(xrow + 8 * i);
    u32x2 x1 = *(const u32x2 *)(xrow + 2 * HALF + 8 * i);
    const f32x4 c0 = Rope<RD>::quad(crow + RB * 4 * i);
    const f32x4 s0 = Rope<RD>::quad(srow + RB * 4 * i);
    f32x4 c1 = c0, s1 = s0;
    if constexpr (FULL) {
        c1 = Rope<RD>::quad(crow + RB * (HALF + 4 * i));
        s1 = Rope<RD>::quad(srow + RB * (HALF + 4 * i));
    }
    if (!valid) {
        x0 = u32x2{0u, 0u};
        x1 = u32x2{0u, 0u};
    }
    rotate_quad<E>(x0, x1, c0, s0, c1, s1, r0w, r1w);
}

// ---- window kernel ------------------------------------------------------------
//
// One workgroup of 4 wavefronts per (segment, group of 4 heads); segment
// length L <= 64.  All HBM traffic is coalesced: consecutive lanes move
// consecutive 16-byte chunks of the group's slab -- 4 heads x D elements,
// contiguous in a [tokens, heads, head_dim] tensor -- and LDS turns the slab
// into MFMA operands (and the output back into slab rows).
//
//   1. every global load is issued up front: cos/sin rows, Q, K, V slabs;
//   2. cos/sin -> LDS as fp32 rows; the Q slab -> LDS (whole, or one
//      32-token half at a time when the LDS budget asks for it), where
//      wavefront w rotates the quads of head 4*hg + w it feeds (fp32, rounded
//      to the storage dtype);
//   3. the same for K;
//   4. V -> LDS transposed (V^T per head, kv pairs packed in dwords);
//   5. per 32-query tile: S^T = K_rot Q_rot^T, softmax, O^T = V^T P^T; the
//      normalised output stays in registers as packed bf16/fp16;
//   6. the output rows go through LDS (over V^T) and leave as slab rows.
//
// Lane (r, g) (r = lane & 31, g = lane >> 5) of a wavefront holds the
// operands of tokens r and r + 32: K_rot rows as the A operand of S^T and
// Q_rot rows as its B operand; MFMA step t, k-slot group g carries
// {x0r[4i..4i+3], x1r[4i..4i+3]} of quad i = g*S + t (the contraction order is
// free as long as Q and K share it).

constexpr int kWinHeads = 4;     // heads (wavefronts) per workgroup
constexpr int kWinWaves = 2;     // wavefronts per SIMD the register budget is sized for
constexpr int kWinThreads = 64 * kWinHeads;

template <int D, bool FULL> struct WinLds {
    static constexpr int W = FULL ? D : D / 2;         // table width
    static constexpr int CS = 2 * W + 4;               // fp32 per [cos | sin] row, +4 pad (conflict-free b128 reads)
    static constexpr int SLAB = kWinHeads * D * 2;     // bytes of one token's slab
    static constexpr int PITCH = SLAB + 16;            // LDS row pitch of a staged slab (one pad chunk)
    static constexpr int VTS = 36;                     // dwords per V^T row: 32 kv pairs + 4 pad
    static constexpr int kTableBytes = 64 * CS * 4;
    static constexpr int kStageRows = kWinWaves == 2 ? 64 : 32;  // slab rows staged at once
    static constexpr int kHalfBytes = kStageRows * PITCH;
    static constexpr int kRotBytes = kTableBytes + kHalfBytes;
    static constexpr int kVtBytes = kWinHeads * D * VTS * 4;
    static constexpr int kOutBytes = 64 * PITCH;
    static constexpr int kMax2 = kVtBytes > kOutBytes ? kVtBytes : kOutBytes;
    static constexpr int kMain = kRotBytes > kMax2 ? kRotBytes : kMax2;
    static constexpr int kBytes = kMain + 16;          // + a 16-byte trash slot
};

template <int D, class E, int RD, bool FULL>
__global__ __launch_bounds__(kWinThreads, kWinWaves) void window_kernel(const KParams p) {
    using LDS = WinLds<D, FULL>;
    constexpr int NQ = D / 8;                 // quads per half
    constexpr int S = (NQ + 1) / 2;           // 16-deep k-steps of QK^T
    constexpr int NDT = (D + 31) / 32;        // 32-row tiles of O^T
    constexpr int VTS = LDS::VTS;
    constexpr int W = LDS::W;
    constexpr int CS = LDS::CS;
    constexpr int PITCH = LDS::PITCH;
    constexpr int HCH = D / 8;                // 16-byte chunks per head row
    constexpr int NCH = kWinHeads * HCH;      // chunks per slab row
    constexpr int RB = Rope<RD>::kBytes;
    constexpr int TQ = W / 4;                 // table quads per row
    constexpr int TITEMS = 64 * TQ * 2;       // (token, quad, table)
    constexpr int TPER = (TITEMS + kWinThreads - 1) / kWinThreads;
    constexpr int SITEMS = 64 * NCH;          // (token, chunk) of a Q/K slab or the output
    constexpr int SPER = (SITEMS + kWinThreads - 1) / kWinThreads;
    constexpr int VITEMS = 32 * NCH;          // (token pair, chunk) of the V slab
    constexpr int VPER = (VITEMS + kWinThreads - 1) / kWinThreads;
    constexpr int OQ = NDT * 4;               // output quads per lane and query tile
    // V^T row rho (= head*D + d) stores kv pair j at dword column
    // j ^ vswz(rho): with the 36-dword pitch this makes both the staging
    // writes and the operand reads (b64, pairs of columns) 2-way at most
    // across the 64 banks.  The xor value is even, so column pairs stay
    // adjacent and 8-byte aligned.
    auto vswz = [](int rho) { return 2 * ((rho >> 4) & 15); };
    __shared__ __attribute__((aligned(16))) char lds[LDS::kBytes];
    float *tab = (float *)lds;                                  // [64][CS] fp32 tables
    char *half = lds + LDS::kTableBytes;                        // [32][PITCH]: half a Q or K slab
    u32 *vt_all = (u32 *)lds;                                   // [4][D][VTS] V^T, after the rotations
    char *oslab = lds;                                          // [64][PITCH] output rows, after PV
    char *trash = lds + LDS::kMain;                             // sink of out-of-range staging items

    const int tid = threadIdx.x;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    const int r = lane & 31, g = lane >> 5;
    const int ngroups = (p.num_heads + kWinHeads - 1) / kWinHeads;
    const int u = xcd_remap(blockIdx.x, gridDim.x);
    const int seg = u / ngroups, hg = u - seg * ngroups;
    const int h0 = hg * kWinHeads;
    const int nh = min(kWinHeads, p.num_heads - h0);            // heads in this group
    const bool active = w < nh;  // wavefronts past the last head still take part in barriers
    int s0 = p.cu[seg], s1 = p.cu[seg + 1];
    s0 = min(max(s0, 0), p.total);
    s1 = min(max(s1, 0), p.total);
    const int L = min(s1 - s0, 64);
    if (L <= 0) return;  // uniform across the workgroup

    // Wave-uniform 64-bit bases plus 32-bit per-lane byte offsets: the host
    // guarantees 64 rows of every tensor span < 2 GiB.
    const char *qb = p.q + ((int64_t)s0 * p.sq_s + (int64_t)h0 * p.sq_h) * 2;
    const char *kb = p.k + ((int64_t)s0 * p.sk_s + (int64_t)h0 * p.sk_h) * 2;
    const char *vb = p.v + ((int64_t)s0 * p.sv_s + (int64_t)h0 * p.sv_h) * 2;
    const char *cb = p.cos + (int64_t)s0 * p.sr_s * RB;
    const char *sb = p.sin + (int64_t)s0 * p.sr_s * RB;
    char *ob = p.out + ((int64_t)s0 * p.so_s + (int64_t)h0 * p.so_h) * 2;
    const uint32_t qrs = (uint32_t)p.sq_s * 2, krs = (uint32_t)p.sk_s * 2, vrs = (uint32_t)p.sv_s * 2;
    const uint32_t qhs = (uint32_t)p.sq_h * 2, khs = (uint32_t)p.sk_h * 2, vhs = (uint32_t)p.sv_h * 2;
    const uint32_t ors = (uint32_t)p.so_s * 2, ohs = (uint32_t)p.so_h * 2;
    const uint32_t trs = (uint32_t)p.sr_s * RB;

    // ---- 1. every global load, back to back: tables, Q, K and V slabs ----------
    // Rows past the segment and chunks of heads past the last one read the
    // segment's first row / the group's first head; their values are never used.
    f32x4 tv[TPER];
    int t1 = fresh(tid);
#pragma unroll
    for (int k = 0; k < TPER; ++k) {
        const int it = min(t1 + k * kWinThreads, TITEMS - 1);
        const int tok = it / (2 * TQ), rem = it - tok * 2 * TQ;
        const int tbl = rem / TQ, qd = rem - tbl * TQ;
        const uint32_t off = (uint32_t)(tok < L ? tok : 0) * trs + (uint32_t)(4 * qd * RB);
        tv[k] = Rope<RD>::quad((tbl ? sb : cb) + off);
    }
    u32x4 qs[SPER], ks[SPER];
    t1 = fresh(tid);
#pragma unroll
    for (int k = 0; k < SPER; ++k) {
        const int it = min(t1 + k * kWinThreads, SITEMS - 1);
        const int tok = it / NCH, wc = it - tok * NCH;
        const int hh = wc / HCH, c = wc - hh * HCH;
        const uint32_t row = tok < L ? tok : 0, hd = hh < nh ? hh : 0;
        qs[k] = *(const u32x4 *)(qb + (row * qrs + hd * qhs + 16 * c));
        ks[k] = *(const u32x4 *)(kb + (row * krs + hd * khs + 16 * c));
    }
    // V rows 2j, 2j+1 of the slab.
    u32x4 va[VPER], vv[VPER];
    t1 = fresh(tid);
#pragma unroll
    for (int k = 0; k < VPER; ++k) {
        const int it = min(t1 + k * kWinThreads, VITEMS - 1);
        const int j = it / NCH, wc = it - j * NCH;
        const int hh = wc / HCH, c = wc - hh * HCH;
        const uint32_t ra = 2 * j < L ? 2 * j : 0, rb = 2 * j + 1 < L ? 2 * j + 1 : 0;
        const uint32_t hd = hh < nh ? hh : 0;
        va[k] = *(const u32x4 *)(vb + (ra * vrs + hd * vhs + 16 * c));
        vv[k] = *(const u32x4 *)(vb + (rb * vrs + hd * vhs + 16 * c));
    }
    __builtin_amdgcn_sched_barrier(0);

    // ---- 2. tables to LDS; Q staged and rotated ---------------------------------
    // Staging writes are branch-free (a branch here would make the compiler
    // wait for every outstanding load): items out of range go to the trash slot.
    t1 = fresh(tid);
#pragma unroll
    for (int k = 0; k < TPER; ++k) {
        const int it = t1 + k * kWinThreads;
        const bool in = TITEMS % kWinThreads == 0 || it < TITEMS;
        const int itc = in ? it : 0;
        const int tok = itc / (2 * TQ), rem = itc - tok * 2 * TQ;
        const int tbl = rem / TQ, qd = rem - tbl * TQ;
        *(f32x4 *)(in ? (char *)(tab + tok * CS + tbl * W + 4 * qd) : trash) = tv[k];
    }
    // Writes the items of tokens [R*hf, R*hf + R) of a slab into `half`
    // (R = kStageRows: all 64 rows at once when LDS allows, else 32).
    constexpr int R = LDS::kStageRows;
    auto stage_half = [&](const u32x4 (&x)[SPER], int hf) {
        const int ts = fresh(tid);
#pragma unroll
        for (int k = 0; k < SPER; ++k) {
            const int it = ts + k * kWinThreads;
            const int tok = it / NCH, wc = it - tok * NCH;
            const bool in = (SITEMS % kWinThreads == 0 || it < SITEMS) && (R == 64 || (tok >> 5) == hf);
            *(u32x4 *)(in ? half + (tok - R * hf) * PITCH + 16 * wc : trash) = x[k];
        }
    };
    // Rotates this wavefront's quads of the staged half into MFMA operands.
    auto rotate_half = [&](u32x4 (&op)[S], int hf) {
        const int tok = r + 32 * hf;
        const float *crow = tab + tok * CS;
        const char *xrow = half + (R == 64 ? tok : r) * PITCH + w * (2 * D);
#pragma unroll
        for (int t = 0; t < S; ++t) {
            const int i = g * S + t;
            const bool has = tok < L && i < NQ;
            const int il = i < NQ ? i : 0;
            const f32x4 c0 = *(const f32x4 *)(crow + 4 * il);
            const f32x4 s0v = *(const f32x4 *)(crow + W + 4 * il);
            f32x4 c1 = c0, s1v = s0v;
            if constexpr (FULL) {
                c1 = *(const f32x4 *)(crow + D / 2 + 4 * il);
                s1v = *(const f32x4 *)(crow + W + D / 2 + 4 * il);
            }
            u32x2 x0 = *(const u32x2 *)(xrow + 8 * il);
            u32x2 x1 = *(const u32x2 *)(xrow + D + 8 * il);
            if (!has) x0 = x1 = u32x2{0u, 0u};
            u32x2 a0, a1;
            rotate_quad<E>(x0, x1, c0, s0v, c1, s1v, a0, a1);
            op[t] = u32x4{a0[0], a0[1], a1[0], a1[1]};
        }
    };
    u32x4 qop[2][S], kop[2][S];
    if constexpr (R == 64) {
        stage_half(qs, 0);
        __syncthreads();
        rotate_half(qop[0], 0);
        rotate_half(qop[1], 1);
        __syncthreads();
        // ---- 3. the K slab -----------------------------------------------------------
        stage_half(ks, 0);
        __syncthreads();
        rotate_half(kop[0], 0);
        rotate_half(kop[1], 1);
    } else {
        stage_half(qs, 0);
        __syncthreads();
        rotate_half(qop[0], 0);
        __syncthreads();
        stage_half(qs, 1);
        __syncthreads();
        rotate_half(qop[1], 1);
        __syncthreads();
        // ---- 3. the K slab -----------------------------------------------------------
        stage_half(ks, 0);
        __syncthreads();
        rotate_half(kop[0], 0);
        __syncthreads();
        stage_half(ks, 1);
        __syncthreads();
        rotate_half(kop[1], 1);
    }
    __syncthreads();  // tables and the staged slab are dead: V^T goes over them

    // ---- 4. V^T: vt[hh][d][j] = {V[2j][d], V[2j+1][d]} ------------------------------
    t1 = fresh(tid);
#pragma unroll
    for (int k = 0; k < VPER; ++k) {
        const int it = t1 + k * kWinThreads;
        const bool in = VITEMS % kWinThreads == 0 || it < VITEMS;
        const int itc = in ? it : 0;
        const int j = itc / NCH, wc = itc - j * NCH;
        const int hh = wc / HCH, c = wc - hh * HCH;
        u32x4 A = va[k], B = vv[k];
        if (2 * j >= L) A = u32x4{0u, 0u, 0u, 0u};
        if (2 * j + 1 >= L) B = u32x4{0u, 0u, 0u, 0u};
        // rho is a multiple of 8, so the item's 8 rows share one swizzle value
        const int rho = hh * D + 8 * c;
        u32 *col = vt_all + rho * VTS + (j ^ vswz(rho));
        const int cs = in ? VTS : 0;  // out-of-range items write the trash slot 8 times
        if (!in) col = (u32 *)trash;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            col[(2 * e) * cs] = perm(B[e], A[e], kSelLo);
            col[(2 * e + 1) * cs] = perm(B[e], A[e], kSelHi);
        }
    }
    __syncthreads();

    // ---- 5. attention per 32-query tile ---------------------------------------------
    // The query-tile loop stays rolled (unrolled, the compiler overlaps the two
    // tiles and runs out of registers); the tile's operands and results are
    // selected with explicit selects, as a register array must not be indexed
    // by the loop variable.
    const float sl = p.scale_log2;
    const int nkt = (L + 31) >> 5;
    const u32 *vt = vt_all + w * (D * VTS);
    u32x2 outq[2][OQ];  // packed normalised output quads (q = 32b + r, d0 = 32dt + 8jq + 4g)
#pragma unroll 1
    for (int b = 0; b < 2; ++b) {
        __builtin_amdgcn_sched_barrier(0);
        if (b * 32 >= L || !active) break;  // uniform within the wavefront; no barrier inside
        u32x4 qcur[S];
#pragma unroll
        for (int t = 0; t < S; ++t) qcur[t] = b ? qop[1][t] : qop[0][t];
        // S^T tiles: rows kv, columns q.  Lane (r, g) holds q = 32b + r and
        // kv = 32a + 8(j/4) + 4g + (j%4) in element j of sacc[a].
        f32x16 sacc[2];
#pragma unroll
        for (int a = 0; a < 2; ++a) {
            sacc[a] = f32x16{};
            if (a < nkt) {
#pragma unroll
                for (int t = 0; t < S; ++t) sacc[a] = E::mma(kop[a][t], qcur[t], sacc[a]);
            }
        }
        float mx = kNegInf;
#pragma unroll
        for (int a = 0; a < 2; ++a) {
#pragma unroll
            for (int j = 0; j < 16; ++j) {
                const int kv = 32 * a + 8 * (j >> 2) + 4 * g + (j & 3);
                if (kv >= L) sacc[a][j] = kNegInf;
                mx = fmaxf(mx, sacc[a][j]);
            }
        }
        mx = fmaxf(mx, xchg32(mx));
        const float mneg = -mx * sl;
        float lsum = 0.f;
#pragma unroll
        for (int a = 0; a < 2; ++a) {
#pragma unroll
            for (int j = 0; j < 16; ++j) {
                const float e = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[a][j], sl, mneg));
                sacc[a][j] = e;
                lsum += e;
            }
        }
        lsum += xchg32(lsum);
        const float inv = 1.0f / lsum;

        // P^T as the B operand of O^T = V^T P^T: step (a, h) uses elements
        // 8h..8h+7 of sacc[a], i.e. kv = 32a + 16h + {4g..4g+3, 8+4g..8+4g+3}.
        u32x4 pop[2][2];
#pragma unroll
        for (int a = 0; a < 2; ++a) {
#pragma unroll
            for (int h = 0; h < 2; ++h)
                pop[a][h] = u32x4{E::pack(sacc[a][8 * h + 0], sacc[a][8 * h + 1]),
                                  E::pack(sacc[a][8 * h + 2], sacc[a][8 * h + 3]),
                                  E::pack(sacc[a][8 * h + 4], sacc[a][8 * h + 5]),
                                  E::pack(sacc[a][8 * h + 6], sacc[a][8 * h + 7])};
        }
        // One 32-row d tile of O^T at a time; element j of oacc is
        // q = 32b + r, d = 32dt + 8(j/4) + 4g + (j%4).
        u32x2 ocur[OQ];
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt) {
            const int d = 32 * dt + r;
            const int dr = min(d, D - 1);
            const u32 *vrow = vt + dr * VTS;
            const int xs = vswz(w * D + dr);
            f32x16 oacc = f32x16{};
#pragma unroll
            for (int a = 0; a < 2; ++a) {
                if (a >= nkt) break;
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    const int kc = 16 * a + 8 * h + 2 * g;  // dword column of kv = 32a + 16h + 4g
                    const u32x2 lo = *(const u32x2 *)(vrow + (kc ^ xs));
                    const u32x2 hi = *(const u32x2 *)(vrow + ((kc + 4) ^ xs));
                    u32x4 vop = {lo[0], lo[1], hi[0], hi[1]};
                    if (d >= D) vop = u32x4{0u, 0u, 0u, 0u};
                    oacc = E::mma(vop, pop[a][h], oacc);
                }
            }
#pragma unroll
            for (int jq = 0; jq < 4; ++jq)
                ocur[4 * dt + jq] = u32x2{E::pack(oacc[4 * jq + 0] * inv, oacc[4 * jq + 1] * inv),
                                          E::pack(oacc[4 * jq + 2] * inv, oacc[4 * jq + 3] * inv)};
        }
#pragma unroll
        for (int i = 0; i < OQ; ++i) {
            if (b) outq[1][i] = ocur[i];
            else outq[0][i] = ocur[i];
        }
    }
    __syncthreads();  // V^T is dead: the output rows go over it

    // ---- 6. output rows through LDS, stored as coalesced slab rows --------------------
    if (active) {
#pragma unroll
        for (int b = 0; b < 2; ++b) {
            if (b * 32 < L) {
                char *orow = oslab + (32 * b + r) * PITCH + w * (2 * D);
#pragma unroll
                for (int dt = 0; dt < NDT; ++dt) {
#pragma unroll
                    for (int jq = 0; jq < 4; ++jq) {
                        const int d0 = 32 * dt + 8 * jq + 4 * g;
                        if (d0 < D) *(u32x2 *)(orow + 2 * d0) = outq[b][4 * dt + jq];
                    }
                }
            }
        }
    }
    __syncthreads();
    const int to = fresh(tid);
#pragma unroll
    for (int k = 0; k < SPER; ++k) {
        const int it = to + k * kWinThreads;
        if (it < SITEMS) {
            const int tok = it / NCH, wc = it - tok * NCH;
            const int hh = wc / HCH, c = wc - hh * HCH;
            if (tok < L && hh < nh)
                *(u32x4 *)(ob + ((uint32_t)tok * ors + (uint32_t)hh * ohs + 16 * c)) =
                    *(const u32x4 *)(oslab + tok * PITCH + 16 * wc);
        }
    }
}

// ---- long kernel ----------------------------------------------------------------
//
// Split-Q flash tiling for segments of any length.  A workgroup of 8
// wavefronts owns 256 query rows of one (segment, head) -- wavefront w rows
// 32w..32w+31 -- and walks the segment's keys in blocks of 64:
//
//   * K_rot (rotated once per block for all 256 rows) and V^T live in LDS,
//     double-buffered; the next block's K/cos/sin/V are loaded into registers
//     while the current block is computed, then rotated / transposed into the
//     other buffer -- one barrier per block.  Loads use a wave-uniform block
//     base and 32-bit lane offsets computed once;
//   * S^T = K_rot Q_rot^T on 32x32x16 MFMA (one query per lane column), exp2
//     online softmax with the row max from v_max3 chains and one exchange
//     with lane^32; the running max is only moved (and O rescaled) when a row
//     max exceeds it by more than 2^8, so in the steady state no rescaling
//     happens and P stays below 2^8;
//   * O^T += V^T P^T with the V^T columns of each 16-key group stored in the
//     order the P^T k-slots visit them, so every A operand is one aligned
//     16-byte LDS read; when head_dim leaves padding rows in the last 32-row
//     tile of V^T, one of them holds ones and the MFMA also produces the row
//     sum of the rounded P (otherwise the sum is taken in fp32 on the VALU).

constexpr int kLongWaves = 4;
constexpr int kLongBQ = 32 * kLongWaves;  // query rows per workgroup
constexpr int kLongBKV = 64;              // key/value rows per LDS stage
constexpr int kLongThreads = 64 * kLongWaves;
constexpr float kRescaleThreshold = 8.0f;  // log2 units

template <int D> struct LongLds {
    static constexpr int DP = (D + 15) / 16 * 16;      // K_rot row padded to the MFMA k-step
    static constexpr int KS = DP + 8;                  // K_rot row stride (bf16 elements), 16 B pad
    static constexpr int NDT = (D + 31) / 32;
    static constexpr int VTS = 36;                     // V^T row stride (dwords): 32 kv pairs + 4 pad
    static constexpr bool kOnesRow = D % 32 != 0;      // a padding row of V^T holds ones
    static constexpr int kKBytes = kLongBKV * KS * 2;
    static constexpr int kVBytes = NDT * 32 * VTS * 4;
    static constexpr int kStage = kKBytes + kVBytes;   // one buffer
    static constexpr int kBytes = 2 * kStage;
};

// Dword column of kv quad kq (keys 4kq..4kq+3) in a V^T row: within each
// 16-key group the quads are stored in the order 0, 2, 1, 3, so the keys
// lane group g feeds to a PV step ({4g..4g+3, 8+4g..8+4g+3}) are 4
// consecutive dwords at column 8 * (group) + 4g.
__device__ __forceinline__ int vt_quad_col(int kq) {
    return 8 * (kq >> 2) + 2 * (((kq & 1) << 1) | ((kq >> 1) & 1));
}

template <int D, class E, int RD, bool FULL>
__global__ __launch_bounds__(kLongThreads, 2) void long_kernel(const KParams p) {
    using LDS = LongLds<D>;
    constexpr int HALF = D / 2;
    constexpr int NQ = D / 8;                  // quads per half
    constexpr int DP = LDS::DP;
    constexpr int S = DP / 16;
    constexpr int KS = LDS::KS;
    constexpr int NDT = LDS::NDT;
    constexpr int VTS = LDS::VTS;
    constexpr int NCH = D / 8;                 // 16-byte chunks per V row
    constexpr int RB = Rope<RD>::kBytes;
    constexpr int KITEMS = kLongBKV * NQ;      // (row, quad) items of a K block
    constexpr int KPER = (KITEMS + kLongThreads - 1) / kLongThreads;
    constexpr int VITEMS = (kLongBKV / 4) * NCH;  // (kv quad, chunk) items of a V block
    constexpr int VPER = (VITEMS + kLongThreads - 1) / kLongThreads;
    constexpr bool ONES = LDS::kOnesRow;
    __shared__ __attribute__((aligned(16))) char lds[LDS::kBytes];

    const int u = xcd_remap(blockIdx.x, gridDim.x);
    const int sh = u / p.qblocks, qblk = u - sh * p.qblocks;
    const int seg = sh / p.num_heads, head = sh - seg * p.num_heads;
    int s0 = p.cu[seg], s1 = p.cu[seg + 1];
    s0 = min(max(s0, 0), p.total);
    s1 = min(max(s1, 0), p.total);
    const int L = s1 - s0;
    if (L <= 0 || qblk * kLongBQ >= L) return;  // uniform across the workgroup

    const int tid = threadIdx.x;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    const int r = lane & 31, g = lane >> 5;

    const char *kbase = p.k + ((int64_t)s0 * p.sk_s + (int64_t)head * p.sk_h) * 2;
    const char *vbase = p.v + ((int64_t)s0 * p.sv_s + (int64_t)head * p.sv_h) * 2;
    const char *cbase = p.cos + (int64_t)s0 * p.sr_s * RB;
    const char *sbase = p.sin + (int64_t)s0 * p.sr_s * RB;
    const int64_t krs = p.sk_s * 2, vrs = p.sv_s * 2, trs = p.sr_s * RB;

    // Constant parts of both buffers: K_rot pad columns [D, DP) and V^T pad
    // rows [D, 32*NDT) are zero (a ones row when it holds the row sum).
    for (int bf = 0; bf < 2; ++bf) {
        u16 *ks = (u16 *)(lds + bf * LDS::kStage);
        u32 *vt = (u32 *)(lds + bf * LDS::kStage + LDS::kKBytes);
        for (int i = tid; i < kLongBKV * (KS - D); i += kLongThreads) {
            const int row = i / (KS - D), col = D + i % (KS - D);
            ks[row * KS + col] = 0;
        }
        const u32 one = E::pack(1.0f, 1.0f);
        for (int i = tid; i < (NDT * 32 - D) * VTS; i += kLongThreads)
            vt[D * VTS + i] = (ONES && i < VTS) ? one : 0u;
    }

    // ---- per-thread staging items, fixed for the whole loop -------------------------
    // K item k: (row, quad i); V item: (chunk c, kv quad kq), kv quad fastest so a
    // wavefront's transposed LDS writes are consecutive columns of one V^T row.
    int krow[KPER], kqd[KPER];
    uint32_t koff[KPER], toff[KPER];
#pragma unroll
    for (int k = 0; k < KPER; ++k) {
        const int it = min(tid + k * kLongThreads, KITEMS - 1);
        krow[k] = it / NQ;
        kqd[k] = it - krow[k] * NQ;
        koff[k] = (uint32_t)(krow[k] * krs) + 8 * kqd[k];
        toff[k] = (uint32_t)(krow[k] * trs) + RB * 4 * kqd[k];
    }
    int vkq[VPER], vch[VPER];
    uint32_t voff[VPER];
#pragma unroll
    for (int k = 0; k < VPER; ++k) {
        const int it = min(tid + k * kLongThreads, VITEMS - 1);
        vch[k] = it / (kLongBKV / 4);
        vkq[k] = it - vch[k] * (kLongBKV / 4);
        voff[k] = (uint32_t)(4 * vkq[k] * vrs) + 16 * vch[k];
    }
    const uint32_t vrs32 = (uint32_t)vrs;

    // ---- prefetch registers of one K/V block ------------------------------------
    u32x2 kx0[KPER], kx1[KPER];
    f32x4 kc0[KPER], ks0[KPER], kc1[KPER], ks1[KPER];
    u32x4 vx[VPER][4];
    // Rows of a partial last block past the segment read row 0 of the block
    // (clamped offsets); their values are replaced by zeros when stored.
    auto load_block = [&](int kb) {
        const bool full = kb + kLongBKV <= L;
        const char *kblk = kbase + kb * krs, *vblk = vbase + kb * vrs;
        const char *cblk = cbase + kb * trs, *sblk = sbase + kb * trs;
#pragma unroll
        for (int k = 0; k < KPER; ++k) {
            const bool ok = full || kb + krow[k] < L;
            const uint32_t ko = ok ? koff[k] : 8u * kqd[k];
            const uint32_t to = ok ? toff[k] : (uint32_t)(RB * 4 * kqd[k]);
            kx0[k] = *(const u32x2 *)(kblk + ko);
            kx1[k] = *(const u32x2 *)(kblk + ko + 2 * HALF);
            kc0[k] = Rope<RD>::quad(cblk + to);
            ks0[k] = Rope<RD>::quad(sblk + to);
            if constexpr (FULL) {
                kc1[k] = Rope<RD>::quad(cblk + to + RB * HALF);
                ks1[k] = Rope<RD>::quad(sblk + to + RB * HALF);
            }
        }
#pragma unroll
        for (int k = 0; k < VPER; ++k) {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const bool ok = full || kb + 4 * vkq[k] + e < L;
                const uint32_t vo = ok ? voff[k] + e * vrs32 : 16u * vch[k];
                vx[k][e] = *(const u32x4 *)(vblk + vo);
            }
        }
    };
    // Rotates / transposes the prefetched block into LDS buffer bf; rows past
    // the segment become zeros.
    auto store_block = [&](int kb, int bf) {
        const bool full = kb + kLongBKV <= L;
        u16 *ks = (u16 *)(lds + bf * LDS::kStage);
        u32 *vt = (u32 *)(lds + bf * LDS::kStage + LDS::kKBytes);
#pragma unroll
        for (int k = 0; k < KPER; ++k) {
            const int it = tid + k * kLongThreads;
            const bool in = KITEMS % kLongThreads == 0 || it < KITEMS;
            u32x2 x0 = kx0[k], x1 = kx1[k];
            if (!full && kb + krow[k] >= L) x0 = x1 = u32x2{0u, 0u};
            u32x2 r0w, r1w;
            rotate_quad<E>(x0, x1, kc0[k], ks0[k], FULL ? kc1[k] : kc0[k], FULL ? ks1[k] : ks0[k], r0w, r1w);
            if (in) {
                *(u32x2 *)(ks + krow[k] * KS + 4 * kqd[k]) = r0w;
                *(u32x2 *)(ks + krow[k] * KS + HALF + 4 * kqd[k]) = r1w;
            }
        }
#pragma unroll
        for (int k = 0; k < VPER; ++k) {
            const int it = tid + k * kLongThreads;
            const bool in = VITEMS % kLongThreads == 0 || it < VITEMS;
            u32x4 x[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                x[e] = vx[k][e];
                if (!full && kb + 4 * vkq[k] + e >= L) x[e] = u32x4{0u, 0u, 0u, 0u};
            }
            if (in) {
                u32 *col = vt + (8 * vch[k]) * VTS + vt_quad_col(vkq[k]);
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    *(u32x2 *)(col + (2 * j) * VTS) =
                        u32x2{perm(x[1][j], x[0][j], kSelLo), perm(x[3][j], x[2][j], kSelLo)};
                    *(u32x2 *)(col + (2 * j + 1) * VTS) =
                        u32x2{perm(x[1][j], x[0][j], kSelHi), perm(x[3][j], x[2][j], kSelHi)};
                }
            }
        }
    };

    load_block(0);

    // Q_rot of this lane's query row, natural order [x0r | x1r | 0], as the
    // B operand of S^T: step t, group g takes elements 16t + 8g .. +7.
    u32x4 qop[S];
    {
        const int q = qblk * kLongBQ + 32 * w + r;
        const bool valid = q < L;
        const int64_t row = s0 + (valid ? q : 0);
        const char *qrow = p.q + (row * p.sq_s + (int64_t)head * p.sq_h) * 2;
        const char *crow = p.cos + row * p.sr_s * RB;
        const char *srow = p.sin + row * p.sr_s * RB;
        u32x2 nat[DP / 4];  // natural quads: 0..NQ-1 = x0r, NQ..2NQ-1 = x1r, rest 0
#pragma unroll
        for (int i = 0; i < NQ; ++i)
            load_rotate_quad<D, E, RD, FULL>(qrow, crow, srow, i, valid, nat[i], nat[NQ + i]);
#pragma unroll
        for (int i = 2 * NQ; i < DP / 4; ++i) nat[i] = u32x2{0u, 0u};
        // Bitwise select: a ?: on the two elements is folded into an index
        // nat[4t + 2g] that would move the array to scratch memory.
        const u32 msk = 0u - (u32)g;
#pragma unroll
        for (int t = 0; t < S; ++t) {
            const u32x2 a = (nat[4 * t] & ~msk) | (nat[4 * t + 2] & msk);
            const u32x2 b = (nat[4 * t + 1] & ~msk) | (nat[4 * t + 3] & msk);
            qop[t] = u32x4{a[0], a[1], b[0], b[1]};
        }
    }

    store_block(0, 0);
    __syncthreads();

    const float sl = p.scale_log2;
    float m_i = kNegInf, l_i = 0.f;
    f32x16 oacc[NDT];
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) oacc[dt] = f32x16{};

    const int nblk = (L + kLongBKV - 1) / kLongBKV;
    for (int j = 0; j < nblk; ++j) {
        const int kb = j * kLongBKV;
        const int bf = j & 1;
        const bool more = j + 1 < nblk;
        if (more) load_block(kb + kLongBKV);
        __builtin_amdgcn_sched_barrier(0);

        const u16 *ks = (const u16 *)(lds + bf * LDS::kStage);
        const u32 *vt = (const u32 *)(lds + bf * LDS::kStage + LDS::kKBytes);
        const int nkv = min(kLongBKV, L - kb);
        const int nkt = (nkv + 31) >> 5;
        f32x16 sacc[2];
#pragma unroll
        for (int a = 0; a < 2; ++a) {
            sacc[a] = f32x16{};
            if (a < nkt) {
                const u16 *krp = ks + (32 * a + r) * KS + 8 * g;
#pragma unroll
                for (int t = 0; t < S; ++t)
                    sacc[a] = E::mma(*(const u32x4 *)(krp + 16 * t), qop[t], sacc[a]);
            }
        }
        if (nkv < kLongBKV) {
#pragma unroll
            for (int a = 0; a < 2; ++a) {
#pragma unroll
                for (int jj = 0; jj < 16; ++jj) {
                    const int kv = 32 * a + 8 * (jj >> 2) + 4 * g + (jj & 3);
                    if (kv >= nkv) sacc[a][jj] = kNegInf;
                }
            }
        }
        float mx = kNegInf;
#pragma unroll
        for (int a = 0; a < 2; ++a) {
#pragma unroll
            for (int jj = 0; jj < 16; jj += 2) mx = max3f(mx, sacc[a][jj], sacc[a][jj + 1]);
        }
        mx = fmaxf(mx, xchg32(mx)) * sl;
        // Lazy rescaling: move the running max only when it grows by more
        // than the threshold (uniform branch over the wavefront).
        if (__builtin_amdgcn_ballot_w64(mx > m_i + kRescaleThreshold) != 0) {
            const float m_new = fmaxf(m_i, mx);
            const float alpha = __builtin_amdgcn_exp2f(m_i - m_new);
#pragma unroll
            for (int dt = 0; dt < NDT; ++dt) oacc[dt] *= alpha;
            l_i *= alpha;
            m_i = m_new;
        }
        float lsum = 0.f;
#pragma unroll
        for (int a = 0; a < 2; ++a) {
#pragma unroll
            for (int jj = 0; jj < 16; ++jj) {
                const float e = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[a][jj], sl, -m_i));
                sacc[a][jj] = e;
                if constexpr (!ONES) lsum += e;
            }
        }
        if constexpr (!ONES) l_i += lsum + xchg32(lsum);

#pragma unroll
        for (int a = 0; a < 2; ++a) {
            if (a >= nkt) break;
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const u32x4 pop = {E::pack(sacc[a][8 * h + 0], sacc[a][8 * h + 1]),
                                   E::pack(sacc[a][8 * h + 2], sacc[a][8 * h + 3]),
                                   E::pack(sacc[a][8 * h + 4], sacc[a][8 * h + 5]),
                                   E::pack(sacc[a][8 * h + 6], sacc[a][8 * h + 7])};
                const int kc = 8 * (2 * a + h) + 4 * g;  // the 16-key group's columns for group g
#pragma unroll
                for (int dt = 0; dt < NDT; ++dt)
                    oacc[dt] = E::mma(*(const u32x4 *)(vt + (32 * dt + r) * VTS + kc), pop, oacc[dt]);
            }
        }
        __builtin_amdgcn_sched_barrier(0);
        if (more) store_block(kb + kLongBKV, bf ^ 1);
        __syncthreads();
    }

    if constexpr (ONES) {
        // O^T row D (the ones row) is in element 4*((D % 32) / 8) of the last
        // d tile, held by the g = 0 lanes.
        constexpr int jl = 4 * ((D - 32 * (NDT - 1)) / 8);
        const float lv = oacc[NDT - 1][jl];
        const float lo = xchg32(lv);
        l_i = g ? lo : lv;
    }
    const int q = qblk * kLongBQ + 32 * w + r;
    if (q < L) {
        const float inv = 1.0f / l_i;
        char *orow = p.out + ((int64_t)(s0 + q) * p.so_s + (int64_t)head * p.so_h) * 2;
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt) {
#pragma unroll
            for (int jq = 0; jq < 4; ++jq) {
                const int d0 = 32 * dt + 8 * jq + 4 * g;
                if (d0 < D) {
                    const u32x2 wv = {E::pack(oacc[dt][4 * jq + 0] * inv, oacc[dt][4 * jq + 1] * inv),
                                      E::pack(oacc[dt][4 * jq + 2] * inv, oacc[dt][4 * jq + 3] * inv)};
                    *(u32x2 *)(orow + 2 * d0) = wv;
                }
            }
        }
    }
}

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

typedef void (*KernelFn)(KParams);

// The window kernel keeps the Q_rot and K_rot operands of 64 tokens in
// registers; above this head_dim the long kernel serves short segments too.
constexpr int kWindowMaxD = 96;

struct Choice {
    KernelFn fn;
    int kernel, grid, block, block_q, block_kv, lds;
    char name[64];
};

template <int D, class E, int RD, bool FULL> void pick_full(bool window, Choice &c) {
    if constexpr (D <= kWindowMaxD) {
        c.fn = window ? (KernelFn)window_kernel<D, E, RD, FULL> : (KernelFn)long_kernel<D, E, RD, FULL>;
    } else {
        c.fn = (KernelFn)long_kernel<D, E, RD, FULL>;
    }
}

template <int D, class E, int RD> void pick_rd(bool window, bool full, Choice &c) {
    if (full) pick_full<D, E, RD, true>(window, c);
    else pick_full<D, E, RD, false>(window, c);
}

template <int D> bool pick_d(bool window, bool full, int qkv, int rd, Choice &c) {
    if (qkv == FRA_DTYPE_BF16) {
        if (rd == FRA_DTYPE_F32) pick_rd<D, BF16, FRA_DTYPE_F32>(window, full, c);
        else if (rd == FRA_DTYPE_BF16) pick_rd<D, BF16, FRA_DTYPE_BF16>(window, full, c);
        else pick_rd<D, BF16, FRA_DTYPE_F16>(window, full, c);
    } else {
        if (rd == FRA_DTYPE_F32) pick_rd<D, F16, FRA_DTYPE_F32>(window, full, c);
        else if (rd == FRA_DTYPE_BF16) pick_rd<D, F16, FRA_DTYPE_BF16>(window, full, c);
        else pick_rd<D, F16, FRA_DTYPE_F16>(window, full, c);
    }
    if (window) {
        c.lds = full ? WinLds<D, true>::kBytes : WinLds<D, false>::kBytes;
    } else {
        c.lds = LongLds<D>::kBytes;
    }
    return true;
}

// Head dims with compiled kernels.  Each must be a multiple of 8 so that
// both halves of a row start on an 8-byte boundary.
bool pick_kernel(int d, bool window, bool full, int qkv, int rd, Choice &c) {
    switch (d) {
        case 64: return pick_d<64>(window, full, qkv, rd, c);
        case 72: return pick_d<72>(window, full, qkv, rd, c);
        case 80: return pick_d<80>(window, full, qkv, rd, c);
        case 96: return pick_d<96>(window, full, qkv, rd, c);
        case 128: return pick_d<128>(window, full, qkv, rd, c);
        default: return false;
    }
}

bool aligned(const void *ptr, int bytes) { return ((uintptr_t)ptr % (uintptr_t)bytes) == 0; }

const char *dtype_name(int dt) {
    switch (dt) {
        case FRA_DTYPE_BF16: return "bf16";
        case FRA_DTYPE_F16: return "f16";
        case FRA_DTYPE_F32: return "f32";
        default: return "?";
    }
}

int plan(const fra_fwd_args *a, Choice &c, KParams &kp) {
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
    if (a->rope_dtype != FRA_DTYPE_F32 && a->rope_dtype != FRA_DTYPE_BF16 && a->rope_dtype != FRA_DTYPE_F16)
        return fail(FRA_EINVAL, "rope_dtype must be f32, bf16 or f16, got %d", a->rope_dtype);
    const int d = a->head_dim;
    if (a->rope_width != d / 2 && a->rope_width != d)
        return fail(FRA_EINVAL, "rope_width must be head_dim/2=%d or head_dim=%d, got %d", d / 2, d, a->rope_width);
    if (!(a->softmax_scale > 0.f) || a->softmax_scale == __builtin_inff())
        return fail(FRA_EINVAL, "softmax_scale must be finite and > 0, got %g", (double)a->softmax_scale);
    if (!a->q || !a->k || !a->v || !a->cos || !a->sin || !a->out || !a->cu_seqlens)
        return fail(FRA_EINVAL, "a tensor pointer is NULL");
    const int64_t strides[9] = {a->q_stride_seq, a->q_stride_head, a->k_stride_seq, a->k_stride_head,
                                a->v_stride_seq, a->v_stride_head, a->out_stride_seq, a->out_stride_head,
                                a->rope_stride_seq};
    for (int i = 0; i < 9; ++i)
        if (strides[i] < 0) return fail(FRA_EINVAL, "strides must be >= 0");

    // The window kernel addresses 64 rows of a tensor with 32-bit offsets.
    const int64_t max_row_bytes = 2 * std::max(std::max(a->q_stride_seq, a->k_stride_seq),
                                               std::max(a->v_stride_seq, a->out_stride_seq));
    const bool small_rows = 64 * max_row_bytes < ((int64_t)1 << 31) && 64 * 4 * a->rope_stride_seq < ((int64_t)1 << 31);
    const bool window = a->max_seqlen <= 64 && d <= kWindowMaxD && small_rows;
    memset(&c, 0, sizeof(c));
    if (!pick_kernel(d, window, a->rope_width == d, a->qkv_dtype, a->rope_dtype, c))
        return fail(FRA_EUNSUPPORTED, "head_dim=%d has no compiled kernel (built: 64, 72, 80, 96, 128)", d);

    // Alignment: Q/K/out are read/written in 8-byte quads, V in 16-byte
    // chunks, fp32 tables in 16-byte quads and 16-bit tables in 8-byte quads.
    const int re = a->rope_dtype == FRA_DTYPE_F32 ? 4 : 2;
    if (!aligned(a->q, 8) || !aligned(a->k, 8) || !aligned(a->out, 8) || !aligned(a->v, 16) ||
        !aligned(a->cos, 4 * re) || !aligned(a->sin, 4 * re))
        return fail(FRA_EUNSUPPORTED, "tensor base pointers are not aligned (q/k/out 8 B, v 16 B, cos/sin %d B)", 4 * re);
    if (a->q_stride_seq % 4 || a->q_stride_head % 4 || a->k_stride_seq % 4 || a->k_stride_head % 4 ||
        a->out_stride_seq % 4 || a->out_stride_head % 4 || a->v_stride_seq % 8 || a->v_stride_head % 8 ||
        a->rope_stride_seq % 4)
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
    kp.sr_s = a->rope_stride_seq;
    kp.total = a->total_seq;
    kp.num_heads = a->num_heads;
    kp.num_seqs = a->num_seqs;
    kp.max_seqlen = a->max_seqlen;
    kp.scale_log2 = a->softmax_scale * kLog2e;

    const int64_t sh = (int64_t)a->num_seqs * a->num_heads;
    int64_t grid;
    if (window) {
        kp.qblocks = 1;
        grid = (int64_t)a->num_seqs * ((a->num_heads + kWinHeads - 1) / kWinHeads);
        c.kernel = FRA_KERNEL_WINDOW;
        c.block = kWinThreads;
        c.block_q = 64;
        c.block_kv = 64;
        snprintf(c.name, sizeof(c.name), "window_d%d_%s_rope%s", d, dtype_name(a->qkv_dtype),
                 dtype_name(a->rope_dtype));
    } else {
        kp.qblocks = (a->max_seqlen + kLongBQ - 1) / kLongBQ;
        grid = sh * kp.qblocks;
        c.kernel = FRA_KERNEL_LONG;
        c.block = kLongThreads;
        c.block_q = kLongBQ;
        c.block_kv = kLongBKV;
        snprintf(c.name, sizeof(c.name), "long_d%d_%s_rope%s", d, dtype_name(a->qkv_dtype),
                 dtype_name(a->rope_dtype));
    }
    if (grid > 0x7fffffff) return fail(FRA_EUNSUPPORTED, "grid of %lld workgroups is too large", (long long)grid);
    c.grid = (int)grid;
    return FRA_OK;
}

}  // namespace

extern "C" {

int fra_fwd_varlen(const fra_fwd_args *args, void *stream) {
    Choice c;
    KParams kp;
    const int rc = plan(args, c, kp);
    if (rc != FRA_OK) return rc;
    g_err[0] = 0;
    if (args->total_seq == 0) return FRA_OK;
    hipLaunchKernelGGL(c.fn, dim3(c.grid), dim3(c.block), 0, (hipStream_t)stream, kp);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(FRA_EHIP, "launch of %s failed: %s", c.name, hipGetErrorString(e));
    return FRA_OK;
}

int fra_query_plan(const fra_fwd_args *args, fra_plan *out) {
    if (!out) return fail(FRA_EINVAL, "plan is NULL");
    Choice c;
    KParams kp;
    const int rc = plan(args, c, kp);
    if (rc != FRA_OK) return rc;
    out->kernel = c.kernel;
    out->grid = c.grid;
    out->block = c.block;
    out->block_q = c.block_q;
    out->block_kv = c.block_kv;
    out->lds_bytes = c.lds;
    memcpy(out->name, c.name, sizeof(out->name));
    g_err[0] = 0;
    return FRA_OK;
}

int fra_supports_head_dim(int32_t head_dim) {
    Choice c;
    return pick_kernel(head_dim, true, false, FRA_DTYPE_BF16, FRA_DTYPE_F32, c) ? 1 : 0;
}

const char *fra_last_error(void) { return g_err; }

const char *fra_version(void) { return "fra 0.1.0 (gfx950)"; }

int32_t fra_abi_version(void) { return FRA_ABI_VERSION; }

int32_t fra_sizeof_args(void) { return (int32_t)sizeof(fra_fwd_args); }

int32_t fra_sizeof_plan(void) { return (int32_t)sizeof(fra_plan); }

}  // extern "C"
