// fra_fwd_kernels.h -- gfx950 forward kernels of the fused RoPE + varlen attention path.
// Included by fra_inst_fwd.hip, which instantiates them for one head_dim.
//
// Two kernel families replace the reference's single Triton kernel
// (reference fused_attn.py:235-423):
//
//   window_kernel  every segment has <= 64 tokens (Qwen2.5-VL window layers).
//                  One workgroup per (segment, group of 2 or 4 heads), one
//                  wavefront per head: Q, K and the cos/sin rows are loaded
//                  as coalesced slab rows, rotated in fp32 through LDS into
//                  MFMA operand registers, V goes from HBM straight to LDS,
//                  and each wavefront does one 64x64 softmax -- no online
//                  rescaling is needed.
//   long_kernel    segments of any length (full-attention layers).  Split-Q
//                  flash tiling: an 8-wave workgroup owns 256 query rows of
//                  one (segment, head); each wave runs an exp2 online softmax
//                  over its 32 rows.  With a workspace, krot_kernel first
//                  writes K rotated for the whole call and the K_rot and V
//                  blocks are staged in LDS by direct loads, with the two
//                  wavefronts of a SIMD half an iteration apart (ping-pong);
//                  without one, raw K and the cos/sin rows are staged and K
//                  is rotated once per block in LDS.  A partly filled last
//                  round of workgroups is split along the key range and
//                  merged by split_merge_kernel.
//
// Both can also write the softmax log-sum-exp for the backward (fra_bwd.hip).
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
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "fra.h"
#include "fra_device.h"
#include "fra_fwd_types.h"

namespace {

using namespace fra_internal;

// ---- rope from positions (fra_fwd_varlen_pos) ----------------------------------------
//
// The table of the position variant is never read: Rope<kRopePos> only
// supplies the element size its (unused) addressing assumes.
template <> struct Rope<kRopePos> {
    static constexpr int kBytes = 4;
    static __device__ __forceinline__ f32x4 quad(const char *) { return f32x4{0.f, 0.f, 0.f, 0.f}; }
};

// cos and sin of quad i (columns 4i .. 4i + 3) of the table row of a token at
// patch position (ph, pw), width D/2: column j < D/4 has the angle
// ph * inv_freq[j], column D/4 + j the angle pw * inv_freq[j] -- one fp32
// product each, the reference's outer product (compute_rope_2d,
// fused_attn.py:109-116, then .cos() / .sin()).
//
// The cosine and sine come from the hardware's v_cos_f32 / v_sin_f32, which
// take revolutions.  The angle's revolutions ang / (2 pi) are formed as an
// unevaluated sum hi + lo (Cody and Waite's split of the constant: hi =
// ang * c_hi rounded, lo = its rounding error, exact by FMA, plus
// ang * c_lo), and only the fraction of hi (exact for |hi| < 2^23) plus lo
// reaches the instruction, so no rounding of the reduction is ever larger
// than one ulp of the fraction.
constexpr float kInv2PiHi = 0.15915494f;            // fp32 of 1 / (2 pi)
constexpr float kInv2PiLo = 6.4206383e-09f;         // 1 / (2 pi) - kInv2PiHi
template <int D>
__device__ __forceinline__ void rope_pos_quad(const float *inv_freq, int ph, int pw, int i, f32x4 &c, f32x4 &s) {
    constexpr int F = D / 4;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const int col = 4 * i + e;
        const bool isw = col >= F;
        const float ang = (float)(isw ? pw : ph) * inv_freq[isw ? col - F : col];
        const float hi = ang * kInv2PiHi;
        const float lo = __builtin_fmaf(ang, kInv2PiHi, -hi) + ang * kInv2PiLo;
        const float fr = __builtin_amdgcn_fractf(hi) + lo;
        c[e] = __builtin_amdgcn_cosf(fr);
        s[e] = __builtin_amdgcn_sinf(fr);
    }
}

// load_rotate_quad (fra_device.h) with the angles of token `row` computed
// from its position instead of read from cos/sin rows.
template <int D, class E>
__device__ __forceinline__ void load_rotate_quad_pos(const char *xrow, const KParams &p, int64_t row, int i,
                                                     bool valid, u32x2 &r0w, u32x2 &r1w) {
    u32x2 x0 = *(const u32x2 *)(xrow + 8 * i);
    u32x2 x1 = *(const u32x2 *)(xrow + D + 8 * i);
    const int2 hw = *(const int2 *)(p.pos + 2 * row);
    f32x4 c, sn;
    rope_pos_quad<D>(p.inv_freq, hw.x, hw.y, i, c, sn);
    if (!valid) {
        x0 = u32x2{0u, 0u};
        x1 = u32x2{0u, 0u};
    }
    rotate_quad<E>(x0, x1, c, sn, c, sn, r0w, r1w);
}

// ---- window kernel ------------------------------------------------------------
//
// One workgroup of HW wavefronts per (segment, group of HW heads), HW = 2
// when that grid fits in one round of resident workgroups, else 4; segment
// length L <= 64.  All HBM traffic is coalesced: consecutive lanes move
// consecutive 16-byte chunks of the group's slab -- HW heads x D elements,
// contiguous in a [tokens, heads, head_dim] tensor -- and LDS turns the slab
// into MFMA operands (and the output back into slab rows).
//
//   1. the cos/sin rows and the Q and K slabs are loaded into registers up
//      front;
//   2. per 32-token half: the half's cos/sin rows -> LDS as fp32 rows, the
//      half's Q slab rows -> LDS, where wavefront w rotates the quads of head
//      HW*hg + w it feeds (fp32, rounded to the storage dtype); then the same
//      for K;
//   3. the V slab goes from HBM straight to LDS (global_load_lds_dwordx4) as
//      padded rows, over the dead staging buffers;
//   4. per 32-query tile: S^T = K_rot Q_rot^T, softmax, O^T = V^T P^T with the
//      V^T operands read by ds_read_b64_tr_b16; the normalised output stays in
//      registers as packed bf16/fp16;
//   5. the output rows go through LDS (over V) and leave as slab rows.
//
// Nothing but the staging buffers of one half lives in LDS while Q and K are
// rotated, and V never passes through registers, so at D = 80 a workgroup
// needs 28 KB of LDS with two heads (five fit on a CU) or 44 KB with four
// (three fit): a 144-window, 16-head layer (1152 two-head workgroups) runs in
// one round on 256 CUs.
//
// Rows past the segment (L < 64) load the segment's first (Q, K) or last (V)
// row: finite values whose keys are masked and whose queries are not stored.
//
// Lane (r, g) (r = lane & 31, g = lane >> 5) of a wavefront holds the
// operands of tokens r and r + 32: K_rot rows as the A operand of S^T and
// Q_rot rows as its B operand; MFMA step t, k-slot group g carries
// {x0r[4i..4i+3], x1r[4i..4i+3]} of quad i = g*S + t (the contraction order is
// free as long as Q and K share it).


// Bytes of an LDS row of V: at least `need`, a multiple of 64 bytes, and
// 16 or 48 dwords past a multiple of 64 dwords, so that the four rows one
// 16-lane group of a transposed read touches fall in disjoint banks.
constexpr int win_vpitch(int need) {
    int dw = (need + 63) / 64 * 16;
    while (dw % 64 != 16 && dw % 64 != 48) dw += 16;
    return 4 * dw;
}

// The items first, first + STEP, ... of a row-major [rows][N] grid as
// (row, col), stepped without divisions: STEP = Q*N + R.
template <int N, int STEP> struct GridWalk {
    static constexpr int Q = STEP / N, R = STEP % N;
    int row, col;
    __device__ __forceinline__ explicit GridWalk(int first) : row(first / N), col(first - (first / N) * N) {}
    // Advances to the next item; true when the column wrapped (one more row).
    __device__ __forceinline__ bool next() {
        row += Q;
        col += R;
        const bool carry = col >= N;
        if (carry) {
            col -= N;
            ++row;
        }
        return carry;
    }
};
template <bool B> struct BoolTag {
    static constexpr bool value = B;
};

template <int D, bool FULL, int HW> struct WinLds {
    static constexpr int W = FULL ? D : D / 2;         // table width
    static constexpr int CS = 2 * W + 4;               // fp32 per [cos | sin] row, +4 pad (conflict-free b128 reads)
    static constexpr int SLAB = HW * D * 2;            // bytes of one token's slab
    static constexpr int PITCH = SLAB + 16;            // LDS row pitch of a staged slab (one pad chunk)
    static constexpr int NDT = (D + 31) / 32;          // 32-row tiles of O^T
    // A V row holds the slab and the columns the last head's padding tile
    // reads past it (values only reach discarded output rows).
    static constexpr int VNEED = 2 * ((HW - 1) * D + 32 * NDT) > SLAB ? 2 * ((HW - 1) * D + 32 * NDT) : SLAB;
    static constexpr int VP = win_vpitch(VNEED);
    static constexpr int VPC = VP / 16;                // 16-byte slots per V row
    static constexpr int kTableBytes = 32 * CS * 4;    // tables of one 32-token half
    static constexpr int kHalfBytes = 32 * PITCH;      // Q or K slab rows of one half
    static constexpr int kRotBytes = kTableBytes + kHalfBytes;
    static constexpr int kVBytes = 64 * VP;
    static constexpr int kOutBytes = 64 * PITCH;
    static constexpr int kMax2 = kVBytes > kOutBytes ? kVBytes : kOutBytes;
    static constexpr int kMain = kRotBytes > kMax2 ? kRotBytes : kMax2;
    static constexpr int kBytes = kMain + 16;          // + a 16-byte trash slot
    // Wavefronts per SIMD the register budget is sized for: three
    // workgroups per CU when their LDS fits and the loads held in registers
    // leave room (half-width tables, D = 64 or 80: at most 166 VGPRs without
    // spills), else two.
    static constexpr int kWaves = !FULL && D <= 80 && D % 16 == 0 && 3 * kBytes <= 160 * 1024 ? 3 : 2;
    // Workgroups per CU (LDS and wavefronts per SIMD), for the planner.
    // Wavefronts per workgroup: one per head, except HW = 1, where two
    // wavefronts split the head's 64 queries (one 32-query tile each).
    static constexpr int kWgWaves = HW == 1 ? 2 : HW;
    static constexpr int kPerCu = (160 * 1024 / kBytes) < (4 * kWaves / kWgWaves) ? (160 * 1024 / kBytes) : (4 * kWaves / kWgWaves);
};

template <int D, class E, int RD, bool FULL, int HW, bool GATHER>
__global__ __launch_bounds__((64 * WinLds<D, FULL, HW>::kWgWaves), (WinLds<D, FULL, HW>::kWaves)) void window_kernel(const KParams p) {
    using LDS = WinLds<D, FULL, HW>;
    constexpr int kWinHeads = HW;
    constexpr int kWinWaves = LDS::kWgWaves;
    constexpr int kWinThreads = 64 * kWinWaves;
    // HW = 1 (query split): both wavefronts work on the one head; wavefront
    // w rotates the queries of tile w and attends them (a layer with few
    // (segment, head) pairs gets twice the wavefronts, each with half the
    // chain).  Otherwise wavefront w owns head w of the group, both tiles.
    constexpr bool QSPLIT = HW == 1;
    constexpr int NQ = D / 8;                 // quads per half
    constexpr int S = (NQ + 1) / 2;           // 16-deep k-steps of QK^T
    constexpr int NDT = LDS::NDT;
    constexpr int W = LDS::W;
    constexpr int CS = LDS::CS;
    constexpr int PITCH = LDS::PITCH;
    constexpr int VP = LDS::VP, VPC = LDS::VPC;
    constexpr int HCH = D / 8;                // 16-byte chunks per head row
    constexpr int NCH = kWinHeads * HCH;      // chunks per slab row
    constexpr int RB = Rope<RD>::kBytes;
    constexpr int TQ = W / 4;                 // table quads per row
    constexpr int TN = 2 * TQ;                // table items per token: cos quads, then sin quads
    constexpr int TITEMS = 64 * TN;
    constexpr int TPER = (TITEMS + kWinThreads - 1) / kWinThreads;
    constexpr int SPER = 64 * NCH / kWinThreads;  // (token, chunk) items of a slab per thread
    static_assert(64 * NCH % kWinThreads == 0, "slab items divide evenly");
    // Item k of a slab belongs to half k / (SPER / 2) when a half is a whole
    // number of item rounds (D != 72); otherwise it is tested per item.
    constexpr bool KHALF = 32 * NCH % kWinThreads == 0;
    constexpr int VPER = (VPC + kWinWaves - 1) / kWinWaves;  // V direct loads per wavefront
    typedef short v4i16 __attribute__((ext_vector_type(4)));
    typedef __attribute__((address_space(3))) v4i16 lds_v4i16;
    typedef __attribute__((address_space(3))) void lds_void;
    typedef __attribute__((address_space(1))) void glb_void;
    __shared__ __attribute__((aligned(16))) char lds[LDS::kBytes];
    float *tab = (float *)lds;                                  // [32][CS] fp32 tables of one half
    char *half = lds + LDS::kTableBytes;                        // [32][PITCH]: one half of a Q or K slab
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
    const bool active = QSPLIT || w < nh;  // wavefronts past the last head still take part in barriers
    const int hw = QSPLIT ? 0 : w;         // this wavefront's head in the group
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
    const uint32_t trs = (uint32_t)p.sr_s * RB;
    // Full window, four heads, each token's heads adjacent in every tensor:
    // chunk c of slab row t is at t * row_stride + 16 c, and row offsets are
    // stepped instead of multiplied.
    const bool fast = !GATHER && p.dense_heads && nh == kWinHeads && L == 64;  // uniform
    // GATHER (fra_fwd_varlen_gather): slot s0 + t of the window is tensor row
    // p.rows[s0 + t] (clamped into the tensors), for every tensor and table;
    // byte offset of that row from row s0 at row stride rs.
    auto grow_bytes = [&](int t, uint32_t rs) -> int64_t {
        const int rr = min(max(p.rows[s0 + t], 0), p.total - 1);
        return (int64_t)(rr - s0) * rs;
    };
    // Byte offset of chunk `col` of a slab row: head col / HCH (heads past
    // the group's last read its first), chunk col % HCH.
    auto chunk_off = [&](int col, uint32_t hs) {
        const int hh = col / HCH;
        const uint32_t hd = hh < nh ? (uint32_t)hh : 0u;
        return hd * hs + (uint32_t)(16 * (col - hh * HCH));
    };

    // ---- 1. global loads into registers, back to back: tables, Q and K slabs -------
    // Q and K are read once and the output is written once: those accesses
    // are non-temporal, so that they neither evict the cos/sin rows the
    // window's other head groups share nor leave dirty output lines in L2
    // for the end of the kernel to write back (measured: 1.6 us of 29 at a
    // 144-window layer).
    // The position variant loads each item's (h, w) instead (items (token,
    // quad) of the cos and sin rows at once) and computes the quads below,
    // while the Q and K slabs are still in flight.
    constexpr bool POS = RD == kRopePos;
    constexpr int PITEMS = 64 * TQ;
    constexpr int PPER = (PITEMS + kWinThreads - 1) / kWinThreads;
    f32x4 tv[POS ? 1 : TPER];
    int2 tpos[POS ? PPER : 1];
    f32x4 tvc[POS ? PPER : 1], tvs[POS ? PPER : 1];
    if constexpr (POS) {
        GridWalk<TQ, kWinThreads> it(fresh(tid));
#pragma unroll
        for (int k = 0; k < PPER; ++k) {
            const int tok = min(it.row, 63);
            const int tt = tok < L ? tok : 0;
            if constexpr (GATHER) tpos[k] = *(const int2 *)(p.pos + 2 * ((int64_t)s0 + grow_bytes(tt, 1)));
            else tpos[k] = *(const int2 *)(p.pos + 2 * ((int64_t)s0 + tt));
            it.next();
        }
    } else {
        GridWalk<TN, kWinThreads> it(fresh(tid));
#pragma unroll
        for (int k = 0; k < TPER; ++k) {
            const int tok = min(it.row, 63), c = it.col;
            const bool is_sin = c >= TQ;
            const uint32_t qoff = (uint32_t)(4 * RB * (is_sin ? c - TQ : c));
            if constexpr (GATHER) {
                tv[k] = Rope<RD>::quad((is_sin ? sb : cb) + grow_bytes(tok < L ? tok : 0, trs) + qoff);
            } else {
                const uint32_t off = (uint32_t)(tok < L ? tok : 0) * trs + qoff;
                tv[k] = Rope<RD>::quad((is_sin ? sb : cb) + off);
            }
            it.next();
        }
    }
    u32x4 qs[SPER], ks[SPER];
    {
        const uint32_t qrs = (uint32_t)p.sq_s * 2, krs = (uint32_t)p.sk_s * 2;
        const uint32_t qhs = (uint32_t)p.sq_h * 2, khs = (uint32_t)p.sk_h * 2;
        auto load_slabs = [&](auto fast_tag) {
            constexpr bool F = decltype(fast_tag)::value;
            GridWalk<NCH, kWinThreads> it(fresh(tid));
            uint32_t qro = (uint32_t)it.row * qrs, kro = (uint32_t)it.row * krs;
#pragma unroll
            for (int k = 0; k < SPER; ++k) {
                if constexpr (F) {
                    qs[k] = __builtin_nontemporal_load((const u32x4 *)(qb + (qro + 16 * it.col)));
                    ks[k] = __builtin_nontemporal_load((const u32x4 *)(kb + (kro + 16 * it.col)));
                } else if constexpr (GATHER) {
                    const int row = it.row < L ? it.row : 0;
                    qs[k] = __builtin_nontemporal_load((const u32x4 *)(qb + grow_bytes(row, qrs) + chunk_off(it.col, qhs)));
                    ks[k] = __builtin_nontemporal_load((const u32x4 *)(kb + grow_bytes(row, krs) + chunk_off(it.col, khs)));
                } else {
                    const uint32_t row = it.row < L ? (uint32_t)it.row : 0u;
                    qs[k] = __builtin_nontemporal_load((const u32x4 *)(qb + (row * qrs + chunk_off(it.col, qhs))));
                    ks[k] = __builtin_nontemporal_load((const u32x4 *)(kb + (row * krs + chunk_off(it.col, khs))));
                }
                const bool cy = it.next();
                if constexpr (F) {
                    qro += GridWalk<NCH, kWinThreads>::Q * qrs + (cy ? qrs : 0u);
                    kro += GridWalk<NCH, kWinThreads>::Q * krs + (cy ? krs : 0u);
                }
            }
        };
        if (fast) load_slabs(BoolTag<true>{});
        else load_slabs(BoolTag<false>{});
    }
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (POS) {
        GridWalk<TQ, kWinThreads> it(fresh(tid));
#pragma unroll
        for (int k = 0; k < PPER; ++k) {
            rope_pos_quad<D>(p.inv_freq, tpos[k].x, tpos[k].y, it.col, tvc[k], tvs[k]);
            it.next();
        }
    }

    // ---- 2. per half: tables and Q staged and rotated, then K ------------------------
    // Staging writes are branch-free (a branch here would make the compiler
    // wait for every outstanding load): items of the other half go to the
    // trash slot unless the half is known per item at compile time.
    auto stage_tab = [&](int hf) {
        if constexpr (POS) {
            GridWalk<TQ, kWinThreads> it(fresh(tid));
#pragma unroll
            for (int k = 0; k < PPER; ++k) {
                const bool in = (PITEMS % kWinThreads == 0 || it.row < 64) && (it.row >> 5) == hf;
                float *dst = tab + (it.row - 32 * hf) * CS + 4 * it.col;
                *(f32x4 *)(in ? (char *)dst : trash) = tvc[k];
                *(f32x4 *)(in ? (char *)(dst + W) : trash) = tvs[k];
                it.next();
            }
            return;
        }
        GridWalk<TN, kWinThreads> it(fresh(tid));
#pragma unroll
        for (int k = 0; k < TPER; ++k) {
            const bool in = (TITEMS % kWinThreads == 0 || it.row < 64) && (it.row >> 5) == hf;
            const int c = it.col, is_sin = c >= TQ ? 1 : 0;
            char *dst = (char *)(tab + (it.row - 32 * hf) * CS + is_sin * W + 4 * (c - is_sin * TQ));
            *(f32x4 *)(in ? dst : trash) = tv[k];
            it.next();
        }
    };
    auto stage_half = [&](const u32x4 (&x)[SPER], int hf) {
        GridWalk<NCH, kWinThreads> it(fresh(tid));
#pragma unroll
        for (int k = 0; k < SPER; ++k) {
            char *dst = half + (it.row - 32 * hf) * PITCH + 16 * it.col;
            if constexpr (KHALF) {
                if (k / (SPER / 2) == hf) *(u32x4 *)dst = x[k];
            } else {
                *(u32x4 *)((it.row >> 5) == hf ? dst : trash) = x[k];
            }
            it.next();
        }
    };
    // Rotates this wavefront's quads of the staged half into MFMA operands.
    // Quad i = g*S + t exists unless NQ is odd and it is the last one.
    auto rotate_half = [&](u32x4 (&op)[S]) {
        const float *crow = tab + r * CS;
        const char *xrow = half + r * PITCH + hw * (2 * D);
#pragma unroll
        for (int t = 0; t < S; ++t) {
            const bool maybe_pad = t >= NQ - S;   // compile time; true only for odd NQ
            const int i = g * S + t;
            const int il = maybe_pad ? (i < NQ ? i : 0) : i;
            const f32x4 c0 = *(const f32x4 *)(crow + 4 * il);
            const f32x4 s0v = *(const f32x4 *)(crow + W + 4 * il);
            f32x4 c1 = c0, s1v = s0v;
            if constexpr (FULL) {
                c1 = *(const f32x4 *)(crow + D / 2 + 4 * il);
                s1v = *(const f32x4 *)(crow + W + D / 2 + 4 * il);
            }
            u32x2 x0 = *(const u32x2 *)(xrow + 8 * il);
            u32x2 x1 = *(const u32x2 *)(xrow + D + 8 * il);
            if (maybe_pad && i >= NQ) x0 = x1 = u32x2{0u, 0u};
            u32x2 a0, a1;
            rotate_quad<E>(x0, x1, c0, s0v, c1, s1v, a0, a1);
            op[t] = u32x4{a0[0], a0[1], a1[0], a1[1]};
        }
        // The packed operands are materialised here: left to itself the
        // compiler sinks the rotation towards the attention that consumes it
        // and keeps its fp32 intermediates (twice the registers) alive
        // across the staging of the next slabs.
#pragma unroll
        for (int t = 0; t < S; ++t) asm volatile("" : "+v"(op[t]));
    };
    u32x4 qop[2][S], kop[2][S];
#pragma unroll
    for (int hf = 0; hf < 2; ++hf) {
        if (hf == 1 && L <= 32) break;  // uniform: no second half (its operands are never read)
        stage_tab(hf);
        stage_half(qs, hf);
        __syncthreads();
        if (!QSPLIT || w == hf) rotate_half(qop[hf]);
        __syncthreads();
        stage_half(ks, hf);
        __syncthreads();
        rotate_half(kop[hf]);
        __syncthreads();  // tables and the staged slab are dead
    }

    // ---- 3. V rows straight from HBM into LDS ------------------------------------------
    // Direct load m moves LDS slots 64m .. 64m + 63 (16 bytes each, lane =
    // slot): slot s is chunk s % VPC of V row s / VPC.  Slots past the slab
    // are padding and not loaded; rows past the segment load its last row.
    {
        const uint32_t vrs = (uint32_t)p.sv_s * 2, vhs = (uint32_t)p.sv_h * 2;
        auto load_v = [&](auto fast_tag) {
            constexpr bool F = decltype(fast_tag)::value;
            GridWalk<VPC, kWinThreads> it(fresh(tid));  // slot 64 (w + waves k) + lane
            uint32_t vro = (uint32_t)it.row * vrs;
#pragma unroll
            for (int k = 0; k < VPER; ++k) {
                const int m = w + kWinWaves * k;
                if (VPC % kWinWaves == 0 || m < VPC) {  // uniform
                    if (it.col < NCH) {
                        const char *src;
                        if constexpr (F) src = vb + (vro + 16 * it.col);
                        else if constexpr (GATHER) src = vb + grow_bytes(min(it.row, L - 1), vrs) + chunk_off(it.col, vhs);
                        else src = vb + ((uint32_t)min(it.row, L - 1) * vrs + chunk_off(it.col, vhs));
                        __builtin_amdgcn_global_load_lds((glb_void *)src, (lds_void *)(lds + 1024 * m), 16, 0, 0);
                    }
                }
                const bool cy = it.next();
                if constexpr (F) vro += GridWalk<VPC, kWinThreads>::Q * vrs + (cy ? vrs : 0u);
            }
        };
        if (fast) load_v(BoolTag<true>{});
        else load_v(BoolTag<false>{});
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    }
    __syncthreads();

    // ---- 4. attention per 32-query tile ---------------------------------------------
    // The two tiles run one after the other (a scheduling barrier between
    // them keeps the compiler from overlapping them, which would need both
    // tiles' registers at once); a tile's packed output is kept in registers
    // until V is dead.
    //
    // V^T operands: ds_read_b64_tr_b16 works on groups of 16 lanes; lane
    // c = 4e + qq of a group addresses the 8 bytes at V[row0 + e][col0 + 4qq],
    // and lane i of the group receives V[row0 + 0..3][col0 + i].  Group G =
    // lane >> 4 takes columns 16 (G & 1) of the 32-column tile and rows 4g,
    // so lane l receives keys 4g .. 4g + 3 of column (l & 31): the A operand
    // of O^T = V^T P^T for k-slots 0..3, and the read 8 rows further down for
    // k-slots 4..7.
    constexpr int OQV = (D / 32) * 4 + (D % 32) / 8;  // quads with d0 < D for g = 0 (D % 8 == 0)
    const float sl = p.scale_log2;
    const int nkt = (L + 31) >> 5;
    const uint32_t v_lane =
        (uint32_t)((4 * g + ((lane >> 2) & 3)) * VP + 2 * (hw * D + 16 * ((lane >> 4) & 1) + 4 * (lane & 3)));
    // Output quad i of a tile: d0 = 32 (i / 4) + 8 (i % 4) + 4g.  Quads past
    // OQV (d0 >= D for both g) are not kept; quad OQV - 1 may be half valid.
    auto tile = [&](const u32x4 (&qcur)[S], u32x2 (&outq)[OQV], int b) {
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
        if (L < 64) {  // uniform: keys past the segment
#pragma unroll
            for (int a = 0; a < 2; ++a) {
#pragma unroll
                for (int j = 0; j < 16; ++j) {
                    const int kv = 32 * a + 8 * (j >> 2) + 4 * g + (j & 3);
                    if (kv >= L) sacc[a][j] = kNegInf;
                }
            }
        }
        float t8[11];
#pragma unroll
        for (int k = 0; k < 10; ++k) {
            const int e = 3 * k;
            t8[k] = max3f(sacc[e >> 4][e & 15], sacc[(e + 1) >> 4][(e + 1) & 15], sacc[(e + 2) >> 4][(e + 2) & 15]);
        }
        t8[10] = fmaxf(sacc[1][14], sacc[1][15]);
        float mx = fmaxf(max3f(max3f(t8[0], t8[1], t8[2]), max3f(t8[3], t8[4], t8[5]), max3f(t8[6], t8[7], t8[8])),
                         fmaxf(t8[9], t8[10]));
        mx = max_pair32(mx);
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
        lsum = sum_pair32(lsum);
        const float inv = 1.0f / lsum;
        if (p.lse != nullptr && g == 0 && 32 * b + r < L)
            p.lse[(int64_t)(h0 + hw) * p.total + s0 + (GATHER ? grow_bytes(32 * b + r, 1) : 32 * b + r)] =
                (__builtin_amdgcn_logf(lsum) - mneg) * kLn2;

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
        // q = 32b + r, d = 32dt + 8(j/4) + 4g + (j%4).  Rows d >= D read
        // columns of the next head or row padding; they are never stored.
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt) {
            f32x16 oacc = f32x16{};
#pragma unroll
            for (int a = 0; a < 2; ++a) {
                if (a >= nkt) break;
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    const char *cp = lds + v_lane + (32 * a + 16 * h) * VP + 64 * dt;
                    const v4i16 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16 *)cp);
                    const v4i16 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16 *)(cp + 8 * VP));
                    const u32x2 l2 = __builtin_bit_cast(u32x2, lo), h2 = __builtin_bit_cast(u32x2, hi);
                    oacc = E::mma(u32x4{l2[0], l2[1], h2[0], h2[1]}, pop[a][h], oacc);
                }
            }
#pragma unroll
            for (int jq = 0; jq < 4; ++jq)
                if (4 * dt + jq < OQV)
                    outq[4 * dt + jq] = u32x2{E::pack(oacc[4 * jq + 0] * inv, oacc[4 * jq + 1] * inv),
                                              E::pack(oacc[4 * jq + 2] * inv, oacc[4 * jq + 3] * inv)};
        }
    };
    u32x2 out0[OQV], out1[OQV];
    if constexpr (QSPLIT) {
        if (w == 0) tile(qop[0], out0, 0);
        else if (L > 32) tile(qop[1], out0, 1);
    } else if (active) {  // uniform within the wavefront; no barrier inside
        tile(qop[0], out0, 0);
        __builtin_amdgcn_sched_barrier(0);
        if (L > 32) tile(qop[1], out1, 1);
    }
    __syncthreads();  // V is dead: the output rows go over it

    // ---- 5. output rows through LDS, stored as coalesced slab rows --------------------
    if (active) {
        auto put = [&](const u32x2 (&outq)[OQV], int b) {
            char *orow = oslab + (32 * b + r) * PITCH + hw * (2 * D);
#pragma unroll
            for (int i = 0; i < OQV; ++i) {
                const int d0 = 32 * (i / 4) + 8 * (i % 4) + 4 * g;
                if (d0 < D) *(u32x2 *)(orow + 2 * d0) = outq[i];
            }
        };
        if constexpr (QSPLIT) {
            if (w == 0 || L > 32) put(out0, w);
        } else {
            put(out0, 0);
            if (L > 32) put(out1, 1);
        }
    }
    __syncthreads();
    {
        char *ob = p.out + ((int64_t)s0 * p.so_s + (int64_t)h0 * p.so_h) * 2;
        const uint32_t ors = (uint32_t)p.so_s * 2, ohs = (uint32_t)p.so_h * 2;
        auto store = [&](auto fast_tag) {
            constexpr bool F = decltype(fast_tag)::value;
            GridWalk<NCH, kWinThreads> it(fresh(tid));
            uint32_t oro = (uint32_t)it.row * ors;
#pragma unroll
            for (int k = 0; k < SPER; ++k) {
                const u32x4 val = *(const u32x4 *)(oslab + it.row * PITCH + 16 * it.col);
                if constexpr (F) {
                    __builtin_nontemporal_store(val, (u32x4 *)(ob + (oro + 16 * it.col)));
                } else if (it.row < L && it.col < nh * HCH) {
                    if constexpr (GATHER)
                        __builtin_nontemporal_store(val, (u32x4 *)(ob + grow_bytes(it.row, ors) + chunk_off(it.col, ohs)));
                    else
                        __builtin_nontemporal_store(val, (u32x4 *)(ob + ((uint32_t)it.row * ors + chunk_off(it.col, ohs))));
                }
                const bool cy = it.next();
                if constexpr (F) oro += GridWalk<NCH, kWinThreads>::Q * ors + (cy ? ors : 0u);
            }
        };
        if (fast) store(BoolTag<true>{});
        else store(BoolTag<false>{});
    }
}

// ---- long kernel ----------------------------------------------------------------
//
// Split-Q flash tiling for segments of any length.  A workgroup of 8
// wavefronts (two per SIMD) owns 256 query rows of one (segment, head) --
// wavefront w rows 32w..32w+31 -- and walks the segment's keys in blocks of 64.
//
// Staging.  Raw K rows, their cos/sin rows and V rows go from HBM straight to
// LDS (global_load_lds_dwordx4: lane l of an instruction writes the 16 bytes
// at LDS base + 16 l).  Each staged block is row-major in LDS, a row of
// 16-byte chunks padded to a pitch that keeps the reads below free of bank
// conflicts, and an instruction moves 64 consecutive chunk slots: whole rows,
// so that its global reads are coalesced (slots of the padding are not
// loaded).  A lane's slot, and so its offset row * row_stride + 16 * chunk,
// is the same in every block.  K is rotated from LDS into a row-major K_rot
// buffer once per block for all query rows of the workgroup (wavefront w
// takes quads w, w + kLongWaves, ... of all 64 rows).  V stays as loaded;
// ds_read_b64_tr_b16 reads it back transposed into the A operand of
// O^T = V^T P^T.
//
// Pipeline.  Iteration j overlaps matrix-core and vector work of one wavefront:
//
//     phase A:  S(j+1) = K_rot(j+1) Q_rot^T  (MFMA)   with  softmax of S(j)  (VALU)
//     phase B:  O^T += V(j)^T P(j)^T          (MFMA)   with  rotation of K(j+2) (VALU)
//
// while the direct loads of raw K(j+3) (+cos/sin) and V(j+1) are in flight;
// one barrier ends the iteration.  Buffers: K_rot and V double-buffered (block
// x in buffer x & 1), raw K/cos/sin double-buffered when LDS allows (else one
// buffer, K(j+2) loaded in iteration j, and a second barrier between the
// phases).
//
// Softmax: exp2 online softmax with the row max from v_max3 chains and one
// exchange with lane^32; the running max is only moved (and O rescaled) when a
// row max exceeds it by more than 2^8, so in the steady state no rescaling
// happens and P stays below 2^8.  When head_dim leaves padding columns in the
// last 32-column tile of V, column D holds ones, so the PV MFMA also produces
// the row sum of the rounded P (otherwise the sum is taken on the VALU).
//
// Rows of the last (partial) block past the segment load row nkv-1 instead
// (finite values), and their scores are masked to -inf, so they add nothing.
//
// ds_read_b64_tr_b16 (gfx950) works on groups of 16 lanes: lane c of a group
// supplies the address of a 4-element (8-byte) chunk, and lane i of the group
// receives element (i & 3) of the chunks of lanes i/4, 4 + i/4, 8 + i/4 and
// 12 + i/4.  With lane c = 4e + qq pointing at V[row0 + e][col0 + 4qq], lane i
// receives V[row0 + 0..3][col0 + i]: four consecutive keys of column col0 + i.

constexpr float kRescaleThreshold = 8.0f;  // log2 units
constexpr int kLdsLimit = 160 * 1024;

// Chunks of an LDS row of V: at least `need`, 4 or 12 mod 16.
constexpr int long_vpitch(int need) {
    int c = need;
    while (c % 16 != 4 && c % 16 != 12) ++c;
    return c;
}

// PRE: K comes rotated (k_rot rows in the caller's workspace, written by
// krot_kernel once per call); the direct loads then fill the K_rot buffers
// themselves and there is no raw staging or rotation in the loop.
template <int D, int RD, bool FULL, bool PRE = false> struct LongLds {
    static constexpr int RB = Rope<RD>::kBytes;
    static constexpr int HALF = D / 2;
    static constexpr int W = FULL ? D : D / 2;         // table width
    static constexpr int DP = (D + 15) / 16 * 16;      // K_rot row padded to the MFMA k-step
    static constexpr int KS = DP + 8;                  // K_rot row pitch (elements), 16 B pad
    static constexpr int NDT = (D + 31) / 32;          // 32-row tiles of O^T
    static constexpr int KCH = D / 8;                  // 16-byte chunks of a K or V row
    static constexpr int TCH = W * RB / 16;            // 16-byte chunks of a table row
    // Row pitches in 16-byte chunks.  Raw K and table rows: an odd number of
    // chunks, so 16 consecutive rows start in 16 different 4-bank groups
    // (16-byte reads conflict-free, 8-byte reads at most 2-way).  V rows:
    // 4 or 12 mod 16 chunks (16 or 48 dwords mod 64), so the four rows a
    // 16-lane group of a transposed read touches fall in disjoint banks; a
    // row also holds the columns [D, 32 NDT) the last O^T tile reads.
    static constexpr int KPC = KCH % 2 ? KCH : KCH + 1;
    static constexpr int TPC = TCH % 2 ? TCH : TCH + 1;
    static constexpr int VPC = long_vpitch(4 * NDT);
    static constexpr bool kOnesCol = D % 32 != 0;      // V column D holds ones
    static constexpr int kRawK = 64 * KPC * 16;
    static constexpr int kRawT = 64 * TPC * 16;
    static constexpr int kRaw = kRawK + 2 * kRawT;     // raw K, cos, sin of one block
    static constexpr int kKrot = kLongBKV * KS * 2;
    static constexpr int kV = 64 * VPC * 16;
    static constexpr int KRC = KS * 2 / 16;            // K_rot row pitch in 16-byte chunks (odd)
    static constexpr int kRawBufs = PRE ? 2 : (2 * (kRaw + kKrot + kV) <= kLdsLimit ? 2 : 1);
    static constexpr int kOffKrot = PRE ? 0 : kRawBufs * kRaw;
    static constexpr int kOffV = kOffKrot + 2 * kKrot;
    static constexpr int kBytes = kOffV + 2 * kV;
    static_assert(kBytes <= kLdsLimit, "long kernel LDS budget");
    static_assert(W * RB % 16 == 0, "table rows must be whole 16-byte chunks");
};

// k_rot = rot(k) for every row, [total, heads, head_dim] dense, into the
// workspace: the long kernel's PRE variant then stages K_rot blocks
// directly instead of staging raw K and the tables and rotating each block
// once per query block (reference fused_attn.py:364-390 recomputes it per
// query block too).  One thread per (token, head, quad i): quads i of both
// halves, rotate_quad's arithmetic.
template <int D, class E, int RD, bool FULL>
__global__ __launch_bounds__(256) void krot_kernel(const KParams p) {
    constexpr int NQ = D / 8, HALF = D / 2, RB = Rope<RD>::kBytes;
    const int64_t it = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (it >= (int64_t)p.total * p.num_heads * NQ) return;
    const int64_t row = it / NQ;
    const int i = (int)(it - row * NQ);
    const int t = (int)(row / p.num_heads), h = (int)(row - (int64_t)t * p.num_heads);
    u32x2 r0, r1;
    if constexpr (RD == kRopePos)
        load_rotate_quad_pos<D, E>(p.k + ((int64_t)t * p.sk_s + (int64_t)h * p.sk_h) * 2, p, t, i, true, r0, r1);
    else
        load_rotate_quad<D, E, RD, FULL>(p.k + ((int64_t)t * p.sk_s + (int64_t)h * p.sk_h) * 2,
                                         p.cos + (int64_t)t * p.sr_s * RB, p.sin + (int64_t)t * p.sr_s * RB, i, true,
                                         r0, r1);
    char *dst = p.krot + row * (D * 2);
    *(u32x2 *)(dst + 8 * i) = r0;
    *(u32x2 *)(dst + 2 * HALF + 8 * i) = r1;
}

// ---- split last round: partial results and their merge ------------------------
//
// Workspace: per (split unit, part), kLongBQ rows of split_row_floats(D) floats:
// O (unnormalised, head_dim values), m (running max in scale*log2e units) and
// l (row sum of P).  split_merge_kernel, launched after the long kernel on
// the same stream, merges the parts of each unit into the output.

// This workgroup's partial rows (one per lane row q < L).
template <int D>
__device__ __forceinline__ void split_write_partial(const KParams &p, int u, int part, int nparts, int q, int L,
                                                    int w, int r, int g, float m_i, float l_i,
                                                    const f32x16 (&oacc)[(D + 31) / 32]) {
    constexpr int NDT = (D + 31) / 32;
    constexpr int RF = split_row_floats(D);
    if (q >= L) return;
    float *row = (float *)p.ws + ((int64_t)((u - p.tail_first) * nparts + part) * kLongBQ + 32 * w + r) * RF;
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) {
#pragma unroll
        for (int jq = 0; jq < 4; ++jq) {
            const int d0 = 32 * dt + 8 * jq + 4 * g;
            if (d0 < D)
                *(f32x4 *)(row + d0) = f32x4{oacc[dt][4 * jq + 0], oacc[dt][4 * jq + 1], oacc[dt][4 * jq + 2],
                                             oacc[dt][4 * jq + 3]};
        }
    }
    if (g == 0) {
        typedef __attribute__((__vector_size__(2 * sizeof(float)))) float f32x2;
        *(f32x2 *)(row + D) = f32x2{m_i, l_i};
    }
}

// O = sum_p 2^(m_p - m) O_p / sum_p 2^(m_p - m) l_p with m = max_p m_p,
// rounded to the output dtype.  Items are (row, 8-column chunk) of a split
// unit, one per thread (consecutive threads on consecutive chunks of a row):
// workgroup (tu, blk) of the grid split_units x split_merge_blocks takes
// items 256 blk .. 256 blk + 255 of unit tu.
template <int D, class E>
__global__ __launch_bounds__(256) void split_merge_kernel(const KParams p) {
    constexpr int RF = split_row_floats(D);
    static_assert(D % 8 == 0, "8-column items");
    constexpr int NC = D / 8;
    constexpr int BPU = split_merge_blocks(D);  // workgroups per unit
    typedef __attribute__((__vector_size__(2 * sizeof(float)))) float f32x2;
    const int tu = blockIdx.x / BPU, blk = blockIdx.x - tu * BPU;
    const int u = p.tail_first + tu, nparts = p.tail_split;
    const int pi = u / p.qblocks, qblk = u - pi * p.qblocks;
    const int sh = long_pair(pi, p.num_seqs * p.num_heads);
    const int seg = sh / p.num_heads, head = sh - seg * p.num_heads;
    int s0 = p.cu[seg], s1 = p.cu[seg + 1];
    s0 = min(max(s0, 0), p.total);
    s1 = min(max(s1, 0), p.total);
    const int L = s1 - s0;
    const int it = blk * 256 + threadIdx.x;
    if (it >= kLongBQ * NC) return;
    const int row = it / NC, c = it - row * NC;
    const int q = qblk * kLongBQ + row;
    if (L <= 0 || q >= L) return;
    const float *base = (const float *)p.ws + ((int64_t)tu * nparts * kLongBQ + row) * RF;
    float mp[kSplitMaxParts], lp[kSplitMaxParts];
    f32x4 op[kSplitMaxParts][2];
#pragma unroll
    for (int pp = 0; pp < kSplitMaxParts; ++pp) {
        if (pp < nparts) {
            const float *pr = base + (int64_t)pp * kLongBQ * RF;
            const f32x2 ml = *(const f32x2 *)(pr + D);  // D % 8 == 0: 8-byte aligned
            mp[pp] = ml[0];
            lp[pp] = ml[1];
            op[pp][0] = *(const f32x4 *)(pr + 8 * c);
            op[pp][1] = *(const f32x4 *)(pr + 8 * c + 4);
        }
    }
    float mx = kNegInf;
#pragma unroll
    for (int pp = 0; pp < kSplitMaxParts; ++pp)
        if (pp < nparts) mx = fmaxf(mx, mp[pp]);
    float l = 0.f;
    f32x4 acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = acc0;
#pragma unroll
    for (int pp = 0; pp < kSplitMaxParts; ++pp) {
        if (pp < nparts && mp[pp] != kNegInf) {  // a part with no keys adds nothing
            const float wt = __builtin_amdgcn_exp2f(mp[pp] - mx);
            l += wt * lp[pp];
            acc0 += wt * op[pp][0];
            acc1 += wt * op[pp][1];
        }
    }
    const float inv = 1.0f / l;
    if (p.lse != nullptr && c == 0) p.lse[(int64_t)head * p.total + s0 + q] = (mx + __builtin_amdgcn_logf(l)) * kLn2;
    char *orow = p.out + ((int64_t)(s0 + q) * p.so_s + (int64_t)head * p.so_h) * 2;
    *(u32x2 *)(orow + 16 * c) = u32x2{E::pack(acc0[0] * inv, acc0[1] * inv), E::pack(acc0[2] * inv, acc0[3] * inv)};
    *(u32x2 *)(orow + 16 * c + 8) =
        u32x2{E::pack(acc1[0] * inv, acc1[1] * inv), E::pack(acc1[2] * inv, acc1[3] * inv)};
}

// Read schedule of the long kernel's matrix half: NOPS MFMA operands, the
// first NV of them two LDS reads each (transposed V), the rest one.  v[i] is
// the number of operands read by the time MFMA i issues: as many as keep at
// most kLimit reads in flight, the most the 4-bit LGKM counter tracks.
template <int NV, int NOPS> struct MatrixReads {
    static constexpr int kLimit = 15;
    int v[NOPS];
    static constexpr MatrixReads make() {
        MatrixReads f{};
        int nx = 0, fl = 0;
        for (int i = 0; i < NOPS; ++i) {
            while (nx < NOPS && fl + (nx < NV ? 2 : 1) <= kLimit) fl += nx++ < NV ? 2 : 1;
            f.v[i] = nx;
            fl -= i < NV ? 2 : 1;  // MFMA i waits for its operand
        }
        return f;
    }
};

template <int D, class E, int RD, bool FULL, bool PRE>
__global__ __launch_bounds__(kLongThreads, 1) void long_kernel(const KParams p) {
    using LDS = LongLds<D, RD, FULL, PRE>;
    constexpr int HALF = D / 2;
    constexpr int NQ = D / 8;                  // quads per half
    constexpr int DP = LDS::DP;
    constexpr int S = DP / 16;
    constexpr int KS = LDS::KS;
    constexpr int NDT = LDS::NDT;
    constexpr int RB = LDS::RB;
    constexpr int KCH = LDS::KCH, TCH = LDS::TCH;
    constexpr int KPC = LDS::KPC, TPC = LDS::TPC, VPC = LDS::VPC;
    constexpr int KRC = LDS::KRC;
    static_assert(KRC % 2 == 1 && KRC * 16 == LDS::KS * 2, "K_rot rows are whole, odd numbers of chunks");
    constexpr int NRAWI = PRE ? KRC : KPC + 2 * TPC;  // direct loads of one raw block (PRE: K_rot rows)
    constexpr int NDMA = NRAWI + VPC;          // ... plus the V block
    constexpr int MPER = (NDMA + kLongWaves - 1) / kLongWaves;
    constexpr int RPER = (NQ + kLongWaves - 1) / kLongWaves;  // rotation quads per wavefront
    constexpr bool ONES = LDS::kOnesCol;
    constexpr int RAWBUFS = LDS::kRawBufs;
    // raw K of block j + DIST is loaded in iteration j (PRE: K_rot of block
    // j + 2, into the K_rot buffer the rotation would otherwise fill then)
    constexpr int DIST = PRE ? 2 : RAWBUFS + 1;
    typedef short v4i16 __attribute__((ext_vector_type(4)));
    typedef __attribute__((address_space(3))) v4i16 lds_v4i16;
    typedef __attribute__((address_space(3))) void lds_void;
    typedef __attribute__((address_space(1))) void glb_void;
    __shared__ __attribute__((aligned(16))) char lds[LDS::kBytes];
    // LDS byte address of lds + off (the direct loads' destination register)
    auto lds_addr = [&](uint32_t off) { return (uint32_t)(uintptr_t)(lds_void *)(lds + off); };

    // Unit u = (segment, head, query block); workgroups past tail_first take
    // part `part` of the key range of a unit of the split last round.
    int u, part = 0, nparts = 1;
    if ((int)blockIdx.x < p.tail_first) {
        u = xcd_remap(blockIdx.x, p.tail_first);
    } else {
        const int t = xcd_remap(blockIdx.x - p.tail_first, gridDim.x - p.tail_first);
        nparts = p.tail_split;
        u = p.tail_first + t / nparts;
        part = t - (t / nparts) * nparts;
    }
    const int pi = u / p.qblocks, qblk = u - pi * p.qblocks;
    const int sh = long_pair(pi, p.num_seqs * p.num_heads);
    const int seg = sh / p.num_heads, head = sh - seg * p.num_heads;
    int s0 = p.cu[seg], s1 = p.cu[seg + 1];
    s0 = min(max(s0, 0), p.total);
    s1 = min(max(s1, 0), p.total);
    const int L = s1 - s0;
    if (L <= 0 || qblk * kLongBQ >= L) return;  // uniform across the workgroup

    const int tid = threadIdx.x;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    const int r = lane & 31, g = lane >> 5;
    // Key blocks [b0, b1) of the segment are this workgroup's (all of them
    // unless the unit is split); Lkv keys, possibly none.
    const int nblk_all = (L + kLongBKV - 1) / kLongBKV;
    const int b0 = part * nblk_all / nparts, b1 = (part + 1) * nblk_all / nparts;
    const int Lkv = min(L, kLongBKV * b1) - kLongBKV * b0;
    const int nblk = (Lkv + kLongBKV - 1) / kLongBKV;

    const int64_t k0 = (int64_t)s0 + (int64_t)kLongBKV * b0;  // first key row
    const char *kbase = PRE ? p.krot + (k0 * p.num_heads + head) * (int64_t)(D * 2)
                            : p.k + (k0 * p.sk_s + (int64_t)head * p.sk_h) * 2;
    const char *vbase = p.v + (k0 * p.sv_s + (int64_t)head * p.sv_h) * 2;
    const char *cbase = p.cos + k0 * p.sr_s * RB;
    const char *sbase = p.sin + k0 * p.sr_s * RB;
    const int64_t krs = PRE ? (int64_t)p.num_heads * D * 2 : p.sk_s * 2, vrs = p.sv_s * 2, trs = p.sr_s * RB;

    const float sl = p.scale_log2;
    float m_i = kNegInf, l_i = 0.f;  // running max (scale*log2e units) and row sum
    f32x16 oacc[NDT];
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) oacc[dt] = f32x16{};
    if (Lkv > 0) {  // uniform; a part of a split unit may have no keys

    // V padding columns [D, 32*NDT) of both buffers: zero, column D ones.
    // They are never overwritten by the staging loads.
    if constexpr (VPC > KCH) {
        constexpr int PADC = VPC - KCH;  // padding chunks of a V row
        const u32 one = E::pack(1.0f, 0.0f) & 0xffffu;
        for (int i = tid; i < 2 * 64 * PADC; i += kLongThreads) {
            const int bf = i / (64 * PADC), rem = i - bf * 64 * PADC;
            const int row = rem / PADC, pc = rem - row * PADC;
            u32x4 val = {0u, 0u, 0u, 0u};
            if (ONES && pc == 0) val[0] = one;  // element 0 of chunk D/8 is column D
            *(u32x4 *)(lds + LDS::kOffV + bf * LDS::kV + row * (VPC * 16) + (KCH + pc) * 16) = val;
        }
    }

    // ---- direct-load jobs ---------------------------------------------------------
    // A block is staged by NDMA direct loads, each moving 64 consecutive
    // 16-byte slots of one region: raw K (KPC loads), cos (TPC), sin (TPC)
    // -- the raw part -- then V (VPC).  Slot s of a region with pitch PC is
    // chunk s % PC of row s / PC; chunks past the row's data are padding and
    // not loaded.  Wavefront w owns loads w, w + kLongWaves, ... (job m is
    // load w + kLongWaves m).  Iteration j loads the raw part of block
    // j + DIST and the V part of block j + 1.
    constexpr int MFULL = NDMA / kLongWaves;  // jobs every wavefront has
    constexpr uint32_t kPadSlot = 0xffffffffu;
    struct Job {
        const char *base;  // the job's tensor at the first row of block 0
        uint32_t rows;     // row stride (bytes)
        uint32_t lds0;     // LDS destination in buffer 0
        uint32_t bufstep;  // bytes between LDS buffers
        int row;           // this lane's row
        uint32_t col;      // this lane's byte offset in the row, kPadSlot for padding
        bool raw;          // raw part (K, cos, sin) or V
    };
    // The bases and strides come in as parameters (values) on the generic
    // path: there, selecting between captured variables would select between
    // their addresses, which keeps them in scratch memory and puts every
    // job's base behind a flat load in every iteration.  (The steady-state
    // setup runs once; its descriptors stay as they are, which keeps the
    // steady loop's registers as they are.)
    auto job_desc_of = [&](int m, const char *kb_, const char *cb_, const char *sb_, const char *vb_, int64_t krs_,
                           int64_t trs_, int64_t vrs_) {
        const int gi = min(w + kLongWaves * m, NDMA - 1);
        Job jb;
        auto slot = [&](int ii, int pc, int dc) {  // pc, dc: compile-time in each branch
            const int s = 64 * ii + lane, row = s / pc, c = s - row * pc;
            jb.row = row;
            jb.col = c < dc ? (uint32_t)(16 * c) : kPadSlot;
        };
        // Base and row stride as selects of values (unary + makes each
        // operand a prvalue), outside the branches: a branch per source that
        // loads its own variable is merged into a load through a select of
        // their addresses, which keeps them in scratch memory.
        const bool is_k = PRE ? gi < NRAWI : gi < KPC;
        const bool is_t = !PRE && !is_k && gi < NRAWI;
        const bool is_c = gi < KPC + TPC;
        if constexpr (PRE) {
            // Two sources: the loaded values pass through empty asm first,
            // or the select is folded back into a load through a select of
            // the captured variables' addresses.
            uint64_t kv = (uint64_t)kb_, vv = (uint64_t)vb_;
            asm volatile("" : "+s"(kv), "+s"(vv));
            jb.base = (const char *)(is_k ? kv : vv);
            jb.rows = (uint32_t)(is_k ? +krs_ : +vrs_);
        } else {
            jb.base = is_k ? +kb_ : is_t ? (is_c ? +cb_ : +sb_) : +vb_;
            jb.rows = (uint32_t)(is_k ? +krs_ : is_t ? +trs_ : +vrs_);
        }
        if (PRE && gi < NRAWI) {
            jb.lds0 = (uint32_t)(LDS::kOffKrot + gi * 1024);
            slot(gi, KRC, KCH);
        } else if (!PRE && gi < KPC) {
            jb.lds0 = (uint32_t)(gi * 1024);
            slot(gi, KPC, KCH);
        } else if (!PRE && gi < NRAWI) {
            const int ii = is_c ? gi - KPC : gi - KPC - TPC;
            jb.lds0 = (uint32_t)(LDS::kRawK + (is_c ? 0 : LDS::kRawT) + ii * 1024);
            slot(ii, TPC, TCH);
        } else {
            const int ii = gi - NRAWI;
            jb.lds0 = (uint32_t)(LDS::kOffV + ii * 1024);
            slot(ii, VPC, KCH);
        }
        jb.raw = gi < NRAWI;
        jb.bufstep = jb.raw ? (PRE ? LDS::kKrot : LDS::kRaw) : LDS::kV;
        return jb;
    };
    auto job_desc = [&](int m) {
        const int gi = min(w + kLongWaves * m, NDMA - 1);
        Job jb;
        auto slot = [&](int ii, int pc, int dc) {  // pc, dc: compile-time in each branch
            const int s = 64 * ii + lane, row = s / pc, c = s - row * pc;
            jb.row = row;
            jb.col = c < dc ? (uint32_t)(16 * c) : kPadSlot;
        };
        if (PRE && gi < NRAWI) {
            jb.base = kbase;
            jb.rows = (uint32_t)krs;
            jb.lds0 = (uint32_t)(LDS::kOffKrot + gi * 1024);
            slot(gi, KRC, KCH);
        } else if (!PRE && gi < KPC) {
            jb.base = kbase;
            jb.rows = (uint32_t)krs;
            jb.lds0 = (uint32_t)(gi * 1024);
            slot(gi, KPC, KCH);
        } else if (!PRE && gi < NRAWI) {
            const bool is_cos = gi < KPC + TPC;
            const int ii = is_cos ? gi - KPC : gi - KPC - TPC;
            jb.base = is_cos ? cbase : sbase;
            jb.rows = (uint32_t)trs;
            jb.lds0 = (uint32_t)(LDS::kRawK + (is_cos ? 0 : LDS::kRawT) + ii * 1024);
            slot(ii, TPC, TCH);
        } else {
            const int ii = gi - NRAWI;
            jb.base = vbase;
            jb.rows = (uint32_t)vrs;
            jb.lds0 = (uint32_t)(LDS::kOffV + ii * 1024);
            slot(ii, VPC, KCH);
        }
        jb.raw = gi < NRAWI;
        jb.bufstep = jb.raw ? (PRE ? LDS::kKrot : LDS::kRaw) : LDS::kV;
        return jb;
    };
    // Does this wavefront have job m?
    auto has_job = [&](int m) { return m < MFULL || w + kLongWaves * m < NDMA; };
    // Job m for block x (raw part: block xr into buffer br; V: block xv into
    // buffer bv), the rows of a partial block clamped to its last row.
    // Generic path: prologue and last iterations.
    auto job_generic = [&](int m, int xr, int br, int xv, int bv) {
        if (!has_job(m)) return;
        const Job jb = job_desc_of(m, kbase, cbase, sbase, vbase, krs, trs, vrs);
        const int x = jb.raw ? xr : xv, bf = jb.raw ? br : bv;
        if (x >= nblk) return;
        const int nkv = min(kLongBKV, Lkv - kLongBKV * x);
        if (jb.col != kPadSlot) {
            const uint32_t voff = (uint32_t)min(jb.row, nkv - 1) * jb.rows + jb.col;
            const char *src = jb.base + (int64_t)x * kLongBKV * jb.rows;
            // (the compiler's own direct load: a generic iteration's
            // transposed reads may wait for it, the steady loops' may not)
            __builtin_amdgcn_global_load_lds((glb_void *)(src + voff), (lds_void *)(lds + jb.lds0 + bf * jb.bufstep),
                                             16, 0, 0);
        }
    };
    // The loads of iteration j (generic path).
    auto dma_iter = [&](int j) {
#pragma unroll
        for (int m = 0; m < MPER; ++m) job_generic(m, j + DIST, (j + DIST) % RAWBUFS, j + 1, (j + 1) & 1);
    };
    // Steady state: running pointers (block j + DIST or j + 1 in iteration j),
    // full blocks, the LDS destination fixed by the iteration parity P.
    const char *jptr[MPER];
    uint32_t jstep[MPER], jdst[MPER][2], jvoff[MPER];
    auto job_steady = [&](int m, int P) {
        if (jvoff[m] != kPadSlot)
            dma16(jptr[m] + jvoff[m], lds_addr(jdst[m][P]));
        jptr[m] += jstep[m];
    };

    // ---- rotation of one raw block into K_rot ---------------------------------------
    // Wavefront w rotates quads i = w, w + kLongWaves, ... of row `lane`
    // (rotate_quad: reference fused_attn.py:389-390), rounded to the storage
    // dtype.
    auto rotate_one = [&](int rawbuf, int kbuf, int i) {
        const char *raw = lds + rawbuf * LDS::kRaw + lane * (KPC * 16);
        const char *ct = lds + rawbuf * LDS::kRaw + LDS::kRawK + lane * (TPC * 16);
        const char *st = ct + LDS::kRawT;
        char *kr = lds + LDS::kOffKrot + kbuf * LDS::kKrot + lane * (KS * 2);
        const u32x2 x0 = *(const u32x2 *)(raw + 8 * i);
        const u32x2 x1 = *(const u32x2 *)(raw + D + 8 * i);
        const f32x4 c0 = Rope<RD>::quad(ct + RB * 4 * i);
        const f32x4 s0v = Rope<RD>::quad(st + RB * 4 * i);
        f32x4 c1 = c0, s1v = s0v;
        if constexpr (FULL) {
            c1 = Rope<RD>::quad(ct + RB * (HALF + 4 * i));
            s1v = Rope<RD>::quad(st + RB * (HALF + 4 * i));
        }
        u32x2 r0w, r1w;
        rotate_quad<E>(x0, x1, c0, s0v, c1, s1v, r0w, r1w);
        *(u32x2 *)(kr + 8 * i) = r0w;
        *(u32x2 *)(kr + D + 8 * i) = r1w;
    };
    auto rotate_rest = [&](int rawbuf, int kbuf) {
#pragma unroll
        for (int m = 1; m < RPER; ++m) {
            const int i = w + kLongWaves * m;
            if (i < NQ) rotate_one(rawbuf, kbuf, i);
        }
    };
    auto rotate = [&](int rawbuf, int kbuf) {
        if (kLongWaves <= NQ || w < NQ) rotate_one(rawbuf, kbuf, w);
        rotate_rest(rawbuf, kbuf);
    };

    auto wait_dma = [] { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); };

    // ---- prologue -----------------------------------------------------------------
    // raw K(0), V(0), and raw K(1) when there are two raw buffers
#pragma unroll
    for (int m = 0; m < MPER; ++m) {
        job_generic(m, 0, 0, 0, 0);
        if (RAWBUFS == 2) job_generic(m, 1, 1, nblk, 0);
    }

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
        for (int i = 0; i < NQ; ++i) {
            if constexpr (RD == kRopePos) load_rotate_quad_pos<D, E>(qrow, p, row, i, valid, nat[i], nat[NQ + i]);
            else load_rotate_quad<D, E, RD, FULL>(qrow, crow, srow, i, valid, nat[i], nat[NQ + i]);
        }
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
    // K_rot zero padding columns [D, KS) of both buffers.
    for (int i = tid; i < 2 * kLongBKV * (KS - D); i += kLongThreads) {
        const int bf = i / (kLongBKV * (KS - D)), rem = i - bf * kLongBKV * (KS - D);
        const int row = rem / (KS - D), col = D + rem % (KS - D);
        *(u16 *)(lds + LDS::kOffKrot + bf * LDS::kKrot + (row * KS + col) * 2) = 0;
    }
    wait_dma();
    __syncthreads();
    if constexpr (PRE) {
        // K_rot(0), K_rot(1) and V(0) are in place; K_rot(2) goes to buffer 0
        // in iteration 0, after the first S^T below has read K_rot(0).
    } else {
        rotate(0, 0);
        if constexpr (RAWBUFS == 2) {
            if (nblk > 1) rotate(1, 1);
            __syncthreads();
#pragma unroll
            for (int m = 0; m < MPER; ++m) job_generic(m, 2, 0, nblk, 0);  // raw K(2)
        } else {
            __syncthreads();
#pragma unroll
            for (int m = 0; m < MPER; ++m) job_generic(m, 1, 0, nblk, 0);  // raw K(1)
            wait_dma();
            __syncthreads();
            if (nblk > 1) rotate(0, 1);
            __syncthreads();
        }
    }

    // Per-lane LDS byte offsets.  K_rot A operand of S^T: row 32a + r, elements
    // 16t + 8g.  V transposed reads: the 16-lane group G = lane >> 4 covers
    // keys 4g + e (e = (lane >> 2) & 3) and columns 16 (G & 1) + 4 (lane & 3) of
    // each 32-column tile.
    const uint32_t k_lane = (uint32_t)(LDS::kOffKrot + (r * KS + 8 * g) * 2);
    const uint32_t v_lane = (uint32_t)(LDS::kOffV + (4 * g + ((lane >> 2) & 3)) * (VPC * 16) +
                                       2 * (16 * ((lane >> 4) & 1) + 4 * (lane & 3)));


    // S^T of block x (K_rot buffer x & 1).
    auto qk = [&](int x, f32x16 (&sacc)[2]) {
        const char *kb = lds + k_lane + (x & 1) * LDS::kKrot;
#pragma unroll
        for (int a = 0; a < 2; ++a) {
            sacc[a] = E::mma(*(const u32x4 *)(kb + a * (32 * KS * 2)), qop[0], f32x16{});
#pragma unroll
            for (int t = 1; t < S; ++t)
                sacc[a] = E::mma(*(const u32x4 *)(kb + a * (32 * KS * 2) + 32 * t), qop[t], sacc[a]);
        }
    };

    // Online softmax of one block's S^T, in two parts.  smax: masks keys
    // past the segment (nkv < 64), takes the row max and moves the running
    // max when needed (lazy rescaling: only when the row max grows by more
    // than the threshold; a uniform branch over the wavefront).
    auto smax = [&](f32x16 (&sacc)[2], int nkv) {
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
        // Row max as a tree of v_max3 (short dependency chains).
        float t[11];
#pragma unroll
        for (int k = 0; k < 10; ++k) {
            const int e = 3 * k;
            t[k] = max3f(sacc[e >> 4][e & 15], sacc[(e + 1) >> 4][(e + 1) & 15], sacc[(e + 2) >> 4][(e + 2) & 15]);
        }
        t[10] = fmaxf(sacc[1][14], sacc[1][15]);
        const float u0 = max3f(t[0], t[1], t[2]), u1 = max3f(t[3], t[4], t[5]);
        const float u2 = max3f(t[6], t[7], t[8]), u3 = fmaxf(t[9], t[10]);
        float mx = fmaxf(max3f(u0, u1, u2), u3);
        mx = max_pair32(mx) * sl;
        if (__builtin_amdgcn_ballot_w64(mx > m_i + kRescaleThreshold) != 0) {
            const float m_new = fmaxf(m_i, mx);
            const float alpha = __builtin_amdgcn_exp2f(m_i - m_new);
#pragma unroll
            for (int dt = 0; dt < NDT; ++dt) oacc[dt] *= alpha;
            l_i *= alpha;
            m_i = m_new;
        }
    };
    // sexp: P = exp2(S * scale * log2e - m), packed as the B operands of the
    // four PV steps.  Step (a, h) covers keys 32a + 16h + {4g..4g+3,
    // 8+4g..8+4g+3}: elements 8h..8h+7 of sacc[a].
    auto sexp = [&](f32x16 (&sacc)[2], u32x4 (&pop)[4]) {
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
        if constexpr (!ONES) l_i += sum_pair32(lsum);
#pragma unroll
        for (int a = 0; a < 2; ++a) {
#pragma unroll
            for (int h = 0; h < 2; ++h)
                pop[2 * a + h] = u32x4{E::pack(sacc[a][8 * h + 0], sacc[a][8 * h + 1]),
                                       E::pack(sacc[a][8 * h + 2], sacc[a][8 * h + 3]),
                                       E::pack(sacc[a][8 * h + 4], sacc[a][8 * h + 5]),
                                       E::pack(sacc[a][8 * h + 6], sacc[a][8 * h + 7])};
        }
    };

    // O^T += V^T P^T for block x (V buffer x & 1): two transposed reads of V
    // rows 32a + 16h + 4g + e and +8 per A operand.
    auto pv = [&](int x, const u32x4 (&pop)[4]) {
        const char *vb = lds + v_lane + (x & 1) * LDS::kV;
#pragma unroll
        for (int st = 0; st < 4; ++st) {
            const char *vrp = vb + 16 * st * (VPC * 16);  // keys 16 st
#pragma unroll
            for (int dt = 0; dt < NDT; ++dt) {
                const char *cp = vrp + 64 * dt;  // 32 columns
                const v4i16 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16 *)cp);
                const v4i16 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16 *)(cp + 8 * (VPC * 16)));
                const u32x2 l2 = __builtin_bit_cast(u32x2, lo), h2 = __builtin_bit_cast(u32x2, hi);
                oacc[dt] = E::mma(u32x4{l2[0], l2[1], h2[0], h2[1]}, pop[st], oacc[dt]);
            }
        }
    };

    // The matrix half of a ping-pong iteration: O^T += V(x)^T P^T (x = V
    // buffer parity) and S^T of the block in K_rot buffer x ^ 1, as one stream
    // of 4 NDT + 2 S MFMAs whose LDS operands are read as far ahead as the
    // LGKM counter allows (MatrixReads), so that the read latency hides
    // behind the matrix core instead of stalling each MFMA on its operand.
    auto matrix_half = [&](int x, const u32x4 (&pop)[4], f32x16 (&nxt)[2]) {
        constexpr int NV = 4 * NDT, NOPS = NV + 2 * S;
        constexpr MatrixReads<NV, NOPS> plan = MatrixReads<NV, NOPS>::make();
        const char *vb = lds + v_lane + x * LDS::kV;
        const char *kb = lds + k_lane + (x ^ 1) * LDS::kKrot;
        u32x4 op[NOPS];
        auto rd = [&](int i) {
            if (i < NV) {
                const char *cp = vb + 16 * (i / NDT) * (VPC * 16) + 64 * (i % NDT);
                const v4i16 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16 *)cp);
                const v4i16 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16 *)(cp + 8 * (VPC * 16)));
                const u32x2 l2 = __builtin_bit_cast(u32x2, lo), h2 = __builtin_bit_cast(u32x2, hi);
                op[i] = u32x4{l2[0], l2[1], h2[0], h2[1]};
            } else {
                const int k = i - NV;
                op[i] = *(const u32x4 *)(kb + (k & 1) * (32 * KS * 2) + 32 * (k >> 1));
            }
        };
#pragma unroll
        for (int i = 0; i < NOPS; ++i) {
#pragma unroll
            for (int k = i == 0 ? 0 : plan.v[i - 1]; k < plan.v[i]; ++k) rd(k);
            if (i < NV) {
                oacc[i % NDT] = E::mma(op[i], pop[i / NDT], oacc[i % NDT]);
            } else {
                const int k = i - NV, ac = k & 1, tt = k >> 1;
                nxt[ac] = E::mma(op[i], qop[tt], tt == 0 ? f32x16{} : nxt[ac]);
            }
            __builtin_amdgcn_sched_barrier(0);
        }
    };

    f32x16 sA[2], sB[2];
    qk(0, sA);
    wait_dma();
    __syncthreads();

    // One iteration j: loads for later blocks, phase A, phase B, barrier.
    // `cur` holds S(j); `nxt` receives S(j+1).  The steady-state variant
    // (P = parity of j) may assume blocks j..j+DIST exist and are full, and
    // keeps phases A and B in one basic block so that the compiler can overlap
    // the MFMAs with the softmax and rotation work; the generic variant checks.
    // Phase A of iteration j: S(j+1) on the matrix core, one MFMA then about
    // three exponentials of S(j) per step, so that the matrix core and the
    // vector unit of this wave both stay busy (the two accumulator chains
    // alternate, and the K_rot operand of a step is read two steps ahead);
    // then P(j) packed as the B operands of the four PV steps.
    auto phase_a = [&](int j, f32x16 (&cur)[2], f32x16 (&nxt)[2], u32x4 (&pop)[4]) {
        {
            constexpr int NA = 2 * S;
            const char *kb = lds + k_lane + ((j + 1) & 1) * LDS::kKrot;
            auto kaddr = [&](int i) { return kb + (i & 1) * (32 * KS * 2) + 32 * (i >> 1); };
            u32x4 kr[3];
            kr[0] = *(const u32x4 *)kaddr(0);
            kr[1] = *(const u32x4 *)kaddr(1);
            float lsum = 0.f;
#pragma unroll
            for (int i = 0; i < NA; ++i) {
                if (i + 2 < NA) kr[(i + 2) % 3] = *(const u32x4 *)kaddr(i + 2);
                const int ac = i & 1, tt = i >> 1;
                nxt[ac] = E::mma(kr[i % 3], qop[tt], tt == 0 ? f32x16{} : nxt[ac]);
#pragma unroll
                for (int e = 32 * i / NA; e < 32 * (i + 1) / NA; ++e) {
                    const float x = __builtin_amdgcn_exp2f(__builtin_fmaf(cur[e >> 4][e & 15], sl, -m_i));
                    cur[e >> 4][e & 15] = x;
                    if constexpr (!ONES) lsum += x;
                }
                __builtin_amdgcn_sched_barrier(0);
            }
            if constexpr (!ONES) l_i += sum_pair32(lsum);
        }
#pragma unroll
        for (int a = 0; a < 2; ++a) {
#pragma unroll
            for (int h = 0; h < 2; ++h)
                pop[2 * a + h] = u32x4{E::pack(cur[a][8 * h + 0], cur[a][8 * h + 1]),
                                       E::pack(cur[a][8 * h + 2], cur[a][8 * h + 3]),
                                       E::pack(cur[a][8 * h + 4], cur[a][8 * h + 5]),
                                       E::pack(cur[a][8 * h + 6], cur[a][8 * h + 7])};
        }
        // P(j) is complete here.  Without the pin the compiler sinks the
        // exponentials and packs to their use, past the ping-pong barrier
        // into phase B, in front of the PV MFMAs that wait for them.
#pragma unroll
        for (int i = 0; i < 4; ++i) asm volatile("" : "+v"(pop[i]));
    };
    auto iteration_steady = [&](auto par_tag, int j, f32x16 (&cur)[2], f32x16 (&nxt)[2]) {
        constexpr int P = decltype(par_tag)::value;
        smax(cur, kLongBKV);
        constexpr int RB2 = RAWBUFS == 2 ? P : 0;  // raw buffer of block j + 2
#pragma unroll
        for (int m = 0; m < MFULL; ++m) job_steady(m, P);
        if constexpr (RAWBUFS == 1 && MPER > MFULL) {
            // one raw buffer: every load of the iteration precedes the mid barrier
            if (has_job(MFULL)) job_steady(MFULL, P);
        }
        __builtin_amdgcn_sched_barrier(0);
        u32x4 pop[4];
        phase_a(j, cur, nxt, pop);
        if constexpr (RAWBUFS == 1) {
            wait_dma();
            __syncthreads();
        }
        pv(j, pop);
        if constexpr (!PRE) {
            if (kLongWaves <= NQ || w < NQ) rotate_one(RB2, P, w);
        }
        if constexpr (RAWBUFS == 2 && MPER > MFULL) {
            if (has_job(MFULL)) job_steady(MFULL, P);
        }
        if constexpr (!PRE) rotate_rest(RB2, P);
        wait_dma();
        __syncthreads();
    };
    auto iteration_generic = [&](int j, f32x16 (&cur)[2], f32x16 (&nxt)[2]) {
        dma_iter(j);
        u32x4 pop[4];
        smax(cur, min(kLongBKV, Lkv - kLongBKV * j));
        if (j + 1 < nblk) qk(j + 1, nxt);
        sexp(cur, pop);
        if constexpr (RAWBUFS == 1) {
            wait_dma();
            __syncthreads();
        }
        pv(j, pop);
        if constexpr (!PRE) {
            if (j + 2 < nblk) rotate((j + 2) % RAWBUFS, j & 1);
        }
        wait_dma();
        __syncthreads();
    };
    typedef std::integral_constant<int, 0> Even;
    typedef std::integral_constant<int, 1> Odd;

    // Steady iterations j need blocks up to j + DIST to exist and be full:
    // j + DIST < nblk - 1, i.e. j < nblk - DIST - 1; taken in pairs.
    int j = 0;
    const int nsteady = nblk - DIST - 1;
    if (nsteady >= 2) {
        bool kjob[MPER];  // job m is a K_rot (raw) job, else a V job
        int nk = 0, nv = 0;
#pragma unroll
        for (int m = 0; m < MPER; ++m) {
            Job jb;
            if constexpr (PRE) jb = job_desc_of(m, kbase, cbase, sbase, vbase, krs, trs, vrs);
            else jb = job_desc(m);
            jstep[m] = kLongBKV * jb.rows;
            jptr[m] = jb.base + (int64_t)(jb.raw ? DIST : 1) * jstep[m];
            jvoff[m] = jb.col == kPadSlot ? kPadSlot : (uint32_t)jb.row * jb.rows + jb.col;
#pragma unroll
            for (int P = 0; P < 2; ++P)
                jdst[m][P] = jb.lds0 + (jb.raw ? (uint32_t)((P + DIST) % RAWBUFS) : (uint32_t)((P + 1) & 1)) * jb.bufstep;
            kjob[m] = jb.raw;
            if (has_job(m)) {
                nk += jb.raw ? 1 : 0;
                nv += jb.raw ? 0 : 1;
            }
        }
        if constexpr (PRE) {
            // Ping-pong: wavefronts 0-3 and 4-7 (one of each per SIMD) run
            // half an iteration apart, with a barrier per half-iteration.  A
            // wavefront's iteration j is a vector half, the softmax of S(j)
            // (row max, lazy rescale, exponentials, P(j) packed), and a matrix
            // half, O += V(j)^T P(j)^T and S(j+1) = K_rot(j+1) Q_rot^T: 22
            // MFMAs with only their LDS operand reads beside them.  While one
            // wavefront of a SIMD feeds the matrix core, the other runs its
            // exponentials on the vector unit; no wavefront's in-order issue
            // holds vector work behind an MFMA that waits for the matrix core.
            // Group 0 runs the vector half of j in half-iteration 2j and the
            // matrix half in 2j + 1; group 1 one half later.  Every wavefront
            // issues its K_rot(j+2) jobs at the start of half-iteration 2j + 1
            // (the buffer last held K_rot(j), whose last reader, group 1's
            // matrix half of j - 1, ran in 2j) and its V(j+1) jobs at the start
            // of 2j + 2 (V(j-1)'s buffer, last read in 2j); the first reader of
            // both (group 0's matrix half of j + 1) runs in 2j + 3.  A half
            // ends with a barrier after the V jobs issued at its start have
            // landed (the K_rot jobs may stay in flight for one more half).
            // The two kinds go in different halves because a burst of direct
            // loads stalls the issuing wavefronts on the CU's memory path.
            static_assert(kLongWaves == 8, "two groups of one wavefront per SIMD");
            const int grp = w >> 2;
            // s_waitcnt takes an immediate; more outstanding jobs than the
            // largest case only wait longer.
            auto half_barrier = [](int keep) {
                if (keep <= 0) asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
                else if (keep == 1) asm volatile("s_waitcnt vmcnt(1) lgkmcnt(0)\n\ts_barrier" ::: "memory");
                else if (keep == 2) asm volatile("s_waitcnt vmcnt(2) lgkmcnt(0)\n\ts_barrier" ::: "memory");
                else asm volatile("s_waitcnt vmcnt(3) lgkmcnt(0)\n\ts_barrier" ::: "memory");
            };
            // Job m of this wavefront for iteration parity P (K_rot(j+2) or
            // V(j+1)).
            auto issue_job = [&](int m, int par) {
                if (has_job(m)) {
                    if (jvoff[m] != kPadSlot) dma16(jptr[m] + jvoff[m], lds_addr(par ? +jdst[m][1] : +jdst[m][0]));
                    jptr[m] += jstep[m];
                }
            };
            auto issue = [&](bool kind, int par) {  // this wavefront's jobs of one kind
#pragma unroll
                for (int m = 0; m < MPER; ++m)
                    if (kjob[m] == kind) issue_job(m, par);
            };
            // Softmax of S(j) into the PV operands, the exponentials in eight
            // groups of four.
            auto vector_half = [&](f32x16 (&cur)[2], u32x4 (&pop)[4]) {
                smax(cur, kLongBKV);
                float lsum = 0.f;
#pragma unroll
                for (int g8 = 0; g8 < 8; ++g8) {
#pragma unroll
                    for (int e = 4 * g8; e < 4 * g8 + 4; ++e) {
                        const float x = __builtin_amdgcn_exp2f(__builtin_fmaf(cur[e >> 4][e & 15], sl, -m_i));
                        cur[e >> 4][e & 15] = x;
                        if constexpr (!ONES) lsum += x;
                    }
                    __builtin_amdgcn_sched_barrier(0);
                }
                if constexpr (!ONES) l_i += sum_pair32(lsum);
#pragma unroll
                for (int a = 0; a < 2; ++a) {
#pragma unroll
                    for (int h = 0; h < 2; ++h)
                        pop[2 * a + h] = u32x4{E::pack(cur[a][8 * h + 0], cur[a][8 * h + 1]),
                                               E::pack(cur[a][8 * h + 2], cur[a][8 * h + 3]),
                                               E::pack(cur[a][8 * h + 4], cur[a][8 * h + 5]),
                                               E::pack(cur[a][8 * h + 6], cur[a][8 * h + 7])};
                }
                // P(j) is complete here.  Without the pin the compiler sinks
                // the exponentials and packs to their use, past the barrier
                // into the matrix half.
#pragma unroll
                for (int i = 0; i < 4; ++i) asm volatile("" : "+v"(pop[i]));
            };
            auto iteration_pp = [&](auto par_tag, f32x16 (&cur)[2], f32x16 (&nxt)[2], bool kmore) {
                constexpr int P = decltype(par_tag)::value;  // parity of j
                u32x4 pop[4];
                if (grp == 0) {
                    vector_half(cur, pop);
                    half_barrier(0);
                }
                if (kmore) issue(true, P);  // K_rot(j+2), where that block exists
                if (grp != 0) {
                    vector_half(cur, pop);
                    half_barrier(nk);
                    issue(false, P);  // V(j+1)
                }
                matrix_half(P, pop, nxt);
                half_barrier(grp == 0 ? nk : 0);
                if (grp == 0) issue(false, P);  // V(j+1), at the start of the next half
            };
            // With a full last block the loop runs through j = nblk - 2 (its
            // last K_rot loads are skipped: those blocks do not exist), and
            // only the last block takes the generic path.  (A partial last
            // block is loaded by the generic path, which clamps its rows.)
            const int npp = Lkv % kLongBKV == 0 ? nblk - 1 : nsteady;
            if (grp == 1) half_barrier(0);  // group 0's vector half of S(0)
            for (; j + 1 < npp; j += 2) {
                iteration_pp(Even{}, sA, sB, j + 2 < nblk);
                iteration_pp(Odd{}, sB, sA, j + 3 < nblk);
            }
            if (j < npp) {  // an odd count: one more, j even
                iteration_pp(Even{}, sA, sB, j + 2 < nblk);
                ++j;
            }
            if (grp == 0) half_barrier(0);  // group 1 finishes the matrix half of the last steady iteration
        } else {
            for (; j + 1 < nsteady; j += 2) {
                iteration_steady(Even{}, j, sA, sB);
                iteration_steady(Odd{}, j + 1, sB, sA);
            }
        }
    }
    // S(j) is in sA for even j, in sB for odd j.
    if ((j & 1) && j < nblk) {
        iteration_generic(j, sB, sA);
        ++j;
    }
    for (; j < nblk; j += 2) {
        iteration_generic(j, sA, sB);
        if (j + 1 < nblk) iteration_generic(j + 1, sB, sA);
    }

    }  // Lkv > 0

    if constexpr (ONES) {
        // O^T row D (the ones column of V) is in element 4*((D % 32) / 8) of
        // the last d tile, held by the g = 0 lanes.
        constexpr int jl = 4 * ((D - 32 * (NDT - 1)) / 8);
        const float lv = oacc[NDT - 1][jl];
        l_i = bcast_lo32(lv);
    }
    const int q = qblk * kLongBQ + 32 * w + r;
    if (nparts > 1) {
        split_write_partial<D>(p, u, part, nparts, q, L, w, r, g, m_i, l_i, oacc);
        return;
    }
    if (q < L) {
        const float inv = 1.0f / l_i;
        if (p.lse != nullptr && g == 0)
            p.lse[(int64_t)head * p.total + s0 + q] = (m_i + __builtin_amdgcn_logf(l_i)) * kLn2;
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

}  // namespace

namespace fra_internal {

// The long kernel stages table rows as whole 16-byte chunks; 16-bit tables
// whose rows are not (head_dim 72 at width head_dim/2) have no long kernel.
template <int D, int RD, bool FULL> constexpr bool long_ok() {
    return (FULL ? D : D / 2) * Rope<RD>::kBytes % 16 == 0;
}

template <int D, class E, int RD, bool FULL> void pick_full(bool window, int hw, Choice &c) {
    c.fn = nullptr;
    if constexpr (D <= kWindowMaxD) {
        if (window) {
            if (hw == 1) {
                // query split: the slab's 16-byte items must divide evenly over
                // two wavefronts (D = 72 has nine chunks a row: no instance)
                if constexpr (64 * (D / 8) % 128 == 0) {
                    c.fn = (KernelFn)window_kernel<D, E, RD, FULL, 1, false>;
                    c.fn_gather = (KernelFn)window_kernel<D, E, RD, FULL, 1, true>;
                    c.lds = WinLds<D, FULL, 1>::kBytes;
                    c.per_cu = WinLds<D, FULL, 1>::kPerCu;
                }
            } else if (hw == 2) {
                c.fn = (KernelFn)window_kernel<D, E, RD, FULL, 2, false>;
                c.fn_gather = (KernelFn)window_kernel<D, E, RD, FULL, 2, true>;
                c.lds = WinLds<D, FULL, 2>::kBytes;
                c.per_cu = WinLds<D, FULL, 2>::kPerCu;
            } else {
                c.fn = (KernelFn)window_kernel<D, E, RD, FULL, 4, false>;
                c.fn_gather = (KernelFn)window_kernel<D, E, RD, FULL, 4, true>;
                c.lds = WinLds<D, FULL, 4>::kBytes;
                c.per_cu = WinLds<D, FULL, 4>::kPerCu;
            }
            c.heads = hw;
            return;
        }
    }
    if constexpr (long_ok<D, RD, FULL>()) {
        // (the position variant has no table rows to stage: rotated-K form only)
        if constexpr (RD != kRopePos) c.fn = (KernelFn)long_kernel<D, E, RD, FULL, false>;
        c.merge = (KernelFn)split_merge_kernel<D, E>;
        c.lds = LongLds<D, RD, FULL>::kBytes;
        c.fn_pre = (KernelFn)long_kernel<D, E, RD, FULL, true>;
        c.krot = (KernelFn)krot_kernel<D, E, RD, FULL>;
        c.lds_pre = LongLds<D, RD, FULL, true>::kBytes;
    }
}

template <int D, class E, int RD> void pick_rd(bool window, int hw, bool full, Choice &c) {
    if (full) pick_full<D, E, RD, true>(window, hw, c);
    else pick_full<D, E, RD, false>(window, hw, c);
}

// The position variant: window kernels, and for long segments only the
// rotated-K (workspace) form, whose K rotation computes the angles.
template <int D, class E> void pick_pos(bool window, int hw, Choice &c) {
    if constexpr (D % 4 == 0) {
        pick_full<D, E, kRopePos, false>(window, hw, c);
    }
}

template <int D> void pick_d(bool window, int hw, bool full, int qkv, int rd, Choice &c) {
    if (rd == kRopePos) {
        if (qkv == FRA_DTYPE_BF16) pick_pos<D, BF16>(window, hw, c);
        else pick_pos<D, F16>(window, hw, c);
        return;
    }
    if (qkv == FRA_DTYPE_BF16) {
        if (rd == FRA_DTYPE_F32) pick_rd<D, BF16, FRA_DTYPE_F32>(window, hw, full, c);
        else if (rd == FRA_DTYPE_BF16) pick_rd<D, BF16, FRA_DTYPE_BF16>(window, hw, full, c);
        else pick_rd<D, BF16, FRA_DTYPE_F16>(window, hw, full, c);
    } else {
        if (rd == FRA_DTYPE_F32) pick_rd<D, F16, FRA_DTYPE_F32>(window, hw, full, c);
        else if (rd == FRA_DTYPE_BF16) pick_rd<D, F16, FRA_DTYPE_BF16>(window, hw, full, c);
        else pick_rd<D, F16, FRA_DTYPE_F16>(window, hw, full, c);
    }
}

}  // namespace fra_internal
