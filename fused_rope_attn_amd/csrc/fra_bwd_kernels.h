// fra_bwd_kernels.h -- gfx950 backward kernels of the fused RoPE + varlen attention op.
// Included by fra_inst_bwd.hip, which instantiates them for one head_dim.
//
// The reference is forward-only (fused_attn.py:139-423 has no autograd and
// no softmax statistics output).  This file adds the training side of the
// same op, as the gradient of the forward's arithmetic (reference
// fused_attn.py:316-423): with q_rot = rot(q), k_rot = rot(k) (fp32 rotation
// rounded to the storage dtype), z = scale * q_rot k_rot^T per segment,
// P = softmax(z), out = P v:
//
//   Dvec = rowsum(dout * out)                      (bwd_dot_kernel)
//   dz   = P * (dout v^T - Dvec)
//   dq   = rot^T(scale * dz k_rot)                 (bwd_dq_kernel)
//   dk   = rot^T(scale * dz^T q_rot),  dv = P^T dout   (bwd_dkdv_kernel)
//
// where rot^T is the transpose of the per-pair rotation (the rounding of
// q_rot / k_rot is taken as the identity, as autograd does for a cast).  P is
// recomputed from the forward's log-sum-exp: P = exp2(z log2(e) - lse log2(e)).
//
// Segments of at most 64 tokens take one kernel, bwd_window_kernel, that does
// all of it per (segment, head) in one pass (below).  Longer segments take
// three: bwd_dot_kernel, then two matrix kernels with the operand layouts of
// the forward (fra_kernels.hip), v_mfma_f32_32x32x16_{bf16,f16}:
//   bwd_dq_kernel    one workgroup per block of 32*NW queries; lane (r, g) of
//                    wave w holds query 32w + r as the column of S^T, dP^T and
//                    dQ^T (the forward's layout), looping over 64-key blocks of
//                    K_rot and V staged in LDS.  dQ^T = K_rot^T dZ^T takes its
//                    A operand from K_rot by ds_read_b64_tr_b16.
//   bwd_dkdv_kernel  one workgroup per block of 32*NW keys; lane (r, g) holds
//                    key 32w + r as the column of S = Q_rot K_rot^T and
//                    dP = dout V^T, looping over 64-query blocks of Q_rot and
//                    dout staged in LDS; dV^T = dout^T P and dK^T = Q_rot^T dZ
//                    take their A operands from dout and Q_rot by transposed
//                    reads.
// dq and dk leave through LDS as fp32 rows, where the inverse rotation pairs
// d with d + head_dim/2.  No atomics: every output row has one writer.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "fra.h"
#include "fra_device.h"
#include "fra_bwd_types.h"

namespace {

using namespace fra_internal;


typedef short v4i16 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) v4i16 lds_v4i16;

__host__ __device__ constexpr int cmax(int a, int b) { return a > b ? a : b; }
__host__ __device__ constexpr int cmin(int a, int b) { return a < b ? a : b; }
__host__ __device__ constexpr int bwd_dp(int d) { return (d + 15) / 16 * 16; }

// LDS row pitch (bytes) of a region read both as rows (16-byte MFMA operand
// reads) and transposed (ds_read_b64_tr_b16 over 32-column tiles, so up to
// 4 * ceil(d / 32) chunks of 16 bytes per row): an odd chunk count.  Rows
// read as 16-byte operands are then conflict-free and the transposed reads
// at most 2-way; a pitch of 4 or 12 mod 16 chunks makes the transposed reads
// conflict-free but puts rows r and r + 4 on the same banks, a 4-way
// conflict on every row read (measured 2.7e8 conflict cycles per backward
// call at 9216 tokens x 16 heads, about a quarter of the kernel's time).
__host__ __device__ constexpr int bwd_pitch_tr(int d) {
    int c = cmax(bwd_dp(d) / 8, 4 * ((d + 31) / 32));
    if (c % 2 == 0) ++c;
    return 16 * c;
}
// ... and of a region read only as rows: an odd chunk count.
__host__ __device__ constexpr int bwd_pitch_rows(int d) { return 16 * (bwd_dp(d) / 8 + 1); }
// fp32 rows of the final transposes (dq, dk before the inverse rotation).
__host__ __device__ constexpr int bwd_pitch_f32(int d) { return 4 * (d + 4); }

// Wavefronts per SIMD the register budget of a backward kernel is sized for
// (two: up to 256 VGPR + AGPR per lane; one at head_dim 128, whose dk/dv
// accumulators alone take 128).
template <int D> struct BwdOcc {
    static constexpr int kWaves = D >= 128 ? 1 : 2;
};

// sched_barrier mask: VALU, SALU and transcendental instructions may be
// scheduled across it; LDS accesses and MFMAs keep their written order.
constexpr int kSchedValuMayCross = 0x0002 | 0x0004 | 0x0400;

constexpr int kBwdBlockQ = 64;   // queries per LDS stage of the dk/dv kernel
constexpr int kBwdBlockKV = 64;  // keys per LDS stage of the dq kernel

// A block of NROWS rows staged through registers: every global load of the
// block is issued first (the item loops have compile-time trip counts and
// unroll), then the values are rotated and written to LDS, so a block costs
// one HBM round trip rather than one per item.
//
// RotBlock: the split-half rotation (fp32, rounded to the storage dtype, as
// the forward computes it) of NX tensors that share token rows (and so their
// cos/sin rows: q and k of one segment), into LDS rows [x0r | x1r | 0-pad to a
// multiple of 16].  Item (row, i) is quad i (entries 4i..4i+3) of both halves.
// Rows >= nvalid are zero.  x[n] points at token tok0's row of the head; xs[n]
// is its row stride in bytes.
template <int D, class E, bool FULL, int NROWS, int NT, int NX>
struct RotBlock {
    static constexpr int NQ = D / 8, HALF = D / 2;
    static constexpr int N = NROWS * NQ, K = (N + NT - 1) / NT;
    static constexpr int PADQ = (bwd_dp(D) - D) / 4;  // zero quads after each row
    u32x2 x0[NX][K], x1[NX][K];
    f32x4 c0[K], s0[K], c1[K], s1[K];

    __device__ __forceinline__ void load(const BParams &p, const char *const (&x)[NX], const int64_t (&xs)[NX],
                                         int tok0, int nvalid, int tid) {
#pragma unroll
        for (int k = 0; k < K; ++k) {
            const int it = tid + k * NT;
            if (N % NT == 0 || it < N) {
                const int row = it / NQ, i = it - row * NQ;
                const int rr = row < nvalid ? row : 0;
                const int64_t tok = (int64_t)tok0 + rr;
#pragma unroll
                for (int n = 0; n < NX; ++n) {
                    const char *xrow = x[n] + rr * xs[n];
                    x0[n][k] = *(const u32x2 *)(xrow + 8 * i);
                    x1[n][k] = *(const u32x2 *)(xrow + 2 * HALF + 8 * i);
                }
                const char *crow = p.cos + tok * p.sr_s * 4, *srow = p.sin + tok * p.sr_s * 4;
                c0[k] = *(const f32x4 *)(crow + 16 * i);
                s0[k] = *(const f32x4 *)(srow + 16 * i);
                if constexpr (FULL) {
                    c1[k] = *(const f32x4 *)(crow + 4 * (HALF + 4 * i));
                    s1[k] = *(const f32x4 *)(srow + 4 * (HALF + 4 * i));
                }
            }
        }
    }

    __device__ __forceinline__ void store(char *const (&dst)[NX], int pitch, int nvalid, int tid) const {
#pragma unroll
        for (int k = 0; k < K; ++k) {
            const int it = tid + k * NT;
            if (N % NT == 0 || it < N) {
                const int row = it / NQ, i = it - row * NQ;
                const bool valid = row < nvalid;
#pragma unroll
                for (int n = 0; n < NX; ++n) {
                    u32x2 r0, r1;
                    rotate_quad<E>(valid ? x0[n][k] : u32x2{0u, 0u}, valid ? x1[n][k] : u32x2{0u, 0u}, c0[k], s0[k],
                                   FULL ? c1[k] : c0[k], FULL ? s1[k] : s0[k], r0, r1);
                    char *drow = dst[n] + row * pitch;
                    *(u32x2 *)(drow + 8 * i) = r0;
                    *(u32x2 *)(drow + 2 * HALF + 8 * i) = r1;
                }
            }
        }
        if constexpr (PADQ > 0) {
            for (int it = tid; it < NROWS * PADQ; it += NT) {
                const int row = it / PADQ, i = it - row * PADQ;
#pragma unroll
                for (int n = 0; n < NX; ++n) *(u32x2 *)(dst[n] + row * pitch + 2 * D + 8 * i) = u32x2{0u, 0u};
            }
        }
    }
};

// RowBlock: rows of x copied as 16-byte chunks, zero past nvalid rows and
// past head_dim up to a multiple of 16.
template <int D, int NROWS, int NT>
struct RowBlock {
    static constexpr int CH = D / 8, N = NROWS * CH, K = (N + NT - 1) / NT;
    static constexpr int PADC = bwd_dp(D) / 8 - CH;  // zero chunks after each row
    u32x4 v[K];

    __device__ __forceinline__ void load(const char *x, int64_t xs, int nvalid, int tid) {
#pragma unroll
        for (int k = 0; k < K; ++k) {
            const int it = tid + k * NT;
            v[k] = u32x4{0u, 0u, 0u, 0u};
            if (N % NT == 0 || it < N) {
                const int row = it / CH, c = it - row * CH;
                if (row < nvalid) v[k] = *(const u32x4 *)(x + row * xs + 16 * c);
            }
        }
    }

    __device__ __forceinline__ void store(char *dst, int pitch, int tid) const {
#pragma unroll
        for (int k = 0; k < K; ++k) {
            const int it = tid + k * NT;
            if (N % NT == 0 || it < N) {
                const int row = it / CH, c = it - row * CH;
                *(u32x4 *)(dst + row * pitch + 16 * c) = v[k];
            }
        }
        if constexpr (PADC > 0) {
            for (int it = tid; it < NROWS * PADC; it += NT) {
                const int row = it / PADC, c = CH + (it - row * PADC);
                *(u32x4 *)(dst + row * pitch + 16 * c) = u32x4{0u, 0u, 0u, 0u};
            }
        }
    }
};

// fp32 gradient rows of x_rot (LDS, `fpf` floats per row) -> gradient of x:
// the transpose of the forward's rotation, x0r = x0 c0 - x1 s0,
// x1r = x0 s1 + x1 c1 (c1 = c0, s1 = s0 for half-width tables), so
// g0 = g0r c0 + g1r s1 and g1 = g1r c1 - g0r s0; rounded to the storage
// dtype and stored to rows [0, nvalid) of dst (row stride ds bytes).
template <int D, class E, bool FULL>
__device__ __forceinline__ void unrotate_store(const float *f, int fpf, const BParams &p, char *dst, int64_t ds,
                                               int tok0, int nvalid, int tid, int nthr) {
    constexpr int NQ = D / 8, HALF = D / 2;
    for (int it = tid; it < nvalid * NQ; it += nthr) {
        const int row = it / NQ, i = it - row * NQ;
        const f32x4 g0 = *(const f32x4 *)(f + row * fpf + 4 * i);
        const f32x4 g1 = *(const f32x4 *)(f + row * fpf + HALF + 4 * i);
        const int64_t tok = (int64_t)tok0 + row;
        const char *crow = p.cos + tok * p.sr_s * 4, *srow = p.sin + tok * p.sr_s * 4;
        const f32x4 c0 = *(const f32x4 *)(crow + 16 * i), s0 = *(const f32x4 *)(srow + 16 * i);
        f32x4 c1 = c0, s1 = s0;
        if constexpr (FULL) {
            c1 = *(const f32x4 *)(crow + 4 * (HALF + 4 * i));
            s1 = *(const f32x4 *)(srow + 4 * (HALF + 4 * i));
        }
        float x0[4], x1[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            x0[e] = __builtin_fmaf(g0[e], c0[e], g1[e] * s1[e]);
            x1[e] = __builtin_fmaf(g1[e], c1[e], -(g0[e] * s0[e]));
        }
        char *drow = dst + row * ds;
        *(u32x2 *)(drow + 8 * i) = u32x2{E::pack(x0[0], x0[1]), E::pack(x0[2], x0[3])};
        *(u32x2 *)(drow + 2 * HALF + 8 * i) = u32x2{E::pack(x1[0], x1[1]), E::pack(x1[2], x1[3])};
    }
}

// Segment bounds of `seg`, clamped to [0, total] as in the forward.
__device__ __forceinline__ void seg_bounds(const BParams &p, int seg, int &s0, int &L) {
    int a = p.cu[seg], b = p.cu[seg + 1];
    a = min(max(a, 0), p.total);
    b = min(max(b, 0), p.total);
    s0 = a;
    L = b - a;
}

// Dvec[h, t] = sum_d dout[t, h, d] * out[t, h, d] in fp32, one thread per
// (token, head) row.
template <int D, class E>
__global__ __launch_bounds__(256) void bwd_dot_kernel(const BParams p) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= (int64_t)p.total * p.num_heads) return;
    const int t = (int)(i / p.num_heads), h = (int)(i - (int64_t)t * p.num_heads);
    const char *o = p.out + ((int64_t)t * p.so_s + (int64_t)h * p.so_h) * 2;
    const char *go = p.dout + ((int64_t)t * p.sdo_s + (int64_t)h * p.sdo_h) * 2;
    float acc = 0.f;
#pragma unroll
    for (int c = 0; c < D / 8; ++c) {
        const u32x4 a = *(const u32x4 *)(o + 16 * c), b = *(const u32x4 *)(go + 16 * c);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            acc = __builtin_fmaf(E::lo(a[e]), E::lo(b[e]), acc);
            acc = __builtin_fmaf(E::hi(a[e]), E::hi(b[e]), acc);
        }
    }
    p.dvec[(int64_t)h * p.total + t] = acc;
}

// q_rot and k_rot into the workspace ([total, heads, head_dim], dense), once
// per call: the dq and dk/dv units then stage plain rows instead of rotating
// every block they load (each K block is loaded by every query block of its
// segment and head, and each Q block by every key block).  One thread per
// (token, head, quad i): quads i of both halves, the forward's rotation.
template <int D, class E, bool FULL>
__global__ __launch_bounds__(256) void bwd_rotate_kernel(const BParams p) {
    constexpr int NQ = D / 8, HALF = D / 2;
    const int64_t it = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (it >= (int64_t)p.total * p.num_heads * NQ) return;
    const int64_t row = it / NQ;
    const int i = (int)(it - row * NQ);
    const int t = (int)(row / p.num_heads), h = (int)(row - (int64_t)t * p.num_heads);
    const char *crow = p.cos + (int64_t)t * p.sr_s * 4, *srow = p.sin + (int64_t)t * p.sr_s * 4;
    const int64_t dst = ((int64_t)t * p.num_heads + h) * D * 2;
    u32x2 r0, r1;
    load_rotate_quad<D, E, FRA_DTYPE_F32, FULL>(p.q + ((int64_t)t * p.sq_s + (int64_t)h * p.sq_h) * 2, crow, srow, i,
                                                true, r0, r1);
    *(u32x2 *)(p.qr + dst + 8 * i) = r0;
    *(u32x2 *)(p.qr + dst + 2 * HALF + 8 * i) = r1;
    load_rotate_quad<D, E, FRA_DTYPE_F32, FULL>(p.k + ((int64_t)t * p.sk_s + (int64_t)h * p.sk_h) * 2, crow, srow, i,
                                                true, r0, r1);
    *(u32x2 *)(p.kr + dst + 8 * i) = r0;
    *(u32x2 *)(p.kr + dst + 2 * HALF + 8 * i) = r1;
}

// A operand of X^T B for a row-major LDS region X (pitch PITCH bytes) by
// ds_read_b64_tr_b16, as in the forward's PV product: for k-step (a, h) of
// 16 rows and d tile dt, lane (r, g) receives X[32a + 16h + {4g..4g+3,
// 8+4g..8+4g+3}][32dt + r] -- the row order in which the accumulator layout
// packs P / dZ as the B operand.
template <int PITCH>
__device__ __forceinline__ u32x4 tr_operand(const char *base, uint32_t lane_off, int a, int h, int dt) {
    const char *cp = base + lane_off + (32 * a + 16 * h) * PITCH + 64 * dt;
    const v4i16 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16 *)cp);
    const v4i16 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16 *)(cp + 8 * PITCH));
    const u32x2 l2 = __builtin_bit_cast(u32x2, lo), h2 = __builtin_bit_cast(u32x2, hi);
    return u32x4{l2[0], l2[1], h2[0], h2[1]};
}

template <int PITCH>
__device__ __forceinline__ uint32_t tr_lane_offset(int lane) {
    const int g = lane >> 5;
    return (uint32_t)((4 * g + ((lane >> 2) & 3)) * PITCH + 2 * (16 * ((lane >> 4) & 1) + 4 * (lane & 3)));
}

// Packs elements 8h..8h+7 of a 32x32 accumulator tile as a B operand.
template <class E>
__device__ __forceinline__ u32x4 pack8(const f32x16 &x, int h) {
    return u32x4{E::pack(x[8 * h + 0], x[8 * h + 1]), E::pack(x[8 * h + 2], x[8 * h + 3]),
                 E::pack(x[8 * h + 4], x[8 * h + 5]), E::pack(x[8 * h + 6], x[8 * h + 7])};
}

// ---- dq -------------------------------------------------------------------------

template <int D, int NW> struct DqLds {
    static constexpr int PTR = bwd_pitch_tr(D), PRD = bwd_pitch_rows(D), FP = bwd_pitch_f32(D);
    static constexpr int BQ = 32 * NW, BKV = kBwdBlockKV;
    // Two stages (key block kb in stage kb & 1), each K_rot then V.
    static constexpr int kKr = 0, kV = BKV * PTR;
    static constexpr int kStage = kV + BKV * PRD;
    static constexpr int kQ = BQ * PRD, kF = BQ * FP;
    static constexpr int kBytes = cmax(2 * kStage, cmax(kQ, kF));
};

// dq of one unit (segment, head, block of 32*NW queries).
template <int D, class E, bool FULL, int NW>
__device__ __forceinline__ void bwd_dq_unit(const BParams &p, char *lds, int unit) {
    using LDS = DqLds<D, NW>;
    constexpr int DP = bwd_dp(D), S = DP / 16, NDT = (D + 31) / 32;
    constexpr int PTR = LDS::PTR, PRD = LDS::PRD, FP = LDS::FP;
    constexpr int BQ = LDS::BQ, BKV = LDS::BKV, NT = 64 * NW;
    constexpr int kKr = LDS::kKr, kV = LDS::kV;

    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, r = lane & 31, g = lane >> 5;
    const int pi = unit / p.blocks, qb = unit - pi * p.blocks;
    const int sh = long_pair(pi, p.num_seqs * p.num_heads);
    const int seg = sh / p.num_heads, head = sh - seg * p.num_heads;
    int s0, L;
    seg_bounds(p, seg, s0, L);
    const int q0 = qb * BQ;
    if (q0 >= L) return;  // uniform
    const int nq = min(BQ, L - q0);

    // Q_rot of the block -> LDS -> the B operands of S^T (one query per lane).
    const int64_t rrs = (int64_t)p.num_heads * D * 2;  // row stride of q_rot / k_rot (bytes)
    {
        RowBlock<D, BQ, NT> qb;
        qb.load(p.qr + ((int64_t)(s0 + q0) * p.num_heads + head) * D * 2, rrs, nq, tid);
        qb.store(lds, PRD, tid);
    }
    __syncthreads();
    const int qi = 32 * w + r;
    const bool qvalid = qi < nq;
    const int qrow = s0 + q0 + (qvalid ? qi : 0);
    u32x4 qop[S], dop[S];
    const char *dorow = p.dout + ((int64_t)qrow * p.sdo_s + (int64_t)head * p.sdo_h) * 2;
#pragma unroll
    for (int t = 0; t < S; ++t) {
        qop[t] = *(const u32x4 *)(lds + qi * PRD + 32 * t + 16 * g);
        const int d0 = 16 * t + 8 * g;
        dop[t] = (qvalid && d0 < D) ? *(const u32x4 *)(dorow + 2 * d0) : u32x4{0u, 0u, 0u, 0u};
    }
    const int64_t srow = (int64_t)head * p.total + qrow;
    const float lse2 = p.lse[srow] * kLog2e;
    const float dvq = p.dvec[srow];
    const float sl = p.scale_log2;

    f32x16 dqacc[NDT];
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) dqacc[dt] = f32x16{};
    const uint32_t trl = tr_lane_offset<PTR>(lane);
    const int nkb = (L + BKV - 1) / BKV;
    // Key blocks through registers, one block ahead: block kb + 1's loads are
    // in flight while block kb is computed.
    RowBlock<D, BKV, NT> kbk;
    RowBlock<D, BKV, NT> vbk;
    auto load_block = [&](int kb) {
        const int k0 = kb * BKV, nk = min(BKV, L - k0);
        // an opaque thread id: the items' addresses are recomputed per block
        // instead of being kept live across the loop
        const int ft = fresh(tid);
        kbk.load(p.kr + ((int64_t)(s0 + k0) * p.num_heads + head) * D * 2, rrs, nk, ft);
        vbk.load(p.v + ((int64_t)(s0 + k0) * p.sv_s + (int64_t)head * p.sv_h) * 2, p.sv_s * 2, nk, ft);
    };
    // Block kb goes to LDS stage kb & 1 at the start of iteration kb - 1, so
    // a wavefront that is ahead stores the next block while the others still
    // read the current one; one barrier per block.
    auto store_block = [&](int kb) {
        const int ft = fresh(tid);
        char *const base = lds + (kb & 1) * LDS::kStage;
        kbk.store(base + kKr, PTR, ft);
        vbk.store(base + kV, PRD, ft);
    };
    load_block(0);
    __syncthreads();  // Q_rot's rows are in registers: stage 0 may go over them
    store_block(0);
    if (nkb > 1) load_block(1);
    __syncthreads();
    for (int kb = 0; kb < nkb; ++kb) {
        const int k0 = kb * BKV, nk = min(BKV, L - k0);
        if (kb + 1 < nkb) {
            store_block(kb + 1);  // the other stage: its last reader (block kb - 1) passed the barrier
            if (kb + 2 < nkb) load_block(kb + 2);
        }
        const char *const stage = lds + (kb & 1) * LDS::kStage;
        // S^T = K_rot Q_rot^T and dP^T = V dout^T: rows key, column query.
        // Tile a = 0's two chains, then tile 1's, alternating S and dP; each
        // MFMA's LDS operand is read two MFMAs ahead (read just before its
        // MFMA, every operand's latency was exposed), and the VALU work of
        // tile 0's dZ may move in beside tile 1's MFMAs.
        f32x16 sacc[2], dpacc[2];
        {
            constexpr int NM = 4 * S;
            auto oaddr = [&](int i) {
                const int a = i / (2 * S), t = (i % (2 * S)) >> 1;
                return (i & 1) ? stage + kV + (32 * a + r) * PRD + 32 * t + 16 * g
                               : stage + kKr + (32 * a + r) * PTR + 32 * t + 16 * g;
            };
            u32x4 op[3];
            op[0] = *(const u32x4 *)oaddr(0);
            op[1] = *(const u32x4 *)oaddr(1);
#pragma unroll
            for (int i = 0; i < NM; ++i) {
                if (i + 2 < NM) op[(i + 2) % 3] = *(const u32x4 *)oaddr(i + 2);
                const int a = i / (2 * S), t = (i % (2 * S)) >> 1;
                if (i & 1) dpacc[a] = E::mma(op[i % 3], dop[t], t == 0 ? f32x16{} : dpacc[a]);
                else sacc[a] = E::mma(op[i % 3], qop[t], t == 0 ? f32x16{} : sacc[a]);
                __builtin_amdgcn_sched_barrier(kSchedValuMayCross);
            }
        }
        // dZ^T = P^T * (dP^T - Dvec), keys past the segment masked.
        u32x4 dsop[2][2];
#pragma unroll
        for (int a = 0; a < 2; ++a) {
#pragma unroll
            for (int j = 0; j < 16; ++j) {
                const int key = 32 * a + 8 * (j >> 2) + 4 * g + (j & 3);
                const float pj = key < nk ? __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[a][j], sl, -lse2)) : 0.f;
                sacc[a][j] = pj * (dpacc[a][j] - dvq);
            }
#pragma unroll
            for (int h = 0; h < 2; ++h) dsop[a][h] = pack8<E>(sacc[a], h);
        }
        // dQ^T += K_rot^T dZ^T.
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt) {
#pragma unroll
            for (int a = 0; a < 2; ++a) {
#pragma unroll
                for (int h = 0; h < 2; ++h)
                    dqacc[dt] = E::mma(tr_operand<PTR>(stage + kKr, trl, a, h, dt), dsop[a][h], dqacc[dt]);
            }
        }
        __syncthreads();  // block kb + 1's stage is written; block kb's is read
    }

    // dQ_rot rows (fp32, scaled) through LDS (free after the loop's last
    // barrier), then the inverse rotation.
    float *f = (float *)lds;
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) {
#pragma unroll
        for (int jq = 0; jq < 4; ++jq) {
            const int d0 = 32 * dt + 8 * jq + 4 * g;
            if (d0 < D)
                *(f32x4 *)(f + qi * (FP / 4) + d0) =
                    f32x4{dqacc[dt][4 * jq + 0], dqacc[dt][4 * jq + 1], dqacc[dt][4 * jq + 2], dqacc[dt][4 * jq + 3]} *
                    p.scale;
        }
    }
    __syncthreads();
    unrotate_store<D, E, FULL>(f, FP / 4, p, p.dq + ((int64_t)(s0 + q0) * p.sdq_s + (int64_t)head * p.sdq_h) * 2,
                               p.sdq_s * 2, s0 + q0, nq, tid, NT);
}

// ---- dk, dv -----------------------------------------------------------------------

template <int D, int NW> struct DkdvLds {
    static constexpr int PTR = bwd_pitch_tr(D), PRD = bwd_pitch_rows(D), FP = bwd_pitch_f32(D);
    static constexpr int BKV = 32 * NW, BQ = kBwdBlockQ;
    // Two stages (query block qb in stage qb & 1), each Q_rot, dO, lse, Dvec.
    static constexpr int kQr = 0, kDo = BQ * PTR, kLse = kDo + BQ * PTR, kDv = kLse + BQ * 4;
    static constexpr int kStage = kDv + BQ * 4;
    static constexpr int kK = BKV * PRD, kF = BKV * FP;
    static constexpr int kBytes = cmax(2 * kStage, cmax(kK, kF));
};

// dk and dv of one unit (segment, head, block of 32*NW keys).
template <int D, class E, bool FULL, int NW>
__device__ __forceinline__ void bwd_dkdv_unit(const BParams &p, char *lds, int unit) {
    using LDS = DkdvLds<D, NW>;
    constexpr int DP = bwd_dp(D), S = DP / 16, NDT = (D + 31) / 32;
    constexpr int PTR = LDS::PTR, PRD = LDS::PRD, FP = LDS::FP;
    constexpr int BKV = LDS::BKV, BQ = LDS::BQ, NT = 64 * NW;
    constexpr int kQr = LDS::kQr, kDo = LDS::kDo, kLse = LDS::kLse, kDv = LDS::kDv;

    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, r = lane & 31, g = lane >> 5;
    const int pi = unit / p.blocks, kb = unit - pi * p.blocks;
    const int sh = long_pair(pi, p.num_seqs * p.num_heads);
    const int seg = sh / p.num_heads, head = sh - seg * p.num_heads;
    int s0, L;
    seg_bounds(p, seg, s0, L);
    const int k0 = kb * BKV;
    if (k0 >= L) return;  // uniform
    const int nk = min(BKV, L - k0);

    // K_rot and V of the block -> the B operands of S and dP (one key per lane).
    const int64_t rrs = (int64_t)p.num_heads * D * 2;  // row stride of q_rot / k_rot (bytes)
    {
        RowBlock<D, BKV, NT> kbk;
        kbk.load(p.kr + ((int64_t)(s0 + k0) * p.num_heads + head) * D * 2, rrs, nk, tid);
        kbk.store(lds, PRD, tid);
    }
    __syncthreads();
    const int ki = 32 * w + r;
    const bool kvalid = ki < nk;
    const int krow = s0 + k0 + (kvalid ? ki : 0);
    u32x4 kop[S], vop[S];
    const char *vrow = p.v + ((int64_t)krow * p.sv_s + (int64_t)head * p.sv_h) * 2;
#pragma unroll
    for (int t = 0; t < S; ++t) {
        kop[t] = *(const u32x4 *)(lds + ki * PRD + 32 * t + 16 * g);
        const int d0 = 16 * t + 8 * g;
        vop[t] = (kvalid && d0 < D) ? *(const u32x4 *)(vrow + 2 * d0) : u32x4{0u, 0u, 0u, 0u};
    }
    const float sl = p.scale_log2;
    f32x16 dvacc[NDT], dkacc[NDT];
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) {
        dvacc[dt] = f32x16{};
        dkacc[dt] = f32x16{};
    }
    const uint32_t trl = tr_lane_offset<PTR>(lane);
    const int nqb = (L + BQ - 1) / BQ;
    // Query blocks through registers, one block ahead: block qb + 1's loads
    // are in flight while block qb is computed.
    RowBlock<D, BQ, NT> qbk;
    RowBlock<D, BQ, NT> dbk;
    float lv, dvv;
    auto load_block = [&](int qb) {
        const int q0 = qb * BQ, nq = min(BQ, L - q0);
        // an opaque thread id: the items' addresses are recomputed per block
        // instead of being kept live across the loop
        const int ft = fresh(tid);
        qbk.load(p.qr + ((int64_t)(s0 + q0) * p.num_heads + head) * D * 2, rrs, nq, ft);
        dbk.load(p.dout + ((int64_t)(s0 + q0) * p.sdo_s + (int64_t)head * p.sdo_h) * 2, p.sdo_s * 2, nq, ft);
        // Rows past the segment: lse = +inf makes their P (and dZ) zero.
        lv = __builtin_inff();
        dvv = 0.f;
        if (ft < nq) {
            const int64_t srow = (int64_t)head * p.total + s0 + q0 + ft;
            lv = p.lse[srow] * kLog2e;
            dvv = p.dvec[srow];
        }
    };
    // Block qb goes to LDS stage qb & 1 at the start of iteration qb - 1, so
    // a wavefront that is ahead stores the next block while the others still
    // read the current one; one barrier per block.
    auto store_block = [&](int qb) {
        const int ft = fresh(tid);
        char *const base = lds + (qb & 1) * LDS::kStage;
        qbk.store(base + kQr, PTR, ft);
        dbk.store(base + kDo, PTR, ft);
        if (ft < BQ) {
            ((float *)(base + kLse))[ft] = lv;
            ((float *)(base + kDv))[ft] = dvv;
        }
    };
    load_block(0);
    __syncthreads();  // K_rot's rows are in registers: stage 0 may go over them
    store_block(0);
    if (nqb > 1) load_block(1);
    __syncthreads();
    for (int qb = 0; qb < nqb; ++qb) {
        const int q0 = qb * BQ, nq = min(BQ, L - q0);
        if (qb + 1 < nqb) {
            store_block(qb + 1);  // the other stage: its last reader (block qb - 1) passed the barrier
            if (qb + 2 < nqb) load_block(qb + 2);
        }
        const char *const stage = lds + (qb & 1) * LDS::kStage;
        const float *lsef = (const float *)(stage + kLse);
        const float *dvf = (const float *)(stage + kDv);
#pragma unroll
        for (int a = 0; a < 2; ++a) {
            if (32 * a >= nq) break;  // uniform
            // S = Q_rot K_rot^T and dP = dout V^T: rows query, column key.
            // The two chains alternate; each MFMA's LDS operand is read two
            // MFMAs ahead.
            f32x16 sacc, dpacc;
            {
                constexpr int NM = 2 * S;
                auto oaddr = [&](int i) {
                    return stage + ((i & 1) ? kDo : kQr) + (32 * a + r) * PTR + 32 * (i >> 1) + 16 * g;
                };
                u32x4 op[3];
                op[0] = *(const u32x4 *)oaddr(0);
                op[1] = *(const u32x4 *)oaddr(1);
#pragma unroll
                for (int i = 0; i < NM; ++i) {
                    if (i + 2 < NM) op[(i + 2) % 3] = *(const u32x4 *)oaddr(i + 2);
                    const int t = i >> 1;
                    if (i & 1) dpacc = E::mma(op[i % 3], vop[t], t == 0 ? f32x16{} : dpacc);
                    else sacc = E::mma(op[i % 3], kop[t], t == 0 ? f32x16{} : sacc);
                    __builtin_amdgcn_sched_barrier(kSchedValuMayCross);
                }
            }
            // Element j holds query 32a + 8(j/4) + 4g + (j%4).
#pragma unroll
            for (int m = 0; m < 4; ++m) {
                const f32x4 l4 = *(const f32x4 *)(lsef + 32 * a + 8 * m + 4 * g);
                const f32x4 d4 = *(const f32x4 *)(dvf + 32 * a + 8 * m + 4 * g);
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int j = 4 * m + i;
                    const float pj = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[j], sl, -l4[i]));
                    sacc[j] = pj;
                    dpacc[j] = pj * (dpacc[j] - d4[i]);
                }
            }
            u32x4 pop[2], dsop[2];
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                pop[h] = pack8<E>(sacc, h);
                dsop[h] = pack8<E>(dpacc, h);
            }
            // dV^T += dout^T P and dK^T += Q_rot^T dZ.
#pragma unroll
            for (int dt = 0; dt < NDT; ++dt) {
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    dvacc[dt] = E::mma(tr_operand<PTR>(stage + kDo, trl, a, h, dt), pop[h], dvacc[dt]);
                    dkacc[dt] = E::mma(tr_operand<PTR>(stage + kQr, trl, a, h, dt), dsop[h], dkacc[dt]);
                }
            }
        }
        __syncthreads();  // block qb + 1's stage is written; block qb's is read
    }

    // dV rows straight from the accumulators (lane (r, g): key ki, d = 32dt +
    // 8jq + 4g .. +3).
    if (kvalid) {
        char *dvr = p.dv + ((int64_t)(s0 + k0 + ki) * p.sdv_s + (int64_t)head * p.sdv_h) * 2;
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt) {
#pragma unroll
            for (int jq = 0; jq < 4; ++jq) {
                const int d0 = 32 * dt + 8 * jq + 4 * g;
                if (d0 < D)
                    *(u32x2 *)(dvr + 2 * d0) = u32x2{E::pack(dvacc[dt][4 * jq + 0], dvacc[dt][4 * jq + 1]),
                                                     E::pack(dvacc[dt][4 * jq + 2], dvacc[dt][4 * jq + 3])};
            }
        }
    }
    // dK_rot rows (fp32, scaled) through LDS, then the inverse rotation.
    __syncthreads();
    float *f = (float *)lds;
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) {
#pragma unroll
        for (int jq = 0; jq < 4; ++jq) {
            const int d0 = 32 * dt + 8 * jq + 4 * g;
            if (d0 < D)
                *(f32x4 *)(f + ki * (FP / 4) + d0) =
                    f32x4{dkacc[dt][4 * jq + 0], dkacc[dt][4 * jq + 1], dkacc[dt][4 * jq + 2], dkacc[dt][4 * jq + 3]} *
                    p.scale;
        }
    }
    __syncthreads();
    unrotate_store<D, E, FULL>(f, FP / 4, p, p.dk + ((int64_t)(s0 + k0) * p.sdk_s + (int64_t)head * p.sdk_h) * 2,
                               p.sdk_s * 2, s0 + k0, nk, tid, NT);
}

// The dq and dk/dv units of a call in one launch: logical unit 2u is the
// dk/dv unit u, 2u + 1 the dq unit u (same segment, head and block, so the
// pair shares its q, k, v and dout lines in one XCD's L2, and every XCD gets
// both kinds).  One grid of both leaves one partly filled last round of
// workgroups instead of two.
template <int D, class E, bool FULL, int NW>
__global__ __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(BwdOcc<D>::kWaves, BwdOcc<D>::kWaves)))
void bwd_long_kernel(const BParams p) {
    __shared__ __attribute__((aligned(16))) char lds[cmax(DqLds<D, NW>::kBytes, DkdvLds<D, NW>::kBytes)];
    const int b = xcd_remap(blockIdx.x, gridDim.x);
    if ((b & 1) == 0)
        bwd_dkdv_unit<D, E, FULL, NW>(p, lds, b >> 1);
    else
        bwd_dq_unit<D, E, FULL, NW>(p, lds, b >> 1);
}

// ---- window layers: the whole backward of one (segment, head) in one pass -------------
//
// Segments of at most 64 tokens (every query block is every key block): one
// workgroup of two wavefronts per (segment, head) stages Q_rot, K_rot, dO and
// V once and produces dq, dk and dv, so each input is read from HBM once (the
// two-kernel path reads q, k, v and dO twice and out and dO once more).
//   phase 1  wave w owns queries 32w..32w+31 (the dq kernel's layout): Dvec of
//            its queries from dO (LDS) and out (HBM), then S^T, dP^T, dZ^T and
//            dQ^T = K_rot^T dZ^T; it takes its keys' K_rot and V rows as
//            registers before the barrier that frees their LDS for dQ's rows;
//   phase 2  wave w owns keys 32w..32w+31 (the dk/dv kernel's layout): S, dP,
//            dZ, dV^T = dO^T P and dK^T = Q_rot^T dZ; dv is stored from
//            registers and dk's rows go through LDS for the inverse rotation.
// VREG = false: V is staged too; dQ's fp32 rows go over K_rot + V after
// phase 1, dK's after them at the end.  VREG = true: a lane's rows of V come
// from HBM as registers, and dQ's then dK's fp32 rows go over the dead
// staging one after the other at the end, so that four workgroups fit on a
// CU at D <= 96 instead of three.  Which pays depends on the grid: four per
// CU took a 1024-workgroup layer (cfg1) from two rounds to one (38 -> 32 µs)
// but made a 2304-workgroup one (cfg2w) 5% slower, so the host takes VREG
// only when the grid fits four per CU and not three.
template <int D, bool VREG> struct WinBwdLds {
    static constexpr int PTR = bwd_pitch_tr(D), PRD = bwd_pitch_rows(D), FP = bwd_pitch_f32(D);
    static constexpr int kKr = 0, kV = 64 * PTR, kQr = kV + (VREG ? 0 : 64 * PRD), kDo = kQr + 64 * PTR;
    static constexpr int kLse = kDo + 64 * PTR, kDvec = kLse + 64 * 4;
    static constexpr int kStage = kDvec + 64 * 4;
    static constexpr int kFq = 0, kFk = VREG ? 0 : 64 * FP;
    static_assert(VREG || 64 * FP <= kQr, "dQ rows must fit over the K_rot and V staging");
    static constexpr int kBytes = cmax(kStage, (VREG ? 1 : 2) * 64 * FP);
    // Workgroups (two wavefronts) per CU: LDS and the waves-per-SIMD budget.
    static constexpr int kPerCu = cmin(160 * 1024 / kBytes, 4 * BwdOcc<D>::kWaves / 2);
};

template <int D, class E, bool FULL, bool VREG>
__global__ __launch_bounds__(128) __attribute__((amdgpu_waves_per_eu(BwdOcc<D>::kWaves, BwdOcc<D>::kWaves)))
void bwd_window_kernel(const BParams p) {
    using LDS = WinBwdLds<D, VREG>;
    constexpr int DP = bwd_dp(D), S = DP / 16, NDT = (D + 31) / 32;
    constexpr int PTR = LDS::PTR, PRD = LDS::PRD, FP = LDS::FP;
    constexpr int NT = 128;
    __shared__ __attribute__((aligned(16))) char lds[LDS::kBytes];

    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, r = lane & 31, g = lane >> 5;
    const int unit = xcd_remap(blockIdx.x, gridDim.x);
    const int seg = unit / p.num_heads, head = unit - seg * p.num_heads;
    int s0, L;
    seg_bounds(p, seg, s0, L);
    if (L <= 0) return;  // uniform
    // Launched when max_seqlen <= 64; a longer segment (an understated
    // max_seqlen) gets unspecified gradients, never an access past 64 rows.
    L = min(L, 64);
    const int64_t qoff = ((int64_t)s0 * p.sq_s + (int64_t)head * p.sq_h) * 2;
    const int64_t koff = ((int64_t)s0 * p.sk_s + (int64_t)head * p.sk_h) * 2;
    const int row = 32 * w + (lane & 31);  // phase 1: this lane's query; phase 2: its key
    const bool rvalid = row < L;
    // Every load of the workgroup first (one HBM round trip), then the
    // rotations and LDS writes.  q and k share their cos/sin loads.
    u32x4 orow[S];  // this lane's row of out, for Dvec in phase 1
    // VREG: V rows 32a + r, elements 16t + 8g..: the A operands of dP^T in
    // phase 1, and (a = w) this lane's key row, the B operand of dP in phase 2.
    u32x4 va[VREG ? 2 : 1][S];
    {
        RotBlock<D, E, FULL, 64, NT, 2> qk;
        RowBlock<D, VREG ? 1 : 64, NT> vb;
        RowBlock<D, 64, NT> db;
        const char *const x[2] = {p.q + qoff, p.k + koff};
        const int64_t xs[2] = {p.sq_s * 2, p.sk_s * 2};
        qk.load(p, x, xs, s0, L, tid);
        const char *vbase = p.v + ((int64_t)s0 * p.sv_s + (int64_t)head * p.sv_h) * 2;
        if constexpr (VREG) {
#pragma unroll
            for (int a = 0; a < 2; ++a) {
                const int vr = 32 * a + r;
#pragma unroll
                for (int t = 0; t < S; ++t) {
                    const int d0 = 16 * t + 8 * g;
                    va[a][t] = (vr < L && d0 < D) ? *(const u32x4 *)(vbase + (int64_t)vr * p.sv_s * 2 + 2 * d0)
                                                  : u32x4{0u, 0u, 0u, 0u};
                }
            }
        } else {
            vb.load(vbase, p.sv_s * 2, L, tid);
        }
        db.load(p.dout + ((int64_t)s0 * p.sdo_s + (int64_t)head * p.sdo_h) * 2, p.sdo_s * 2, L, tid);
        const char *op = p.out + ((int64_t)(s0 + (rvalid ? row : 0)) * p.so_s + (int64_t)head * p.so_h) * 2;
#pragma unroll
        for (int t = 0; t < S; ++t) {
            const int d0 = 16 * t + 8 * (lane >> 5);
            orow[t] = (rvalid && d0 < D) ? *(const u32x4 *)(op + 2 * d0) : u32x4{0u, 0u, 0u, 0u};
        }
        // rows past the segment: lse = +inf makes their P (and dZ) zero
        const float lv = tid < L ? p.lse[(int64_t)head * p.total + s0 + tid] * kLog2e : __builtin_inff();
        char *const dst[2] = {lds + LDS::kQr, lds + LDS::kKr};
        qk.store(dst, PTR, L, tid);
        if constexpr (!VREG) vb.store(lds + LDS::kV, PRD, tid);
        db.store(lds + LDS::kDo, PTR, tid);
        if (tid < 64) ((float *)(lds + LDS::kLse))[tid] = lv;
    }
    __syncthreads();

    const float sl = p.scale_log2;
    const uint32_t trl = tr_lane_offset<PTR>(lane);
    const int ntile = (L + 31) >> 5;  // 32-row tiles of queries (and of keys)

    // ---- phase 1: dQ for queries 32w..32w+31 -----------------------------------------
    f32x16 dqacc[NDT];
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) dqacc[dt] = f32x16{};
    {
        u32x4 qop[S], dop[S];
        float dot = 0.f;
#pragma unroll
        for (int t = 0; t < S; ++t) {
            qop[t] = *(const u32x4 *)(lds + LDS::kQr + row * PTR + 32 * t + 16 * g);
            dop[t] = *(const u32x4 *)(lds + LDS::kDo + row * PTR + 32 * t + 16 * g);
#pragma unroll
            for (int e = 0; e < 4; ++e) {  // orow is zero past the row and the segment
                dot = __builtin_fmaf(E::lo(orow[t][e]), E::lo(dop[t][e]), dot);
                dot = __builtin_fmaf(E::hi(orow[t][e]), E::hi(dop[t][e]), dot);
            }
        }
        const float dvq = sum_pair32(dot);  // rowsum(dO * O) of query `row`
        if (g == 0) ((float *)(lds + LDS::kDvec))[row] = dvq;
        const float lse2 = ((const float *)(lds + LDS::kLse))[row];
        if (w < ntile) {  // uniform per wavefront
            f32x16 sacc[2], dpacc[2];
#pragma unroll
            for (int a = 0; a < 2; ++a) {
                sacc[a] = f32x16{};
                dpacc[a] = f32x16{};
                if (a < ntile) {
#pragma unroll
                    for (int t = 0; t < S; ++t)
                        sacc[a] = E::mma(*(const u32x4 *)(lds + LDS::kKr + (32 * a + r) * PTR + 32 * t + 16 * g),
                                         qop[t], sacc[a]);
#pragma unroll
                    for (int t = 0; t < S; ++t) {
                        if constexpr (VREG)
                            dpacc[a] = E::mma(va[a][t], dop[t], dpacc[a]);
                        else
                            dpacc[a] = E::mma(*(const u32x4 *)(lds + LDS::kV + (32 * a + r) * PRD + 32 * t + 16 * g),
                                              dop[t], dpacc[a]);
                    }
                }
            }
            u32x4 dsop[2][2];
#pragma unroll
            for (int a = 0; a < 2; ++a) {
#pragma unroll
                for (int j = 0; j < 16; ++j) {
                    const int key = 32 * a + 8 * (j >> 2) + 4 * g + (j & 3);
                    const float pj = key < L ? __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[a][j], sl, -lse2)) : 0.f;
                    sacc[a][j] = pj * (dpacc[a][j] - dvq);
                }
#pragma unroll
                for (int h = 0; h < 2; ++h) dsop[a][h] = pack8<E>(sacc[a], h);
            }
#pragma unroll
            for (int dt = 0; dt < NDT; ++dt) {
#pragma unroll
                for (int a = 0; a < 2; ++a) {
                    if (a >= ntile) break;
#pragma unroll
                    for (int h = 0; h < 2; ++h)
                        dqacc[dt] = E::mma(tr_operand<PTR>(lds + LDS::kKr, trl, a, h, dt), dsop[a][h], dqacc[dt]);
                }
            }
        }
    }
    // Phase 2's B operands: this lane's key row of K_rot, and of V (VREG:
    // tile w of the phase-1 operands, a select of values, not of the array
    // slots), before their LDS is reused.
    u32x4 kop[S], vop[S];
#pragma unroll
    for (int t = 0; t < S; ++t) {
        kop[t] = *(const u32x4 *)(lds + LDS::kKr + row * PTR + 32 * t + 16 * g);
        if constexpr (VREG) vop[t] = w ? +va[VREG ? 1 : 0][t] : +va[0][t];
        else vop[t] = *(const u32x4 *)(lds + LDS::kV + row * PRD + 32 * t + 16 * g);
    }
    __syncthreads();  // Dvec is complete (and, without VREG, K_rot and V are dead)
    // fp32 rows of dQ_rot, then of dK_rot, each followed by the inverse
    // rotation and the store.
    auto rows_out = [&](float *f, const f32x16 (&acc)[NDT]) {
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt) {
#pragma unroll
            for (int jq = 0; jq < 4; ++jq) {
                const int d0 = 32 * dt + 8 * jq + 4 * g;
                if (d0 < D)
                    *(f32x4 *)(f + row * (FP / 4) + d0) =
                        f32x4{acc[dt][4 * jq + 0], acc[dt][4 * jq + 1], acc[dt][4 * jq + 2], acc[dt][4 * jq + 3]} *
                        p.scale;
            }
        }
    };
    float *fq = (float *)(lds + LDS::kFq), *fk = (float *)(lds + LDS::kFk);
    if constexpr (!VREG) rows_out(fq, dqacc);

    // ---- phase 2: dK, dV for keys 32w..32w+31 ----------------------------------------
    f32x16 dvacc[NDT], dkacc[NDT];
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) {
        dvacc[dt] = f32x16{};
        dkacc[dt] = f32x16{};
    }
    if (w < ntile) {  // uniform per wavefront
        const float *lsef = (const float *)(lds + LDS::kLse);
        const float *dvf = (const float *)(lds + LDS::kDvec);
#pragma unroll
        for (int a = 0; a < 2; ++a) {
            if (a >= ntile) break;
            f32x16 sacc = f32x16{}, dpacc = f32x16{};
#pragma unroll
            for (int t = 0; t < S; ++t)
                sacc = E::mma(*(const u32x4 *)(lds + LDS::kQr + (32 * a + r) * PTR + 32 * t + 16 * g), kop[t], sacc);
#pragma unroll
            for (int t = 0; t < S; ++t)
                dpacc = E::mma(*(const u32x4 *)(lds + LDS::kDo + (32 * a + r) * PTR + 32 * t + 16 * g), vop[t], dpacc);
#pragma unroll
            for (int m = 0; m < 4; ++m) {
                const f32x4 l4 = *(const f32x4 *)(lsef + 32 * a + 8 * m + 4 * g);
                const f32x4 d4 = *(const f32x4 *)(dvf + 32 * a + 8 * m + 4 * g);
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int j = 4 * m + i;
                    const float pj = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[j], sl, -l4[i]));
                    sacc[j] = pj;
                    dpacc[j] = pj * (dpacc[j] - d4[i]);
                }
            }
            u32x4 pop[2], dsop[2];
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                pop[h] = pack8<E>(sacc, h);
                dsop[h] = pack8<E>(dpacc, h);
            }
#pragma unroll
            for (int dt = 0; dt < NDT; ++dt) {
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    dvacc[dt] = E::mma(tr_operand<PTR>(lds + LDS::kDo, trl, a, h, dt), pop[h], dvacc[dt]);
                    dkacc[dt] = E::mma(tr_operand<PTR>(lds + LDS::kQr, trl, a, h, dt), dsop[h], dkacc[dt]);
                }
            }
        }
    }
    if (rvalid) {
        char *dvr = p.dv + ((int64_t)(s0 + row) * p.sdv_s + (int64_t)head * p.sdv_h) * 2;
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt) {
#pragma unroll
            for (int jq = 0; jq < 4; ++jq) {
                const int d0 = 32 * dt + 8 * jq + 4 * g;
                if (d0 < D)
                    *(u32x2 *)(dvr + 2 * d0) = u32x2{E::pack(dvacc[dt][4 * jq + 0], dvacc[dt][4 * jq + 1]),
                                                     E::pack(dvacc[dt][4 * jq + 2], dvacc[dt][4 * jq + 3])};
            }
        }
    }
    __syncthreads();  // Q_rot and dO are dead
    if constexpr (VREG) {
        rows_out(fq, dqacc);
        __syncthreads();
        unrotate_store<D, E, FULL>(fq, FP / 4, p, p.dq + ((int64_t)s0 * p.sdq_s + (int64_t)head * p.sdq_h) * 2,
                                   p.sdq_s * 2, s0, L, tid, NT);
        __syncthreads();  // dQ's rows are read
        rows_out(fk, dkacc);
        __syncthreads();
    } else {
        rows_out(fk, dkacc);
        __syncthreads();
        unrotate_store<D, E, FULL>(fq, FP / 4, p, p.dq + ((int64_t)s0 * p.sdq_s + (int64_t)head * p.sdq_h) * 2,
                                   p.sdq_s * 2, s0, L, tid, NT);
    }
    unrotate_store<D, E, FULL>(fk, FP / 4, p, p.dk + ((int64_t)s0 * p.sdk_s + (int64_t)head * p.sdk_h) * 2,
                               p.sdk_s * 2, s0, L, tid, NT);
}

}  // namespace

namespace fra_internal {

template <int D, class E, bool FULL, int NW>
BwdKernels bwd_kernels_nw() {
    // A register-V instance only where it fits more workgroups per CU than
    // the staged kernel (the planner could never choose it otherwise: D = 64,
    // whose staged kernel fits four, and D >= 128, two either way), and not
    // at D = 96 with full-width tables (it spills).
    constexpr bool kVreg = !(D == 96 && FULL) && WinBwdLds<D, true>::kPerCu > WinBwdLds<D, false>::kPerCu;
    BwdFn vreg = nullptr;
    if constexpr (kVreg) vreg = (BwdFn)bwd_window_kernel<D, E, FULL, true>;
    return BwdKernels{(BwdFn)bwd_dot_kernel<D, E>,
                      (BwdFn)bwd_rotate_kernel<D, E, FULL>,
                      (BwdFn)bwd_long_kernel<D, E, FULL, NW>,
                      NW,
                      (BwdFn)bwd_window_kernel<D, E, FULL, false>,
                      vreg,
                      WinBwdLds<D, false>::kPerCu,
                      kVreg ? WinBwdLds<D, true>::kPerCu : 0};
}

template <int D, class E>
BwdKernels bwd_kernels_e(bool full) {
    return full ? bwd_kernels_nw<D, E, true, 4>() : bwd_kernels_nw<D, E, false, 4>();
}

template <int D>
BwdKernels bwd_kernels_d(int qkv, bool full) {
    return qkv == FRA_DTYPE_BF16 ? bwd_kernels_e<D, BF16>(full) : bwd_kernels_e<D, F16>(full);
}

}  // namespace fra_internal
