// fra_device.h -- device-side types and helpers shared by the forward
// (fra_kernels.hip) and backward (fra_bwd.hip) kernels of libfra.so.
//
// Everything here sits in an anonymous namespace: each translation unit gets
// its own copy of these inline helpers, and none of them is exported.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "fra.h"

// Records a failure message for fra_last_error() (thread-local) and returns
// `code`.  Defined in fra_kernels.hip; hidden, not part of the C ABI.
__attribute__((visibility("hidden"), format(printf, 2, 3))) int fra_fail(int code, const char *fmt, ...);

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
constexpr float kLn2 = 0.6931471805599453f;

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

// ---- unit order of the long kernels (forward and backward) ----------------------------
//
// Units u = (pair position i, block) with u = i * blocks + block, and
// pairs (segment, head) sh = seg * heads + head taken in an order that deals
// them out to the eight XCDs by residue: position i is pair 8k + r for the
// i-th (r, k) in r-major order.  xcd_remap gives XCD x a contiguous range of
// units, so XCD x works on pairs x, x + 8, x + 16, ...: the heads of every
// segment are spread over all XCDs, which keeps layers of unequal segments
// balanced (in segment order, one XCD took nearly all units of the longest
// image of a ragged batch), while the query blocks of one pair stay on one
// XCD, sharing its K/V rows in L2.
__device__ __forceinline__ int long_pair(int i, int pairs) {
    const int q = pairs >> 3, rem = pairs & 7;
    const int big = rem * (q + 1);  // the first rem residues hold q + 1 pairs
    int r, k;
    if (i < big) {
        r = i / (q + 1);
        k = i - r * (q + 1);
    } else {
        const int j = i - big;
        r = rem + j / q;
        k = j - (j / q) * q;
    }
    return 8 * k + r;
}

// v_permlane32_swap with both operands in a and b: lanes 32..63 of a trade
// places with lanes 0..31 of b, so when both start as x, one of them holds
// x of lanes 0..31 in both halves and the other x of lanes 32..63.  It is a
// VALU op: no LDS round trip (and no wait on other LDS reads in flight) on
// the softmax's critical path.  The clang builtin of this toolchain returns
// the first register for both results, hence the asm; the s_nop gives the
// two wait states a VALU write needs before the permlane reads it.
__device__ __forceinline__ void permlane32_swap(float &a, float &b) {
    asm("s_nop 1\n\tv_permlane32_swap_b32 %0, %1" : "+v"(a), "+v"(b));
}

// One direct load per lane: 16 bytes from src to LDS byte address
// lds_addr + 16 * lane (lds_addr wave-uniform).  The compiler counts a
// direct load as an LDS store of unknown place, and then makes every later
// transposed LDS read wait (vmcnt(0)) for every direct load in flight,
// whichever buffer either touches; issued from asm, the loads are the
// caller's to wait for (s_waitcnt vmcnt and a barrier before the
// destination is read).  M0 is a reserved register, which a clobber list
// does not protect, so the asm saves and restores it; the s_nops are the
// wait states between writing M0 and the load that reads it, and between
// the load and the restore.
__device__ __forceinline__ void dma16(const void *src, uint32_t lds_addr) {
    const uint32_t m0v = __builtin_amdgcn_readfirstlane(lds_addr);  // uniform: already scalar, or one readlane
    uint32_t saved;
    asm volatile(
        "s_mov_b32 %0, m0\n\ts_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off\n\t"
        "s_nop 0\n\ts_mov_b32 m0, %0"
        : "=&s"(saved)
        : "v"(src), "s"(m0v)
        : "memory");
}

// Compute units of the current device (host code; cached per device and
// translation unit; 256 when no device can be queried, e.g. planning on a
// host without a GPU).
inline int device_cus() {
    static int cached[64] = {0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) {
        (void)hipGetLastError();
        return 256;
    }
    if (cached[dev] == 0) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) {
            (void)hipGetLastError();
            n = 256;
        }
        cached[dev] = n;
    }
    return cached[dev];
}

// max and sum of x over lanes l and l ^ 32 (symmetric, so the result does
// not depend on which operand receives which half).
__device__ __forceinline__ float max_pair32(float x) {
    float a = x, b = x;
    permlane32_swap(a, b);
    return fmaxf(a, b);
}
__device__ __forceinline__ float sum_pair32(float x) {
    float a = x, b = x;
    permlane32_swap(a, b);
    return a + b;
}

// x of lane (l & 31) in every lane l: the upper half is zeroed first, so the
// sum of the two swapped registers is the lower half's value whichever
// register it lands in.
__device__ __forceinline__ float bcast_lo32(float x) {
    float a = (threadIdx.x & 32) ? 0.f : x, b = a;
    permlane32_swap(a, b);
    return a + b;
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

// Split-half rotation of one quad pair in fp32 (reference
// fused_attn.py:340-345 and :385-390: x0*cos - x1*sin, x0*sin + x1*cos),
// packed to the storage dtype.  Each output is one product and one FMA, the
// form FP contraction (on by default in Triton) gives the reference
// expression; it differs from separately rounded products by at most one
// fp32 rounding before the result is rounded to 16 bits.
template <class E>
__device__ __forceinline__ void rotate_quad(u32x2 x0w, u32x2 x1w, f32x4 c0, f32x4 s0, f32x4 c1, f32x4 s1,
                                            u32x2 &r0w, u32x2 &r1w) {
    const float x0[4] = {E::lo(x0w[0]), E::hi(x0w[0]), E::lo(x0w[1]), E::hi(x0w[1])};
    const float x1[4] = {E::lo(x1w[0]), E::hi(x1w[0]), E::lo(x1w[1]), E::hi(x1w[1])};
    float r0[4], r1[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        r0[i] = __builtin_fmaf(x0[i], c0[i], -(x1[i] * s0[i]));
        r1[i] = __builtin_fmaf(x0[i], s1[i], x1[i] * c1[i]);
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

}  // namespace
