// Device helpers shared by the gfx950 kernels: bf16 rounding, the MLX-affine
// 4-bit unpack into bf16 pairs, wave reductions, and bounded spin waits.
//
// Numerics: storage is bf16, accumulation f32, and values are rounded to bf16
// (round to nearest even) at the points where the reference's MLX graph
// materialises a bf16 array (src/ming_fused.zig:17-25).  The library is built
// with -ffp-contract=off, so an expression rounds exactly as written; fused
// multiply-adds appear only where a kernel calls fmaf() or a dot builtin.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace ming {

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

constexpr int kWave = 64;

// ---- bf16 -----------------------------------------------------------------

__device__ __forceinline__ float bf2f(uint16_t h) { return __uint_as_float((uint32_t)h << 16); }
__device__ __forceinline__ float bf_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// f32 -> bf16, round to nearest even, NaN stays NaN: gfx950's
// v_cvt_pk_bf16_f32 (one instruction per pair).  It agrees bit for bit with
// the integer sequence u += 0x7fff + ((u >> 16) & 1), u >>= 16 on all 2^32
// inputs whose value is not NaN, denormals included.
typedef float f32x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint16_t f2bf(float f) { return __builtin_bit_cast(uint16_t, (__bf16)f); }
__device__ __forceinline__ float rb(float f) { return bf2f(f2bf(f)); }
__device__ __forceinline__ uint32_t pack_bf2(float lo, float hi) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{lo, hi}, bf16x2_t));
}

// e^x for the flow head's softmax and sigmoids, built only from correctly
// rounded f32 operations (multiply, rint, fma, ldexp), so that a CPU that
// evaluates the same steps gets the same bits: Cody-Waite reduction
// x = n ln2 + r with ln2 split into a 15-bit head and its f32 tail (|r| <=
// ln2/2 + a few ulps), the degree-7 Taylor polynomial of e^r in Horner form
// (truncation below 2^-27 relative) and an exact scaling by 2^n.  Measured
// against double exp over [-86, 88]: at most 0.92 ulp.  Below -86 the result
// is 0 (e^-86 < 2^-124; the scaled polynomial would reach denormals), above 88
// +inf; NaN stays NaN.
__device__ __forceinline__ float exp_rep(float x) {
    if (x < -86.0f) return 0.0f;
    if (x > 88.0f) return __builtin_inff();
    const float n = __builtin_rintf(x * 0x1.715476p+0f);
    float r = __builtin_fmaf(n, -0x1.62e4p-1f, x);
    r = __builtin_fmaf(n, -0x1.7f7d1cp-20f, r);
    float p = 0x1.a01a02p-13f;              // 1/7!
    p = __builtin_fmaf(p, r, 0x1.6c16c2p-10f);  // 1/6!
    p = __builtin_fmaf(p, r, 0x1.111112p-7f);   // 1/5!
    p = __builtin_fmaf(p, r, 0x1.555556p-5f);   // 1/4!
    p = __builtin_fmaf(p, r, 0x1.555556p-3f);   // 1/3!
    p = __builtin_fmaf(p, r, 0.5f);
    p = __builtin_fmaf(p, r, 1.0f);
    p = __builtin_fmaf(p, r, 1.0f);
    return __builtin_ldexpf(p, (int)n);
}

// acc + a.lo*b.lo + a.hi*b.hi with bf16 pairs packed in u32 (v_dot2c_f32_bf16).
// Not an IEEE sequence: measured on gfx950, the two exact products are
// truncated toward zero onto the grid 2^(e_p - 24) (e_p: the larger product's
// exponent-field sum) and summed; acc joins on the grid 2^(e_acc - 31) when its
// exponent exceeds e_p (the product sum floored onto it), else floored onto the
// product grid; the sum is rounded once to nearest even (a zero result is +0).
// Each 8-k block of v_mfma_f32_16x16x32_bf16 accumulates the same way.
__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float acc) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a), __builtin_bit_cast(bf16x2_t, b), acc,
                                           false);
}

// ---- MLX affine 4-bit unpack ------------------------------------------------
// A u32 word holds 8 nibbles, element 8j+i in bits [4i, 4i+4) (low first).
// OR-ing a nibble q into the mantissa of bf16(128) gives bf16(128 + q)
// exactly, so one v_and_or_b32 turns two nibbles into a bf16 pair.  The pairs
// are (q0,q4), (q1,q5), (q2,q6), (q3,q7); the activation vector is staged in
// the same pair order, and the +128 offset is removed in the group epilogue:
//   sum_k (s q_k + b) x_k = s * sum_k (128 + q_k) x_k + (b - 128 s) * sum_k x_k.
constexpr uint32_t kQ4Magic = 0x43004300u;  // bf16(128) | bf16(128) << 16

__device__ __forceinline__ void q4_pairs(uint32_t w, uint32_t& p0, uint32_t& p1, uint32_t& p2, uint32_t& p3) {
    p0 = (w & 0x000f000fu) | kQ4Magic;
    p1 = ((w >> 4) & 0x000f000fu) | kQ4Magic;
    p2 = ((w >> 8) & 0x000f000fu) | kQ4Magic;
    p3 = ((w >> 12) & 0x000f000fu) | kQ4Magic;
}

// Dot product of one 8-element word of nibbles with the pair-ordered
// activations xp[0..3] = (x0,x4),(x1,x5),(x2,x6),(x3,x7).
__device__ __forceinline__ float q4_word_dot(uint32_t w, const uint32_t* xp, float acc) {
    uint32_t p0, p1, p2, p3;
    q4_pairs(w, p0, p1, p2, p3);
    acc = dot2(p0, xp[0], acc);
    acc = dot2(p1, xp[1], acc);
    acc = dot2(p2, xp[2], acc);
    acc = dot2(p3, xp[3], acc);
    return acc;
}

// ---- reductions -------------------------------------------------------------

// Butterfly reductions over aligned teams of W lanes (W = 2..64) on VALU
// data paths: DPP quad_perm for lane distance 1 and 2, DPP half-row and row
// mirrors to complete 8- and 16-lane groups, and gfx950's permlane16/32 swaps
// across rows.  Each step combines two values symmetrically, so every lane of
// a team ends with the bit-identical result.
template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false));
}

template <int W, class Op>
__device__ __forceinline__ float team_reduce(float v, Op op) {
    if (W > 1) v = op(v, dpp<0xB1>(v));   // quad_perm [1,0,3,2]
    if (W > 2) v = op(v, dpp<0x4E>(v));   // quad_perm [2,3,0,1]
    if (W > 4) v = op(v, dpp<0x141>(v));  // row_half_mirror
    if (W > 8) v = op(v, dpp<0x140>(v));  // row_mirror
    if (W > 16) {
        const auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
        v = op(__uint_as_float(p[0]), __uint_as_float(p[1]));
    }
    if (W > 32) {
        const auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
        v = op(__uint_as_float(p[0]), __uint_as_float(p[1]));
    }
    return v;
}

// Combine the four lanes l, l ^ 16, l ^ 32, l ^ 48 (the same place in each
// 16-lane row) with the permlane swaps: the butterfly of __shfl_xor over 16
// and 32, bit for bit (add and max are commutative), without LDS round trips.
template <class Op>
__device__ __forceinline__ float rows_reduce(float v, Op op) {
    auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = op(__uint_as_float(p[0]), __uint_as_float(p[1]));
    p = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return op(__uint_as_float(p[0]), __uint_as_float(p[1]));
}
__device__ __forceinline__ float rows_sum(float v) { return rows_reduce(v, [](float a, float b) { return a + b; }); }
__device__ __forceinline__ float rows_max(float v) { return rows_reduce(v, [](float a, float b) { return fmaxf(a, b); }); }

// e^x for attention softmaxes and their merges: the native base-2 exponential
// (v_exp_f32, about one ulp) of x log2(e), two instructions where expf takes
// about ten (range reduction, special cases); -inf gives 0.
__device__ __forceinline__ float att_exp(float x) { return __builtin_amdgcn_exp2f(x * 1.44269504088896341f); }

// The value of lane l ^ 1 (DPP quad_perm [1,0,3,2]) and of lane l ^ 32
// (v_permlane32_swap: its first result holds the low half twice, its second the
// high half twice), exactly what __shfl(v, l ^ 1) and __shfl(v, l ^ 32) read,
// without an LDS round trip.
__device__ __forceinline__ float lane_xor1(float v) { return dpp<0xB1>(v); }
__device__ __forceinline__ float lane_xor32(float v, int lane) {
    const auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(lane < 32 ? p[1] : p[0]);
}

// Lane `lane`'s value (a constant lane) for the whole wave, by v_readlane.
__device__ __forceinline__ float lane_of(float v, int lane) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}

template <int W>
__device__ __forceinline__ float team_sum(float v) {
    return team_reduce<W>(v, [](float a, float b) { return a + b; });
}

template <int W>
__device__ __forceinline__ float team_max(float v) {
    return team_reduce<W>(v, [](float a, float b) { return fmaxf(a, b); });
}

// Workgroup barrier that orders LDS accesses only.  __syncthreads() also
// drains every outstanding global load of the calling wave (its fence waits
// for the memory counters); this one lets weight prefetches stay in flight.
__device__ __forceinline__ void lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Block-wide sum over blockDim.x threads (multiple of 64); `red` holds one
// float per wave.  All threads get the result.
__device__ __forceinline__ float block_sum(float v, float* red) {
    v = team_sum<kWave>(v);
    const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave, nw = blockDim.x / kWave;
    lds_sync();
    if (lane == 0) red[wave] = v;
    lds_sync();
    float s = 0.0f;
    for (int i = 0; i < nw; i++) s += red[i];
    return s;
}

__device__ __forceinline__ float block_max(float v, float* red) {
    v = team_max<kWave>(v);
    const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave, nw = blockDim.x / kWave;
    lds_sync();
    if (lane == 0) red[wave] = v;
    lds_sync();
    float s = -INFINITY;
    for (int i = 0; i < nw; i++) s = fmaxf(s, red[i]);
    return s;
}

// ---- global memory -------------------------------------------------------------
// Accesses through these views compile to global_* instructions.  Through a
// generic pointer whose origin the compiler cannot see (one loaded from an
// argument block) they would be flat_* instructions, which also count against
// the LDS counter: the next LDS access would then wait for them, which turns a
// weight prefetch into a stall.
#define MING_GLOBAL __attribute__((address_space(1)))

typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

template <class T>  // scalar T
__device__ __forceinline__ T gld(const T* p) {
    return *(const MING_GLOBAL T*)p;
}
template <class T>  // scalar T
__device__ __forceinline__ void gst(T* p, T v) {
    *(MING_GLOBAL T*)p = v;
}
__device__ __forceinline__ void gst(uint4* p, uint4 v) {
    *(MING_GLOBAL u32x4_t*)p = u32x4_t{v.x, v.y, v.z, v.w};
}
__device__ __forceinline__ uint4 ldg4(const void* p) {
    const u32x4_t v = *(const MING_GLOBAL u32x4_t*)p;
    return make_uint4(v.x, v.y, v.z, v.w);
}

// MFMA operand and accumulator types (v_mfma_f32_16x16x32_bf16).
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ bf16x8_t as_bf8(uint4 v) { return __builtin_bit_cast(bf16x8_t, u32x4_t{v.x, v.y, v.z, v.w}); }

}  // namespace ming
