// Batched MLX-affine 4-bit GEMM on MFMA: Y[M][N] = g * X[M][K] W^T with W in
// the MLX affine format (u32 [N][K/8], 8 nibbles low first; bf16 scale and
// bias per group of 64) -- mlx_quantized_matmul / gather_qmm with M > 1
// (src/mlx.zig:279-282), the multi-request shape where the weight bytes are
// shared by M rows and the contraction is dense enough for the matrix cores.
//
// Arithmetic (exact as the batch-1 GEMV's): OR-ing a nibble q into the
// mantissa of bf16(128) gives bf16(128 + q) exactly, so v_mfma_f32_16x16x32_bf16
// computes sum_k (128 + q_k) x_k per group of 64 without rounding the weights;
// the group is then folded in f32 as s * acc + (b - 128 s) * sum_k x_k.  The
// activations are staged once per call (stage_kernel) in the MFMA A operand's
// layout: 16-byte words of 8 values in nibble-pair order (x0,x4), (x1,x5),
// (x2,x6), (x3,x7), matching the unpacked weight word, plus the f32 group sums.
//
// MFMA 16x16x32 bf16 lane layout on gfx950 (checked on the device): the A
// operand of lane l is row l % 16, k-block l / 16 (8 values); B is column
// l % 16, the same k-block; C[r] is (row 4 (l / 16) + r, column l % 16).
// Here rows are activation rows (M), columns weight rows (N).  Within a group
// (8 words) lane l takes words 2j and 2j+1 (j = l / 16), one per MFMA, so each
// MFMA's 32 k lie in one group and a lane loads 8 contiguous bytes per row.
//
// Workgroup (column block x, row-tile group y): KW waves split the groups of
// K; each wave accumulates MT x 16 rows by NW x 16 columns, with two groups'
// loads in flight while one group's MFMAs run; the waves' partial sums are
// added through LDS and every wave applies the epilogue (QEpi) to its share of
// the rows.  One call may concatenate up to three matrices along N (q/k/v;
// gate/up), each a run of workgroups.  Staged activations are group-major:
// xs [K/64][Mp][8] 16-byte words, xsum [K/64][Mp] (Mp = M rounded up to 16).
#include "batch.h"
#include "common.h"
#include "internal.h"

namespace ming {

namespace {

typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ uint2 ldg2(const void* p) {
    const u32x2_t v = *(const MING_GLOBAL u32x2_t*)p;
    return make_uint2(v.x, v.y);
}

// A value the compiler must keep in a register: with the nibble mask and the
// magic constant in registers, each pair is one v_and_or_b32 (gfx9 VOP3 takes
// no literal operands, so with literals it would be an AND and an OR).
__device__ __forceinline__ uint32_t in_reg(uint32_t v) {
    asm volatile("" : "+v"(v));
    return v;
}

// bf16 pairs (128 + q_i, 128 + q_{i+4}) of one packed word, as the 8-value B operand.
__device__ __forceinline__ bf16x8_t unpack_b(uint32_t w, uint32_t mask, uint32_t magic) {
    return __builtin_bit_cast(bf16x8_t, u32x4_t{(w & mask) | magic, ((w >> 4) & mask) | magic,
                                                ((w >> 8) & mask) | magic, ((w >> 12) & mask) | magic});
}

__device__ __forceinline__ bf16x8_t as_a(uint4 v) { return __builtin_bit_cast(bf16x8_t, u32x4_t{v.x, v.y, v.z, v.w}); }

__device__ __forceinline__ const QSeg& pick(const QgemmArgs& a, int si) {
    return si == 0 ? a.seg[0] : (si == 1 ? a.seg[1] : a.seg[2]);
}

// One group's operands of one lane.
template <int MT, int NW>
struct GroupIn {
    uint2 wq[NW];       // words 2j, 2j+1 of the group, weight row of tile t
    float sc[NW], bi[NW];
    uint4 xa[MT][2];    // A operand words 2j, 2j+1 of row 16 mt + c
    float4 xsv[MT];     // group sums of rows 16 mt + 4j + r, r = 0..3
};

// Per-lane 32-bit byte offsets from the uniform bases: the loads then take a
// scalar base plus a 32-bit vector offset, with no per-load 64-bit arithmetic.
template <int MT, int NW>
struct Offs {
    uint32_t w[NW];     // row n_t * K/2 + 8j
    uint32_t s[NW];     // row n_t * G * 2
    uint32_t x;         // ((16 mt0 + c) * 8 + 2j) * 16     (+ g * Mp * 128 + 2048 mt)
    uint32_t xs;        // (16 mt0 + 4j) * 4                  (+ g * Mp * 4 + 64 mt)
};

template <class T>
__device__ __forceinline__ const T* at(const T* base, uint32_t byte_off) {
    return reinterpret_cast<const T*>(reinterpret_cast<const char*>(base) + byte_off);
}

template <int MT, int NW>
__device__ __forceinline__ void group_load(const QgemmArgs& a, const uint32_t* const (&wb)[NW],
                                           const uint16_t* const (&sb)[NW], const uint16_t* const (&bb)[NW],
                                           const Offs<MT, NW>& o, int Mp, int g, GroupIn<MT, NW>& in) {
    const uint4* xs = static_cast<const uint4*>(a.xs);
#pragma unroll
    for (int t = 0; t < NW; t++) {
        in.wq[t] = ldg2(at(wb[t], o.w[t] + 32u * g));
        in.sc[t] = bf2f(gld(at(sb[t], o.s[t] + 2u * g)));
        in.bi[t] = bf2f(gld(at(bb[t], o.s[t] + 2u * g)));
    }
    const uint32_t xg = o.x + (uint32_t)g * Mp * 128u, sg = o.xs + (uint32_t)g * Mp * 4u;
#pragma unroll
    for (int mt = 0; mt < MT; mt++) {
        in.xa[mt][0] = ldg4(at(xs, xg + 2048u * mt));
        in.xa[mt][1] = ldg4(at(xs, xg + 2048u * mt + 16u));
        const uint4 v = ldg4(at(a.xsum, sg + 64u * mt));
        in.xsv[mt] = make_float4(__uint_as_float(v.x), __uint_as_float(v.y), __uint_as_float(v.z), __uint_as_float(v.w));
    }
}

// acc += s * sum_k (128 + q_k) x_k + (b - 128 s) * sum_k x_k for one group.  The
// MFMAs of tile t + 1 are issued before tile t is folded, so the fold's VALU
// work covers the matrix core's latency.
template <int MT, int NW>
__device__ __forceinline__ void group_mma(const GroupIn<MT, NW>& in, f32x4_t (&acc)[MT][NW], uint32_t mask,
                                          uint32_t magic) {
    f32x4_t ag[2][MT];
    auto issue = [&](int t, f32x4_t (&dst)[MT]) {
        const bf16x8_t b0 = unpack_b(in.wq[t].x, mask, magic), b1 = unpack_b(in.wq[t].y, mask, magic);
#pragma unroll
        for (int mt = 0; mt < MT; mt++)
            dst[mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_a(in.xa[mt][0]), b0, f32x4_t{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
#pragma unroll
        for (int mt = 0; mt < MT; mt++)
            dst[mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_a(in.xa[mt][1]), b1, dst[mt], 0, 0, 0);
    };
    auto fold = [&](int t, const f32x4_t (&src)[MT]) {
        const float s = in.sc[t], off = fmaf(-128.0f, in.sc[t], in.bi[t]);
#pragma unroll
        for (int mt = 0; mt < MT; mt++) {
            const float xv[4] = {in.xsv[mt].x, in.xsv[mt].y, in.xsv[mt].z, in.xsv[mt].w};
#pragma unroll
            for (int r = 0; r < 4; r++) acc[mt][t][r] = fmaf(off, xv[r], fmaf(s, src[mt][r], acc[mt][t][r]));
        }
    };
    issue(0, ag[0]);
#pragma unroll
    for (int t = 0; t < NW; t++) {
        if (t + 1 < NW) issue(t + 1, ag[(t + 1) & 1]);
        fold(t, ag[t & 1]);
    }
}

// q/k/v epilogue of one activation row m: bias, rope (q, k), qkv row, k/v append.
template <int MT, int NW>
__device__ __forceinline__ void qkv_row(const QgemmArgs& a, const QSeg& S, int si, int n0, int c, int m,
                                        const float (&v)[NW]) {
    static_assert(NW == 4, "one head of 64 columns per workgroup");
    const QPaged& P = a.pg;
    const int pos = gld(P.pos + m);
    float e[4];
#pragma unroll
    for (int t = 0; t < 4; t++) e[t] = rb(rb(v[t] * S.gscale) + bf2f(gld(S.bias + n0 + 16 * t + c)));
    const bool pos_ok = pos >= 0 && pos < P.max_ctx && pos / 64 < P.pages_per_seq;
    if (si < 2 && pos_ok) {  // MLX fast::rope, non-traditional: pairs (d, d + 32)
#pragma unroll
        for (int t = 0; t < 2; t++) {
            const int d = 16 * t + c;
            const float2 cs = *reinterpret_cast<const float2*>(P.rope_cs + ((size_t)pos * 32 + d) * 2);
            const float o1 = e[t] * cs.x - e[t + 2] * cs.y, o2 = e[t] * cs.y + e[t + 2] * cs.x;
            e[t] = rb(o1);
            e[t + 2] = rb(o2);
        }
    }
#pragma unroll
    for (int t = 0; t < 4; t++) gst(a.y + (size_t)m * a.ldy + S.col0 + n0 + 16 * t + c, f2bf(e[t]));
    if (si == 0) return;
    int page = -1;
    if (pos_ok) page = gld(P.table + (size_t)m * P.pages_per_seq + pos / 64);
    if (page < 0 || page >= P.n_pages) {
        if (c == 0) gst(P.flags, 1);
        return;
    }
    const int kh = n0 / 64, slot = pos % 64;
    const size_t base = ((size_t)page * P.kvh + kh) * 64 * 64;
#pragma unroll
    for (int t = 0; t < 4; t++) {
        const int d = 16 * t + c;
        if (si == 1)
            gst(P.kp + base + (size_t)slot * 64 + d, f2bf(e[t]));
        else
            gst(P.vp + base + (size_t)d * 64 + slot, f2bf(e[t]));
    }
}

// Per-row argmax of the workgroup's columns (lowest index on ties): lanes of
// one j hold one row; v[t] is column n0 + 16t + c.
template <int NW>
__device__ __forceinline__ void row_argmax(const QgemmArgs& a, int n0, int c, int m, const float (&v)[NW], int N) {
    float best = -INFINITY;
    int idx = 0x7fffffff;
#pragma unroll
    for (int t = 0; t < NW; t++) {
        const int n = n0 + 16 * t + c;
        if (n < N && v[t] > best) {
            best = v[t];
            idx = n;
        }
    }
#pragma unroll
    for (int d = 1; d < 16; d <<= 1) {
        const float ov = __shfl_xor(best, d);
        const int oi = __shfl_xor(idx, d);
        if (ov > best || (ov == best && oi < idx)) {
            best = ov;
            idx = oi;
        }
    }
    if (c == 0) {
        const int blk = n0 / (16 * NW);
        gst(a.pmax + (size_t)m * a.nblk + blk, best);
        gst(a.pidx + (size_t)m * a.nblk + blk, idx);
    }
}

// The epilogue of activation row m: v[t] is the sum of column tile t of this lane.
template <int MT, int NW, int EPI>
__device__ __forceinline__ void epi_row(const QgemmArgs& a, const QSeg& S, int si, int n0, int c, int m,
                                        float (&v)[NW]) {
    constexpr int TPS = EPI == QE_SWIGLU ? NW / 2 : NW;  // column tiles per segment and workgroup
    if constexpr (EPI == QE_QKV) {
        qkv_row<MT, NW>(a, S, si, n0, c, m, v);
    } else if constexpr (EPI == QE_SWIGLU) {
        const float gg = a.seg[0].gscale, gu = a.seg[1].gscale;
#pragma unroll
        for (int t = 0; t < TPS; t++) {
            const int n = n0 + 16 * t + c;
            if (n >= S.N) continue;
            const float gv = rb(v[t] * gg), u = rb(v[t + TPS] * gu);
            const float sg = rb(1.0f / (1.0f + expf(-gv)));
            gst(a.y + (size_t)m * a.ldy + n, f2bf(rb(gv * sg) * u));
        }
    } else {
#pragma unroll
        for (int t = 0; t < NW; t++) {
            v[t] *= S.gscale;
            const int n = n0 + 16 * t + c;
            if (n >= S.N) continue;
            const size_t off = (size_t)m * a.ldy + S.col0 + n;
            if constexpr (EPI == QE_RES) {
                gst(a.y + off, f2bf(bf2f(gld(a.res + (size_t)m * a.ldres + S.col0 + n)) + rb(v[t])));
            } else {
                if (a.y) gst(a.y + off, f2bf(v[t]));
                if (a.yf) gst(a.yf + off, v[t]);
            }
        }
        if constexpr (EPI == QE_PLAIN)
            if (a.pmax) row_argmax<NW>(a, n0, c, m, v, S.N);
    }
}

// KW = blockDim.x / 64 waves (<= KWMAX) split the K/64 groups; each wave takes
// its groups either through a three-deep register ring (GPW = 0) or in chunks
// of GPW whose loads are all issued before the chunk's MFMAs.
template <int MT, int NW, int GPW, int KWMAX, int EPI>
__global__ __launch_bounds__(64 * KWMAX) void qgemm_kernel(QgemmArgs a) {
    extern __shared__ float red[];  // [KW][MT * 4][NW][64]
    constexpr int TPS = EPI == QE_SWIGLU ? NW / 2 : NW;  // column tiles per segment and workgroup
    const int KW = blockDim.x / kWave;
    const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave, c = lane % 16, j = lane / 16;
    int blk = blockIdx.x, si = 0;
    if (EPI != QE_SWIGLU && a.nseg > 1 && blk >= a.blocks[0]) {
        blk -= a.blocks[0];
        si = 1;
        if (a.nseg > 2 && blk >= a.blocks[1]) {
            blk -= a.blocks[1];
            si = 2;
        }
    }
    const int n0 = blk * 16 * TPS;
    const int G = a.K / 64, KW8 = a.K / 8, MTT = (a.M + 15) / 16, Mp = 16 * MTT;
    const int mt0 = blockIdx.y * MT;  // the launcher picks MT dividing MTT
    const uint32_t* wb[NW];
    const uint16_t* sb[NW];
    const uint16_t* bb[NW];
    Offs<MT, NW> o;
#pragma unroll
    for (int t = 0; t < NW; t++) {
        const QSeg& S = pick(a, EPI == QE_SWIGLU ? (t < TPS ? 0 : 1) : si);
        const int n = min(n0 + 16 * (t % TPS) + c, S.N - 1);
        wb[t] = S.w;
        sb[t] = S.s;
        bb[t] = S.b;
        o.w[t] = (uint32_t)n * KW8 * 4u + 8u * j;
        o.s[t] = (uint32_t)n * G * 2u;
    }
    o.x = ((uint32_t)(16 * mt0 + c) * 8u + 2u * j) * 16u;
    o.xs = (uint32_t)(16 * mt0 + 4 * j) * 4u;
    const int gper = (G + KW - 1) / KW, g0 = wave * gper, g1 = min(G, g0 + gper);
    f32x4_t acc[MT][NW];
#pragma unroll
    for (int mt = 0; mt < MT; mt++)
#pragma unroll
        for (int t = 0; t < NW; t++) acc[mt][t] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
    const uint32_t mask = in_reg(0x000f000fu), magic = in_reg(kQ4Magic);
    if constexpr (GPW == 0) {
        // a ring of three groups in registers: two groups' loads in flight while one computes
        if (g0 < g1) {
            GroupIn<MT, NW> b0, b1, b2;
            group_load<MT, NW>(a, wb, sb, bb, o, Mp, g0, b0);
            if (g0 + 1 < g1) group_load<MT, NW>(a, wb, sb, bb, o, Mp, g0 + 1, b1);
            for (int g = g0; g < g1; g += 3) {
                if (g + 2 < g1) group_load<MT, NW>(a, wb, sb, bb, o, Mp, g + 2, b2);
                group_mma<MT, NW>(b0, acc, mask, magic);
                if (g + 1 >= g1) break;
                if (g + 3 < g1) group_load<MT, NW>(a, wb, sb, bb, o, Mp, g + 3, b0);
                group_mma<MT, NW>(b1, acc, mask, magic);
                if (g + 2 >= g1) break;
                if (g + 4 < g1) group_load<MT, NW>(a, wb, sb, bb, o, Mp, g + 4, b1);
                group_mma<MT, NW>(b2, acc, mask, magic);
            }
        }
    } else {
        // chunks of GPW groups whose loads are all issued before the chunk's MFMAs
        for (int gb = g0; gb < g1; gb += GPW) {
            GroupIn<MT, NW> in[GPW];
#pragma unroll
            for (int u = 0; u < GPW; u++)
                if (gb + u < g1) group_load<MT, NW>(a, wb, sb, bb, o, Mp, gb + u, in[u]);
#pragma unroll
            for (int u = 0; u < GPW; u++)
                if (gb + u < g1) group_mma<MT, NW>(in[u], acc, mask, magic);
        }
    }
    // the waves' partial sums through LDS; wave w then owns the row slots u = mt * 4 + r with u % KW == w
    if (KWMAX > 1) {
#pragma unroll
        for (int mt = 0; mt < MT; mt++)
#pragma unroll
            for (int r = 0; r < 4; r++)
#pragma unroll
                for (int t = 0; t < NW; t++) red[(((wave * MT + mt) * 4 + r) * NW + t) * kWave + lane] = acc[mt][t][r];
        __syncthreads();
    }
    const QSeg& S = pick(a, si);
#pragma unroll
    for (int mt = 0; mt < MT; mt++)
#pragma unroll
        for (int r = 0; r < 4; r++) {
            if ((mt * 4 + r) % KW != wave) continue;
            const int m = 16 * (mt0 + mt) + 4 * j + r;
            if (m >= a.M) continue;
            float v[NW];
#pragma unroll
            for (int t = 0; t < NW; t++) {
                if (KWMAX > 1) {
                    float sum = 0.0f;
                    for (int w = 0; w < KW; w++) sum += red[(((w * MT + mt) * 4 + r) * NW + t) * kWave + lane];
                    v[t] = sum;
                } else {
                    v[t] = acc[mt][t][r];
                }
            }
            epi_row<MT, NW, EPI>(a, S, si, n0, c, m, v);
        }
}

// ---- more than 64 rows (prompt prefill) ------------------------------------------
// A workgroup of 4 waves in a WM x WN grid owns a tile of 16 WM MT rows and
// WN NW 16 weight columns (of one segment; for SwiGLU each wave's NW/2 gate
// and NW/2 up tiles), wave (wm, wn) the MT x NW tiles at (wm, wn).  K runs in
// chunks of kLdsGK groups through two LDS buffers: the workgroup loads a
// chunk's activation words and group sums (coalesced, from the staged
// layout) and its weights, which it unpacks once into (128 + q) bf16 pairs --
// the B operand group_mma builds in registers, bit for bit -- with each
// column's scale and b - 128 s; the next chunk's global loads are issued
// before this chunk's MFMAs and stored after them.  Every wave walks all of K;
// where a K slice of the shape's <= 64-row launch ends (kslices slices of
// ceil(G / kslices) groups, summed by that launch's waves and added through
// LDS from zero in slice order) it adds the slice's sum to a running total in
// the same order, so a row's bits do not depend on the number of rows.
constexpr int kLdsGK = 2;                    // groups per LDS chunk
constexpr int kRowStride = kLdsGK * 8 + 1;   // uint4 per row / column in LDS (one of padding)

template <int MT>
struct AIn {
    uint4 xa[MT][2];   // A operand words 2j, 2j+1 of row 16 mt + c
    float4 xsv[MT];    // group sums of rows 16 mt + 4j + r
};

// One group from pre-unpacked B operands, in group_mma's order and arithmetic.
template <int MT, int NW>
__device__ __forceinline__ void group_mma_pre(const AIn<MT>& in, const uint4 (&b)[NW][2], const float (&sc)[NW],
                                              const float (&off)[NW], f32x4_t (&acc)[MT][NW]) {
    f32x4_t ag[2][MT];
    auto issue = [&](int t, f32x4_t (&dst)[MT]) {
        const bf16x8_t b0 = as_a(b[t][0]), b1 = as_a(b[t][1]);
#pragma unroll
        for (int mt = 0; mt < MT; mt++)
            dst[mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_a(in.xa[mt][0]), b0, f32x4_t{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
#pragma unroll
        for (int mt = 0; mt < MT; mt++)
            dst[mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_a(in.xa[mt][1]), b1, dst[mt], 0, 0, 0);
    };
    auto fold = [&](int t, const f32x4_t (&src)[MT]) {
#pragma unroll
        for (int mt = 0; mt < MT; mt++) {
            const float xv[4] = {in.xsv[mt].x, in.xsv[mt].y, in.xsv[mt].z, in.xsv[mt].w};
#pragma unroll
            for (int r = 0; r < 4; r++) acc[mt][t][r] = fmaf(off[t], xv[r], fmaf(sc[t], src[mt][r], acc[mt][t][r]));
        }
    };
    issue(0, ag[0]);
#pragma unroll
    for (int t = 0; t < NW; t++) {
        if (t + 1 < NW) issue(t + 1, ag[(t + 1) & 1]);
        fold(t, ag[t & 1]);
    }
}

template <int WM, int WN, int MT, int NW, int EPI>
__global__ __launch_bounds__(256) void qgemm_lds_kernel(QgemmArgs a, int kslices) {
    static_assert(WM * WN == 4, "four waves");
    constexpr int TPS = EPI == QE_SWIGLU ? NW / 2 : NW;
    constexpr int BM = 16 * WM * MT, NC = 16 * WN * NW;         // rows, weight columns of the tile
    constexpr int AQ = BM * kLdsGK * 8 / 256;                   // activation uint4 per thread per chunk
    static_assert(AQ * 256 == BM * kLdsGK * 8, "whole activation chunk per thread");
    __shared__ uint4 As[2][BM * kRowStride];
    __shared__ __align__(16) float Xs[2][kLdsGK * BM];          // group sums [group][row], read as float4
    __shared__ uint4 Bs[2][NC * kRowStride];
    __shared__ float2 Ss[2][NC * kLdsGK];                       // (scale, b - 128 scale)
    const int tid = threadIdx.x, wave = tid / kWave, lane = tid % kWave, c = lane % 16, j = lane / 16;
    const int wm = wave / WN, wn = wave % WN;
    int blk = blockIdx.x, si = 0;
    if (EPI != QE_SWIGLU && a.nseg > 1 && blk >= a.blocks[0]) {
        blk -= a.blocks[0];
        si = 1;
        if (a.nseg > 2 && blk >= a.blocks[1]) {
            blk -= a.blocks[1];
            si = 2;
        }
    }
    // output column c0 of the tile: tile columns (wn, t) are n0 + 16 (wn TPS + t % TPS) + c
    const int n0 = blk * 16 * TPS * WN;
    const int G = a.K / 64, KW8 = a.K / 8, MTT = (a.M + 15) / 16, Mp = 16 * MTT;
    const int r0 = blockIdx.y * BM;  // the tile's first row (rows past Mp are clamped for the loads)
    // weight column k of the tile (k = 16 (wn NW + t) + cc): its segment and row
    auto wcol = [&](int k, const QSeg*& S) {
        const int wq = k / (16 * NW), t = (k / 16) % NW;
        S = &pick(a, EPI == QE_SWIGLU ? (t < TPS ? 0 : 1) : si);
        return min(n0 + 16 * (wq * TPS + t % TPS) + k % 16, S->N - 1);
    };
    // loads of a chunk: activations (AQ uint4 per thread), group sums (threads < kLdsGK BM / 4, one uint4),
    // weights (threads < 2 kLdsGK NC: column k, group, half of 4 words), scales (threads < kLdsGK NC)
    const int wk = tid / (2 * kLdsGK), wgg = (tid / 2) % kLdsGK, wh = tid % 2;
    const bool wload = tid < NC * kLdsGK * 2;
    const QSeg* WS;
    const int wn_row = wcol(min(wk, NC - 1), WS);
    const uint32_t* wrow = WS->w + (size_t)wn_row * KW8;
    const int sk = tid / kLdsGK, sgg = tid % kLdsGK;
    const bool sload = tid < NC * kLdsGK;
    const QSeg* SS;
    const int sn = wcol(min(sk, NC - 1), SS);
    const bool xload = tid < kLdsGK * BM / 4;
    const int xgg = tid / (BM / 4), xr = (tid % (BM / 4)) * 4;  // group, first of 4 rows
    const uint32_t mask = in_reg(0x000f000fu), magic = in_reg(kQ4Magic);
    const uint4* xs = static_cast<const uint4*>(a.xs);
    const int nch = (G + kLdsGK - 1) / kLdsGK;
    struct Raw {
        uint4 a[AQ], w, x;
        uint32_t s, b;
    };
    auto fetch = [&](int ch, Raw& R) {
#pragma unroll
        for (int i = 0; i < AQ; i++) {  // uint4 q = tid + 256 i of the chunk: row q / (8 kLdsGK), group, word
            const int q = tid + 256 * i, row = q / (8 * kLdsGK), gg = (q / 8) % kLdsGK, wd = q % 8;
            const int g = min(ch * kLdsGK + gg, G - 1), m = min(r0 + row, Mp - 1);
            R.a[i] = ldg4(xs + ((size_t)g * Mp + m) * 8 + wd);
        }
        if (xload) {
            const int g = min(ch * kLdsGK + xgg, G - 1), m = min(r0 + xr, Mp - 4);
            R.x = ldg4(a.xsum + (size_t)g * Mp + m);
        }
        const int g = ch * kLdsGK + wgg;
        if (wload && g < G) R.w = ldg4(wrow + 8 * g + 4 * wh);
        const int gs = ch * kLdsGK + sgg;
        if (sload && gs < G) {
            R.s = gld(SS->s + (size_t)sn * G + gs);
            R.b = gld(SS->b + (size_t)sn * G + gs);
        }
    };
    auto store = [&](const Raw& R, int buf) {
#pragma unroll
        for (int i = 0; i < AQ; i++) {
            const int q = tid + 256 * i, row = q / (8 * kLdsGK), gg = (q / 8) % kLdsGK, wd = q % 8;
            As[buf][row * kRowStride + gg * 8 + wd] = R.a[i];
        }
        if (xload) {
            Xs[buf][xgg * BM + xr] = __uint_as_float(R.x.x);
            Xs[buf][xgg * BM + xr + 1] = __uint_as_float(R.x.y);
            Xs[buf][xgg * BM + xr + 2] = __uint_as_float(R.x.z);
            Xs[buf][xgg * BM + xr + 3] = __uint_as_float(R.x.w);
        }
        if (wload) {
            const uint32_t w4[4] = {R.w.x, R.w.y, R.w.z, R.w.w};
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const uint32_t w = w4[i];
                Bs[buf][wk * kRowStride + wgg * 8 + 4 * wh + i] =
                    make_uint4((w & mask) | magic, ((w >> 4) & mask) | magic, ((w >> 8) & mask) | magic,
                               ((w >> 12) & mask) | magic);
            }
        }
        if (sload) {
            const float sv = bf2f((uint16_t)R.s), bv = bf2f((uint16_t)R.b);
            Ss[buf][sk * kLdsGK + sgg] = make_float2(sv, fmaf(-128.0f, sv, bv));
        }
    };
    f32x4_t acc[MT][NW], run[MT][NW];
#pragma unroll
    for (int mt = 0; mt < MT; mt++)
#pragma unroll
        for (int t = 0; t < NW; t++) acc[mt][t] = run[mt][t] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
    const int gper = (G + kslices - 1) / kslices;
    auto chunk = [&](int ch, int buf) {
#pragma unroll
        for (int gg = 0; gg < kLdsGK; gg++) {
            const int g = ch * kLdsGK + gg;
            if (g >= G) break;
            AIn<MT> in;
#pragma unroll
            for (int mt = 0; mt < MT; mt++) {
                const int row = 16 * (wm * MT + mt);
                in.xa[mt][0] = As[buf][(row + c) * kRowStride + gg * 8 + 2 * j];
                in.xa[mt][1] = As[buf][(row + c) * kRowStride + gg * 8 + 2 * j + 1];
                in.xsv[mt] = *reinterpret_cast<const float4*>(&Xs[buf][gg * BM + row + 4 * j]);
            }
            uint4 b[NW][2];
            float sc[NW], off[NW];
#pragma unroll
            for (int t = 0; t < NW; t++) {
                const int col = 16 * (wn * NW + t) + c;
                b[t][0] = Bs[buf][col * kRowStride + gg * 8 + 2 * j];
                b[t][1] = Bs[buf][col * kRowStride + gg * 8 + 2 * j + 1];
                const float2 f = Ss[buf][col * kLdsGK + gg];
                sc[t] = f.x;
                off[t] = f.y;
            }
            group_mma_pre<MT, NW>(in, b, sc, off, acc);
            if ((g + 1) % gper == 0 || g + 1 == G) {
#pragma unroll
                for (int mt = 0; mt < MT; mt++)
#pragma unroll
                    for (int t = 0; t < NW; t++) {
                        run[mt][t] = run[mt][t] + acc[mt][t];
                        acc[mt][t] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
                    }
            }
        }
    };
    // two chunks' global loads in flight (register sets R0, R1) while one computes from LDS
    Raw R0{}, R1{};
    fetch(0, R0);
    store(R0, 0);
    if (nch > 1) fetch(1, R1);
    if (nch > 2) fetch(2, R0);
    __syncthreads();
    for (int ch = 0; ch < nch; ch += 2) {
        chunk(ch, 0);
        if (ch + 1 < nch) store(R1, 1);
        __syncthreads();
        if (ch + 3 < nch) fetch(ch + 3, R1);
        if (ch + 1 >= nch) break;
        chunk(ch + 1, 1);
        if (ch + 2 < nch) store(R0, 0);
        __syncthreads();
        if (ch + 4 < nch) fetch(ch + 4, R0);
    }
    // slices of the <= 64-row launch that hold no group add zero partials there
    for (int sidx = (G + gper - 1) / gper; sidx < kslices; sidx++)
#pragma unroll
        for (int mt = 0; mt < MT; mt++)
#pragma unroll
            for (int t = 0; t < NW; t++) run[mt][t] = run[mt][t] + f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
    const QSeg& S = pick(a, si);
    const int nw0 = n0 + 16 * wn * TPS;  // this wave's first output column
#pragma unroll
    for (int mt = 0; mt < MT; mt++)
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int m = r0 + 16 * (wm * MT + mt) + 4 * j + r;
            if (m >= a.M) continue;
            float v[NW];
#pragma unroll
            for (int t = 0; t < NW; t++) v[t] = run[mt][t][r];
            epi_row<MT, NW, EPI>(a, S, si, nw0, c, m, v);
        }
}

// One group from packed weight words: as group_mma_pre (the same MFMA chain and
// fold, so the same bits), with each column tile's two B operands unpacked from
// its two u32 words (8 nibbles each, pair order) right before their MFMAs.
template <int MT, int NW>
__device__ __forceinline__ void group_mma_packed(const AIn<MT>& in, const uint32_t (&bw)[NW][2], const float (&sc)[NW],
                                                 const float (&off)[NW], f32x4_t (&acc)[MT][NW], uint32_t mask,
                                                 uint32_t magic) {
    f32x4_t ag[2][MT];
    auto unpack = [&](uint32_t w) {
        return make_uint4((w & mask) | magic, ((w >> 4) & mask) | magic, ((w >> 8) & mask) | magic,
                          ((w >> 12) & mask) | magic);
    };
    auto issue = [&](int t, f32x4_t (&dst)[MT]) {
        const bf16x8_t b0 = as_a(unpack(bw[t][0])), b1 = as_a(unpack(bw[t][1]));
#pragma unroll
        for (int mt = 0; mt < MT; mt++)
            dst[mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_a(in.xa[mt][0]), b0, f32x4_t{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
#pragma unroll
        for (int mt = 0; mt < MT; mt++)
            dst[mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_a(in.xa[mt][1]), b1, dst[mt], 0, 0, 0);
    };
    auto fold = [&](int t, const f32x4_t (&src)[MT]) {
#pragma unroll
        for (int mt = 0; mt < MT; mt++) {
            const float xv[4] = {in.xsv[mt].x, in.xsv[mt].y, in.xsv[mt].z, in.xsv[mt].w};
#pragma unroll
            for (int r = 0; r < 4; r++) acc[mt][t][r] = fmaf(off[t], xv[r], fmaf(sc[t], src[mt][r], acc[mt][t][r]));
        }
    };
    issue(0, ag[0]);
#pragma unroll
    for (int t = 0; t < NW; t++) {
        if (t + 1 < NW) issue(t + 1, ag[(t + 1) & 1]);
        fold(t, ag[t & 1]);
    }
}

// More than 64 rows, wide tiles: qgemm_lds_kernel's arithmetic (group order,
// K slices of the <= 64-row launch, fold) on WM x WN waves with MT x NW tiles
// each, the weights kept packed in LDS (4 bits a value instead of the 16 of an
// unpacked B operand) so that a tile of 16 NW WN columns fits: every column
// and group word is stored word-major, Bp[word][column] with a row of kBPad
// words, so the 64 lanes of an operand read (16 columns x 4 words 2 j + h)
// fall in 64 distinct banks.  The activation rows are re-read once per 16 TPS
// WN output columns instead of once per 32.
constexpr int kBWords = kLdsGK * 8;  // packed words of one column per chunk
template <int NC>
struct BPad {
    static constexpr int v = NC + 8;  // 2 j rows apart = 16 j banks: with c, 64 distinct banks
};

template <int WM, int WN, int MT, int NW, int EPI>
__global__ __launch_bounds__(64 * WM * WN) void qgemm_wide_kernel(QgemmArgs a, int kslices) {
    constexpr int T = 64 * WM * WN;
    constexpr int TPS = EPI == QE_SWIGLU ? NW / 2 : NW;
    constexpr int BM = 16 * WM * MT, NC = 16 * WN * NW;  // rows, weight columns of the tile
    constexpr int AQ = BM * kLdsGK * 8 / T;              // activation uint4 per thread per chunk
    constexpr int WQ = NC * kBWords / 4 / T;             // packed weight uint4 per thread per chunk
    constexpr int SQ = NC * kLdsGK / T;                  // (scale, bias) pairs per thread per chunk
    constexpr int BP = BPad<NC>::v;
    static_assert(AQ * T == BM * kLdsGK * 8 && WQ * T * 4 == NC * kBWords && SQ * T == NC * kLdsGK, "whole chunk");
    __shared__ uint4 As[2][BM * kRowStride];
    __shared__ __align__(16) float Xs[2][kLdsGK * BM];
    __shared__ uint32_t Bp[2][kBWords * BP];
    __shared__ float2 Ss[2][NC * kLdsGK];
    const int tid = threadIdx.x, lane = tid % kWave, c = lane % 16, j = lane / 16;
    const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
    const int wm = wave / WN, wn = wave % WN;
    int blk = blockIdx.x, si = 0;
    if (EPI != QE_SWIGLU && a.nseg > 1 && blk >= a.blocks[0]) {
        blk -= a.blocks[0];
        si = 1;
        if (a.nseg > 2 && blk >= a.blocks[1]) {
            blk -= a.blocks[1];
            si = 2;
        }
    }
    const int n0 = blk * 16 * TPS * WN;
    const int G = a.K / 64, KW8 = a.K / 8, MTT = (a.M + 15) / 16, Mp = 16 * MTT;
    const int r0 = blockIdx.y * BM;
    auto wcol = [&](int k, const QSeg*& S) {
        const int wq = k / (16 * NW), t = (k / 16) % NW;
        S = &pick(a, EPI == QE_SWIGLU ? (t < TPS ? 0 : 1) : si);
        return min(n0 + 16 * (wq * TPS + t % TPS) + k % 16, S->N - 1);
    };
    // this thread's packed-weight loads: uint4 q = tid + T i -> column q / 4, group (q / 2) % 2, half q % 2
    const uint32_t* wrow[WQ];
#pragma unroll
    for (int i = 0; i < WQ; i++) {
        const QSeg* WS;
        const int q = tid + T * i;
        const int n = wcol(q / 4, WS);
        wrow[i] = WS->w + (size_t)n * KW8;
    }
    const uint16_t* srow[SQ];
    const uint16_t* brow[SQ];
#pragma unroll
    for (int i = 0; i < SQ; i++) {
        const QSeg* SS;
        const int q = tid + T * i, n = wcol(q / kLdsGK, SS);
        srow[i] = SS->s + (size_t)n * G;
        brow[i] = SS->b + (size_t)n * G;
    }
    const bool xload = tid < kLdsGK * BM / 4;
    const int xgg = tid / (BM / 4), xr = (tid % (BM / 4)) * 4;
    const uint32_t mask = in_reg(0x000f000fu), magic = in_reg(kQ4Magic);
    const uint4* xs = static_cast<const uint4*>(a.xs);
    const int nch = (G + kLdsGK - 1) / kLdsGK;
    struct Raw {
        uint4 a[AQ], w[WQ], x;
        uint32_t s[SQ], b[SQ];
    };
    auto fetch = [&](int ch, Raw& R) {
#pragma unroll
        for (int i = 0; i < AQ; i++) {
            const int q = tid + T * i, row = q / (8 * kLdsGK), gg = (q / 8) % kLdsGK, wd = q % 8;
            const int g = min(ch * kLdsGK + gg, G - 1), m = min(r0 + row, Mp - 1);
            R.a[i] = ldg4(xs + ((size_t)g * Mp + m) * 8 + wd);
        }
        if (xload) {
            const int g = min(ch * kLdsGK + xgg, G - 1), m = min(r0 + xr, Mp - 4);
            R.x = ldg4(a.xsum + (size_t)g * Mp + m);
        }
#pragma unroll
        for (int i = 0; i < WQ; i++) {
            const int q = tid + T * i, gg = (q / 2) % kLdsGK, wh = q % 2, g = min(ch * kLdsGK + gg, G - 1);
            R.w[i] = ldg4(wrow[i] + 8 * g + 4 * wh);
        }
#pragma unroll
        for (int i = 0; i < SQ; i++) {
            const int q = tid + T * i, g = min(ch * kLdsGK + q % kLdsGK, G - 1);
            R.s[i] = gld(srow[i] + g);
            R.b[i] = gld(brow[i] + g);
        }
    };
    auto store = [&](const Raw& R, int buf) {
#pragma unroll
        for (int i = 0; i < AQ; i++) {
            const int q = tid + T * i, row = q / (8 * kLdsGK), gg = (q / 8) % kLdsGK, wd = q % 8;
            As[buf][row * kRowStride + gg * 8 + wd] = R.a[i];
        }
        if (xload) {
            Xs[buf][xgg * BM + xr] = __uint_as_float(R.x.x);
            Xs[buf][xgg * BM + xr + 1] = __uint_as_float(R.x.y);
            Xs[buf][xgg * BM + xr + 2] = __uint_as_float(R.x.z);
            Xs[buf][xgg * BM + xr + 3] = __uint_as_float(R.x.w);
        }
#pragma unroll
        for (int i = 0; i < WQ; i++) {
            const int q = tid + T * i, col = q / 4, gg = (q / 2) % kLdsGK, wh = q % 2, w0 = gg * 8 + 4 * wh;
            Bp[buf][(w0 + 0) * BP + col] = R.w[i].x;
            Bp[buf][(w0 + 1) * BP + col] = R.w[i].y;
            Bp[buf][(w0 + 2) * BP + col] = R.w[i].z;
            Bp[buf][(w0 + 3) * BP + col] = R.w[i].w;
        }
#pragma unroll
        for (int i = 0; i < SQ; i++) {
            const int q = tid + T * i;
            const float sv = bf2f((uint16_t)R.s[i]), bv = bf2f((uint16_t)R.b[i]);
            Ss[buf][q] = make_float2(sv, fmaf(-128.0f, sv, bv));  // q = column * kLdsGK + group
        }
    };
    f32x4_t acc[MT][NW], run[MT][NW];
#pragma unroll
    for (int mt = 0; mt < MT; mt++)
#pragma unroll
        for (int t = 0; t < NW; t++) acc[mt][t] = run[mt][t] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
    const int gper = (G + kslices - 1) / kslices;
    auto chunk = [&](int ch, int buf) {
#pragma unroll
        for (int gg = 0; gg < kLdsGK; gg++) {
            const int g = ch * kLdsGK + gg;
            if (g >= G) break;
            AIn<MT> in;
#pragma unroll
            for (int mt = 0; mt < MT; mt++) {
                const int row = 16 * (wm * MT + mt);
                in.xa[mt][0] = As[buf][(row + c) * kRowStride + gg * 8 + 2 * j];
                in.xa[mt][1] = As[buf][(row + c) * kRowStride + gg * 8 + 2 * j + 1];
                in.xsv[mt] = *reinterpret_cast<const float4*>(&Xs[buf][gg * BM + row + 4 * j]);
            }
            uint32_t bw[NW][2];
            float sc[NW], off[NW];
#pragma unroll
            for (int t = 0; t < NW; t++) {
                const int col = 16 * (wn * NW + t) + c;
                bw[t][0] = Bp[buf][(gg * 8 + 2 * j) * BP + col];
                bw[t][1] = Bp[buf][(gg * 8 + 2 * j + 1) * BP + col];
                const float2 f = Ss[buf][col * kLdsGK + gg];
                sc[t] = f.x;
                off[t] = f.y;
            }
            group_mma_packed<MT, NW>(in, bw, sc, off, acc, mask, magic);
            if ((g + 1) % gper == 0 || g + 1 == G) {
#pragma unroll
                for (int mt = 0; mt < MT; mt++)
#pragma unroll
                    for (int t = 0; t < NW; t++) {
                        run[mt][t] = run[mt][t] + acc[mt][t];
                        acc[mt][t] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
                    }
            }
        }
    };
    Raw R0{}, R1{};
    fetch(0, R0);
    store(R0, 0);
    if (nch > 1) fetch(1, R1);
    if (nch > 2) fetch(2, R0);
    __syncthreads();
    for (int ch = 0; ch < nch; ch += 2) {
        chunk(ch, 0);
        if (ch + 1 < nch) store(R1, 1);
        __syncthreads();
        if (ch + 3 < nch) fetch(ch + 3, R1);
        if (ch + 1 >= nch) break;
        chunk(ch + 1, 1);
        if (ch + 2 < nch) store(R0, 0);
        __syncthreads();
        if (ch + 4 < nch) fetch(ch + 4, R0);
    }
    for (int sidx = (G + gper - 1) / gper; sidx < kslices; sidx++)
#pragma unroll
        for (int mt = 0; mt < MT; mt++)
#pragma unroll
            for (int t = 0; t < NW; t++) run[mt][t] = run[mt][t] + f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
    const QSeg& S = pick(a, si);
    const int nw0 = n0 + 16 * wn * TPS;
#pragma unroll
    for (int mt = 0; mt < MT; mt++)
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int m = r0 + 16 * (wm * MT + mt) + 4 * j + r;
            if (m >= a.M) continue;
            float v[NW];
#pragma unroll
            for (int t = 0; t < NW; t++) v[t] = run[mt][t][r];
            epi_row<MT, NW, EPI>(a, S, si, nw0, c, m, v);
        }
}

// kw_in > 0 sets the number of waves splitting K (at most KWMAX).
template <int MT, int NW, int GPW, int KWMAX, int EPI>
hipError_t launch_k(hipStream_t st, const QgemmArgs& a, int kw_in = 0) {
    const int grid = a.blocks[0] + (a.nseg > 1 ? a.blocks[1] : 0) + (a.nseg > 2 ? a.blocks[2] : 0);
    const int mtt = (a.M + 15) / 16, gy = mtt / MT;
    const int G = a.K / 64;
    const int kw = kw_in > 0 ? min(KWMAX, kw_in) : (GPW == 0 ? KWMAX : min(KWMAX, (G + GPW - 1) / GPW));
    const size_t lds = KWMAX > 1 ? sizeof(float) * (size_t)kw * MT * 4 * NW * kWave : 0;
    hipLaunchKernelGGL((qgemm_kernel<MT, NW, GPW, KWMAX, EPI>), dim3(grid, gy), dim3(64 * kw), lds, st, a);
    return hipGetLastError();
}

// ---- the wide head, at most 64 rows --------------------------------------------
// QE_PLAIN with N >= 16384 or argmax partials (the LM head) and M <= 64, for
// K = 896: each workgroup (one per CU, W waves) copies the staged
// activations of all rows into LDS once (rows padded to 9 uint4 so that a
// 16-lane b128 read hits 8 distinct 16-byte bank groups), then every wave
// streams units of 32 weight columns (2 column tiles x all MT row tiles), unit
// u = the wave's grid index + k x the grid's waves.  A wave's weights are read
// once from HBM and its A operands come from LDS, shared by its two column
// tiles.  A unit's 32 rows are consecutive, so its scales (and biases) are one
// contiguous run of 32 x 14 bf16: a wave loads the next unit's two runs with
// one 16-byte load a lane while the current unit runs, and writes them into
// its LDS block once the current unit's are read (two loads a unit instead of
// four 2-byte loads a group).  A wave's (unit, group) items run in order through a ring of R
// groups in registers: item i + R's load is issued as soon as item i's slot
// is read, unconditionally (past the end the last item is loaded again), and
// held there by a scheduling barrier, so R groups are in flight.  The wave
// index is read as a scalar, so the item loop's control is uniform (with a
// divergent loop the compiler waits for every load at each step).  Only two
// stores leave per unit when no logits are asked for (the argmax partials,
// one row slot per lane), so the wait counter's bound never forces a full
// wait.  Per row and column the arithmetic is group_mma's over the groups in
// order with one K slice, exactly as qgemm_kernel computes this shape, so the
// logits are the same bits; the argmax partials cover 32 columns each.
constexpr int kHeadNW = 2;     // column tiles per unit
constexpr int kHeadRow = 9;    // uint4 per staged row in LDS (8 + 1 of padding)

__host__ __device__ constexpr size_t head_lds_bytes(int G, int Mp) {
    return (size_t)G * Mp * kHeadRow * 16 + (size_t)G * Mp * 4;
}


// Maximum / minimum over the 16 lanes of a DPP row (the butterfly of team_reduce: every lane
// gets the result).
__device__ __forceinline__ float head_row_max(float v) {
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0xB1, 0xf, 0xf, true)));
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x4E, 0xf, 0xf, true)));
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x141, 0xf, 0xf, true)));
    return fmaxf(v, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x140, 0xf, 0xf, true)));
}

__device__ __forceinline__ int head_row_min(int v) {
    v = min(v, __builtin_amdgcn_mov_dpp(v, 0xB1, 0xf, 0xf, true));
    v = min(v, __builtin_amdgcn_mov_dpp(v, 0x4E, 0xf, 0xf, true));
    v = min(v, __builtin_amdgcn_mov_dpp(v, 0x141, 0xf, 0xf, true));
    return min(v, __builtin_amdgcn_mov_dpp(v, 0x140, 0xf, 0xf, true));
}

struct HeadGroup {
    uint2 wq[kHeadNW];
};

// A wave's scale/bias block in LDS: the bf16 scales of its unit's 32 rows x G groups, then the
// biases (rows of a unit are consecutive, so each block is one contiguous run of 64 G bytes).
template <int G>
__host__ __device__ constexpr int head_sb_bytes() { return 2 * 32 * G * 2; }

// OUT: the logits are written (a.y / a.yf); without, only the argmax partials leave the kernel.
// W waves per workgroup, R groups in flight per wave.
template <int MT, int G, bool OUT, int W, int R>
__global__ __launch_bounds__(64 * W) void qgemm_head_kernel(QgemmArgs a) {
    extern __shared__ uint4 hl[];  // As [G][Mp][kHeadRow] uint4, then Xs [G][Mp] f32
    constexpr int Mp = 16 * MT, KW8 = 8 * G;
    static_assert(R >= 2 && R <= 12, "ring slots named below");
    // the wave index as a scalar: the unit loop's bounds are then uniform, its branches scalar
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    const int lane = threadIdx.x % kWave, c = lane % 16, j = lane / 16;
    const QSeg& S = a.seg[0];
    const int N = S.N, units = (N + 16 * kHeadNW - 1) / (16 * kHeadNW);
    const int gw = blockIdx.x * W + wave, stride = gridDim.x * W;
    const int my_units = gw < units ? (units - gw + stride - 1) / stride : 0;
    const int items = my_units * G;  // (unit, group) pairs of this wave, unit-major
    // Item it's weights into a ring slot; past the last item the last one is loaded again (unused),
    // so that every load is unconditional and the ring's waits are static.
    auto load = [&](int it, HeadGroup& h) {
        it = min(it, items - 1);
        const int u = gw + (it / G) * stride, g = it % G;
        // a uniform base (the group) plus a 32-bit per-lane offset (the row)
        const char* wb = reinterpret_cast<const char*>(S.w) + 32 * g;
#pragma unroll
        for (int t = 0; t < kHeadNW; t++) {
            const uint32_t n = (uint32_t)min(16 * (kHeadNW * u + t) + c, N - 1);
            h.wq[t] = ldg2(wb + (n * (uint32_t)(4 * KW8) + 8u * j));
        }
    };
    // unit u's scale and bias blocks, 16 bytes a lane (lanes past the block load its last word)
    constexpr int kSbWords = 32 * G * 2 / 16;  // uint4 per block
    auto load_sb = [&](int u, uint4& vs, uint4& vb) {
        const size_t w0 = (size_t)u * kSbWords + min(lane, kSbWords - 1);
        vs = ldg4(reinterpret_cast<const uint4*>(S.s) + w0);
        vb = ldg4(reinterpret_cast<const uint4*>(S.b) + w0);
    };
    HeadGroup ring[R];
    if (items > 0) {
#pragma unroll
        for (int k = 0; k < R; k++) load(k, ring[k]);
    }
    uint4 nbs, nbb;  // the next unit's scale and bias blocks, in flight during a unit
    load_sb(min(gw, units - 1), nbs, nbb);
    // the staged activations of all rows into LDS
    uint4* As = hl;
    float* Xs = reinterpret_cast<float*>(hl + (size_t)G * Mp * kHeadRow);
    uint4* SB = reinterpret_cast<uint4*>(Xs + G * Mp) + wave * (2 * kSbWords);  // this wave's blocks
    const uint16_t* SBs = reinterpret_cast<const uint16_t*>(SB);
    const uint16_t* SBb = SBs + 32 * G;
    auto store_sb = [&]() {
        if (lane < kSbWords) {
            SB[lane] = nbs;
            SB[kSbWords + lane] = nbb;
        }
    };
    {
        const uint4* xs = static_cast<const uint4*>(a.xs);
        constexpr int total = G * Mp * 8, nsum = G * Mp, T = 64 * W, U = 8;
        const int t = threadIdx.x;
        float sv[(nsum + T - 1) / T];
#pragma unroll
        for (int k = 0; k < (nsum + T - 1) / T; k++)
            if (t + k * T < nsum) sv[k] = gld(a.xsum + t + k * T);
#pragma unroll 1
        for (int base = 0; base < total; base += U * T) {  // passes of U loads a thread, then U stores
            uint4 v[U];
#pragma unroll
            for (int k = 0; k < U; k++)
                if (base + t + k * T < total) v[k] = ldg4(xs + base + t + k * T);
#pragma unroll
            for (int k = 0; k < U; k++) {
                const int i = base + t + k * T;
                if (i < total) As[(i / 8) * kHeadRow + i % 8] = v[k];
            }
        }
#pragma unroll
        for (int k = 0; k < (nsum + T - 1) / T; k++)
            if (t + k * T < nsum) Xs[t + k * T] = sv[k];
    }
    store_sb();
    __syncthreads();
    if (items == 0) return;
    const uint32_t mask = in_reg(0x000f000fu), magic = in_reg(kQ4Magic);
    f32x4_t acc[MT][kHeadNW];
    // One item: group g of its unit from ring slot h, whose next item is loaded as soon as the slot
    // is read; the unit's epilogue after its last group.
    auto step = [&](int it, HeadGroup& h) __attribute__((always_inline)) {
        const int g = it % G;
        const int u = gw + (it / G) * stride;
        if (g == 0) {
#pragma unroll
            for (int mt = 0; mt < MT; mt++)
#pragma unroll
                for (int t = 0; t < kHeadNW; t++) acc[mt][t] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
            load_sb(u + stride < units ? u + stride : u, nbs, nbb);  // the next unit's blocks
        }
        bf16x8_t b[kHeadNW][2];
        float sc[kHeadNW], off[kHeadNW];
#pragma unroll
        for (int t = 0; t < kHeadNW; t++) {
            b[t][0] = unpack_b(h.wq[t].x, mask, magic);
            b[t][1] = unpack_b(h.wq[t].y, mask, magic);
            const int row = (16 * t + c) * G + g;
            sc[t] = bf2f(SBs[row]);
            off[t] = fmaf(-128.0f, sc[t], bf2f(SBb[row]));
        }
        load(it + R, h);
        // the loads stay here, R items ahead of their use (the scheduler would sink them to the use
        // to save registers, which serialises the ring); ALU, MFMA and LDS work may still cross
        __builtin_amdgcn_sched_barrier(0x38F);
        // row tile by row tile, tile mt + 1's MFMAs issued before tile mt is folded (group_mma's
        // arithmetic: two MFMAs from zero, then s * sum + (b - 128 s) * sum_k x_k)
        f32x4_t agA[kHeadNW], agB[kHeadNW];  // two row tiles' MFMA sums in flight (named: no indexing)
        struct AOp {
            bf16x8_t a0, a1;
            float4 xs;
        };
        // row tile mt's A operands and group sums from LDS
        auto read = [&](int mt, AOp& o) __attribute__((always_inline)) {
            const uint4* ar = As + (size_t)(g * Mp + 16 * mt + c) * kHeadRow + 2 * j;
            o.a0 = as_a(ar[0]);
            o.a1 = as_a(ar[1]);
            o.xs = *reinterpret_cast<const float4*>(Xs + g * Mp + 16 * mt + 4 * j);
        };
        auto mma = [&](const AOp& o, f32x4_t (&dst)[kHeadNW]) __attribute__((always_inline)) {
#pragma unroll
            for (int t = 0; t < kHeadNW; t++)
                dst[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(o.a0, b[t][0], f32x4_t{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
#pragma unroll
            for (int t = 0; t < kHeadNW; t++)
                dst[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(o.a1, b[t][1], dst[t], 0, 0, 0);
        };
        auto fold = [&](int mt, const f32x4_t (&src)[kHeadNW], const float4& xs4) __attribute__((always_inline)) {
            const float xv[4] = {xs4.x, xs4.y, xs4.z, xs4.w};
#pragma unroll
            for (int t = 0; t < kHeadNW; t++)
#pragma unroll
                for (int r = 0; r < 4; r++) acc[mt][t][r] = fmaf(off[t], xv[r], fmaf(sc[t], src[t][r], acc[mt][t][r]));
        };
        // tile mt + 1's LDS reads are issued before tile mt's fold, its MFMAs after it: the fold's
        // VALU work covers both the MFMA latency of tile mt and the LDS latency of tile mt + 1
        AOp oA, oB;
        read(0, oA);
        mma(oA, agA);
#pragma unroll
        for (int mt = 0; mt < MT; mt += 2) {
            if (mt + 1 < MT) read(mt + 1, oB);
            fold(mt, agA, oA.xs);
            if (mt + 1 < MT) {
                mma(oB, agB);
                if (mt + 2 < MT) read(mt + 2, oA);
                fold(mt + 1, agB, oB.xs);
                if (mt + 2 < MT) mma(oA, agA);
            }
        }
        if (g + 1 < G) return;
        // the unit's epilogue: g acc, the logits, one argmax partial per row.  Lane c of each
        // 16-lane group keeps the partial of row slot c (row 16 (c / 4) + 4 j + c % 4), so the
        // partials leave in one store per array: few stores keep the ring's waits exact (the
        // wait counter holds at most 63 outstanding operations).
        float keep_v = -INFINITY;
        int keep_i = 0x7fffffff;
#pragma unroll
        for (int mt = 0; mt < MT; mt++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int m = 16 * mt + 4 * j + r;
                // this lane's two columns (every column of a unit is < N): the larger, the lower
                // column on ties, -inf and NaN never chosen -- the sequential rule "v > best"
                float bv = -INFINITY;
                int bn = 0x7fffffff;
#pragma unroll
                for (int t = 0; t < kHeadNW; t++) {
                    const float v = acc[mt][t][r] * S.gscale;
                    const int n = 16 * (kHeadNW * u + t) + c;
                    if (OUT && m < a.M) {
                        const size_t o = (size_t)m * a.ldy + S.col0 + n;
                        if (a.y) gst(a.y + o, f2bf(v));
                        if (a.yf) gst(a.yf + o, v);
                    }
                    if (v > bv) {
                        bv = v;
                        bn = n;
                    }
                }
                // the 16 lanes of one j (one DPP row) hold one row: its maximum, then the lowest
                // column holding a value equal to it (-0 equals +0, as in the sequential rule);
                // a row of -inf / NaN keeps no column
                const float rm = head_row_max(bv);
                const int ri = head_row_min(bv == rm && rm > -INFINITY ? bn : 0x7fffffff);
                if (c == 4 * mt + r) {
                    keep_v = rm;
                    keep_i = ri;
                }
            }
        if (a.pmax && c < 4 * MT) {
            const int m = 16 * (c / 4) + 4 * j + c % 4;
            if (m < a.M) {
                gst(a.pmax + (size_t)m * a.nblk + u, keep_v);
                gst(a.pidx + (size_t)m * a.nblk + u, keep_i);
            }
        }
        store_sb();  // this unit's scales are read: the next unit's blocks take their place
    };
    for (int it = 0; it < items; it += R) {  // slots named one by one: the ring must not be indexed
#define MING_HEAD_STEP(K)                     \
    if (K < R) {                              \
        if (it + K >= items) break;           \
        step(it + K, ring[K % R]);            \
    }
        MING_HEAD_STEP(0) MING_HEAD_STEP(1) MING_HEAD_STEP(2) MING_HEAD_STEP(3)
        MING_HEAD_STEP(4) MING_HEAD_STEP(5) MING_HEAD_STEP(6) MING_HEAD_STEP(7)
        MING_HEAD_STEP(8) MING_HEAD_STEP(9) MING_HEAD_STEP(10) MING_HEAD_STEP(11)
#undef MING_HEAD_STEP
    }
}

int head_grid() {
    static int cus[64] = {0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    if (!cus[dev]) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
        cus[dev] = n;
    }
    return cus[dev];
}

// K = 896 (14 groups), whole units of 32 rows, scale and bias blocks 16-byte aligned
bool head_fits(const QgemmArgs& a) {
    return a.nseg == 1 && a.M <= 64 && a.K == 896 && a.seg[0].N % 32 == 0 &&
           reinterpret_cast<uintptr_t>(a.seg[0].s) % 16 == 0 && reinterpret_cast<uintptr_t>(a.seg[0].b) % 16 == 0;
}

template <int MT, int G, bool OUT, int W, int R>
hipError_t launch_head_g(hipStream_t st, QgemmArgs a) {
    constexpr size_t lds = head_lds_bytes(G, 16 * MT) + (size_t)W * head_sb_bytes<G>();
    static_assert(lds <= 160 * 1024, "staged rows and scale blocks fit in LDS");
    const int units = (a.seg[0].N + 16 * kHeadNW - 1) / (16 * kHeadNW);
    a.nblk = units;
    static bool raised[64] = {false};  // the kernel's LDS limit, raised once per device
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return hipErrorInvalidDevice;
    if (!raised[dev]) {
        const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&qgemm_head_kernel<MT, G, OUT, W, R>),
                                                 hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) return e;
        raised[dev] = true;
    }
    const int grid = min(head_grid(), (units + W - 1) / W);
    hipLaunchKernelGGL((qgemm_head_kernel<MT, G, OUT, W, R>), dim3(grid), dim3(64 * W), lds, st, a);
    return hipGetLastError();
}

template <int G, bool OUT>
hipError_t launch_head_k(hipStream_t st, const QgemmArgs& a) {
    const int mt = (a.M + 15) / 16;
    if (mt == 1) return launch_head_g<1, G, OUT, 8, 6>(st, a);
    if (mt == 2) return launch_head_g<2, G, OUT, 8, 6>(st, a);
    if (mt == 3) return launch_head_g<3, G, OUT, 8, 6>(st, a);
    // four row tiles (N = 151936, K = 896, 64 rows): 12 waves (3 a SIMD) with 4 groups in flight
    // each 42.6 us; 12 x 6 42.5, 8 x 6 45.2, 16 x 4 and 16 x 3 50.3-50.4 (more waves are slower)
    return launch_head_g<4, G, OUT, 12, 4>(st, a);
}

hipError_t launch_head(hipStream_t st, const QgemmArgs& a) {
    return a.y || a.yf ? launch_head_k<14, true>(st, a) : launch_head_k<14, false>(st, a);
}

// row tiles per workgroup: 2 when MTMAX allows and the row-tile count is even, else 1
template <int NW, int GPW, int KWMAX, int EPI, int MTMAX>
hipError_t launch_mt(hipStream_t st, const QgemmArgs& a) {
    const int mtt = (a.M + 15) / 16;
    if constexpr (MTMAX >= 2)
        if (mtt % 2 == 0) return launch_k<2, NW, GPW, KWMAX, EPI>(st, a);
    return launch_k<1, NW, GPW, KWMAX, EPI>(st, a);
}

// More than 64 rows: qgemm_lds_kernel with the K slices of the shape's launch for
// <= 64 rows (GPW, KWMAX as there); WM x WN waves of MT x NW tiles.
template <int WM, int WN, int MT, int NW, int GPW, int KWMAX, int EPI>
hipError_t launch_big(hipStream_t st, QgemmArgs a) {
    constexpr int TPS = EPI == QE_SWIGLU ? NW / 2 : NW, CB = 16 * TPS * WN, BM = 16 * WM * MT;
    const int G = a.K / 64, kw = GPW == 0 ? KWMAX : min(KWMAX, (G + GPW - 1) / GPW);
    for (int i = 0; i < 3; i++) a.blocks[i] = i < a.nseg ? (a.seg[i].N + CB - 1) / CB : 0;
    if (EPI == QE_SWIGLU) a.blocks[1] = 0;
    for (int i = 0; i < a.nseg; i++)  // a tile never straddles two segments
        if (EPI != QE_SWIGLU && a.nseg > 1 && a.seg[i].N % CB) return hipErrorInvalidValue;
    const int grid = a.blocks[0] + a.blocks[1] + a.blocks[2];
    const int mtt = (a.M + 15) / 16, gy = (16 * mtt + BM - 1) / BM;
    hipLaunchKernelGGL((qgemm_lds_kernel<WM, WN, MT, NW, EPI>), dim3(grid, gy), dim3(256), 0, st, a, kw);
    return hipGetLastError();
}

// More than 64 rows on qgemm_wide_kernel (same K slices as launch_big); false
// when the shape does not tile: the caller takes launch_big.
bool qgemm_wide_enabled() {
    static const bool v = [] {
        const char* e = std::getenv("MING_QGEMM_WIDE");
        return !(e && e[0] == '0' && e[1] == '\0');
    }();
    return v;
}

template <int WM, int WN, int MT, int NW, int GPW, int KWMAX, int EPI>
bool launch_wide(hipStream_t st, QgemmArgs a, hipError_t& err) {
    constexpr int TPS = EPI == QE_SWIGLU ? NW / 2 : NW, CB = 16 * TPS * WN, BM = 16 * WM * MT;
    if (!qgemm_wide_enabled()) return false;
    for (int i = 0; i < a.nseg; i++)
        if (a.seg[i].N % CB) return false;
    const int G = a.K / 64, kw = GPW == 0 ? KWMAX : min(KWMAX, (G + GPW - 1) / GPW);
    for (int i = 0; i < 3; i++) a.blocks[i] = i < a.nseg ? a.seg[i].N / CB : 0;
    if (EPI == QE_SWIGLU) a.blocks[1] = 0;
    const int grid = a.blocks[0] + a.blocks[1] + a.blocks[2];
    const int mtt = (a.M + 15) / 16, gy = (16 * mtt + BM - 1) / BM;
    hipLaunchKernelGGL((qgemm_wide_kernel<WM, WN, MT, NW, EPI>), dim3(grid, gy), dim3(64 * WM * WN), 0, st, a, kw);
    err = hipGetLastError();
    return true;
}

}  // namespace

// a.blocks is filled here.  Shapes: the LM head 4 column tiles x 2 row tiles
// per wave, one wave per workgroup streaming all of K through the register
// ring; gate/up 2 + 2 column tiles x 2 row tiles, two waves splitting K; q/k/v
// one head (4 tiles) x 1 row tile, K in chunks of 2 groups over up to 8
// waves; the narrow o/down projections 1 x 1, K in chunks of 5 groups over up
// to 16 waves, so that they still spread over the CUs.  (Four row tiles per
// wave would keep the accumulators in AGPRs.)  More than 64 rows: LDS-tiled
// 64 x 64 tiles, except the narrow o/down projections (residual epilogue),
// whose 32 x 32 tiles (one 16 x 16 tile per wave) give a 512-row chunk 448
// workgroups at N = 896 instead of 112 (512-token prefill 3.58 -> 3.20 ms;
// 64 x 32, 32 x 64, 64 x 16 and 16 x 64 tiles measured 3.24-3.35 ms).
hipError_t launch_qgemm_epi(hipStream_t st, QgemmArgs a, int epi) {
    if (a.M < 1 || a.M > kQgemmMaxRows || a.K % 64 || a.nseg < 1 || a.nseg > 3) return hipErrorInvalidValue;
    const bool big = a.M > 64;
    auto set_blocks = [&a](int cols) {
        for (int i = 0; i < 3; i++) a.blocks[i] = i < a.nseg ? (a.seg[i].N + cols - 1) / cols : 0;
    };
    switch (epi) {
        case QE_PLAIN:
            if (a.nseg == 1 && (a.seg[0].N >= 16384 || a.pmax)) {
                if (head_fits(a)) return launch_head(st, a);  // argmax partials: blocks of 32 columns
                set_blocks(64);                               // argmax partials: blocks of 64 columns
                a.nblk = a.blocks[0];
                return launch_mt<4, 0, 1, QE_PLAIN, 2>(st, a);
            }
            if (a.pmax) return hipErrorInvalidValue;
            set_blocks(16);
            return big ? launch_big<2, 2, 2, 2, 5, 16, QE_PLAIN>(st, a) : launch_mt<1, 5, 16, QE_PLAIN, 1>(st, a);
        case QE_RES:
            set_blocks(16);
            return big ? launch_big<2, 2, 1, 1, 5, 16, QE_RES>(st, a) : launch_mt<1, 5, 16, QE_RES, 1>(st, a);
        case QE_SWIGLU:
            if (a.nseg != 2 || a.seg[0].N != a.seg[1].N) return hipErrorInvalidValue;
            set_blocks(32);
            a.blocks[1] = 0;
            if (big) {
                hipError_t e;
                if (launch_wide<2, 4, 2, 4, 0, 2, QE_SWIGLU>(st, a, e)) return e;
                return launch_big<2, 2, 2, 2, 0, 2, QE_SWIGLU>(st, a);
            }
            return launch_mt<4, 0, 2, QE_SWIGLU, 2>(st, a);
        case QE_QKV:
            if (a.nseg != 3) return hipErrorInvalidValue;
            for (int i = 0; i < 3; i++)
                if (a.seg[i].N % 64) return hipErrorInvalidValue;
            set_blocks(64);
            return big ? launch_big<4, 1, 1, 4, 2, 8, QE_QKV>(st, a) : launch_mt<4, 2, 8, QE_QKV, 1>(st, a);
        default:
            return hipErrorInvalidValue;
    }
}

// Final argmax over the head GEMM's per-workgroup partials: one workgroup per row.
__global__ __launch_bounds__(256) void argmax_partials_kernel(const float* __restrict__ pmax,
                                                              const int32_t* __restrict__ pidx, int nblk,
                                                              int32_t* __restrict__ out) {
    __shared__ float bv[4];
    __shared__ int bi[4];
    const float* pm = pmax + (size_t)blockIdx.x * nblk;
    const int32_t* pi = pidx + (size_t)blockIdx.x * nblk;
    float best = -INFINITY;
    int idx = 0x7fffffff;
    for (int i = threadIdx.x; i < nblk; i += 256) {
        const float v = gld(pm + i);
        const int k = gld(pi + i);
        if (v > best || (v == best && k < idx)) {
            best = v;
            idx = k;
        }
    }
#pragma unroll
    for (int d = 32; d >= 1; d >>= 1) {
        const float ov = __shfl_xor(best, d);
        const int oi = __shfl_xor(idx, d);
        if (ov > best || (ov == best && oi < idx)) {
            best = ov;
            idx = oi;
        }
    }
    const int wave = threadIdx.x / kWave;
    if (threadIdx.x % kWave == 0) {
        bv[wave] = best;
        bi[wave] = idx;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < 4; w++)
            if (bv[w] > best || (bv[w] == best && bi[w] < idx)) {
                best = bv[w];
                idx = bi[w];
            }
        gst(out + blockIdx.x, idx == 0x7fffffff ? 0 : idx);
    }
}

int qgemm_argmax_blocks(int M, int K, int N) {
    QgemmArgs a{};
    a.M = M;
    a.K = K;
    a.nseg = 1;
    return head_fits(a) ? (N + 16 * kHeadNW - 1) / (16 * kHeadNW) : (N + 63) / 64;
}

hipError_t launch_argmax_partials(hipStream_t st, const float* pmax, const int32_t* pidx, int nblk, int n,
                                  int32_t* out) {
    hipLaunchKernelGGL(argmax_partials_kernel, dim3(n), dim3(256), 0, st, pmax, pidx, nblk, out);
    return hipGetLastError();
}

}  // namespace ming
