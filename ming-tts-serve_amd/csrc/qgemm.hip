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
// Workgroup: KW waves split the groups of K; each wave accumulates MT x 16
// rows by NW x 16 columns, keeping the next group's loads in flight while the
// current group's MFMAs run; the waves' partial sums are added through LDS and
// the first wave applies the epilogue (QEpi).  One call may concatenate up to
// three matrices along N (q/k/v; gate/up), each a run of workgroups.
#include "batch.h"
#include "common.h"
#include "internal.h"

namespace ming {

namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ uint2 ldg2(const void* p) {
    const u32x2_t v = *(const MING_GLOBAL u32x2_t*)p;
    return make_uint2(v.x, v.y);
}

// bf16 pairs (128 + q_i, 128 + q_{i+4}) of one packed word, as the 8-value B operand.
__device__ __forceinline__ bf16x8_t unpack_b(uint32_t w) {
    return __builtin_bit_cast(bf16x8_t, u32x4_t{(w & 0x000f000fu) | kQ4Magic, ((w >> 4) & 0x000f000fu) | kQ4Magic,
                                                ((w >> 8) & 0x000f000fu) | kQ4Magic,
                                                ((w >> 12) & 0x000f000fu) | kQ4Magic});
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
    uint4 xa[MT][2];    // A operand words 2j, 2j+1 of row 16mt + c
    float xsv[MT][4];   // group sums of rows 16mt + 4j + r
};

template <int MT, int NW>
struct Rows {
    const uint32_t* w[NW];
    const uint16_t* s[NW];
    const uint16_t* b[NW];
};

template <int MT, int NW>
__device__ __forceinline__ void group_load(const QgemmArgs& a, const Rows<MT, NW>& R, int g, int c, int j,
                                           GroupIn<MT, NW>& in) {
    const int G = a.K / 64, KW8 = a.K / 8;
    const uint4* xs = static_cast<const uint4*>(a.xs);
#pragma unroll
    for (int t = 0; t < NW; t++) {
        in.wq[t] = ldg2(R.w[t] + 8 * g + 2 * j);
        in.sc[t] = bf2f(gld(R.s[t] + g));
        in.bi[t] = bf2f(gld(R.b[t] + g));
    }
#pragma unroll
    for (int mt = 0; mt < MT; mt++) {
        const uint4* xp = xs + (size_t)(16 * mt + c) * KW8 + 8 * g + 2 * j;
        in.xa[mt][0] = ldg4(xp);
        in.xa[mt][1] = ldg4(xp + 1);
#pragma unroll
        for (int r = 0; r < 4; r++) in.xsv[mt][r] = gld(a.xsum + (size_t)(16 * mt + 4 * j + r) * G + g);
    }
}

template <int MT, int NW>
__device__ __forceinline__ void group_mma(const GroupIn<MT, NW>& in, f32x4_t (&acc)[MT][NW]) {
#pragma unroll
    for (int t = 0; t < NW; t++) {
        const bf16x8_t b0 = unpack_b(in.wq[t].x), b1 = unpack_b(in.wq[t].y);
        const float s = in.sc[t], off = in.bi[t] - 128.0f * in.sc[t];
#pragma unroll
        for (int mt = 0; mt < MT; mt++) {
            f32x4_t ag = {0.0f, 0.0f, 0.0f, 0.0f};
            ag = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_a(in.xa[mt][0]), b0, ag, 0, 0, 0);
            ag = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_a(in.xa[mt][1]), b1, ag, 0, 0, 0);
#pragma unroll
            for (int r = 0; r < 4; r++) acc[mt][t][r] += s * ag[r] + off * in.xsv[mt][r];
        }
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

template <int MT, int NW, int KW, int EPI>
__global__ __launch_bounds__(64 * KW) void qgemm_kernel(QgemmArgs a) {
    extern __shared__ float red[];  // [KW - 1][MT][NW][4][64]
    constexpr int TPS = EPI == QE_SWIGLU ? NW / 2 : NW;  // column tiles per segment and workgroup
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
    const int G = a.K / 64, KW8 = a.K / 8;
    Rows<MT, NW> R;
#pragma unroll
    for (int t = 0; t < NW; t++) {
        const QSeg& S = pick(a, EPI == QE_SWIGLU ? (t < TPS ? 0 : 1) : si);
        const int n = min(n0 + 16 * (t % TPS) + c, S.N - 1);
        R.w[t] = S.w + (size_t)n * KW8;
        R.s[t] = S.s + (size_t)n * G;
        R.b[t] = S.b + (size_t)n * G;
    }
    const int gper = (G + KW - 1) / KW, g0 = wave * gper, g1 = min(G, g0 + gper);
    f32x4_t acc[MT][NW];
#pragma unroll
    for (int mt = 0; mt < MT; mt++)
#pragma unroll
        for (int t = 0; t < NW; t++) acc[mt][t] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
    if (g0 < g1) {
        GroupIn<MT, NW> cur, nxt;
        group_load<MT, NW>(a, R, g0, c, j, cur);
        for (int g = g0; g < g1; g++) {
            if (g + 1 < g1) group_load<MT, NW>(a, R, g + 1, c, j, nxt);
            group_mma<MT, NW>(cur, acc);
            if (g + 1 < g1) cur = nxt;
        }
    }
    if (KW > 1) {
        if (wave > 0)
#pragma unroll
            for (int mt = 0; mt < MT; mt++)
#pragma unroll
                for (int t = 0; t < NW; t++)
#pragma unroll
                    for (int r = 0; r < 4; r++)
                        red[((((wave - 1) * MT + mt) * NW + t) * 4 + r) * kWave + lane] = acc[mt][t][r];
        __syncthreads();
        if (wave > 0) return;
#pragma unroll
        for (int mt = 0; mt < MT; mt++)
#pragma unroll
            for (int t = 0; t < NW; t++)
#pragma unroll
                for (int r = 0; r < 4; r++)
                    for (int w = 1; w < KW; w++) acc[mt][t][r] += red[((((w - 1) * MT + mt) * NW + t) * 4 + r) * kWave + lane];
    }
    const QSeg& S = pick(a, si);
#pragma unroll
    for (int mt = 0; mt < MT; mt++)
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int m = 16 * mt + 4 * j + r;
            if (m >= a.M) continue;
            if constexpr (EPI == QE_QKV) {
                float v[NW];
#pragma unroll
                for (int t = 0; t < NW; t++) v[t] = acc[mt][t][r];
                qkv_row<MT, NW>(a, S, si, n0, c, m, v);
            } else if constexpr (EPI == QE_SWIGLU) {
                const float gg = a.seg[0].gscale, gu = a.seg[1].gscale;
#pragma unroll
                for (int t = 0; t < TPS; t++) {
                    const int n = n0 + 16 * t + c;
                    if (n >= S.N) continue;
                    const float gv = rb(acc[mt][t][r] * gg), u = rb(acc[mt][t + TPS][r] * gu);
                    const float sg = rb(1.0f / (1.0f + expf(-gv)));
                    gst(a.y + (size_t)m * a.ldy + n, f2bf(rb(gv * sg) * u));
                }
            } else {
#pragma unroll
                for (int t = 0; t < NW; t++) {
                    const int n = n0 + 16 * t + c;
                    if (n >= S.N) continue;
                    const float v = acc[mt][t][r] * S.gscale;
                    const size_t o = (size_t)m * a.ldy + S.col0 + n;
                    if constexpr (EPI == QE_RES) {
                        gst(a.y + o, f2bf(bf2f(gld(a.res + (size_t)m * a.ldres + S.col0 + n)) + rb(v)));
                    } else {
                        if (a.y) gst(a.y + o, f2bf(v));
                        if (a.yf) gst(a.yf + o, v);
                    }
                }
            }
        }
}

template <int MT, int NW, int KW, int EPI>
hipError_t launch_k(hipStream_t st, const QgemmArgs& a) {
    const int grid = a.blocks[0] + (a.nseg > 1 ? a.blocks[1] : 0) + (a.nseg > 2 ? a.blocks[2] : 0);
    const size_t lds = sizeof(float) * (size_t)(KW - 1) * MT * NW * 4 * kWave;
    hipLaunchKernelGGL((qgemm_kernel<MT, NW, KW, EPI>), dim3(grid), dim3(64 * KW), lds, st, a);
    return hipGetLastError();
}

template <int NW, int EPI>
hipError_t launch_mt(hipStream_t st, const QgemmArgs& a) {
    switch ((a.M + 15) / 16) {
        case 1: return launch_k<1, NW, 4, EPI>(st, a);
        case 2: return launch_k<2, NW, 4, EPI>(st, a);
        case 3: return launch_k<3, NW, 4, EPI>(st, a);
        case 4: return launch_k<4, NW, 4, EPI>(st, a);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace

// a.blocks is filled here: wide matrices (plain epilogue, N >= 16384) take 4
// column tiles per wave, narrow ones 1 so that they still spread over the CUs;
// q/k/v take one head (4 tiles) per workgroup, gate/up 2 + 2 tiles.
hipError_t launch_qgemm_epi(hipStream_t st, QgemmArgs a, int epi) {
    if (a.M < 1 || a.M > 64 || a.K % 64 || a.nseg < 1 || a.nseg > 3) return hipErrorInvalidValue;
    auto set_blocks = [&a](int cols) {
        for (int i = 0; i < 3; i++) a.blocks[i] = i < a.nseg ? (a.seg[i].N + cols - 1) / cols : 0;
    };
    switch (epi) {
        case QE_PLAIN:
            if (a.nseg == 1 && a.seg[0].N >= 16384) {
                set_blocks(64);
                return launch_mt<4, QE_PLAIN>(st, a);
            }
            set_blocks(16);
            return launch_mt<1, QE_PLAIN>(st, a);
        case QE_RES:
            set_blocks(16);
            return launch_mt<1, QE_RES>(st, a);
        case QE_SWIGLU:
            if (a.nseg != 2 || a.seg[0].N != a.seg[1].N) return hipErrorInvalidValue;
            set_blocks(32);
            a.blocks[1] = 0;
            return launch_mt<4, QE_SWIGLU>(st, a);
        case QE_QKV:
            if (a.nseg != 3) return hipErrorInvalidValue;
            for (int i = 0; i < 3; i++)
                if (a.seg[i].N % 64) return hipErrorInvalidValue;
            set_blocks(64);
            return launch_mt<4, QE_QKV>(st, a);
        default:
            return hipErrorInvalidValue;
    }
}

}  // namespace ming
