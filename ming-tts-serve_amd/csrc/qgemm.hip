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
// activations are staged once per call (qgemm_stage_kernel) in the MFMA A
// operand's layout: 16-byte words of 8 values in nibble-pair order (x0,x4),
// (x1,x5), (x2,x6), (x3,x7), matching the unpacked weight word, plus the f32
// group sums.
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
// current group's MFMAs run; the waves' partial sums are added through LDS.
#include "common.h"
#include "internal.h"

namespace ming {

namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

struct QgemmArgs {
    const uint4* xs;       // [Mp][K/8] staged activations
    const float* xsum;     // [Mp][K/64]
    int M, Mp, N, K;
    const uint32_t* w;     // [N][K/8]
    const uint16_t* s;     // [N][K/64]
    const uint16_t* b;
    float gscale;
    uint16_t* y;           // [M][N] bf16, or null
    float* yf;             // [M][N] f32, or null
};

__global__ __launch_bounds__(256) void qgemm_stage_kernel(const uint16_t* __restrict__ x, int M, int Mp, int K,
                                                          uint4* __restrict__ xs, float* __restrict__ xsum) {
    // one thread per (row, group of 64): 8 words in pair order and the group's sum
    const int G = K / 64;
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i >= Mp * G) return;
    const int m = i / G, g = i % G;
    float sum = 0.0f;
#pragma unroll
    for (int wd = 0; wd < 8; wd++) {
        uint4 v = make_uint4(0, 0, 0, 0);
        if (m < M) v = ldg4(x + (size_t)m * K + 64 * g + 8 * wd);
        const uint32_t e[4] = {v.x, v.y, v.z, v.w};  // (x0,x1) (x2,x3) (x4,x5) (x6,x7)
        float f[8];
#pragma unroll
        for (int p = 0; p < 4; p++) {
            f[2 * p] = bf_lo(e[p]);
            f[2 * p + 1] = bf_hi(e[p]);
        }
#pragma unroll
        for (int q = 0; q < 8; q++) sum += f[q];
        const uint4 o = make_uint4((e[0] & 0xffffu) | (e[2] << 16), (e[0] >> 16) | (e[2] & 0xffff0000u),
                                   (e[1] & 0xffffu) | (e[3] << 16), (e[1] >> 16) | (e[3] & 0xffff0000u));
        gst(xs + (size_t)m * (K / 8) + 8 * g + wd, o);
    }
    gst(xsum + (size_t)m * G + g, sum);
}

// bf16 pairs (128 + q_i, 128 + q_{i+4}) of one packed word, as the 8-value B operand.
__device__ __forceinline__ bf16x8_t unpack_b(uint32_t w) {
    const uint32_t p[4] = {(w & 0x000f000fu) | kQ4Magic, ((w >> 4) & 0x000f000fu) | kQ4Magic,
                           ((w >> 8) & 0x000f000fu) | kQ4Magic, ((w >> 12) & 0x000f000fu) | kQ4Magic};
    typedef uint32_t u32x4v __attribute__((ext_vector_type(4)));
    return __builtin_bit_cast(bf16x8_t, u32x4v{p[0], p[1], p[2], p[3]});
}

__device__ __forceinline__ bf16x8_t as_a(uint4 v) {
    typedef uint32_t u32x4v __attribute__((ext_vector_type(4)));
    return __builtin_bit_cast(bf16x8_t, u32x4v{v.x, v.y, v.z, v.w});
}

// One group's operands of one lane.
template <int MT, int NW>
struct GroupIn {
    uint2 wq[NW];       // words 2j, 2j+1 of the group, row n0 + 16t + c
    float sc[NW], bi[NW];
    uint4 xa[MT][2];    // A operand words 2j, 2j+1 of row 16mt + c
    float xsv[MT][4];   // group sums of rows 16mt + 4j + r
};

template <int MT, int NW>
__device__ __forceinline__ void group_load(const QgemmArgs& a, int n0, int g, int c, int j, GroupIn<MT, NW>& in) {
    const int G = a.K / 64, KW8 = a.K / 8;
#pragma unroll
    for (int t = 0; t < NW; t++) {
        const int n = min(n0 + 16 * t + c, a.N - 1);
        const uint32_t* wp = a.w + (size_t)n * KW8 + 8 * g + 2 * j;
        const uint32_t lo = gld(wp), hi = gld(wp + 1);
        in.wq[t] = make_uint2(lo, hi);
        in.sc[t] = bf2f(gld(a.s + (size_t)n * G + g));
        in.bi[t] = bf2f(gld(a.b + (size_t)n * G + g));
    }
#pragma unroll
    for (int mt = 0; mt < MT; mt++) {
        const uint4* xp = a.xs + (size_t)(16 * mt + c) * KW8 + 8 * g + 2 * j;
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

template <int MT, int NW, int KW>
__global__ __launch_bounds__(64 * KW) void qgemm_kernel(QgemmArgs a) {
    extern __shared__ float red[];  // [KW - 1][MT][NW][4][64]
    const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave, c = lane % 16, j = lane / 16;
    const int n0 = blockIdx.x * 16 * NW;
    const int G = a.K / 64, gper = (G + KW - 1) / KW, g0 = wave * gper, g1 = min(G, g0 + gper);
    f32x4_t acc[MT][NW];
#pragma unroll
    for (int mt = 0; mt < MT; mt++)
#pragma unroll
        for (int t = 0; t < NW; t++) acc[mt][t] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
    if (g0 < g1) {
        GroupIn<MT, NW> cur, nxt;
        group_load<MT, NW>(a, n0, g0, c, j, cur);
        for (int g = g0; g < g1; g++) {
            if (g + 1 < g1) group_load<MT, NW>(a, n0, g + 1, c, j, nxt);
            group_mma<MT, NW>(cur, acc);
            if (g + 1 < g1) cur = nxt;
        }
    }
    // the waves' partial sums, in wave order
    if (wave > 0)
#pragma unroll
        for (int mt = 0; mt < MT; mt++)
#pragma unroll
            for (int t = 0; t < NW; t++)
#pragma unroll
                for (int r = 0; r < 4; r++) red[((((wave - 1) * MT + mt) * NW + t) * 4 + r) * kWave + lane] = acc[mt][t][r];
    __syncthreads();
    if (wave > 0) return;
#pragma unroll
    for (int mt = 0; mt < MT; mt++)
#pragma unroll
        for (int t = 0; t < NW; t++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                float v = acc[mt][t][r];
                for (int w = 1; w < KW; w++) v += red[((((w - 1) * MT + mt) * NW + t) * 4 + r) * kWave + lane];
                const int m = 16 * mt + 4 * j + r, n = n0 + 16 * t + c;
                if (m < a.M && n < a.N) {
                    const float y = v * a.gscale;
                    if (a.y) gst(a.y + (size_t)m * a.N + n, f2bf(y));
                    if (a.yf) gst(a.yf + (size_t)m * a.N + n, y);
                }
            }
}

template <int MT, int NW, int KW>
hipError_t launch_mt(hipStream_t st, const QgemmArgs& a) {
    const int grid = (a.N + 16 * NW - 1) / (16 * NW);
    const size_t lds = sizeof(float) * (size_t)(KW - 1) * MT * NW * 4 * kWave;
    hipLaunchKernelGGL((qgemm_kernel<MT, NW, KW>), dim3(grid), dim3(64 * KW), lds, st, a);
    return hipGetLastError();
}

}  // namespace

// Staging of X [M][K] (bf16, K % 64 == 0) into xs [Mp][K/8] and xsum [Mp][K/64]
// (Mp = M rounded up to 16; rows past M are zero).
hipError_t launch_qgemm_stage(hipStream_t st, const uint16_t* x, int M, int K, uint4* xs, float* xsum) {
    const int Mp = (M + 15) / 16 * 16, n = Mp * (K / 64);
    hipLaunchKernelGGL(qgemm_stage_kernel, dim3((n + 255) / 256), dim3(256), 0, st, x, M, Mp, K, xs, xsum);
    return hipGetLastError();
}

// Y = g * X W^T from staged X; M <= 64.  Wide N: 4 column tiles per wave;
// narrow N: 1, so that small matrices still spread over the CUs.
hipError_t launch_qgemm(hipStream_t st, const uint4* xs, const float* xsum, int M, int N, int K, const uint32_t* w,
                        const uint16_t* s, const uint16_t* b, float gscale, uint16_t* y, float* yf) {
    QgemmArgs a{xs, xsum, M, (M + 15) / 16 * 16, N, K, w, s, b, gscale, y, yf};
    const int mt = (M + 15) / 16;
    const bool wide = N >= 64 * 256;
#define MING_QG(MT)                                                                                   \
    case MT:                                                                                          \
        return wide ? launch_mt<MT, 4, 4>(st, a) : launch_mt<MT, 1, 4>(st, a);
    switch (mt) {
        MING_QG(1)
        MING_QG(2)
        MING_QG(3)
        MING_QG(4)
        default:
            return hipErrorInvalidValue;
    }
#undef MING_QG
}

}  // namespace ming
