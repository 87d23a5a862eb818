// The flow head for many sequences at once (config 5's DiT head per step):
// cfmSample (src/ming_model.zig:1143-1151, :1161-1203) over R = 6 n rows
// (n sequences x 2 CFG halves x 3 positions), every DiT linear one bf16 GEMM
// on the matrix cores.  Per sequence the arithmetic is the fused DiT path's
// (src/ming_fused.zig:145-289): bias adds rounded once with the product
// (addmm), residuals rounded, gelu with every op rounded, interleaved rotary
// as four f32 products, CFG + Euler (+ SDE) with every op rounded.
//
// GEMM: Y [R][N] = X [R][K] W^T, bf16 in, f32 accumulate.  MFMA 16x16x32 bf16
// lane layout (gfx950): A lane l = row l % 16, k-block l / 16 (8 values); B
// lane l = column l % 16, same k-block; C[r] = (row 4 (l / 16) + r, column
// l % 16).  A rows and W rows are both K-contiguous, so each lane loads 16
// contiguous bytes per operand per MFMA.  Workgroup (column block x, row-tile
// group y): KW <= 4 waves split K; a wave holds MT row tiles x NW column tiles;
// two groups of 64 k in flight while one computes; partial sums meet in LDS.
#include "args.h"
#include "common.h"
#include "internal.h"

namespace ming {

namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

enum DEpi : int { DE_BIAS = 0, DE_RES = 1, DE_GELU = 2, DE_QKV = 3, DE_CFM = 4 };

struct DGemm {
    const uint16_t* x;     // A rows [R][ldx]
    int ldx, R, N, K;
    const uint16_t* w[3];  // [N][K] (DE_QKV: q, k, v of N / 3 rows each)
    const uint16_t* b[3];
    uint16_t* out;         // [R][ldo] (DE_QKV: [3][R][N / 3])
    int ldo;
    const uint16_t* res;   // DE_RES: [R][ldo]
    // DE_QKV
    const float *cos_t, *sin_t;
    int L, hd;
    // DE_CFM: rows 2b (cond) and 2b + 1 (uncond) of sequence b
    const uint16_t *y, *dt, *sq, *sde;  // y [n][N], sde [n][steps][N]
    int step, steps;
    float cfg, shift;
    uint16_t* y_out;       // [n][N]
    uint16_t* y_steps;     // optional [n][steps][N]
};

__device__ __forceinline__ bf16x8_t as8(uint4 v) { return __builtin_bit_cast(bf16x8_t, u32x4_t{v.x, v.y, v.z, v.w}); }

__device__ __forceinline__ float gelu_chain_b(float x) {
    const float c0 = rb(0.044715f), c1 = rb(0.7978845608f);
    const float x3 = rb((float)((double)x * (double)x * (double)x));
    const float inner = rb(x + rb(c0 * x3));
    const float th = rb(tanhf(rb(c1 * inner)));
    return rb(rb(0.5f * x) * rb(1.0f + th));
}

template <int MT, int NW>
struct DIn {
    uint4 a[MT][2], b[NW][2];
};

template <int MT, int NW>
__device__ __forceinline__ void dload(const uint16_t* const (&xr)[MT], const uint16_t* const (&wr)[NW], int g,
                                      DIn<MT, NW>& in) {
#pragma unroll
    for (int mt = 0; mt < MT; mt++) {
        in.a[mt][0] = ldg4(xr[mt] + 64 * g);
        in.a[mt][1] = ldg4(xr[mt] + 64 * g + 32);
    }
#pragma unroll
    for (int t = 0; t < NW; t++) {
        in.b[t][0] = ldg4(wr[t] + 64 * g);
        in.b[t][1] = ldg4(wr[t] + 64 * g + 32);
    }
}

template <int MT, int NW>
__device__ __forceinline__ void dmma(const DIn<MT, NW>& in, f32x4_t (&acc)[MT][NW]) {
#pragma unroll
    for (int h = 0; h < 2; h++)
#pragma unroll
        for (int t = 0; t < NW; t++)
#pragma unroll
            for (int mt = 0; mt < MT; mt++)
                acc[mt][t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as8(in.a[mt][h]), as8(in.b[t][h]), acc[mt][t], 0, 0, 0);
}

template <int MT, int NW, int E>
__global__ __launch_bounds__(256) void dgemm_kernel(DGemm a) {
    extern __shared__ float red[];  // [KW][MT * 4][NW][64]
    const int KW = blockDim.x / kWave;
    const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave, c = lane % 16, j = lane / 16;
    const int NS = E == DE_QKV ? a.N / 3 : a.N;  // columns per segment
    const int n0 = blockIdx.x * 16 * NW, si = E == DE_QKV ? n0 / NS : 0, ns0 = n0 - si * NS;
    const uint16_t* W = si == 0 ? a.w[0] : (si == 1 ? a.w[1] : a.w[2]);
    const uint16_t* B = si == 0 ? a.b[0] : (si == 1 ? a.b[1] : a.b[2]);
    const int MTT = (a.R + 15) / 16, mt0 = blockIdx.y * MT, G = a.K / 64;
    const uint16_t* xr[MT];
    const uint16_t* wr[NW];
#pragma unroll
    for (int mt = 0; mt < MT; mt++) {
        const int r = min(16 * min(mt0 + mt, MTT - 1) + c, a.R - 1);
        xr[mt] = a.x + (size_t)r * a.ldx + 8 * j;
    }
#pragma unroll
    for (int t = 0; t < NW; t++) {
        const int n = min(ns0 + 16 * t + c, NS - 1);
        wr[t] = W + (size_t)n * a.K + 8 * j;
    }
    const int gper = (G + KW - 1) / KW, g0 = wave * gper, g1 = min(G, g0 + gper);
    f32x4_t acc[MT][NW];
#pragma unroll
    for (int mt = 0; mt < MT; mt++)
#pragma unroll
        for (int t = 0; t < NW; t++) acc[mt][t] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
    if (g0 < g1) {
        DIn<MT, NW> b0, b1, b2;
        dload<MT, NW>(xr, wr, g0, b0);
        if (g0 + 1 < g1) dload<MT, NW>(xr, wr, g0 + 1, b1);
        for (int g = g0; g < g1; g += 3) {
            if (g + 2 < g1) dload<MT, NW>(xr, wr, g + 2, b2);
            dmma<MT, NW>(b0, acc);
            if (g + 1 >= g1) break;
            if (g + 3 < g1) dload<MT, NW>(xr, wr, g + 3, b0);
            dmma<MT, NW>(b1, acc);
            if (g + 2 >= g1) break;
            if (g + 4 < g1) dload<MT, NW>(xr, wr, g + 4, b1);
            dmma<MT, NW>(b2, acc);
        }
    }
    if (KW > 1) {
#pragma unroll
        for (int mt = 0; mt < MT; mt++)
#pragma unroll
            for (int r = 0; r < 4; r++)
#pragma unroll
                for (int t = 0; t < NW; t++) red[(((wave * MT + mt) * 4 + r) * NW + t) * kWave + lane] = acc[mt][t][r];
        __syncthreads();
    }
    auto sum = [&](int mt, int r, int t) {
        if (KW == 1) return acc[mt][t][r];
        float s = 0.0f;
        for (int w = 0; w < KW; w++) s += red[(((w * MT + mt) * 4 + r) * NW + t) * kWave + lane];
        return s;
    };
    if constexpr (E == DE_CFM) {
        // lane rows 4j + {0,1} and 4j + {2,3}: (cond, uncond) of two sequences; wave w takes the pairs u % KW == w
#pragma unroll
        for (int mt = 0; mt < MT; mt++)
#pragma unroll
            for (int pr = 0; pr < 2; pr++) {
                if ((mt * 2 + pr) % KW != wave) continue;
                const int m = 16 * (mt0 + mt) + 4 * j + 2 * pr;
                if (mt0 + mt >= MTT || m + 1 >= a.R) continue;
                const int sb = m / 2;
#pragma unroll
                for (int t = 0; t < NW; t++) {
                    const int n = n0 + 16 * t + c;
                    if (n >= a.N) continue;
                    const float bb = bf2f(gld(B + n));
                    const float pc = rb(sum(mt, 2 * pr, t) + bb), pn = rb(sum(mt, 2 * pr + 1, t) + bb);
                    const float f0 = rb(pc + rb(rb(pc - pn) * rb(a.cfg)));
                    float y = rb(bf2f(gld(a.y + (size_t)sb * a.N + n)) + rb(bf2f(gld(a.dt + a.step)) * f0));
                    if (a.shift != 0.0f)
                        y = rb(y + rb(rb(rb(a.shift) * bf2f(gld(a.sq + a.step))) *
                                      bf2f(gld(a.sde + ((size_t)sb * a.steps + a.step) * a.N + n))));
                    gst(a.y_out + (size_t)sb * a.N + n, f2bf(y));
                    if (a.y_steps) gst(a.y_steps + ((size_t)sb * a.steps + a.step) * a.N + n, f2bf(y));
                }
            }
        return;
    }
#pragma unroll
    for (int mt = 0; mt < MT; mt++)
#pragma unroll
        for (int r = 0; r < 4; r++) {
            if ((mt * 4 + r) % KW != wave) continue;
            const int m = 16 * (mt0 + mt) + 4 * j + r;
            const bool row_ok = mt0 + mt < MTT && m < a.R;
#pragma unroll
            for (int t = 0; t < NW; t++) {
                const int nn = ns0 + 16 * t + c;  // column within the segment
                const float e = rb(sum(mt, r, t) + bf2f(gld(B + min(nn, NS - 1))));
                if constexpr (E == DE_QKV) {
                    // interleaved rotary on q, k: the pair (2i, 2i+1) is lanes (c, c ^ 1)
                    const float other = __shfl_xor(e, 1, kWave);
                    if (!row_ok) continue;
                    float o = e;
                    if (si < 2) {
                        const int half = a.hd / 2, i = (nn % a.hd) / 2, l = m % a.L;
                        const float cs = gld(a.cos_t + l * half + i), sn = gld(a.sin_t + l * half + i);
                        const float ev = (c & 1) == 0 ? e : other, od = (c & 1) == 0 ? other : e;
                        const float p = ev * cs, q = od * sn, s2 = ev * sn, u = od * cs;
                        o = (c & 1) == 0 ? p - q : s2 + u;
                    }
                    gst(a.out + ((size_t)si * a.R + m) * NS + nn, f2bf(o));
                } else {
                    if (!row_ok || nn >= NS) continue;
                    const size_t off = (size_t)m * a.ldo + nn;
                    if constexpr (E == DE_BIAS) gst(a.out + off, f2bf(e));
                    if constexpr (E == DE_RES) gst(a.out + off, f2bf(bf2f(gld(a.res + off)) + e));
                    if constexpr (E == DE_GELU) gst(a.out + off, f2bf(gelu_chain_b(e)));
                }
            }
        }
}

// Rows rms-normalised (MLX fast::rms_norm: bf16(w * bf16(x * rsqrt(mean x^2 + eps)))),
// one workgroup per output row o; gather > 0: output row o = 2b + h is input
// row (2b + h) * gather + gather - 1 (the last position of each CFG half).
__global__ __launch_bounds__(256) void drms_kernel(const uint16_t* __restrict__ x, int K, int gather,
                                                   const uint16_t* __restrict__ w, float eps,
                                                   uint16_t* __restrict__ out) {
    __shared__ float red[4];
    const int o = blockIdx.x, src = gather > 0 ? o * gather + gather - 1 : o;
    const uint16_t* row = x + (size_t)src * K;
    float ss = 0.0f;
    for (int i = threadIdx.x; i < K / 8; i += 256) {
        const uint4 v = ldg4(row + 8 * i);
        const uint32_t e[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int p = 0; p < 4; p++) {
            const float lo = bf_lo(e[p]), hi = bf_hi(e[p]);
            ss += lo * lo;
            ss += hi * hi;
        }
    }
    ss = block_sum(ss, red);
    const float inv = 1.0f / sqrtf(ss / (float)K + eps);
    for (int i = threadIdx.x; i < K / 8; i += 256) {
        const uint4 v = ldg4(row + 8 * i), wv = ldg4(w + 8 * i);
        const uint32_t e[4] = {v.x, v.y, v.z, v.w}, we[4] = {wv.x, wv.y, wv.z, wv.w};
        uint32_t r4[4];
#pragma unroll
        for (int p = 0; p < 4; p++)
            r4[p] = pack_bf2(bf_lo(we[p]) * rb(bf_lo(e[p]) * inv), bf_hi(we[p]) * rb(bf_hi(e[p]) * inv));
        gst(reinterpret_cast<uint4*>(out + (size_t)o * K) + i, make_uint4(r4[0], r4[1], r4[2], r4[3]));
    }
}

// The CFM input rows of every sequence b (cfm `embed`, src/ming_fused.zig:559-561):
// rows (2b + h) * 3 + {0, 1, 2} = [te[h] + ce[b][h], xh[b], xe[b]].
__global__ __launch_bounds__(256) void cfm_rows_kernel(const uint16_t* __restrict__ te, const uint16_t* __restrict__ ce,
                                                       const uint16_t* __restrict__ bc, const uint16_t* __restrict__ xh,
                                                       const uint16_t* __restrict__ xe, int n, int D,
                                                       uint16_t* __restrict__ rows) {
    const int k = blockIdx.x * 256 + threadIdx.x;
    if (k >= n * D) return;
    const int b = k / D, d = k % D;
    const uint16_t xv = gld(xh + k), ev = gld(xe + k);
#pragma unroll
    for (int h = 0; h < 2; h++) {
        // c_emb([z, 0]): the unconditional half is the bias alone
        const float cev = h == 0 ? bf2f(gld(ce + k)) : bf2f(gld(bc + d));
        uint16_t* r = rows + (size_t)(2 * b + h) * 3 * D + d;
        gst(r, f2bf(bf2f(gld(te + (size_t)h * D + d)) + cev));
        gst(r + D, xv);
        gst(r + 2 * D, ev);
    }
}

template <int MT, int NW, int E>
hipError_t dlaunch(hipStream_t st, const DGemm& a, int kw) {
    const int mtt = (a.R + 15) / 16, gy = (mtt + MT - 1) / MT, gx = (a.N + 16 * NW - 1) / (16 * NW);
    const size_t lds = kw > 1 ? sizeof(float) * (size_t)kw * MT * 4 * NW * kWave : 0;
    hipLaunchKernelGGL((dgemm_kernel<MT, NW, E>), dim3(gx, gy), dim3(64 * kw), lds, st, a);
    return hipGetLastError();
}

// Row tiles per wave and K split from the shape: enough workgroups to cover
// the CUs, at most 4 row tiles, at most 4 waves (one per SIMD: a wave may
// hold 512 registers), LDS for the K split within 64 KB.
template <int E>
hipError_t dpick(hipStream_t st, const DGemm& a) {
    const int mtt = (a.R + 15) / 16, G = a.K / 64, gx = (a.N + 63) / 64;
    int mt = 1;
    if (mtt % 4 == 0 && gx * (mtt / 4) >= 128) mt = 4;
    else if (mtt % 2 == 0 && gx * (mtt / 2) >= 128) mt = 2;
    int kw = G >= 8 ? 4 : (G >= 2 ? 2 : 1);
    while (kw > 1 && (size_t)kw * mt * 4 * 4 * kWave * 4 > 65536) kw /= 2;
    if (E == DE_CFM) mt = 1;
    switch (mt) {
        case 4: return dlaunch<4, 4, E>(st, a, kw);
        case 2: return dlaunch<2, 4, E>(st, a, kw);
        default: return dlaunch<1, 4, E>(st, a, kw);
    }
}

DGemm gemm_args(const uint16_t* x, int R, int N, int K, const uint16_t* w, const uint16_t* b, uint16_t* out) {
    DGemm a{};
    a.x = x;
    a.ldx = K;
    a.R = R;
    a.N = N;
    a.K = K;
    a.w[0] = a.w[1] = a.w[2] = w;
    a.b[0] = a.b[1] = a.b[2] = b;
    a.out = out;
    a.ldo = N;
    return a;
}

}  // namespace

// One DiT block over R rows of L positions: rms1 -> q/k/v (+ rotary) -> attention
// -> out_proj + residual -> rms2 -> ff1 + gelu -> ff2 + residual.  x and out may
// not alias; hn [R][D], qkv [3][R][D], att [R][D], x1 [R][D], hh [R][F] scratch.
hipError_t launch_dit_block_gemm(hipStream_t st, const DitBlockDev& w, const uint16_t* x, int R, int L,
                                 const float* cos_t, const float* sin_t, uint16_t* hn, uint16_t* qkv, uint16_t* att,
                                 uint16_t* x1, uint16_t* hh, uint16_t* out) {
    const int D = w.D, F = w.F;
    hipError_t e;
    hipLaunchKernelGGL(drms_kernel, dim3(R), dim3(256), 0, st, x, D, 0, w.norm1, w.eps, hn);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    DGemm a = gemm_args(hn, R, 3 * D, D, w.wq, w.bq, qkv);
    a.w[1] = w.wk;
    a.w[2] = w.wv;
    a.b[1] = w.bk;
    a.b[2] = w.bv;
    a.cos_t = cos_t;
    a.sin_t = sin_t;
    a.L = L;
    a.hd = w.hd;
    if ((e = dpick<DE_QKV>(st, a)) != hipSuccess) return e;
    if ((e = launch_dit_attn(st, qkv, R / L, L, D, w.heads, w.hd, att)) != hipSuccess) return e;
    a = gemm_args(att, R, D, D, w.wo, w.bo, x1);
    a.res = x;
    if ((e = dpick<DE_RES>(st, a)) != hipSuccess) return e;
    hipLaunchKernelGGL(drms_kernel, dim3(R), dim3(256), 0, st, x1, D, 0, w.norm2, w.eps, hn);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    a = gemm_args(hn, R, F, D, w.w1, w.b1, hh);
    if ((e = dpick<DE_GELU>(st, a)) != hipSuccess) return e;
    a = gemm_args(hh, R, D, F, w.w2, w.b2, out);
    a.res = x1;
    return dpick<DE_RES>(st, a);
}

// out [R][N] = bf16(x W^T + b) (x [R][K]).
hipError_t launch_dit_linear_gemm(hipStream_t st, const uint16_t* x, int R, const uint16_t* w, int N, int K,
                                  const uint16_t* b, uint16_t* out) {
    return dpick<DE_BIAS>(st, gemm_args(x, R, N, K, w, b, out));
}

hipError_t launch_cfm_rows_batch(hipStream_t st, const uint16_t* te, const uint16_t* ce, const uint16_t* bc,
                                 const uint16_t* xh, const uint16_t* xe, int n, int D, uint16_t* rows) {
    hipLaunchKernelGGL(cfm_rows_kernel, dim3((n * D + 255) / 256), dim3(256), 0, st, te, ce, bc, xh, xe, n, D, rows);
    return hipGetLastError();
}

// The final layer of n sequences at Euler step `step`: rms(norm) of the last
// position of both CFG halves (rows of L positions in h [2n L][D]) -> linear
// [latent, D] + bias -> CFG + Euler (+ SDE) -> y_out [n][latent].
hipError_t launch_cfm_final_batch(hipStream_t st, const uint16_t* h, int n, int L, int D, const uint16_t* norm,
                                  float eps, const uint16_t* wf, const uint16_t* bf, int latent, const uint16_t* y,
                                  const uint16_t* dt, const uint16_t* sq, const uint16_t* sde, int step, int steps,
                                  float cfg, float shift, uint16_t* hn, uint16_t* y_out, uint16_t* y_steps) {
    hipLaunchKernelGGL(drms_kernel, dim3(2 * n), dim3(256), 0, st, h, D, L, norm, eps, hn);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    DGemm a = gemm_args(hn, 2 * n, latent, D, wf, bf, nullptr);
    a.y = y;
    a.dt = dt;
    a.sq = sq;
    a.sde = sde;
    a.step = step;
    a.steps = steps;
    a.cfg = cfg;
    a.shift = shift;
    a.y_out = y_out;
    a.y_steps = y_steps;
    return dpick<DE_CFM>(st, a);
}

}  // namespace ming
