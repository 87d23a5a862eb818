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
// l % 16).  A rows and W rows are both K-contiguous: the workgroup stages
// 64-k slices of both through LDS (dgemm_kernel below) and each lane reads
// its 16-byte fragments from there.
#include "args.h"
#include "common.h"
#include "internal.h"
#include "tanh_tab.h"

namespace ming {

namespace {


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
    // split K: grid z = ks slices of K / ks; f32 partials [ks][R][N] (bias and
    // epilogue applied by dreduce_kernel).  vs: the slices a row's sum is taken
    // over (a function of K alone); a workgroup that covers several of them (ks <
    // vs) sums each slice from zero and adds the slice sums in slice order, as
    // dreduce_kernel adds the partials, so the bits do not depend on ks
    float* part;
    int ks, vs;
};

__device__ __forceinline__ bf16x8_t as8(uint4 v) { return __builtin_bit_cast(bf16x8_t, u32x4_t{v.x, v.y, v.z, v.w}); }

// this file's copy of the tanh table (tanh_tab.h), filled at context creation
__device__ float dit_batch_tanh_tab[kTanhTabN];

__device__ __forceinline__ float gelu_chain_b(float x) {
    const float c0 = rb(0.044715f), c1 = rb(0.7978845608f);
    const float x3 = rb((float)((double)x * (double)x * (double)x));
    const float inner = rb(x + rb(c0 * x3));
    const float th = rb(tanh_bf16(dit_batch_tanh_tab, rb(c1 * inner)));  // as gelu_chain (dit.hip)
    return rb(rb(0.5f * x) * rb(1.0f + th));
}

// LDS-tiled GEMM: workgroup tile BM rows x 64 columns, K staged kBK (128 where
// K allows, else 64) at a time through two LDS buffers (rows padded by 8
// values: the 16 rows a fragment read touches fall in distinct banks).  256 threads load each stage
// cooperatively (16 bytes each, coalesced) while the previous stage's MFMAs
// run; wave w owns rows 32 (w / 2) .. + 32 and columns 32 (w % 2) .. + 32 of
// a 64-row tile (BM = 64), or rows 0 .. 32 and columns 16 w .. + 16 (BM = 32).
constexpr int kBN = 64;

template <int BM, int kBK>
struct DTile {
    static constexpr int NT = BM == 64 ? 2 : 1;       // 16-column tiles per wave
    static constexpr int AL = BM * kBK / 8 / 256;    // A chunks (16 B) per thread per stage
    static constexpr int BL = kBN * kBK / 8 / 256;   // B chunks per thread per stage
};

template <int BM, int kBK, int E>
__global__ __launch_bounds__(256) void dgemm_kernel(DGemm a) {
    constexpr int kPad = kBK + 8, kCPR = kBK / 8;
    using T = DTile<BM, kBK>;
    constexpr int NT = T::NT;
    __shared__ __align__(16) uint16_t As[2][BM * kPad];
    __shared__ __align__(16) uint16_t Bs[2][kBN * kPad];
    const int tid = threadIdx.x, wave = tid / kWave, lane = tid % kWave, c = lane % 16, j = lane / 16;
    const int NS = E == DE_QKV ? a.N / 3 : a.N;  // columns per segment (a tile never straddles two)
    const int n0 = blockIdx.x * kBN, si = E == DE_QKV ? n0 / NS : 0, ns0 = n0 - si * NS;
    const uint16_t* W = si == 0 ? a.w[0] : (si == 1 ? a.w[1] : a.w[2]);
    const uint16_t* B = si == 0 ? a.b[0] : (si == 1 ? a.b[1] : a.b[2]);
    const int m0 = blockIdx.y * BM, S = a.K / kBK / a.ks, s0 = blockIdx.z * S;
    const int wm = BM == 64 ? wave / 2 : 0, wn = BM == 64 ? wave % 2 : wave;
    // this thread's global chunks: chunk q -> (row q / kCPR, k 8 (q % kCPR))
    const uint16_t* ag[T::AL];
    const uint16_t* bg[T::BL];
#pragma unroll
    for (int i = 0; i < T::AL; i++) {
        const int q = tid + 256 * i, r = min(m0 + q / kCPR, a.R - 1);
        ag[i] = a.x + (size_t)r * a.ldx + 8 * (q % kCPR);
    }
#pragma unroll
    for (int i = 0; i < T::BL; i++) {
        const int q = tid + 256 * i, n = min(ns0 + q / kCPR, NS - 1);
        bg[i] = W + (size_t)n * a.K + 8 * (q % kCPR);
    }
    // two register sets: the stage about to be stored to LDS and the one after it, in flight
    uint4 ar[2][T::AL], br[2][T::BL];
    auto gload = [&](int s, int set) {
#pragma unroll
        for (int i = 0; i < T::AL; i++) ar[set][i] = ldg4(ag[i] + kBK * (s0 + s));
#pragma unroll
        for (int i = 0; i < T::BL; i++) br[set][i] = ldg4(bg[i] + kBK * (s0 + s));
    };
    auto lstore = [&](int buf, int set) {
#pragma unroll
        for (int i = 0; i < T::AL; i++) {
            const int q = tid + 256 * i;
            *reinterpret_cast<uint4*>(&As[buf][(q / kCPR) * kPad + 8 * (q % kCPR)]) = ar[set][i];
        }
#pragma unroll
        for (int i = 0; i < T::BL; i++) {
            const int q = tid + 256 * i;
            *reinterpret_cast<uint4*>(&Bs[buf][(q / kCPR) * kPad + 8 * (q % kCPR)]) = br[set][i];
        }
    };
    f32x4_t acc[2][NT], tot[2][NT];
#pragma unroll
    for (int mt = 0; mt < 2; mt++)
#pragma unroll
        for (int t = 0; t < NT; t++) acc[mt][t] = tot[mt][t] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
    // after stage s: at the end of a K slice (not the last one of this workgroup), add the
    // slice's sum to the total and start the next slice from zero
    const int Sv = a.K / kBK / a.vs;
    const bool fold = a.ks < a.vs;
    auto slice_end = [&](int s) {
        if (fold && (s + 1) % Sv == 0 && s + 1 < S) {
#pragma unroll
            for (int mt = 0; mt < 2; mt++)
#pragma unroll
                for (int t = 0; t < NT; t++) {
                    tot[mt][t] = tot[mt][t] + acc[mt][t];
                    acc[mt][t] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
                }
        }
    };
    auto compute = [&](int buf) {
#pragma unroll
        for (int ks = 0; ks < kBK / 32; ks++) {
            uint4 af[2], bfr[NT];
#pragma unroll
            for (int mt = 0; mt < 2; mt++)
                af[mt] = *reinterpret_cast<const uint4*>(&As[buf][(32 * wm + 16 * mt + c) * kPad + 32 * ks + 8 * j]);
#pragma unroll
            for (int t = 0; t < NT; t++)
                bfr[t] = *reinterpret_cast<const uint4*>(
                    &Bs[buf][((BM == 64 ? 32 : 16) * wn + 16 * t + c) * kPad + 32 * ks + 8 * j]);
#pragma unroll
            for (int mt = 0; mt < 2; mt++)
#pragma unroll
                for (int t = 0; t < NT; t++)
                    acc[mt][t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as8(af[mt]), as8(bfr[t]), acc[mt][t], 0, 0, 0);
        }
    };
    // stages in pairs so that every register-set and LDS-buffer index is a constant:
    // stage s computes from buffer s & 1 while stage s + 1 waits in set (s + 1) & 1
    // and stage s + 2 loads into set s & 1
    gload(0, 0);
    if (S > 1) gload(1, 1);
    lstore(0, 0);
    __syncthreads();
    for (int s = 0; s < S; s += 2) {
        if (s + 2 < S) gload(s + 2, 0);
        compute(0);
        slice_end(s);
        if (s + 1 < S) lstore(1, 1);
        __syncthreads();
        if (s + 1 >= S) break;
        if (s + 3 < S) gload(s + 3, 1);
        compute(1);
        slice_end(s + 1);
        if (s + 2 < S) lstore(0, 0);
        __syncthreads();
    }
    if (fold) {
#pragma unroll
        for (int mt = 0; mt < 2; mt++)
#pragma unroll
            for (int t = 0; t < NT; t++) acc[mt][t] = tot[mt][t] + acc[mt][t];
    }
    if (a.ks > 1) {  // split K: f32 partials of this slice; dreduce_kernel finishes
#pragma unroll
        for (int mt = 0; mt < 2; mt++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int m = m0 + 32 * wm + 16 * mt + 4 * j + r;
                if (m >= a.R) continue;
#pragma unroll
                for (int t = 0; t < NT; t++) {
                    const int n = ns0 + (BM == 64 ? 32 : 16) * wn + 16 * t + c;
                    if (n < NS) gst(a.part + ((size_t)blockIdx.z * a.R + m) * a.N + n, acc[mt][t][r]);
                }
            }
        return;
    }
    const int cb = ns0 + (BM == 64 ? 32 : 16) * wn;  // this wave's first column within the segment
    if constexpr (E == DE_CFM) {
        // lane rows 4j + {0,1} and 4j + {2,3}: (cond, uncond) of two sequences
#pragma unroll
        for (int mt = 0; mt < 2; mt++)
#pragma unroll
            for (int pr = 0; pr < 2; pr++) {
                const int m = m0 + 32 * wm + 16 * mt + 4 * j + 2 * pr;
                if (m + 1 >= a.R) continue;
                const int sb = m / 2;
#pragma unroll
                for (int t = 0; t < NT; t++) {
                    const int n = cb + 16 * t + c;
                    if (n >= a.N) continue;
                    const float bb = bf2f(gld(B + n));
                    const float pc = rb(acc[mt][t][2 * pr] + bb), pn = rb(acc[mt][t][2 * pr + 1] + bb);
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
    for (int mt = 0; mt < 2; mt++)
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int m = m0 + 32 * wm + 16 * mt + 4 * j + r;
            const bool row_ok = m < a.R;
#pragma unroll
            for (int t = 0; t < NT; t++) {
                const int nn = cb + 16 * t + c;  // column within the segment
                const float e = rb(acc[mt][t][r] + bf2f(gld(B + min(nn, NS - 1))));
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

// Split-K epilogue: sum the ks partials in slice order, then bias and the epilogue.
template <int E>
__global__ __launch_bounds__(256) void dreduce_kernel(DGemm a) {
    const int k = blockIdx.x * 256 + threadIdx.x;
    if (k >= a.R * a.N) return;
    const int m = k / a.N, n = k % a.N;
    float sum = 0.0f;
    for (int z = 0; z < a.ks; z++) sum += gld(a.part + (size_t)z * a.R * a.N + k);
    const float e = rb(sum + bf2f(gld(a.b[0] + n)));
    const size_t off = (size_t)m * a.ldo + n;
    if constexpr (E == DE_BIAS) gst(a.out + off, f2bf(e));
    if constexpr (E == DE_RES) gst(a.out + off, f2bf(bf2f(gld(a.res + off)) + e));
    if constexpr (E == DE_GELU) gst(a.out + off, f2bf(gelu_chain_b(e)));
}

// Split-K reduce with the residual epilogue (dreduce_kernel<DE_RES>'s arithmetic) followed
// by the row norm of the result (drms_kernel's): one workgroup per row m, thread t holding
// the 8-column chunks t, t + 256; writes the row to a.out and its normalised form to hn.
// The same bits as the two kernels back to back, one launch fewer.
__global__ __launch_bounds__(256) void dreduce_res_rms_kernel(DGemm a, const uint16_t* __restrict__ w, float eps,
                                                              uint16_t* __restrict__ hn) {
    __shared__ float red[4];
    const int m = blockIdx.x, N = a.N;
    constexpr int kMaxC = 2;  // chunks per thread: N <= 4096
    uint32_t xv[kMaxC][4];
    float ss = 0.0f;
#pragma unroll
    for (int k = 0; k < kMaxC; k++) {
        const int i = threadIdx.x + 256 * k;
        if (i >= N / 8) break;
#pragma unroll
        for (int p = 0; p < 4; p++) {
            float v[2];
#pragma unroll
            for (int h = 0; h < 2; h++) {
                const int n = 8 * i + 2 * p + h;
                float sum = 0.0f;
                for (int z = 0; z < a.ks; z++) sum += gld(a.part + ((size_t)z * a.R + m) * a.N + n);
                const float e = rb(sum + bf2f(gld(a.b[0] + n)));
                v[h] = rb(bf2f(gld(a.res + (size_t)m * a.ldo + n)) + e);
            }
            xv[k][p] = pack_bf2(v[0], v[1]);
            ss += v[0] * v[0];
            ss += v[1] * v[1];
        }
        gst(reinterpret_cast<uint4*>(a.out + (size_t)m * a.ldo) + i, make_uint4(xv[k][0], xv[k][1], xv[k][2], xv[k][3]));
    }
    ss = block_sum(ss, red);
    const float inv = 1.0f / sqrtf(ss / (float)N + eps);
#pragma unroll
    for (int k = 0; k < kMaxC; k++) {
        const int i = threadIdx.x + 256 * k;
        if (i >= N / 8) break;
        const uint4 wv = ldg4(w + 8 * i);
        const uint32_t we[4] = {wv.x, wv.y, wv.z, wv.w};
        uint32_t r4[4];
#pragma unroll
        for (int p = 0; p < 4; p++)
            r4[p] = pack_bf2(bf_lo(we[p]) * rb(bf_lo(xv[k][p]) * inv), bf_hi(we[p]) * rb(bf_hi(xv[k][p]) * inv));
        gst(reinterpret_cast<uint4*>(hn + (size_t)m * N) + i, make_uint4(r4[0], r4[1], r4[2], r4[3]));
    }
}

// 64-row tiles when they still give >= 128 workgroups, else 32-row tiles.
// K >= 2048 (plain epilogues, with a partials buffer) splits four ways across
// workgroups; the split depends on K alone, so a row's arithmetic does not
// depend on how many rows are batched.
template <int E>
void dsplit(DGemm& a) {
    constexpr bool SPLIT = E == DE_BIAS || E == DE_RES || E == DE_GELU;
    const int gx = (a.N + kBN - 1) / kBN, tiles = gx * ((a.R + 31) / 32);
    a.vs = SPLIT && a.K >= 2048 && a.K % (4 * 64) == 0 ? 4 : (SPLIT && a.K >= 1024 && a.K % (2 * 64) == 0 ? 2 : 1);
    a.ks = !a.part ? 1 : (a.vs == 4 ? 4 : (a.vs == 2 && tiles < 512 ? 2 : 1));
}

template <int E>
hipError_t dpick(hipStream_t st, DGemm a, const uint16_t* rms_w = nullptr, float rms_eps = 0.0f,
                 uint16_t* rms_out = nullptr) {
    const int gx = (a.N + kBN - 1) / kBN;
    // The sum over K is taken in vs slices fixed by K alone (4 from K = 2048, 2 from K = 1024,
    // for the epilogues the reduce kernel applies), so a sequence's bits do not depend on the
    // batch it is in.  How many workgroups share a row's K (ks) is a launch choice: latency
    // bound at these sizes, K split over workgroups keeps more of them per CU in flight
    // (measured on the 16- and 64-sequence server step: +9-11 %), except where the grid
    // already has >= 512 workgroups (splitting one at 768 loses 5 %); with ks < vs each
    // workgroup folds its slices in the reduce kernel's order.
    dsplit<E>(a);
    if (a.K % (64 * a.vs)) return hipErrorInvalidValue;
    // 128-wide K stages put twice the bytes of each stage in flight (measured: +10 % at 96 rows);
    // slices are whole stages
    if (a.K % (128 * a.vs) == 0)
        hipLaunchKernelGGL((dgemm_kernel<32, 128, E>), dim3(gx, (a.R + 31) / 32, a.ks), dim3(256), 0, st, a);
    else
        hipLaunchKernelGGL((dgemm_kernel<32, 64, E>), dim3(gx, (a.R + 31) / 32, a.ks), dim3(256), 0, st, a);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    // rms_out: the caller wants the rows' norm next (DE_RES only); with split K the reduce does it
    if (a.ks == 1) {
        if (rms_out) {
            hipLaunchKernelGGL(drms_kernel, dim3(a.R), dim3(256), 0, st, a.out, a.N, 0, rms_w, rms_eps, rms_out);
            e = hipGetLastError();
        }
        return e;
    }
    if constexpr (E == DE_RES) {
        if (rms_out) {
            if (a.N % 8 || a.N > 4096 || a.ldo != a.N) return hipErrorInvalidValue;
            hipLaunchKernelGGL(dreduce_res_rms_kernel, dim3(a.R), dim3(256), 0, st, a, rms_w, rms_eps, rms_out);
            return hipGetLastError();
        }
    }
    if constexpr (E == DE_BIAS || E == DE_RES || E == DE_GELU) {
        hipLaunchKernelGGL(dreduce_kernel<E>, dim3((a.R * a.N + 255) / 256), dim3(256), 0, st, a);
        e = hipGetLastError();
    }
    return e;
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
    a.ks = a.vs = 1;
    return a;
}

}  // namespace

// One DiT block over R rows of L positions: rms1 -> q/k/v (+ rotary) -> attention
// -> out_proj + residual -> rms2 -> ff1 + gelu -> ff2 + residual.  x and out may
// not alias; hn [R][D], qkv [3][R][D], att [R][D], x1 [R][D], hh [R][F] and
// part f32 scratch of max(4 R D, 2 R F) floats (split-K partials).  hn_ready: hn
// already holds rms1(x) (the block before wrote it); next: the following block,
// whose rms1 of this block's output is left in hn.  A residual projection with
// split K takes the norm after it into its reduce kernel (dreduce_res_rms_kernel).
hipError_t launch_dit_block_gemm(hipStream_t st, const DitBlockDev& w, const uint16_t* x, int R, int L,
                                 const float* cos_t, const float* sin_t, uint16_t* hn, uint16_t* qkv, uint16_t* att,
                                 uint16_t* x1, uint16_t* hh, uint16_t* out, float* part, bool hn_ready,
                                 const DitBlockDev* next) {
    const int D = w.D, F = w.F;
    hipError_t e;
    if (!hn_ready) {
        hipLaunchKernelGGL(drms_kernel, dim3(R), dim3(256), 0, st, x, D, 0, w.norm1, w.eps, hn);
        if ((e = hipGetLastError()) != hipSuccess) return e;
    }
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
    a.part = part;  // [2][R][D] of the [4][R][D] scratch
    if ((e = dpick<DE_RES>(st, a, w.norm2, w.eps, hn)) != hipSuccess) return e;  // x1, then rms2(x1) into hn
    a = gemm_args(hn, R, F, D, w.w1, w.b1, hh);
    a.part = part;  // [2][R][F]
    if ((e = dpick<DE_GELU>(st, a)) != hipSuccess) return e;
    a = gemm_args(hh, R, D, F, w.w2, w.b2, out);
    a.res = x1;
    a.part = part;  // [4][R][D] f32: ff2's K = F splits
    return next ? dpick<DE_RES>(st, a, next->norm1, next->eps, hn) : dpick<DE_RES>(st, a);
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

hipError_t tanh_upload_dit_batch(const float* host) {
    return hipMemcpyToSymbol(HIP_SYMBOL(dit_batch_tanh_tab), host, sizeof(float) * kTanhTabN);
}

}  // namespace ming
