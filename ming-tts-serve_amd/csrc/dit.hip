// DiT flow head (CFM) and aggregator for gfx950: the reference's fused
// kernels A-F (src/ming_fused.zig:145-289) rebuilt as bf16 GEMVs over at
// most 6 activation rows, with MLX-graph numerics (src/ming_model.zig:783-795,
// :1078-1091, :1161-1188): rms_norm rounds the normalised row to bf16 before
// the product, each linear is addmm (one rounding of acc + bias), the
// interleaved-pair rotary is computed in f32 against f32 tables and rounded
// once, attention is f32 with the output rounded once, and every op of the
// gelu chain and of the CFG/Euler update rounds to bf16.
//
// GEMV layout: a workgroup of 4 waves owns 8 output rows (two 32-lane teams
// per wave, one output row each); the R input rows (R <= 6, K <= 4096) are
// staged in LDS once per workgroup (normalised there when the stage has an
// rms_norm); a lane holds K/256 16-byte weight chunks in registers, loaded
// before the staging so the HBM latency overlaps it; team sums use DPP.
// Rows past N load the last row again and write nothing.
#include "gemv.h"
#include "internal.h"

namespace ming {

namespace {

constexpr int kDB = 256;     // threads per workgroup
constexpr int kDRows = 8;    // output rows per workgroup
constexpr int kMaxR = 6;     // activation rows

enum DitEpi {
    E_BIAS = 0,     // out[r][n] = bf16(acc + b)
    E_RES = 1,      // out[r][n] = bf16(res[r][n] + bf16(acc + b))
    E_GELU = 2,     // out = gelu_approx(bf16(acc + b)), every op rounded
    E_SILU = 3,     // out = bf16(v * bf16(sigmoid(v))), v = bf16(acc + b)
    E_QKV = 4,      // q|k|v columns of [3][R][D] + interleaved rotary on q, k
    E_CFMROWS = 5,  // x_emb(y) column n into the 6 CFM input rows (+ t_emb + c_emb, x_emb(hist))
    E_CFM = 6,      // CFG combine + Euler update of latent channel n (rows: cond, uncond)
    E_STOP = 7,     // softmax of the 2 stop logits (f32), probability of class 1
};

struct DitGemv {
    const uint16_t* x;  // input row r = x + (xrow0 + r * xstride) * K
    int64_t xrow0, xstride;
    int R;
    const uint16_t* norm;  // rms_norm weight [K] or null
    float eps;
    const uint16_t* w;  // bf16 [N, K]
    int N, K;
    const uint16_t* bias;  // [N]
    uint16_t* out;         // out[r * ostride + n] (layouts per epilogue)
    int64_t ostride;
    const uint16_t* res;   // E_RES: res[r * ostride + n]
    // E_QKV: rows [0, D) of wq, then wk, then wv (N = 3*D)
    const uint16_t* w3[3];
    const uint16_t* b3[3];
    const float* cos_t;    // [L][hd/2]
    const float* sin_t;
    int L, D, hd;
    // E_CFMROWS: te [2][D], ce [2][D], xh [D] -> out rows [2*3][D]
    const uint16_t* te;
    const uint16_t* ce;
    const uint16_t* xh;
    // E_CFM
    const uint16_t* y;
    const uint16_t* dt;
    const uint16_t* sq;
    const uint16_t* sde;   // [steps][latent]
    int step;
    float cfg, shift;
    uint16_t* y_out;
    float* p_out;          // E_STOP
};

__device__ __forceinline__ float gelu_chain(float x) {
    const float c0 = rb(0.044715f), c1 = rb(0.7978845608f);
    const float x3 = rb(powf(x, 3.0f));
    const float inner = rb(x + rb(c0 * x3));
    const float th = rb(tanhf(rb(c1 * inner)));
    return rb(rb(0.5f * x) * rb(1.0f + th));
}

template <int E, bool NORM, int NCH>
__global__ __launch_bounds__(kDB) void dit_gemv_kernel(DitGemv a) {
    extern __shared__ uint32_t xs[];  // [R][K/2] bf16 pairs, natural order
    __shared__ float red[kDB / kWave][kMaxR];
    __shared__ float inv_s[kMaxR];
    const int t = threadIdx.x, wave = t / kWave, lane = t % kWave, team = lane / 32, tl = lane % 32;
    const int K = a.K, R = a.R, NCk = K / 8, K2 = K / 2;
    const int n = blockIdx.x * kDRows + wave * 2 + team;
    const int nn = min(n, a.N - 1);
    // weight matrix and row of output n (q/k/v: D % 8 == 0 keeps a workgroup in one matrix)
    const int which = E == E_QKV ? nn / a.D : 0;
    const int nrow = E == E_QKV ? nn % a.D : nn;
    const uint16_t* W = E == E_QKV ? a.w3[which] : a.w;
    const uint16_t* Bv = E == E_QKV ? a.b3[which] : a.bias;
    // weight loads first (lanes past the row's end reload its last chunk)
    uint4 wr[NCH];
    const uint16_t* wrow = W + (size_t)nrow * K;
#pragma unroll
    for (int j = 0; j < NCH; j++) wr[j] = ldg4(wrow + 8 * min(tl + 32 * j, NCk - 1));
    // stage the R input rows (rms-normalised when NORM)
    if (NORM) {
        float ss[kMaxR];
#pragma unroll
        for (int r = 0; r < kMaxR; r++) {
            ss[r] = 0.0f;
            if (r < R) {
                const uint16_t* xr = a.x + (a.xrow0 + r * a.xstride) * K;
                for (int i = t; i < K2; i += kDB) {
                    const uint32_t v = gld(reinterpret_cast<const uint32_t*>(xr) + i);
                    const float lo = bf_lo(v), hi = bf_hi(v);
                    ss[r] += lo * lo;
                    ss[r] += hi * hi;
                }
            }
            ss[r] = team_sum<kWave>(ss[r]);
        }
        if (lane == 0)
#pragma unroll
            for (int r = 0; r < kMaxR; r++) red[wave][r] = ss[r];
        __syncthreads();
        if (t < kMaxR) {
            float s = 0.0f;
            for (int w = 0; w < kDB / kWave; w++) s += red[w][t];
            inv_s[t] = 1.0f / sqrtf(s / (float)K + a.eps);
        }
        __syncthreads();
        for (int r = 0; r < R; r++) {
            const uint16_t* xr = a.x + (a.xrow0 + r * a.xstride) * K;
            const float inv = inv_s[r];
            for (int i = t; i < K2; i += kDB) {
                const uint32_t v = gld(reinterpret_cast<const uint32_t*>(xr) + i);
                const uint32_t wn = gld(reinterpret_cast<const uint32_t*>(a.norm) + i);
                xs[r * K2 + i] = pack_bf2(bf_lo(wn) * rb(bf_lo(v) * inv), bf_hi(wn) * rb(bf_hi(v) * inv));
            }
        }
    } else {
        for (int r = 0; r < R; r++) {
            const uint16_t* xr = a.x + (a.xrow0 + r * a.xstride) * K;
            for (int i = t; i < K / 8; i += kDB)
                reinterpret_cast<uint4*>(xs + r * K2)[i] = ldg4(xr + 8 * i);
        }
    }
    __syncthreads();
    // dot products of this team's row with the R staged rows
    float acc[kMaxR];
#pragma unroll
    for (int r = 0; r < kMaxR; r++) acc[r] = 0.0f;
#pragma unroll
    for (int j = 0; j < NCH; j++) {
        const int c = tl + 32 * j;
        if (c < NCk) {
#pragma unroll
            for (int r = 0; r < kMaxR; r++)
                if (r < R) {
                    const uint4 xv = reinterpret_cast<const uint4*>(xs + r * K2)[c];
                    float s = dot2(wr[j].x, xv.x, acc[r]);
                    s = dot2(wr[j].y, xv.y, s);
                    s = dot2(wr[j].z, xv.z, s);
                    acc[r] = dot2(wr[j].w, xv.w, s);
                }
        }
    }
#pragma unroll
    for (int r = 0; r < kMaxR; r++) acc[r] = team_sum<32>(acc[r]);
    // epilogue: lane tl = r of each team handles row r
    float v = 0.0f;
#pragma unroll
    for (int r = 0; r < kMaxR; r++)
        if (tl == r) v = acc[r];
    const int r = tl;
    if (E == E_QKV) {
        // the rotary pair (2i, 2i+1) is (team 0, team 1) of this wave: D and 8 are even
        const float e = r < R ? rb(v + bf2f(gld(Bv + nrow))) : 0.0f;
        const float other = __shfl(e, lane ^ 32, kWave);
        if (r >= R || n >= a.N) return;
        const int col = nrow;
        float o = e;
        if (which < 2) {
            // four separate f32 products, no fused multiply-add (MLX evaluates mul, then sub/add)
#pragma clang fp contract(off)
            const int l = r % a.L, i = (col % a.hd) / 2, half = a.hd / 2;
            const float cs = gld(a.cos_t + l * half + i), sn = gld(a.sin_t + l * half + i);
            const float ev = team == 0 ? e : other, od = team == 0 ? other : e;
            const float p = ev * cs, q = od * sn, s2 = ev * sn, u = od * cs;
            o = team == 0 ? p - q : s2 + u;
        }
        gst(a.out + ((size_t)which * R + r) * a.D + col, f2bf(o));
        return;
    }
    if (E == E_CFM) {
        // every lane of the team holds both rows' sums: row 0 cond, row 1 uncond
        if (tl != 0 || n >= a.N) return;
        const float b = bf2f(gld(a.bias + n));
        const float pc = rb(acc[0] + b), pn = rb(acc[1] + b);
        const float f0 = rb(pc + rb(rb(pc - pn) * rb(a.cfg)));
        float y = rb(bf2f(gld(a.y + n)) + rb(bf2f(gld(a.dt + a.step)) * f0));
        if (a.shift != 0.0f)
            y = rb(y + rb(rb(rb(a.shift) * bf2f(gld(a.sq + a.step))) * bf2f(gld(a.sde + (size_t)a.step * a.N + n))));
        gst(a.y_out + n, f2bf(y));
        return;
    }
    if (E == E_STOP) {
        const float l1 = __shfl(v, lane ^ 32, kWave);
        if (blockIdx.x != 0 || wave != 0 || lane != 0) return;
        const float x0 = rb(v + bf2f(gld(a.bias))), x1 = rb(l1 + bf2f(gld(a.bias + 1)));
        const float m = fmaxf(x0, x1), e0 = expf(x0 - m), e1 = expf(x1 - m);
        gst(a.p_out, e1 / (e0 + e1));
        return;
    }
    if (r >= R || n >= a.N) return;
    const float e = rb(v + bf2f(gld(a.bias + n)));
    if (E == E_BIAS) {
        gst(a.out + r * a.ostride + n, f2bf(e));
    } else if (E == E_RES) {
        gst(a.out + r * a.ostride + n, f2bf(bf2f(gld(a.res + r * a.ostride + n)) + e));
    } else if (E == E_GELU) {
        gst(a.out + r * a.ostride + n, f2bf(gelu_chain(e)));
    } else if (E == E_SILU) {
        gst(a.out + r * a.ostride + n, f2bf(e * rb(1.0f / (1.0f + expf(-e)))));
    } else if (E == E_CFMROWS) {
        // rows [t_emb + c_emb, x_emb(hist), x_emb(y)] of both CFG halves
        const uint16_t xe = f2bf(e), xh = gld(a.xh + n);
#pragma unroll
        for (int b = 0; b < 2; b++) {
            gst(a.out + (size_t)(b * 3 + 0) * a.N + n,
                f2bf(bf2f(gld(a.te + (size_t)b * a.N + n)) + bf2f(gld(a.ce + (size_t)b * a.N + n))));
            gst(a.out + (size_t)(b * 3 + 1) * a.N + n, xh);
            gst(a.out + (size_t)(b * 3 + 2) * a.N + n, xe);
        }
    }
}

// Attention over the L positions of each sequence, one wave per (sequence,
// head): lane d owns dimension d; f32 scores with the 1/8 scale on q, f32
// softmax, output rounded once.
__global__ __launch_bounds__(kWave) void dit_attn_kernel(const uint16_t* qkv, int R, int L, int D, int heads, int hd,
                                                         uint16_t* att) {
    // lanes past head_dim take part in the wave sums with zeros
    const int b = blockIdx.x / heads, h = blockIdx.x % heads, d = threadIdx.x, dd = min(d, hd - 1);
    const bool on = d < hd;
    const uint16_t* q = qkv;
    const uint16_t* k = qkv + (size_t)R * D;
    const uint16_t* v = qkv + (size_t)2 * R * D;
    const float scale = 1.0f / 8.0f;
    for (int i = 0; i < L; i++) {
        const float qd = on ? scale * bf2f(gld(q + (size_t)(b * L + i) * D + h * hd + dd)) : 0.0f;
        float sc[8], m = -INFINITY;
        for (int j = 0; j < L; j++) {
            sc[j] = team_sum<kWave>(qd * bf2f(gld(k + (size_t)(b * L + j) * D + h * hd + dd)));
            m = fmaxf(m, sc[j]);
        }
        float l = 0.0f, o = 0.0f;
        for (int j = 0; j < L; j++) {
            const float p = expf(sc[j] - m);
            l += p;
            o += p * bf2f(gld(v + (size_t)(b * L + j) * D + h * hd + dd));
        }
        if (on) gst(att + (size_t)(b * L + i) * D + h * hd + d, f2bf(o / l));
    }
}

template <int E, bool NORM>
hipError_t launch_gemv(hipStream_t st, const DitGemv& a) {
    const int grid = (a.N + kDRows - 1) / kDRows;
    const size_t lds = sizeof(uint32_t) * (size_t)a.R * (a.K / 2);
    if (a.K <= 256)
        hipLaunchKernelGGL((dit_gemv_kernel<E, NORM, 1>), dim3(grid), dim3(kDB), lds, st, a);
    else if (a.K <= 1024)
        hipLaunchKernelGGL((dit_gemv_kernel<E, NORM, 4>), dim3(grid), dim3(kDB), lds, st, a);
    else
        hipLaunchKernelGGL((dit_gemv_kernel<E, NORM, 16>), dim3(grid), dim3(kDB), lds, st, a);
    return hipGetLastError();
}

DitGemv gemv_args(const uint16_t* x, int R, const uint16_t* w, int N, int K, const uint16_t* bias, uint16_t* out) {
    DitGemv a{};
    a.x = x;
    a.xrow0 = 0;
    a.xstride = 1;
    a.R = R;
    a.w = w;
    a.N = N;
    a.K = K;
    a.bias = bias;
    a.out = out;
    a.ostride = N;
    a.eps = 1e-6f;
    return a;
}

}  // namespace

// ---- entry points used by the C ABI (csrc/api_dit.cpp) ---------------------------

// One stage of a DiT block on x [R][D] (R = B*L):
//   0  A: rms1 + q/k/v + bias + rotary -> qkv [3][R][D], attention -> out
//   1  B: out = x + out_proj(in)          (in = attention output)
//   2  C: out = gelu(ff1(rms2(x)))        ([R][F])
//   3  D: out = x + ff2(in)               (in = C's output)
hipError_t launch_dit_stage(hipStream_t st, int which, const DitBlockDev& w, const uint16_t* x, const uint16_t* in,
                            int B, int L, const float* cos_t, const float* sin_t, uint16_t* qkv, uint16_t* out) {
    const int R = B * L, D = w.D, F = w.F;
    DitGemv a;
    switch (which) {
        case 0: {
            a = gemv_args(x, R, nullptr, 3 * D, D, nullptr, qkv);
            a.w3[0] = w.wq;
            a.w3[1] = w.wk;
            a.w3[2] = w.wv;
            a.b3[0] = w.bq;
            a.b3[1] = w.bk;
            a.b3[2] = w.bv;
            a.norm = w.norm1;
            a.eps = w.eps;
            a.cos_t = cos_t;
            a.sin_t = sin_t;
            a.L = L;
            a.D = D;
            a.hd = w.hd;
            hipError_t e = launch_gemv<E_QKV, true>(st, a);
            if (e != hipSuccess) return e;
            hipLaunchKernelGGL(dit_attn_kernel, dim3(B * w.heads), dim3(kWave), 0, st, qkv, R, L, D, w.heads, w.hd,
                               out);
            return hipGetLastError();
        }
        case 1:
            a = gemv_args(in, R, w.wo, D, D, w.bo, out);
            a.res = x;
            return launch_gemv<E_RES, false>(st, a);
        case 2:
            a = gemv_args(x, R, w.w1, F, D, w.b1, out);
            a.norm = w.norm2;
            a.eps = w.eps;
            return launch_gemv<E_GELU, true>(st, a);
        default:
            a = gemv_args(in, R, w.w2, D, F, w.b2, out);
            a.res = x;
            return launch_gemv<E_RES, false>(st, a);
    }
}

// One DiT block: the four stages in order.
hipError_t launch_dit_block(hipStream_t st, const DitBlockDev& w, const uint16_t* x, int B, int L,
                            const float* cos_t, const float* sin_t, uint16_t* qkv, uint16_t* att, uint16_t* x1,
                            uint16_t* hh, uint16_t* x2) {
    hipError_t e;
    if ((e = launch_dit_stage(st, 0, w, x, nullptr, B, L, cos_t, sin_t, qkv, att)) != hipSuccess) return e;
    if ((e = launch_dit_stage(st, 1, w, x, att, B, L, cos_t, sin_t, qkv, x1)) != hipSuccess) return e;
    if ((e = launch_dit_stage(st, 2, w, x1, nullptr, B, L, cos_t, sin_t, qkv, hh)) != hipSuccess) return e;
    return launch_dit_stage(st, 3, w, x1, hh, B, L, cos_t, sin_t, qkv, x2);
}

// y [N] = bf16(W x + b) over R rows (optionally rms-normalised input rows,
// rows xrow0 + r*xstride of x), E_BIAS or E_SILU epilogue.
hipError_t launch_dit_linear(hipStream_t st, const uint16_t* x, int64_t xrow0, int64_t xstride, int R,
                             const uint16_t* norm, float eps, const uint16_t* w, int N, int K, const uint16_t* bias,
                             uint16_t* out, bool silu) {
    DitGemv a = gemv_args(x, R, w, N, K, bias, out);
    a.xrow0 = xrow0;
    a.xstride = xstride;
    a.norm = norm;
    a.eps = eps;
    if (norm) return silu ? launch_gemv<E_SILU, true>(st, a) : launch_gemv<E_BIAS, true>(st, a);
    return silu ? launch_gemv<E_SILU, false>(st, a) : launch_gemv<E_BIAS, false>(st, a);
}

// fused.embed: rows [2*3][D] = [te + ce, xh, x_emb(y)] per CFG half.
hipError_t launch_cfm_embed(hipStream_t st, const uint16_t* y, const uint16_t* wx, const uint16_t* bx, int D, int latent,
                            const uint16_t* te, const uint16_t* ce, const uint16_t* xh, uint16_t* rows) {
    DitGemv a = gemv_args(y, 1, wx, D, latent, bx, rows);
    a.te = te;
    a.ce = ce;
    a.xh = xh;
    return launch_gemv<E_CFMROWS, false>(st, a);
}

// fused.final: rms + final linear on rows L-1 and 2L-1 of h, CFG + Euler.
hipError_t launch_cfm_final(hipStream_t st, const uint16_t* h, int L, int D, const uint16_t* norm, float eps,
                            const uint16_t* wf, const uint16_t* bf, int latent, const uint16_t* y, const uint16_t* dt,
                            const uint16_t* sq, const uint16_t* sde, int step, float cfg, float shift,
                            uint16_t* y_out) {
    DitGemv a = gemv_args(h, 2, wf, latent, D, bf, nullptr);
    a.xrow0 = L - 1;
    a.xstride = L;
    a.norm = norm;
    a.eps = eps;
    a.y = y;
    a.dt = dt;
    a.sq = sq;
    a.sde = sde;
    a.step = step;
    a.cfg = cfg;
    a.shift = shift;
    a.y_out = y_out;
    return launch_gemv<E_CFM, true>(st, a);
}

// stopProb: p = softmax(f32(bf16(W z + b)))[1] (W [2][K]).
hipError_t launch_stop_prob(hipStream_t st, const uint16_t* z, const uint16_t* w, const uint16_t* b, int K, float* p) {
    DitGemv a = gemv_args(z, 1, w, 2, K, b, nullptr);
    a.p_out = p;
    return launch_gemv<E_STOP, false>(st, a);
}

}  // namespace ming
