// DiT flow head (CFM) and aggregator for gfx950: the reference's fused
// kernels A-F (src/ming_fused.zig:145-289) rebuilt as bf16 GEMVs over at
// most 6 activation rows, with MLX-graph numerics (src/ming_model.zig:783-795,
// :1078-1091, :1161-1188): rms_norm rounds the normalised row to bf16 before
// the product, each linear is addmm (one rounding of acc + bias), the
// interleaved-pair rotary is computed in f32 against f32 tables and rounded
// once, attention is f32 with the output rounded once, and every op of the
// gelu chain and of the CFG/Euler update rounds to bf16.
//
// GEMV layout: a workgroup of W waves (W = 2 or 4) owns 2W output rows, one
// per 32-lane team; a lane holds K/256 16-byte weight chunks in registers.
// Each lane adds its products with v_dot2c_f32_bf16 (two products per step,
// chunks in order), and the team's lane sums meet in the DPP tree; that order
// and the instruction's own fixed-grid accumulation are what the oracle's
// device order restates, so the flow head is reproducible on a CPU bit for bit.
// The weight loads go first, then the epilogue's operands (bias, residual,
// rotary table, CFM inputs), then the R input rows (R <= 6) in one batch of
// loads -- every load is issued before the first one is used, so the kernel
// waits for memory once.  The rows are staged in LDS as they are or
// rms-normalised (the row sums reduced from the registers of the batch).
// These kernels are latency-bound (a few MB per launch, every workgroup
// resident at once), so the code keeps the dependent instruction chain of a
// wave short: native bf16 rounding, one reciprocal square root per row shared
// by readlane, no loads after the reduction.  Team sums use DPP; rows past N
// load the last row again and write nothing.
#include <algorithm>
#include <cmath>
#include <cstring>
#include <mutex>
#include <vector>

#include "gemv.h"
#include "internal.h"
#include "tanh_tab.h"

namespace ming {

namespace {

constexpr int kMaxR = 6;       // activation rows of a reference-shape block (2 x 3)
constexpr int kMaxSlots = 20;  // row slots of the widest launch (adaLN modulations: 10 steps x 2 halves)
// 16-byte LDS vector (the staged rows are 16-byte aligned: K % 8 == 0)
typedef uint32_t lds_u32x4_t __attribute__((ext_vector_type(4), aligned(16)));
constexpr int kMaxL = 8;  // positions per sequence (attention)
constexpr int kMaxH = 4;  // heads per wave in dit_attn_out_kernel (16 heads, 4 waves)

enum DitEpi {
    E_BIAS = 0,     // out[r][n] = bf16(acc + b)
    E_RES = 1,      // out[r][n] = bf16(res[r][n] + bf16(acc + b))
    E_GELU = 2,     // out = gelu_approx(bf16(acc + b)), every op rounded
    E_SILU = 3,     // out = bf16(v * bf16(sigmoid(v))), v = bf16(acc + b)
    E_QKV = 4,      // q|k|v columns of [3][R][D] + interleaved rotary on q, k
    E_CFMROWS = 5,  // x_emb(y) column n into the 6 CFM input rows (+ t_emb + c_emb, x_emb(hist))
    E_CFM = 6,      // CFG combine + Euler update of latent channel n (rows: cond, uncond)
    E_STOP = 7,     // softmax of the 2 stop logits (f32), probability of class 1
    E_GATE = 8,     // out[r][n] = bf16(res + bf16(gate * bf16(acc + b))), adaLN gated residual
    E_CFMF = 9,     // CFG + Euler of frame f = lane: rows f (cond) and F + f (uncond)
    E_PATCH = 10,   // x_emb of frame r into rows r and R + r (both CFG halves)
};

enum StageMode { M_PLAIN = 0, M_NORM = 1, M_ADANORM = 2 };  // M_ADANORM: rms_norm, then modulate

struct DitGemv {
    const uint16_t* x;  // input row r = x + (xrow0 + r * xstride) * K
    int64_t xrow0, xstride;
    int R;
    const uint16_t* norm;  // M_NORM: rms_norm weight [K]
    float eps;
    const uint16_t* w;  // bf16 [N, K]
    int N, K;
    const uint16_t* bias;  // [N]
    uint16_t* out;         // out[r * ostride + n] (layouts per epilogue)
    int64_t ostride;
    const uint16_t* res;   // E_RES, E_GATE: res[r * ostride + n]
    // adaLN: modulation vectors of the CFG half of row r = mod + (r / rph) * mstride + {soff, coff, goff} * K|N
    const uint16_t* mod;
    int64_t mstride;
    int rph, soff, coff, goff;
    int F;                 // E_CFMF: frames per half
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
    const int32_t* flags_in;  // E_STOP: when set, flags_in[0..2] are copied to p_out[1..3] (as int32)
};

// (float)tanh((double)u) for every bf16 u in [0, 16] (tanh_tab.h), filled at
// context creation
__device__ float dit_tanh_tab[kTanhTabN];

__device__ __forceinline__ float gelu_chain(float x) {
    const float c0 = rb(0.044715f), c1 = rb(0.7978845608f);
    // x^3 in f64: x*x is exact there and the product rounds once, so the f32
    // result is x^3 correctly rounded (up to double rounding, which bf16 hides)
    const float x3 = rb((float)((double)x * (double)x * (double)x));
    const float inner = rb(x + rb(c0 * x3));
    // tanh of the bf16 argument: f64 tanh rounded to f32 (by table), then to
    // bf16 -- the CPU restatement's expression, so the two agree bit for bit
    const float th = rb(tanh_bf16(dit_tanh_tab, rb(c1 * inner)));
    return rb(rb(0.5f * x) * rb(1.0f + th));
}

// ---- staging ------------------------------------------------------------------------

// Rows as they are, or rms-normalised: bf16(w * bf16(x * inv)),
// inv = 1 / sqrt(mean(x^2) + eps) per row.  RC >= R row slots (slots past R
// repeat row R-1), XCH chunks of 8 per thread per row; the loops carry no
// branches, so the compiler issues every load, and later every LDS store,
// back to back.  Threads whose chunk is past the row's end store nothing and
// add nothing to the sums.
//
// stage_finish is the arithmetic on operands already in registers (xr the
// rows' chunks c = min(t + T j, K/8 - 1), gn the norm weight's, msh / msc the
// adaLN shift and scale of the two CFG halves); stage_rows loads them first.
template <int MODE, int RC, int XCH, int T>
__device__ __forceinline__ void stage_finish(const DitGemv& a, uint32_t* xs, float* red, int t,
                                             const uint4 (&xr)[RC][XCH], const uint4 (&gn)[XCH],
                                             const uint4 (&msh)[2][XCH], const uint4 (&msc)[2][XCH]) {
    constexpr bool NORM = MODE != M_PLAIN, ADA = MODE == M_ADANORM;
    const int K = a.K, NC = K / 8, K2 = K / 2, R = a.R;
    if (!NORM) {
#pragma unroll
        for (int j = 0; j < XCH; j++) {
            const int c = t + T * j;
            if (c < NC)
#pragma unroll
                for (int r = 0; r < RC; r++)
                    reinterpret_cast<lds_u32x4_t*>(xs)[r * (K2 / 4) + c] = u32x4_t{xr[r][j].x, xr[r][j].y, xr[r][j].z, xr[r][j].w};
        }
        return;
    }
    float ss[RC];
#pragma unroll
    for (int r = 0; r < RC; r++) {
        ss[r] = 0.0f;
#pragma unroll
        for (int j = 0; j < XCH; j++) {
            const float on = t + T * j < NC ? 1.0f : 0.0f;
            const uint32_t q[4] = {xr[r][j].x, xr[r][j].y, xr[r][j].z, xr[r][j].w};
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const float lo = on * bf_lo(q[e]), hi = on * bf_hi(q[e]);
                ss[r] += lo * lo;
                ss[r] += hi * hi;
            }
        }
        ss[r] = team_sum<kWave>(ss[r]);
    }
    const int wave = t / kWave, lane = t % kWave;
    if (lane == 0)
#pragma unroll
        for (int r = 0; r < RC; r++) red[wave * kMaxSlots + r] = ss[r];
    __syncthreads();
    // lane r of every wave finishes row r (waves summed in order), then broadcasts it
    float s = 0.0f;
#pragma unroll
    for (int w = 0; w < T / kWave; w++) s += red[w * kMaxSlots + min(lane, RC - 1)];
    const float my_inv = 1.0f / sqrtf(s / (float)K + a.eps);
    float inv[RC];
#pragma unroll
    for (int r = 0; r < RC; r++) inv[r] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(my_inv), r));
#pragma unroll
    for (int j = 0; j < XCH; j++) {
        const int c = t + T * j;
        const uint32_t g[4] = {gn[j].x, gn[j].y, gn[j].z, gn[j].w};
        uint4 o[RC];
#pragma unroll
        for (int r = 0; r < RC; r++) {
            const uint32_t q[4] = {xr[r][j].x, xr[r][j].y, xr[r][j].z, xr[r][j].w};
            uint32_t w4[4];
            if (ADA) {
                // modulate(n) = bf16(bf16(n * bf16(1 + scale)) + shift), half of the row's slot
                const bool h1 = min(r, R - 1) / a.rph != 0;
                const uint4 s4 = h1 ? msh[1][j] : msh[0][j], c4 = h1 ? msc[1][j] : msc[0][j];
                const uint32_t sh[4] = {s4.x, s4.y, s4.z, s4.w}, sc[4] = {c4.x, c4.y, c4.z, c4.w};
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const float nl = rb(bf_lo(g[e]) * rb(bf_lo(q[e]) * inv[r]));
                    const float nh2 = rb(bf_hi(g[e]) * rb(bf_hi(q[e]) * inv[r]));
                    const float vl = rb(nl * rb(1.0f + bf_lo(sc[e]))), vh = rb(nh2 * rb(1.0f + bf_hi(sc[e])));
                    w4[e] = pack_bf2(vl + bf_lo(sh[e]), vh + bf_hi(sh[e]));
                }
            } else {
#pragma unroll
                for (int e = 0; e < 4; e++)
                    w4[e] = pack_bf2(bf_lo(g[e]) * rb(bf_lo(q[e]) * inv[r]), bf_hi(g[e]) * rb(bf_hi(q[e]) * inv[r]));
            }
            o[r] = make_uint4(w4[0], w4[1], w4[2], w4[3]);
        }
        if (c < NC)
#pragma unroll
            for (int r = 0; r < RC; r++)
                reinterpret_cast<lds_u32x4_t*>(xs)[r * (K2 / 4) + c] = u32x4_t{o[r].x, o[r].y, o[r].z, o[r].w};
    }
}

template <int MODE, int RC, int XCH, int T>
__device__ __forceinline__ void stage_rows(const DitGemv& a, uint32_t* xs, float* red, int t) {
    constexpr bool NORM = MODE != M_PLAIN, ADA = MODE == M_ADANORM;
    const int K = a.K, NC = K / 8, R = a.R;
    uint4 xr[RC][XCH];
    uint4 gn[XCH];
    uint4 msh[2][XCH], msc[2][XCH];  // adaLN shift / scale chunks of the (at most 2) CFG halves
    const int nh = ADA ? (R + a.rph - 1) / a.rph : 1;
#pragma unroll
    for (int j = 0; j < XCH; j++) {
        const int c = min(t + T * j, NC - 1);
        if (NORM) gn[j] = ldg4(a.norm + 8 * c);
#pragma unroll
        for (int r = 0; r < RC; r++) xr[r][j] = ldg4(a.x + (a.xrow0 + min(r, R - 1) * a.xstride) * K + 8 * c);
        if (ADA)
#pragma unroll
            for (int h = 0; h < 2; h++) {
                const uint16_t* mh = a.mod + min(h, nh - 1) * a.mstride;
                msh[h][j] = ldg4(mh + (size_t)a.soff * K + 8 * c);
                msc[h][j] = ldg4(mh + (size_t)a.coff * K + 8 * c);
            }
    }
    stage_finish<MODE, RC, XCH, T>(a, xs, red, t, xr, gn, msh, msc);
}

// Operands of the epilogue of lane tl (row r = tl, output n), loaded at
// kernel start so that no load waits at the end.
struct EpiIn {
    float b;        // bias
    float res;      // E_RES, E_GATE: residual
    float gate;     // E_GATE
    float cs, sn;   // E_QKV: rotary
    float te0, te1, ce0, ce1;  // E_CFMROWS
    uint16_t xh;
    float y, dt, sq, sde;      // E_CFM
};

template <int E>
__device__ __forceinline__ EpiIn epi_load(const DitGemv& a, int n, int nrow, int which, int r, const uint16_t* Bv) {
    EpiIn p{};
    const int rr = min(r, a.R - 1);
    if (E == E_QKV) {
        p.b = bf2f(gld(Bv + nrow));
        const int l = rr % a.L, i = (nrow % a.hd) / 2, half = a.hd / 2;
        p.cs = gld(a.cos_t + l * half + i);
        p.sn = gld(a.sin_t + l * half + i);
    } else {
        p.b = bf2f(gld(a.bias + n));
    }
    if (E == E_RES || E == E_GATE) p.res = bf2f(gld(a.res + rr * a.ostride + n));
    if (E == E_GATE) p.gate = bf2f(gld(a.mod + (rr / a.rph) * a.mstride + (size_t)a.goff * a.N + n));
    if (E == E_CFMF) {
        const int f = min(r, a.F - 1);
        p.y = bf2f(gld(a.y + (size_t)f * a.N + n));
        p.dt = bf2f(gld(a.dt + a.step));
        p.sq = bf2f(gld(a.sq + a.step));
        p.sde = a.shift != 0.0f ? bf2f(gld(a.sde + ((size_t)a.step * a.F + f) * a.N + n)) : 0.0f;
    }
    if (E == E_CFMROWS) {
        p.te0 = bf2f(gld(a.te + n));
        p.te1 = bf2f(gld(a.te + a.N + n));
        p.ce0 = bf2f(gld(a.ce + n));
        p.ce1 = bf2f(gld(a.ce + a.N + n));
        p.xh = gld(a.xh + n);
    }
    if (E == E_CFM) {
        p.y = bf2f(gld(a.y + n));
        p.dt = bf2f(gld(a.dt + a.step));
        p.sq = bf2f(gld(a.sq + a.step));
        p.sde = a.shift != 0.0f ? bf2f(gld(a.sde + (size_t)a.step * a.N + n)) : 0.0f;
    }
    return p;
}

// Dot products of a team's weight chunks (chunk tl + TEAM j of its row;
// chunks past the row's end are zeroed here) with the RC row slots staged in
// LDS: each lane's products in chunk order by v_dot2c, then the team's DPP
// tree, so every lane of the team holds acc[r].  No branches, so all LDS
// reads issue ahead of the dot chains.
template <int NCH, int RC, int TEAM>
__device__ __forceinline__ void gemv_dots(uint4 (&wr)[NCH], const uint32_t* xs, int tl, int K, float (&acc)[RC]) {
    const int NCk = K / 8, K2 = K / 2;
#pragma unroll
    for (int j = 0; j < NCH; j++) {
        const uint32_t m = tl + TEAM * j < NCk ? 0xffffffffu : 0u;
        wr[j].x &= m;
        wr[j].y &= m;
        wr[j].z &= m;
        wr[j].w &= m;
    }
    const lds_u32x4_t* xv4 = reinterpret_cast<const lds_u32x4_t*>(xs);
#pragma unroll
    for (int r = 0; r < RC; r++) acc[r] = 0.0f;
    // up to 6 row slots, chunk j + 1's row reads are issued before chunk j's
    // products, so they overlap the math instead of each waiting out its own
    // latency (wider slot counts would need the registers twice over)
    constexpr int NB = RC <= 6 ? 2 : 1;
    u32x4_t xv[NB][RC];
    if constexpr (NB == 2) {
#pragma unroll
        for (int r = 0; r < RC; r++) xv[0][r] = xv4[r * (K2 / 4) + min(tl, NCk - 1)];
    }
#pragma unroll
    for (int j = 0; j < NCH; j++) {
        const int jn = NB == 2 ? j + 1 : j;  // the chunk read here
        if (jn < NCH) {
            const int c = min(tl + TEAM * jn, NCk - 1);
#pragma unroll
            for (int r = 0; r < RC; r++) xv[jn % NB][r] = xv4[r * (K2 / 4) + c];
        }
        const u32x4_t(&x)[RC] = xv[j % NB];
#pragma unroll
        for (int r = 0; r < RC; r++) {
            float s = dot2(wr[j].x, x[r].x, acc[r]);
            s = dot2(wr[j].y, x[r].y, s);
            s = dot2(wr[j].z, x[r].z, s);
            acc[r] = dot2(wr[j].w, x[r].w, s);
        }
    }
#pragma unroll
    for (int r = 0; r < RC; r++) acc[r] = team_sum<TEAM>(acc[r]);
}

// ---- the GEMV kernel ----------------------------------------------------------------

// W waves, RPW output rows per wave (a team of 64 / RPW lanes per row), NCH
// 16-byte weight chunks per lane, RC row slots.
// (workgroup vb of the launch; xs the staged rows [R][K/2] as bf16 pairs in
// natural order, red W * kMaxSlots floats)
template <int E, int MODE, int NCH, int W, int RC, int RPW>
__device__ __forceinline__ void gemv_body(const DitGemv& a, int vb, uint32_t* xs, float* red) {
    constexpr int T = 64 * W, TEAM = kWave / RPW, ROWS = RPW * W, XCH = (NCH * TEAM + T - 1) / T;
    static_assert((E != E_QKV && E != E_STOP && E != E_CFMF) || RPW == 2, "per-row lanes live in a half wave");
    static_assert(RC <= kMaxSlots, "row slots");
    const int t = threadIdx.x, wave = t / kWave, lane = t % kWave, team = lane / TEAM, tl = lane % TEAM;
    const int K = a.K, R = a.R, NCk = K / 8, K2 = K / 2;
    const int n = vb * ROWS + wave * RPW + team;
    const int nn = min(n, a.N - 1);
    // weight matrix and row of output n (q/k/v: D % 8 == 0 keeps a row pair in one matrix)
    const int which = E == E_QKV ? nn / a.D : 0;
    const int nrow = E == E_QKV ? nn % a.D : nn;
    const uint16_t* Wm = E == E_QKV ? (which == 0 ? a.w3[0] : which == 1 ? a.w3[1] : a.w3[2]) : a.w;
    const uint16_t* Bv = E == E_QKV ? (which == 0 ? a.b3[0] : which == 1 ? a.b3[1] : a.b3[2]) : a.bias;
    // weight loads first (lanes past the row's end reload its last chunk and
    // zero it below), then the epilogue's operands, then the rows
    uint4 wr[NCH];
    const uint16_t* wrow = Wm + (size_t)nrow * K;
#pragma unroll
    for (int j = 0; j < NCH; j++) wr[j] = ldg4(wrow + 8 * min(tl + TEAM * j, NCk - 1));
    const EpiIn ep = epi_load<E>(a, nn, nrow, which, tl, Bv);
    stage_rows<MODE, RC, XCH, T>(a, xs, red, t);
    __syncthreads();
    float acc[RC];
    gemv_dots<NCH, RC, TEAM>(wr, xs, tl, K, acc);
    // epilogue: lane tl = r of each team handles row r
    float v = 0.0f;
#pragma unroll
    for (int r = 0; r < RC; r++)
        if (tl == r) v = acc[r];
    const int r = tl;
    if (E == E_QKV) {
        // the rotary pair (2i, 2i+1) is (team 0, team 1) of this wave: D and 2W are even
        const float e = rb(v + ep.b);
        const float other = lane_xor32(e, lane);
        if (r >= R || n >= a.N) return;
        float o = e;
        if (which < 2) {
            // four separate f32 products (MLX evaluates mul, then sub/add)
            const float ev = team == 0 ? e : other, od = team == 0 ? other : e;
            const float p = ev * ep.cs, q = od * ep.sn, s2 = ev * ep.sn, u = od * ep.cs;
            o = team == 0 ? p - q : s2 + u;
        }
        gst(a.out + ((size_t)which * R + r) * a.D + nrow, f2bf(o));
        return;
    }
    if (E == E_CFM) {
        // every lane of the team holds both rows' sums: row 0 cond, row 1 uncond
        if (tl != 0 || n >= a.N) return;
        const float pc = rb(acc[0] + ep.b), pn = rb(acc[RC > 1 ? 1 : 0] + ep.b);
        const float f0 = rb(pc + rb(rb(pc - pn) * rb(a.cfg)));
        float y = rb(ep.y + rb(ep.dt * f0));
        if (a.shift != 0.0f) y = rb(y + rb(rb(rb(a.shift) * ep.sq) * ep.sde));
        gst(a.y_out + n, f2bf(y));
        return;
    }
    if (E == E_CFMF) {
        // lane tl < F: frame tl, rows tl (cond) and F + tl (uncond)
        float vc = 0.0f, vu = 0.0f;
#pragma unroll
        for (int q = 0; q < RC; q++) {
            if (tl == q) vc = acc[q];
            if (tl + a.F == q) vu = acc[q];
        }
        if (tl >= a.F || n >= a.N) return;
        const float pc = rb(vc + ep.b), pn = rb(vu + ep.b);
        const float f0 = rb(pc + rb(rb(pc - pn) * rb(a.cfg)));
        float y = rb(ep.y + rb(ep.dt * f0));
        if (a.shift != 0.0f) y = rb(y + rb(rb(rb(a.shift) * ep.sq) * ep.sde));
        gst(a.y_out + (size_t)tl * a.N + n, f2bf(y));
        return;
    }
    if (E == E_STOP) {
        // lane 0 holds logit 0 (bias 0), lane 32 logit 1 (bias 1)
        const float x = rb(v + ep.b);
        const float x1 = lane_xor32(x, lane);
        if (vb != 0 || wave != 0 || lane != 0) return;
        const float m = fmaxf(x, x1), e0 = exp_rep(x - m), e1 = exp_rep(x1 - m);
        gst(a.p_out, e1 / (e0 + e1));
        if (a.flags_in)
            for (int i = 0; i < 3; i++) gst(reinterpret_cast<int32_t*>(a.p_out) + 1 + i, gld(a.flags_in + i));
        return;
    }
    if (r >= R || n >= a.N) return;
    const float e = rb(v + ep.b);
    if (E == E_BIAS) {
        gst(a.out + r * a.ostride + n, f2bf(e));
    } else if (E == E_RES) {
        gst(a.out + r * a.ostride + n, f2bf(ep.res + e));
    } else if (E == E_GATE) {
        gst(a.out + r * a.ostride + n, f2bf(ep.res + rb(ep.gate * e)));
    } else if (E == E_PATCH) {
        const uint16_t xe = f2bf(e);
        gst(a.out + (size_t)r * a.N + n, xe);
        gst(a.out + (size_t)(R + r) * a.N + n, xe);
    } else if (E == E_GELU) {
        gst(a.out + r * a.ostride + n, f2bf(gelu_chain(e)));
    } else if (E == E_SILU) {
        gst(a.out + r * a.ostride + n, f2bf(e * rb(1.0f / (1.0f + exp_rep(-e)))));
    } else if (E == E_CFMROWS) {
        // rows [t_emb + c_emb, x_emb(hist), x_emb(y)] of both CFG halves
        const uint16_t xe = f2bf(e);
        gst(a.out + n, f2bf(ep.te0 + ep.ce0));
        gst(a.out + (size_t)a.N + n, ep.xh);
        gst(a.out + (size_t)2 * a.N + n, xe);
        gst(a.out + (size_t)3 * a.N + n, f2bf(ep.te1 + ep.ce1));
        gst(a.out + (size_t)4 * a.N + n, ep.xh);
        gst(a.out + (size_t)5 * a.N + n, xe);
    }
}

template <int E, int MODE, int NCH, int W, int RC, int RPW>
__global__ __launch_bounds__(64 * W) void dit_gemv_kernel(DitGemv a) {
    extern __shared__ uint32_t xs[];
    __shared__ float red[W * kMaxSlots];
    gemv_body<E, MODE, NCH, W, RC, RPW>(a, blockIdx.x, xs, red);
}

// The three one-row GEMVs that sit between an LM step and the next flow-head
// sample, in one launch: c_emb(z) (row 0 of the flow head's c_emb rows;
// workgroups [0, nc)), x_emb(hist) ([nc, nc + nx)) and the stop head on z
// (the last workgroup) -- each workgroup runs the body that its own launch
// would (two waves, rows of 32 lanes, chunks by K), so the same bits.
template <int NCHC, int NCHX>
__global__ __launch_bounds__(128) void dit_pre_kernel(DitGemv c, DitGemv x, DitGemv s, int nc, int nx) {
    extern __shared__ uint32_t xs[];
    __shared__ float red[2 * kMaxSlots];
    const int b = blockIdx.x;
    if (b < nc)
        gemv_body<E_BIAS, M_PLAIN, NCHC, 2, 1, 2>(c, b, xs, red);
    else if (b < nc + nx)
        gemv_body<E_BIAS, M_PLAIN, NCHX, 2, 1, 2>(x, b - nc, xs, red);
    else
        gemv_body<E_STOP, M_PLAIN, NCHC, 2, 1, 2>(s, 0, xs, red);
}

// adaLN conditions of every Euler step and CFG half: out [steps][2][D] =
// silu(bf16(te[s][b] + ce[b])) with each op rounded (silu = x * sigmoid(x)).
__global__ __launch_bounds__(256) void adaln_cond_kernel(const uint16_t* te, const uint16_t* ce, int steps, int D,
                                                         uint16_t* out) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i >= steps * 2 * D) return;
    const float v = rb(bf2f(gld(te + i)) + bf2f(gld(ce + i % (2 * D))));
    const float sg = rb(1.0f / (1.0f + exp_rep(-v)));
    gst(out + i, f2bf(v * sg));
}

// Attention of one (sequence, head) over its L positions on the wave, lane d
// holding dimension d of q, k and v (lanes past head_dim: on = false, adding
// zeros): scores sum_d (q/8) k in f32 (wave sums), p = exp(s - max),
// l = sum p, o[i] = (sum_j p_j v_j) / l, to be rounded once by the caller.
__device__ __forceinline__ void attn_math(const float (&qv)[kMaxL], const float (&kv)[kMaxL],
                                          const float (&vv)[kMaxL], int L, bool on, float (&o)[kMaxL]) {
    const float scale = 1.0f / 8.0f;
#pragma unroll
    for (int i = 0; i < kMaxL; i++)
        if (i < L) {
            const float qd = on ? scale * qv[i] : 0.0f;
            float sc[kMaxL], m = -INFINITY;
#pragma unroll
            for (int j = 0; j < kMaxL; j++)
                if (j < L) {
                    sc[j] = team_sum<kWave>(qd * kv[j]);
                    m = fmaxf(m, sc[j]);
                }
            float l = 0.0f, acc = 0.0f;
#pragma unroll
            for (int j = 0; j < kMaxL; j++)
                if (j < L) {
                    const float p = exp_rep(sc[j] - m);
                    l += p;
                    acc += p * vv[j];
                }
            o[i] = acc / l;
        }
}

// Attention over the L positions of each sequence, one wave per (sequence,
// head), lane d owning dimension d: every q/k/v load is issued first, then
// attn_math, each output rounded once.
__global__ __launch_bounds__(kWave) void dit_attn_kernel(const uint16_t* qkv, int R, int L, int D, int heads,
                                                         int hd, uint16_t* att) {
    const int b = blockIdx.x / heads, h = blockIdx.x % heads, d = threadIdx.x, dd = min(d, hd - 1);
    const bool on = d < hd;
    const uint16_t* q = qkv + (size_t)(b * L) * D + h * hd + dd;
    const uint16_t* k = q + (size_t)R * D;
    const uint16_t* v = q + (size_t)2 * R * D;
    float qv[kMaxL], kv[kMaxL], vv[kMaxL];
#pragma unroll
    for (int i = 0; i < kMaxL; i++)
        if (i < L) {
            qv[i] = bf2f(gld(q + (size_t)i * D));
            kv[i] = bf2f(gld(k + (size_t)i * D));
            vv[i] = bf2f(gld(v + (size_t)i * D));
        }
    float o[kMaxL];
    attn_math(qv, kv, vv, L, on, o);
#pragma unroll
    for (int i = 0; i < kMaxL; i++)
        if (i < L && on) gst(att + (size_t)(b * L + i) * D + h * hd + d, f2bf(o[i]));
}

template <int E, int MODE, int W, int RC, int RPW>
hipError_t launch_wr(hipStream_t st, const DitGemv& a) {
    constexpr int ROWS = RPW * W, TEAM = kWave / RPW;
    const int grid = (a.N + ROWS - 1) / ROWS;
    const size_t lds = sizeof(uint32_t) * (size_t)RC * (a.K / 2);
    if (a.K <= 8 * TEAM)
        hipLaunchKernelGGL((dit_gemv_kernel<E, MODE, 1, W, RC, RPW>), dim3(grid), dim3(64 * W), lds, st, a);
    else if (a.K <= 32 * TEAM)
        hipLaunchKernelGGL((dit_gemv_kernel<E, MODE, 4, W, RC, RPW>), dim3(grid), dim3(64 * W), lds, st, a);
    else
        hipLaunchKernelGGL((dit_gemv_kernel<E, MODE, 4096 / (8 * TEAM), W, RC, RPW>), dim3(grid), dim3(64 * W),
                           lds, st, a);
    return hipGetLastError();
}

// Row slots.  Reference-shape stages: 1, 2 or 6 (3..6 rows run in 6 slots);
// adaLN stages: 2 or 8; the modulation GEMV (bias epilogue, plain rows) also
// 20.  Only the sets a stage uses are compiled.
template <int E, int MODE, int W, int RPW>
hipError_t launch_rc(hipStream_t st, const DitGemv& a) {
    constexpr bool kAda = MODE == M_ADANORM || E == E_GATE || E == E_CFMF || E == E_PATCH;
    if constexpr (kAda) {
        if (a.R <= 2) return launch_wr<E, MODE, W, 2, RPW>(st, a);
        return launch_wr<E, MODE, W, 8, RPW>(st, a);
    } else {
        if (E == E_CFM) return launch_wr<E, MODE, W, 2, RPW>(st, a);
        if (a.R == 1) return launch_wr<E, MODE, W, 1, RPW>(st, a);
        if (a.R == 2) return launch_wr<E, MODE, W, 2, RPW>(st, a);
        if constexpr (E == E_BIAS && MODE == M_PLAIN)
            if (a.R > kMaxR) return launch_wr<E, MODE, W, kMaxSlots, RPW>(st, a);
        return launch_wr<E, MODE, W, kMaxR, RPW>(st, a);
    }
}

// Long rows (K > 1024) get a whole wave each, shorter ones a half wave.
template <int E, int MODE, int W>
hipError_t launch_w(hipStream_t st, const DitGemv& a) {
    constexpr bool kPairs = E == E_QKV || E == E_STOP || E == E_CFMF;
    if constexpr (!kPairs)
        if (a.K > 1024) return launch_rc<E, MODE, W, 1>(st, a);
    return launch_rc<E, MODE, W, 2>(st, a);
}

// Four-wave workgroups when that still gives >= 256 of them (one per CU),
// else two-wave ones: N = 1024 runs as 256 workgroups of 4 rows (long rows:
// 4 waves of one row each).
template <int E, int MODE>
hipError_t launch_gemv(hipStream_t st, const DitGemv& a) {
    constexpr bool kPairs = E == E_QKV || E == E_STOP || E == E_CFMF;
    if (!kPairs && a.K > 1024) return launch_w<E, MODE, 4>(st, a);
    return (a.N + 7) / 8 >= 256 ? launch_w<E, MODE, 4>(st, a) : launch_w<E, MODE, 2>(st, a);
}

__host__ __device__ DitGemv gemv_args(const uint16_t* x, int R, const uint16_t* w, int N, int K, const uint16_t* bias, uint16_t* out) {
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

// ---- attention + out_proj in one launch (one sequence of two rows) ------------------
// The aggregator's blocks (one sequence, L = 2) run stage B without the
// attention launch before it: each out_proj workgroup of four waves computes
// the attention of every head itself (heads wave, wave + 4, ...: attn_math,
// the attention kernel's arithmetic, rounded once, so the same bits) into
// its staged rows, then the E_RES stage as dit_gemv_kernel computes it (rows
// of 32 lanes, chunk split and dot order by K alone: plain staged rows make
// the bits independent of the workgroup's width).  Eight launches fewer per
// aggregate; a workgroup's attention work (16 heads x 2 rows) is a few
// hundred cycles.
constexpr int kAoW = 4;  // waves per workgroup

template <int NCH>
__global__ __launch_bounds__(64 * kAoW) void dit_attn_out_kernel(DitGemv a) {
    constexpr int RPW = 2, TEAM = kWave / RPW, ROWS = RPW * kAoW, RC = 2;
    extern __shared__ uint32_t xs[];  // [2][D/2] the attention rows
    const int t = threadIdx.x, wave = t / kWave, lane = t % kWave, team = lane / TEAM, tl = lane % TEAM;
    const int D = a.K, NCk = D / 8, hd = a.hd, heads = D / hd;
    const int n = blockIdx.x * ROWS + wave * RPW + team, nn = min(n, a.N - 1);
    uint4 wr[NCH];
    const uint16_t* wrow = a.w + (size_t)nn * D;
#pragma unroll
    for (int j = 0; j < NCH; j++) wr[j] = ldg4(wrow + 8 * min(tl + TEAM * j, NCk - 1));
    const EpiIn ep = epi_load<E_RES>(a, nn, nn, 0, tl, a.bias);
    // q, k, v of rows 0 and 1 at a.x = qkv [3][2][D]; waves past the last head repeat it (not stored)
    const int d = lane, dd = min(d, hd - 1);
    float o[kMaxH][kMaxL];
#pragma unroll
    for (int k = 0; k < kMaxH; k++) {
        const int h = min(wave + kAoW * k, heads - 1);
        float qv[kMaxL], kv[kMaxL], vv[kMaxL];
#pragma unroll
        for (int i = 0; i < 2; i++) {
            const uint16_t* p = a.x + (size_t)i * D + h * hd + dd;
            qv[i] = bf2f(gld(p));
            kv[i] = bf2f(gld(p + (size_t)2 * D));
            vv[i] = bf2f(gld(p + (size_t)4 * D));
        }
        attn_math(qv, kv, vv, 2, d < hd, o[k]);
    }
    uint16_t* xh = reinterpret_cast<uint16_t*>(xs);
#pragma unroll
    for (int k = 0; k < kMaxH; k++) {
        const int h = wave + kAoW * k;
        if (h < heads && d < hd)
#pragma unroll
            for (int i = 0; i < 2; i++) xh[i * D + h * hd + d] = f2bf(o[k][i]);
    }
    __syncthreads();
    float acc[RC];
    gemv_dots<NCH, RC, TEAM>(wr, xs, tl, D, acc);
    float v = 0.0f;
#pragma unroll
    for (int r = 0; r < RC; r++)
        if (tl == r) v = acc[r];
    const int r = tl;
    if (r >= 2 || n >= a.N) return;
    gst(a.out + r * a.ostride + n, f2bf(ep.res + rb(v + ep.b)));
}

// Stage A's GEMV: rms1 + q/k/v + bias + rotary of R rows (sequences of L) -> qkv [3][R][D].
hipError_t launch_dit_qkv(hipStream_t st, const DitBlockDev& w, const uint16_t* x, int R, int L, const float* cos_t,
                          const float* sin_t, uint16_t* qkv) {
    const int D = w.D;
    DitGemv a = gemv_args(x, R, nullptr, 3 * D, D, nullptr, qkv);
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
    return launch_gemv<E_QKV, M_NORM>(st, a);
}

// Attention + out_proj + residual of one sequence of two rows (dit_attn_out_kernel), where its
// shape allows: hidden <= 1024 in chunks of 8, at most 16 heads of at most 64.
bool attn_out_fits(const DitBlockDev& w) {
    return w.D <= 1024 && w.D % 8 == 0 && w.hd >= 1 && w.hd <= kWave && w.D % w.hd == 0 && w.D / w.hd <= kAoW * kMaxH;
}

hipError_t launch_attn_out(hipStream_t st, const DitBlockDev& w, const uint16_t* qkv, const uint16_t* x,
                           uint16_t* out) {
    const int D = w.D;
    DitGemv a = gemv_args(qkv, 2, w.wo, D, D, w.bo, out);
    a.res = x;
    a.hd = w.hd;
    const int grid = (D + 2 * kAoW - 1) / (2 * kAoW);
    const size_t lds = sizeof(uint32_t) * (size_t)D;  // two rows of D bf16
    if (D <= 8 * (kWave / 2))
        hipLaunchKernelGGL(dit_attn_out_kernel<1>, dim3(grid), dim3(64 * kAoW), lds, st, a);
    else
        hipLaunchKernelGGL(dit_attn_out_kernel<4>, dim3(grid), dim3(64 * kAoW), lds, st, a);
    return hipGetLastError();
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
            hipError_t e = launch_dit_qkv(st, w, x, R, L, cos_t, sin_t, qkv);
            if (e != hipSuccess) return e;
            hipLaunchKernelGGL(dit_attn_kernel, dim3(B * w.heads), dim3(kWave), 0, st, qkv, R, L, D, w.heads, w.hd,
                               out);
            return hipGetLastError();
        }
        case 1:
            a = gemv_args(in, R, w.wo, D, D, w.bo, out);
            a.res = x;
            return launch_gemv<E_RES, M_PLAIN>(st, a);
        case 2:
            a = gemv_args(x, R, w.w1, F, D, w.b1, out);
            a.norm = w.norm2;
            a.eps = w.eps;
            return launch_gemv<E_GELU, M_NORM>(st, a);
        default:
            a = gemv_args(in, R, w.w2, D, F, w.b2, out);
            a.res = x;
            return launch_gemv<E_RES, M_PLAIN>(st, a);
    }
}

// Attention of B sequences of L rows on qkv [3][B L][D] (one wave per (sequence, head)).
hipError_t launch_dit_attn(hipStream_t st, const uint16_t* qkv, int B, int L, int D, int heads, int hd, uint16_t* att) {
    if (L > kMaxL) return hipErrorInvalidValue;
    hipLaunchKernelGGL(dit_attn_kernel, dim3(B * heads), dim3(kWave), 0, st, qkv, B * L, L, D, heads, hd, att);
    return hipGetLastError();
}

// One DiT block: the four stages in order.  fuse_attn: for one sequence of
// two rows, attention and out_proj in one launch where the shape allows
// (dit_attn_out_kernel: the same bits; att is then not written).
hipError_t launch_dit_block(hipStream_t st, const DitBlockDev& w, const uint16_t* x, int B, int L,
                            const float* cos_t, const float* sin_t, uint16_t* qkv, uint16_t* att, uint16_t* x1,
                            uint16_t* hh, uint16_t* x2, bool fuse_attn) {
    hipError_t e;
    if (fuse_attn && B == 1 && L == 2 && attn_out_fits(w)) {
        if ((e = launch_dit_qkv(st, w, x, 2, 2, cos_t, sin_t, qkv)) != hipSuccess) return e;
        if ((e = launch_attn_out(st, w, qkv, x, x1)) != hipSuccess) return e;
    } else {
        if ((e = launch_dit_stage(st, 0, w, x, nullptr, B, L, cos_t, sin_t, qkv, att)) != hipSuccess) return e;
        if ((e = launch_dit_stage(st, 1, w, x, att, B, L, cos_t, sin_t, qkv, x1)) != hipSuccess) return e;
    }
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
    if (norm) return silu ? launch_gemv<E_SILU, M_NORM>(st, a) : launch_gemv<E_BIAS, M_NORM>(st, a);
    return silu ? launch_gemv<E_SILU, M_PLAIN>(st, a) : launch_gemv<E_BIAS, M_PLAIN>(st, a);
}

// fused.embed: rows [2*3][D] = [te + ce, xh, x_emb(y)] per CFG half.
hipError_t launch_cfm_embed(hipStream_t st, const uint16_t* y, const uint16_t* wx, const uint16_t* bx, int D, int latent,
                            const uint16_t* te, const uint16_t* ce, const uint16_t* xh, uint16_t* rows) {
    DitGemv a = gemv_args(y, 1, wx, D, latent, bx, rows);
    a.te = te;
    a.ce = ce;
    a.xh = xh;
    return launch_gemv<E_CFMROWS, M_PLAIN>(st, a);
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
    return launch_gemv<E_CFM, M_NORM>(st, a);
}

// ---- adaLN flow head (config 4) -----------------------------------------------------

// One stage of an adaLN block on x [R][D] (R = B*L, half b = rows [bL, bL + L)),
// mod [B][6D] = [shift_a, scale_a, gate_a, shift_m, scale_m, gate_m] per half:
//   0  modulate(rms1(x)) -> q/k/v + rotary -> qkv, attention -> out
//   1  out = bf16(x + bf16(gate_a * out_proj(in)))
//   2  out = gelu(ff1(modulate(rms2(x))))
//   3  out = bf16(x + bf16(gate_m * ff2(in)))
hipError_t launch_adaln_stage(hipStream_t st, int which, const DitBlockDev& w, const uint16_t* mod, const uint16_t* x,
                              const uint16_t* in, int B, int L, const float* cos_t, const float* sin_t, uint16_t* qkv,
                              uint16_t* out) {
    const int R = B * L, D = w.D, F = w.F;
    DitGemv a;
    switch (which) {
        case 0:
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
            a.soff = 0;
            a.coff = 1;
            break;
        case 1:
            a = gemv_args(in, R, w.wo, D, D, w.bo, out);
            a.res = x;
            a.goff = 2;
            break;
        case 2:
            a = gemv_args(x, R, w.w1, F, D, w.b1, out);
            a.norm = w.norm2;
            a.eps = w.eps;
            a.soff = 3;
            a.coff = 4;
            break;
        default:
            a = gemv_args(in, R, w.w2, D, F, w.b2, out);
            a.res = x;
            a.goff = 5;
            break;
    }
    a.mod = mod;
    a.mstride = 6 * (int64_t)D;
    a.rph = L;
    switch (which) {
        case 0: {
            hipError_t e = launch_gemv<E_QKV, M_ADANORM>(st, a);
            if (e != hipSuccess) return e;
            hipLaunchKernelGGL(dit_attn_kernel, dim3(B * w.heads), dim3(kWave), 0, st, qkv, R, L, D, w.heads, w.hd,
                               out);
            return hipGetLastError();
        }
        case 1:
            return launch_gemv<E_GATE, M_PLAIN>(st, a);
        case 2:
            return launch_gemv<E_GELU, M_ADANORM>(st, a);
        default:
            return launch_gemv<E_GATE, M_PLAIN>(st, a);
    }
}

hipError_t launch_adaln_block(hipStream_t st, const DitBlockDev& w, const uint16_t* mod, const uint16_t* x, int B,
                              int L, const float* cos_t, const float* sin_t, uint16_t* qkv, uint16_t* att, uint16_t* x1,
                              uint16_t* hh, uint16_t* x2) {
    hipError_t e;
    if ((e = launch_adaln_stage(st, 0, w, mod, x, nullptr, B, L, cos_t, sin_t, qkv, att)) != hipSuccess) return e;
    if ((e = launch_adaln_stage(st, 1, w, mod, x, att, B, L, cos_t, sin_t, qkv, x1)) != hipSuccess) return e;
    if ((e = launch_adaln_stage(st, 2, w, mod, x1, nullptr, B, L, cos_t, sin_t, qkv, hh)) != hipSuccess) return e;
    return launch_adaln_stage(st, 3, w, mod, x1, hh, B, L, cos_t, sin_t, qkv, x2);
}

hipError_t launch_adaln_cond(hipStream_t st, const uint16_t* te, const uint16_t* ce, int steps, int D, uint16_t* out) {
    const int n = steps * 2 * D;
    hipLaunchKernelGGL(adaln_cond_kernel, dim3((n + 255) / 256), dim3(256), 0, st, te, ce, steps, D, out);
    return hipGetLastError();
}

// Input rows of a patch: rows [2][F][D] = x_emb(y_f) for both halves; y [F][latent].
hipError_t launch_adaln_rows(hipStream_t st, const uint16_t* y, int F, const uint16_t* wx, const uint16_t* bx, int D,
                             int latent, uint16_t* rows) {
    DitGemv a = gemv_args(y, F, wx, D, latent, bx, rows);
    return launch_gemv<E_PATCH, M_PLAIN>(st, a);
}

// Final adaLN layer on h [2F][D]: modulate(rms(h)) with mod [2][2D] = [shift | scale]
// per half, linear to the latent, CFG + Euler (+ SDE) per frame: y [F][latent] -> y_out.
hipError_t launch_adaln_final(hipStream_t st, const uint16_t* h, int F, int D, const uint16_t* norm, float eps,
                              const uint16_t* mod, const uint16_t* wf, const uint16_t* bf, int latent, const uint16_t* y,
                              const uint16_t* dt, const uint16_t* sq, const uint16_t* sde, int step, float cfg,
                              float shift, uint16_t* y_out) {
    DitGemv a = gemv_args(h, 2 * F, wf, latent, D, bf, nullptr);
    a.norm = norm;
    a.eps = eps;
    a.mod = mod;
    a.mstride = 2 * (int64_t)D;
    a.rph = F;
    a.soff = 0;
    a.coff = 1;
    a.F = F;
    a.y = y;
    a.dt = dt;
    a.sq = sq;
    a.sde = sde;
    a.step = step;
    a.cfg = cfg;
    a.shift = shift;
    a.y_out = y_out;
    return launch_gemv<E_CFMF, M_ADANORM>(st, a);
}

// stopProb: p = softmax(f32(bf16(W z + b)))[1] (W [2][K]).
hipError_t launch_stop_prob(hipStream_t st, const uint16_t* z, const uint16_t* w, const uint16_t* b, int K, float* p,
                            const int32_t* flags_in) {
    DitGemv a = gemv_args(z, 1, w, 2, K, b, nullptr);
    a.p_out = p;
    a.flags_in = flags_in;
    return launch_gemv<E_STOP, M_PLAIN>(st, a);
}

// c_emb(z) -> ce row 0, x_emb(hist) -> xh and the stop head on z -> p_out (with the error flags
// beside it when flags_in is set) as one launch where the shapes allow it (z of 256 < K <= 1024,
// hist of K <= 256, hidden < 2041, all 16-byte aligned); false: the caller launches them apart.
bool launch_cfm_pre(hipStream_t st, const uint16_t* z, int H, const uint16_t* wc, const uint16_t* bc, int D,
                    uint16_t* ce, const uint16_t* hist, int lat, const uint16_t* wx, const uint16_t* bx, uint16_t* xh,
                    const uint16_t* ws, const uint16_t* bs, float* p_out, const int32_t* flags_in, hipError_t* err) {
    auto al = [](const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; };
    if (H <= 256 || H > 1024 || H % 8 || lat < 8 || lat > 256 || lat % 8 || (D + 7) / 8 >= 256 || !al(z) || !al(hist))
        return false;
    DitGemv c = gemv_args(z, 1, wc, D, H, bc, ce);
    DitGemv x = gemv_args(hist, 1, wx, D, lat, bx, xh);
    DitGemv s = gemv_args(z, 1, ws, 2, H, bs, nullptr);
    s.p_out = p_out;
    s.flags_in = flags_in;
    const int nb = (D + 3) / 4;  // rows of two waves x 2
    const size_t lds = sizeof(uint32_t) * (size_t)(H / 2);
    hipLaunchKernelGGL((dit_pre_kernel<4, 1>), dim3(2 * nb + 1), dim3(128), lds, st, c, x, s, nb, nb);
    *err = hipGetLastError();
    return true;
}

hipError_t tanh_upload_dit(const float* host) {
    return hipMemcpyToSymbol(HIP_SYMBOL(dit_tanh_tab), host, sizeof(float) * kTanhTabN);
}

const float* tanh_table_host() {
    static const std::vector<float> tab = [] {
        std::vector<float> t(kTanhTabN);
        for (int h = 0; h < kTanhTabN; h++) {
            const uint32_t bits = (uint32_t)h << 16;
            float u;
            std::memcpy(&u, &bits, sizeof u);
            t[h] = (float)std::tanh((double)u);
        }
        return t;
    }();
    return tab.data();
}

hipError_t tanh_tables_init(int device) {
    static std::mutex mu;
    static std::vector<int> done;  // devices whose arrays are filled
    std::lock_guard<std::mutex> lock(mu);
    for (int d : done)
        if (d == device) return hipSuccess;
    const float* t = tanh_table_host();
    hipError_t e = tanh_upload_dit(t);
    if (e == hipSuccess) e = tanh_upload_dit_batch(t);
    if (e == hipSuccess) e = tanh_upload_cfmp(t);
    if (e == hipSuccess) e = hipDeviceSynchronize();
    if (e == hipSuccess) done.push_back(device);
    return e;
}

}  // namespace ming
