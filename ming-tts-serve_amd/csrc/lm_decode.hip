// Qwen2 decode step for gfx950: the reference's five fused layer kernels
// LA..LE (src/ming_fused.zig:296-399), rebuilt for 64-wide wavefronts, with
// the KV cache written in place, split-K GQA attention for long contexts, and
// the tied LM head with a greedy argmax.
//
// Each GEMV stage is split into three device functions: `load` issues one
// wave's weight loads into registers, `prepare` stages the activation vector
// in LDS (and normalises it), `compute` finishes the dot products and the
// epilogue.  A workgroup loads its first unit's weights before `prepare`, so
// the HBM latency of the weights overlaps the normalisation, and prefetches
// the next unit while computing the current one.  This file is the per-stage
// schedule (one kernel per stage, the reference's schedule, used by
// ming_lm_layer and by ming_lm_step in MING_LM_KERNELS mode); the one-kernel
// schedule with tagged hand-offs is in lm_persistent.hip.
//
// Numerics follow the MLX graph (src/ming_model.zig:588-611): h =
// rms_norm(x) is rounded to bf16 before the q/k/v and gate/up products, every
// linear output is rounded to bf16, the residual adds round once more, rope
// and swiglu round like the reference (src/ming_fused.zig:296-324, :384-394),
// attention scores and softmax are f32 with the output rounded once.
#include "gemv.h"
#include "internal.h"

namespace ming {

namespace {

constexpr int kBlock = 256;
constexpr int kWpb = kBlock / kWave;  // waves per block
constexpr int kLdsWords = 8192;       // 32 KB static LDS per workgroup
constexpr int kHOff = 4608;           // bf16 temp (rms output), up to 2048 values
constexpr int kRedOff = 5632;         // block reduction scratch
constexpr int kTile = 64;             // attention positions per LDS tile
constexpr int kMaxSplit = 256;        // attention positions per split

// Chunks per lane held in registers (32- and 64-lane teams): one batch covers
// a whole row of the Qwen2-0.5B shapes (K = 896 or 4864).
template <int Q4>
struct Nch {
    static constexpr int t32 = Q4 ? 1 : 4;
    static constexpr int t64 = Q4 ? 3 : 5;
};

enum Stage { S_EMBED, S_QKV, S_ATTN, S_MERGE, S_O, S_UP, S_DOWN, S_HEAD, S_ARGMAX, S_FINAL };

__device__ __forceinline__ XStage xstage(uint32_t* lds, int K) { return XStage{lds, reinterpret_cast<float*>(lds + K / 2)}; }
__device__ __forceinline__ uint16_t* htemp(uint32_t* lds) { return reinterpret_cast<uint16_t*>(lds + kHOff); }
__device__ __forceinline__ float* red(uint32_t* lds) { return reinterpret_cast<float*>(lds + kRedOff); }

__device__ __forceinline__ int attn_nsplit(const StepArgs& a) { return (a.pos + 1 + a.split_len - 1) / a.split_len; }

// MLX fast::rms_norm of x [H] into LDS: bf16(w * bf16(x * rsqrt(mean(x^2) + eps))).
__device__ void rms_to_lds(const uint16_t* x, const uint16_t* w, int H, float eps, uint16_t* h, float* rd) {
    float ss = 0.0f;
    for (int i = threadIdx.x; i < H; i += blockDim.x) {
        const float v = bf2f(x[i]);
        ss += v * v;
    }
    ss = block_sum(ss, rd);
    const float inv = 1.0f / sqrtf(ss / (float)H + eps);
    for (int i = threadIdx.x; i < H; i += blockDim.x) h[i] = f2bf(bf2f(w[i]) * rb(bf2f(x[i]) * inv));
    __syncthreads();
}

__host__ __device__ __forceinline__ int units_of(Stage s, int H, int kvh, int hd, int heads, int I, int V, int n_attn) {
    switch (s) {
        case S_EMBED: return 1;
        case S_QKV: return ((H + 2 * kvh * hd) / 2 + kWpb - 1) / kWpb;
        case S_ATTN: return n_attn;
        case S_MERGE: return heads;
        case S_O: return (H + 2 * kWpb - 1) / (2 * kWpb);
        case S_UP: return (I + kWpb - 1) / kWpb;
        case S_DOWN: return (H + kWpb - 1) / kWpb;
        case S_HEAD: return (V + 2 * kWpb - 1) / (2 * kWpb);
        case S_ARGMAX: return 1;
        case S_FINAL: return 1;
    }
    return 1;
}

__device__ __forceinline__ int stage_units(Stage s, const StepArgs& a) {
    return units_of(s, a.H, a.kvh, a.hd, a.heads, a.I, a.head.N, a.kvh * attn_nsplit(a));
}

// ---- embed: x[0] = embed(token) ---------------------------------------------
__device__ void embed_unit(const StepArgs& a) {
    const LinearDev& E = a.embed;
    int id = *a.token_in;
    id = id < 0 ? 0 : (id >= E.N ? E.N - 1 : id);
    if (E.kind == 1) {
        const uint32_t* wr = E.w + (size_t)id * (E.K / 8);
        const uint16_t* sr = E.s + (size_t)id * (E.K / 64);
        const uint16_t* br = E.b + (size_t)id * (E.K / 64);
        for (int wi = threadIdx.x; wi < E.K / 8; wi += blockDim.x) {
            const float sc = bf2f(sr[wi / 8]), bi = bf2f(br[wi / 8]);
            const uint32_t word = wr[wi];
            uint32_t o[4];
#pragma unroll
            for (int p = 0; p < 4; p++) {
                float v0 = sc * (float)((word >> (8 * p)) & 0xfu) + bi;
                float v1 = sc * (float)((word >> (8 * p + 4)) & 0xfu) + bi;
                if (E.gscale != 1.0f) {
                    v0 *= E.gscale;
                    v1 *= E.gscale;
                }
                o[p] = pack_bf2(v0, v1);
            }
            *reinterpret_cast<uint4*>(a.x + 8 * wi) = make_uint4(o[0], o[1], o[2], o[3]);
        }
    } else {
        const uint16_t* row = reinterpret_cast<const uint16_t*>(E.w) + (size_t)id * E.K;
        for (int i = threadIdx.x; i < E.K / 8; i += blockDim.x)
            reinterpret_cast<uint4*>(a.x)[i] = reinterpret_cast<const uint4*>(row)[i];
    }
}

// ---- LA: rms(ln1) + q/k/v + bias + rope; k/v written into the cache at pos ----
// A wave owns one rope pair of rows (r, r + hd/2) of the concatenated
// [q | k | v] rows: team 0 the first, team 1 the second.
struct QkvRow {
    int r1, which, base;
};

__device__ __forceinline__ QkvRow qkv_row(const StepArgs& a, int u) {
    const int half = a.hd / 2, kvd = a.kvh * a.hd;
    const int pi = u * kWpb + threadIdx.x / kWave;
    QkvRow q;
    q.r1 = (pi / half) * a.hd + pi % half;
    q.which = pi >= (a.H + 2 * kvd) / 2 ? -1 : (q.r1 < a.H ? 0 : (q.r1 < a.H + kvd ? 1 : 2));
    q.base = q.which == 0 ? 0 : (q.which == 1 ? a.H : a.H + kvd);
    return q;
}

__device__ __forceinline__ const LinearDev& qkv_lin(const LayerDev& Ld, int which) {
    return which == 0 ? Ld.q : (which == 1 ? Ld.k : Ld.v);
}

template <int Q4>
__device__ void qkv_load(const StepArgs& a, const LayerDev& Ld, int u, RowRegs<Nch<Q4>::t32>& r) {
    const QkvRow q = qkv_row(a, u);
    if (q.which < 0) return;
    const int lane = threadIdx.x % kWave;
    row_load<Q4, 32, Nch<Q4>::t32>(qkv_lin(Ld, q.which), q.r1 - q.base + (lane / 32) * (a.hd / 2), lane % 32, 0, r);
}

template <int Q4>
__device__ void qkv_prepare(const StepArgs& a, const LayerDev& Ld, int l, uint32_t* lds) {
    uint16_t* h = htemp(lds);
    rms_to_lds(a.x + l * a.sx, Ld.ln1, a.H, a.eps, h, red(lds));
    stage_xk<Q4>(h, a.H, xstage(lds, a.H));
}

template <int Q4>
__device__ void qkv_compute(const StepArgs& a, const LayerDev& Ld, int l, uint32_t* lds, int u,
                            const RowRegs<Nch<Q4>::t32>& r) {
    const QkvRow q = qkv_row(a, u);
    if (q.which < 0) return;
    const int lane = threadIdx.x % kWave, half = a.hd / 2;
    const LinearDev& L = qkv_lin(Ld, q.which);
    const uint16_t* bias = q.which == 0 ? Ld.bq : (q.which == 1 ? Ld.bk : Ld.bv);
    const float acc = row_dot_pf<Q4, 32, Nch<Q4>::t32>(L, q.r1 - q.base + (lane / 32) * half, xstage(lds, a.H), lane % 32, r);
    const float v1 = __shfl(acc, 0, kWave), v2 = __shfl(acc, 32, kWave);
    if (lane != 0) return;
    const int lr = q.r1 - q.base;
    float e1, e2;
    if (Q4) {  // quantized_matmul, then + bias
        e1 = rb(rb(v1) + bf2f(bias[lr]));
        e2 = rb(rb(v2) + bf2f(bias[lr + half]));
    } else {            // addmm
        e1 = rb(v1 + bf2f(bias[lr]));
        e2 = rb(v2 + bf2f(bias[lr + half]));
    }
    if (q.which < 2) {  // MLX fast::rope, non-traditional: pair (d, d + hd/2)
        const int d = lr % a.hd;
        const float inv_freq = exp2f(-((float)d / (float)half) * a.log2_theta);
        const float th = (float)a.pos * inv_freq;
        const float c = cosf(th), s = sinf(th);
        const float o1 = e1 * c - e2 * s, o2 = e1 * s + e2 * c;
        e1 = rb(o1);
        e2 = rb(o2);
    }
    uint16_t* out = a.qkv + l * a.sq;
    out[q.r1] = f2bf(e1);
    out[q.r1 + half] = f2bf(e2);
    if (q.which > 0) {
        uint16_t* cache = q.which == 1 ? a.kc : a.vc;
        const int kh = lr / a.hd, d = lr % a.hd;
        uint16_t* dst = cache + (((size_t)l * a.kvh + kh) * a.cap + a.pos) * a.hd;
        dst[d] = f2bf(e1);
        dst[d + half] = f2bf(e2);
    }
}

// ---- LB: split-K GQA attention; one unit = (kv head, split of positions) ----
// The grp query heads sharing a kv head are processed together, so each K/V
// row is read once.  A split is walked in tiles of 64 positions staged in LDS
// with coalesced 16-byte loads (the next tile's loads are issued before the
// current tile is computed), with an online softmax across tiles.  The unit
// writes (max, sum, P.V) partials per head; MERGE combines the splits.
struct AttnLds {
    float* q;      // [8][64]   scaled q (f32)
    uint16_t* k;   // [64][64]  K tile
    uint16_t* v;   // [64][64]  V tile
    float* p;      // [8][64]   scores -> probabilities
    float* ml;     // [8][4]    running max, running sum, tile correction
};

__device__ __forceinline__ AttnLds attn_lds(uint32_t* lds) {
    AttnLds s;
    s.q = reinterpret_cast<float*>(lds);
    s.k = reinterpret_cast<uint16_t*>(lds + 512);
    s.v = reinterpret_cast<uint16_t*>(lds + 512 + 2048);
    s.p = reinterpret_cast<float*>(lds + 512 + 4096);
    s.ml = reinterpret_cast<float*>(lds + 512 + 4096 + 512);
    return s;
}

__device__ void attn_unit(const StepArgs& a, int l, uint32_t* lds, int u) {
    const int ns = attn_nsplit(a), n = a.pos + 1, grp = a.heads / a.kvh, hd = a.hd;
    const int g = u / ns, sp = u % ns;
    const int j0 = sp * a.split_len, j1 = min(n, j0 + a.split_len);
    const AttnLds S = attn_lds(lds);
    const int t = threadIdx.x, wave = t / kWave, lane = t % kWave;
    const float scale = 1.0f / sqrtf((float)hd);
    const uint16_t* q = a.qkv + l * a.sq + (size_t)g * grp * hd;
    for (int i = t; i < grp * hd; i += blockDim.x) S.q[i] = scale * bf2f(q[i]);
    if (t < 8 * 4) S.ml[t] = (t % 4 == 0) ? -INFINITY : 0.0f;
    const uint16_t* kbase = a.kc + (((size_t)l * a.kvh + g) * a.cap) * hd;
    const uint16_t* vbase = a.vc + (((size_t)l * a.kvh + g) * a.cap) * hd;
    // tile loads: 64 rows x 128 B = 512 x 16 B for K and for V; two of each per thread
    uint4 kr[2], vr[2];
    auto load_tile = [&](int t0) {
#pragma unroll
        for (int i = 0; i < 2; i++) {
            const int idx = t + i * kBlock, row = idx / 8, col = idx % 8;
            if (t0 + row < j1) {
                kr[i] = ldg4(kbase + (size_t)(t0 + row) * hd + 8 * col);
                vr[i] = ldg4(vbase + (size_t)(t0 + row) * hd + 8 * col);
            } else {
                kr[i] = make_uint4(0, 0, 0, 0);
                vr[i] = make_uint4(0, 0, 0, 0);
            }
        }
    };
    load_tile(j0);
    const int hs = t / 64, d = t % 64;  // P.V: thread owns dim d of heads hs, hs+4
    float acc0 = 0.0f, acc1 = 0.0f;
    for (int t0 = j0; t0 < j1; t0 += kTile) {
        const int cnt = min(kTile, j1 - t0);
        __syncthreads();  // previous tile fully consumed
#pragma unroll
        for (int i = 0; i < 2; i++) {
            const int idx = t + i * kBlock;
            reinterpret_cast<uint4*>(S.k)[idx] = kr[i];
            reinterpret_cast<uint4*>(S.v)[idx] = vr[i];
        }
        __syncthreads();
        if (t0 + kTile < j1) load_tile(t0 + kTile);
        // scores: thread = (position p, quarter qt of the head dim)
        {
            const int p = t >> 2, qt = t & 3;
            const uint4* kp = reinterpret_cast<const uint4*>(S.k + p * hd + qt * 16);
            const uint4 k0 = kp[0], k1 = kp[1];
            const uint32_t kw[8] = {k0.x, k0.y, k0.z, k0.w, k1.x, k1.y, k1.z, k1.w};
            for (int h = 0; h < grp; h++) {
                const float* qh = S.q + h * hd + qt * 16;
                float s = 0.0f;
#pragma unroll
                for (int i = 0; i < 8; i++) {
                    s += qh[2 * i] * bf_lo(kw[i]);
                    s += qh[2 * i + 1] * bf_hi(kw[i]);
                }
                s = team_sum<4>(s);
                if (qt == 0) S.p[h * kTile + p] = p < cnt ? s : -INFINITY;
            }
        }
        __syncthreads();
        // online softmax: wave w takes heads w, w+4; lane = position
        for (int h = wave; h < grp; h += kWpb) {
            const float s = S.p[h * kTile + lane];
            const float mt = team_max<kWave>(s);
            const float mo = S.ml[4 * h], mn = fmaxf(mo, mt);
            const float e = lane < cnt ? expf(s - mn) : 0.0f;
            S.p[h * kTile + lane] = e;
            const float sum = team_sum<kWave>(e);
            if (lane == 0) {
                const float corr = expf(mo - mn);  // exp(-inf) = 0 on the first tile
                S.ml[4 * h] = mn;
                S.ml[4 * h + 1] = S.ml[4 * h + 1] * corr + sum;
                S.ml[4 * h + 2] = corr;
            }
        }
        __syncthreads();
        if (hs < grp) {
            const float c0 = S.ml[4 * hs + 2];
            const bool h1 = hs + 4 < grp;
            const float c1 = h1 ? S.ml[4 * (hs + 4) + 2] : 0.0f;
            const float* p0 = S.p + hs * kTile;
            const float* p1 = S.p + (hs + 4) * kTile;
            float s0 = 0.0f, s1 = 0.0f;
            for (int p = 0; p < cnt; p++) {
                const float vv = bf2f(S.v[p * hd + d]);
                s0 += p0[p] * vv;
                if (h1) s1 += p1[p] * vv;
            }
            acc0 = acc0 * c0 + s0;
            acc1 = acc1 * c1 + s1;
        }
    }
    __syncthreads();
    if (hs < grp) {
        float* out = a.part + ((size_t)(g * ns + sp) * grp + hs) * (hd + 2);
        out[2 + d] = acc0;
        if (d == 0) {
            out[0] = S.ml[4 * hs];
            out[1] = S.ml[4 * hs + 1];
        }
        if (hs + 4 < grp) {
            float* out1 = a.part + ((size_t)(g * ns + sp) * grp + hs + 4) * (hd + 2);
            out1[2 + d] = acc1;
            if (d == 0) {
                out1[0] = S.ml[4 * (hs + 4)];
                out1[1] = S.ml[4 * (hs + 4) + 1];
            }
        }
    }
    __syncthreads();
}

// ---- merge of the split partials, one workgroup per query head -------------
// att[h] = sum_s e^(m_s - M) acc_s / sum_s e^(m_s - M) l_s.  Wave w takes the
// splits s = w, w + 4, ...; the waves' sums meet in LDS.
__device__ void merge_unit(const StepArgs& a, int l, uint32_t* lds, int h) {
    const int t = threadIdx.x, wave = t / kWave, lane = t % kWave;
    const int grp = a.heads / a.kvh, g = h / grp, hl = h % grp, ns = attn_nsplit(a), hd = a.hd;
    const float* base = a.part + ((size_t)(g * ns) * grp + hl) * (hd + 2);
    const size_t stride = (size_t)grp * (hd + 2);
    float* sm = reinterpret_cast<float*>(lds);  // [4][64] partial O, [8] scratch
    // M over all splits (lane-parallel)
    float m = -INFINITY;
    for (int s = lane; s < ns; s += kWave) m = fmaxf(m, base[s * stride]);
    const float M = team_max<kWave>(m);
    float Lw = 0.0f, O = 0.0f;
    for (int s = wave; s < ns; s += kWpb) {
        const float* p = base + s * stride;
        const float e = expf(p[0] - M);
        Lw += p[1] * e;
        O += p[2 + lane] * e;
    }
    sm[wave * 64 + lane] = O;
    if (lane == 0) sm[256 + wave] = Lw;
    __syncthreads();
    if (wave == 0) {
        const float Ls = (sm[256] + sm[257]) + (sm[258] + sm[259]);
        const float Os = (sm[lane] + sm[64 + lane]) + (sm[128 + lane] + sm[192 + lane]);
        a.att[l * a.sx + h * hd + lane] = f2bf(Os / Ls);
    }
    __syncthreads();
}

// ---- LC: o_proj + residual ----------------------------------------------------
template <int Q4>
__device__ void o_load(const StepArgs& a, const LayerDev& Ld, int u, RowRegs<Nch<Q4>::t32>& r) {
    const int lane = threadIdx.x % kWave, r0 = (u * kWpb + threadIdx.x / kWave) * 2;
    if (r0 >= a.H) return;
    row_load<Q4, 32, Nch<Q4>::t32>(Ld.o, min(r0 + lane / 32, a.H - 1), lane % 32, 0, r);
}

template <int Q4>
__device__ void o_prepare(const StepArgs& a, const LayerDev& Ld, int l, uint32_t* lds) {
    stage_xk<Q4>(a.att + l * a.sx, a.H, xstage(lds, a.H));
}

template <int Q4>
__device__ void o_compute(const StepArgs& a, const LayerDev& Ld, int l, uint32_t* lds, int u,
                          const RowRegs<Nch<Q4>::t32>& rr) {
    const int lane = threadIdx.x % kWave, r0 = (u * kWpb + threadIdx.x / kWave) * 2;
    if (r0 >= a.H) return;
    const int team = lane / 32, tl = lane % 32, r = min(r0 + team, a.H - 1);
    const float acc = row_dot_pf<Q4, 32, Nch<Q4>::t32>(Ld.o, r, xstage(lds, a.H), tl, rr);
    if (tl == 0 && r0 + team < a.H) {
        const int64_t i = l * a.sx + r;
        a.x1[i] = f2bf(bf2f(a.x[i]) + rb(acc));
    }
}

// ---- LD: rms(ln2) + gate/up + swiglu ------------------------------------------
template <int Q4>
__device__ void up_load(const StepArgs& a, const LayerDev& Ld, int u, RowRegs<Nch<Q4>::t32>& r) {
    const int lane = threadIdx.x % kWave, n = u * kWpb + threadIdx.x / kWave;
    if (n >= a.I) return;
    row_load<Q4, 32, Nch<Q4>::t32>(lane < 32 ? Ld.g : Ld.u, n, lane % 32, 0, r);
}

template <int Q4>
__device__ void up_prepare(const StepArgs& a, const LayerDev& Ld, int l, uint32_t* lds) {
    uint16_t* h = htemp(lds);
    rms_to_lds(a.x1 + l * a.sx, Ld.ln2, a.H, a.eps, h, red(lds));
    stage_xk<Q4>(h, a.H, xstage(lds, a.H));
}

template <int Q4>
__device__ void up_compute(const StepArgs& a, const LayerDev& Ld, int l, uint32_t* lds, int u,
                           const RowRegs<Nch<Q4>::t32>& rr) {
    const int lane = threadIdx.x % kWave, n = u * kWpb + threadIdx.x / kWave;
    if (n >= a.I) return;
    const float acc = row_dot_pf<Q4, 32, Nch<Q4>::t32>(lane < 32 ? Ld.g : Ld.u, n, xstage(lds, a.H), lane % 32, rr);
    const float ga = __shfl(acc, 0, kWave), ua = __shfl(acc, 32, kWave);
    if (lane == 0) {
        const float g = rb(ga), up = rb(ua);
        const float sg = rb(1.0f / (1.0f + expf(-g)));
        a.hh[l * a.sh + n] = f2bf(rb(g * sg) * up);
    }
}

// ---- LE: down + residual --------------------------------------------------------
template <int Q4>
__device__ void down_load(const StepArgs& a, const LayerDev& Ld, int u, RowRegs<Nch<Q4>::t64>& r) {
    const int r0 = u * kWpb + threadIdx.x / kWave;
    if (r0 >= a.H) return;
    row_load<Q4, 64, Nch<Q4>::t64>(Ld.d, r0, threadIdx.x % kWave, 0, r);
}

template <int Q4>
__device__ void down_prepare(const StepArgs& a, const LayerDev& Ld, int l, uint32_t* lds) {
    stage_xk<Q4>(a.hh + l * a.sh, a.I, xstage(lds, a.I));
}

template <int Q4>
__device__ void down_compute(const StepArgs& a, const LayerDev& Ld, int l, uint32_t* lds, int u,
                             const RowRegs<Nch<Q4>::t64>& rr) {
    const int lane = threadIdx.x % kWave, r = u * kWpb + threadIdx.x / kWave;
    if (r >= a.H) return;
    const float acc = row_dot_pf<Q4, 64, Nch<Q4>::t64>(Ld.d, r, xstage(lds, a.I), lane, rr);
    if (lane == 0) {
        const int64_t i = l * a.sx + r;
        a.xo[i] = f2bf(bf2f(a.x1[i]) + rb(acc));
    }
}

// ---- final norm + tied LM head + per-workgroup argmax partial -----------------
template <int Q4>
__device__ void head_load(const StepArgs& a, int u, RowRegs<Nch<Q4>::t32>& r) {
    const int lane = threadIdx.x % kWave, r0 = (u * kWpb + threadIdx.x / kWave) * 2;
    if (r0 >= a.head.N) return;
    row_load<Q4, 32, Nch<Q4>::t32>(a.head, min(r0 + lane / 32, a.head.N - 1), lane % 32, 0, r);
}

template <int Q4>
__device__ void head_prepare(const StepArgs& a, uint32_t* lds) {
    uint16_t* h = htemp(lds);
    rms_to_lds(a.x + a.n_layers * a.sx, a.final_norm, a.H, a.eps, h, red(lds));
    if (blockIdx.x == 0)
        for (int i = threadIdx.x; i < a.H; i += blockDim.x) a.hidden[i] = h[i];
    stage_xk<Q4>(h, a.H, xstage(lds, a.H));
}

// Better (value, index) pair: larger value, lower index on ties; NaN never wins.
__device__ __forceinline__ bool better(float v, int i, float bv, int bi) { return v > bv || (v == bv && i < bi); }

template <int Q4>
__device__ void head_compute(const StepArgs& a, uint32_t* lds, int u, const RowRegs<Nch<Q4>::t32>& rr, float& bv, int& bi) {
    const int lane = threadIdx.x % kWave, r0 = (u * kWpb + threadIdx.x / kWave) * 2;
    if (r0 >= a.head.N) return;
    const int team = lane / 32, tl = lane % 32, r = min(r0 + team, a.head.N - 1);
    const float acc = row_dot_pf<Q4, 32, Nch<Q4>::t32>(a.head, r, xstage(lds, a.H), tl, rr);
    if (tl == 0 && r0 + team < a.head.N) {
        if (a.logits) a.logits[r] = acc;
        if (better(acc, r, bv, bi)) {
            bv = acc;
            bi = r;
        }
    }
}

__device__ void argmax_block(float bv, int bi, float* rv, int* ri) {
    // reduce (bv, bi) over the block; result in rv[0], ri[0]
    for (int o = kWave / 2; o > 0; o >>= 1) {
        const float ov = __shfl_xor(bv, o, kWave);
        const int oi = __shfl_xor(bi, o, kWave);
        if (better(ov, oi, bv, bi)) {
            bv = ov;
            bi = oi;
        }
    }
    const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
    __syncthreads();
    if (lane == 0) {
        rv[wave] = bv;
        ri[wave] = bi;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < (int)(blockDim.x / kWave); w++)
            if (better(rv[w], ri[w], bv, bi)) {
                bv = rv[w];
                bi = ri[w];
            }
        rv[0] = bv;
        ri[0] = bi;
    }
    __syncthreads();
}

__device__ void head_finish(const StepArgs& a, uint32_t* lds, float bv, int bi) {
    float* rv = red(lds);
    int* ri = reinterpret_cast<int*>(rv + 16);
    argmax_block(bv, bi, rv, ri);
    if (threadIdx.x == 0) {
        a.amax_v[blockIdx.x] = rv[0];
        a.amax_i[blockIdx.x] = ri[0];
    }
}

__device__ void argmax_unit(const StepArgs& a, uint32_t* lds, int nparts) {
    float bv = -INFINITY;
    int bi = 0x7fffffff;
    for (int i = threadIdx.x; i < nparts; i += blockDim.x)
        if (better(a.amax_v[i], a.amax_i[i], bv, bi)) {
            bv = a.amax_v[i];
            bi = a.amax_i[i];
        }
    float* rv = red(lds);
    int* ri = reinterpret_cast<int*>(rv + 16);
    argmax_block(bv, bi, rv, ri);
    if (threadIdx.x == 0 && a.argmax_out) *a.argmax_out = ri[0] == 0x7fffffff ? 0 : ri[0];
}

// ---- stage driver shared by both schedules ------------------------------------
// GEMV stages: load the first unit's weights, prepare, then walk the units
// blockIdx.x, blockIdx.x + grid, ... with the next unit's loads in flight.
#define GEMV_STAGE(NCH, LOAD, PREPARE, COMPUTE)                          \
    {                                                                    \
        if (bid >= nu) break;                                            \
        RowRegs<NCH> cur;                                                \
        LOAD(bid, cur);                                                  \
        PREPARE;                                                         \
        for (int u = bid; u < nu; u += grid) {                           \
            RowRegs<NCH> nxt;                                            \
            const bool more = u + grid < nu;                             \
            if (more) LOAD(u + grid, nxt);                               \
            COMPUTE(u, cur);                                             \
            if (more) cur = nxt;                                         \
        }                                                                \
    }

template <int Q4>
__device__ void run_stage(Stage s, const StepArgs& a, const LayerDev& Ld, int l, uint32_t* lds, int nparts) {
    const int nu = stage_units(s, a);
    const int bid = blockIdx.x, grid = gridDim.x;
#define QKV_LOAD(u, r) qkv_load<Q4>(a, Ld, u, r)
#define QKV_COMPUTE(u, r) qkv_compute<Q4>(a, Ld, l, lds, u, r)
#define O_LOAD(u, r) o_load<Q4>(a, Ld, u, r)
#define O_COMPUTE(u, r) o_compute<Q4>(a, Ld, l, lds, u, r)
#define UP_LOAD(u, r) up_load<Q4>(a, Ld, u, r)
#define UP_COMPUTE(u, r) up_compute<Q4>(a, Ld, l, lds, u, r)
#define DOWN_LOAD(u, r) down_load<Q4>(a, Ld, u, r)
#define DOWN_COMPUTE(u, r) down_compute<Q4>(a, Ld, l, lds, u, r)
#define HEAD_LOAD(u, r) head_load<Q4>(a, u, r)
#define HEAD_COMPUTE(u, r) head_compute<Q4>(a, lds, u, r, bv, bi)
    switch (s) {
        case S_EMBED:
            if (bid == 0) embed_unit(a);
            break;
        case S_QKV:
            GEMV_STAGE(Nch<Q4>::t32, QKV_LOAD, qkv_prepare<Q4>(a, Ld, l, lds), QKV_COMPUTE);
            break;
        case S_ATTN:
            for (int u = bid; u < nu; u += grid) attn_unit(a, l, lds, u);
            break;
        case S_MERGE:
            for (int u = bid; u < nu; u += grid) merge_unit(a, l, lds, u);
            break;
        case S_O:
            GEMV_STAGE(Nch<Q4>::t32, O_LOAD, o_prepare<Q4>(a, Ld, l, lds), O_COMPUTE);
            break;
        case S_UP:
            GEMV_STAGE(Nch<Q4>::t32, UP_LOAD, up_prepare<Q4>(a, Ld, l, lds), UP_COMPUTE);
            break;
        case S_DOWN:
            GEMV_STAGE(Nch<Q4>::t64, DOWN_LOAD, down_prepare<Q4>(a, Ld, l, lds), DOWN_COMPUTE);
            break;
        case S_HEAD: {
            float bv = -INFINITY;
            int bi = 0x7fffffff;
            do {
                GEMV_STAGE(Nch<Q4>::t32, HEAD_LOAD, head_prepare<Q4>(a, lds), HEAD_COMPUTE);
            } while (0);
            head_finish(a, lds, bv, bi);
            break;
        }
        case S_ARGMAX:
            if (bid == 0) argmax_unit(a, lds, nparts);
            break;
        case S_FINAL:  // final norm only (no head): the hidden output
            if (bid == 0) {
                uint16_t* h = htemp(lds);
                rms_to_lds(a.x + a.n_layers * a.sx, a.final_norm, a.H, a.eps, h, red(lds));
                for (int i = threadIdx.x; i < a.H; i += blockDim.x) a.hidden[i] = h[i];
            }
            break;
    }
#undef QKV_LOAD
#undef QKV_COMPUTE
#undef O_LOAD
#undef O_COMPUTE
#undef UP_LOAD
#undef UP_COMPUTE
#undef DOWN_LOAD
#undef DOWN_COMPUTE
#undef HEAD_LOAD
#undef HEAD_COMPUTE
}

// ---- per-stage schedule ----------------------------------------------------------
template <int Q4, Stage S>
__global__ __launch_bounds__(kBlock) void stage_kernel(StepArgs a, LayerDev Ld, int l, int nparts) {
    __shared__ uint32_t lds[kLdsWords];
    run_stage<Q4>(S, a, Ld, l, lds, nparts);
}

int host_units(Stage s, const StepArgs& a) {
    return units_of(s, a.H, a.kvh, a.hd, a.heads, a.I, a.head.N,
                    a.kvh * ((a.pos + 1 + a.split_len - 1) / a.split_len));
}

template <Stage S>
hipError_t launch_stage(hipStream_t st, const StepArgs& a, const LayerDev& Ld, int l, int grid, int nparts) {
    if (Ld.q.kind == 1)
        hipLaunchKernelGGL((stage_kernel<1, S>), dim3(grid), dim3(kBlock), 0, st, a, Ld, l, nparts);
    else
        hipLaunchKernelGGL((stage_kernel<0, S>), dim3(grid), dim3(kBlock), 0, st, a, Ld, l, nparts);
    return hipGetLastError();
}

}  // namespace

// Positions per attention split: 64 (one tile) while that gives at most 64
// splits per kv head, doubling up to kMaxSplit for longer contexts.
int attn_split_len(int n) {
    int sl = 64;
    while (sl < kMaxSplit && (n + sl - 1) / sl > 64) sl *= 2;
    return sl;
}

// Partials for any context length up to n: below the largest split length a
// context uses at most 64 splits; at kMaxSplit it uses ceil(n / kMaxSplit).
size_t attn_part_floats(int kvh, int heads, int hd, int n) {
    const int ns_big = (n + kMaxSplit - 1) / kMaxSplit;
    const int ns = ns_big > 64 ? ns_big : 64;
    return (size_t)kvh * ns * (heads / kvh) * (hd + 2);
}

// One layer on the per-stage schedule (ming_lm_layer).
hipError_t launch_lm_layer(hipStream_t st, const StepArgs& a, const LayerDev& Ld, int l) {
    hipError_t e;
    if ((e = launch_stage<S_QKV>(st, a, Ld, l, host_units(S_QKV, a), 0)) != hipSuccess) return e;
    if ((e = launch_stage<S_ATTN>(st, a, Ld, l, host_units(S_ATTN, a), 0)) != hipSuccess) return e;
    if ((e = launch_stage<S_MERGE>(st, a, Ld, l, host_units(S_MERGE, a), 0)) != hipSuccess) return e;
    if ((e = launch_stage<S_O>(st, a, Ld, l, host_units(S_O, a), 0)) != hipSuccess) return e;
    if ((e = launch_stage<S_UP>(st, a, Ld, l, host_units(S_UP, a), 0)) != hipSuccess) return e;
    return launch_stage<S_DOWN>(st, a, Ld, l, host_units(S_DOWN, a), 0);
}

// Whole step on the per-stage schedule; host_layers mirrors a.layers.
hipError_t launch_lm_step_kernels(hipStream_t st, const StepArgs& a, const LayerDev* host_layers) {
    hipError_t e;
    if (a.token_in && (e = launch_stage<S_EMBED>(st, a, host_layers[0], 0, 1, 0)) != hipSuccess) return e;
    for (int l = 0; l < a.n_layers; l++)
        if ((e = launch_lm_layer(st, a, host_layers[l], l)) != hipSuccess) return e;
    if (!a.logits && !a.argmax_out) return launch_stage<S_FINAL>(st, a, host_layers[0], 0, 1, 0);
    const int hg = host_units(S_HEAD, a) < 2048 ? host_units(S_HEAD, a) : 2048;
    if ((e = launch_stage<S_HEAD>(st, a, host_layers[0], 0, hg, 0)) != hipSuccess) return e;
    return launch_stage<S_ARGMAX>(st, a, host_layers[0], 0, 1, hg);
}

}  // namespace ming
