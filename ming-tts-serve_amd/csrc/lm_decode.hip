// Qwen2 decode step for gfx950: the reference's five fused layer kernels
// LA..LE (src/ming_fused.zig:296-399), rebuilt for 64-wide wavefronts, with
// the KV cache written in place, split-K GQA attention for long contexts, and
// the tied LM head with a greedy argmax.
//
// Each stage is a pair of device functions: `prepare` stages the stage's
// activation vector in LDS once per workgroup, `unit` computes one
// workgroup-sized slice of the outputs.  Two schedules run the same stages:
//   - per-stage launches (one kernel per stage, the reference's schedule);
//   - one persistent kernel per token whose workgroups walk the stages,
//     separated by grid barriers.
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
constexpr int kMaxSplit = 256;        // attention positions per split

enum Stage { S_EMBED, S_QKV, S_ATTN, S_MERGE, S_O, S_UP, S_DOWN, S_HEAD, S_ARGMAX };

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

__device__ __forceinline__ int stage_units(Stage s, const StepArgs& a) {
    switch (s) {
        case S_EMBED: return 1;
        case S_QKV: return ((a.H + 2 * a.kvh * a.hd) / 2 + kWpb - 1) / kWpb;
        case S_ATTN: return a.kvh * attn_nsplit(a);
        case S_MERGE: return (a.heads + kWpb - 1) / kWpb;
        case S_O: return (a.H + 2 * kWpb - 1) / (2 * kWpb);
        case S_UP: return (a.I + kWpb - 1) / kWpb;
        case S_DOWN: return (a.H + kWpb - 1) / kWpb;
        case S_HEAD: return (a.head.N + 2 * kWpb - 1) / (2 * kWpb);
        case S_ARGMAX: return 1;
    }
    return 0;
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
__device__ void qkv_prepare(const StepArgs& a, const LayerDev& Ld, int l, uint32_t* lds) {
    uint16_t* h = htemp(lds);
    rms_to_lds(a.x + l * a.sx, Ld.ln1, a.H, a.eps, h, red(lds));
    stage_x(Ld.q, h, xstage(lds, a.H));
}

__device__ void qkv_unit(const StepArgs& a, const LayerDev& Ld, int l, uint32_t* lds, int u) {
    const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
    const int half = a.hd / 2, kvd = a.kvh * a.hd, nq = a.H + 2 * kvd;
    const int pi = u * kWpb + wave;
    if (pi >= nq / 2) return;
    const int r1 = (pi / half) * a.hd + pi % half;  // row in the concatenated [q | k | v] space
    const int which = r1 < a.H ? 0 : (r1 < a.H + kvd ? 1 : 2);
    const int base = which == 0 ? 0 : (which == 1 ? a.H : a.H + kvd);
    const LinearDev& L = which == 0 ? Ld.q : (which == 1 ? Ld.k : Ld.v);
    const uint16_t* bias = which == 0 ? Ld.bq : (which == 1 ? Ld.bk : Ld.bv);
    const int team = lane / 32, tl = lane % 32;
    const int row = r1 - base + team * half;
    const float acc = row_dot<32>(L, row, xstage(lds, a.H), tl);
    const float v1 = __shfl(acc, 0, kWave), v2 = __shfl(acc, 32, kWave);
    if (lane != 0) return;
    const int lr = r1 - base;
    float e1, e2;
    if (L.kind == 1) {  // quantized_matmul, then + bias
        e1 = rb(rb(v1) + bf2f(bias[lr]));
        e2 = rb(rb(v2) + bf2f(bias[lr + half]));
    } else {            // addmm
        e1 = rb(v1 + bf2f(bias[lr]));
        e2 = rb(v2 + bf2f(bias[lr + half]));
    }
    if (which < 2) {  // MLX fast::rope, non-traditional: pair (d, d + hd/2)
        const int d = lr % a.hd;
        const float inv_freq = exp2f(-((float)d / (float)half) * a.log2_theta);
        const float th = (float)a.pos * inv_freq;
        const float c = cosf(th), s = sinf(th);
        const float o1 = e1 * c - e2 * s, o2 = e1 * s + e2 * c;
        e1 = rb(o1);
        e2 = rb(o2);
    }
    uint16_t* q = a.qkv + l * a.sq;
    q[r1] = f2bf(e1);
    q[r1 + half] = f2bf(e2);
    if (which > 0) {
        uint16_t* cache = which == 1 ? a.kc : a.vc;
        const int kh = lr / a.hd, d = lr % a.hd;
        uint16_t* dst = cache + (((size_t)l * a.kvh + kh) * a.cap + a.pos) * a.hd;
        dst[d] = f2bf(e1);
        dst[d + half] = f2bf(e2);
    }
}

// ---- LB: split-K GQA attention; one unit = (kv head, split of positions) ----
// Scores, softmax partials (max, sum) and P.V for the grp query heads that
// share the kv head, over positions [j0, j1) of the cache (the new row at
// `pos` included).  Partials are merged by the MERGE stage.
__device__ void attn_unit(const StepArgs& a, int l, uint32_t* lds, int u) {
    const int ns = attn_nsplit(a), n = a.pos + 1, grp = a.heads / a.kvh, hd = a.hd;
    const int g = u / ns, sp = u % ns;
    const int j0 = sp * a.split_len, j1 = min(n, j0 + a.split_len), cnt = j1 - j0;
    float* qf = reinterpret_cast<float*>(lds);        // [grp][hd]
    float* sc = qf + 8 * 64;                          // [grp][kMaxSplit]
    float* ml = sc + 8 * kMaxSplit;                   // [grp][2]
    const float scale = 1.0f / sqrtf((float)hd);
    const uint16_t* q = a.qkv + l * a.sq + (size_t)g * grp * hd;
    for (int i = threadIdx.x; i < grp * hd; i += blockDim.x) qf[i] = scale * bf2f(q[i]);
    __syncthreads();
    const uint16_t* kbase = a.kc + (((size_t)l * a.kvh + g) * a.cap) * hd;
    const uint16_t* vbase = a.vc + (((size_t)l * a.kvh + g) * a.cap) * hd;
    const int hs = threadIdx.x / 64, t64 = threadIdx.x % 64;
    for (int t0 = 0; t0 < cnt; t0 += 64) {
        const int jj = t0 + t64;
        if (jj < cnt) {
            const uint4* kr = reinterpret_cast<const uint4*>(kbase + (size_t)(j0 + jj) * hd);
            float kv[64];
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const uint4 w = kr[i];
                kv[8 * i + 0] = bf_lo(w.x); kv[8 * i + 1] = bf_hi(w.x);
                kv[8 * i + 2] = bf_lo(w.y); kv[8 * i + 3] = bf_hi(w.y);
                kv[8 * i + 4] = bf_lo(w.z); kv[8 * i + 5] = bf_hi(w.z);
                kv[8 * i + 6] = bf_lo(w.w); kv[8 * i + 7] = bf_hi(w.w);
            }
            for (int h = hs; h < grp; h += 4) {
                const float* qh = qf + h * hd;
                float p[8] = {0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
                for (int d = 0; d < 64; d++) p[d % 8] += qh[d] * kv[d];
                sc[h * kMaxSplit + jj] = ((p[0] + p[1]) + (p[2] + p[3])) + ((p[4] + p[5]) + (p[6] + p[7]));
            }
        }
    }
    __syncthreads();
    // per-head max and sum: wave w takes heads w, w+4
    const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
    for (int h = wave; h < grp; h += kWpb) {
        float* s = sc + h * kMaxSplit;
        float m = -INFINITY;
        for (int j = lane; j < cnt; j += kWave) m = fmaxf(m, s[j]);
        m = team_max<kWave>(m);
        float sum = 0.0f;
        for (int j = lane; j < cnt; j += kWave) {
            const float p = expf(s[j] - m);
            s[j] = p;
            sum += p;
        }
        sum = team_sum<kWave>(sum);
        if (lane == 0) {
            ml[2 * h] = m;
            ml[2 * h + 1] = sum;
        }
    }
    __syncthreads();
    // P.V: thread (hs, d) accumulates heads hs, hs+4 over the split
    {
        const int d = t64;
        float acc0 = 0.0f, acc1 = 0.0f;
        const bool h1 = hs + 4 < grp;
        const float* s0 = sc + hs * kMaxSplit;
        const float* s1 = sc + (hs + 4) * kMaxSplit;
        if (hs < grp) {
            for (int jj = 0; jj < cnt; jj++) {
                const float v = bf2f(vbase[(size_t)(j0 + jj) * hd + d]);
                acc0 += s0[jj] * v;
                if (h1) acc1 += s1[jj] * v;
            }
            float* out = a.part + ((size_t)(g * ns + sp) * grp + hs) * (hd + 2);
            out[2 + d] = acc0;
            if (d == 0) {
                out[0] = ml[2 * hs];
                out[1] = ml[2 * hs + 1];
            }
            if (h1) {
                float* out1 = a.part + ((size_t)(g * ns + sp) * grp + hs + 4) * (hd + 2);
                out1[2 + d] = acc1;
                if (d == 0) {
                    out1[0] = ml[2 * (hs + 4)];
                    out1[1] = ml[2 * (hs + 4) + 1];
                }
            }
        }
    }
    __syncthreads();
}

// ---- merge of the split partials: att[h] = sum_s e^(m_s-M) acc_s / sum_s e^(m_s-M) l_s ----
__device__ void merge_unit(const StepArgs& a, int l, int u) {
    const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
    const int h = u * kWpb + wave;
    if (h >= a.heads) return;
    const int grp = a.heads / a.kvh, g = h / grp, hl = h % grp, ns = attn_nsplit(a), hd = a.hd;
    float M = -INFINITY;
    for (int s = 0; s < ns; s++) M = fmaxf(M, a.part[((size_t)(g * ns + s) * grp + hl) * (hd + 2)]);
    float Lsum = 0.0f, O = 0.0f;
    for (int s = 0; s < ns; s++) {
        const float* p = a.part + ((size_t)(g * ns + s) * grp + hl) * (hd + 2);
        const float e = expf(p[0] - M);
        Lsum += p[1] * e;
        if (lane < hd) O += p[2 + lane] * e;
    }
    if (lane < hd) a.att[l * a.sx + h * hd + lane] = f2bf(O / Lsum);
}

// ---- LC: o_proj + residual ----------------------------------------------------
__device__ void o_prepare(const StepArgs& a, const LayerDev& Ld, int l, uint32_t* lds) {
    stage_x(Ld.o, a.att + l * a.sx, xstage(lds, a.H));
}

__device__ void o_unit(const StepArgs& a, const LayerDev& Ld, int l, uint32_t* lds, int u) {
    const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
    const int r0 = (u * kWpb + wave) * 2;
    if (r0 >= a.H) return;
    const int team = lane / 32, tl = lane % 32, r = min(r0 + team, a.H - 1);
    const float acc = row_dot<32>(Ld.o, r, xstage(lds, a.H), tl);
    if (tl == 0 && r0 + team < a.H) {
        const int64_t i = l * a.sx + r;
        a.x1[i] = f2bf(bf2f(a.x[i]) + rb(acc));
    }
}

// ---- LD: rms(ln2) + gate/up + swiglu ------------------------------------------
__device__ void up_prepare(const StepArgs& a, const LayerDev& Ld, int l, uint32_t* lds) {
    uint16_t* h = htemp(lds);
    rms_to_lds(a.x1 + l * a.sx, Ld.ln2, a.H, a.eps, h, red(lds));
    stage_x(Ld.g, h, xstage(lds, a.H));
}

__device__ void up_unit(const StepArgs& a, const LayerDev& Ld, int l, uint32_t* lds, int u) {
    const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
    const int n = u * kWpb + wave;
    if (n >= a.I) return;
    const int team = lane / 32, tl = lane % 32;
    const float acc = row_dot<32>(team == 0 ? Ld.g : Ld.u, n, xstage(lds, a.H), tl);
    const float ga = __shfl(acc, 0, kWave), ua = __shfl(acc, 32, kWave);
    if (lane == 0) {
        const float g = rb(ga), up = rb(ua);
        const float sg = rb(1.0f / (1.0f + expf(-g)));
        a.hh[l * a.sh + n] = f2bf(rb(g * sg) * up);
    }
}

// ---- LE: down + residual --------------------------------------------------------
__device__ void down_prepare(const StepArgs& a, const LayerDev& Ld, int l, uint32_t* lds) {
    stage_x(Ld.d, a.hh + l * a.sh, xstage(lds, a.I));
}

__device__ void down_unit(const StepArgs& a, const LayerDev& Ld, int l, uint32_t* lds, int u) {
    const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
    const int r = u * kWpb + wave;
    if (r >= a.H) return;
    const float acc = row_dot<64>(Ld.d, r, xstage(lds, a.I), lane);
    if (lane == 0) {
        const int64_t i = l * a.sx + r;
        a.xo[i] = f2bf(bf2f(a.x1[i]) + rb(acc));
    }
}

// ---- final norm + tied LM head + per-workgroup argmax partial -----------------
__device__ void head_prepare(const StepArgs& a, uint32_t* lds) {
    uint16_t* h = htemp(lds);
    rms_to_lds(a.x + a.n_layers * a.sx, a.final_norm, a.H, a.eps, h, red(lds));
    if (blockIdx.x == 0)
        for (int i = threadIdx.x; i < a.H; i += blockDim.x) a.hidden[i] = h[i];
    stage_x(a.head, h, xstage(lds, a.H));
}

// Better (value, index) pair: larger value, lower index on ties; NaN never wins.
__device__ __forceinline__ bool better(float v, int i, float bv, int bi) { return v > bv || (v == bv && i < bi); }

__device__ void head_unit(const StepArgs& a, uint32_t* lds, int u, float& bv, int& bi) {
    const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
    const int r0 = (u * kWpb + wave) * 2;
    if (r0 >= a.head.N) return;
    const int team = lane / 32, tl = lane % 32, r = min(r0 + team, a.head.N - 1);
    const float acc = row_dot<32>(a.head, r, xstage(lds, a.H), tl);
    if (tl == 0 && r0 + team < a.head.N) {
        if (a.logits) a.logits[r] = acc;
        if (better(acc, r, bv, bi)) {
            bv = acc;
            bi = r;
        }
    }
}

__device__ void argmax_block(float bv, int bi, float* rv, int* ri) {
    // reduce (bv, bi) over the block; result in thread 0
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
// Runs `s` for layer l over units blockIdx.x, blockIdx.x + grid, ...
__device__ void run_stage(Stage s, const StepArgs& a, const LayerDev& Ld, int l, uint32_t* lds, int nparts) {
    const int nu = stage_units(s, a);
    const int bid = blockIdx.x, grid = gridDim.x;
    switch (s) {
        case S_EMBED:
            if (bid == 0) embed_unit(a);
            break;
        case S_QKV:
            if (bid >= nu) break;
            qkv_prepare(a, Ld, l, lds);
            for (int u = bid; u < nu; u += grid) qkv_unit(a, Ld, l, lds, u);
            break;
        case S_ATTN:
            for (int u = bid; u < nu; u += grid) attn_unit(a, l, lds, u);
            break;
        case S_MERGE:
            for (int u = bid; u < nu; u += grid) merge_unit(a, l, u);
            break;
        case S_O:
            if (bid >= nu) break;
            o_prepare(a, Ld, l, lds);
            for (int u = bid; u < nu; u += grid) o_unit(a, Ld, l, lds, u);
            break;
        case S_UP:
            if (bid >= nu) break;
            up_prepare(a, Ld, l, lds);
            for (int u = bid; u < nu; u += grid) up_unit(a, Ld, l, lds, u);
            break;
        case S_DOWN:
            if (bid >= nu) break;
            down_prepare(a, Ld, l, lds);
            for (int u = bid; u < nu; u += grid) down_unit(a, Ld, l, lds, u);
            break;
        case S_HEAD: {
            float bv = -INFINITY;
            int bi = 0x7fffffff;
            if (bid < nu) {
                head_prepare(a, lds);
                for (int u = bid; u < nu; u += grid) head_unit(a, lds, u, bv, bi);
            }
            head_finish(a, lds, bv, bi);
            break;
        }
        case S_ARGMAX:
            if (bid == 0) argmax_unit(a, lds, nparts);
            break;
    }
}

// ---- per-stage schedule ----------------------------------------------------------
template <Stage S>
__global__ __launch_bounds__(kBlock) void stage_kernel(StepArgs a, LayerDev Ld, int l, int nparts) {
    __shared__ uint32_t lds[kLdsWords];
    run_stage(S, a, Ld, l, lds, nparts);
}

// ---- persistent schedule -------------------------------------------------------
// Grid barrier on a monotonic counter (flags[1], zeroed before the launch).
// Each workgroup publishes its writes (device-scope release), adds one, and
// waits for gridDim.x * k arrivals at its k-th barrier.  The wait is bounded:
// past the spin limit the workgroup raises flags[0] and goes on, so the grid
// always drains; the host reports MING_E_TIMEOUT.
constexpr unsigned kSpinLimit = 1u << 22;

__device__ void grid_barrier(int32_t* flags, unsigned& target) {
    __syncthreads();
    target += gridDim.x;
    if (threadIdx.x == 0) {
        unsigned* ctr = reinterpret_cast<unsigned*>(flags + 1);
        __threadfence();
        atomicAdd(ctr, 1u);
        unsigned spins = 0;
        while (__hip_atomic_load(ctr, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_AGENT) < target) {
            __builtin_amdgcn_s_sleep(1);
            if (++spins >= kSpinLimit) {
                atomicOr(flags, 1);
                break;
            }
            if ((spins & 1023u) == 0 && __hip_atomic_load(flags, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) break;
        }
        __threadfence();
    }
    __syncthreads();
}

__global__ __launch_bounds__(kBlock) void step_persistent_kernel(StepArgs a) {
    __shared__ uint32_t lds[kLdsWords];
    unsigned target = 0;
    const LayerDev& L0 = a.layers[0];
    if (a.token_in) {
        run_stage(S_EMBED, a, L0, 0, lds, 0);
        grid_barrier(a.flags, target);
    }
    for (int l = 0; l < a.n_layers; l++) {
        const LayerDev& Ld = a.layers[l];
        run_stage(S_QKV, a, Ld, l, lds, 0);
        grid_barrier(a.flags, target);
        run_stage(S_ATTN, a, Ld, l, lds, 0);
        grid_barrier(a.flags, target);
        run_stage(S_MERGE, a, Ld, l, lds, 0);
        grid_barrier(a.flags, target);
        run_stage(S_O, a, Ld, l, lds, 0);
        grid_barrier(a.flags, target);
        run_stage(S_UP, a, Ld, l, lds, 0);
        grid_barrier(a.flags, target);
        run_stage(S_DOWN, a, Ld, l, lds, 0);
        grid_barrier(a.flags, target);
    }
    run_stage(S_HEAD, a, L0, 0, lds, 0);
    grid_barrier(a.flags, target);
    run_stage(S_ARGMAX, a, L0, 0, lds, gridDim.x);
}

__global__ void zero_counter_kernel(int32_t* flags) { flags[1] = 0; }

__global__ void copy_token_kernel(const int32_t* src, int32_t* dst) { *dst = *src; }

int host_units(Stage s, const StepArgs& a) {
    switch (s) {
        case S_EMBED: return 1;
        case S_QKV: return ((a.H + 2 * a.kvh * a.hd) / 2 + kWpb - 1) / kWpb;
        case S_ATTN: return a.kvh * ((a.pos + 1 + a.split_len - 1) / a.split_len);
        case S_MERGE: return (a.heads + kWpb - 1) / kWpb;
        case S_O: return (a.H + 2 * kWpb - 1) / (2 * kWpb);
        case S_UP: return (a.I + kWpb - 1) / kWpb;
        case S_DOWN: return (a.H + kWpb - 1) / kWpb;
        case S_HEAD: return (a.head.N + 2 * kWpb - 1) / (2 * kWpb);
        case S_ARGMAX: return 1;
    }
    return 1;
}

template <Stage S>
hipError_t launch_stage(hipStream_t st, const StepArgs& a, const LayerDev& Ld, int l, int grid, int nparts) {
    hipLaunchKernelGGL(stage_kernel<S>, dim3(grid), dim3(kBlock), 0, st, a, Ld, l, nparts);
    return hipGetLastError();
}

}  // namespace

// Positions per attention split: enough splits to spread the cache over
// the chip, each a multiple of 64 and at most kMaxSplit.
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
    const int hg = host_units(S_HEAD, a) < 2048 ? host_units(S_HEAD, a) : 2048;
    if ((e = launch_stage<S_HEAD>(st, a, host_layers[0], 0, hg, 0)) != hipSuccess) return e;
    return launch_stage<S_ARGMAX>(st, a, host_layers[0], 0, 1, hg);
}

// Whole step as one persistent kernel of `grid` co-resident workgroups.
hipError_t launch_lm_step_persistent(hipStream_t st, const StepArgs& a, int grid) {
    hipLaunchKernelGGL(zero_counter_kernel, dim3(1), dim3(1), 0, st, a.flags);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    StepArgs args = a;
    void* params[] = {&args};
    return hipLaunchCooperativeKernel(reinterpret_cast<const void*>(step_persistent_kernel), dim3(grid),
                                      dim3(kBlock), params, 0, st);
}

int persistent_grid(int num_cus) {
    int per_cu = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, step_persistent_kernel, kBlock, 0) != hipSuccess ||
        per_cu < 1)
        return 0;
    if (per_cu > 2) per_cu = 2;
    return num_cus * per_cu;
}

hipError_t launch_copy_token(hipStream_t st, const int32_t* src, int32_t* dst) {
    hipLaunchKernelGGL(copy_token_kernel, dim3(1), dim3(1), 0, st, src, dst);
    return hipGetLastError();
}

}  // namespace ming
