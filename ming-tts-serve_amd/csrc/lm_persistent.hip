// One persistent kernel per decode token (the whole of QStack.decodeFused,
// src/ming_model.zig:530-544, plus the tied LM head and argmax), with the
// stages handing their outputs over through tagged words instead of grid
// barriers.
//
// Hand-off: a stage's output vector is written as u64 words {bf16 pair, epoch}
// with device-coherent (sc1) stores, and a consumer polls the words it needs
// with device-coherent loads until every tag equals the step's epoch.  Data
// and flag travel in one single-copy-atomic word, so no fence (no L2
// write-back or invalidate) is needed and a hand-off costs one cross-XCD
// store->load trip.  Buffers start zeroed and epochs start at 1, so a stale
// word never matches.
//
// Overlap: every workgroup issues the weight loads of its next units (and
// attention workgroups their first K/V tile) before it polls for the stage's
// input, so HBM latency is hidden behind the dependency chain.
//
// Attention splits meet through a per-(layer, kv head) arrival counter: the
// workgroup that arrives last merges the partials.  The LM head's
// per-workgroup argmax partials meet the same way.  Partials are written with
// device-coherent stores and waited on (s_waitcnt) before the arrival.
//
// Every wait is bounded: past the spin limit a workgroup raises flags[0] and
// continues, so the grid always drains; the host reports MING_E_TIMEOUT.
// The kernel needs all workgroups co-resident (cooperative launch, one per
// CU).
#include "gemv.h"
#include "internal.h"

namespace ming {

namespace {

constexpr int kT = 512;          // threads per workgroup (8 waves, 2 per SIMD)
constexpr int kW = kT / kWave;   // waves per workgroup
constexpr int kLds = 12288;      // LDS words (48 KB)
constexpr int kXsOff = 0;        // XStage, K <= 8192: 4352 words
constexpr int kRecvOff = 4400;   // received payloads, <= 4096 words
constexpr int kHtOff = 8496;     // rms output, <= 2048 bf16
constexpr int kRedOff = 9520;    // reduction scratch (64 words)
constexpr int kFlagOff = 9584;   // broadcast flags (16 words)
constexpr unsigned kSpin = 1u << 22;
constexpr int kTile = 64;

template <int Q4>
struct Nc {
    static constexpr int t32 = Q4 ? 1 : 4;   // chunks per lane, K = hidden
    static constexpr int down = Q4 ? 5 : 5;  // chunks per lane, K = inter (32-lane teams)
    static constexpr int up_units = Q4 ? 2 : 1;
};

__device__ __forceinline__ void tstore(uint64_t* p, uint32_t payload, uint32_t tag) {
    __hip_atomic_store(p, ((uint64_t)tag << 32) | payload, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t tload(const uint64_t* p) {
    return __hip_atomic_load(const_cast<uint64_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void cstore(float* p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float cload(const float* p) {
    return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ int flag_set(int32_t* flags) {
    return __hip_atomic_load(flags, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Pollers back off between rounds (s_sleep of about 64 cycles per unit, up
// to 4 units), so a few hundred workgroups waiting on one small vector do not
// crowd out the stores they are waiting for.
__device__ __forceinline__ void poll_pause(unsigned s) {
    if (s < 2)
        __builtin_amdgcn_s_sleep(1);
    else if (s < 8)
        __builtin_amdgcn_s_sleep(2);
    else
        __builtin_amdgcn_s_sleep(4);
}

// Poll one tagged word until it carries `tag` (bounded); returns its payload.
__device__ __forceinline__ uint32_t trecv1(const uint64_t* p, uint32_t tag, int32_t* flags) {
    uint64_t w = tload(p);
    unsigned s = 0;
    while ((uint32_t)(w >> 32) != tag) {
        if (++s >= kSpin) {
            atomicOr(flags, 1);
            break;
        }
        if ((s & 255u) == 0 && flag_set(flags)) break;
        poll_pause(s);
        w = tload(p);
    }
    return (uint32_t)w;
}

// Finish a tagged word whose first load was issued earlier.
__device__ __forceinline__ uint32_t tfinish(const uint64_t* p, uint64_t w, uint32_t tag, int32_t* flags) {
    return (uint32_t)(w >> 32) == tag ? (uint32_t)w : trecv1(p, tag, flags);
}

// Whole tagged vector of n words (n <= 8 * blockDim.x) into LDS (u32
// payloads); ends with a barrier.  A thread issues the loads of all its words
// at once and re-polls only the stale ones, so the wait is one round trip
// after the last producer, not one per word.
__device__ void trecv(const uint64_t* src, int n, uint32_t tag, uint32_t* dst, int32_t* flags) {
    constexpr int kMaxPer = 8;
    uint64_t w[kMaxPer];
#pragma unroll
    for (int k = 0; k < kMaxPer; k++) {
        const int i = threadIdx.x + k * blockDim.x;
        w[k] = i < n ? tload(src + i) : ((uint64_t)tag << 32);
    }
    unsigned s = 0;
    while (true) {
        bool ready = true;
#pragma unroll
        for (int k = 0; k < kMaxPer; k++) ready &= (uint32_t)(w[k] >> 32) == tag;
        if (ready) break;
        if (++s >= kSpin) {
            atomicOr(flags, 1);
            break;
        }
        if ((s & 255u) == 0 && flag_set(flags)) break;
        poll_pause(s);
#pragma unroll
        for (int k = 0; k < kMaxPer; k++) {
            const int i = threadIdx.x + k * blockDim.x;
            if ((uint32_t)(w[k] >> 32) != tag) w[k] = tload(src + i);
        }
    }
#pragma unroll
    for (int k = 0; k < kMaxPer; k++) {
        const int i = threadIdx.x + k * blockDim.x;
        if (i < n) dst[i] = (uint32_t)w[k];
    }
    __syncthreads();
}

// Optional profile: wall-clock stamps of this workgroup.  Slot 0 is the
// kernel start; stage s (0 qkv, 1 attn, 2 o, 3 up, 4 down) of layer l has
// slot 1 + 2 (5 l + s) when its input has arrived and the next slot when it is
// done; the head takes the two slots after the last layer.
__device__ __forceinline__ void stamp(const StepArgs& a, int k) {
    if (a.tstamp && threadIdx.x == 0) a.tstamp[(size_t)k * gridDim.x + blockIdx.x] = wall_clock64();
}
__device__ __forceinline__ int slot_in(int l, int s) { return 1 + 2 * (5 * l + s); }

struct Ctx {
    const StepArgs& a;
    uint32_t* lds;
    int G, wg, wave, lane, team, tl;
};

__device__ __forceinline__ XStage xs_of(uint32_t* lds, int K) {
    return XStage{lds + kXsOff, reinterpret_cast<float*>(lds + kXsOff + K / 2)};
}
__device__ __forceinline__ uint16_t* recv16(uint32_t* lds) { return reinterpret_cast<uint16_t*>(lds + kRecvOff); }

// MLX fast::rms_norm of x (LDS) into LDS.
__device__ void rms_lds(const uint16_t* x, const uint16_t* w, int H, float eps, uint16_t* h, float* rd) {
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

// Receive a tagged bf16 vector of K values, optionally rms-normalise it, and
// stage it for a GEMV.
template <int Q4>
__device__ void recv_stage(const Ctx& c, const uint64_t* src, int K, const uint16_t* norm_w, uint16_t* h_out = nullptr) {
    const StepArgs& a = c.a;
    trecv(src, K / 2, a.epoch, c.lds + kRecvOff, a.flags);
    const uint16_t* x = recv16(c.lds);
    if (norm_w) {
        uint16_t* h = reinterpret_cast<uint16_t*>(c.lds + kHtOff);
        rms_lds(x, norm_w, K, a.eps, h, reinterpret_cast<float*>(c.lds + kRedOff));
        if (h_out)
            for (int i = threadIdx.x; i < K; i += blockDim.x) h_out[i] = h[i];
        x = h;
    }
    stage_xk<Q4>(x, K, xs_of(c.lds, K));
}

// ---- embed / input row -> tx[0] ----------------------------------------------
__device__ void st_embed(const Ctx& c) {
    const StepArgs& a = c.a;
    const int nw = a.H / 2;
    for (int i = c.wg * kT + threadIdx.x; i < nw; i += c.G * kT) {
        uint32_t v;
        if (a.token_in) {
            const LinearDev& E = a.embed;
            int id = *a.token_in;
            id = id < 0 ? 0 : (id >= E.N ? E.N - 1 : id);
            const int k = 2 * i;
            if (E.kind == 1) {
                const uint32_t word = E.w[(size_t)id * (E.K / 8) + k / 8];
                const float sc = bf2f(E.s[(size_t)id * (E.K / 64) + k / 64]);
                const float bi = bf2f(E.b[(size_t)id * (E.K / 64) + k / 64]);
                float v0 = sc * (float)((word >> (4 * (k % 8))) & 0xfu) + bi;
                float v1 = sc * (float)((word >> (4 * (k % 8) + 4)) & 0xfu) + bi;
                if (E.gscale != 1.0f) {
                    v0 *= E.gscale;
                    v1 *= E.gscale;
                }
                v = pack_bf2(v0, v1);
            } else {
                v = reinterpret_cast<const uint32_t*>(E.w)[((size_t)id * E.K + k) / 2];
            }
            reinterpret_cast<uint32_t*>(a.x)[i] = v;
        } else {
            v = reinterpret_cast<const uint32_t*>(a.x)[i];
        }
        tstore(a.tx + i, v, a.epoch);
    }
}

// ---- LA: q/k/v + bias + rope ----------------------------------------------------
// Unit = quad of rows (c, c+1, c+hd/2, c+hd/2+1) of the concatenated [q|k|v]
// rows, c even; team 0 computes the first two, team 1 the other two, so each
// output word (c, c+1) has one writer.  Units are packed: unit = wg*kW + wave.
//
// Every GEMV stage is split into `load` (issue this workgroup's weight loads
// into registers) and `run` (wait for the input vector, compute, hand over).
// The kernel issues stage s+1's loads before it runs stage s, so weights are
// in flight one stage ahead across the whole chain, layers included.
struct QkvGeom {
    bool any, has;
    int cr, which, base, r0;
};

__device__ __forceinline__ QkvGeom qkv_geom(const Ctx& c) {
    const StepArgs& a = c.a;
    const int half = a.hd / 2, kvd = a.kvh * a.hd, nq = a.H + 2 * kvd;
    const int nunits = nq / 4, qpb = half / 2;  // quads per head block
    QkvGeom g;
    g.any = c.wg * kW < nunits;
    const int q = c.wg * kW + c.wave;
    g.has = q < nunits;
    g.cr = (q / qpb) * a.hd + (q % qpb) * 2;  // concatenated row c
    g.which = g.cr < a.H ? 0 : (g.cr < a.H + kvd ? 1 : 2);
    g.base = g.which == 0 ? 0 : (g.which == 1 ? a.H : a.H + kvd);
    g.r0 = g.cr - g.base + c.team * half;  // this team's rows r0, r0 + 1
    return g;
}

template <int Q4>
struct QkvW {
    RowRegs<Nc<Q4>::t32> w0, w1;
};

template <int Q4>
__device__ void qkv_load(const Ctx& c, const LayerDev& Ld, QkvW<Q4>& W) {
    const QkvGeom g = qkv_geom(c);
    if (!g.has) return;
    const LinearDev& L = g.which == 0 ? Ld.q : (g.which == 1 ? Ld.k : Ld.v);
    row_load<Q4, 32, Nc<Q4>::t32>(L, g.r0, c.tl, 0, W.w0);
    row_load<Q4, 32, Nc<Q4>::t32>(L, g.r0 + 1, c.tl, 0, W.w1);
}

template <int Q4>
__device__ void st_qkv(const Ctx& c, const LayerDev& Ld, int l, const QkvW<Q4>& W) {
    const StepArgs& a = c.a;
    const int half = a.hd / 2, kvd = a.kvh * a.hd, nq = a.H + 2 * kvd;
    const QkvGeom g = qkv_geom(c);
    if (!g.any) return;
    const bool has = g.has;
    const int cr = g.cr, which = g.which, base = g.base, r0 = g.r0;
    const LinearDev& L = which == 0 ? Ld.q : (which == 1 ? Ld.k : Ld.v);
    recv_stage<Q4>(c, a.tx + (size_t)l * (a.H / 2), a.H, Ld.ln1);
    stamp(a, slot_in(l, 0));
    if (!has) return;
    const XStage st = xs_of(c.lds, a.H);
    const float acc0 = row_dot_pf<Q4, 32, Nc<Q4>::t32>(L, r0, st, c.tl, W.w0);
    const float acc1 = row_dot_pf<Q4, 32, Nc<Q4>::t32>(L, r0 + 1, st, c.tl, W.w1);
    const float v[4] = {__shfl(acc0, 0, kWave), __shfl(acc1, 0, kWave), __shfl(acc0, 32, kWave),
                        __shfl(acc1, 32, kWave)};
    if (c.lane != 0) return;
    const uint16_t* bias = which == 0 ? Ld.bq : (which == 1 ? Ld.bk : Ld.bv);
    const int lr = cr - base;
    float e[4];
    const int off[4] = {0, 1, half, half + 1};
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const float bv = bf2f(bias[lr + off[i]]);
        e[i] = Q4 ? rb(rb(v[i]) + bv) : rb(v[i] + bv);
    }
    if (which < 2) {  // MLX fast::rope, non-traditional: pairs (d, d + hd/2)
#pragma unroll
        for (int i = 0; i < 2; i++) {
            const int d = (lr + i) % a.hd;
            const float inv_freq = exp2f(-((float)d / (float)half) * a.log2_theta);
            const float th = (float)a.pos * inv_freq;
            const float cs = cosf(th), sn = sinf(th);
            const float x1 = e[i], x2 = e[i + 2];
            const float o1 = x1 * cs - x2 * sn, o2 = x1 * sn + x2 * cs;
            e[i] = rb(o1);
            e[i + 2] = rb(o2);
        }
    }
    uint64_t* tq = a.tq + (size_t)l * (nq / 2);
    const uint32_t w_lo = pack_bf2(e[0], e[1]), w_hi = pack_bf2(e[2], e[3]);
    tstore(tq + cr / 2, w_lo, a.epoch);
    tstore(tq + (cr + half) / 2, w_hi, a.epoch);
    uint32_t* pq = reinterpret_cast<uint32_t*>(a.qkv + l * a.sq);
    pq[cr / 2] = w_lo;
    pq[(cr + half) / 2] = w_hi;
    if (which > 0) {
        uint16_t* cache = which == 1 ? a.kc : a.vc;
        const int kh = lr / a.hd, d = lr % a.hd;
        uint32_t* dst = reinterpret_cast<uint32_t*>(cache + (((size_t)l * a.kvh + kh) * a.cap + a.pos) * a.hd);
        dst[d / 2] = w_lo;
        dst[(d + half) / 2] = w_hi;
    }
}

// ---- LB: split-K GQA attention + last-arriver merge ----------------------------
// Unit = (kv head g, split of positions), on the last workgroups of the grid.
// The split is walked in tiles of 64 positions: each thread loads one 16 B
// chunk of K and one of V per tile (the next tile's loads are issued before
// the current one is computed); scores use 8 lanes per position, the online
// softmax one wave per head, P.V one thread per (head, dim).
struct ALds {
    float* q;       // [8][64]
    uint16_t* k;    // [64][64]
    uint16_t* v;    // [64][64]
    float* p;       // [8][64]
    float* ml;      // [8][4]: running max, running sum, tile correction
    uint32_t* kn;   // [32] new k row (bf16 pairs)
    uint32_t* vn;   // [32] new v row
    float* mw;      // merge: [8][64] split weights
    float* mlsum;   // merge: [8]
};

__device__ __forceinline__ ALds alds(uint32_t* lds) {
    ALds s;
    s.q = reinterpret_cast<float*>(lds);
    s.k = reinterpret_cast<uint16_t*>(lds + 512);
    s.v = reinterpret_cast<uint16_t*>(lds + 2560);
    s.p = reinterpret_cast<float*>(lds + 4608);
    s.ml = reinterpret_cast<float*>(lds + 5120);
    s.kn = lds + 5152;
    s.vn = lds + 5184;
    s.mw = reinterpret_cast<float*>(lds + 5216);
    s.mlsum = reinterpret_cast<float*>(lds + 5728);
    return s;
}

__device__ void st_attn(const Ctx& c, int l) {
    const StepArgs& a = c.a;
    const int n = a.pos + 1, ns = (n + a.split_len - 1) / a.split_len, grp = a.heads / a.kvh, hd = a.hd;
    const int U = a.kvh * ns;
    const int u = c.G - 1 - c.wg;  // attention units on the last workgroups
    if (u < 0 || u >= U) return;
    const int g = u / ns, sp = u % ns;
    const int j0 = sp * a.split_len, j1 = min(n, j0 + a.split_len);
    const ALds S = alds(c.lds);
    const int t = threadIdx.x;
    const uint16_t* kbase = a.kc + (((size_t)l * a.kvh + g) * a.cap) * hd;
    const uint16_t* vbase = a.vc + (((size_t)l * a.kvh + g) * a.cap) * hd;
    const int trow = t / 8, tcol = t % 8;  // this thread's 16 B chunk of a 64 x 128 B tile
    uint4 kr, vr;
    // cached rows (< pos) come from the cache; row pos from the tagged q|k|v
    auto load_tile = [&](int t0) {
        const int row = t0 + trow;
        if (row < j1 && row < a.pos) {
            kr = ldg4(kbase + (size_t)row * hd + 8 * tcol);
            vr = ldg4(vbase + (size_t)row * hd + 8 * tcol);
        } else {
            kr = make_uint4(0, 0, 0, 0);
            vr = make_uint4(0, 0, 0, 0);
        }
    };
    load_tile(j0);
    const int nq = a.H + 2 * a.kvh * hd;
    const uint64_t* tq = a.tq + (size_t)l * (nq / 2);
    const float scale = 1.0f / sqrtf((float)hd);
    for (int i = t; i < grp * hd / 2; i += kT) {
        const uint32_t w = trecv1(tq + (g * grp * hd) / 2 + i, a.epoch, a.flags);
        S.q[2 * i] = scale * bf_lo(w);
        S.q[2 * i + 1] = scale * bf_hi(w);
    }
    if (j1 > a.pos && t < hd) {  // this split holds the new row
        const uint64_t* src =
            t < hd / 2 ? tq + (a.H + g * hd) / 2 + t : tq + (a.H + a.kvh * hd + g * hd) / 2 + t - hd / 2;
        const uint32_t w = trecv1(src, a.epoch, a.flags);
        if (t < hd / 2)
            S.kn[t] = w;
        else
            S.vn[t - hd / 2] = w;
    }
    if (t < 32) S.ml[t] = (t % 4 == 0) ? -INFINITY : 0.0f;
    stamp(a, slot_in(l, 1));
    const int hp = t / 64, d = t % 64;  // P.V: thread owns dim d of head hp
    float acc = 0.0f;
    for (int t0 = j0; t0 < j1; t0 += kTile) {
        const int cnt = min(kTile, j1 - t0);
        __syncthreads();
        reinterpret_cast<uint4*>(S.k)[t] = kr;
        reinterpret_cast<uint4*>(S.v)[t] = vr;
        __syncthreads();
        if (a.pos >= t0 && a.pos < t0 + cnt && t < hd / 2) {  // new row
            reinterpret_cast<uint32_t*>(S.k + (a.pos - t0) * hd)[t] = S.kn[t];
            reinterpret_cast<uint32_t*>(S.v + (a.pos - t0) * hd)[t] = S.vn[t];
        }
        __syncthreads();
        if (t0 + kTile < j1) load_tile(t0 + kTile);
        {   // scores: 8 lanes per position, 8 dims each
            const int p = t >> 3, qt = t & 7;
            const uint4 kk = *reinterpret_cast<const uint4*>(S.k + p * hd + qt * 8);
            const uint32_t kw[4] = {kk.x, kk.y, kk.z, kk.w};
            for (int h = 0; h < grp; h++) {
                const float* qh = S.q + h * hd + qt * 8;
                float s = 0.0f;
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    s += qh[2 * i] * bf_lo(kw[i]);
                    s += qh[2 * i + 1] * bf_hi(kw[i]);
                }
                s = team_sum<8>(s);
                if (qt == 0) S.p[h * kTile + p] = p < cnt ? s : -INFINITY;
            }
        }
        __syncthreads();
        if (c.wave < grp) {  // online softmax, one wave per head, lane = position
            const int h = c.wave;
            const float s = S.p[h * kTile + c.lane];
            const float mt = team_max<kWave>(s);
            const float mo = S.ml[4 * h], mn = fmaxf(mo, mt);
            const float e = c.lane < cnt ? expf(s - mn) : 0.0f;
            S.p[h * kTile + c.lane] = e;
            const float sum = team_sum<kWave>(e);
            if (c.lane == 0) {
                const float corr = expf(mo - mn);  // 0 on the first tile
                S.ml[4 * h] = mn;
                S.ml[4 * h + 1] = S.ml[4 * h + 1] * corr + sum;
                S.ml[4 * h + 2] = corr;
            }
        }
        __syncthreads();
        if (hp < grp) {
            const float* ph = S.p + hp * kTile;
            float s0 = 0.0f, s1 = 0.0f;
#pragma unroll 8
            for (int p = 0; p < kTile; p += 2) {  // probabilities past cnt are 0
                s0 += ph[p] * bf2f(S.v[p * hd + d]);
                s1 += ph[p + 1] * bf2f(S.v[(p + 1) * hd + d]);
            }
            acc = acc * S.ml[4 * hp + 2] + (s0 + s1);
        }
    }
    __syncthreads();
    // partials: device-coherent stores, completed before the arrival
    if (hp < grp) {
        float* out = a.part + ((size_t)(g * ns + sp) * grp + hp) * (hd + 2);
        cstore(out + 2 + d, acc);
        if (d == 0) {
            cstore(out, S.ml[4 * hp]);
            cstore(out + 1, S.ml[4 * hp + 1]);
        }
    }
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    int* last = reinterpret_cast<int*>(c.lds + kFlagOff);
    if (t == 0) {
        int* ctr = a.counters + l * a.kvh + g;
        const int old = __hip_atomic_fetch_add(ctr, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        *last = old == ns - 1;
        if (old == ns - 1) __hip_atomic_store(ctr, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    if (!*last) return;
    // merge the ns (<= 64) splits of the grp heads of kv head g
    const float* pbase = a.part + (size_t)(g * ns) * grp * (hd + 2);
    const size_t sstride = (size_t)grp * (hd + 2);
    if (c.wave < grp) {
        const int h = c.wave;
        const float m = c.lane < ns ? cload(pbase + c.lane * sstride + h * (hd + 2)) : -INFINITY;
        const float lsum = c.lane < ns ? cload(pbase + c.lane * sstride + h * (hd + 2) + 1) : 0.0f;
        const float M = team_max<kWave>(m);
        const float w = c.lane < ns ? expf(m - M) : 0.0f;
        const float lw = team_sum<kWave>(w * lsum);
        S.mw[h * 64 + c.lane] = w;
        if (c.lane == 0) S.mlsum[h] = lw;
    }
    __syncthreads();
    if (hp < grp) {
        constexpr int B = 8;
        float o = 0.0f;
        for (int s0 = 0; s0 < ns; s0 += B) {
            float v[B];
#pragma unroll
            for (int i = 0; i < B; i++)
                v[i] = s0 + i < ns ? cload(pbase + (s0 + i) * sstride + hp * (hd + 2) + 2 + d) : 0.0f;
#pragma unroll
            for (int i = 0; i < B; i++)
                if (s0 + i < ns) o += v[i] * S.mw[hp * 64 + s0 + i];
        }
        const float val = o / S.mlsum[hp];
        const float nxt = __shfl_down(val, 1, kWave);
        const int col = (g * grp + hp) * hd + d;
        if ((d & 1) == 0) {
            const uint32_t w = pack_bf2(val, nxt);
            tstore(a.ta + (size_t)l * (a.H / 2) + col / 2, w, a.epoch);
            reinterpret_cast<uint32_t*>(a.att + l * a.sx)[col / 2] = w;
        }
    }
}

// ---- LC: o_proj + residual (unit = row pair, packed) -----------------------------
template <int Q4>
struct OW {
    RowRegs<Nc<Q4>::t32> w;
};

template <int Q4>
__device__ void o_load(const Ctx& c, const LayerDev& Ld, OW<Q4>& W) {
    const int p = c.wg * kW + c.wave;
    if (p < c.a.H / 2) row_load<Q4, 32, Nc<Q4>::t32>(Ld.o, 2 * p + c.team, c.tl, 0, W.w);
}

template <int Q4>
__device__ void st_o(const Ctx& c, const LayerDev& Ld, int l, const OW<Q4>& W) {
    const StepArgs& a = c.a;
    const int nunits = a.H / 2;
    if (c.wg * kW >= nunits) return;
    const int p = c.wg * kW + c.wave;
    const bool has = p < nunits;
    const int r = 2 * p + c.team;
    const uint64_t* xsrc = a.tx + (size_t)l * (a.H / 2) + p;  // residual, produced two stages ago
    const uint64_t xpre = has && c.lane == 0 ? tload(xsrc) : 0;
    recv_stage<Q4>(c, a.ta + (size_t)l * (a.H / 2), a.H, nullptr);
    stamp(a, slot_in(l, 2));
    if (!has) return;
    const float acc = row_dot_pf<Q4, 32, Nc<Q4>::t32>(Ld.o, r, xs_of(c.lds, a.H), c.tl, W.w);
    const float a0 = __shfl(acc, 0, kWave), a1 = __shfl(acc, 32, kWave);
    if (c.lane == 0) {
        const uint32_t xw = tfinish(xsrc, xpre, a.epoch, a.flags);
        const uint32_t w = pack_bf2(bf_lo(xw) + rb(a0), bf_hi(xw) + rb(a1));
        tstore(a.tx1 + (size_t)l * (a.H / 2) + p, w, a.epoch);
        reinterpret_cast<uint32_t*>(a.x1 + l * a.sx)[p] = w;
    }
}

// ---- LD: rms(ln2) + gate/up + swiglu (unit = output pair, spread) -----------------
// Unit p -> workgroup p % G, slot p / G; slot s -> wave s % kW.  Team 0 takes
// the gate rows 2p, 2p+1, team 1 the up rows.
template <int Q4>
struct UpW {
    RowRegs<Nc<Q4>::t32> w[Nc<Q4>::up_units][2];
};

__device__ __forceinline__ int up_slots(const Ctx& c) { return (c.a.I / 2 - c.wg + c.G - 1) / c.G; }

template <int Q4>
__device__ void up_load(const Ctx& c, const LayerDev& Ld, UpW<Q4>& W) {
    const int slots = up_slots(c);
    const LinearDev& L = c.team == 0 ? Ld.g : Ld.u;
#pragma unroll
    for (int i = 0; i < Nc<Q4>::up_units; i++) {
        const int s = c.wave + i * kW;
        if (s < slots) {
            const int p = c.wg + s * c.G;
            row_load<Q4, 32, Nc<Q4>::t32>(L, 2 * p, c.tl, 0, W.w[i][0]);
            row_load<Q4, 32, Nc<Q4>::t32>(L, 2 * p + 1, c.tl, 0, W.w[i][1]);
        }
    }
}

template <int Q4>
__device__ void st_up(const Ctx& c, const LayerDev& Ld, int l, const UpW<Q4>& W) {
    const StepArgs& a = c.a;
    constexpr int MU = Nc<Q4>::up_units;
    const int slots = up_slots(c);
    if (slots <= 0) return;
    const LinearDev& L = c.team == 0 ? Ld.g : Ld.u;
    recv_stage<Q4>(c, a.tx1 + (size_t)l * (a.H / 2), a.H, Ld.ln2);
    stamp(a, slot_in(l, 3));
    const XStage st = xs_of(c.lds, a.H);
    auto finish = [&](int p, float acc0, float acc1) {
        const float g0 = rb(__shfl(acc0, 0, kWave)), g1 = rb(__shfl(acc1, 0, kWave));
        const float u0 = rb(__shfl(acc0, 32, kWave)), u1 = rb(__shfl(acc1, 32, kWave));
        if (c.lane == 0) {
            const float s0 = rb(1.0f / (1.0f + expf(-g0))), s1 = rb(1.0f / (1.0f + expf(-g1)));
            const uint32_t wv = pack_bf2(rb(g0 * s0) * u0, rb(g1 * s1) * u1);
            tstore(a.th + (size_t)l * (a.I / 2) + p, wv, a.epoch);
            reinterpret_cast<uint32_t*>(a.hh + l * a.sh)[p] = wv;
        }
    };
#pragma unroll
    for (int i = 0; i < MU; i++) {
        const int s = c.wave + i * kW;
        if (s < slots) {
            const int p = c.wg + s * c.G;
            const float acc0 = row_dot_pf<Q4, 32, Nc<Q4>::t32>(L, 2 * p, st, c.tl, W.w[i][0]);
            const float acc1 = row_dot_pf<Q4, 32, Nc<Q4>::t32>(L, 2 * p + 1, st, c.tl, W.w[i][1]);
            finish(p, acc0, acc1);
        }
    }
    // units beyond the prefetched ones (only when MU is small)
    for (int s = c.wave + MU * kW; s < slots; s += kW) {
        const int p = c.wg + s * c.G;
        RowRegs<Nc<Q4>::t32> r0, r1;
        row_load<Q4, 32, Nc<Q4>::t32>(L, 2 * p, c.tl, 0, r0);
        row_load<Q4, 32, Nc<Q4>::t32>(L, 2 * p + 1, c.tl, 0, r1);
        const float acc0 = row_dot_pf<Q4, 32, Nc<Q4>::t32>(L, 2 * p, st, c.tl, r0);
        const float acc1 = row_dot_pf<Q4, 32, Nc<Q4>::t32>(L, 2 * p + 1, st, c.tl, r1);
        finish(p, acc0, acc1);
    }
}

// ---- LE: down + residual (unit = row pair, packed) ---------------------------------
template <int Q4>
struct DownW {
    RowRegs<Nc<Q4>::down> w;
};

template <int Q4>
__device__ void down_load(const Ctx& c, const LayerDev& Ld, DownW<Q4>& W) {
    const int p = c.wg * kW + c.wave;
    if (p < c.a.H / 2) row_load<Q4, 32, Nc<Q4>::down>(Ld.d, 2 * p + c.team, c.tl, 0, W.w);
}

template <int Q4>
__device__ void st_down(const Ctx& c, const LayerDev& Ld, int l, const DownW<Q4>& W) {
    const StepArgs& a = c.a;
    const int nunits = a.H / 2;
    if (c.wg * kW >= nunits) return;
    const int p = c.wg * kW + c.wave;
    const bool has = p < nunits;
    const int r = 2 * p + c.team;
    const uint64_t* xsrc = a.tx1 + (size_t)l * (a.H / 2) + p;  // residual, produced two stages ago
    const uint64_t xpre = has && c.lane == 0 ? tload(xsrc) : 0;
    recv_stage<Q4>(c, a.th + (size_t)l * (a.I / 2), a.I, nullptr);
    stamp(a, slot_in(l, 4));
    if (!has) return;
    const float acc = row_dot_pf<Q4, 32, Nc<Q4>::down>(Ld.d, r, xs_of(c.lds, a.I), c.tl, W.w);
    const float a0 = __shfl(acc, 0, kWave), a1 = __shfl(acc, 32, kWave);
    if (c.lane == 0) {
        const uint32_t xw = tfinish(xsrc, xpre, a.epoch, a.flags);
        const uint32_t w2 = pack_bf2(bf_lo(xw) + rb(a0), bf_hi(xw) + rb(a1));
        tstore(a.tx + (size_t)(l + 1) * (a.H / 2) + p, w2, a.epoch);
        reinterpret_cast<uint32_t*>(a.xo + l * a.sx)[p] = w2;
    }
}

// ---- final norm + tied LM head + argmax ---------------------------------------------
__device__ __forceinline__ bool better(float v, int i, float bv, int bi) { return v > bv || (v == bv && i < bi); }

__device__ void block_best(float& bv, int& bi, float* rv, int* ri) {
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
    if (threadIdx.x == 0)
        for (int w = 1; w < kW; w++)
            if (better(rv[w], ri[w], bv, bi)) {
                bv = rv[w];
                bi = ri[w];
            }
}

// The head keeps kHeadDepth row pairs per wave in flight: each register slot
// is refilled with the row pair kHeadDepth positions further on as soon as it
// has been used (slots are indexed statically, the loop is unrolled by the
// depth), so the stream of head rows never waits for a whole batch.
constexpr int kHeadDepth = 8;

template <int Q4>
struct HeadW {
    RowRegs<Nc<Q4>::t32> w[kHeadDepth];
};

template <int Q4>
__device__ __forceinline__ void head_slot_load(const Ctx& c, int p, RowRegs<Nc<Q4>::t32>& w) {
    const int V = c.a.head.N, nunits = V / 2 + (V & 1);
    if (p < nunits) row_load<Q4, 32, Nc<Q4>::t32>(c.a.head, min(2 * p + c.team, V - 1), c.tl, 0, w);
}

template <int Q4>
__device__ void head_load(const Ctx& c, HeadW<Q4>& W) {
    const int nw = c.G * kW, me = c.wg * kW + c.wave;
#pragma unroll
    for (int i = 0; i < kHeadDepth; i++) head_slot_load<Q4>(c, me + i * nw, W.w[i]);
}

template <int Q4>
__device__ void st_head(const Ctx& c, HeadW<Q4>& W) {
    const StepArgs& a = c.a;
    const int V = a.head.N, nunits = V / 2 + (V & 1);
    const int nw = c.G * kW, me = c.wg * kW + c.wave;
    recv_stage<Q4>(c, a.tx + (size_t)a.n_layers * (a.H / 2), a.H, a.final_norm,
                   c.wg == 0 ? a.hidden : nullptr);
    stamp(a, slot_in(a.n_layers, 0));
    const XStage st = xs_of(c.lds, a.H);
    float bv = -INFINITY;
    int bi = 0x7fffffff;
    for (int first = me; first < nunits; first += kHeadDepth * nw) {
#pragma unroll
        for (int i = 0; i < kHeadDepth; i++) {
            const int p = first + i * nw;
            if (p < nunits) {
                const int r = min(2 * p + c.team, V - 1);
                const float acc = row_dot_pf<Q4, 32, Nc<Q4>::t32>(a.head, r, st, c.tl, W.w[i]);
                head_slot_load<Q4>(c, p + kHeadDepth * nw, W.w[i]);
                if (c.tl == 0 && 2 * p + c.team < V) {
                    if (a.logits) a.logits[r] = acc;
                    if (better(acc, r, bv, bi)) {
                        bv = acc;
                        bi = r;
                    }
                }
            }
        }
    }
    float* rv = reinterpret_cast<float*>(c.lds + kRedOff);
    int* ri = reinterpret_cast<int*>(c.lds + kRedOff + 16);
    block_best(bv, bi, rv, ri);
    if (threadIdx.x == 0) {
        cstore(a.amax_v + c.wg, bv);
        __hip_atomic_store(a.amax_i + c.wg, bi, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    int* last = reinterpret_cast<int*>(c.lds + kFlagOff);
    if (threadIdx.x == 0) {
        int* ctr = a.counters + a.n_layers * a.kvh;
        const int old = __hip_atomic_fetch_add(ctr, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        *last = old == c.G - 1;
        if (old == c.G - 1) __hip_atomic_store(ctr, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    if (!*last) return;
    bv = -INFINITY;
    bi = 0x7fffffff;
    for (int i = threadIdx.x; i < c.G; i += kT) {
        const float v = cload(a.amax_v + i);
        const int ix = __hip_atomic_load(a.amax_i + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (better(v, ix, bv, bi)) {
            bv = v;
            bi = ix;
        }
    }
    block_best(bv, bi, rv, ri);
    if (threadIdx.x == 0 && a.argmax_out) *a.argmax_out = bi == 0x7fffffff ? 0 : bi;
}


template <int Q4>
__global__ __launch_bounds__(kT) void decode_tagged_kernel(StepArgs a) {
    __shared__ uint32_t lds[kLds];
    const int lane = threadIdx.x % kWave;
    const Ctx c{a, lds, (int)gridDim.x, (int)blockIdx.x, (int)(threadIdx.x / kWave), lane, lane / 32, lane % 32};
    stamp(a, 0);
    QkvW<Q4> qw;
    OW<Q4> ow;
    UpW<Q4> uw;
    DownW<Q4> dw;
    qkv_load<Q4>(c, a.layers[0], qw);
    st_embed(c);
    for (int l = 0; l < a.n_layers; l++) {
        const LayerDev& Ld = a.layers[l];
        o_load<Q4>(c, Ld, ow);
        st_qkv<Q4>(c, Ld, l, qw);
        __syncthreads();
        stamp(a, slot_in(l, 0) + 1);
        st_attn(c, l);
        __syncthreads();
        stamp(a, slot_in(l, 1) + 1);
        up_load<Q4>(c, Ld, uw);
        st_o<Q4>(c, Ld, l, ow);
        __syncthreads();
        stamp(a, slot_in(l, 2) + 1);
        down_load<Q4>(c, Ld, dw);
        st_up<Q4>(c, Ld, l, uw);
        __syncthreads();
        stamp(a, slot_in(l, 3) + 1);
        if (l + 1 < a.n_layers) qkv_load<Q4>(c, a.layers[l + 1], qw);
        st_down<Q4>(c, Ld, l, dw);
        __syncthreads();
        stamp(a, slot_in(l, 4) + 1);
    }
    HeadW<Q4> hw;
    head_load<Q4>(c, hw);
    st_head<Q4>(c, hw);
    stamp(a, slot_in(a.n_layers, 0) + 1);
}

}  // namespace

// Positions per attention split on this schedule: a multiple of the 64-row
// tile, doubled until a kv head has at most 24 splits (each split is one
// workgroup; the last one to finish merges them).
int tagged_split_len(int n) {
    int sl = kTile;
    while ((n + sl - 1) / sl > 24 && sl < 16 * kTile) sl *= 2;
    return sl;
}

hipError_t launch_lm_step_tagged(hipStream_t st, const StepArgs& a, int q4, int grid) {
    StepArgs args = a;
    void* params[] = {&args};
    const void* f = q4 ? reinterpret_cast<const void*>(decode_tagged_kernel<1>)
                       : reinterpret_cast<const void*>(decode_tagged_kernel<0>);
    return hipLaunchCooperativeKernel(f, dim3(grid), dim3(kT), params, 0, st);
}

int tagged_grid(int num_cus) {
    int per_cu = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, decode_tagged_kernel<1>, kT, 0) != hipSuccess ||
        per_cu < 1)
        return 0;
    return num_cus;
}

}  // namespace ming
