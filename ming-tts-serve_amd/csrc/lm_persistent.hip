// One persistent kernel per decode token (the whole of QStack.decodeFused,
// src/ming_model.zig:530-544, plus the tied LM head and argmax), with the
// stages handing their outputs over through tagged words and per-XCD hubs
// instead of grid barriers.
//
// Producers: a stage's output vector is written as u64 words {bf16 pair,
// epoch} with device-coherent (sc1) stores.  Data and tag travel in one
// single-copy-atomic word, so no fence (no L2 write-back or invalidate) is
// needed.  Buffers start zeroed and epochs start at 1, so a stale word never
// matches.
//
// Hubs: workgroups 0..7 run one per XCD (the dispatcher places workgroup i on
// XCD i % 8; every workgroup reads its XCC id, and a workgroup whose XCD has
// no hub polls and stages its inputs itself).  A hub polls each stage's input
// vector with device-coherent loads, rms-normalises it where the stage does,
// builds the GEMV stage image (nibble pair order plus chunk sums) and writes
// it with ordinary stores, which stay in its XCD's L2.  A flag raised after
// the image's stores have completed tells the workers of the XCD to copy the
// image into LDS with device-scope loads, which the L2 serves because the
// lines were written on this XCD.  A broadcast to 248 workgroups thus costs 8
// device-coherent readers instead of 248, and a waiting worker polls one
// word instead of the whole vector.
//
// Overlap: in a worker, wave 0 receives each stage's input while waves 1..7
// have the stage's weight loads in flight.  Vector loads complete in issue
// order, so a wave with outstanding weight loads could not see a poll result
// before its weights; the split keeps the receive path free of them.  A
// worker issues a stage's loads as soon as it enters the stage, which for
// most workers is long before the input arrives (they skip the stages in
// between), and attention workers hold their split's K/V in LDS before they
// wait for q.
//
// Attention splits hold their K rows and V^T in LDS, loaded a layer ahead,
// and meet through a per-(layer, kv head) arrival counter: the workgroup that
// arrives last merges the partials.  The LM head's per-workgroup argmax
// partials meet the same way.  Partials are written with device-coherent
// stores and waited on (s_waitcnt) before the arrival.
//
// Every wait is bounded: past the spin limit a workgroup raises flags[0] and
// continues, so the grid always drains; the host reports MING_E_TIMEOUT.
// The kernel needs all workgroups co-resident (cooperative launch).
#include "gemv.h"
#include "internal.h"
#include "tagged.h"

namespace ming {

namespace {

constexpr int kT = 512;          // threads per workgroup (8 waves, 2 per SIMD)
constexpr int kW = kT / kWave;   // waves per workgroup
constexpr int kCW = kW - 1;      // compute waves (1..7); wave 0 receives each stage's input
constexpr int kLds = 12288;      // LDS words (48 KB)
constexpr int kXsOff = 0;        // stage image, K <= 8192: 4352 words (+3 copy padding)
constexpr int kRedOff = 9520;    // reduction scratch (64 words)
constexpr int kFlagOff = 9584;   // broadcast flags (16 words)
constexpr int kLayOff = 12288;   // the layer table, copied once per launch: a stage's weight pointers and
                                 // shapes are then LDS reads, not global loads that would queue behind prefetches
constexpr int kMaxLdsLayers = 32;
constexpr int kLayWords = (int)(sizeof(LayerDev) / 4);
constexpr int kLdsTotal = kLayOff + kMaxLdsLayers * kLayWords;
static_assert(sizeof(LayerDev) % 8 == 0, "layer table entries must keep 8-byte alignment in LDS");
// Attention: a split of kAttTiles tiles of kTileP positions per workgroup, its
// K rows and V^T resident in LDS after the layer table.  Four tiles of 96
// positions take one compute wave on each SIMD (six of 64 put two on two SIMDs).
constexpr int kTileP = 96;
constexpr int kTileSub = kTileP / 16;  // 16-position score sub-tiles of a tile
constexpr int kTileU = kTileP / 32;    // 32-position P.V chunks of a tile
constexpr int kAttTiles = 4;
constexpr int kAttP = kAttTiles * kTileP;     // positions per split
constexpr int kVtRowP = kAttP / 2 + 4;        // u32 per V^T row (position pairs), padded: conflict-free reads
constexpr int kKvOff = kLdsTotal;             // K rows [kAttP][64] bf16
constexpr int kVtOffP = kKvOff + kAttP * 32;  // V^T [64][kVtRowP]
constexpr int kLdsAll = kVtOffP + 64 * kVtRowP;
constexpr int kAttOt = 5248;                  // the tiles' partials [kAttTiles][8][66] f32 (attention stage)
constexpr int kAttWords = 5248;               // a merged attention row, H/2 u32 (o_proj staging)
static_assert(kKvOff % 4 == 0 && kVtOffP % 4 == 0 && kVtRowP % 4 == 0, "16-byte LDS operands");
static_assert(kLdsAll * 4 <= 160 * 1024, "LDS of one workgroup");
static_assert(kAttOt + kAttTiles * 8 * 66 <= kRedOff, "attention partials below the reduction scratch");
constexpr int kSc1 = 16;         // buffer-load cache policy bit: device scope

// A tagged word for readers on this workgroup's own XCD (loc): a plain store,
// which stays in the XCD's L2 where the readers' device-scope loads find it;
// otherwise device-coherent.
__device__ __forceinline__ void tstore_loc(uint64_t* p, uint32_t payload, uint32_t tag, bool loc) {
    if (loc)
        gst(p, ((uint64_t)tag << 32) | payload);
    else
        tagged::tstore(p, payload, tag);
}

template <int Q4>
struct Nc {
    static constexpr int t32 = Q4 ? 1 : 4;   // chunks per lane, K = hidden
    static constexpr int down = Q4 ? 5 : 5;  // chunks per lane, K = inter (32-lane teams)
    static constexpr int up_units = Q4 ? 2 : 1;
};

using namespace tagged;

// Optional profile: wall-clock stamps of this workgroup.  Slot 0 is the
// kernel start; stage s (0 qkv, 1 attn, 2 o, 3 up, 4 down) of layer l has
// slot 1 + 2 (5 l + s) when its input has arrived and the next slot when it is
// done; the head takes the two slots after the last layer.
__device__ __forceinline__ void stamp(const StepArgs& a, int k) {
    if (a.tstamp && tix() == 0) gst(a.tstamp + (size_t)k * gridDim.x + blockIdx.x, (uint64_t)wall_clock64());
}
__device__ __forceinline__ int slot_in(int l, int s) { return 1 + 2 * (5 * l + s); }
// A stage's "done" stamp, taken when every wave of the workgroup is done.
__device__ __forceinline__ void done_stamp(const StepArgs& a, int k) {
    if (a.tstamp) {
        lds_sync();
        stamp(a, k);
    }
}

// A worker: W workers, this one is w; hub is the hub workgroup of its XCD
// (or -1: stage inputs itself).
struct Ctx {
    const StepArgs& a;
    uint32_t* lds;
    int W, w, wave, lane, team, tl, hub;
};

__device__ __forceinline__ XStage xs_of(uint32_t* lds, int K) {
    return XStage{lds + kXsOff, reinterpret_cast<float*>(lds + kXsOff + K / 2)};
}

// ---- stage images ------------------------------------------------------------------
// Receive the tagged bf16 vector src [K/2 words], optionally rms-normalise it
// with norm_w (MLX fast::rms_norm: bf16(w * bf16(x * rsqrt(mean(x^2) + eps)))),
// and write its GEMV stage image to dst (LDS or global): xs [K/2] and, for
// affine weights, the chunk sums xh [K/32] right after it.  `hidden`, if not
// null, receives the (normalised) vector.  Thread t owns the 8-value groups
// t and t + kT (K <= 8192).  All threads of the block call it.
template <int Q4, bool TO_LDS>
__device__ __forceinline__ void image_finish(const StepArgs& a, uint32_t* lds, uint32_t (&v)[8], const uint4 (&nw)[2],
                                             int K, const uint16_t* norm_w, uint32_t* dst, uint16_t* hidden,
                                             int stamp_slot);

template <int Q4, bool TO_LDS>
__device__ __forceinline__ void build_image(const StepArgs& a, uint32_t* lds, const uint64_t* src, int K,
                                            const uint16_t* norm_w, uint32_t* dst, uint16_t* hidden,
                                            int stamp_slot = -1) {
    const int ng = K / 8;
    uint4 nw[2];
#pragma unroll
    for (int p = 0; p < 2; p++) {
        const int g = tix() + p * kT;
        nw[p] = (norm_w && g < ng) ? ldg4(norm_w + 8 * g) : make_uint4(0, 0, 0, 0);
    }
    uint32_t v[8];
    trecv_groups<kT>(src, ng, a.epoch, v, a.flags);
    image_finish<Q4, TO_LDS>(a, lds, v, nw, K, norm_w, dst, hidden, stamp_slot);
}

// The rest of build_image for the groups v[] a thread holds (groups t and
// t + kT of the vector, 4 u32 each), with its rms weight chunks nw.  dst is
// LDS (a worker staging for itself) or global memory (a hub image).
template <int Q4, bool TO_LDS>
__device__ __forceinline__ void image_finish(const StepArgs& a, uint32_t* lds, uint32_t (&v)[8], const uint4 (&nw)[2],
                                             int K, const uint16_t* norm_w, uint32_t* dst, uint16_t* hidden,
                                             int stamp_slot) {
    auto put4 = [&](int word, uint4 v) {
        if (TO_LDS)
            *reinterpret_cast<uint4*>(dst + word) = v;
        else
            gst(reinterpret_cast<uint4*>(dst + word), v);
    };
    auto put1 = [&](int word, float v) {
        if (TO_LDS)
            reinterpret_cast<float*>(dst)[word] = v;
        else
            gst(reinterpret_cast<float*>(dst) + word, v);
    };
    const int ng = K / 8, NC = K / 32;
    if (norm_w) {
        float ss = 0.0f;
#pragma unroll
        for (int k = 0; k < 8; k++) {
            const float lo = bf_lo(v[k]), hi = bf_hi(v[k]);
            ss += lo * lo;
            ss += hi * hi;
        }
        ss = block_sum(ss, reinterpret_cast<float*>(lds + kRedOff));
        if (stamp_slot >= 0) stamp(a, stamp_slot);  // past block_sum's barrier: every group received
        const float inv = 1.0f / sqrtf(ss / (float)K + a.eps);
#pragma unroll
        for (int p = 0; p < 2; p++) {
            const uint32_t wn[4] = {nw[p].x, nw[p].y, nw[p].z, nw[p].w};
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const uint32_t x = v[4 * p + j];
                v[4 * p + j] = pack_bf2(bf_lo(wn[j]) * rb(bf_lo(x) * inv), bf_hi(wn[j]) * rb(bf_hi(x) * inv));
            }
        }
    }
#pragma unroll
    for (int p = 0; p < 2; p++) {
        const int g = tix() + p * kT;
        const bool act = g < ng;
        const uint4 x = make_uint4(v[4 * p], v[4 * p + 1], v[4 * p + 2], v[4 * p + 3]);
        if (hidden && act) gst(reinterpret_cast<uint4*>(hidden + 8 * g), x);
        if (Q4) {
            float s;
            const uint4 o = q4_group(x, s);
            if (act) put4(((g & 3) * NC + (g >> 2)) * 4, o);
            s = team_sum<4>(s);  // ng is a multiple of 4: a quad of lanes is active or idle together
            if (act && (g & 3) == 0) put1(K / 2 + (g >> 2), s);
        } else if (act) {
            put4(4 * g, x);
        }
    }
}

// Worker: the stage image of flag fidx / image slot `slot` into LDS (xs at
// kXsOff).  With a hub serving this stage, wave 0 waits for its flag and
// copies the image (waves 1..7 meanwhile have their weight loads in flight);
// otherwise all waves build it here.  The first barrier also ends the previous stage's use of LDS.
__device__ __forceinline__ bool hub_on(const StepArgs& a, int stage) { return a.nhubs > 0 && (a.hub_stages & stage); }

template <int Q4>
__device__ __forceinline__ void copy_hub_image(const Ctx& c, int fidx, int slot, int K);

template <int Q4>
__device__ __forceinline__ void get_image(const Ctx& c, int stage, int fidx, int slot, const uint64_t* src, int K,
                                          const uint16_t* norm_w, uint16_t* hidden) {
    const StepArgs& a = c.a;
    if (c.hub < 0 || !(a.hub_stages & stage)) {
        lds_sync();
        build_image<Q4, true>(a, c.lds, src, K, norm_w, c.lds + kXsOff, hidden);
        lds_sync();
        return;
    }
    copy_hub_image<Q4>(c, fidx, slot, K);
}

// Worker: wave 0 waits for the hub's flag fidx and copies image slot `slot`
// (an image of K values) into LDS.
template <int Q4>
__device__ __forceinline__ void copy_hub_image(const Ctx& c, int fidx, int slot, int K) {
    const StepArgs& a = c.a;
    if (c.wave == 0 && c.lane == 0) wait_flag(a.hflag + (size_t)c.hub * a.nflag + fidx, a.epoch, a.flags);
    lds_sync();
    if (c.wave == 0) {
        // direct buffer loads into LDS: lane l's 16 bytes land at the round's
        // base + 16 l; the last round's lanes past the image read past it
        // inside the slot's range (or get zeros beyond the range) and write
        // inside the stage-image area, which holds K <= 8192
        const int n4 = ((Q4 ? K / 2 + K / 32 : K / 2) + 3) / 4;
        const uint32_t* img = a.img + ((size_t)c.hub * kImgSlots + slot) * a.img_stride;
        const __amdgpu_buffer_rsrc_t rs =
            __builtin_amdgcn_make_buffer_rsrc(const_cast<uint32_t*>(img), 0, a.img_stride * 4, 0x00020000);
        for (int i0 = 0; i0 < n4; i0 += kWave)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (__attribute__((address_space(3))) void*)(c.lds + kXsOff + 4 * i0),
                                                     16, (i0 + c.lane) * 16, 0, 0, kSc1);
        __builtin_amdgcn_s_waitcnt(0);
    }
    lds_sync();
}

// Hub: build and publish one stage image, then raise its flag.  The barrier
// waits for every thread's stores to complete (its release fence drains the
// memory counters), so the flag is raised after the whole image is in L2.
// With stage stamps on, a hub writes the stage's slots as a worker does: its
// input arrived (for a normalised stage: every group received), and done
// (the flag raised).
template <int Q4>
__device__ __forceinline__ void hub_publish(const StepArgs& a, uint32_t* lds, const uint64_t* src, int K, const uint16_t* norm_w,
                            uint32_t* img, uint32_t* flag, uint16_t* hidden, int slot) {
    build_image<Q4, false>(a, lds, src, K, norm_w, img, hidden, norm_w ? slot : -1);
    __syncthreads();
    if (tix() == 0) gst(flag, a.epoch);
    stamp(a, slot + 1);
}

template <int Q4>
__device__ __forceinline__ void hub_main(const StepArgs& a, const LayerDev* __restrict__ layers, uint32_t* lds, int b,
                                         uint32_t xcc) {
    if (tix() == 0) tstore(a.hubtab + b, xcc, a.epoch);
    uint32_t* img = a.img + (size_t)b * kImgSlots * a.img_stride;
    uint32_t* fl = a.hflag + (size_t)b * a.nflag;
    const int H = a.H, L = a.n_layers;
    const size_t st = a.img_stride;
    for (int l = 0; l < L; l++) {
        const LayerDev& Ld = layers[l];
        const int hs = a.hub_stages;
        if (hs & HUB_QKV)
            hub_publish<Q4>(a, lds, a.tx + (size_t)l * (H / 2), H, Ld.ln1, img, fl + 4 * l, nullptr, slot_in(l, 0));
        if (hs & HUB_O)
            hub_publish<Q4>(a, lds, a.ta + (size_t)l * (H / 2), H, nullptr, img + st, fl + 4 * l + 1, nullptr,
                            slot_in(l, 2));
        if (hs & HUB_UP)
            hub_publish<Q4>(a, lds, a.tx1 + (size_t)l * (H / 2), H, Ld.ln2, img + 2 * st, fl + 4 * l + 2, nullptr,
                            slot_in(l, 3));
        if (hs & HUB_DOWN)
            hub_publish<Q4>(a, lds, a.th + (size_t)l * (a.I / 2), a.I, nullptr, img + 3 * st, fl + 4 * l + 3, nullptr,
                            slot_in(l, 4));
    }
    if (a.hub_stages & HUB_HEAD)
        hub_publish<Q4>(a, lds, a.tx + (size_t)L * (H / 2), H, a.final_norm, img + 4 * st, fl + 4 * L,
                        b == 0 ? a.hidden : nullptr, slot_in(L, 0));
}

// Worker: the first hub whose XCC id equals this workgroup's, or -1.
__device__ __forceinline__ int find_hub(const StepArgs& a, uint32_t* lds, uint32_t xcc) {
    int* sel = reinterpret_cast<int*>(lds + kFlagOff + 1);
    if (tix() < kWave) {
        uint32_t hx = 0xffffffffu;
        if ((int)tix() < a.nhubs) hx = trecv1(a.hubtab + tix(), a.epoch, a.flags);
        const unsigned long long m = __ballot(hx == xcc);
        if (tix() == 0) *sel = m ? __ffsll(m) - 1 : -1;
    }
    __syncthreads();
    return *sel;
}

// ---- embed / input row -> tx[0] ----------------------------------------------
__device__ __forceinline__ void st_embed(const Ctx& c) {
    const StepArgs& a = c.a;
    const int nw = a.H / 2;
    for (int i = c.w * kT + tix(); i < nw; i += c.W * kT) {
        uint32_t v;
        if (a.token_in) {
            const LinearDev& E = a.embed;
            int id = gld(a.token_in);
            id = id < 0 ? 0 : (id >= E.N ? E.N - 1 : id);
            const int k = 2 * i;
            if (E.kind == 1) {
                const uint32_t word = gld(E.w + (size_t)id * (E.K / 8) + k / 8);
                const float sc = bf2f(gld(E.s + (size_t)id * (E.K / 64) + k / 64));
                const float bi = bf2f(gld(E.b + (size_t)id * (E.K / 64) + k / 64));
                float v0 = sc * (float)((word >> (4 * (k % 8))) & 0xfu) + bi;
                float v1 = sc * (float)((word >> (4 * (k % 8) + 4)) & 0xfu) + bi;
                if (E.gscale != 1.0f) {
                    v0 *= E.gscale;
                    v1 *= E.gscale;
                }
                v = pack_bf2(v0, v1);
            } else {
                v = gld(reinterpret_cast<const uint32_t*>(E.w) + ((size_t)id * E.K + k) / 2);
            }
            gst(reinterpret_cast<uint32_t*>(a.x) + i, v);
        } else {
            v = gld(reinterpret_cast<const uint32_t*>(a.x) + i);
        }
        tstore(a.tx + i, v, a.epoch);
    }
}

// ---- LA: q/k/v + bias + rope ----------------------------------------------------
// Unit = quad of rows (c, c+1, c+hd/2, c+hd/2+1) of the concatenated [q|k|v]
// rows, c even; team 0 computes the first two, team 1 the other two, so each
// output word (c, c+1) has one writer.  Units are packed on the compute waves:
// unit = w*kCW + wave - 1.
struct QkvGeom {
    bool any, has;
    int cr, which, base, r0;
};

__device__ __forceinline__ QkvGeom qkv_geom(const Ctx& c) {
    const StepArgs& a = c.a;
    const int half = a.hd / 2, kvd = a.kvh * a.hd, nq = a.H + 2 * kvd;
    const int nunits = nq / 4, qpb = half / 2;  // quads per head block
    QkvGeom g;
    const int u = c.w * kCW + c.wave - 1;
    g.any = c.w * kCW < nunits;
    g.has = c.wave > 0 && u < nunits;
    const int q = max(0, min(u, nunits - 1));
    g.cr = (q / qpb) * a.hd + (q % qpb) * 2;  // concatenated row c
    g.which = g.cr < a.H ? 0 : (g.cr < a.H + kvd ? 1 : 2);
    g.base = g.which == 0 ? 0 : (g.which == 1 ? a.H : a.H + kvd);
    g.r0 = g.cr - g.base + c.team * half;  // this team's rows r0, r0 + 1
    return g;
}

__device__ __forceinline__ bool in_qkv(const Ctx& c) { return qkv_geom(c).any; }

template <int Q4>
struct QkvW {
    RowRegs<Nc<Q4>::t32> w0, w1;
    uint32_t bias[2];    // bias pairs (lr, lr+1) and (lr+hd/2, lr+hd/2+1)
    float cs[2], sn[2];  // rope factors of dims d, d+1 (they do not depend on the input)
};

// The q/k/v stage for this wave's unit g (every wave of the workgroup calls it).
template <int Q4>
__device__ __forceinline__ void st_qkv_g(const Ctx& c, const LayerDev& Ld, int l, const QkvGeom& g,
                                         bool loc = false) {
    const StepArgs& a = c.a;
    const int half = a.hd / 2, kvd = a.kvh * a.hd, nq = a.H + 2 * kvd;
    const int cr = g.cr, which = g.which, base = g.base, r0 = g.r0, lr = cr - base;
    const LinearDev& L = which == 0 ? Ld.q : (which == 1 ? Ld.k : Ld.v);
    QkvW<Q4> W;
    if (g.has) {
        // MLX fast::rope, non-traditional: pairs (d, d + hd/2); computed
        // before the weight loads are issued, as large angles may read
        // reduction tables
#pragma unroll
        for (int i = 0; i < 2; i++) {
            const int d = (lr + i) % a.hd;
            const float inv_freq = exp2f(-((float)d / (float)half) * a.log2_theta);
            const float th = (float)a.pos * inv_freq;
            W.cs[i] = cosf(th);
            W.sn[i] = sinf(th);
        }
        asm volatile("" ::: "memory");
        const uint32_t* b32 = reinterpret_cast<const uint32_t*>(which == 0 ? Ld.bq : (which == 1 ? Ld.bk : Ld.bv));
        W.bias[0] = gld(b32 + lr / 2);
        W.bias[1] = gld(b32 + (lr + half) / 2);
        row_load<Q4, 32, Nc<Q4>::t32>(L, r0, c.tl, 0, W.w0);
        row_load<Q4, 32, Nc<Q4>::t32>(L, r0 + 1, c.tl, 0, W.w1);
    }
    get_image<Q4>(c, HUB_QKV, 4 * l, 0, a.tx + (size_t)l * (a.H / 2), a.H, Ld.ln1, nullptr);
    stamp(a, slot_in(l, 0));
    if (!g.has) return;
    const XStage st = xs_of(c.lds, a.H);
    const float acc0 = row_dot_pf<Q4, 32, Nc<Q4>::t32>(L, r0, st, c.tl, W.w0);
    const float acc1 = row_dot_pf<Q4, 32, Nc<Q4>::t32>(L, r0 + 1, st, c.tl, W.w1);
    const float v[4] = {lane_of(acc0, 0), lane_of(acc1, 0), lane_of(acc0, 32), lane_of(acc1, 32)};
    if (c.lane != 0) return;
    const float bias[4] = {bf_lo(W.bias[0]), bf_hi(W.bias[0]), bf_lo(W.bias[1]), bf_hi(W.bias[1])};
    float e[4];
#pragma unroll
    for (int i = 0; i < 4; i++) e[i] = Q4 ? rb(rb(v[i]) + bias[i]) : rb(v[i] + bias[i]);
    if (which < 2) {
#pragma unroll
        for (int i = 0; i < 2; i++) {
            const float cs = W.cs[i], sn = W.sn[i];
            const float x1 = e[i], x2 = e[i + 2];
            const float o1 = x1 * cs - x2 * sn, o2 = x1 * sn + x2 * cs;
            e[i] = rb(o1);
            e[i + 2] = rb(o2);
        }
    }
    uint64_t* tq = a.tq + (size_t)l * (nq / 2);
    const uint32_t w_lo = pack_bf2(e[0], e[1]), w_hi = pack_bf2(e[2], e[3]);
    tstore_loc(tq + cr / 2, w_lo, a.epoch, loc);
    tstore_loc(tq + (cr + half) / 2, w_hi, a.epoch, loc);
    uint32_t* pq = reinterpret_cast<uint32_t*>(a.qkv + l * a.sq);
    gst(pq + cr / 2, w_lo);
    gst(pq + (cr + half) / 2, w_hi);
    if (which > 0) {
        uint16_t* cache = which == 1 ? a.kc : a.vc;
        const int kh = lr / a.hd, d = lr % a.hd;
        uint32_t* dst = reinterpret_cast<uint32_t*>(cache + (((size_t)l * a.kvh + kh) * a.cap + a.pos) * a.hd);
        gst(dst + d / 2, w_lo);
        gst(dst + (d + half) / 2, w_hi);
    }
}

template <int Q4>
__device__ __forceinline__ void st_qkv(const Ctx& c, const LayerDev& Ld, int l) {
    st_qkv_g<Q4>(c, Ld, l, qkv_geom(c));
}

// 1 / (1 + e^-x) from the native exponential and reciprocal (about one ulp
// each; the SwiGLU rounds the result to bf16).
__device__ __forceinline__ float sigmoid_fast(float x) { return __builtin_amdgcn_rcpf(1.0f + att_exp(-x)); }

// ---- LB: split GQA attention over LDS-resident K/V + last-arriver merge ------------------
// Unit = (kv head g, split of kAttP positions), on the last workers.  A
// split's K rows and V^T stay in this workgroup's LDS: they are loaded one
// layer ahead (attn_prefetch, after the workgroup's gate/up stage of the
// layer before, or at launch for layer 0), so that once q arrives the four
// 96-position tiles of the split are computed at once, one per compute wave,
// on the matrix cores, and merged through LDS into one partial per split
// (per q head: max, sum, unnormalised output).  The splits of a kv head meet
// through a per-(layer, kv head) arrival counter: every split stores its
// partial device-coherently and waits for the stores before it counts itself
// in, and the last to arrive merges all of them (a kv head has a few splits of
// six tiles each -- 6 at ctx 2048 -- where one-tile splits made it 33).
struct ALds {
    uint4* qb;      // [64 lanes][2] the score MFMAs' B operands: q * 1/8 in bf16, per lane (head c, dims 16 j ..)
    float* ot;      // [kAttTiles][8 heads][66] each tile's (max, sum, o[64])
};

__device__ __forceinline__ ALds alds(uint32_t* lds) {
    ALds s;
    s.qb = reinterpret_cast<uint4*>(lds);
    s.ot = reinterpret_cast<float*>(lds + kAttOt);
    return s;
}

// K rows in LDS are stored with their 16-byte chunks permuted within the row
// (chunk q of row p at slot q ^ kswz(p)), so that the 16 rows that one pass
// of the score MFMAs' A-operand reads touches fall in distinct banks.
__device__ __forceinline__ int kswz(int p) { return ((p >> 2) & 6) | ((p >> 1) & 1); }

// This worker's attention unit: kv head g, positions [j0, j1) of split sp of ns.
struct AttnGeom {
    int u, ns, g, sp, j0, j1;
};

__device__ __forceinline__ int attn_splits(int pos) { return (pos + 1 + kAttP - 1) / kAttP; }

__device__ __forceinline__ AttnGeom attn_geom(const Ctx& c) {
    const StepArgs& a = c.a;
    AttnGeom q;
    const int n = a.pos + 1;
    q.ns = attn_splits(a.pos);
    const int d = c.W - 1 - c.w;  // attention units on the last workers
    if (a.att_xl) {  // split sp of kv head g on worker W-1-(8 sp + g): a kv head's splits 8 workgroups apart
        q.g = d % 8;
        q.sp = d / 8;
        q.u = q.g < a.kvh && q.sp < q.ns ? q.g * q.ns + q.sp : -1;
    } else {
        q.u = d;
        q.g = q.u / q.ns;
        q.sp = q.u % q.ns;
    }
    q.j0 = q.sp * kAttP;
    q.j1 = min(n, q.j0 + kAttP);
    return q;
}

__device__ __forceinline__ bool in_attn(const Ctx& c) {
    const AttnGeom q = attn_geom(c);
    return q.u >= 0 && q.u < c.a.kvh * q.ns;
}

// With XCD-grouped splits (att_xl), every split publishes its XCC id and reads
// those of its kv head's splits: if all agree, the kv head's partials and its
// arrival counter go through that XCD's L2 (plain stores, L2 atomics) instead
// of device-coherent memory.  The same ids give every split of a kv head the
// same answer; kept in LDS for the launch.
__device__ __forceinline__ void attn_xl_publish(const Ctx& c, uint32_t xcc) {
    if (c.a.att_xl && tix() == 0) tstore(c.a.hubtab + kAttXlBase + (c.W - 1 - c.w), xcc, c.a.epoch);
}

__device__ __forceinline__ void attn_xl_check(const Ctx& c, uint32_t xcc) {
    const StepArgs& a = c.a;
    int* xl = reinterpret_cast<int*>(c.lds + kFlagOff + 2);
    if (tix() < kWave) {
        bool same = a.att_xl != 0;
        if (same) {
            const AttnGeom q = attn_geom(c);
            const int sp = tix();
            uint32_t x = xcc;
            if (sp < q.ns) x = trecv1(a.hubtab + kAttXlBase + 8 * sp + q.g, a.epoch, a.flags);
            same = __ballot(x != xcc) == 0ull;
        }
        if (tix() == 0) *xl = same;
    }
    __syncthreads();
}

// The split's K rows [j0, j0 + kAttP) of layer l into LDS (direct buffer
// loads: each 16 bytes of a row land at the row's place, no registers) and
// its V rows through registers into V^T (u32 at vt[dim * kVtRowP + m] holds
// dimension dim of positions 2m and 2m + 1; rows 2m and 2m + 1 meet through a
// lane shuffle).  Rows the cache does not hold yet read as whatever the cache
// holds there (rows past its capacity as zeros) and are masked by the
// attention; the new row pos arrives with q.  Every wave waits for its loads.
__device__ __forceinline__ void attn_prefetch(const Ctx& c, int l) {
    const StepArgs& a = c.a;
    const AttnGeom q = attn_geom(c);
    const size_t base = (((size_t)l * a.kvh + q.g) * a.cap + q.j0) * a.hd;  // element offset of row j0
    const int rows = max(0, min(kAttP, a.cap - q.j0));
    const uint32_t nbytes = (uint32_t)rows * (uint32_t)a.hd * 2u;
    const __amdgpu_buffer_rsrc_t rk = __builtin_amdgcn_make_buffer_rsrc(a.kc + base, 0, nbytes, 0x00020000);
    const __amdgpu_buffer_rsrc_t rv = __builtin_amdgcn_make_buffer_rsrc(a.vc + base, 0, nbytes, 0x00020000);
    // K: kAttP rows x 8 chunks of 16 bytes; wave w loads rounds of 64 chunks w, w + 8, ...
    for (int i0 = kWave * c.wave; i0 < kAttP * 8; i0 += kT) {
        const int i = i0 + c.lane, r = i / 8;  // this lane fills slot i % 8 of LDS row r
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rk, (__attribute__((address_space(3))) void*)(c.lds + kKvOff + 4 * i0),
                                                 16, (8 * r + ((i % 8) ^ kswz(r))) * 16, 0, 0, 0);
    }
    // V: chunk i = tix() + kT k is row i / 8, dimensions 8 (i % 8) .. + 7
    constexpr int NV = kAttP * 8 / kT;
    uint4 vv[NV];
#pragma unroll
    for (int k = 0; k < NV; k++) {
        const auto v = __builtin_amdgcn_raw_buffer_load_b128(rv, (tix() + kT * k) * 16, 0, 0);
        vv[k] = make_uint4(v[0], v[1], v[2], v[3]);
    }
    uint32_t* vt = c.lds + kVtOffP;
    const int t = tix(), ch = t % 8;
#pragma unroll
    for (int k = 0; k < NV; k++) {
        const uint32_t e1[4] = {(uint32_t)__shfl((int)vv[k].x, c.lane + 8, kWave),
                                (uint32_t)__shfl((int)vv[k].y, c.lane + 8, kWave),
                                (uint32_t)__shfl((int)vv[k].z, c.lane + 8, kWave),
                                (uint32_t)__shfl((int)vv[k].w, c.lane + 8, kWave)};
        if (((t / 8) & 1) == 0) {
            const uint32_t e0[4] = {vv[k].x, vv[k].y, vv[k].z, vv[k].w};
            const int m = t / 16 + 32 * k;  // pair of rows 2m, 2m + 1
#pragma unroll
            for (int d = 0; d < 4; d++) {
                vt[(8 * ch + 2 * d) * kVtRowP + m] = (e0[d] & 0xffffu) | (e1[d] << 16);
                vt[(8 * ch + 2 * d + 1) * kVtRowP + m] = (e0[d] >> 16) | (e1[d] & 0xffff0000u);
            }
        }
    }
    __builtin_amdgcn_s_waitcnt(0);  // this wave's K rows are in LDS
}

// Wait for this unit's q rows (and, in the split holding position pos, the
// new k/v row, which replaces its row in the LDS K and V^T) and stage q.
__device__ __forceinline__ void attn_recv(const Ctx& c, int l) {
    const StepArgs& a = c.a;
    const AttnGeom q = attn_geom(c);
    const int grp = a.heads / a.kvh, hd = a.hd, g = q.g, t = tix();
    const ALds S = alds(c.lds);
    const int nq = a.H + 2 * a.kvh * hd;
    const uint64_t* tq = a.tq + (size_t)l * (nq / 2);
    const float scale = 1.0f / sqrtf((float)hd);
    lds_sync();  // the previous stage is done with LDS; every wave's prefetched K rows are visible
    if (t < 2 * kWave) {
        // B operand h of lane (head c, j): q of head c, dimensions 16 j + 8 h .. + 7, times 1/8 (exact in bf16)
        const int ln = t % kWave, h = t / kWave, cc = ln % 16, jj = ln / 16;
        uint4 b = make_uint4(0u, 0u, 0u, 0u);
        if (cc < grp) {
            const uint64_t* src = tq + (g * grp + cc) * (hd / 2) + 8 * jj + 4 * h;
            uint32_t w[4];
#pragma unroll
            for (int k = 0; k < 4; k++) w[k] = trecv1(src + k, a.epoch, a.flags);
#pragma unroll
            for (int k = 0; k < 4; k++) w[k] = pack_bf2(scale * bf_lo(w[k]), scale * bf_hi(w[k]));
            b = make_uint4(w[0], w[1], w[2], w[3]);
        }
        S.qb[2 * ln + h] = b;
    }
    if (q.j1 > a.pos && t >= 2 * kWave && t < 2 * kWave + hd) {  // this split holds the new row (waves 2, 3)
        const int r = a.pos - q.j0, u = t - 2 * kWave;
        const uint64_t* src =
            u < hd / 2 ? tq + (a.H + g * hd) / 2 + u : tq + (a.H + a.kvh * hd + g * hd) / 2 + u - hd / 2;
        const uint32_t w = trecv1(src, a.epoch, a.flags);
        if (u < hd / 2) {
            c.lds[kKvOff + r * (hd / 2) + 4 * ((u / 4) ^ kswz(r)) + u % 4] = w;
        } else {
            const int d = 2 * (u - hd / 2);
            uint16_t* vt16 = reinterpret_cast<uint16_t*>(c.lds + kVtOffP);
            vt16[d * (2 * kVtRowP) + r] = (uint16_t)(w & 0xffffu);
            vt16[(d + 1) * (2 * kVtRowP) + r] = (uint16_t)(w >> 16);
        }
    }
    stamp(a, slot_in(l, 1));
}

// The split's tiles on the matrix cores, compute wave 1 + t taking tile t
// (positions j0 + 64 t ..), each with its own max / sum / output.  Scores:
// C[position][head] over two v_mfma_f32_16x16x32_bf16 per 16 positions, A =
// the K rows (position 32 (s/2) + 8 (c/4) + 4 (s%2) + c%4 in A row c of
// sub-tile s, so that lane (c, j) ends with head c's scores of positions
// 32 (s/2) + 8 j + 4 (s%2) + r -- the k order P.V wants), B = q of head c
// pre-scaled by 1/8 (exact in bf16), dimensions 16 j + 8 h .. + 7.  P.V:
// C[dim][head], A = V^T rows, B = the probabilities split into bf16 hi + lo
// (two MFMAs, so P keeps about 16 bits).  The tiles' partials meet through
// LDS (in tile order) into the split's partial, which leaves as tagged words.
__device__ __forceinline__ void attn_run(const Ctx& c, int l, bool loc = false, bool direct = false) {
    const StepArgs& a = c.a;
    const AttnGeom q = attn_geom(c);
    const int grp = a.heads / a.kvh, hd = a.hd;
    const ALds S = alds(c.lds);
    lds_sync();  // q and the new row staged
    const int tile = c.wave - 1, p0 = q.j0 + kTileP * tile;
    const int cnt = (c.wave >= 1 && c.wave <= kAttTiles) ? max(0, min(kTileP, q.j1 - p0)) : 0;
    const int cc = c.lane % 16, jj = c.lane / 16;
    if (cnt > 0) {
        const uint4 qb[2] = {S.qb[2 * c.lane], S.qb[2 * c.lane + 1]};
        const uint4* kt = reinterpret_cast<const uint4*>(c.lds + kKvOff) + (size_t)kTileP * tile * 8;  // 8 chunks a row
        f32x4_t sc[kTileSub];
#pragma unroll
        for (int tt = 0; tt < kTileSub; tt++) {
            const int p = 32 * (tt / 2) + 8 * (cc / 4) + 4 * (tt % 2) + cc % 4, pr = kTileP * tile + p;
            const uint4* kr = kt + 8 * p;
            sc[tt] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
            sc[tt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf8(kr[(2 * jj) ^ kswz(pr)]), as_bf8(qb[0]), sc[tt],
                                                            0, 0, 0);
            sc[tt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf8(kr[(2 * jj + 1) ^ kswz(pr)]), as_bf8(qb[1]),
                                                            sc[tt], 0, 0, 0);
        }
        if (cnt < kTileP) {  // (wave-uniform) only the tile that holds the newest position is partial
#pragma unroll
            for (int tt = 0; tt < kTileSub; tt++)
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const int p = 32 * (tt / 2) + 8 * jj + 4 * (tt % 2) + r;
                    if (p >= cnt) sc[tt][r] = -INFINITY;
                }
        }
        float mx = -INFINITY;
#pragma unroll
        for (int tt = 0; tt < kTileSub; tt++)
#pragma unroll
            for (int r = 0; r < 4; r++) mx = fmaxf(mx, sc[tt][r]);
        mx = rows_max(mx);
        float lp = 0.0f;
#pragma unroll
        for (int tt = 0; tt < kTileSub; tt++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const float e = att_exp(sc[tt][r] - mx);  // masked scores (-inf) give 0
                sc[tt][r] = e;
                lp += e;
            }
        lp = rows_sum(lp);
        const uint32_t* vt = c.lds + kVtOffP + (kTileP / 2) * tile;
        f32x4_t o[4];
#pragma unroll
        for (int dt = 0; dt < 4; dt++) o[dt] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int u = 0; u < kTileU; u++) {
            uint32_t hi[4], lo[4];
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const float e0 = sc[2 * u + k / 2][2 * (k % 2)], e1 = sc[2 * u + k / 2][2 * (k % 2) + 1];
                hi[k] = pack_bf2(e0, e1);
                lo[k] = pack_bf2(e0 - bf_lo(hi[k]), e1 - bf_hi(hi[k]));
            }
            const bf16x8_t ph = as_bf8(make_uint4(hi[0], hi[1], hi[2], hi[3]));
            const bf16x8_t pl = as_bf8(make_uint4(lo[0], lo[1], lo[2], lo[3]));
#pragma unroll
            for (int dt = 0; dt < 4; dt++) {
                const uint4 va = *reinterpret_cast<const uint4*>(vt + (16 * dt + cc) * kVtRowP + 16 * u + 4 * jj);
                o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf8(va), ph, o[dt], 0, 0, 0);
                o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf8(va), pl, o[dt], 0, 0, 0);
            }
        }
        // lane (c, j) holds head c's o at dimensions 16 dt + 4 j + r
        float* ot = S.ot + (size_t)tile * 8 * (hd + 2);
        if (cc < grp) {
#pragma unroll
            for (int dt = 0; dt < 4; dt++)
#pragma unroll
                for (int r = 0; r < 4; r++) ot[cc * (hd + 2) + 2 + 16 * dt + 4 * jj + r] = o[dt][r];
            if (jj == 0) {
                ot[cc * (hd + 2)] = mx;
                ot[cc * (hd + 2) + 1] = lp;
            }
        }
    }
    lds_sync();
    // the split's partial: per head the max over its tiles, the sum and output rescaled to it;
    // device-coherent stores, completed before the arrival (direct: tagged words of the layer's
    // own partial slots, which the o_proj workers poll and merge; no arrival)
    const int ntl = min(kAttTiles, (q.j1 - q.j0 + kTileP - 1) / kTileP);  // tiles holding positions
    const int t = tix();
    const bool xl = *reinterpret_cast<const int*>(c.lds + kFlagOff + 2) != 0;
    {
        const int h = t / hd, d = t % hd;
        if (h < grp) {
            float M = -INFINITY;
            for (int i = 0; i < ntl; i++) M = fmaxf(M, S.ot[(i * 8 + h) * (hd + 2)]);
            float o = 0.0f, Ls = 0.0f;
            for (int i = 0; i < ntl; i++) {
                const float* pi = S.ot + (i * 8 + h) * (hd + 2);
                const float wgt = att_exp(pi[0] - M);
                o += wgt * pi[2 + d];
                Ls += wgt * pi[1];
            }
            if (direct) {  // tagged words of this layer's partials, merged by the o_proj workers
                uint64_t* out = a.tpa + ((((size_t)l * a.kvh + q.g) * a.xnsm + q.sp) * grp + h) * (hd + 2);
                tstore_loc(out + 2 + d, __float_as_uint(o), a.epoch, loc);
                if (d == 0) {
                    tstore_loc(out, __float_as_uint(M), a.epoch, loc);
                    tstore_loc(out + 1, __float_as_uint(Ls), a.epoch, loc);
                }
            } else if (xl) {  // to this XCD's L2
                float* out = a.part + (((size_t)q.g * q.ns + q.sp) * grp + h) * (hd + 2);
                gst(out + 2 + d, o);
                if (d == 0) {
                    gst(out, M);
                    gst(out + 1, Ls);
                }
            } else {
                float* out = a.part + (((size_t)q.g * q.ns + q.sp) * grp + h) * (hd + 2);
                cstore(out + 2 + d, o);
                if (d == 0) {
                    cstore(out, M);
                    cstore(out + 1, Ls);
                }
            }
        }
    }
    if (direct) return;
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    int* last = reinterpret_cast<int*>(c.lds + kFlagOff);
    if (t == 0) {
        if (xl) {  // the kv head's splits share this XCD: an L2 atomic
            int* ctr = a.counters + a.n_layers * a.kvh + 1 + l * a.kvh + q.g;
            const int old = __hip_atomic_fetch_add((MING_GLOBAL int*)ctr, 1, __ATOMIC_RELAXED,
                                                   __HIP_MEMORY_SCOPE_WORKGROUP);
            *last = old == q.ns - 1;
            if (old == q.ns - 1) __hip_atomic_store((MING_GLOBAL int*)ctr, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        } else {
            int* ctr = a.counters + l * a.kvh + q.g;
            const int old = __hip_atomic_fetch_add((MING_GLOBAL int*)ctr, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            *last = old == q.ns - 1;
            if (old == q.ns - 1) astore(ctr, 0);
        }
    }
    lds_sync();
    if (!*last) return;
    // the last split to arrive merges the kv head's splits, in split order: a running (M, L, o),
    // M' = max(M, m_s), L' = L e^(M - M') + l_s e^(m_s - M'), o likewise; the row is o / L
    for (int w = t; w < grp * hd / 2; w += kT) {
        const int h = (2 * w) / hd, d = (2 * w) % hd;
        const float* base = a.part + ((size_t)q.g * q.ns * grp + h) * (hd + 2);
        const size_t sstride = (size_t)grp * (hd + 2);
        float M = -INFINITY, L = 0.0f, o0 = 0.0f, o1 = 0.0f;
        for (int s0 = 0; s0 < q.ns; s0 += 8) {
            const int nb = min(8, q.ns - s0);
            float v[8][4];
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const float* p = base + (size_t)(s0 + min(i, nb - 1)) * sstride;
                v[i][0] = cload(p);
                v[i][1] = cload(p + 1);
                v[i][2] = cload(p + 2 + d);
                v[i][3] = cload(p + 3 + d);
            }
#pragma unroll
            for (int i = 0; i < 8; i++) {
                if (i >= nb) break;
                const float Mn = fmaxf(M, v[i][0]);
                const float cold = M == -INFINITY ? 0.0f : att_exp(M - Mn), cnew = att_exp(v[i][0] - Mn);
                L = L * cold + cnew * v[i][1];
                o0 = o0 * cold + cnew * v[i][2];
                o1 = o1 * cold + cnew * v[i][3];
                M = Mn;
            }
        }
        const uint32_t wv = pack_bf2(o0 / L, o1 / L);
        const int cw = (q.g * grp * hd) / 2 + w;
        tstore_loc(a.ta + (size_t)l * (a.H / 2) + cw, wv, a.epoch, loc);
        gst(reinterpret_cast<uint32_t*>(a.att + l * a.sx) + cw, wv);
    }
}

// ---- LC: o_proj + residual (unit = row pair, packed on the compute waves) ------
// O and down workers (the same set): row pairs 2p, 2p+1 with p = w*kCW + wave - 1.
__device__ __forceinline__ bool in_rowpairs(const Ctx& c) { return c.w * kCW < c.a.H / 2; }

template <int Q4>
__device__ __forceinline__ void st_o(const Ctx& c, const LayerDev& Ld, int l) {
    const StepArgs& a = c.a;
    const int p = c.w * kCW + c.wave - 1;
    const bool has = c.wave > 0 && p < a.H / 2;
    const int r = 2 * p + c.team;
    const uint64_t* xsrc = a.tx + (size_t)l * (a.H / 2) + p;  // residual, produced two stages ago
    uint64_t xpre = 0;
    RowRegs<Nc<Q4>::t32> W;
    if (has) {
        if (c.lane == 0) xpre = tload(xsrc);
        row_load<Q4, 32, Nc<Q4>::t32>(Ld.o, r, c.tl, 0, W);
    }
    get_image<Q4>(c, HUB_O, 4 * l + 1, 1, a.ta + (size_t)l * (a.H / 2), a.H, nullptr, nullptr);
    stamp(a, slot_in(l, 2));
    if (!has) return;
    const float acc = row_dot_pf<Q4, 32, Nc<Q4>::t32>(Ld.o, r, xs_of(c.lds, a.H), c.tl, W);
    const float a0 = lane_of(acc, 0), a1 = lane_of(acc, 32);
    if (c.lane == 0) {
        const uint32_t xw = tfinish(xsrc, xpre, a.epoch, a.flags);
        const uint32_t w = pack_bf2(bf_lo(xw) + rb(a0), bf_hi(xw) + rb(a1));
        tstore(a.tx1 + (size_t)l * (a.H / 2) + p, w, a.epoch);
        gst(reinterpret_cast<uint32_t*>(a.x1 + l * a.sx) + p, w);
    }
}

// ---- LD: rms(ln2) + gate/up + swiglu (unit = output pair, spread) -----------------
// Unit p -> worker p % W, slot s = p / W; slot s -> compute wave 1 + s % kCW.
// Team 0 takes the gate rows 2p, 2p+1, team 1 the up rows.
__device__ __forceinline__ int up_slots(const Ctx& c) { return (c.a.I / 2 - c.w + c.W - 1) / c.W; }

template <int Q4>
__device__ __forceinline__ void st_up(const Ctx& c, const LayerDev& Ld, int l) {
    const StepArgs& a = c.a;
    constexpr int MU = Nc<Q4>::up_units;
    const int slots = up_slots(c);
    if (slots <= 0) return;
    const LinearDev& L = c.team == 0 ? Ld.g : Ld.u;
    RowRegs<Nc<Q4>::t32> W[MU][2];
    if (c.wave > 0) {
#pragma unroll
        for (int i = 0; i < MU; i++) {
            const int s = c.wave - 1 + i * kCW;
            if (s < slots) {
                const int p = c.w + s * c.W;
                row_load<Q4, 32, Nc<Q4>::t32>(L, 2 * p, c.tl, 0, W[i][0]);
                row_load<Q4, 32, Nc<Q4>::t32>(L, 2 * p + 1, c.tl, 0, W[i][1]);
            }
        }
    }
    get_image<Q4>(c, HUB_UP, 4 * l + 2, 2, a.tx1 + (size_t)l * (a.H / 2), a.H, Ld.ln2, nullptr);
    stamp(a, slot_in(l, 3));
    if (c.wave == 0) return;
    const XStage st = xs_of(c.lds, a.H);
    auto finish = [&](int p, float acc0, float acc1) {
        const float g0 = rb(lane_of(acc0, 0)), g1 = rb(lane_of(acc1, 0));
        const float u0 = rb(lane_of(acc0, 32)), u1 = rb(lane_of(acc1, 32));
        if (c.lane == 0) {
            const float s0 = rb(sigmoid_fast(g0)), s1 = rb(sigmoid_fast(g1));
            const uint32_t wv = pack_bf2(rb(g0 * s0) * u0, rb(g1 * s1) * u1);
            tstore(a.th + (size_t)l * (a.I / 2) + p, wv, a.epoch);
            gst(reinterpret_cast<uint32_t*>(a.hh + l * a.sh) + p, wv);
        }
    };
    // Every preloaded unit's dot products before any unit's stores: stores
    // count in the same memory counter as loads, so a dot product issued
    // after a store would wait for that store's device-coherent round trip.
    float acc[MU][2];
#pragma unroll
    for (int i = 0; i < MU; i++) {
        const int s = c.wave - 1 + i * kCW;
        acc[i][0] = acc[i][1] = 0.0f;
        if (s < slots) {
            const int p = c.w + s * c.W;
            acc[i][0] = row_dot_pf<Q4, 32, Nc<Q4>::t32>(L, 2 * p, st, c.tl, W[i][0]);
            acc[i][1] = row_dot_pf<Q4, 32, Nc<Q4>::t32>(L, 2 * p + 1, st, c.tl, W[i][1]);
        }
    }
#pragma unroll
    for (int i = 0; i < MU; i++) {
        const int s = c.wave - 1 + i * kCW;
        if (s < slots) finish(c.w + s * c.W, acc[i][0], acc[i][1]);
    }
    // units beyond the preloaded ones (only when a worker has more than MU * kCW)
    for (int s = c.wave - 1 + MU * kCW; s < slots; s += kCW) {
        const int p = c.w + s * c.W;
        RowRegs<Nc<Q4>::t32> r0, r1;
        row_load<Q4, 32, Nc<Q4>::t32>(L, 2 * p, c.tl, 0, r0);
        row_load<Q4, 32, Nc<Q4>::t32>(L, 2 * p + 1, c.tl, 0, r1);
        const float acc0 = row_dot_pf<Q4, 32, Nc<Q4>::t32>(L, 2 * p, st, c.tl, r0);
        const float acc1 = row_dot_pf<Q4, 32, Nc<Q4>::t32>(L, 2 * p + 1, st, c.tl, r1);
        finish(p, acc0, acc1);
    }
}

// ---- LE: down + residual (unit = row pair, packed on the compute waves) --------------
// The weight loads are issued before the gate/up stage (down_pre): a wave's
// loads complete in issue order, so loads issued after gate/up would hold
// back this stage's receipt of its input behind them.
template <int Q4>
struct DownPre {
    RowRegs<Nc<Q4>::down> W;
};

template <int Q4>
__device__ __forceinline__ void down_pre(const Ctx& c, const LayerDev& Ld, DownPre<Q4>& d) {
    const int p = c.w * kCW + c.wave - 1;
    if (c.wave > 0 && p < c.a.H / 2) row_load<Q4, 32, Nc<Q4>::down>(Ld.d, 2 * p + c.team, c.tl, 0, d.W);
}

template <int Q4>
__device__ __forceinline__ void st_down(const Ctx& c, const LayerDev& Ld, int l, const DownPre<Q4>& d) {
    const StepArgs& a = c.a;
    const int p = c.w * kCW + c.wave - 1;
    const bool has = c.wave > 0 && p < a.H / 2;
    const int r = 2 * p + c.team;
    const uint64_t* xsrc = a.tx1 + (size_t)l * (a.H / 2) + p;  // residual, produced two stages ago
    uint64_t xpre = 0;
    if (has && c.lane == 0) xpre = tload(xsrc);
    get_image<Q4>(c, HUB_DOWN, 4 * l + 3, 3, a.th + (size_t)l * (a.I / 2), a.I, nullptr, nullptr);
    stamp(a, slot_in(l, 4));
    if (!has) return;
    const float acc = row_dot_pf<Q4, 32, Nc<Q4>::down>(Ld.d, r, xs_of(c.lds, a.I), c.tl, d.W);
    const float a0 = lane_of(acc, 0), a1 = lane_of(acc, 32);
    if (c.lane == 0) {
        const uint32_t xw = tfinish(xsrc, xpre, a.epoch, a.flags);
        const uint32_t w2 = pack_bf2(bf_lo(xw) + rb(a0), bf_hi(xw) + rb(a1));
        tstore(a.tx + (size_t)(l + 1) * (a.H / 2) + p, w2, a.epoch);
        gst(reinterpret_cast<uint32_t*>(a.xo + l * a.sx) + p, w2);
    }
}

// ---- final norm + tied LM head + argmax ---------------------------------------------
__device__ __forceinline__ bool better(float v, int i, float bv, int bi) { return v > bv || (v == bv && i < bi); }

__device__ __forceinline__ void block_best(float& bv, int& bi, float* rv, int* ri) {
    for (int o = kWave / 2; o > 0; o >>= 1) {
        const float ov = __shfl_xor(bv, o, kWave);
        const int oi = __shfl_xor(bi, o, kWave);
        if (better(ov, oi, bv, bi)) {
            bv = ov;
            bi = oi;
        }
    }
    const int wave = tix() / kWave, lane = tix() % kWave;
    lds_sync();
    if (lane == 0) {
        rv[wave] = bv;
        ri[wave] = bi;
    }
    lds_sync();
    if (tix() == 0)
        for (int w = 1; w < kW; w++)
            if (better(rv[w], ri[w], bv, bi)) {
                bv = rv[w];
                bi = ri[w];
            }
}

// The row-pair head (head_rows) keeps kHeadDepth row pairs per compute wave in flight: each
// register slot is refilled with the row pair kHeadDepth positions further on
// as soon as it has been used (slots are indexed statically, the loop is
// unrolled by the depth), so the stream of head rows never waits for a whole
// batch.  Loads past the last row pair reload the last one.
constexpr int kHeadDepth = 8;

template <int Q4>
struct HeadW {
    RowRegs<Nc<Q4>::t32> w[kHeadDepth];
};

template <int Q4>
__device__ __forceinline__ void head_slot_load(const Ctx& c, int p, RowRegs<Nc<Q4>::t32>& w) {
    const int V = c.a.head.N;
    row_load<Q4, 32, Nc<Q4>::t32>(c.a.head, min(2 * p + c.team, V - 1), c.tl, 0, w);
}

// The head's rows through the register ring (bf16 heads, and affine heads
// that q4tile_fits rejects), compute waves only.
template <int Q4>
__device__ __forceinline__ void head_rows(const Ctx& c, float& bv, int& bi) {
    const StepArgs& a = c.a;
    const int V = a.head.N, nunits = V / 2 + (V & 1);
    const int nw = c.W * kCW, me = c.w * kCW + c.wave - 1;
    HeadW<Q4> W;
    if (c.wave > 0) {
#pragma unroll
        for (int i = 0; i < kHeadDepth; i++) head_slot_load<Q4>(c, me + i * nw, W.w[i]);
    }
    // the hidden output comes from hub 0, or from worker 0 when no hub serves the head
    get_image<Q4>(c, HUB_HEAD, 4 * a.n_layers, 4, a.tx + (size_t)a.n_layers * (a.H / 2), a.H, a.final_norm,
                  !hub_on(a, HUB_HEAD) && c.w == 0 ? a.hidden : nullptr);
    stamp(a, slot_in(a.n_layers, 0));
    const XStage st = xs_of(c.lds, a.H);
    if (c.wave > 0) {
        for (int first = me; first < nunits; first += kHeadDepth * nw) {
#pragma unroll
            for (int i = 0; i < kHeadDepth; i++) {
                const int p = first + i * nw;
                if (p < nunits) {
                    const int r = min(2 * p + c.team, V - 1);
                    const float acc = row_dot_pf<Q4, 32, Nc<Q4>::t32>(a.head, r, st, c.tl, W.w[i]);
                    head_slot_load<Q4>(c, p + kHeadDepth * nw, W.w[i]);
                    if (c.tl == 0 && 2 * p + c.team < V) {
                        if (a.logits) gst(a.logits + r, acc);
                        if (better(acc, r, bv, bi)) {
                            bv = acc;
                            bi = r;
                        }
                    }
                }
            }
        }
    }
}

// The affine head with an even number of groups up to 16 (q4tile_fits) on
// the matrix cores: 16-row tiles
// (q4tile_mma / q4tile_finish), DEPTH tiles per wave in flight (two in the
// XCD-local kernel, whose registers allow it; one in the first schedule's
// kernel, which two would make spill), and all eight waves computing.  Tile t
// goes to wave slot t mod 8W, where the compute waves 1..7 of every worker
// come first and the receiving waves last: a receiving wave starts its loads
// only once the head's input has arrived, so it gets the fewer tiles.
template <int DEPTH>
__device__ __forceinline__ void head_tiles(const Ctx& c, float& bv, int& bi) {
    static_assert(DEPTH >= 1 && DEPTH <= 3, "one to three tiles in flight");
    const StepArgs& a = c.a;
    const LinearDev& L = a.head;
    const int V = L.N, G = L.K / 64, ntiles = (V + 15) / 16, nq = c.W * kW;
    const int q = c.wave > 0 ? c.w * kCW + c.wave - 1 : c.W * kCW + c.w;
    const int n16 = c.lane % 16, kq = c.lane / 16;
    const __amdgpu_buffer_rsrc_t rs = q4tile_rsrc(L.s, V, G), rb = q4tile_rsrc(L.b, V, G);
    auto load = [&](int t, Q4Tile& r) { q4tile_load(L, min(t * 16 + n16, V - 1), kq, rs, rb, r); };
    Q4Tile r0, r1, r2;  // tile t in r0, t + nq in r1 (DEPTH >= 2), t + 2 nq in r2 (DEPTH 3)
    auto first = [&]() {
        if (q < ntiles) load(q, r0);
        if (DEPTH >= 2 && q + nq < ntiles) load(q + nq, r1);
        if (DEPTH >= 3 && q + 2 * nq < ntiles) load(q + 2 * nq, r2);
    };
    if (c.wave > 0) first();
    get_image<1>(c, HUB_HEAD, 4 * a.n_layers, 4, a.tx + (size_t)a.n_layers * (a.H / 2), a.H, a.final_norm,
                 !hub_on(a, HUB_HEAD) && c.w == 0 ? a.hidden : nullptr);
    stamp(a, slot_in(a.n_layers, 0));
    if (c.wave == 0) first();
    const Q4TileX tx = q4tile_x(xs_of(c.lds, a.H), a.H, c.lane);
    auto step = [&](int t, Q4Tile& r) {
        const f32x4_t C = q4tile_mma(L, r, tx, c.lane);
        const uint2 s = r.s, b = r.b;
        if (t + DEPTH * nq < ntiles) load(t + DEPTH * nq, r);
        const float y = q4tile_finish(L, C, s, b, tx, c.lane);
        const int n = t * 16 + n16;
        if (kq == 0 && n < V) {
            if (a.logits) gst(a.logits + n, y);
            if (better(y, n, bv, bi)) {
                bv = y;
                bi = n;
            }
        }
    };
    for (int t = q; t < ntiles; t += DEPTH * nq) {
        step(t, r0);
        if (DEPTH >= 2 && t + nq < ntiles) step(t + nq, r1);
        if (DEPTH >= 3 && t + 2 * nq < ntiles) step(t + 2 * nq, r2);
    }
}

template <int Q4, int DEPTH = 1>
__device__ __forceinline__ void st_head(const Ctx& c) {
    const StepArgs& a = c.a;
    if (!a.logits && !a.argmax_out) {  // hidden only: hub 0 (or worker 0) writes it, no head
        if (!hub_on(a, HUB_HEAD) && c.w == 0)
            get_image<Q4>(c, HUB_HEAD, 4 * a.n_layers, 4, a.tx + (size_t)a.n_layers * (a.H / 2), a.H, a.final_norm,
                          a.hidden);
        return;
    }
    float bv = -INFINITY;
    int bi = 0x7fffffff;
    if constexpr (Q4) {
        if (q4tile_fits(a.head.K))
            head_tiles<DEPTH>(c, bv, bi);
        else
            head_rows<Q4>(c, bv, bi);
    } else {
        head_rows<Q4>(c, bv, bi);
    }
    float* rv = reinterpret_cast<float*>(c.lds + kRedOff);
    int* ri = reinterpret_cast<int*>(c.lds + kRedOff + 16);
    block_best(bv, bi, rv, ri);
    if (tix() == 0) {
        cstore(a.amax_v + c.w, bv);
        astore(a.amax_i + c.w, bi);
    }
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    int* last = reinterpret_cast<int*>(c.lds + kFlagOff);
    if (tix() == 0) {
        int* ctr = a.counters + a.n_layers * a.kvh;
        const int old = __hip_atomic_fetch_add((MING_GLOBAL int*)ctr, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        *last = old == c.W - 1;
        if (old == c.W - 1) astore(ctr, 0);
    }
    lds_sync();
    if (!*last) return;
    bv = -INFINITY;
    bi = 0x7fffffff;
    for (int i = tix(); i < c.W; i += kT) {
        const float v = cload(a.amax_v + i);
        const int ix = aload(a.amax_i + i);
        if (better(v, ix, bv, bi)) {
            bv = v;
            bi = ix;
        }
    }
    block_best(bv, bi, rv, ri);
    if (tix() == 0 && a.argmax_out) gst(a.argmax_out, bi == 0x7fffffff ? 0 : bi);
}

template <int Q4>
__global__ __launch_bounds__(kT) void decode_tagged_kernel(StepArgs args, const LayerDev* __restrict__ layers) {
    // Read the arguments in place, in the kernel-argument segment (uniform
    // scalar loads), instead of letting the compiler copy the block to scratch
    // for the references that the stages take.
    (void)args;
    const StepArgs& a = *(const StepArgs*)__builtin_amdgcn_kernarg_segment_ptr();
    __shared__ __align__(16) uint32_t lds[kLdsAll];
    stamp(a, 0);
    uint32_t xcc;
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(xcc));
    xcc &= 0xfu;
    const int nh = a.nhubs;
    if ((int)blockIdx.x < nh) {
        hub_main<Q4>(a, layers, lds, blockIdx.x, xcc);
        return;
    }
    // the wave index is uniform across the wave: say so, so that per-wave
    // selections (which rows, which linear) live in scalar registers
    const int lane = tix() % kWave, wave = __builtin_amdgcn_readfirstlane(tix() / kWave);
    const int W = (int)gridDim.x - nh, w = (int)blockIdx.x - nh;
    {
        const Ctx c0{a, lds, W, w, wave, lane, lane / 32, lane % 32, -1};
        st_embed(c0);
        // layer table into LDS (find_hub's barrier publishes it)
        const uint32_t* src = reinterpret_cast<const uint32_t*>(layers);
        for (int i = tix(); i < a.n_layers * kLayWords; i += kT) lds[kLayOff + i] = gld(src + i);
    }
    const LayerDev* lay = reinterpret_cast<const LayerDev*>(lds + kLayOff);
    const int hub = find_hub(a, lds, xcc);
    const Ctx c0{a, lds, W, w, wave, lane, lane / 32, lane % 32, hub};
    const bool pq = in_qkv(c0), pa = in_attn(c0), po = in_rowpairs(c0);
    const int L = a.n_layers;
    if (pa) {
        attn_xl_publish(c0, xcc);
        attn_prefetch(c0, 0);
        attn_xl_check(c0, xcc);
    }
    for (int l = 0; l < L; l++) {
        const int ln = tix() % kWave;
        const Ctx c{a, lds, W, w, wave, ln, ln / 32, ln % 32, hub};
        const LayerDev& Ld = lay[l];
        if (pq) {
            st_qkv<Q4>(c, Ld, l);
            done_stamp(a, slot_in(l, 0) + 1);
        }
        if (pa) {
            attn_recv(c, l);
            attn_run(c, l);
            done_stamp(a, slot_in(l, 1) + 1);
        }
        if (po) {
            st_o<Q4>(c, Ld, l);
            done_stamp(a, slot_in(l, 2) + 1);
        }
        DownPre<Q4> dp;
        if (po) down_pre<Q4>(c, Ld, dp);
        st_up<Q4>(c, Ld, l);
        done_stamp(a, slot_in(l, 3) + 1);
        if (pa && l + 1 < L) attn_prefetch(c, l + 1);  // the next layer's K/V while down and q/k/v run
        if (po) {
            st_down<Q4>(c, Ld, l, dp);
            done_stamp(a, slot_in(l, 4) + 1);
        }
    }
    const int ln = tix() % kWave;
    const Ctx c{a, lds, W, w, wave, ln, ln / 32, ln % 32, hub};
    st_head<Q4>(c);
    done_stamp(a, slot_in(L, 0) + 1);
}

// ==== The XCD-local layer (second schedule of the same step) =====================
// For a grid of 8 R workgroups, workgroup b on XCD slot x = b % 8 with rank
// r = b / 8 (rank 0 is the slot's hub).  Kv head g's q/k/v rows, its attention
// splits and its share of o_proj run on the workers of slot 7 - g (the slot
// that attn_geom's XCD grouping gives kv head g), so those hand-offs stay in
// one XCD's L2.  o_proj is split over K by kv head: slot 7 - g computes every
// output row over kv head g's 448 columns.  Gate/up units of slot x are the
// SwiGLU outputs of its own 64-column groups, and down is split over K the
// same way: slot x computes every output row over its groups.  The hubs of all
// slots gather the partials (tagged f32 words), sum them in slot order, apply
// the global scale, add the residual (which each hub keeps in LDS) and build
// the normalised stage images.  A layer thus has two grid-wide exchanges (o
// partials -> hubs, down partials -> hubs) where the first schedule has five.
// Hand-offs inside a slot use the same device-coherent tagged words, so the
// results do not depend on where the dispatcher places the workgroups; only
// the speed does.
constexpr int kXs = 8;             // XCD slots
constexpr int kHubRes = kLdsTotal;  // hub LDS, after the layer table: the residual stream, bf16 pairs [H/2] (H <= 1024)
static_assert(kHubRes + 512 <= kLdsAll, "hub LDS regions");
constexpr int kSliceT = 8;         // lanes per team of the split-K rows (8 rows per wave)

// A partial as an f32 word whose lowest mantissa bit is the epoch's parity
// (device-coherent store).  A reader that sees the parity of its own epoch
// has this step's value, since the word was last written a step earlier,
// with the other parity; it then clears the bit (every partial is thus
// truncated to 23 mantissa bits, the same way at every step).
__device__ __forceinline__ void pstore(uint32_t* p, float v, uint32_t epoch) {
    astore(p, (__float_as_uint(v) & ~1u) | (epoch & 1u));
}

// SwiGLU groups [gs, ge) of 64 outputs of slot x (slots x < xslots have some).
__device__ __forceinline__ void xslot_groups(const StepArgs& a, int x, int& gs, int& ge) {
    const int ng = a.I / 64, n = a.xslots;
    gs = x < n ? x * ng / n : ng;
    ge = x < n ? (x + 1) * ng / n : ng;
}

// A lane's chunks of row n's K slice: chunks [cb, cb + nc) of the row, a chunk
// being 32 values of an affine matrix (Q4) or 8 of a bf16 one; the lane takes
// slice chunks c0 + tl + T j, clamped to the slice's last chunk (and then not
// selected), as row_load does for whole rows.  Affine chunks carry their
// group's scale and bias.
template <int Q4, int NCH>
struct SliceRegs {
    uint4 w[NCH];
    uint32_t s[NCH], b[NCH];
};
template <int NCH>
struct SliceRegs<0, NCH> {
    uint4 w[NCH];
};

// Values per chunk and the chunks per lane of the split-K rows (8-lane
// teams): o_proj over a kv head's grp hd <= 512 columns, down over a slot's
// SwiGLU columns (<= 10 groups of 64 for Qwen2-0.5B; more run in further
// batches).
template <int Q4>
struct XcdN {
    static constexpr int cv = Q4 ? 32 : 8;
    static constexpr int o = Q4 ? 2 : 7;
    static constexpr int d = Q4 ? 3 : 10;
};

template <int Q4, int T, int NCH>
__device__ __forceinline__ void slice_load(const LinearDev& L, int n, int cb, int nc, int tl, int c0,
                                           SliceRegs<Q4, NCH>& r) {
    const uint32_t* wrow = L.w + (size_t)n * (Q4 ? L.K / 8 : L.K / 2);
#pragma unroll
    for (int j = 0; j < NCH; j++) {
        const int c = cb + min(c0 + tl + T * j, nc - 1);
        r.w[j] = ldg4(wrow + 4 * c);
        if constexpr (Q4 != 0) {
            const int G = L.K / 64;
            r.s[j] = gld(L.s + (size_t)n * G + (c >> 1));
            r.b[j] = gld(L.b + (size_t)n * G + (c >> 1));
        }
    }
}

// Partial dot of those chunks with the stage image of the slice (nc chunks).
template <int Q4, int T, int NCH>
__device__ __forceinline__ float slice_compute(const SliceRegs<Q4, NCH>& r, const XStage& st, int nc, int tl, int c0) {
    float acc = 0.0f;
    if constexpr (Q4 != 0) {
#pragma unroll
        for (int j = 0; j < NCH; j++) {
            const int cr = c0 + tl + T * j;
            const bool in = cr < nc;
            const int c = in ? cr : nc - 1;
            const uint4 x0 = *reinterpret_cast<const uint4*>(st.xs + (0 * nc + c) * 4);
            const uint4 x1 = *reinterpret_cast<const uint4*>(st.xs + (1 * nc + c) * 4);
            const uint4 x2 = *reinterpret_cast<const uint4*>(st.xs + (2 * nc + c) * 4);
            const uint4 x3 = *reinterpret_cast<const uint4*>(st.xs + (3 * nc + c) * 4);
            const float xh = st.xh[c];
            float a0 = q4_word_dot(r.w[j].x, reinterpret_cast<const uint32_t*>(&x0), 0.0f);
            float a1 = q4_word_dot(r.w[j].y, reinterpret_cast<const uint32_t*>(&x1), 0.0f);
            a0 = q4_word_dot(r.w[j].z, reinterpret_cast<const uint32_t*>(&x2), a0);
            a1 = q4_word_dot(r.w[j].w, reinterpret_cast<const uint32_t*>(&x3), a1);
            const float s = bf2f((uint16_t)r.s[j]), b = bf2f((uint16_t)r.b[j]);
            const float t = fmaf(b - 128.0f * s, xh, fmaf(s, a0 + a1, acc));
            acc = in ? t : acc;
        }
    } else {  // bf16 rows: the image holds the values in order, two accumulators as row_compute
        float a1 = 0.0f;
#pragma unroll
        for (int j = 0; j < NCH; j++) {
            const int cr = c0 + tl + T * j;
            const bool in = cr < nc;
            const uint4 x = *reinterpret_cast<const uint4*>(st.xs + 4 * (in ? cr : nc - 1));
            const float t0 = dot2(r.w[j].z, x.z, dot2(r.w[j].x, x.x, acc));
            const float t1 = dot2(r.w[j].w, x.w, dot2(r.w[j].y, x.y, a1));
            acc = in ? t0 : acc;
            a1 = in ? t1 : a1;
        }
        acc += a1;
    }
    return acc;
}

// Row n's dot over the slice, its first batch of chunks in `first`; team
// reduced, without the global scale (the hubs apply it to the summed slices).
template <int Q4, int T, int NCH>
__device__ __forceinline__ float slice_dot(const LinearDev& L, int n, const SliceRegs<Q4, NCH>& first,
                                           const XStage& st, int cb, int nc, int tl) {
    float acc = slice_compute<Q4, T, NCH>(first, st, nc, tl, 0);
    for (int c0 = T * NCH; c0 < nc; c0 += T * NCH) {
        SliceRegs<Q4, NCH> r;
        slice_load<Q4, T, NCH>(L, n, cb, nc, tl, c0, r);
        acc += slice_compute<Q4, T, NCH>(r, st, nc, tl, c0);
    }
    return team_sum<T>(acc);
}

// q/k/v unit u of kv head gh: quads of head blocks [q heads of the group | k | v].
__device__ __forceinline__ QkvGeom qkv_geom_x(const Ctx& c, int gh, int u) {
    const StepArgs& a = c.a;
    const int kvd = a.kvh * a.hd, grp = a.heads / a.kvh, qpb = a.hd / 4;
    const int nu = (grp + 2) * qpb;
    QkvGeom g;
    g.any = true;
    g.has = c.wave > 0 && u < nu;
    const int uq = max(0, min(u, nu - 1));
    const int hb = uq / qpb, qd = uq % qpb;
    g.cr = (hb < grp ? (gh * grp + hb) * a.hd : (hb == grp ? a.H + gh * a.hd : a.H + kvd + gh * a.hd)) + 2 * qd;
    g.which = g.cr < a.H ? 0 : (g.cr < a.H + kvd ? 1 : 2);
    g.base = g.which == 0 ? 0 : (g.which == 1 ? a.H : a.H + kvd);
    g.r0 = g.cr - g.base + c.team * (a.hd / 2);
    return g;
}

// o_proj workers of the XCD-local schedule: kv head g's attention row of layer
// l (grp heads x hd) merged here from its splits' tagged partials, in split
// order, as the last arriver merges them in the first schedule (a running
// (M, L, o): M' = max(M, m_s), L' = L e^(M - M') + l_s e^(m_s - M'), o
// likewise; the row is o / L), then left in LDS as the stage image of its
// K = grp hd values.  Every word a thread needs is polled at once, and a
// split's four words again while any is stale.  With `trace` the row also
// goes to the attention trace.  All threads call it.
template <int Q4>
__device__ __forceinline__ void attn_merge_image(const Ctx& c, int l, int g, bool trace) {
    const StepArgs& a = c.a;
    const int grp = a.heads / a.kvh, hd = a.hd, K = grp * hd, ns = attn_splits(a.pos);
    const size_t sstride = (size_t)grp * (hd + 2);
    const uint64_t* base = a.tpa + ((size_t)l * a.kvh + g) * a.xnsm * sstride;
    uint32_t* words = c.lds + kAttOt;
    const uint32_t ep = a.epoch;
    for (int w = tix(); w < K / 2; w += kT) {
        const int h = (2 * w) / hd, d = (2 * w) % hd;
        const uint64_t* hb = base + (size_t)h * (hd + 2);
        float M = -INFINITY, L = 0.0f, o0 = 0.0f, o1 = 0.0f;
        for (int s0 = 0; s0 < ns; s0 += 8) {
            const int nb = min(8, ns - s0);
            uint64_t v[8][4];
            auto load = [&](int i) {
                const uint64_t* p = hb + (size_t)(s0 + min(i, nb - 1)) * sstride;
                v[i][0] = tload(p);
                v[i][1] = tload(p + 1);
                v[i][2] = tload(p + 2 + d);
                v[i][3] = tload(p + 3 + d);
            };
            auto here = [&](int i) {
                return ((uint32_t)(v[i][0] >> 32) == ep) & ((uint32_t)(v[i][1] >> 32) == ep) &
                       ((uint32_t)(v[i][2] >> 32) == ep) & ((uint32_t)(v[i][3] >> 32) == ep);
            };
#pragma unroll
            for (int i = 0; i < 8; i++) load(i);
            unsigned sp = 0;
            while (true) {
                bool ready = true;
#pragma unroll
                for (int i = 0; i < 8; i++) ready &= here(i);
                if (ready) break;
                if (++sp >= kSpin) {
                    raise_flag(a.flags);
                    break;
                }
                if ((sp & 255u) == 0 && flag_set(a.flags)) break;
#pragma unroll
                for (int i = 0; i < 8; i++)
                    if (!here(i)) load(i);
            }
#pragma unroll
            for (int i = 0; i < 8; i++) {
                if (i >= nb) break;
                const float mi = __uint_as_float((uint32_t)v[i][0]), li = __uint_as_float((uint32_t)v[i][1]);
                const float v0 = __uint_as_float((uint32_t)v[i][2]), v1 = __uint_as_float((uint32_t)v[i][3]);
                const float Mn = fmaxf(M, mi);
                const float cold = M == -INFINITY ? 0.0f : att_exp(M - Mn), cnew = att_exp(mi - Mn);
                L = L * cold + cnew * li;
                o0 = o0 * cold + cnew * v0;
                o1 = o1 * cold + cnew * v1;
                M = Mn;
            }
        }
        const uint32_t wv = pack_bf2(o0 / L, o1 / L);
        words[w] = wv;
        if (trace) gst(reinterpret_cast<uint32_t*>(a.att + l * a.sx) + (g * K) / 2 + w, wv);
    }
    lds_sync();
    uint32_t v[8];
#pragma unroll
    for (int p = 0; p < 2; p++) {
        const int gi = tix() + p * kT;
#pragma unroll
        for (int j = 0; j < 4; j++) v[4 * p + j] = gi < K / 8 ? words[4 * gi + j] : 0u;
    }
    const uint4 nw[2] = {make_uint4(0, 0, 0, 0), make_uint4(0, 0, 0, 0)};
    image_finish<Q4, true>(a, c.lds, v, nw, K, nullptr, c.lds + kXsOff, nullptr, -1);
    lds_sync();
}

// o_proj partial of kv head g: rows 8 s + lane / 8 over the head's columns
// [g grp hd, (g + 1) grp hd), from the head's merged attention row.
template <int Q4>
__device__ __forceinline__ void st_opart(const Ctx& c, const LayerDev& Ld, int l, int g, int s, bool trace) {
    const StepArgs& a = c.a;
    constexpr int NO = XcdN<Q4>::o;
    const int K = (a.heads / a.kvh) * a.hd, nc = K / XcdN<Q4>::cv, cb = g * nc;
    const int n = kSliceT * s + c.lane / kSliceT, tl = c.lane % kSliceT;
    const bool has = c.wave > 0 && n < a.H;
    SliceRegs<Q4, NO> W;
    if (has) slice_load<Q4, kSliceT, NO>(Ld.o, n, cb, nc, tl, 0, W);
    lds_sync();
    attn_merge_image<Q4>(c, l, g, trace);
    stamp(a, slot_in(l, 2));
    if (!has) return;
    const float acc = slice_dot<Q4, kSliceT, NO>(Ld.o, n, W, xs_of(c.lds, K), cb, nc, tl);
    if (tl == 0) pstore(a.tpo + ((size_t)l * a.kvh + g) * a.H + n, acc, a.epoch);
}

// Gate/up units p in [p0, p1) of this slot: unit p0 + (r - 1) kCW + wave - 1 + i (R - 1) kCW.
template <int Q4>
__device__ __forceinline__ void st_up_x(const Ctx& c, const LayerDev& Ld, int l, int p0, int p1, int r, int R,
                                        bool loc) {
    const StepArgs& a = c.a;
    constexpr int MU = Nc<Q4>::up_units;
    const int step = (R - 1) * kCW, pw = p0 + (r - 1) * kCW + c.wave - 1;
    if (p0 + (r - 1) * kCW >= p1) return;  // no unit on this workgroup
    const LinearDev& L = c.team == 0 ? Ld.g : Ld.u;
    RowRegs<Nc<Q4>::t32> W[MU][2];
    if (c.wave > 0) {
#pragma unroll
        for (int i = 0; i < MU; i++) {
            const int p = pw + i * step;
            if (p < p1) {
                row_load<Q4, 32, Nc<Q4>::t32>(L, 2 * p, c.tl, 0, W[i][0]);
                row_load<Q4, 32, Nc<Q4>::t32>(L, 2 * p + 1, c.tl, 0, W[i][1]);
            }
        }
    }
    get_image<Q4>(c, HUB_UP, 4 * l + 2, 2, a.tx1 + (size_t)l * (a.H / 2), a.H, Ld.ln2, nullptr);
    stamp(a, slot_in(l, 3));
    if (c.wave == 0) return;
    const XStage st = xs_of(c.lds, a.H);
    auto finish = [&](int p, float acc0, float acc1) {
        const float g0 = rb(lane_of(acc0, 0)), g1 = rb(lane_of(acc1, 0));
        const float u0 = rb(lane_of(acc0, 32)), u1 = rb(lane_of(acc1, 32));
        if (c.lane == 0) {
            const float s0 = rb(sigmoid_fast(g0)), s1 = rb(sigmoid_fast(g1));
            const uint32_t wv = pack_bf2(rb(g0 * s0) * u0, rb(g1 * s1) * u1);
            tstore_loc(a.th + (size_t)l * (a.I / 2) + p, wv, a.epoch, loc);
            gst(reinterpret_cast<uint32_t*>(a.hh + l * a.sh) + p, wv);
        }
    };
    float acc[MU][2];
#pragma unroll
    for (int i = 0; i < MU; i++) {
        const int p = pw + i * step;
        acc[i][0] = acc[i][1] = 0.0f;
        if (p < p1) {
            acc[i][0] = row_dot_pf<Q4, 32, Nc<Q4>::t32>(L, 2 * p, st, c.tl, W[i][0]);
            acc[i][1] = row_dot_pf<Q4, 32, Nc<Q4>::t32>(L, 2 * p + 1, st, c.tl, W[i][1]);
        }
    }
#pragma unroll
    for (int i = 0; i < MU; i++) {
        const int p = pw + i * step;
        if (p < p1) finish(p, acc[i][0], acc[i][1]);
    }
    for (int p = pw + MU * step; p < p1; p += step) {
        RowRegs<Nc<Q4>::t32> r0, r1;
        row_load<Q4, 32, Nc<Q4>::t32>(L, 2 * p, c.tl, 0, r0);
        row_load<Q4, 32, Nc<Q4>::t32>(L, 2 * p + 1, c.tl, 0, r1);
        const float acc0 = row_dot_pf<Q4, 32, Nc<Q4>::t32>(L, 2 * p, st, c.tl, r0);
        const float acc1 = row_dot_pf<Q4, 32, Nc<Q4>::t32>(L, 2 * p + 1, st, c.tl, r1);
        finish(p, acc0, acc1);
    }
}

// Down partial of slot x: rows 8 s + lane / 8 over the slot's SwiGLU columns
// (chunks [cb, cb + nc)); the first batch of weights is loaded before gate/up.
template <int Q4>
struct DownX {
    SliceRegs<Q4, XcdN<Q4>::d> W;
};

// The slot's SwiGLU values [v0, v0 + K) are chunks [v0 / cv, (v0 + K) / cv) of a down row.
template <int Q4>
__device__ __forceinline__ void down_pre_x(const Ctx& c, const LayerDev& Ld, int s, int v0, int K, DownX<Q4>& d) {
    constexpr int CV = XcdN<Q4>::cv;
    const int n = kSliceT * s + c.lane / kSliceT;
    if (c.wave > 0 && n < c.a.H)
        slice_load<Q4, kSliceT, XcdN<Q4>::d>(Ld.d, n, v0 / CV, K / CV, c.lane % kSliceT, 0, d.W);
}

template <int Q4>
__device__ __forceinline__ void st_dpart(const Ctx& c, const LayerDev& Ld, int l, int x, int s, int v0, int K,
                                         const DownX<Q4>& d) {
    const StepArgs& a = c.a;
    constexpr int CV = XcdN<Q4>::cv;
    const int n = kSliceT * s + c.lane / kSliceT, tl = c.lane % kSliceT;
    const bool has = c.wave > 0 && n < a.H;
    lds_sync();
    build_image<Q4, true>(a, c.lds, a.th + (size_t)l * (a.I / 2) + v0 / 2, K, nullptr, c.lds + kXsOff, nullptr);
    lds_sync();
    stamp(a, slot_in(l, 4));
    if (!has) return;
    const float acc = slice_dot<Q4, kSliceT, XcdN<Q4>::d>(Ld.d, n, d.W, xs_of(c.lds, K), v0 / CV, K / CV, tl);
    if (tl == 0) pstore(a.tpd + ((size_t)l * kXs + x) * a.H + n, acc, a.epoch);
}

// Whether all four values of a polled quad carry the epoch's parity.
__device__ __forceinline__ bool quad_ready(uint4 v, uint32_t par) {
    return ((v.x & v.y & v.z & v.w & 1u) == par) && (((v.x | v.y | v.z | v.w) & 1u) == par);
}

// Hub: the next residual from the np partial vectors src[q H ..]: thread t
// (t < H/4) polls quad t (rows 4t .. 4t + 3) of every partial (device-scope
// 16-byte loads, all issued at once; stale quads polled again after a short
// sleep), sums them in partial order with the tag bits cleared, applies the
// global scale and updates residual words 2t, 2t + 1 in LDS:
// res = bf16(res + bf16(gs * sum over q of part[q])).  Then v gets the groups
// t and t + kT of 8 values as image_finish owns them.
__device__ __forceinline__ void hub_residual(const StepArgs& a, uint32_t* lds, const uint32_t* src, int np, float gs,
                                             uint32_t (&v)[8]) {
    uint32_t* res = lds + kHubRes;
    const int H = a.H, t = tix(), nq = H / 4;
    const uint32_t par = a.epoch & 1u;
    if (t < nq) {
        const __amdgpu_buffer_rsrc_t rs =
            __builtin_amdgcn_make_buffer_rsrc(const_cast<uint32_t*>(src), 0, (uint32_t)(np * H) * 4u, 0x00020000);
        const uint4 ok = make_uint4(par, par, par, par);
        uint4 w[kXs];
        auto load = [&](int q) {
            const auto x = __builtin_amdgcn_raw_buffer_load_b128(rs, (q * nq + t) * 16, 0, kSc1);
            w[q] = make_uint4(x[0], x[1], x[2], x[3]);
        };
#pragma unroll
        for (int q = 0; q < kXs; q++) {
            if (q < np)
                load(q);
            else
                w[q] = ok;
        }
        unsigned sp = 0;
        while (true) {
            bool ready = true;
#pragma unroll
            for (int q = 0; q < kXs; q++) ready &= quad_ready(w[q], par);
            if (ready) break;
            if (++sp >= kSpin) {
                raise_flag(a.flags);
                break;
            }
            if ((sp & 255u) == 0 && flag_set(a.flags)) break;
            __builtin_amdgcn_s_sleep(1);
            // (one statement per quad: the compiler declines to unroll this loop of conditional loads)
            auto again = [&](int q) {
                if (!quad_ready(w[q], par)) load(q);
            };
            static_assert(kXs == 8, "the re-poll below names each slot");
            again(0);
            again(1);
            again(2);
            again(3);
            again(4);
            again(5);
            again(6);
            again(7);
        }
        float s[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int q = 0; q < kXs; q++) {
            const uint32_t e[4] = {w[q].x, w[q].y, w[q].z, w[q].w};
#pragma unroll
            for (int j = 0; j < 4; j++) s[j] = q < np ? s[j] + __uint_as_float(e[j] & ~1u) : s[j];
        }
        const uint32_t x0 = res[2 * t], x1 = res[2 * t + 1];
        res[2 * t] = pack_bf2(bf_lo(x0) + rb(s[0] * gs), bf_hi(x0) + rb(s[1] * gs));
        res[2 * t + 1] = pack_bf2(bf_lo(x1) + rb(s[2] * gs), bf_hi(x1) + rb(s[3] * gs));
    }
    lds_sync();
#pragma unroll
    for (int p = 0; p < 2; p++) {
        const int gi = t + p * kT;
#pragma unroll
        for (int j = 0; j < 4; j++) v[4 * p + j] = gi < H / 8 ? res[4 * gi + j] : 0u;
    }
}

// The hubs also publish each residual as tagged words (for workers that find
// no hub on their XCD and stage their own inputs) and as the trace copy, hub
// b the groups gi with gi % 8 == b (so that no hub's next poll queues behind
// many stores).
__device__ __forceinline__ void hub_trace(const StepArgs& a, int b, const uint32_t (&v)[8], uint64_t* tdst,
                                          uint16_t* dst) {
    const int ng = a.H / 8;
#pragma unroll
    for (int p = 0; p < 2; p++) {
        const int gi = tix() + p * kT;
        if (gi < ng && gi % kXs == b) {
#pragma unroll
            for (int j = 0; j < 4; j++) tstore(tdst + 4 * gi + j, v[4 * p + j], a.epoch);
            gst(reinterpret_cast<uint4*>(dst) + gi, make_uint4(v[4 * p], v[4 * p + 1], v[4 * p + 2], v[4 * p + 3]));
        }
    }
}

// Hub: this thread's rms weight chunks of norm_w, loaded before the gather
// whose result they normalise.
__device__ __forceinline__ void hub_norm_pre(const StepArgs& a, const uint16_t* norm_w, uint4 (&nw)[2]) {
#pragma unroll
    for (int p = 0; p < 2; p++) {
        const int g = tix() + p * kT;
        nw[p] = g < a.H / 8 ? ldg4(norm_w + 8 * g) : make_uint4(0, 0, 0, 0);
    }
}

// Hub: image of the residual v (normalised with norm_w, whose chunks nw
// holds) into image slot `slot`, then flag fidx.  Stamps as hub_publish.
template <int Q4>
__device__ __forceinline__ void hub_image(const StepArgs& a, uint32_t* lds, int b, const uint32_t (&v0)[8],
                                          const uint16_t* norm_w, const uint4 (&nw)[2], int slot, int fidx,
                                          uint16_t* hidden, int ss) {
    uint32_t v[8];
#pragma unroll
    for (int k = 0; k < 8; k++) v[k] = v0[k];
    uint32_t* img = a.img + ((size_t)b * kImgSlots + slot) * a.img_stride;
    image_finish<Q4, false>(a, lds, v, nw, a.H, norm_w, img, hidden, ss);
    __syncthreads();
    if (tix() == 0) gst(a.hflag + (size_t)b * a.nflag + fidx, a.epoch);
    stamp(a, ss + 1);
}

template <int Q4>
__device__ __forceinline__ void hub_main_x(const StepArgs& a, const LayerDev* __restrict__ layers, uint32_t* lds, int b,
                                           uint32_t xcc) {
    if (tix() == 0) tstore(a.hubtab + b, xcc, a.epoch);
    const int H = a.H, L = a.n_layers;
    {  // the layer table into LDS: the stages' norm weights and global scales are then LDS reads
        const uint32_t* src = reinterpret_cast<const uint32_t*>(layers);
        for (int i = tix(); i < L * kLayWords; i += kT) lds[kLayOff + i] = gld(src + i);
    }
    const LayerDev* lay = reinterpret_cast<const LayerDev*>(lds + kLayOff);
    uint32_t v[8];
    uint4 nw[2];
    hub_norm_pre(a, layers[0].ln1, nw);
    {  // the embedded row
        trecv_groups<kT>(a.tx, H / 8, a.epoch, v, a.flags);
        uint32_t* res = lds + kHubRes;
#pragma unroll
        for (int p = 0; p < 2; p++) {
            const int gi = tix() + p * kT;
            if (gi < H / 8)
#pragma unroll
                for (int j = 0; j < 4; j++) res[4 * gi + j] = v[4 * p + j];
        }
    }
    __syncthreads();  // the layer table and the residual are in LDS
    for (int l = 0; l <= L; l++) {
        const uint16_t* n1 = l < L ? lay[l].ln1 : a.final_norm;
        if (l > 0) {  // layer l - 1's down partials
            const float gs = lay[l - 1].d.gscale;
            hub_norm_pre(a, n1, nw);
            hub_residual(a, lds, a.tpd + (size_t)(l - 1) * kXs * H, a.xslots, gs, v);
        }
        if (l == L) {
            hub_image<Q4>(a, lds, b, v, n1, nw, 4, 4 * L, b == 0 ? a.hidden : nullptr, slot_in(L, 0));
            hub_trace(a, b, v, a.tx + (size_t)L * (H / 2), a.xo + (size_t)(L - 1) * a.sx);
            break;
        }
        hub_image<Q4>(a, lds, b, v, n1, nw, 0, 4 * l, nullptr, slot_in(l, 0));
        if (l > 0) hub_trace(a, b, v, a.tx + (size_t)l * (H / 2), a.xo + (size_t)(l - 1) * a.sx);
        const uint16_t* n2 = lay[l].ln2;
        const float gs = lay[l].o.gscale;
        hub_norm_pre(a, n2, nw);
        hub_residual(a, lds, a.tpo + (size_t)l * a.kvh * H, a.kvh, gs, v);
        hub_image<Q4>(a, lds, b, v, n2, nw, 2, 4 * l + 2, nullptr, slot_in(l, 3));
        hub_trace(a, b, v, a.tx1 + (size_t)l * (H / 2), a.x1 + (size_t)l * a.sx);
    }
}

// Whether every workgroup of slot x (b = x, x + 8, ..., R of them) runs on
// this workgroup's XCD, from the XCC ids all workgroups publish at launch; the
// same answer in every workgroup of the slot.
__device__ __forceinline__ bool slot_on_one_xcd(const StepArgs& a, uint32_t* lds, int x, int R, uint32_t xcc) {
    int* res = reinterpret_cast<int*>(lds + kFlagOff + 3);
    if (tix() < kWave) {
        bool diff = false;
        for (int i = tix(); i < R; i += kWave) diff |= trecv1(a.hubtab + kXcdBase + kXs * i + x, a.epoch, a.flags) != xcc;
        const bool any = __ballot(diff) != 0ull;
        if (tix() == 0) *res = !any;
    }
    __syncthreads();
    return *res != 0;
}

template <int Q4>
__global__ __launch_bounds__(kT) void decode_xcd_kernel(StepArgs args, const LayerDev* __restrict__ layers) {
    (void)args;
    const StepArgs& a = *(const StepArgs*)__builtin_amdgcn_kernarg_segment_ptr();
    __shared__ __align__(16) uint32_t lds[kLdsAll];
    stamp(a, 0);
    uint32_t xcc;
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(xcc));
    xcc &= 0xfu;
    const int b = blockIdx.x;
    if (a.xloc && tix() == 0) tstore(a.hubtab + kXcdBase + b, xcc, a.epoch);
    if (b < kXs) {
        hub_main_x<Q4>(a, layers, lds, b, xcc);
        return;
    }
    const int lane = tix() % kWave, wave = __builtin_amdgcn_readfirstlane(tix() / kWave);
    const int W = (int)gridDim.x - kXs, w = b - kXs;
    const int x = b % kXs, r = b / kXs, R = (int)gridDim.x / kXs;
    {
        const Ctx c0{a, lds, W, w, wave, lane, lane / 32, lane % 32, -1};
        st_embed(c0);
        const uint32_t* src = reinterpret_cast<const uint32_t*>(layers);
        for (int i = tix(); i < a.n_layers * kLayWords; i += kT) lds[kLayOff + i] = gld(src + i);
    }
    const LayerDev* lay = reinterpret_cast<const LayerDev*>(lds + kLayOff);
    const int hub = find_hub(a, lds, xcc);
    const bool loc = a.xloc && slot_on_one_xcd(a, lds, x, R, xcc);
    const Ctx c0{a, lds, W, w, wave, lane, lane / 32, lane % 32, hub};
    const int gh = kXs - 1 - x;  // the kv head of this slot, if < kvh
    const int grp = a.heads / a.kvh, nu = (grp + 2) * (a.hd / 4);
    const int s0 = (r - 1) * kCW;  // wave slot of this workgroup's wave 1
    const bool onh = gh < a.kvh;
    const bool pq = onh && s0 < nu, pa = in_attn(c0), po = onh && kSliceT * s0 < a.H;
    int gs, ge;
    xslot_groups(a, x, gs, ge);
    const bool pd = ge > gs && kSliceT * s0 < a.H;
    const int L = a.n_layers;
    if (pa) {
        attn_xl_publish(c0, xcc);
        attn_prefetch(c0, 0);
        attn_xl_check(c0, xcc);
    }
    for (int l = 0; l < L; l++) {
        const int ln = tix() % kWave;
        const Ctx c{a, lds, W, w, wave, ln, ln / 32, ln % 32, hub};
        const LayerDev& Ld = lay[l];
        const int s = s0 + wave - 1;
        if (pq) {
            st_qkv_g<Q4>(c, Ld, l, qkv_geom_x(c, gh, s), loc);
            done_stamp(a, slot_in(l, 0) + 1);
        }
        if (pa) {
            attn_recv(c, l);
            attn_run(c, l, loc, true);
            done_stamp(a, slot_in(l, 1) + 1);
        }
        if (po) {
            st_opart<Q4>(c, Ld, l, gh, s, r == 1);
            done_stamp(a, slot_in(l, 2) + 1);
        }
        DownX<Q4> dx;
        if (pd) down_pre_x<Q4>(c, Ld, s, 64 * gs, 64 * (ge - gs), dx);
        if (ge > gs) {
            st_up_x<Q4>(c, Ld, l, 32 * gs, 32 * ge, r, R, loc);
            done_stamp(a, slot_in(l, 3) + 1);
        }
        if (pa && l + 1 < L) attn_prefetch(c, l + 1);
        if (pd) {
            st_dpart<Q4>(c, Ld, l, x, s, 64 * gs, 64 * (ge - gs), dx);
            done_stamp(a, slot_in(l, 4) + 1);
        }
    }
    const int ln = tix() % kWave;
    const Ctx c{a, lds, W, w, wave, ln, ln / 32, ln % 32, hub};
    st_head<Q4, 3>(c);
    done_stamp(a, slot_in(L, 0) + 1);
}

}  // namespace

// Positions per attention split on this schedule: a workgroup holds the
// split's K rows and V^T in LDS, one 96-position tile on each of four compute waves.
int tagged_split_len(int) { return kAttP; }

// Hubs for a grid of `grid` workgroups: one per XCD when the grid is large
// enough to spare them.
int tagged_hubs(int grid) { return grid >= 64 ? kMaxHubs : 0; }

// u32 words of one image slot: the largest stage image (K = max(H, I)),
// rounded up to 256 bytes.
int tagged_img_stride(int H, int I) {
    const int K = H > I ? H : I;
    return (xstage_words(K) + 63) / 64 * 64;
}

int tagged_max_layers() { return kMaxLdsLayers; }
int tagged_units_per_worker() { return kCW; }

// The grid is one workgroup per CU and every workgroup waits on others, so all
// of them must be resident at once.  A cooperative launch guarantees it; an
// ordinary one (about 16 us less per step) relies on the caller keeping other
// work off the device while the step runs.  Either way each wait is bounded:
// a workgroup that never starts turns into MING_E_TIMEOUT, not a hang.
hipError_t launch_lm_step_tagged(hipStream_t st, const StepArgs& a, int q4, int grid, bool cooperative) {
    StepArgs args = a;
    const LayerDev* layers = a.layers;
    void* params[] = {&args, &layers};
    const void* f = q4 ? reinterpret_cast<const void*>(decode_tagged_kernel<1>)
                       : reinterpret_cast<const void*>(decode_tagged_kernel<0>);
    if (cooperative) return hipLaunchCooperativeKernel(f, dim3(grid), dim3(kT), params, 0, st);
    return hipLaunchKernel(f, dim3(grid), dim3(kT), params, 0, st);
}

// The XCD-local schedule (decode_xcd_kernel): 4-bit (q4) or bf16 weights,
// grid of 8 R workgroups.
hipError_t launch_lm_step_xcd(hipStream_t st, const StepArgs& a, int q4, int grid, bool cooperative) {
    StepArgs args = a;
    const LayerDev* layers = a.layers;
    void* params[] = {&args, &layers};
    const void* f = q4 ? reinterpret_cast<const void*>(decode_xcd_kernel<1>)
                       : reinterpret_cast<const void*>(decode_xcd_kernel<0>);
    if (cooperative) return hipLaunchCooperativeKernel(f, dim3(grid), dim3(kT), params, 0, st);
    return hipLaunchKernel(f, dim3(grid), dim3(kT), params, 0, st);
}

// Whether the XCD-local schedule takes this shape on a grid of `grid`
// workgroups (one per CU); a step also needs at most grid / 8 - 1 attention
// splits per kv head.
bool xcd_fits(int q4, int grid, int H, int heads, int kvh, int hd, int I, int n_layers) {
    if (grid % kXs != 0 || grid > kXcdSlots || hd != 64 || kvh < 1 || kvh > kXs || heads % kvh != 0 || heads / kvh > 8) return false;
    int per_cu = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, q4 ? decode_xcd_kernel<1> : decode_xcd_kernel<0>, kT,
                                                     0) != hipSuccess ||
        per_cu < 1)
        return false;
    const int R = grid / kXs, waves = (R - 1) * kCW, grp = heads / kvh;
    return R >= 2 && H % 64 == 0 && H <= 1024 && I % 64 == 0 && I <= 8192 && (grp + 2) * hd / 4 <= waves &&
           H <= kSliceT * waves && n_layers <= kMaxLdsLayers;
}

// SwiGLU slots of the XCD-local schedule: every slot while there are at
// least 8 groups of 64 outputs, else one slot per group.
int xcd_slots(int I) { return I / 64 < kXs ? I / 64 : kXs; }

int tagged_grid(int num_cus) {
    int per_cu = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, decode_tagged_kernel<1>, kT, 0) != hipSuccess ||
        per_cu < 1)
        return 0;
    return num_cus;
}

}  // namespace ming
