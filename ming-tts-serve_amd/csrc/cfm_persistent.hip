// Persistent flow head for gfx950: one launch runs the ten Euler steps of
// cfmSample (src/ming_model.zig:1193-1203) -- per step the input rows
// (fused.embed), every DiT block's four stages (src/ming_fused.zig:145-289:
// rms1 + q/k/v + rotary, attention, out_proj + residual, rms2 + ff1 + gelu,
// ff2 + residual) and the final layer with the CFG combine and Euler update
// -- instead of about 42 launches per step.
//
// Results are bit-identical to the launch path (dit.hip): every output row
// is computed by a team of the same width holding the same weight chunks,
// the activation rows are staged with the same values in the same order, the
// row sums of the rms norms meet in the same order, and every epilogue is the
// same expression.
//
// Roles.  Workgroup x < 8 is the head of XCD x (the dispatcher places
// workgroup i on XCD i % 8; every workgroup checks this against its XCC id).
// The other workgroups are workers: worker w sits on XCD w % 8 as that XCD's
// worker j = w / 8.  In a worker, waves 1..7 compute and wave 0 receives.
//  - A stage's outputs leave a worker as tagged words {bf16 pair, epoch}
//    with device-coherent stores; every output word of a launch has its own
//    address, so a word carrying this launch's epoch is final.
//  - Each XCD rebuilds every stage input (an "image") in its own L2, in
//    slices: the receiving wave of worker j polls only slice j (a half row of
//    the rows an rms norm takes, with that half row's sum of squares; one
//    (CFG half, head) attention task over the received q/k/v; 128 units
//    (column pairs) of the ff1 rows, whose tagged words are unit-major),
//    writes it with ordinary stores, which stay in the
//    XCD's L2, and raises the slice's flag once the stores have completed.
//    The XCD's workers wait for every slice flag, then copy the image into
//    LDS with device-scope loads, which that L2 serves, normalising the rows
//    on the way where the stage takes rms-normalised rows.  A small vector
//    polled by many receivers arrives sooner than a large one polled by one.
//  - The head of each XCD computes the final layer (64 latent rows, CFG,
//    Euler, SDE) and the next step's input rows (x_emb(y): 1024 rows of 64,
//    with x_embedder held in its LDS for the whole launch) and publishes the
//    first block's rms1 image of that step itself.
// An image slot is rewritten only after every worker that read its previous
// contents has produced outputs that the slice owners have received since
// (each stage needs all of the previous stage's outputs).
//
// Every wait is bounded: past the spin limit a workgroup raises flags[0] and
// continues, so the grid always drains; the host reports MING_E_TIMEOUT.  The
// kernel needs all workgroups co-resident (cooperative launch, or an ordinary
// one on a device the caller keeps to this work).
#include "cfmp.h"
#include "common.h"
#include "tagged.h"
#include "tanh_tab.h"

namespace ming {

namespace {

using namespace tagged;

constexpr int kT = 512;  // threads per workgroup: 8 waves, 2 per SIMD
constexpr int kCW = 7;   // compute waves of a worker (1..7)
constexpr int kSc1 = 16; // buffer-load cache policy bit: device scope
constexpr int kD2 = kPD / 2, kF2 = kPF / 2;  // u32 words of a hidden row, an ff row
constexpr int kUA = 3 * kPD / 2, kUB = kPD / 2, kUC = kPF / 2, kUD = kPD / 2;  // row pairs per stage
constexpr int kNormSlices = 2 * kPR;          // half rows of an rms image
constexpr int kTasks = 2 * kPHeads;           // (CFG half, head) attention tasks
constexpr int kHhSlices = 16;                 // ff1 image slices: 128 units (column pairs) x 6 rows each
enum { SA = 0, SB = 1, SC = 2, SD = 3 };      // stage images: rms1 rows, attention rows, rms2 rows, ff1 rows

// LDS (u32 words).  Shared: the block table, row-sum partials, the rows'
// inverse norms.  A worker's stage image and gelu's tanh table follow; a
// head's area holds the latent y, x_emb(y), the final-normed rows and, for
// the whole launch, x_embedder's weights and bias.
constexpr int kBlkWords = (int)(sizeof(CfmPBlock) / 4);
constexpr int kLBlk = 0;                                // block table
constexpr int kLRed = kLBlk + kPMaxBlocks * kBlkWords;  // row-sum partials (12 floats)
constexpr int kLInv = kLRed + 16;                       // inverse norms of the 6 rows
constexpr int kLY = kLInv + 8;                          // head: the current latent y (64 bf16)
constexpr int kLXe = kLY + kPLat / 2;                   // head: x_emb(y) (1024 bf16)
constexpr int kLFx = kLXe + kD2;                        // head: final-normed rows L-1, 2L-1 [2][512]
constexpr int kLBx = kLFx + 2 * kD2;                    // head: x_embedder bias (1024 bf16)
constexpr int kLArea = kLBx + kD2;
constexpr int kLXs = kLArea;                            // worker: stage image (<= 6 x 2048 words)
constexpr int kLTanh = kLXs + kPR * kF2;                // worker: gelu's tanh table (tanh_tab.h)
constexpr int kLWx = kLArea;                            // head: x_embedder [1024][64] bf16
constexpr int kLdsW = kLTanh + kTanhTabN, kLdsH = kLWx + kPD * kPLat / 2;
constexpr int kLds = kLdsW > kLdsH ? kLdsW : kLdsH;
static_assert(kLY % 4 == 0 && kLXe % 4 == 0 && kLFx % 4 == 0 && kLXs % 4 == 0 && kLWx % 4 == 0 && kLTanh % 4 == 0,
              "LDS alignment");
static_assert(kLds * 4 <= 160 * 1024, "LDS of one workgroup");
static_assert(sizeof(CfmPBlock) % 8 == 0, "block table entries are copied as u64");

typedef uint32_t lds_u32x4_t __attribute__((ext_vector_type(4), aligned(16)));

// (float)tanh((double)u) for every bf16 u in [0, 16] (tanh_tab.h), filled at
// context creation; each worker copies it into LDS once per launch
__device__ float cfmp_tanh_tab[kTanhTabN];

// gelu_approx with every op rounded to bf16 (the launch path's chain), tanh from the LDS table
__device__ __forceinline__ float gelu_chain_p(const float* tab, float x) {
    const float c0 = rb(0.044715f), c1 = rb(0.7978845608f);
    const float x3 = rb((float)((double)x * (double)x * (double)x));
    const float inner = rb(x + rb(c0 * x3));
    const float th = rb(tanh_bf16(tab, rb(c1 * inner)));
    return rb(rb(0.5f * x) * rb(1.0f + th));
}

__device__ __forceinline__ int fidx(const CfmPArgs& a, int s, int b, int k) { return (s * a.nblk + b) * 4 + k; }
// tag of image f's slice flags: above every tag of earlier images and launches
__device__ __forceinline__ uint32_t ftag(const CfmPArgs& a, int f) { return a.epoch + (uint32_t)f; }

// Optional stage stamps (device wall clock), [6][nflag]: 0 worker 0's
// receiving wave published its slice of image f; 1 worker 0 holds image f;
// 2 worker 0's first compute wave issued its stores of stage f; 3 worker 0's
// receiving wave holds its slice's inputs; 4 head 0 done with the final layer
// of step f; 5 as 2 for the last worker.
__device__ __forceinline__ void stamp_at(const CfmPArgs& a, int row, int i) {
    if (a.tstamp) gst(a.tstamp + (size_t)row * a.nflag + i, (uint64_t)wall_clock64());
}

// Poll the 4 words of each group g = tix() + kT k (k < NG, g < ng) of a tagged
// vector, group g at word 4 map(g) of src, until all carry `tag` (bounded);
// payloads into v[4k + j].  Every load is issued at once and only groups with
// a stale word are polled again.
template <int NG, class Map>
__device__ __forceinline__ void recv(const uint64_t* src, int ng, Map map, uint32_t tag, uint32_t (&v)[4 * NG],
                                     int32_t* flags) {
    const uint64_t* gp[NG];
#pragma unroll
    for (int k = 0; k < NG; k++) {
        const int g = tix() + k * kT;
        gp[k] = g < ng ? src + 4 * (size_t)map(g) : nullptr;
    }
    uint64_t w[4 * NG];
#pragma unroll
    for (int k = 0; k < 4 * NG; k++) w[k] = gp[k >> 2] ? tload(gp[k >> 2] + (k & 3)) : ((uint64_t)tag << 32);
    unsigned s = 0;
    while (true) {
        bool ready = true;
#pragma unroll
        for (int k = 0; k < 4 * NG; k++) ready &= (uint32_t)(w[k] >> 32) == tag;
        if (ready) break;
        if (++s >= kSpin) {
            raise_flag(flags);
            break;
        }
        if ((s & 255u) == 0 && flag_set(flags)) break;
#pragma unroll
        for (int k = 0; k < NG; k++) {
            bool stale = false;
#pragma unroll
            for (int j = 0; j < 4; j++) stale |= (uint32_t)(w[4 * k + j] >> 32) != tag;
            if (stale)
#pragma unroll
                for (int j = 0; j < 4; j++) w[4 * k + j] = tload(gp[k] + j);
        }
    }
#pragma unroll
    for (int k = 0; k < 4 * NG; k++) v[k] = (uint32_t)w[k];
}

// N tagged words of one lane at p + off(i) until all carry `tag` (bounded);
// a round that finds a stale word sleeps briefly before polling again, so
// the receiving waves leave the memory path to the stage's producers
// (s_sleep 28: 8 to 64 measured, the sample time is not monotonic in it and
// its best value moved as the stages' own chains changed).
template <int N, class Off>
__device__ __forceinline__ void poll_words(const uint64_t* p, Off off, uint32_t tag, uint32_t (&v)[N],
                                           int32_t* flags) {
    uint64_t w[N];
#pragma unroll
    for (int i = 0; i < N; i++) w[i] = tload(p + off(i));
    unsigned s = 0;
    while (true) {
        bool ready = true;
#pragma unroll
        for (int i = 0; i < N; i++) ready &= (uint32_t)(w[i] >> 32) == tag;
        if (ready) break;
        if (++s >= kSpin) {
            raise_flag(flags);
            break;
        }
        if ((s & 255u) == 0 && flag_set(flags)) break;
        __builtin_amdgcn_s_sleep(28);
#pragma unroll
        for (int i = 0; i < N; i++)
            if ((uint32_t)(w[i] >> 32) != tag) w[i] = tload(p + off(i));
    }
#pragma unroll
    for (int i = 0; i < N; i++) v[i] = (uint32_t)w[i];
}

// Poll a slice flag until it carries `tag` (bounded), sleeping between polls.
__device__ __forceinline__ void wait_slice(const uint32_t* f, uint32_t tag, int32_t* flags) {
    unsigned s = 0;
    while (aload(f) != tag) {
        if (++s >= kSpin) {
            raise_flag(flags);
            break;
        }
        if ((s & 255u) == 0 && flag_set(flags)) break;
        __builtin_amdgcn_s_sleep(1);
    }
}

// Every store this wave has issued has completed (they count against the
// memory counter); the following store cannot move above.
__device__ __forceinline__ void stores_done() {
    __builtin_amdgcn_s_waitcnt(0);
    asm volatile("" ::: "memory");
}

// ---- row dot products (the launch path's inner loop) -------------------------------

// acc[u][r] = team sum over the TEAM lanes of row slot r (6 slots) dotted
// with unit u's NCH weight chunks of this lane (chunk tl + TEAM j), rows at
// xs with KW4 16-byte chunks each.  Units share each LDS read; chunk j + 1's
// six reads are issued before chunk j's products, so the reads overlap the
// math instead of each waiting out its own latency (the chains keep their
// order: chunk j's four words after chunk j - 1's).
template <int NCH, int TEAM, int NU>
__device__ __forceinline__ void dots6(const uint4 (&wr)[NU][NCH], const uint32_t* xs, int KW4, int tl,
                                      float (&acc)[NU][kPR]) {
    const lds_u32x4_t* xv4 = reinterpret_cast<const lds_u32x4_t*>(xs);
#pragma unroll
    for (int u = 0; u < NU; u++)
#pragma unroll
        for (int r = 0; r < kPR; r++) acc[u][r] = 0.0f;
    u32x4_t xv[2][kPR];  // chunk j's six row words, chunk j + 1's in flight
#pragma unroll
    for (int r = 0; r < kPR; r++) xv[0][r] = xv4[r * KW4 + tl];
#pragma unroll
    for (int j = 0; j < NCH; j++) {
        if (j + 1 < NCH) {
#pragma unroll
            for (int r = 0; r < kPR; r++) xv[(j + 1) & 1][r] = xv4[r * KW4 + tl + TEAM * (j + 1)];
        }
        const u32x4_t(&x)[kPR] = xv[j & 1];
#pragma unroll
        for (int r = 0; r < kPR; r++) {
#pragma unroll
            for (int u = 0; u < NU; u++) {
                float s = dot2(wr[u][j].x, x[r].x, acc[u][r]);
                s = dot2(wr[u][j].y, x[r].y, s);
                s = dot2(wr[u][j].z, x[r].z, s);
                acc[u][r] = dot2(wr[u][j].w, x[r].w, s);
            }
        }
    }
#pragma unroll
    for (int u = 0; u < NU; u++)
#pragma unroll
        for (int r = 0; r < kPR; r++) acc[u][r] = team_sum<TEAM>(acc[u][r]);
}

__device__ __forceinline__ float pick6(const float (&acc)[kPR], int tl) {
    float v = 0.0f;
#pragma unroll
    for (int r = 0; r < kPR; r++)
        if (tl == r) v = acc[r];
    return v;
}

// Attention of one (CFG half, head) task as the launch path's attention
// kernel computes it: lane d owns dimension d; scores sum_d (q/8) k over the
// wave, p = exp(s - max), o = sum_j p_j v_j / sum_j p_j (rounded by the caller).
__device__ __forceinline__ void attn_math(const float (&qv)[kPL], const float (&kv)[kPL], const float (&vv)[kPL],
                                          float (&r)[kPL]) {
    const float scale = 1.0f / 8.0f;
#pragma unroll
    for (int i = 0; i < kPL; i++) {
        const float qd = scale * qv[i];
        float sc[kPL], m = -INFINITY;
#pragma unroll
        for (int jj = 0; jj < kPL; jj++) {
            sc[jj] = team_sum<kWave>(qd * kv[jj]);
            m = fmaxf(m, sc[jj]);
        }
        float l = 0.0f, o = 0.0f;
#pragma unroll
        for (int jj = 0; jj < kPL; jj++) {
            const float p = exp_rep(sc[jj] - m);
            l += p;
            o += p * vv[jj];
        }
        r[i] = o / l;
    }
}

// ---- workers -----------------------------------------------------------------------

struct Wk {
    const CfmPArgs& a;
    uint32_t* lds;
    int W, w, nj, j, wave, lane;
    uint32_t* img;  // this XCD's images
    uint32_t* flg;  // this XCD's slice flags [4][32]
};

__device__ __forceinline__ const CfmPBlock& blk(const uint32_t* lds, int b) {
    return reinterpret_cast<const CfmPBlock*>(lds + kLBlk)[b];
}

__device__ __forceinline__ uint32_t* img_of(const CfmPArgs& a, int x) { return a.img + (size_t)x * kPImgWords; }
__device__ __forceinline__ uint32_t* flg_of(const CfmPArgs& a, int x) { return a.flg + (size_t)x * 4 * kPFlagLine; }

// Slice owner (receiving wave): half row j of the 6 rows (tagged, [6][512]
// words) -- lane l holds chunk 64 (j % 2) + l of row j / 2, as the launch
// path's staging lane l of wave j % 2 does -- its sum of squares met over
// the 64 lanes, raw words and sum into the image, then the slice flag.
__device__ __forceinline__ void own_rows(const Wk& c, const uint64_t* src, int raw, int part, int kind, int f) {
    const CfmPArgs& a = c.a;
    if (c.j >= kNormSlices) return;
    const int r = c.j / 2, h = c.j % 2, l = c.lane, word = r * kD2 + h * (kD2 / 2) + 4 * l;
    uint32_t v[4];
    poll_words<4>(src + word, [](int i) { return i; }, a.epoch, v, a.flags);
    if (c.w == 0 && l == 0) stamp_at(a, 3, f);
    float ss = 0.0f;
#pragma unroll
    for (int e = 0; e < 4; e++) {
        const float lo = bf_lo(v[e]), hi = bf_hi(v[e]);
        ss += lo * lo;
        ss += hi * hi;
    }
    ss = team_sum<kWave>(ss);
    gst(reinterpret_cast<uint4*>(c.img + raw + word), make_uint4(v[0], v[1], v[2], v[3]));
    if (l == 0) gst(reinterpret_cast<float*>(c.img + part) + c.j, ss);
    stores_done();
    if (l == 0) gst(c.flg + kind * kPFlagLine + c.j, ftag(a, f));
    if (c.w == 0 && l == 0) stamp_at(a, 0, f);
}

// Attention task `task` (CFG half task / 16, head task % 16) of block (s, b)
// on one wave, its rows into the image at img: q, k, v of positions 0..2 of
// the half are words (which * 6 + 3 half + i) * 512 + col / 2 of the tagged q|k|v.
__device__ __forceinline__ void attn_task(const CfmPArgs& a, uint32_t* img, int s, int b, int task, int d) {
    const uint64_t* tq = a.tq + (size_t)(s * a.nblk + b) * kPTq;
    const int hb = task / kPHeads, hd = task % kPHeads, col = hd * kPHd + d;
    uint32_t w[3 * kPL];
    // unit-major q | k | v: word (which, column pair, row) at (which kD2 + pair) kPR + row
    poll_words<3 * kPL>(tq + (size_t)(col / 2) * kPR + 3 * hb, [](int i) { return (i / kPL) * (kD2 * kPR) + i % kPL; },
                        a.epoch, w, a.flags);
    float qv[kPL], kv[kPL], vv[kPL], o[kPL];
#pragma unroll
    for (int i = 0; i < kPL; i++) {
        qv[i] = (d & 1) ? bf_hi(w[i]) : bf_lo(w[i]);
        kv[i] = (d & 1) ? bf_hi(w[kPL + i]) : bf_lo(w[kPL + i]);
        vv[i] = (d & 1) ? bf_hi(w[2 * kPL + i]) : bf_lo(w[2 * kPL + i]);
    }
    attn_math(qv, kv, vv, o);
#pragma unroll
    for (int i = 0; i < kPL; i++) {
        const float o1 = lane_xor1(o[i]);  // d is the lane
        if ((d & 1) == 0) gst(img + kPImgB + (3 * hb + i) * kD2 + col / 2, pack_bf2(o[i], o1));
    }
}

// Slice owner: attention task j of block (s, b) (tasks from nj on are the head's).
__device__ __forceinline__ void own_attn(const Wk& c, int s, int b, int f) {
    const CfmPArgs& a = c.a;
    if (c.j >= kTasks) return;
    attn_task(a, c.img, s, b, c.j, c.lane);
    if (c.w == 0 && c.lane == 0) stamp_at(a, 3, f);
    stores_done();
    if (c.lane == 0) gst(c.flg + SB * kPFlagLine + c.j, ftag(a, f));
    if (c.w == 0 && c.lane == 0) stamp_at(a, 0, f);
}

// Slice owner: units 128 j .. 128 j + 127 of the ff1 outputs of block (s, b),
// all six rows.  The tagged outputs are unit-major (a unit's 6 row words are
// contiguous, one producer's 48 bytes), so lane l polls the 12 contiguous
// words of units 128 j + 2l and + 1 and writes them into the row-major image.
__device__ __forceinline__ void own_hh(const Wk& c, int s, int b, int f) {
    const CfmPArgs& a = c.a;
    if (c.j >= kHhSlices) return;
    const uint64_t* th = a.th + (size_t)(s * a.nblk + b) * kPTh;
    const int u = (kUC / kHhSlices) * c.j + 2 * c.lane;
    uint32_t v[2 * kPR];
    poll_words<2 * kPR>(th + (size_t)u * kPR, [](int i) { return i; }, a.epoch, v, a.flags);
    if (c.w == 0 && c.lane == 0) stamp_at(a, 3, f);
    typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
#pragma unroll
    for (int r = 0; r < kPR; r++)
        *(MING_GLOBAL u32x2*)(c.img + kPImgD + r * kF2 + u) = u32x2{v[r], v[kPR + r]};
    stores_done();
    if (c.lane == 0) gst(c.flg + SD * kPFlagLine + c.j, ftag(a, f));
    if (c.w == 0 && c.lane == 0) stamp_at(a, 0, f);
}

// Wait for every slice flag of image f (wave 0), then copy `words` u32 from
// slot offset `off` of this XCD's image into LDS at kLXs.  With `part` >= 0
// the image holds raw rows whose half-row sums of squares are at `part`:
// each row is normalised on the way with the weights nw of the thread's
// chunks (bf16(w * bf16(x * inv)), inv = 1 / sqrt((s0 + s1) / D + eps)).
template <int NG>
__device__ __forceinline__ void wait_image(const Wk& c, int kind, int nslices, int f, int off, int words, int part,
                                           const uint4* nw) {
    const CfmPArgs& a = c.a;
    if (c.wave == 0) {
        if (c.lane < nslices) wait_slice(c.flg + kind * kPFlagLine + c.lane, ftag(a, f), a.flags);
        if (part >= 0 && c.lane < kPR) {
            const float* ps = reinterpret_cast<const float*>(c.img + part);
            const float sum = aload(ps + 2 * c.lane) + aload(ps + 2 * c.lane + 1);
            reinterpret_cast<float*>(c.lds + kLInv)[c.lane] = 1.0f / sqrtf(sum / (float)kPD + a.eps);
        }
    }
    lds_sync();
    const int n4 = words / 4;
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(c.img + off, 0, n4 * 16, 0x00020000);
    const float* inv = reinterpret_cast<const float*>(c.lds + kLInv);
    if (part < 0) {
        // images used as they are: each wave's 64 chunks go straight to LDS
        // (a direct buffer load: lane l's 16 bytes land at the wave's base +
        // 16 l); n4 is a multiple of 64, so a wave is wholly in or out
#pragma unroll
        for (int k = 0; k < NG; k++) {
            const int i0 = kWave * c.wave + kT * k;
            if (i0 < n4)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(
                    rs, (__attribute__((address_space(3))) void*)(c.lds + kLXs + 4 * i0), 16, (i0 + c.lane) * 16, 0,
                    0, kSc1);
        }
        __builtin_amdgcn_s_waitcnt(0);
        lds_sync();
        if (c.w == 0 && tix() == 0) stamp_at(a, 1, f);
        return;
    }
#pragma unroll
    for (int k = 0; k < NG; k++) {
        const int i = tix() + kT * k;
        if (i < n4) {
            const auto v = __builtin_amdgcn_raw_buffer_load_b128(rs, i * 16, 0, kSc1);
            uint32_t o[4] = {v[0], v[1], v[2], v[3]};
            if (part >= 0) {
                const float iv = inv[i / (kD2 / 4)];
                const uint32_t g[4] = {nw[k].x, nw[k].y, nw[k].z, nw[k].w};
#pragma unroll
                for (int e = 0; e < 4; e++)
                    o[e] = pack_bf2(bf_lo(g[e]) * rb(bf_lo(o[e]) * iv), bf_hi(g[e]) * rb(bf_hi(o[e]) * iv));
            }
            reinterpret_cast<lds_u32x4_t*>(c.lds + kLXs)[i] = u32x4_t{o[0], o[1], o[2], o[3]};
        }
    }
    lds_sync();
    if (c.w == 0 && tix() == 0) stamp_at(a, 1, f);
}

// rms weight chunks of the image chunks a thread copies (chunk i % 128 of i = tix() + 512 k)
__device__ __forceinline__ void norm_chunks(const uint16_t* w, uint4 (&nw)[2]) {
#pragma unroll
    for (int k = 0; k < 2; k++) nw[k] = ldg4(w + 8 * ((tix() + kT * k) % (kPD / 8)));
}

// The raw-row word (row r, column pair u) of this XCD's image at `off`.
__device__ __forceinline__ uint32_t raw_word(const Wk& c, int off, int r, int u) {
    return aload(c.img + off + r * kD2 + u);
}

__device__ __forceinline__ void stamp_stores(const Wk& c, int f) {
    if (c.a.tstamp && c.wave == 1 && c.lane == 0 && (c.w == 0 || c.w == c.W - 1))
        gst(c.a.tstamp + (size_t)(c.w == 0 ? 2 : 5) * c.a.nflag + f, (uint64_t)wall_clock64());
}

// A: q/k/v row pairs of rms1(x) with bias and the interleaved rotary on q, k
// (the launch path's E_QKV: 32-lane teams, 4 chunks per lane).
__device__ __forceinline__ void wk_qkv(const Wk& c, const CfmPBlock& B, int s, int b) {
    const CfmPArgs& a = c.a;
    const int cw = c.wave - 1, u = c.w + c.W * cw;
    const bool act = cw >= 0 && u < kUA;
    const int team = c.lane >> 5, tl = c.lane & 31;
    const int n = 2 * (act ? u : 0) + team, which = n / kPD, nrow = n % kPD;
    uint4 wr[1][4];
    float bias = 0.0f, cs = 0.0f, sn = 0.0f;
    if (act) {
        const uint16_t* Wm = which == 0 ? B.wq : which == 1 ? B.wk : B.wv;
        const uint16_t* Bv = which == 0 ? B.bq : which == 1 ? B.bk : B.bv;
#pragma unroll
        for (int j = 0; j < 4; j++) wr[0][j] = ldg4(Wm + (size_t)nrow * kPD + 8 * (tl + 32 * j));
        bias = bf2f(gld(Bv + nrow));
        const int rr = min(tl, kPR - 1), l = rr % kPL, i = (nrow % kPHd) / 2;
        cs = gld(a.cos_t + l * (kPHd / 2) + i);
        sn = gld(a.sin_t + l * (kPHd / 2) + i);
    }
    uint4 nw[2];
    norm_chunks(B.norm1, nw);
    const int f = fidx(a, s, b, SA);
    if (c.wave == 0 && b > 0) own_rows(c, a.txo + (size_t)(s * a.nblk + b - 1) * kPTx, kPImgA, kPImgAp, SA, f);
    wait_image<2>(c, SA, kNormSlices, f, kPImgA, kPR * kD2, kPImgAp, nw);
    if (!act) return;
    float acc[1][kPR];
    dots6<4, 32, 1>(wr, c.lds + kLXs, kPD / 8, tl, acc);
    const float e = rb(pick6(acc[0], tl) + bias);
    const float other = lane_xor32(e, c.lane);
    float o = e;
    if (which < 2) {
        const float ev = team == 0 ? e : other, od = team == 0 ? other : e;
        const float p = ev * cs, q = od * sn, s2 = ev * sn, uu = od * cs;
        o = team == 0 ? p - q : s2 + uu;
    }
    const float o1 = lane_xor32(o, c.lane);
    if (team == 0 && tl < kPR)
        tstore(a.tq + (size_t)(s * a.nblk + b) * kPTq + ((size_t)which * kD2 + nrow / 2) * kPR + tl, pack_bf2(o, o1),
               a.epoch);
    stamp_stores(c, f);
}

// B: x1 = x + out_proj(attention) (E_RES: 32-lane teams, 4 chunks per lane).
__device__ __forceinline__ void wk_out(const Wk& c, const CfmPBlock& B, int s, int b) {
    const CfmPArgs& a = c.a;
    const int cw = c.wave - 1, u = c.w + c.W * cw;
    const bool act = cw >= 0 && u < kUB;
    const int team = c.lane >> 5, tl = c.lane & 31;
    const int n = 2 * (act ? u : 0) + team;
    uint4 wr[1][4];
    float bias = 0.0f;
    if (act) {
#pragma unroll
        for (int j = 0; j < 4; j++) wr[0][j] = ldg4(B.wo + (size_t)n * kPD + 8 * (tl + 32 * j));
        bias = bf2f(gld(B.bo + n));
    }
    const int f = fidx(a, s, b, SB);
    if (c.wave == 0) own_attn(c, s, b, f);
    wait_image<2>(c, SB, kTasks, f, kPImgB, kPR * kD2, -1, nullptr);
    if (!act) return;
    const uint32_t rw = tl < kPR ? raw_word(c, kPImgA, tl, u) : 0u;
    float acc[1][kPR];
    dots6<4, 32, 1>(wr, c.lds + kLXs, kPD / 8, tl, acc);
    const float res = team == 0 ? bf_lo(rw) : bf_hi(rw);
    const float o = res + rb(pick6(acc[0], tl) + bias);
    const float o1 = lane_xor32(o, c.lane);
    if (team == 0 && tl < kPR)
        tstore(a.tx1 + (size_t)(s * a.nblk + b) * kPTx + tl * kD2 + u, pack_bf2(o, o1), a.epoch);
    stamp_stores(c, f);
}

// C: gelu(ff1(rms2(x1))) (E_GELU: 32-lane teams, 4 chunks per lane).  Compute
// wave q of worker w takes row pairs w + W (2q) and w + W (2q + 1), sharing
// every image read, every dot product before any store: 2,048 pairs on five
// waves per worker measured faster (1.548 vs 1.646 ms per sample) than one
// or two pairs on each of the seven.
__device__ __forceinline__ void wk_ff1(const Wk& c, const CfmPBlock& B, int s, int b) {
    const CfmPArgs& a = c.a;
    const int cw = c.wave - 1;
    const int u0 = c.w + c.W * (2 * cw), u1 = c.w + c.W * (2 * cw + 1);
    const bool act0 = cw >= 0 && u0 < kUC, act1 = cw >= 0 && u1 < kUC;
    const int team = c.lane >> 5, tl = c.lane & 31;
    const int n0 = 2 * (act0 ? u0 : 0) + team, n1 = 2 * (act1 ? u1 : 0) + team;
    uint4 wr[2][4];
    float b0 = 0.0f, b1 = 0.0f;
    if (act0) {
#pragma unroll
        for (int j = 0; j < 4; j++) wr[0][j] = ldg4(B.w1 + (size_t)n0 * kPD + 8 * (tl + 32 * j));
        b0 = bf2f(gld(B.b1 + n0));
    }
    if (act1) {
#pragma unroll
        for (int j = 0; j < 4; j++) wr[1][j] = ldg4(B.w1 + (size_t)n1 * kPD + 8 * (tl + 32 * j));
        b1 = bf2f(gld(B.b1 + n1));
    }
    uint4 nw[2];
    norm_chunks(B.norm2, nw);
    const int f = fidx(a, s, b, SC);
    if (c.wave == 0) own_rows(c, a.tx1 + (size_t)(s * a.nblk + b) * kPTx, kPImgC, kPImgCp, SC, f);
    wait_image<2>(c, SC, kNormSlices, f, kPImgC, kPR * kD2, kPImgCp, nw);
    if (!act0) return;
    float acc[2][kPR];
    if (act1) {
        dots6<4, 32, 2>(wr, c.lds + kLXs, kPD / 8, tl, acc);
    } else {
        const uint4(&w1)[1][4] = reinterpret_cast<const uint4(&)[1][4]>(wr);
        float (&a1)[1][kPR] = reinterpret_cast<float(&)[1][kPR]>(acc);
        dots6<4, 32, 1>(w1, c.lds + kLXs, kPD / 8, tl, a1);
    }
    uint64_t* out = a.th + (size_t)(s * a.nblk + b) * kPTh;
    const float* tab = reinterpret_cast<const float*>(c.lds + kLTanh);
    {
        const float g = gelu_chain_p(tab, rb(pick6(acc[0], tl) + b0));
        const float g1 = lane_xor32(g, c.lane);
        if (team == 0 && tl < kPR) tstore(out + (size_t)u0 * kPR + tl, pack_bf2(g, g1), a.epoch);
    }
    if (act1) {
        const float g = gelu_chain_p(tab, rb(pick6(acc[1], tl) + b1));
        const float g1 = lane_xor32(g, c.lane);
        if (team == 0 && tl < kPR) tstore(out + (size_t)u1 * kPR + tl, pack_bf2(g, g1), a.epoch);
    }
    stamp_stores(c, f);
}

// D: x2 = x1 + ff2(h) (E_RES with K = 4096: one 64-lane team per row, 8
// chunks per lane).  Compute wave q of worker w takes both rows of pair
// u = w + W q; the two rows share every image read.
__device__ __forceinline__ void wk_ff2(const Wk& c, const CfmPBlock& B, int s, int b) {
    const CfmPArgs& a = c.a;
    const int cw = c.wave - 1, u = c.w + c.W * cw;
    const bool act = cw >= 0 && u < kUD;
    const int n = 2 * (act ? u : 0);
    uint4 wr[2][8];
    float b0 = 0.0f, b1 = 0.0f;
    if (act) {
#pragma unroll
        for (int j = 0; j < 8; j++) {
            wr[0][j] = ldg4(B.w2 + (size_t)n * kPF + 8 * (c.lane + 64 * j));
            wr[1][j] = ldg4(B.w2 + (size_t)(n + 1) * kPF + 8 * (c.lane + 64 * j));
        }
        b0 = bf2f(gld(B.b2 + n));
        b1 = bf2f(gld(B.b2 + n + 1));
    }
    const int f = fidx(a, s, b, SD);
    if (c.wave == 0) own_hh(c, s, b, f);
    wait_image<6>(c, SD, kHhSlices, f, kPImgD, kPR * kF2, -1, nullptr);
    if (!act) return;
    const uint32_t rw = c.lane < kPR ? raw_word(c, kPImgC, c.lane, u) : 0u;
    float acc[2][kPR];
    dots6<8, 64, 2>(wr, c.lds + kLXs, kPF / 8, c.lane, acc);
    const float o0 = bf_lo(rw) + rb(pick6(acc[0], c.lane) + b0);
    const float o1 = bf_hi(rw) + rb(pick6(acc[1], c.lane) + b1);
    if (c.lane < kPR) tstore(a.txo + (size_t)(s * a.nblk + b) * kPTx + c.lane * kD2 + u, pack_bf2(o0, o1), a.epoch);
    stamp_stores(c, f);
}

// ---- heads -------------------------------------------------------------------------

// The head of Euler step s on XCD x (s > 0: first the final layer of step s - 1):
//   final: rms(final_norm) of rows L-1, 2L-1 of the last block's output, the
//     64 latent rows (32-lane teams, 4 chunks per lane, 2 row slots), CFG
//     combine and Euler update (+ SDE) -> y (the launch path's E_CFM);
//   embed: x_emb(y) (one 8-lane team per row: the launch path's 32-lane team
//     has its lanes 8..31 at +0, which its butterfly adds in two more exact
//     steps), the six rows [t_emb + c_emb, x_emb(hist), x_emb(y)] per CFG
//     half -> image A of (s, 0) on XCD x: raw rows, the half-row sums of
//     squares (as the slice owners compute them) and every slice flag.
// Every weight of the final layer is loaded before the wait for the block output.
__device__ __forceinline__ void head_step(const CfmPArgs& a, uint32_t* lds, int x, int s) {
    const int t = tix(), wave = t / kWave, lane = t % kWave;
    const bool fin = s > 0, emb = s < a.steps;
    uint32_t* img = img_of(a, x);
    const int team = lane >> 5, tl = lane & 31;
    uint4 wf[4][4];
    float bfv[4];
    if (fin) {
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int n = 2 * (wave + 8 * j) + team;
#pragma unroll
            for (int jj = 0; jj < 4; jj++) wf[j][jj] = ldg4(a.wf + (size_t)n * kPD + 8 * (tl + 32 * jj));
            bfv[j] = bf2f(gld(a.bf + n));
        }
    }
    // the input rows' other operands (group g = t + 512 k: row g / 128, chunk g % 128)
    uint4 ra[2], rc[2];
    if (emb) {
#pragma unroll
        for (int k = 0; k < 2; k++) {
            const int g = t + kT * k, r = min(g / 128, kPR - 1), cc = g % 128, half = r / kPL;
            if (r % kPL == 0) {
                ra[k] = ldg4(a.te + ((size_t)s * 2 + half) * kPD + 8 * cc);
                rc[k] = ldg4(a.ce + (size_t)half * kPD + 8 * cc);
            } else {
                ra[k] = ldg4(a.xh + 8 * cc);
                rc[k] = ra[k];
            }
        }
    }
    float* red = reinterpret_cast<float*>(lds + kLRed);
    if (fin) {
        // final norm rows L-1 and 2L-1 (waves 0..3: row slot wave / 2, half wave % 2)
        const int g = t;  // chunk g % 128 of row slot g / 128 (g < 256)
        const uint4 fw = ldg4(a.fnorm + 8 * (g % 128));
        const float dtv = bf2f(gld(a.dt + s - 1)), sqv = bf2f(gld(a.sq + s - 1));
        float sdes[4];
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int n = 2 * (wave + 8 * j) + team;
            sdes[j] = a.shift != 0.0f ? bf2f(gld(a.sde + (size_t)(s - 1) * kPLat + n)) : 0.0f;
        }
        uint32_t v[4];
        const uint64_t* src = a.txo + (size_t)((s - 1) * a.nblk + a.nblk - 1) * kPTx;
        recv<1>(src, 2 * kPD / 8, [](int gg) { return (gg / 128 == 0 ? kPL - 1 : 2 * kPL - 1) * (kD2 / 4) + gg % 128; },
                a.epoch, v, a.flags);
        float ss = 0.0f;
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const float lo = bf_lo(v[e]), hi = bf_hi(v[e]);
            ss += lo * lo;
            ss += hi * hi;
        }
        ss = team_sum<kWave>(ss);
        if (g < 256 && lane == 0) red[g / 64] = ss;
        lds_sync();
        if (g < 256) {
            const int rs = g / 128, cc = g % 128;
            const float sum = red[2 * rs] + red[2 * rs + 1];
            const float inv = 1.0f / sqrtf(sum / (float)kPD + a.eps);
            const uint32_t gn[4] = {fw.x, fw.y, fw.z, fw.w};
            uint32_t o[4];
#pragma unroll
            for (int e = 0; e < 4; e++)
                o[e] = pack_bf2(bf_lo(gn[e]) * rb(bf_lo(v[e]) * inv), bf_hi(gn[e]) * rb(bf_hi(v[e]) * inv));
            reinterpret_cast<lds_u32x4_t*>(lds + kLFx)[rs * (kPD / 8) + cc] = u32x4_t{o[0], o[1], o[2], o[3]};
        }
        lds_sync();
        // 64 latent rows: 2 row slots (cond, uncond)
        const lds_u32x4_t* xv4 = reinterpret_cast<const lds_u32x4_t*>(lds + kLFx);
        uint16_t* y16 = reinterpret_cast<uint16_t*>(lds + kLY);
        const float cfg = rb(a.cfg);
        u32x4_t xr[2][4];  // this lane's chunks of both rows, shared by its 4 row pairs
#pragma unroll
        for (int jj = 0; jj < 4; jj++)
#pragma unroll
            for (int r = 0; r < 2; r++) xr[r][jj] = xv4[r * (kPD / 8) + tl + 32 * jj];
#pragma unroll
        for (int j = 0; j < 4; j++) {
            float acc[2] = {0.0f, 0.0f};
#pragma unroll
            for (int jj = 0; jj < 4; jj++) {
#pragma unroll
                for (int r = 0; r < 2; r++) {
                    const u32x4_t xv = xr[r][jj];
                    float sacc = dot2(wf[j][jj].x, xv.x, acc[r]);
                    sacc = dot2(wf[j][jj].y, xv.y, sacc);
                    sacc = dot2(wf[j][jj].z, xv.z, sacc);
                    acc[r] = dot2(wf[j][jj].w, xv.w, sacc);
                }
            }
            acc[0] = team_sum<32>(acc[0]);
            acc[1] = team_sum<32>(acc[1]);
            const int n = 2 * (wave + 8 * j) + team;
            if (tl == 0) {
                const float pc = rb(acc[0] + bfv[j]), pn = rb(acc[1] + bfv[j]);
                const float f0 = rb(pc + rb(rb(pc - pn) * cfg));
                float y = rb(bf2f(y16[n]) + rb(dtv * f0));
                if (a.shift != 0.0f) y = rb(y + rb(rb(rb(a.shift) * sqv) * sdes[j]));
                const uint16_t yb = f2bf(y);
                y16[n] = yb;
                if (x == 0) {
                    if (a.y_steps) gst(a.y_steps + (size_t)(s - 1) * kPLat + n, yb);
                    if (!emb) gst(a.y_out + n, yb);
                }
            }
        }
        lds_sync();
        if (x == 0 && t == 0) stamp_at(a, 4, s - 1);
    }
    if (!emb) return;
    // x_emb(y): 1024 rows of K = 64, row n = 64 j + 8 wave + lane / 8, chunk lane % 8
    {
        const int tm = lane >> 3, t8 = lane & 7;
        const u32x4_t yv = reinterpret_cast<const lds_u32x4_t*>(lds + kLY)[t8];
        const lds_u32x4_t* wx4 = reinterpret_cast<const lds_u32x4_t*>(lds + kLWx);
        const uint16_t* bx16 = reinterpret_cast<const uint16_t*>(lds + kLBx);
        uint16_t* xe16 = reinterpret_cast<uint16_t*>(lds + kLXe);
        u32x4_t wvs[16];  // every row's weight chunk first, so the reads overlap
#pragma unroll
        for (int j = 0; j < 16; j++) wvs[j] = wx4[(64 * j + 8 * wave + tm) * (kPLat / 8) + t8];
#pragma unroll
        for (int j = 0; j < 16; j++) {
            const int n = 64 * j + 8 * wave + tm;
            const u32x4_t wv = wvs[j];
            float acc = dot2(wv.x, yv.x, 0.0f);
            acc = dot2(wv.y, yv.y, acc);
            acc = dot2(wv.z, yv.z, acc);
            acc = dot2(wv.w, yv.w, acc);
            acc = team_sum<8>(acc);
            acc = (acc + 0.0f) + 0.0f;
            if (t8 == 0) xe16[n] = f2bf(rb(acc + bf2f(bx16[n])));
        }
    }
    lds_sync();
    // the rows: group g (< 768) = chunk g % 128 of row g / 128; a wave's 64 groups form half row g / 64
    const int f = fidx(a, s, 0, SA);
#pragma unroll
    for (int k = 0; k < 2; k++) {
        const int g = t + kT * k, r = min(g / 128, kPR - 1), cc = g % 128;
        uint4 xv;
        if (r % kPL == 0)
            xv = make_uint4(pack_bf2(bf_lo(ra[k].x) + bf_lo(rc[k].x), bf_hi(ra[k].x) + bf_hi(rc[k].x)),
                            pack_bf2(bf_lo(ra[k].y) + bf_lo(rc[k].y), bf_hi(ra[k].y) + bf_hi(rc[k].y)),
                            pack_bf2(bf_lo(ra[k].z) + bf_lo(rc[k].z), bf_hi(ra[k].z) + bf_hi(rc[k].z)),
                            pack_bf2(bf_lo(ra[k].w) + bf_lo(rc[k].w), bf_hi(ra[k].w) + bf_hi(rc[k].w)));
        else if (r % kPL == 1)
            xv = ra[k];
        else {
            const u32x4_t e = reinterpret_cast<const lds_u32x4_t*>(lds + kLXe)[cc];
            xv = make_uint4(e[0], e[1], e[2], e[3]);
        }
        const uint32_t q[4] = {xv.x, xv.y, xv.z, xv.w};
        float ss = 0.0f;
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const float lo = bf_lo(q[e]), hi = bf_hi(q[e]);
            ss += lo * lo;
            ss += hi * hi;
        }
        ss = team_sum<kWave>(ss);
        if (g < kPR * kPD / 8) {
            gst(reinterpret_cast<uint4*>(img + kPImgA + r * kD2 + 4 * cc), xv);
            if (lane == 0) gst(reinterpret_cast<float*>(img + kPImgAp) + g / 64, ss);
        }
    }
    __syncthreads();  // every store of the image has completed
    if (t < kNormSlices) gst(flg_of(a, x) + SA * kPFlagLine + t, ftag(a, f));
    // the attention tasks the XCD's workers do not cover (tasks nj .. 31), block by block, on wave 0
    const int nj = ((int)gridDim.x - kPXcds) / kPXcds;
    if (wave == 0 && nj < kTasks)
        for (int b = 0; b < a.nblk; b++) {
            for (int task = nj; task < kTasks; task++) attn_task(a, img, s, b, task, lane);
            stores_done();
            for (int task = nj; task < kTasks; task++)
                if (lane == 0) gst(flg_of(a, x) + SB * kPFlagLine + task, ftag(a, fidx(a, s, b, SB)));
        }
}

__device__ __forceinline__ void head_main(const CfmPArgs& a, uint32_t* lds, int x) {
    if (tix() < kPLat / 2) lds[kLY + tix()] = gld(reinterpret_cast<const uint32_t*>(a.noise) + tix());
    // x_embedder weights and bias, for every step of this launch
    for (int i = tix(); i < kPD * kPLat / 8; i += kT) {
        const uint4 w = ldg4(a.wx + 8 * i);
        reinterpret_cast<lds_u32x4_t*>(lds + kLWx)[i] = u32x4_t{w.x, w.y, w.z, w.w};
    }
    for (int i = tix(); i < kPD / 8; i += kT) {
        const uint4 w = ldg4(a.bx + 8 * i);
        reinterpret_cast<lds_u32x4_t*>(lds + kLBx)[i] = u32x4_t{w.x, w.y, w.z, w.w};
    }
    lds_sync();
    for (int s = 0; s <= a.steps; s++) head_step(a, lds, x, s);
}

__global__ __launch_bounds__(kT, 1) void cfm_persistent_kernel(CfmPArgs a) {
    __shared__ __align__(16) uint32_t lds[kLds];
    uint32_t xcc;
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(xcc));
    {
        const int nw = a.nblk * (int)(sizeof(CfmPBlock) / 8);
        for (int i = tix(); i < nw; i += kT)
            reinterpret_cast<uint64_t*>(lds + kLBlk)[i] = gld(reinterpret_cast<const uint64_t*>(a.blocks) + i);
    }
    __syncthreads();
    if ((int)blockIdx.x < kPXcds) {
        if (tix() == 0) tstore(a.xcctab + blockIdx.x, xcc, a.epoch);
        head_main(a, lds, blockIdx.x);
        return;
    }
    const int w = (int)blockIdx.x - kPXcds, W = (int)gridDim.x - kPXcds, x = w % kPXcds;
    Wk c{a, lds, W, w, W / kPXcds, w / kPXcds, (int)(tix() / kWave), (int)(tix() % kWave), img_of(a, x), flg_of(a, x)};
    // the XCD's head must share this workgroup's XCC (their L2 holds the images)
    int* ok = reinterpret_cast<int*>(lds + kLInv);
    if (tix() == 0) *ok = trecv1(a.xcctab + x, a.epoch, a.flags) == xcc;
    __syncthreads();
    if (!*ok) {
        if (tix() == 0) raise_flag(a.flags);
        return;
    }
    for (int i = tix(); i < kTanhTabN; i += kT) reinterpret_cast<float*>(lds + kLTanh)[i] = gld(cfmp_tanh_tab + i);
    for (int s = 0; s < a.steps; s++)
        for (int b = 0; b < a.nblk; b++) {
            const CfmPBlock& B = blk(lds, b);
            wk_qkv(c, B, s, b);
            wk_out(c, B, s, b);
            wk_ff1(c, B, s, b);
            wk_ff2(c, B, s, b);
        }
}

}  // namespace

hipError_t tanh_upload_cfmp(const float* host) {
    return hipMemcpyToSymbol(HIP_SYMBOL(cfmp_tanh_tab), host, sizeof(float) * kTanhTabN);
}

// Workgroups of the persistent flow head on a device of num_cus CUs (one per
// CU, every one resident), or 0 if the kernel cannot keep one per CU or the
// device's CUs do not fit its plan (the same number of workers on each XCD,
// enough of them for the q/k/v row pairs in one round and for every slice).
int cfmp_grid(int num_cus) {
    int per_cu = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, cfm_persistent_kernel, kT, 0) != hipSuccess ||
        per_cu < 1)
        return 0;
    const int W = num_cus - kPXcds;
    return W >= kPMinWorkers && W % kPXcds == 0 && W / kPXcds >= kHhSlices ? num_cus : 0;
}

hipError_t launch_cfm_persistent(hipStream_t st, const CfmPArgs& a, int grid, bool cooperative) {
    CfmPArgs args = a;
    void* params[] = {&args};
    const void* f = reinterpret_cast<const void*>(cfm_persistent_kernel);
    if (cooperative) return hipLaunchCooperativeKernel(f, dim3(grid), dim3(kT), params, 0, st);
    return hipLaunchKernel(f, dim3(grid), dim3(kT), params, 0, st);
}

}  // namespace ming
