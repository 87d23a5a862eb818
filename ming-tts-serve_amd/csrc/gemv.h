// Batch-1 (and few-row) GEMV building blocks for gfx950.
//
// The activation vector is staged once per workgroup in LDS; a "team" of T
// lanes (32 or 64) owns one weight row and walks it in 16-byte chunks, so a
// team's loads of a row are contiguous and one wave instruction covers
// 64 x 16 B.  Partial sums stay in f32 and meet with a team reduction.
//
// MLX-affine 4-bit rows: a 16 B chunk is 4 u32 words = 32 nibbles = half a
// quantization group of 64.  The staged activations are bf16 pairs in nibble
// pair order (see q4_pairs) laid out [word j][chunk c][pair p] so that the
// lanes of one ds_read_b128 hit consecutive 16 B (no LDS bank conflicts), and
// xh[c] holds the f32 sum of chunk c's 32 activations for the +128 offset
// correction and the bias term.
//
// bf16 rows: a 16 B chunk is 8 weights, dotted with the activations in their
// natural pair order with v_dot2c_f32_bf16.
#pragma once

#include "args.h"
#include "common.h"

namespace ming {

// LDS image of one activation vector of K elements (K % 64 == 0).
struct XStage {
    uint32_t* xs;  // K/2 u32
    float* xh;     // K/32 f32 (affine only)
};

__host__ __device__ constexpr int xstage_words(int K) { return K / 2 + K / 32; }

// One group of 8 activations x[8g..8g+7], held as the bf16 pairs
// (0,1),(2,3),(4,5),(6,7) in v: returns the nibble pair order
// (0,4),(1,5),(2,6),(3,7) that goes to xs word j = g % 4 of chunk c = g / 4
// (at (j * NC + c) * 4), and the f32 sum of the 8 values (the 4 groups of a
// chunk add up to xh[c]).
__device__ __forceinline__ uint4 q4_group(uint4 v, float& s) {
    uint4 o;
    o.x = (v.x & 0xffffu) | (v.z << 16);
    o.y = (v.x >> 16) | (v.z & 0xffff0000u);
    o.z = (v.y & 0xffffu) | (v.w << 16);
    o.w = (v.y >> 16) | (v.w & 0xffff0000u);
    s = ((bf_lo(v.x) + bf_hi(v.x)) + (bf_lo(v.y) + bf_hi(v.y))) +
        ((bf_lo(v.z) + bf_hi(v.z)) + (bf_lo(v.w) + bf_hi(v.w)));
    return o;
}

// Stage bf16 x [K] (global or LDS) for an affine matrix.  All threads of the
// block participate; ends with __syncthreads().
__device__ __forceinline__ void stage_q4(const uint16_t* x, int K, XStage st) {
    const int NC = K / 32, nw = K / 8;
    // blockDim.x and nw are multiples of 4, so the 4 words of a chunk are
    // handled by 4 adjacent lanes in the same iteration; their sums meet
    // with two lane exchanges.
    for (int wi = threadIdx.x; wi < nw; wi += blockDim.x) {
        const int c = wi >> 2, j = wi & 3;
        float s;
        const uint4 o = q4_group(*reinterpret_cast<const uint4*>(x + 8 * wi), s);
        *reinterpret_cast<uint4*>(st.xs + (j * NC + c) * 4) = o;
        s = team_sum<4>(s);
        if (j == 0) st.xh[c] = s;
    }
    __syncthreads();
}

// Stage bf16 x [K] for a bf16 matrix (natural order).
__device__ __forceinline__ void stage_bf16(const uint16_t* x, int K, XStage st) {
    for (int i = threadIdx.x; i < K / 8; i += blockDim.x)
        reinterpret_cast<uint4*>(st.xs)[i] = reinterpret_cast<const uint4*>(x)[i];
    __syncthreads();
}

__device__ __forceinline__ void stage_x(const LinearDev& L, const uint16_t* x, XStage st) {
    if (L.kind == 1)
        stage_q4(x, L.K, st);
    else
        stage_bf16(x, L.K, st);
}

// Partial dot of affine row n over the chunks c = tl, tl+T, ... (no team
// reduction; the caller reduces).  Global scale not applied.
template <int T>
__device__ __forceinline__ float q4_row_partial(const LinearDev& L, int n, const XStage& st, int tl) {
    const int NC = L.K / 32, G = L.K / 64;
    const uint32_t* wrow = L.w + (size_t)n * (L.K / 8);
    const uint16_t* srow = L.s + (size_t)n * G;
    const uint16_t* brow = L.b + (size_t)n * G;
    float acc = 0.0f;
    for (int c = tl; c < NC; c += T) {
        const uint4 w = ldg4(wrow + 4 * c);
        const float s = bf2f(srow[c >> 1]), b = bf2f(brow[c >> 1]);
        const uint4 x0 = *reinterpret_cast<const uint4*>(st.xs + (0 * NC + c) * 4);
        const uint4 x1 = *reinterpret_cast<const uint4*>(st.xs + (1 * NC + c) * 4);
        const uint4 x2 = *reinterpret_cast<const uint4*>(st.xs + (2 * NC + c) * 4);
        const uint4 x3 = *reinterpret_cast<const uint4*>(st.xs + (3 * NC + c) * 4);
        float a0 = q4_word_dot(w.x, reinterpret_cast<const uint32_t*>(&x0), 0.0f);
        float a1 = q4_word_dot(w.y, reinterpret_cast<const uint32_t*>(&x1), 0.0f);
        a0 = q4_word_dot(w.z, reinterpret_cast<const uint32_t*>(&x2), a0);
        a1 = q4_word_dot(w.w, reinterpret_cast<const uint32_t*>(&x3), a1);
        const float a = a0 + a1;
        acc = fmaf(s, a, acc);
        acc = fmaf(b - 128.0f * s, st.xh[c], acc);
    }
    return acc;
}

// Partial dot of bf16 row n over 16 B chunks c = tl, tl+T, ...
template <int T>
__device__ __forceinline__ float bf16_row_partial(const LinearDev& L, int n, const XStage& st, int tl) {
    const int NC = L.K / 8;
    const uint32_t* wrow = L.w + (size_t)n * (L.K / 2);
    float a0 = 0.0f, a1 = 0.0f;
    for (int c = tl; c < NC; c += T) {
        const uint4 w = ldg4(wrow + 4 * c);
        const uint4 x = *reinterpret_cast<const uint4*>(st.xs + 4 * c);
        a0 = dot2(w.x, x.x, a0);
        a1 = dot2(w.y, x.y, a1);
        a0 = dot2(w.z, x.z, a0);
        a1 = dot2(w.w, x.w, a1);
    }
    return a0 + a1;
}

// Full row dot (team-reduced, global scale applied): every lane of the team
// gets the f32 accumulator of row n.
template <int T>
__device__ __forceinline__ float row_dot(const LinearDev& L, int n, const XStage& st, int tl) {
    float a = L.kind == 1 ? q4_row_partial<T>(L, n, st, tl) : bf16_row_partial<T>(L, n, st, tl);
    a = team_sum<T>(a);
    return L.kind == 1 ? a * L.gscale : a;
}

// ---- register-prefetched rows ----------------------------------------------
// A lane's share of one weight row: NCH 16-byte chunks c = c0 + tl + T*j and,
// for affine rows, each chunk's scale and bias (bf16 bits, zero-extended).
// Loading is split from computing so that a stage can issue its weight loads
// before the activation vector is ready (the HBM latency then overlaps the
// wait for the input).  Nothing touches the loaded registers until the
// compute step: an ALU use right after the load would make the compiler wait
// for it there.  Lanes past the end of the row load the row's last chunk
// again (same cache line) and mask it in the compute step, so the number of
// loads does not depend on the lane.  Q4 selects the weight format at compile
// time (1: MLX affine 4-bit, 0: bf16).
template <int NCH>
struct RowRegs {
    uint4 w[NCH];
    uint32_t s[NCH], b[NCH];
};

template <int Q4>
__device__ __forceinline__ int row_chunks(const LinearDev& L) { return Q4 ? L.K / 32 : L.K / 8; }

template <int Q4, int T, int NCH>
__device__ __forceinline__ void row_load(const LinearDev& L, int n, int tl, int c0, RowRegs<NCH>& r) {
    const int NC = row_chunks<Q4>(L), G = L.K / 64;
    const uint32_t* wrow = L.w + (size_t)n * (Q4 ? L.K / 8 : L.K / 2);
#pragma unroll
    for (int j = 0; j < NCH; j++) {
        const int c = min(c0 + tl + T * j, NC - 1);
        r.w[j] = ldg4(wrow + 4 * c);
        if (Q4) {
            r.s[j] = gld(L.s + (size_t)n * G + (c >> 1));
            r.b[j] = gld(L.b + (size_t)n * G + (c >> 1));
        } else {
            r.s[j] = r.b[j] = 0u;
        }
    }
}


// Partial (not team-reduced) dot of the chunks held in r.  Branch-free: a
// chunk past the row's end reads the last chunk (as row_load loads it) and
// its result is not selected, so every chunk's LDS reads can issue ahead of
// the first products instead of one chunk's round trip after another.
template <int Q4, int T, int NCH>
__device__ __forceinline__ float row_compute(const LinearDev& L, const RowRegs<NCH>& r, const XStage& st, int tl,
                                             int c0) {
    const int NC = row_chunks<Q4>(L);
    float acc = 0.0f;
    if (Q4) {
#pragma unroll
        for (int j = 0; j < NCH; j++) {
            const int cr = c0 + tl + T * j;
            const bool in = cr < NC;
            const int c = in ? cr : NC - 1;
            const uint4 x0 = *reinterpret_cast<const uint4*>(st.xs + (0 * NC + c) * 4);
            const uint4 x1 = *reinterpret_cast<const uint4*>(st.xs + (1 * NC + c) * 4);
            const uint4 x2 = *reinterpret_cast<const uint4*>(st.xs + (2 * NC + c) * 4);
            const uint4 x3 = *reinterpret_cast<const uint4*>(st.xs + (3 * NC + c) * 4);
            const float xh = st.xh[c];
            float a0 = q4_word_dot(r.w[j].x, reinterpret_cast<const uint32_t*>(&x0), 0.0f);
            float a1 = q4_word_dot(r.w[j].y, reinterpret_cast<const uint32_t*>(&x1), 0.0f);
            a0 = q4_word_dot(r.w[j].z, reinterpret_cast<const uint32_t*>(&x2), a0);
            a1 = q4_word_dot(r.w[j].w, reinterpret_cast<const uint32_t*>(&x3), a1);
            const float s = bf2f((uint16_t)r.s[j]), b = bf2f((uint16_t)r.b[j]);
            const float t = fmaf(b - 128.0f * s, xh, fmaf(s, a0 + a1, acc));
            acc = in ? t : acc;
        }
    } else {
        float a1 = 0.0f;
#pragma unroll
        for (int j = 0; j < NCH; j++) {
            const int cr = c0 + tl + T * j;
            const bool in = cr < NC;
            const uint4 x = *reinterpret_cast<const uint4*>(st.xs + 4 * (in ? cr : NC - 1));
            const float t0 = dot2(r.w[j].z, x.z, dot2(r.w[j].x, x.x, acc));
            const float t1 = dot2(r.w[j].w, x.w, dot2(r.w[j].y, x.y, a1));
            acc = in ? t0 : acc;
            a1 = in ? t1 : a1;
        }
        acc += a1;
    }
    return acc;
}

// Row n with its first batch of chunks already in `first`; the remaining
// batches (rows longer than T*NCH chunks) are loaded here.  Team-reduced,
// global scale applied.
template <int Q4, int T, int NCH>
__device__ __forceinline__ float row_dot_pf(const LinearDev& L, int n, const XStage& st, int tl,
                                            const RowRegs<NCH>& first) {
    float acc = row_compute<Q4, T, NCH>(L, first, st, tl, 0);
    const int NC = row_chunks<Q4>(L);
    for (int c0 = T * NCH; c0 < NC; c0 += T * NCH) {
        RowRegs<NCH> r;
        row_load<Q4, T, NCH>(L, n, tl, c0, r);
        acc += row_compute<Q4, T, NCH>(L, r, st, tl, c0);
    }
    acc = team_sum<T>(acc);
    return Q4 ? acc * L.gscale : acc;
}

// ---- 16-row MFMA tiles of an affine matrix, K <= 1024 and K % 128 == 0 --------
// A wave computes rows n0 .. n0 + 15 with one v_mfma_f32_16x16x32_bf16 per
// half group (lane layout: A row l % 16, B column l % 16, k-block l / 16;
// C[r] = (row 4 (l / 16) + r, column l % 16)).  Lane (n = l % 16, kq = l / 16)
// holds words 2 kq and 2 kq + 1 of every group of row n0 + n as the B
// operands of the group's two MFMAs, unpacked to (128 + q) bf16 pairs (the
// order of q4_pairs); the A operand is x at the same k positions in the row of
// the group's index and zero in every other row.  C[g][n] is then row n's sum
// over group g alone, and each (row, group) sum meets its scale and bias once:
// y[n] = g_s * sum_g (s_g C[g][n] + (b_g - 128 s_g) xsum_g).  The K order of
// the sums is the matrix cores', so rows differ from row_dot's in the last
// bits (within the f32 error of either).
constexpr int kTileMaxG = 16;

// The tiles need G = K / 64 even as well: a lane's scales (and biases) are one
// 8-byte buffer load at byte n * 2G + 8 kq, which must be 4-byte aligned.
__host__ __device__ constexpr bool q4tile_fits(int K) {
    return K % 128 == 0 && K <= 64 * kTileMaxG;
}

struct Q4Tile {
    uint2 w[kTileMaxG];  // words 2 kq, 2 kq + 1 of group g
    uint2 s, b;          // bf16 scales / biases of groups 4 kq .. 4 kq + 3
};

// Per-lane operands that do not depend on the rows: x of this lane's group
// (g = l % 16) at words 2 kq + h, and the x sums of groups 4 kq + i.
struct Q4TileX {
    uint4 x[2];
    float xsum[4];
};

__device__ __forceinline__ __amdgpu_buffer_rsrc_t q4tile_rsrc(const uint16_t* p, int N, int G) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(p), 0, N * G * 2, 0x00020000);
}

// Row n's words and scales for this lane (n clamped by the caller; scale
// words past the row read the next row's, or zero past the matrix: unused).
// Requires q4tile_fits(L.K).
__device__ __forceinline__ void q4tile_load(const LinearDev& L, int n, int kq, __amdgpu_buffer_rsrc_t rs,
                                            __amdgpu_buffer_rsrc_t rb, Q4Tile& r) {
    const int G = L.K / 64;
    const uint32_t* wrow = L.w + (size_t)n * (L.K / 8) + 2 * kq;
    typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
#pragma unroll
    for (int g = 0; g < kTileMaxG; g++)
        if (g < G) {
            const u32x2 v = *(const MING_GLOBAL u32x2*)(wrow + 8 * g);
            r.w[g] = make_uint2(v.x, v.y);
        }
    const auto s2 = __builtin_amdgcn_raw_buffer_load_b64(rs, n * G * 2 + 8 * kq, 0, 0);
    const auto b2 = __builtin_amdgcn_raw_buffer_load_b64(rb, n * G * 2 + 8 * kq, 0, 0);
    r.s = make_uint2(s2[0], s2[1]);
    r.b = make_uint2(b2[0], b2[1]);
}

__device__ __forceinline__ Q4TileX q4tile_x(const XStage& st, int K, int lane) {
    const int G = K / 64, NC = K / 32, n16 = lane % 16, kq = lane / 16;
    Q4TileX t;
    const int g = min(n16, G - 1);
#pragma unroll
    for (int h = 0; h < 2; h++) {
        const int wi = 2 * kq + h, c = 2 * g + wi / 4, j = wi % 4;
        t.x[h] = *reinterpret_cast<const uint4*>(st.xs + (j * NC + c) * 4);
    }
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int gi = min(4 * kq + i, G - 1);
        t.xsum[i] = st.xh[2 * gi] + st.xh[2 * gi + 1];
    }
    return t;
}

// The tile's group sums C (lane: groups 4 kq + r of row n0 + l % 16).  The A
// operands are selected here, per MFMA, rather than kept for every group
// (which would hold 32 x 4 registers per lane).
__device__ __forceinline__ f32x4_t q4tile_mma(const LinearDev& L, const Q4Tile& r, const Q4TileX& t, int lane) {
    const int G = L.K / 64;
    int n16 = lane % 16;
    asm volatile("" : "+v"(n16));  // keeps the selects at the MFMAs
    f32x4_t C = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int g = 0; g < kTileMaxG; g++) {
        if (g < G) {
            const bool on = n16 == g;
#pragma unroll
            for (int h = 0; h < 2; h++) {
                const uint32_t w = h == 0 ? r.w[g].x : r.w[g].y;
                uint32_t p0, p1, p2, p3;
                q4_pairs(w, p0, p1, p2, p3);
                const uint4 a = on ? t.x[h] : make_uint4(0u, 0u, 0u, 0u);
                C = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf8(a), as_bf8(make_uint4(p0, p1, p2, p3)), C, 0, 0, 0);
            }
        }
    }
    return C;
}

// Row n0 + l % 16 of the tile (every lane of that column holds it), global
// scale applied, from the group sums and the row's scales s and biases b.
__device__ __forceinline__ float q4tile_finish(const LinearDev& L, f32x4_t C, uint2 s, uint2 b, const Q4TileX& t,
                                               int lane) {
    const int G = L.K / 64, kq = lane / 16;
    const uint32_t sw[4] = {s.x << 16, s.x & 0xffff0000u, s.y << 16, s.y & 0xffff0000u};
    const uint32_t bw[4] = {b.x << 16, b.x & 0xffff0000u, b.y << 16, b.y & 0xffff0000u};
    float p = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        if (4 * kq + i < G) {
            const float sc = __uint_as_float(sw[i]), bi = __uint_as_float(bw[i]);
            p = fmaf(sc, C[i], p);
            p = fmaf(bi - 128.0f * sc, t.xsum[i], p);
        }
    }
    p = rows_sum(p);
    return p * L.gscale;
}

template <int Q4>
__device__ __forceinline__ void stage_xk(const uint16_t* x, int K, XStage st) {
    if (Q4)
        stage_q4(x, K, st);
    else
        stage_bf16(x, K, st);
}

}  // namespace ming
