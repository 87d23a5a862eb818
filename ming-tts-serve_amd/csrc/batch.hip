// Batched decode of many sequences over a paged KV cache: the element-wise and
// attention kernels around the batched 4-bit GEMM (qgemm.hip).  One step of
// n_seq sequences runs, per layer: rms + staging, q/k/v GEMM (bias, rope and
// the k/v append in its epilogue), paged attention over splits of 4 pages,
// split merge + staging, o GEMM + residual, rms + staging, gate/up GEMM +
// swiglu, staging, down GEMM + residual.  Rounding points are those of the
// batch-1 layer (src/ming_fused.zig:296-324, :384-394).
#include "batch.h"
#include "common.h"
#include "internal.h"

namespace ming {

namespace {


// 8 bf16 of a 16-byte word in natural order -> pair order (x0,x4) (x1,x5) (x2,x6) (x3,x7).
__device__ __forceinline__ uint4 pair_order(uint4 e) {
    return make_uint4((e.x & 0xffffu) | (e.z << 16), (e.x >> 16) | (e.z & 0xffff0000u), (e.y & 0xffffu) | (e.w << 16),
                      (e.y >> 16) | (e.w & 0xffff0000u));
}

// ---- staging: (optional rms) of rows of x into the GEMM's A layout -----------------
// One workgroup per row m < Mp (rows >= M are written as zeros).  rms_norm as
// MLX fast::rms_norm: bf16(w * bf16(x * rsqrt(mean(x^2) + eps))).  hout, when
// set, receives the (normed) bf16 row; pos_inc, when set, is incremented per row.
template <bool NORM>
__global__ __launch_bounds__(256) void stage_kernel(const uint16_t* __restrict__ x, int ldx, int M, int K,
                                                    const uint16_t* __restrict__ w, float eps, uint4* __restrict__ xs,
                                                    float* __restrict__ xsum, uint16_t* __restrict__ hout,
                                                    int32_t* __restrict__ pos_inc) {
    __shared__ float red[4];
    const int m = blockIdx.x, Mp = gridDim.x, tid = threadIdx.x, KW8 = K / 8, G = K / 64;
    // group-major: word wi = 8 g + w of row m at xs[(g Mp + m) 8 + w], its group sum at xsum[g Mp + m]
    auto xw = [&](int wi) { return xs + ((size_t)(wi / 8) * Mp + m) * 8 + wi % 8; };
    if (m >= M) {
        for (int wi = tid; wi < KW8; wi += 256) gst(xw(wi), make_uint4(0, 0, 0, 0));
        for (int g = tid; g < G; g += 256) gst(xsum + (size_t)g * Mp + m, 0.0f);
        return;
    }
    const uint16_t* row = x + (size_t)m * ldx;
    float inv = 1.0f;
    if (NORM) {
        float ss = 0.0f;
        for (int wi = tid; wi < KW8; wi += 256) {
            const uint4 v = ldg4(row + 8 * wi);
            const uint32_t e[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
            for (int p = 0; p < 4; p++) {
                const float lo = bf_lo(e[p]), hi = bf_hi(e[p]);
                ss += lo * lo;
                ss += hi * hi;
            }
        }
        ss = block_sum(ss, red);
        inv = 1.0f / sqrtf(ss / (float)K + eps);
    }
    // K % 64 == 0: the 8 lanes holding one group's words are active together
    for (int wi = tid; wi < KW8; wi += 256) {
        uint4 v = ldg4(row + 8 * wi);
        if (NORM) {
            const uint4 wv = ldg4(w + 8 * wi);
            const uint32_t e[4] = {v.x, v.y, v.z, v.w}, we[4] = {wv.x, wv.y, wv.z, wv.w};
            uint32_t o[4];
#pragma unroll
            for (int p = 0; p < 4; p++)
                o[p] = pack_bf2(bf_lo(we[p]) * rb(bf_lo(e[p]) * inv), bf_hi(we[p]) * rb(bf_hi(e[p]) * inv));
            v = make_uint4(o[0], o[1], o[2], o[3]);
        }
        if (hout) gst(reinterpret_cast<uint4*>(hout + (size_t)m * K) + wi, v);
        gst(xw(wi), pair_order(v));
        const uint32_t e[4] = {v.x, v.y, v.z, v.w};
        float s = 0.0f;
#pragma unroll
        for (int p = 0; p < 4; p++) s += bf_lo(e[p]) + bf_hi(e[p]);
        s += __shfl_xor(s, 1);
        s += __shfl_xor(s, 2);
        s += __shfl_xor(s, 4);
        if (tid % 8 == 0) gst(xsum + (size_t)(wi / 8) * Mp + m, s);
    }
    if (pos_inc && tid == 0) gst(pos_inc + m, gld(pos_inc + m) + 1);
}

// ---- embedding rows (the batch-1 embed, one row per sequence) -------------------------
__global__ __launch_bounds__(256) void embed_rows_kernel(LinearDev E, const int32_t* __restrict__ tokens,
                                                         uint16_t* __restrict__ x) {
    const int b = blockIdx.x;
    int id = gld(tokens + b);
    id = id < 0 ? 0 : (id >= E.N ? E.N - 1 : id);
    uint4* xo = reinterpret_cast<uint4*>(x + (size_t)b * E.K);
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
            gst(xo + wi, make_uint4(o[0], o[1], o[2], o[3]));
        }
    } else {
        const uint4* row = reinterpret_cast<const uint4*>(reinterpret_cast<const uint16_t*>(E.w) + (size_t)id * E.K);
        for (int i = threadIdx.x; i < E.K / 8; i += blockDim.x) gst(xo + i, ldg4(row + i));
    }
}

// ---- rope table: (cos, sin) of p * inv_freq[i], as the batch-1 layer computes them ----
__global__ __launch_bounds__(256) void rope_table_kernel(float* __restrict__ cs, int max_ctx, int half,
                                                         float log2_theta) {
    const int k = blockIdx.x * 256 + threadIdx.x;
    if (k >= max_ctx * half) return;
    const int p = k / half, d = k % half;
    const float inv_freq = exp2f(-((float)d / (float)half) * log2_theta);
    const float th = (float)p * inv_freq;
    gst(cs + 2 * k, cosf(th));
    gst(cs + 2 * k + 1, sinf(th));
}

// ---- paged attention ------------------------------------------------------------------
// Workgroup (split s, kv head g, sequence b); wave w takes page 4s + w (64
// positions).  Both products run on the matrix cores with the kv head's grp
// query heads as the 16-wide MFMA column (heads >= grp are zero):
//   S^T [64 positions][heads] = K q^T: A = K rows, B = q^T (q * scale, exact
//   for scale 2^-3); the A row i of tile t is position 32(t/2) + 8(i/4) +
//   4(t%2) + i%4, so that lane (c, j) ends with positions 32u + 8j + 0..7 of
//   k-block u in the C registers of tiles 2u, 2u+1 -- exactly the B operand
//   P^T of the next product.
//   O^T [64 dims][heads] = V^T P^T: A = V^T (the page is stored transposed:
//   8 positions of one dim are 16 contiguous bytes), B = P^T split as
//   bf16 hi + bf16 lo (two MFMAs), which keeps p to ~2^-17 relative.
// The four waves' (max, sum, o) are combined through LDS into one partial.
__global__ __launch_bounds__(256) void paged_attn_kernel(PagedAttnArgs a) {
    __shared__ float so[3][16][64];
    __shared__ float sm[4][16], sl[4][16];
    const int s = blockIdx.x, g = blockIdx.y, b = blockIdx.z;
    const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave, c = lane % 16, j = lane / 16;
    const int pos = gld(a.pos + b);
    if (pos < 0 || pos >= a.pages_per_seq * 64) {
        if (threadIdx.x == 0 && s == 0 && g == 0) gst(a.flags, 1);
        return;
    }
    const int len = pos + 1, nsplit = (len + 255) / 256;
    if (s >= nsplit) return;
    const int pi = 4 * s + wave;
    bool has = pi * 64 < len;
    int page = 0;
    if (has) {
        page = gld(a.table + (size_t)b * a.pages_per_seq + pi);
        if (page < 0 || page >= a.n_pages) {
            has = false;
            if (lane == 0) gst(a.flags, 1);
        }
    }
    float mrun = -INFINITY, lrun = 0.0f;
    f32x4_t o[4];
#pragma unroll
    for (int dt = 0; dt < 4; dt++) o[dt] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
    if (has) {
        const size_t pbase = ((size_t)page * a.kvh + g) * 64 * 64;
        const uint16_t* kb = a.kp + pbase;
        const uint16_t* vb = a.vp + pbase;
        uint4 ka[4][2], va[4][2];
#pragma unroll
        for (int t = 0; t < 4; t++) {
            const int p = 32 * (t / 2) + 8 * (c / 4) + 4 * (t % 2) + c % 4;
            const uint16_t* kr = kb + p * 64 + 16 * j;
            ka[t][0] = ldg4(kr);
            ka[t][1] = ldg4(kr + 8);
        }
#pragma unroll
        for (int dt = 0; dt < 4; dt++)
#pragma unroll
            for (int u = 0; u < 2; u++) va[dt][u] = ldg4(vb + (16 * dt + c) * 64 + 32 * u + 8 * j);
        uint4 q[2] = {make_uint4(0, 0, 0, 0), make_uint4(0, 0, 0, 0)};
        if (c < a.grp) {
            const uint16_t* qr = a.qkv + (size_t)b * a.ldq + (g * a.grp + c) * 64 + 16 * j;
#pragma unroll
            for (int h = 0; h < 2; h++) {
                const uint4 v = ldg4(qr + 8 * h);
                const uint32_t e[4] = {v.x, v.y, v.z, v.w};
                uint32_t r4[4];
#pragma unroll
                for (int p = 0; p < 4; p++) r4[p] = pack_bf2(bf_lo(e[p]) * a.scale, bf_hi(e[p]) * a.scale);
                q[h] = make_uint4(r4[0], r4[1], r4[2], r4[3]);
            }
        }
        f32x4_t sc[4];
#pragma unroll
        for (int t = 0; t < 4; t++) {
            sc[t] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
            sc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf8(ka[t][0]), as_bf8(q[0]), sc[t], 0, 0, 0);
            sc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf8(ka[t][1]), as_bf8(q[1]), sc[t], 0, 0, 0);
        }
        const int base = pi * 64;
        float mx = -INFINITY;
#pragma unroll
        for (int t = 0; t < 4; t++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int p = 32 * (t / 2) + 8 * j + 4 * (t % 2) + r;
                if (base + p >= len) sc[t][r] = -INFINITY;
                mx = fmaxf(mx, sc[t][r]);
            }
        mx = rows_max(mx);
        float l = 0.0f;
#pragma unroll
        for (int t = 0; t < 4; t++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const float e = att_exp(sc[t][r] - mx);  // masked scores (-inf) give 0
                sc[t][r] = e;
                l += e;
            }
        l = rows_sum(l);
#pragma unroll
        for (int u = 0; u < 2; u++) {
            uint32_t hi[4], lo[4];
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const float p0 = sc[2 * u + k / 2][2 * (k % 2)], p1 = sc[2 * u + k / 2][2 * (k % 2) + 1];
                hi[k] = pack_bf2(p0, p1);
                lo[k] = pack_bf2(p0 - bf_lo(hi[k]), p1 - bf_hi(hi[k]));
            }
            const bf16x8_t ph = as_bf8(make_uint4(hi[0], hi[1], hi[2], hi[3]));
            const bf16x8_t pl = as_bf8(make_uint4(lo[0], lo[1], lo[2], lo[3]));
#pragma unroll
            for (int dt = 0; dt < 4; dt++) {
                o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf8(va[dt][u]), ph, o[dt], 0, 0, 0);
                o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf8(va[dt][u]), pl, o[dt], 0, 0, 0);
            }
        }
        mrun = mx;
        lrun = l;
    }
    // lane (c, j): o[dt][r] = O[head c][dim 16 dt + 4 j + r]
    if (wave > 0)
#pragma unroll
        for (int dt = 0; dt < 4; dt++)
#pragma unroll
            for (int r = 0; r < 4; r++) so[wave - 1][dt * 4 + r][lane] = o[dt][r];
    if (j == 0) {
        sm[wave][c] = mrun;
        sl[wave][c] = lrun;
    }
    __syncthreads();
    if (wave > 0) return;
    float M = sm[0][c];
#pragma unroll
    for (int w = 1; w < 4; w++) M = fmaxf(M, sm[w][c]);
    float f[4], L = 0.0f;
#pragma unroll
    for (int w = 0; w < 4; w++) {
        f[w] = sm[w][c] == -INFINITY ? 0.0f : att_exp(sm[w][c] - M);
        L += f[w] * sl[w][c];
    }
    if (c >= a.grp) return;
    float* pp = a.part + ((((size_t)b * a.kvh + g) * a.max_splits + s) * a.grp + c) * 68;
#pragma unroll
    for (int dt = 0; dt < 4; dt++) {
        float v[4];
#pragma unroll
        for (int r = 0; r < 4; r++) {
            v[r] = f[0] * o[dt][r];
#pragma unroll
            for (int w = 1; w < 4; w++) v[r] += f[w] * so[w - 1][dt * 4 + r][lane];
        }
        gst(reinterpret_cast<uint4*>(pp + 16 * dt + 4 * j),
            make_uint4(__float_as_uint(v[0]), __float_as_uint(v[1]), __float_as_uint(v[2]), __float_as_uint(v[3])));
    }
    if (j == 0) {
        gst(pp + 64, M);
        gst(pp + 65, L);
    }
}

// ---- split merge + staging for the o projection ------------------------------------------
// One wave per (sequence, head); lane = dim.  att = bf16(sum_s f_s o_s / sum_s f_s l_s),
// f_s = exp(m_s - max m); written as the attention row and as the staged A words
// (the head's 64 dims are one group of the o projection's K).
__global__ __launch_bounds__(256) void merge_stage_kernel(MergeArgs a) {
    const int item = blockIdx.x * 4 + threadIdx.x / kWave, lane = threadIdx.x % kWave;
    if (item >= a.n_seq * a.heads) return;
    const int b = item / a.heads, h = item % a.heads, g = h / a.grp, c = h % a.grp;
    const int pos = gld(a.pos + b);
    const int nsplit = min(max((pos + 256) / 256, 1), a.max_splits);
    const size_t stride = (size_t)a.grp * 68;
    const float* pp = a.part + (((size_t)b * a.kvh + g) * a.max_splits * a.grp + c) * 68;
    float M = -INFINITY;
    for (int s = lane; s < nsplit; s += kWave) M = fmaxf(M, gld(pp + s * stride + 64));
    M = team_max<kWave>(M);
    float o = 0.0f, L = 0.0f;
    for (int s = 0; s < nsplit; s++) {
        const float ms = gld(pp + s * stride + 64), ls = gld(pp + s * stride + 65);
        const float f = ms == -INFINITY ? 0.0f : att_exp(ms - M);
        L += f * ls;
        o += f * gld(pp + s * stride + lane);
    }
    const uint32_t hb = f2bf(o / L);
    const int H = a.heads * 64;
    gst(a.att + (size_t)b * H + h * 64 + lane, (uint16_t)hb);
    const uint32_t word = hb | (__shfl_down(hb, 4) << 16);  // lanes with lane % 8 < 4
    const uint32_t w1 = __shfl_down(word, 1), w2 = __shfl_down(word, 2), w3 = __shfl_down(word, 3);
    // the head's 64 dims are group h of the o projection's K (group-major staging)
    if (lane % 8 == 0)
        gst(static_cast<uint4*>(a.xs) + ((size_t)h * a.Mp + b) * 8 + lane / 8, make_uint4(word, w1, w2, w3));
    const float sum = team_sum<kWave>(bf2f((uint16_t)hb));
    if (lane == 0) gst(a.xsum + (size_t)h * a.Mp + b, sum);
}

// ---- prefill rows: n virtual sequences over one sequence's pages ----------------------
// Row i of the chunk is position p0 + i of the same sequence: its page-table
// row is the sequence's table and its position p0 + i.
__global__ __launch_bounds__(256) void prefill_rows_kernel(const int32_t* __restrict__ table, int pps, int n, int p0,
                                                           int32_t* __restrict__ rows, int32_t* __restrict__ pos) {
    const int k = blockIdx.x * 256 + threadIdx.x;
    if (k < n * pps) gst(rows + k, gld(table + k % pps));
    if (k < n) gst(pos + k, p0 + k);
}

// ---- pages -> contiguous cache rows -------------------------------------------------
// Positions [p0, p0 + n) of one sequence whose pages are 0, 1, 2, ... in
// position order, copied into a contiguous cache [n_layers][kvh][cap][64].
// Thread = (layer, head, position, 8-dim chunk): K rows are contiguous in
// both layouts (one 16-byte load and store); a V page is stored transposed
// ([dim][64 positions]), so its 8 dims are gathered 64 elements apart.
__global__ __launch_bounds__(256) void pages_to_rows_kernel(const uint16_t* __restrict__ kp,
                                                            const uint16_t* __restrict__ vp, int n_layers, int kvh,
                                                            int n_pages, int p0, int n, uint16_t* __restrict__ kc,
                                                            uint16_t* __restrict__ vc, int cap) {
    const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int64_t total = (int64_t)n_layers * kvh * n * 8;
    if (t >= total) return;
    const int c = (int)(t & 7);
    int64_t r = t >> 3;
    const int i = (int)(r % n);
    r /= n;
    const int h = (int)(r % kvh);
    const int l = (int)(r / kvh);
    const int p = p0 + i;
    const int64_t page = ((int64_t)l * n_pages + p / 64) * kvh + h;  // [layer][page][head] block of 64 x 64
    const int64_t dst = (((int64_t)l * kvh + h) * cap + p) * 64 + c * 8;
    gst(reinterpret_cast<uint4*>(kc + dst), ldg4(kp + page * 4096 + (p % 64) * 64 + c * 8));
    const uint16_t* vs = vp + page * 4096 + (c * 8) * 64 + p % 64;
    uint16_t v8[8];
#pragma unroll
    for (int j = 0; j < 8; j++) v8[j] = gld(vs + j * 64);
    uint4 o;
    o.x = v8[0] | (uint32_t)v8[1] << 16;
    o.y = v8[2] | (uint32_t)v8[3] << 16;
    o.z = v8[4] | (uint32_t)v8[5] << 16;
    o.w = v8[6] | (uint32_t)v8[7] << 16;
    gst(reinterpret_cast<uint4*>(vc + dst), o);
}

}  // namespace

hipError_t launch_pages_to_rows(hipStream_t st, const uint16_t* kp, const uint16_t* vp, int n_layers, int kvh,
                                int n_pages, int p0, int n, uint16_t* kc, uint16_t* vc, int cap) {
    if (n_layers < 1 || kvh < 1 || n < 1 || p0 < 0 || p0 + n > n_pages * 64 || p0 + n > cap)
        return hipErrorInvalidValue;
    const int64_t total = (int64_t)n_layers * kvh * n * 8;
    hipLaunchKernelGGL(pages_to_rows_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, st, kp, vp,
                       n_layers, kvh, n_pages, p0, n, kc, vc, cap);
    return hipGetLastError();
}

hipError_t launch_stage(hipStream_t st, const uint16_t* x, int ldx, int M, int K, const uint16_t* norm_w, float eps,
                        void* xs, float* xsum, uint16_t* hout, int32_t* pos_inc) {
    const int Mp = (M + 15) / 16 * 16;
    if (norm_w)
        hipLaunchKernelGGL(stage_kernel<true>, dim3(Mp), dim3(256), 0, st, x, ldx, M, K, norm_w, eps,
                           static_cast<uint4*>(xs), xsum, hout, pos_inc);
    else
        hipLaunchKernelGGL(stage_kernel<false>, dim3(Mp), dim3(256), 0, st, x, ldx, M, K, norm_w, eps,
                           static_cast<uint4*>(xs), xsum, hout, pos_inc);
    return hipGetLastError();
}

hipError_t launch_embed_rows(hipStream_t st, const LinearDev& E, const int32_t* tokens, int n, uint16_t* x) {
    hipLaunchKernelGGL(embed_rows_kernel, dim3(n), dim3(256), 0, st, E, tokens, x);
    return hipGetLastError();
}

hipError_t launch_rope_table(hipStream_t st, float* cs, int max_ctx, int half, float log2_theta) {
    const int n = max_ctx * half;
    hipLaunchKernelGGL(rope_table_kernel, dim3((n + 255) / 256), dim3(256), 0, st, cs, max_ctx, half, log2_theta);
    return hipGetLastError();
}

hipError_t launch_paged_attn(hipStream_t st, const PagedAttnArgs& a, int n_seq) {
    hipLaunchKernelGGL(paged_attn_kernel, dim3(a.max_splits, a.kvh, n_seq), dim3(256), 0, st, a);
    return hipGetLastError();
}

hipError_t launch_prefill_rows(hipStream_t st, const int32_t* table, int pps, int n, int p0, int32_t* rows,
                               int32_t* pos) {
    const int k = n * pps > n ? n * pps : n;
    hipLaunchKernelGGL(prefill_rows_kernel, dim3((k + 255) / 256), dim3(256), 0, st, table, pps, n, p0, rows, pos);
    return hipGetLastError();
}

hipError_t launch_merge_stage(hipStream_t st, const MergeArgs& a) {
    const int items = a.n_seq * a.heads;
    hipLaunchKernelGGL(merge_stage_kernel, dim3((items + 3) / 4), dim3(256), 0, st, a);
    return hipGetLastError();
}

}  // namespace ming
