/*
 * oracle_vae.c -- CPU restatement of the reference's VAE decoder
 * (Model.vaeDecode, src/ming_model.zig:1257-1309): fc1, the 4x linear
 * upsample (:1316-1340), the 24-layer sliding-window Qwen2 stack
 * (QStack.forward with window 64, :566-614, mask :618-636) and the ISTFT head
 * (exp/min magnitude, phase, irfft n_fft, window, overlap-add, envelope,
 * "same" trim).
 *
 * TEST INFRASTRUCTURE ONLY (see oracle.h).
 *
 * Precision follows the MLX graph: fc1 runs on the bf16 latents (addmm, one
 * bf16 rounding); the upsample casts to f32, so every later array of the
 * graph is f32 (bf16 weights and norms are promoted), and nothing after it is
 * rounded to bf16.  irfft is evaluated as a direct sum in double and rounded
 * to f32 once (MLX's pocketfft c2r rounds differently at the f32 ulp level).
 */
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "oracle.h"

#ifndef M_PI
#define M_PI 3.14159265358979323846
#endif

/* Dequantized weight (n, k) in f32, as MLX's f32 kernels see it: bf16 weights
 * widened exactly; affine weights scale * q + bias (times the global scale). */
static float wf32(const or_linear* L, int64_t n, int64_t k) {
    if (L->kind == OR_W_BF16) return or_f32(((const uint16_t*)L->w)[n * L->K + k]);
    const int64_t per = 32 / L->bits, wpr = L->K / per;
    const uint32_t word = ((const uint32_t*)L->w)[n * wpr + k / per];
    const uint32_t q = (word >> (L->bits * (k % per))) & ((1u << L->bits) - 1u);
    const int64_t g = n * (L->K / L->group) + k / L->group;
    float v = or_f32(L->scales[g]) * (float)q + or_f32(L->biases[g]);
    if (L->gscale != 1.0f) v *= L->gscale;
    return v;
}

void or_linear_f32(const or_linear* L, const float* x, int64_t M, const uint16_t* bias, float* y) {
    const int64_t N = L->N, K = L->K;
    float* wt = malloc(sizeof(float) * (size_t)(N * K));
#pragma omp parallel for schedule(static)
    for (int64_t n = 0; n < N; n++)
        for (int64_t k = 0; k < K; k++) wt[n * K + k] = wf32(L, n, k);
#pragma omp parallel for collapse(2) schedule(static)
    for (int64_t m = 0; m < M; m++)
        for (int64_t n = 0; n < N; n++) {
            const float* xr = x + m * K;
            const float* wr = wt + n * K;
            float p[8] = {0};
            for (int64_t k = 0; k < K; k++) p[k % 8] += wr[k] * xr[k];
            float acc = ((p[0] + p[1]) + (p[2] + p[3])) + ((p[4] + p[5]) + (p[6] + p[7]));
            if (bias) acc += or_f32(bias[n]);
            y[m * N + n] = acc;
        }
    free(wt);
}

/* MLX fast::rms_norm on f32 rows with a bf16 weight: w * (x * rsqrt(mean(x^2) + eps)). */
void or_rms_f32(const float* x, const uint16_t* w, int64_t M, int64_t n, float eps, float* out) {
    for (int64_t m = 0; m < M; m++) {
        const float* xr = x + m * n;
        float p[8] = {0};
        for (int64_t i = 0; i < n; i++) p[i % 8] += xr[i] * xr[i];
        const float ss = ((p[0] + p[1]) + (p[2] + p[3])) + ((p[4] + p[5]) + (p[6] + p[7]));
        const float inv = 1.0f / sqrtf(ss / (float)n + eps);
        for (int64_t i = 0; i < n; i++) out[m * n + i] = or_f32(w[i]) * (xr[i] * inv);
    }
}

/* MLX fast::rope, traditional=false, on f32 heads x [nh][hd] at position pos. */
void or_rope_f32(float* x, int nh, int hd, int pos, float log2_base) {
    const int half = hd / 2;
    for (int i = 0; i < half; i++) {
        const float inv_freq = exp2f(-((float)i / (float)half) * log2_base);
        const float th = (float)pos * inv_freq;
        const float c = cosf(th), s = sinf(th);
        for (int h = 0; h < nh; h++) {
            float* r = x + h * hd;
            const float x1 = r[i], x2 = r[i + half];
            r[i] = x1 * c - x2 * s;
            r[i + half] = x1 * s + x2 * c;
        }
    }
}

/* Decoder._linear_upsample_1d, align_corners=False (src/ming_model.zig:1316-1340):
 * bf16 x [T][C] -> f32 y [T*scale][C]; pos = (i + 0.5) / scale - 0.5, clamped
 * neighbours, y = x[l] * (1 - w) + x[r] * w. */
void or_linear_upsample(const uint16_t* x, int T, int C, int scale, float* y) {
    const float sc = (float)scale;
    for (int i = 0; i < T * scale; i++) {
        const float pos = ((float)i + 0.5f) / sc - 0.5f;
        const float lf = floorf(pos);
        const int left = (int)lf;
        const float wr = pos - (float)left, wl = 1.0f - wr;
        const int l = left < 0 ? 0 : (left > T - 1 ? T - 1 : left);
        const int r = left + 1 < 0 ? 0 : (left + 1 > T - 1 ? T - 1 : left + 1);
        for (int c = 0; c < C; c++) y[(int64_t)i * C + c] = or_f32(x[(int64_t)l * C + c]) * wl + or_f32(x[(int64_t)r * C + c]) * wr;
    }
}

/* Sliding-window causal attention over F rows (the mask of
 * src/ming_model.zig:618-636: key j is visible to query i when
 * i - window < j <= i).  q [F][heads][hd], k/v [F][kv_heads][hd] f32 -> out
 * [F][heads][hd] f32; softmax in f32 over the visible keys. */
void or_window_attention(const float* q, const float* k, const float* v, int F, int heads, int kv_heads, int hd,
                         int window, float scale, float* out) {
    const int grp = heads / kv_heads;
#pragma omp parallel for collapse(2) schedule(static)
    for (int i = 0; i < F; i++)
        for (int h = 0; h < heads; h++) {
            const float* qi = q + ((int64_t)i * heads + h) * hd;
            const int kh = h / grp;
            const int j0 = i - window + 1 > 0 ? i - window + 1 : 0;
            const int n = i - j0 + 1;
            float* s = malloc(sizeof(float) * (size_t)n);
            float mx = -INFINITY;
            for (int j = j0; j <= i; j++) {
                const float* kj = k + ((int64_t)j * kv_heads + kh) * hd;
                float p[8] = {0};
                for (int d = 0; d < hd; d++) p[d % 8] += qi[d] * kj[d];
                const float dot = ((p[0] + p[1]) + (p[2] + p[3])) + ((p[4] + p[5]) + (p[6] + p[7]));
                s[j - j0] = dot * scale;
                if (s[j - j0] > mx) mx = s[j - j0];
            }
            float l = 0.0f;
            for (int t = 0; t < n; t++) {
                s[t] = expf(s[t] - mx);
                l += s[t];
            }
            float* o = out + ((int64_t)i * heads + h) * hd;
            for (int d = 0; d < hd; d++) {
                float acc = 0.0f;
                for (int j = j0; j <= i; j++) acc += s[j - j0] * v[((int64_t)j * kv_heads + kh) * hd + d];
                o[d] = acc / l;
            }
            free(s);
        }
}

/* One Qwen2 layer of the VAE backbone on all F rows (QStack.forward, no
 * cache, offset 0: row i sits at position i). */
void or_vae_layer(const or_vae_cfg* c, const or_lm_layer* l, const float* x, int F, float* x_out, or_vae_trace* tr) {
    const int H = c->hidden, hd = c->head_dim, kvd = c->kv_heads * hd, I = c->inter;
    float* h = malloc(sizeof(float) * (size_t)F * H);
    float* q = malloc(sizeof(float) * (size_t)F * H);
    float* k = malloc(sizeof(float) * (size_t)F * kvd);
    float* v = malloc(sizeof(float) * (size_t)F * kvd);
    float* att = malloc(sizeof(float) * (size_t)F * H);
    float* o = malloc(sizeof(float) * (size_t)F * H);
    float* x1 = malloc(sizeof(float) * (size_t)F * H);
    float* g = malloc(sizeof(float) * (size_t)F * I);
    float* u = malloc(sizeof(float) * (size_t)F * I);
    float* d = malloc(sizeof(float) * (size_t)F * H);
    or_rms_f32(x, l->ln1, F, H, c->eps, h);
    or_linear_f32(&l->q, h, F, l->bq, q);
    or_linear_f32(&l->k, h, F, l->bk, k);
    or_linear_f32(&l->v, h, F, l->bv, v);
    for (int i = 0; i < F; i++) {
        or_rope_f32(q + (int64_t)i * H, c->heads, hd, i, c->log2_theta);
        or_rope_f32(k + (int64_t)i * kvd, c->kv_heads, hd, i, c->log2_theta);
    }
    or_window_attention(q, k, v, F, c->heads, c->kv_heads, hd, c->window, 1.0f / sqrtf((float)hd), att);
    or_linear_f32(&l->o, att, F, NULL, o);
    for (int64_t i = 0; i < (int64_t)F * H; i++) x1[i] = x[i] + o[i];
    or_rms_f32(x1, l->ln2, F, H, c->eps, h);
    or_linear_f32(&l->gate, h, F, NULL, g);
    or_linear_f32(&l->up, h, F, NULL, u);
    /* compiled swiglu in f32: (g * sigmoid(g)) * u */
    for (int64_t i = 0; i < (int64_t)F * I; i++) {
        const float sg = 1.0f / (1.0f + expf(-g[i]));
        g[i] = (g[i] * sg) * u[i];
    }
    or_linear_f32(&l->down, g, F, NULL, d);
    for (int64_t i = 0; i < (int64_t)F * H; i++) x_out[i] = x1[i] + d[i];
    if (tr) {
        if (tr->qkv)
            for (int i = 0; i < F; i++) {
                float* r = tr->qkv + (int64_t)i * (H + 2 * kvd);
                memcpy(r, q + (int64_t)i * H, sizeof(float) * H);
                memcpy(r + H, k + (int64_t)i * kvd, sizeof(float) * kvd);
                memcpy(r + H + kvd, v + (int64_t)i * kvd, sizeof(float) * kvd);
            }
        if (tr->att) memcpy(tr->att, att, sizeof(float) * (size_t)F * H);
        if (tr->x1) memcpy(tr->x1, x1, sizeof(float) * (size_t)F * H);
        if (tr->hh) memcpy(tr->hh, g, sizeof(float) * (size_t)F * I);
    }
    free(h);
    free(q);
    free(k);
    free(v);
    free(att);
    free(o);
    free(x1);
    free(g);
    free(u);
    free(d);
}

/* The ISTFT head after dec_head (src/ming_model.zig:1264-1308): p [F][n_fft+2]
 * f32 -> wave [F*hop] f32 (n_fft = 4 hop).  frames (optional) [F][n_fft]. */
void or_vae_istft(const float* p, int F, int n_fft, int hop, const float* win, float* wave, float* frames_out) {
    const int nb = n_fft / 2 + 1, N = n_fft;
    float* fr = malloc(sizeof(float) * (size_t)F * N);
    /* twiddles by (k n) mod N, in double */
    double* cs = malloc(sizeof(double) * (size_t)N);
    double* sn = malloc(sizeof(double) * (size_t)N);
    for (int i = 0; i < N; i++) {
        cs[i] = cos(2.0 * M_PI * (double)i / (double)N);
        sn[i] = sin(2.0 * M_PI * (double)i / (double)N);
    }
#pragma omp parallel for schedule(static)
    for (int f = 0; f < F; f++) {
        const float* pr = p + (int64_t)f * (N + 2);
        double* re = malloc(sizeof(double) * (size_t)nb);
        double* im = malloc(sizeof(double) * (size_t)nb);
        for (int k = 0; k < nb; k++) {
            float mag = expf(pr[k]);
            mag = mag < 100.0f ? mag : 100.0f;
            const float ph = pr[nb + k];
            re[k] = (double)(mag * cosf(ph));
            im[k] = (double)(mag * sinf(ph));
        }
        for (int n = 0; n < N; n++) {
            /* irfft, backward norm: the imaginary parts of bins 0 and N/2 are ignored */
            double acc = re[0] + ((n & 1) ? -re[N / 2] : re[N / 2]);
            for (int k = 1; k < N / 2; k++) {
                const int64_t t = ((int64_t)k * n) % N;
                acc += 2.0 * (re[k] * cs[t] - im[k] * sn[t]);
            }
            fr[(int64_t)f * N + n] = (float)(acc / (double)N) * win[n];
        }
        free(re);
        free(im);
    }
    /* overlap-add: block b sums ((frame b-3 part 3 + frame b-2 part 2) + frame b-1 part 1) + frame b part 0 */
    const int total = (F + 3) * hop, pad = (N - hop) / 2, n_out = total - 2 * pad;
    for (int i = 0; i < n_out; i++) {
        const int s = pad + i, b = s / hop, kk = s % hop;
        float acc = 0.0f, env = 0.0f;
        for (int j = 3; j >= 0; j--) {
            const int t = b - j;
            const float fv = (t >= 0 && t < F) ? fr[(int64_t)t * N + j * hop + kk] : 0.0f;
            const float w2 = (t >= 0 && t < F) ? win[j * hop + kk] * win[j * hop + kk] : 0.0f;
            acc = j == 3 ? fv : acc + fv;
            env = env + w2;
        }
        wave[i] = acc / (env > 1e-11f ? env : 1e-11f);
    }
    if (frames_out) memcpy(frames_out, fr, sizeof(float) * (size_t)F * N);
    free(fr);
    free(cs);
    free(sn);
}

/* Model.vaeDecode: latents bf16 [T][latent] -> wave f32 [T * patch * hop]. */
void or_vae_decode(const or_vae_model* m, const uint16_t* latents, int T, float* wave, float* xs, float* head_out) {
    const or_vae_cfg* c = &m->cfg;
    const int H = c->hidden, F = T * c->patch;
    uint16_t* x0 = malloc(sizeof(uint16_t) * (size_t)T * H);
    or_linear_fwd(&m->fc1, latents, T, m->fc1_bias, x0);
    float* x = malloc(sizeof(float) * (size_t)F * H);
    float* y = malloc(sizeof(float) * (size_t)F * H);
    or_linear_upsample(x0, T, H, c->patch, x);
    if (xs) memcpy(xs, x, sizeof(float) * (size_t)F * H);
    for (int li = 0; li < c->n_layers; li++) {
        or_vae_layer(c, &m->layers[li], x, F, y, NULL);
        float* t = x;
        x = y;
        y = t;
        if (xs) memcpy(xs + (int64_t)(li + 1) * F * H, x, sizeof(float) * (size_t)F * H);
    }
    or_rms_f32(x, m->norm, F, H, c->eps, y);
    const int P = c->n_fft + 2;
    float* p = malloc(sizeof(float) * (size_t)F * P);
    or_linear_f32(&m->head, y, F, m->head_bias, p);
    if (head_out) memcpy(head_out, p, sizeof(float) * (size_t)F * P);
    or_vae_istft(p, F, c->n_fft, c->hop, m->window_fn, wave, NULL);
    free(x0);
    free(x);
    free(y);
    free(p);
}
