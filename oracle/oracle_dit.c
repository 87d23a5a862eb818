/*
 * oracle_dit.c -- CPU restatement of the DiT flow head (CFM) and the
 * aggregator, MLX graph semantics (TEST INFRASTRUCTURE ONLY; see oracle.h).
 *
 *   DiT block graph ..... src/ming_model.zig:783-795 (rms, q/k/v addmm, Rotary,
 *                         sdpa scale 1/8, out, rms, gelu_approx, ff2)
 *   Rotary .............. src/ming_model.zig:681-721 (x_transformers interleaved pairs)
 *   ditCfgEmb ........... src/ming_model.zig:1078-1091
 *   cfmSampleRaw ........ src/ming_model.zig:1161-1188 (Euler + CFG, SDE when shift != 0)
 *   flowSchedule ........ src/ming_model.zig:1207-1215
 *   timestepEmbed ....... src/ming_model.zig:1064-1076, t_freq :976-983
 *   aggregateRaw ........ src/ming_model.zig:1042-1053
 *   stopProb ............ src/ming_model.zig:1033-1038
 *
 * Every op of the MLX graph that produces a bf16 array rounds here (or_rb);
 * scalars the graph creates in the array's dtype (g.scalar(v, dt)) are bf16.
 */
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "oracle.h"

static float sum8(const float* p) { return ((p[0] + p[1]) + (p[2] + p[3])) + ((p[4] + p[5]) + (p[6] + p[7])); }

/* Rotary.table (:688-696): pos = arange(L) in inv_freq's dtype (f32), outer product, cos/sin in f32. */
void or_rotary_table(const float* inv_freq, int half, int L, float* cos_t, float* sin_t) {
    for (int l = 0; l < L; l++)
        for (int i = 0; i < half; i++) {
            const float f = (float)l * inv_freq[i];
            cos_t[l * half + i] = cosf(f);
            sin_t[l * half + i] = sinf(f);
        }
}

/* Rotary.apply (:706-720): xe = x[..., 0::2], xo = x[..., 1::2];
 * oe = xe*c - xo*s, oo = xe*s + xo*c (bf16 x f32 -> f32), interleaved, astype bf16. */
void or_rotary(uint16_t* x, int R, int L, int heads, int hd, const float* cos_t, const float* sin_t) {
    const int half = hd / 2;
    for (int r = 0; r < R; r++) {
        const int l = r % L;
        for (int h = 0; h < heads; h++) {
            uint16_t* v = x + ((int64_t)r * heads + h) * hd;
            for (int i = 0; i < half; i++) {
                const float c = cos_t[l * half + i], s = sin_t[l * half + i];
                const float xe = or_f32(v[2 * i]), xo = or_f32(v[2 * i + 1]);
                const float a = xe * c, b = xo * s, e = xe * s, f = xo * c;
                v[2 * i] = or_bf16(a - b);
                v[2 * i + 1] = or_bf16(e + f);
            }
        }
    }
}

/* sdpa over the L positions of each of the B sequences (no mask, L <= 8):
 * f32 scores with the scale on q, f32 softmax, output rounded once. */
static void sdpa_small(const uint16_t* q, const uint16_t* k, const uint16_t* v, int B, int L, int heads, int hd,
                       float scale, uint16_t* out) {
    const int D = heads * hd;
    for (int b = 0; b < B; b++)
        for (int h = 0; h < heads; h++)
            for (int i = 0; i < L; i++) {
                const uint16_t* qr = q + ((int64_t)(b * L + i)) * D + h * hd;
                float sc[8], m = -INFINITY;
                for (int j = 0; j < L; j++) {
                    const uint16_t* kr = k + ((int64_t)(b * L + j)) * D + h * hd;
                    float p[8] = {0};
                    for (int d = 0; d < hd; d++) p[d % 8] += (scale * or_f32(qr[d])) * or_f32(kr[d]);
                    sc[j] = sum8(p);
                    m = fmaxf(m, sc[j]);
                }
                float l = 0.0f;
                for (int j = 0; j < L; j++) {
                    sc[j] = expf(sc[j] - m);
                    l += sc[j];
                }
                for (int d = 0; d < hd; d++) {
                    float a = 0.0f;
                    for (int j = 0; j < L; j++) a += sc[j] * or_f32(v[((int64_t)(b * L + j)) * D + h * hd + d]);
                    out[((int64_t)(b * L + i)) * D + h * hd + d] = or_bf16(a / l);
                }
            }
}

/* adaLN modulation of rows h [R][D] in place: half = r / L selects mod + half * 6D;
 * h = bf16(bf16(h * bf16(1 + scale)) + shift), each op a materialised bf16 array. */
static void modulate(uint16_t* h, int R, int L, int D, const uint16_t* mod, int mstride, int soff, int coff) {
    for (int r = 0; r < R; r++) {
        const uint16_t* sh = mod + (size_t)(r / L) * mstride + (size_t)soff * D;
        const uint16_t* sc = mod + (size_t)(r / L) * mstride + (size_t)coff * D;
        for (int i = 0; i < D; i++) {
            const float t1 = or_rb(1.0f + or_f32(sc[i]));
            const float v = or_rb(or_f32(h[(size_t)r * D + i]) * t1);
            h[(size_t)r * D + i] = or_bf16(v + or_f32(sh[i]));
        }
    }
}

/* Gated residual: out = bf16(x + bf16(gate * a)), gate from the row's half. */
static void gated_add(const uint16_t* x, const uint16_t* a, int R, int L, int D, const uint16_t* mod, int mstride,
                      int goff, uint16_t* out) {
    for (int r = 0; r < R; r++) {
        const uint16_t* g = mod + (size_t)(r / L) * mstride + (size_t)goff * D;
        for (int i = 0; i < D; i++) {
            const size_t k = (size_t)r * D + i;
            out[k] = or_bf16(or_f32(x[k]) + or_rb(or_f32(g[i]) * or_f32(a[k])));
        }
    }
}

/* One block; mod (optional) [B][6D] = per half [shift_a, scale_a, gate_a, shift_m, scale_m, gate_m]. */
static void block_fwd(const or_dit_cfg* c, const or_dit_block* b, const uint16_t* mod, const uint16_t* x, int B,
                      int L, const float* cos_t, const float* sin_t, uint16_t* out, or_dit_trace* tr) {
    const int R = B * L, D = c->D, F = c->ff;
    uint16_t* h = malloc(sizeof(uint16_t) * (size_t)R * D);
    uint16_t* qkv = malloc(sizeof(uint16_t) * (size_t)3 * R * D);
    uint16_t* att = malloc(sizeof(uint16_t) * (size_t)R * D);
    uint16_t* t1 = malloc(sizeof(uint16_t) * (size_t)R * D);
    uint16_t* x1 = malloc(sizeof(uint16_t) * (size_t)R * D);
    uint16_t* f1 = malloc(sizeof(uint16_t) * (size_t)R * F);
    uint16_t* hh = malloc(sizeof(uint16_t) * (size_t)R * F);
    or_rms_norm(x, b->norm1, R, D, c->eps, h);
    if (mod) modulate(h, R, L, D, mod, 6 * D, 0, 1);
    or_linear_fwd(&b->q, h, R, b->bq, qkv);
    or_linear_fwd(&b->k, h, R, b->bk, qkv + (size_t)R * D);
    or_linear_fwd(&b->v, h, R, b->bv, qkv + (size_t)2 * R * D);
    or_rotary(qkv, R, L, c->heads, c->head_dim, cos_t, sin_t);
    or_rotary(qkv + (size_t)R * D, R, L, c->heads, c->head_dim, cos_t, sin_t);
    sdpa_small(qkv, qkv + (size_t)R * D, qkv + (size_t)2 * R * D, B, L, c->heads, c->head_dim, 1.0f / 8.0f, att);
    or_linear_fwd(&b->o, att, R, b->bo, t1);
    if (mod)
        gated_add(x, t1, R, L, D, mod, 6 * D, 2, x1);
    else
        or_add(x, t1, (int64_t)R * D, x1);
    or_rms_norm(x1, b->norm2, R, D, c->eps, h);
    if (mod) modulate(h, R, L, D, mod, 6 * D, 3, 4);
    or_linear_fwd(&b->ff1, h, R, b->b1, f1);
    or_gelu_approx(f1, (int64_t)R * F, hh);
    or_linear_fwd(&b->ff2, hh, R, b->b2, t1);
    if (mod)
        gated_add(x1, t1, R, L, D, mod, 6 * D, 5, out);
    else
        or_add(x1, t1, (int64_t)R * D, out);
    if (tr) {
        if (tr->qkv) memcpy(tr->qkv, qkv, sizeof(uint16_t) * (size_t)3 * R * D);
        if (tr->att) memcpy(tr->att, att, sizeof(uint16_t) * (size_t)R * D);
        if (tr->x1) memcpy(tr->x1, x1, sizeof(uint16_t) * (size_t)R * D);
        if (tr->hh) memcpy(tr->hh, hh, sizeof(uint16_t) * (size_t)R * F);
    }
    free(h);
    free(qkv);
    free(att);
    free(t1);
    free(x1);
    free(f1);
    free(hh);
}

void or_dit_block_fwd(const or_dit_cfg* c, const or_dit_block* b, const uint16_t* x, int B, int L,
                      const float* cos_t, const float* sin_t, uint16_t* out, or_dit_trace* tr) {
    block_fwd(c, b, NULL, x, B, L, cos_t, sin_t, out, tr);
}

void or_adaln_block_fwd(const or_dit_cfg* c, const or_dit_block* b, const uint16_t* mod, const uint16_t* x, int B,
                        int L, const float* cos_t, const float* sin_t, uint16_t* out, or_dit_trace* tr) {
    block_fwd(c, b, mod, x, B, L, cos_t, sin_t, out, tr);
}

/* flowSchedule (:1207-1215) in bf16: t = (1/32) * sched; t = t + (-1) * (cos(pi/2 * t) - 1 + t). */
void or_flow_schedule(uint16_t* t) {
    static const float sched[11] = {0, 2, 4, 6, 8, 12, 16, 20, 24, 28, 32};
    const float c32 = or_rb(1.0f / 32.0f), hpi = or_rb((float)(3.14159265358979323846 / 2.0)), one = 1.0f, m1 = -1.0f;
    for (int i = 0; i < 11; i++) {
        const float ti = or_rb(c32 * or_rb(sched[i]));
        const float ct = or_rb(cosf(or_rb(hpi * ti)));
        const float sw = or_rb(or_rb(ct - one) + ti);
        t[i] = or_bf16(ti + or_rb(m1 * sw));
    }
}

/* flow_dt = t[1:] - t[:-1], flow_sq = |flow_dt| ** 0.5 (Model.load, bf16). */
void or_flow_steps(const uint16_t* t, uint16_t* dt, uint16_t* sq) {
    for (int i = 0; i < 10; i++) {
        const float d = or_rb(or_f32(t[i + 1]) - or_f32(t[i]));
        dt[i] = or_bf16(d);
        sq[i] = or_bf16(powf(fabsf(d), or_rb(0.5f)));
    }
}

/* t_freq = exp(arange(128) * -(ln(1e4)/127)), f32 (Model.load). */
void or_t_freq(float* f) {
    const float e = (float)(log(10000.0) / 127.0);
    for (int k = 0; k < 128; k++) f[k] = expf((float)k * -e);
}

/* timestepEmbed (:1064-1076): ts = bf16(1000 * t); emb = f32(ts) * t_freq (f32);
 * [sin | cos] -> bf16 -> t_mlp0 (addmm) -> silu (compiled) -> t_mlp2 (addmm). */
void or_timestep_embed(const or_linear* mlp0, const uint16_t* b0, const or_linear* mlp2, const uint16_t* b2,
                       const float* t_freq, uint16_t t, uint16_t* out) {
    const float ts = or_rb(or_rb(1000.0f) * or_f32(t));
    uint16_t sc[2 * 256];
    for (int r = 0; r < 2; r++)
        for (int k = 0; k < 128; k++) {
            const float e = ts * t_freq[k];
            sc[r * 256 + k] = or_bf16(sinf(e));
            sc[r * 256 + 128 + k] = or_bf16(cosf(e));
        }
    const int64_t D = mlp0->N;
    uint16_t* te = malloc(sizeof(uint16_t) * 2 * D);
    or_linear_fwd(mlp0, sc, 2, b0, te);
    for (int64_t i = 0; i < 2 * D; i++) {  /* silu: x * sigmoid(x), each op rounded */
        const float v = or_f32(te[i]);
        const float sg = or_rb(1.0f / (1.0f + expf(-v)));
        te[i] = or_bf16(v * sg);
    }
    or_linear_fwd(mlp2, te, 2, b2, out);
    free(te);
}

/* ditCfgEmb rows (:1078-1091): x_now = x_emb([y, y]), x_hist = x_emb([hist, hist]),
 * c_embed = c_emb([z, 0]), y0 = t_emb + c_embed; rows [y0, x_hist, x_now] per half. */
void or_cfm_rows(const or_cfm_model* m, const uint16_t* z, const uint16_t* hist, const uint16_t* y, int step,
                 uint16_t* rows) {
    const int D = m->c.D;
    const int64_t H = m->c_emb.K;
    uint16_t* xn = malloc(sizeof(uint16_t) * D);
    uint16_t* xh = malloc(sizeof(uint16_t) * D);
    uint16_t* ce = malloc(sizeof(uint16_t) * 2 * D);
    uint16_t* zc = calloc((size_t)2 * H, sizeof(uint16_t));
    memcpy(zc, z, sizeof(uint16_t) * H);  /* [z, zeros] */
    or_linear_fwd(&m->x_emb, y, 1, m->bx, xn);
    or_linear_fwd(&m->x_emb, hist, 1, m->bx, xh);
    or_linear_fwd(&m->c_emb, zc, 2, m->bc, ce);
    const uint16_t* te = m->t_emb + (size_t)step * 2 * D;
    for (int b = 0; b < 2; b++) {
        or_add(te + (size_t)b * D, ce + (size_t)b * D, D, rows + (size_t)(b * 3 + 0) * D);
        memcpy(rows + (size_t)(b * 3 + 1) * D, xh, sizeof(uint16_t) * D);
        memcpy(rows + (size_t)(b * 3 + 2) * D, xn, sizeof(uint16_t) * D);
    }
    free(xn);
    free(xh);
    free(ce);
    free(zc);
}

/* dit_final(rms(h)) on the last row of each half, then (:1172-1186):
 * f0 = pc + (pc - pu) * cfg; y = y + dt * f0; y += (shift_k * sq) * sde when shift_k != 0. */
void or_cfm_final(const or_cfm_model* m, const uint16_t* h, int L, const uint16_t* y, const uint16_t* sde, int step,
                  float cfg, float shift_k, uint16_t* y_out) {
    const int D = m->c.D;
    const int64_t n = m->final.N;
    uint16_t hn[2 * 4096];
    uint16_t last[2 * 4096];
    memcpy(last, h + (size_t)(L - 1) * D, sizeof(uint16_t) * D);
    memcpy(last + D, h + (size_t)(2 * L - 1) * D, sizeof(uint16_t) * D);
    or_rms_norm(last, m->final_norm, 2, D, m->c.eps, hn);
    uint16_t* o = malloc(sizeof(uint16_t) * 2 * n);
    or_linear_fwd(&m->final, hn, 2, m->bf, o);
    const float cf = or_rb(cfg), dt = or_f32(m->dt[step]), sq = or_f32(m->sq[step]), sk = or_rb(shift_k);
    for (int64_t i = 0; i < n; i++) {
        const float pc = or_f32(o[i]), pu = or_f32(o[n + i]);
        const float f0 = or_rb(pc + or_rb(or_rb(pc - pu) * cf));
        float v = or_rb(or_f32(y[i]) + or_rb(dt * f0));
        if (shift_k != 0.0f) v = or_rb(v + or_rb(or_rb(sk * sq) * or_f32(sde[(size_t)step * n + i])));
        y_out[i] = or_bf16(v);
    }
    free(o);
}

void or_cfm_sample(const or_cfm_model* m, const uint16_t* z, const uint16_t* hist, const uint16_t* noise,
                   const uint16_t* sde, float cfg, float shift_k, uint16_t* out, uint16_t* y_steps) {
    const int D = m->c.D, L = 3;
    const int64_t n = m->final.N;
    uint16_t* y = malloc(sizeof(uint16_t) * n);
    uint16_t* a = malloc(sizeof(uint16_t) * 2 * L * D);
    uint16_t* b2 = malloc(sizeof(uint16_t) * 2 * L * D);
    memcpy(y, noise, sizeof(uint16_t) * n);
    for (int i = 0; i < m->steps; i++) {
        or_cfm_rows(m, z, hist, y, i, a);
        for (int k = 0; k < m->n_blocks; k++) {
            or_dit_block_fwd(&m->c, &m->blocks[k], a, 2, L, m->cos_t, m->sin_t, b2, NULL);
            uint16_t* t = a;
            a = b2;
            b2 = t;
        }
        or_cfm_final(m, a, L, y, sde, i, cfg, shift_k, y);
        if (y_steps) memcpy(y_steps + (size_t)i * n, y, sizeof(uint16_t) * n);
    }
    memcpy(out, y, sizeof(uint16_t) * n);
    free(y);
    free(a);
    free(b2);
}

/* aggregateRaw (:1042-1053): x = x_emb(latent); h = [cls, x]; 8 blocks (L = 2);
 * final(rms(h)) -> row 0. */
void or_aggregate(const or_agg_model* m, const uint16_t* latent, uint16_t* out) {
    const int D = m->c.D;
    uint16_t* a = malloc(sizeof(uint16_t) * 2 * D);
    uint16_t* b2 = malloc(sizeof(uint16_t) * 2 * D);
    memcpy(a, m->cls, sizeof(uint16_t) * D);
    or_linear_fwd(&m->x_emb, latent, 1, m->bx, a + D);
    for (int k = 0; k < m->n_blocks; k++) {
        or_dit_block_fwd(&m->c, &m->blocks[k], a, 1, 2, m->cos_t, m->sin_t, b2, NULL);
        uint16_t* t = a;
        a = b2;
        b2 = t;
    }
    uint16_t* hn = malloc(sizeof(uint16_t) * D);
    or_rms_norm(a, m->final_norm, 1, D, m->c.eps, hn);  /* row 0 only: rms and the linear are per row */
    or_linear_fwd(&m->final, hn, 1, m->bf, out);
    free(hn);
    free(a);
    free(b2);
}

/* stopProb (:1033-1038): softmax(f32(stop_head(z)))[1]. */
float or_stop_prob(const or_linear* head, const uint16_t* bias, const uint16_t* z) {
    uint16_t lg[2];
    or_linear_fwd(head, z, 1, bias, lg);
    const float l0 = or_f32(lg[0]), l1 = or_f32(lg[1]);
    const float mx = fmaxf(l0, l1);
    const float e0 = expf(l0 - mx), e1 = expf(l1 - mx);
    return e1 / (e0 + e1);
}

/* ---- adaLN flow head (config 4; the build's definition, see oracle.h) ---------------- */

static void silu_rows(const uint16_t* c, int64_t n, uint16_t* out) {
    for (int64_t i = 0; i < n; i++) {  /* silu: x * sigmoid(x), each op rounded (as the timestep MLP) */
        const float v = or_f32(c[i]);
        const float sg = or_rb(1.0f / (1.0f + expf(-v)));
        out[i] = or_bf16(v * sg);
    }
}

void or_adaln_cond(const or_adaln_model* m, const uint16_t* z, uint16_t* silu_c) {
    const int D = m->c.D;
    const int64_t H = m->c_emb.K;
    uint16_t* zc = calloc((size_t)2 * H, sizeof(uint16_t));
    uint16_t* ce = malloc(sizeof(uint16_t) * 2 * D);
    uint16_t* cc = malloc(sizeof(uint16_t) * 2 * D);
    memcpy(zc, z, sizeof(uint16_t) * H);  /* [z, zeros] */
    or_linear_fwd(&m->c_emb, zc, 2, m->bc, ce);
    for (int s = 0; s < m->steps; s++) {
        or_add(m->t_emb + (size_t)s * 2 * D, ce, 2 * D, cc);
        silu_rows(cc, 2 * D, silu_c + (size_t)s * 2 * D);
    }
    free(zc);
    free(ce);
    free(cc);
}

void or_adaln_mods(const or_adaln_model* m, const uint16_t* silu_c, uint16_t* mods, uint16_t* modf) {
    const int D = m->c.D, rows = 2 * m->steps;
    for (int k = 0; k < m->n_blocks; k++)
        or_linear_fwd(&m->blocks[k].ada, silu_c, rows, m->blocks[k].bada, mods + (size_t)k * rows * 6 * D);
    or_linear_fwd(&m->final_ada, silu_c, rows, m->bfa, modf);
}

void or_adaln_rows(const or_adaln_model* m, const uint16_t* y, uint16_t* rows) {
    const int D = m->c.D, F = m->frames;
    or_linear_fwd(&m->x_emb, y, F, m->bx, rows);
    memcpy(rows + (size_t)F * D, rows, sizeof(uint16_t) * (size_t)F * D);
}

void or_adaln_final(const or_adaln_model* m, const uint16_t* h, const uint16_t* modf_step, const uint16_t* y,
                    const uint16_t* sde, int step, float cfg, float shift_k, uint16_t* y_out) {
    const int D = m->c.D, F = m->frames, R = 2 * F;
    const int64_t n = m->final.N;
    uint16_t* hn = malloc(sizeof(uint16_t) * (size_t)R * D);
    uint16_t* o = malloc(sizeof(uint16_t) * (size_t)R * n);
    or_rms_norm(h, m->final_norm, R, D, m->c.eps, hn);
    modulate(hn, R, F, D, modf_step, 2 * D, 0, 1);
    or_linear_fwd(&m->final, hn, R, m->bf, o);
    const float cf = or_rb(cfg), dt = or_f32(m->dt[step]), sq = or_f32(m->sq[step]), sk = or_rb(shift_k);
    for (int f = 0; f < F; f++)
        for (int64_t i = 0; i < n; i++) {
            const float pc = or_f32(o[(size_t)f * n + i]), pu = or_f32(o[(size_t)(F + f) * n + i]);
            const float f0 = or_rb(pc + or_rb(or_rb(pc - pu) * cf));
            float v = or_rb(or_f32(y[(size_t)f * n + i]) + or_rb(dt * f0));
            if (shift_k != 0.0f)
                v = or_rb(v + or_rb(or_rb(sk * sq) * or_f32(sde[((size_t)step * F + f) * n + i])));
            y_out[(size_t)f * n + i] = or_bf16(v);
        }
    free(hn);
    free(o);
}

void or_adaln_sample(const or_adaln_model* m, const uint16_t* z, const uint16_t* noise, const uint16_t* sde,
                     float cfg, float shift_k, uint16_t* out, uint16_t* y_steps) {
    const int D = m->c.D, F = m->frames, R = 2 * F, rows = 2 * m->steps;
    const int64_t n = (int64_t)F * m->final.N;
    uint16_t* silu_c = malloc(sizeof(uint16_t) * (size_t)rows * D);
    uint16_t* mods = malloc(sizeof(uint16_t) * (size_t)m->n_blocks * rows * 6 * D);
    uint16_t* modf = malloc(sizeof(uint16_t) * (size_t)rows * 2 * D);
    uint16_t* y = malloc(sizeof(uint16_t) * n);
    uint16_t* a = malloc(sizeof(uint16_t) * (size_t)R * D);
    uint16_t* b2 = malloc(sizeof(uint16_t) * (size_t)R * D);
    or_adaln_cond(m, z, silu_c);
    or_adaln_mods(m, silu_c, mods, modf);
    memcpy(y, noise, sizeof(uint16_t) * n);
    for (int i = 0; i < m->steps; i++) {
        or_adaln_rows(m, y, a);
        for (int k = 0; k < m->n_blocks; k++) {
            const uint16_t* mk = mods + ((size_t)k * rows + 2 * i) * 6 * D;
            or_adaln_block_fwd(&m->c, &m->blocks[k].blk, mk, a, 2, F, m->cos_t, m->sin_t, b2, NULL);
            uint16_t* t = a;
            a = b2;
            b2 = t;
        }
        or_adaln_final(m, a, modf + (size_t)2 * i * 2 * D, y, sde, i, cfg, shift_k, y);
        if (y_steps) memcpy(y_steps + (size_t)i * n, y, sizeof(uint16_t) * n);
    }
    memcpy(out, y, sizeof(uint16_t) * n);
    free(silu_c);
    free(mods);
    free(modf);
    free(y);
    free(a);
    free(b2);
}
