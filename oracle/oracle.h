/*
 * oracle.h -- CPU restatement of Ming-3.0-tts's per-token generation loop.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product library links, loads or
 * calls this code.  It is the checker for the HIP path (tests/, the smoke
 * entry and the cpu_baseline leg of bench.py) and nothing else.
 *
 * It restates the MLX graph path of the reference (MING_FUSED=0 semantics):
 * bf16 storage, f32 accumulation, and a bf16 rounding at every point where
 * MLX materialises a bf16 array.  Citations are to the reference tree
 * (sbusso/ming-tts-serve).
 *
 *   LM layer graph ............ src/ming_model.zig:588-611
 *   decode gate / final norm .. src/ming_model.zig:530-544, :566-575
 *   rounding points ........... src/ming_fused.zig:17-25
 *   swiglu / gelu op order .... src/ming_model.zig:800-862
 *   DiT block graph ........... src/ming_model.zig:783-795
 *   CFM / CFG / Euler ......... src/ming_model.zig:1161-1188, :1193-1203
 *   flow schedule ............. src/ming_model.zig:1207-1215
 *   aggregator ................ src/ming_model.zig:1042-1053
 *   stop head ................. src/ming_model.zig:1033-1038
 *
 * The MLX-affine quantizer, dequantizer and quantized matmul restate the
 * published MLX 0.32 CPU algorithm (mlx/backend/cpu/quantized.cpp), which the
 * reference binds at src/mlx.zig:279-292 but never calls.
 *
 * Where each function is pinned (closed forms, library routines, brute force)
 * is stated in the test that checks it (tests/test_oracle_*.py).
 */
#ifndef MING_ORACLE_H
#define MING_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- bf16 ---------------------------------------------------------------- */
uint16_t or_bf16(float f);             /* f32 -> bf16, round to nearest even */
float or_f32(uint16_t h);              /* bf16 -> f32 (exact) */
float or_rb(float f);                  /* round through bf16 */
void or_to_bf16(const float* x, uint16_t* y, int64_t n);
void or_to_f32(const uint16_t* x, float* y, int64_t n);

/* ---- MLX affine quantization (mode "affine", transpose=true layout) ------ */
/* w bf16 [N,K] -> wq u32 [N, K*bits/32], scales/biases bf16 [N, K/group];
 * each group quantized as w / gscale (gscale > 0; 1 = plain MLX affine). */
int or_quantize(const uint16_t* w, int64_t N, int64_t K, int group, int bits, float gscale,
                uint32_t* wq, uint16_t* scales, uint16_t* biases);
/* -> bf16 [N,K]: bf16(gscale * (s*q + b)) */
int or_dequantize(const uint32_t* wq, const uint16_t* scales, const uint16_t* biases,
                  int64_t N, int64_t K, int group, int bits, float gscale, uint16_t* out);

/* ---- linear layers -------------------------------------------------------- */
enum { OR_W_BF16 = 0, OR_W_AFFINE = 1 };
typedef struct {
    int kind;                 /* OR_W_BF16 or OR_W_AFFINE */
    int64_t N, K;             /* out_features, in_features */
    const void* w;            /* bf16 [N,K] or u32 [N,K*bits/32] */
    const uint16_t* scales;   /* bf16 [N,K/group] (affine) */
    const uint16_t* biases;   /* bf16 [N,K/group] (affine) */
    float gscale;             /* global scale (affine); 1.0 = plain MLX affine */
    int group, bits;
} or_linear;

/* y[n] = f32 accumulation of W x (no rounding). rows x[M][K] -> y[M][N]. */
void or_linear_acc(const or_linear* L, const uint16_t* x, int64_t M, float* y);
/* MLX linear output: bf16 [M,N].
 *   bf16 weights:  addmm  -> bf16(acc + bias)                (one rounding)
 *   affine weights: quantized_matmul then + bias -> bf16(bf16(acc) + bias)  */
void or_linear_fwd(const or_linear* L, const uint16_t* x, int64_t M, const uint16_t* bias, uint16_t* y);

/* ---- element-wise / normalisation ---------------------------------------- */
/* MLX fast::rms_norm: out = bf16(w * bf16(x * rsqrt(mean(x^2) + eps))), rows [M][n]. */
void or_rms_norm(const uint16_t* x, const uint16_t* w, int64_t M, int64_t n, float eps, uint16_t* out);
/* MLX fast::rope, traditional=false: pairs (d, d + hd/2); x [nh][hd] bf16 in place. */
void or_rope(uint16_t* x, int nh, int hd, int pos, float log2_base);
/* compiled swiglu: bf16(bf16(g * bf16(sigmoid(g))) * u) */
void or_swiglu(const uint16_t* g, const uint16_t* u, int64_t n, uint16_t* out);
/* compiled mlx.nn.gelu_approx with bf16 weak scalars, every op rounded */
void or_gelu_approx(const uint16_t* x, int64_t n, uint16_t* out);
/* bf16 add */
void or_add(const uint16_t* a, const uint16_t* b, int64_t n, uint16_t* out);

/* ---- Qwen2 decode --------------------------------------------------------- */
typedef struct {
    int hidden, heads, kv_heads, head_dim, inter;
    float eps, log2_theta;
} or_lm_cfg;

typedef struct {
    const uint16_t *ln1, *ln2;
    or_linear q, k, v, o, gate, up, down;
    const uint16_t *bq, *bk, *bv;
} or_lm_layer;

/* Intermediates of one layer (all optional, bf16 unless noted). */
typedef struct {
    uint16_t* h;    /* rms(x, ln1)        [hidden] */
    uint16_t* qkv;  /* roped q | roped k | v  [hidden + 2*kv_heads*head_dim] */
    uint16_t* att;  /* attention output   [hidden] */
    uint16_t* x1;   /* x + o_proj         [hidden] */
    uint16_t* hh;   /* swiglu             [inter] */
} or_lm_trace;

/* GQA decode attention of one token at position `pos` over the cache rows
 * [0, pos] (the new row already appended).  q [heads][hd] bf16;
 * kc/vc [kv_heads][cap][hd] bf16; out [heads][hd] bf16. */
void or_attention(const uint16_t* q, const uint16_t* kc, const uint16_t* vc, int heads, int kv_heads,
                  int hd, int cap, int pos, float scale, uint16_t* out);

/* One Qwen2 layer on x [hidden] at position pos.  k/v are appended in place
 * at row pos of kc/vc ([kv_heads][cap][hd]).  x_out [hidden]. */
void or_lm_layer_step(const or_lm_cfg* c, const or_lm_layer* l, const uint16_t* x, int pos,
                      uint16_t* kc, uint16_t* vc, int cap, uint16_t* x_out, or_lm_trace* tr);

/* Final norm + tied LM head + greedy argmax.  hidden_out bf16 [hidden];
 * logits f32 [vocab] (accumulator before rounding; may be NULL);
 * returns the argmax over the f32 logits, lowest index on ties. */
int or_lm_head(const or_lm_cfg* c, const uint16_t* norm, const or_linear* head, const uint16_t* x,
               uint16_t* hidden_out, float* logits, uint16_t* logits_bf16, float* margin);

/* Embedding row gather: bf16 table [V,H] or affine-quantized table. */
void or_embed(const or_linear* table, int id, uint16_t* out);

/* ---- DiT flow head and aggregator ------------------------------------------ */
typedef struct {
    int D, heads, head_dim, ff;   /* 1024, 16, 64, 4096 in the reference */
    float eps;                    /* rms_norm eps, 1e-6 */
} or_dit_cfg;

/* One DiT block: bf16 [out,in] linears with biases (addmm), two RMSNorms. */
typedef struct {
    const uint16_t *norm1, *norm2;
    or_linear q, k, v, o, ff1, ff2;
    const uint16_t *bq, *bk, *bv, *bo, *b1, *b2;
} or_dit_block;

/* Intermediates of one block (optional). */
typedef struct {
    uint16_t* qkv;  /* [3][R][D]: rotated q, rotated k, v */
    uint16_t* att;  /* [R][D] attention output */
    uint16_t* x1;   /* [R][D] x + out(att) */
    uint16_t* hh;   /* [R][ff] gelu_approx(ff1(rms(x1))) */
} or_dit_trace;

/* Summation order of every DiT function below (blocks, flow head, aggregator, stop head,
 * adaLN head): OR_DIT_ORDER_MLX (default) sums dot products over 8 interleaved f32 partials and
 * uses libm expf; OR_DIT_ORDER_DEVICE takes each f32 sum in the order and with the arithmetic of
 * the library's batch-1 DiT kernels (team lanes over 16-byte chunks, v_dot2c_f32_bf16 steps
 * restated by or_acc_step, the pairwise lane tree, wave sums in order) and e^x by or_exp_rep;
 * OR_DIT_ORDER_MFMA is the device order with the dot products of the batched flow head's matrix
 * core GEMM (or_dot_mfma).  Same graph and rounding points in every mode. */
enum { OR_DIT_ORDER_MLX = 0, OR_DIT_ORDER_DEVICE = 1, OR_DIT_ORDER_MFMA = 2 };
void or_set_dit_order(int mode);
int or_get_dit_order(void);
/* e^x from correctly rounded f32 steps (Cody-Waite reduction, degree-7 Taylor, 2^n scaling). */
float or_exp_rep(float x);
/* acc + sum_{i<n} a_i b_i (bf16, n <= 32) as one accumulation step of gfx950's v_dot2c_f32_bf16
 * (n = 2) or of one 8-k block of v_mfma_f32_16x16x32_bf16 (n = 8); other n for tests. */
float or_acc_step(float acc, const uint16_t* a, const uint16_t* b, int n);
/* Batches of or_acc_step: dot2 over u32 bf16 pairs; 16x16x32 matrix tiles (A [t][16][32],
 * B [t][32][16], C, D [t][16][16]). */
void or_dot2_batch(const uint32_t* a, const uint32_t* b, const float* c, float* d, int64_t n);
void or_mfma_batch(const uint16_t* A, const uint16_t* B, const float* C, float* D, int64_t ntests);
/* One dot product of bf16 w, x [K] in the device order with a team of T (32 or 64) lanes. */
float or_dot_dev(const uint16_t* w, const uint16_t* x, int64_t K, int T);
/* One dot product of bf16 w, x [K] in the batched (matrix core) order over vs K slices. */
float or_dot_mfma(const uint16_t* w, const uint16_t* x, int64_t K, int vs);
/* Sum of squares of x [K] (K <= 1024) in the device order. */
float or_sumsq_dev(const uint16_t* x, int64_t K);

/* x_transformers RotaryEmbedding table: cos/sin[l][i] = cos/sin(l * inv_freq[i]) in f32. */
void or_rotary_table(const float* inv_freq, int half, int L, float* cos_t, float* sin_t);
/* Interleaved-pair rotary (2i, 2i+1) of every head of the R = B*L rows of x [R][heads*hd]
 * (row r at position r % L): bf16 * f32 table products in f32, rounded once. */
void or_rotary(uint16_t* x, int R, int L, int heads, int hd, const float* cos_t, const float* sin_t);
/* One block on x [B*L][D] -> out [B*L][D]. */
void or_dit_block_fwd(const or_dit_cfg* c, const or_dit_block* b, const uint16_t* x, int B, int L,
                      const float* cos_t, const float* sin_t, uint16_t* out, or_dit_trace* tr);

/* EPSS + sway flow schedule, 11 bf16 values. */
void or_flow_schedule(uint16_t* t);
/* Step sizes dt[i] = t[i+1] - t[i] and sq[i] = |dt[i]|^0.5, bf16 [10] each. */
void or_flow_steps(const uint16_t* t, uint16_t* dt, uint16_t* sq);
/* Timestep sinusoid frequencies exp(-k ln(1e4)/127), f32 [128]. */
void or_t_freq(float* f);
/* TimestepEmbedder for scalar t (bf16): out [2][D] (both CFG rows equal). */
void or_timestep_embed(const or_linear* mlp0, const uint16_t* b0, const or_linear* mlp2, const uint16_t* b2,
                       const float* t_freq, uint16_t t, uint16_t* out);

typedef struct {
    or_dit_cfg c;
    int n_blocks;
    const or_dit_block* blocks;
    or_linear x_emb;                 /* latent (64) -> D */
    const uint16_t* bx;
    or_linear c_emb;                 /* LM hidden (896) -> D */
    const uint16_t* bc;
    const uint16_t* final_norm;      /* [D] */
    or_linear final;                 /* D -> latent */
    const uint16_t* bf;
    const uint16_t* t_emb;           /* [steps][2][D] */
    const uint16_t* dt;              /* [steps] */
    const uint16_t* sq;              /* [steps] */
    const float *cos_t, *sin_t;      /* rotary tables for L = 3 */
    int steps;
} or_cfm_model;

/* CFM.sample for one LM step: z [hidden], hist [latent], noise [latent],
 * sde [steps][latent] -> out [latent]; y_steps [steps][latent] (optional)
 * receives the latent after every Euler step. */
void or_cfm_sample(const or_cfm_model* m, const uint16_t* z, const uint16_t* hist, const uint16_t* noise,
                   const uint16_t* sde, float cfg, float shift_k, uint16_t* out, uint16_t* y_steps);
/* The 6 DiT input rows [t_emb+c_emb, x_emb(hist), x_emb(y)] x 2 CFG halves for step i. */
void or_cfm_rows(const or_cfm_model* m, const uint16_t* z, const uint16_t* hist, const uint16_t* y, int step,
                 uint16_t* rows);
/* Final norm + linear on the last row of each half, CFG combine and Euler
 * update for step i: h [2*L][D], y [latent] -> y_out [latent]. */
void or_cfm_final(const or_cfm_model* m, const uint16_t* h, int L, const uint16_t* y, const uint16_t* sde, int step,
                  float cfg, float shift_k, uint16_t* y_out);

typedef struct {
    or_dit_cfg c;
    int n_blocks;
    const or_dit_block* blocks;
    or_linear x_emb;                 /* latent -> D */
    const uint16_t* bx;
    const uint16_t* cls;             /* [D] */
    const uint16_t* final_norm;      /* [D] */
    or_linear final;                 /* D -> LM hidden */
    const uint16_t* bf;
    const float *cos_t, *sin_t;      /* rotary tables for L = 2 */
} or_agg_model;

/* Aggregator: latent [latent] -> next LM input row [final.N]. */
void or_aggregate(const or_agg_model* m, const uint16_t* latent, uint16_t* out);
/* softmax(f32(stop_head(z)))[1]. */
float or_stop_prob(const or_linear* head, const uint16_t* bias, const uint16_t* z);

/* ---- adaLN DiT flow head (config 4) -----------------------------------------
 * No reference implementation exists; this build defines it as the standard
 * adaLN-Zero DiT (Peebles & Xie) on the reference block's RMSNorm.  Per CFG half
 * b (uncond: z = 0) and Euler step s: c = bf16(t_emb[s] + c_emb(z)); silu(c)
 * with each op rounded; per block mod = bf16(addmm(b_ada, silu(c), W_ada^T)) =
 * [shift_a | scale_a | gate_a | shift_m | scale_m | gate_m] (6 x D);
 * modulate(n) = bf16(bf16(n * bf16(1 + scale)) + shift) on the rms_norm output;
 * x1 = bf16(x + bf16(gate_a * out_proj(...))), x2 likewise with gate_m.  The
 * sequence is the F patch frames x_emb(y_f) per half (rotary positions 0..F-1);
 * the final layer is modulate(rms(h)) with [shift | scale] = addmm(b_fa,
 * silu(c), W_fa^T), a linear to the latent, and CFG + Euler (+ SDE) per frame.
 * With shift = scale = 0 and gate = 1 a block is the reference block. */
void or_adaln_block_fwd(const or_dit_cfg* c, const or_dit_block* b, const uint16_t* mod, const uint16_t* x, int B,
                        int L, const float* cos_t, const float* sin_t, uint16_t* out, or_dit_trace* tr);

typedef struct {
    or_dit_block blk;
    or_linear ada;                   /* D -> 6D */
    const uint16_t* bada;
} or_adaln_block;

typedef struct {
    or_dit_cfg c;
    int n_blocks;
    const or_adaln_block* blocks;
    or_linear x_emb;                 /* latent -> D */
    const uint16_t* bx;
    or_linear c_emb;                 /* LM hidden -> D */
    const uint16_t* bc;
    const uint16_t* final_norm;      /* [D] */
    or_linear final;                 /* D -> latent */
    const uint16_t* bf;
    or_linear final_ada;             /* D -> 2D */
    const uint16_t* bfa;
    const uint16_t* t_emb;           /* [steps][2][D] */
    const uint16_t* dt;              /* [steps] */
    const uint16_t* sq;              /* [steps] */
    const float *cos_t, *sin_t;      /* rotary tables for L = frames */
    int steps, frames;
} or_adaln_model;

/* silu(c) rows [steps][2][D] for LM hidden z. */
void or_adaln_cond(const or_adaln_model* m, const uint16_t* z, uint16_t* silu_c);
/* Modulations of every step and half: mods [n_blocks][steps*2][6D], modf [steps*2][2D]. */
void or_adaln_mods(const or_adaln_model* m, const uint16_t* silu_c, uint16_t* mods, uint16_t* modf);
/* Input rows [2][F][D] = x_emb(y_f) for both halves; y [F][latent]. */
void or_adaln_rows(const or_adaln_model* m, const uint16_t* y, uint16_t* rows);
/* Final adaLN layer on h [2F][D] with modf_step [2][2D], CFG + Euler of step: y [F][latent] -> y_out. */
void or_adaln_final(const or_adaln_model* m, const uint16_t* h, const uint16_t* modf_step, const uint16_t* y,
                    const uint16_t* sde, int step, float cfg, float shift_k, uint16_t* y_out);
/* The whole sample: noise [F][latent], sde [steps][F][latent] -> out [F][latent]. */
void or_adaln_sample(const or_adaln_model* m, const uint16_t* z, const uint16_t* noise, const uint16_t* sde,
                     float cfg, float shift_k, uint16_t* out, uint16_t* y_steps);

/* ---- CPU threads ---------------------------------------------------------- */
void or_set_threads(int n);
int or_get_threads(void);

/* ---- VAE decoder (oracle_vae.c; src/ming_model.zig:1257-1340, :566-636) ---- */
typedef struct {
    int hidden, heads, kv_heads, head_dim, inter, n_layers;
    float eps, log2_theta;
    int window;                 /* sliding attention window (64) */
    int latent, patch;          /* latent width (64), upsample factor (4) */
    int n_fft, hop;             /* ISTFT (3528, 882; n_fft = 4 hop) */
} or_vae_cfg;

typedef struct {
    or_vae_cfg cfg;
    or_linear fc1;              /* [hidden, latent] */
    const uint16_t* fc1_bias;   /* bf16 [hidden] or NULL */
    const or_lm_layer* layers;  /* [n_layers]; q/k/v biases may be NULL */
    const uint16_t* norm;       /* bf16 [hidden] */
    or_linear head;             /* [n_fft + 2, hidden] */
    const uint16_t* head_bias;  /* bf16 [n_fft + 2] or NULL */
    const float* window_fn;     /* f32 [n_fft] */
} or_vae_model;

/* Intermediates of one VAE layer over F rows (optional, f32). */
typedef struct {
    float* qkv;  /* [F][hidden + 2 kv_heads head_dim] roped q | roped k | v */
    float* att;  /* [F][hidden] */
    float* x1;   /* [F][hidden] */
    float* hh;   /* [F][inter] */
} or_vae_trace;

/* f32 activations through a bf16 or affine linear (+ bf16 bias): y [M][N] f32. */
void or_linear_f32(const or_linear* L, const float* x, int64_t M, const uint16_t* bias, float* y);
/* fast::rms_norm on f32 rows, bf16 weight: out = w * (x * rsqrt(mean(x^2) + eps)) in f32. */
void or_rms_f32(const float* x, const uint16_t* w, int64_t M, int64_t n, float eps, float* out);
/* fast::rope, traditional=false, f32 heads [nh][hd] in place. */
void or_rope_f32(float* x, int nh, int hd, int pos, float log2_base);
/* linear upsample x scale, align_corners=False: bf16 [T][C] -> f32 [T*scale][C]. */
void or_linear_upsample(const uint16_t* x, int T, int C, int scale, float* y);
/* sliding-window causal attention: q [F][heads][hd], k/v [F][kv_heads][hd] f32 -> [F][heads][hd]. */
void or_window_attention(const float* q, const float* k, const float* v, int F, int heads, int kv_heads, int hd,
                         int window, float scale, float* out);
/* one backbone layer over F rows (positions 0..F-1): x [F][hidden] -> x_out. */
void or_vae_layer(const or_vae_cfg* c, const or_lm_layer* l, const float* x, int F, float* x_out, or_vae_trace* tr);
/* ISTFT head: p [F][n_fft + 2] (log-magnitudes | phases) -> wave [F * hop]; frames (optional) [F][n_fft]. */
void or_vae_istft(const float* p, int F, int n_fft, int hop, const float* win, float* wave, float* frames);
/* Model.vaeDecode: latents bf16 [T][latent] -> wave f32 [T * patch * hop]; xs (optional)
 * [n_layers + 1][F][hidden] layer inputs (xs[0] = upsampled fc1 rows); head_out (optional) [F][n_fft + 2]. */
void or_vae_decode(const or_vae_model* m, const uint16_t* latents, int T, float* wave, float* xs, float* head_out);

#ifdef __cplusplus
}
#endif
#endif
