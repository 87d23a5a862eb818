/*
 * ming_hip.h -- C ABI of the MI355X (gfx950) per-token generation loop of
 * Ming-3.0-tts: the KV-cached Qwen2 decode step over MLX-affine 4-bit (or
 * bf16) weights, and the fused DiT flow-head / aggregator path.
 *
 * This is the drop-in boundary for the reference's fused-kernel module
 * (sbusso/ming-tts-serve src/ming_fused.zig) and the quantized-matmul entry
 * points of its mlx-c FFI (src/mlx.zig:278-292).  Names keep the reference's
 * with a `ming_` prefix; argument order follows the reference function each
 * one replaces (cited per declaration).
 *
 * Conventions (src/ming_fused.zig:444-446, src/ming_model.zig:262-274):
 *  - Every tensor/weight pointer is DEVICE memory, row-major contiguous.
 *    Inputs are borrowed; outputs go to caller-provided buffers (no per-call
 *    allocation on the hot path).
 *  - Calls are asynchronous on the context's stream, like MLX's lazy graph;
 *    ming_sync() is the eval point.
 *  - Every function returns a status (0 = MING_OK), like mlx-c's int return;
 *    ming_last_error() gives the message.  A context is single-threaded, like
 *    the reference's one engine thread (src/ming_service.zig:11-14).
 *  - dtypes: bf16 activations/weights/scales/biases, u32 packed weights,
 *    f32 accumulators and logits, i32 token ids.
 */
#ifndef MING_HIP_H
#define MING_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes ---------------------------------------------------------
 * Replace the reference's Zig error set: error.MlxError (src/mlx.zig:431-433),
 * error.CacheTooLong (src/ming_fused.zig:601), error.PromptTooLong
 * (src/ming_model.zig:1391). */
enum ming_status {
    MING_OK = 0,
    MING_E_SHAPE = 1,               /* tensor shape/dtype does not fit the kernel */
    MING_E_CTX_OVER_CAPACITY = 2,   /* KV cache full (error.CacheTooLong) */
    MING_E_HIP = 3,                 /* a HIP runtime call failed */
    MING_E_NOT_INIT = 4,            /* null or destroyed context / model */
    MING_E_ARG = 5,                 /* invalid argument */
    MING_E_UNSUPPORTED = 6,         /* valid MLX request this build does not implement */
    MING_E_TIMEOUT = 7              /* a device-side wait exceeded its spin limit */
};

enum ming_dtype { MING_DT_BF16 = 1, MING_DT_F32 = 2, MING_DT_U32 = 3, MING_DT_I32 = 4 };

/* Replaces mlx_array (src/mlx.zig) on the hot path: a borrowed device view. */
typedef struct {
    void* data;
    int32_t dtype;      /* enum ming_dtype */
    int32_t ndim;
    int64_t shape[4];
} ming_tensor;

/* Replaces mlx_stream: owns a HIP stream (or borrows one), workspaces and
 * per-device state. */
typedef struct ming_ctx ming_ctx;

int ming_ctx_create(ming_ctx** out, int device);
int ming_ctx_destroy(ming_ctx* ctx);
/* Run on a caller-owned hipStream_t, used as given: NULL is HIP's null
 * (default) stream.  A new context runs on a stream of its own until this is
 * called; ming_ctx_use_own_stream() returns to it. */
int ming_ctx_set_stream(ming_ctx* ctx, void* hip_stream);
int ming_ctx_use_own_stream(ming_ctx* ctx);
void* ming_ctx_stream(ming_ctx* ctx);
/* The eval point (mlx_eval, src/ming_model.zig:269-274); also reports any
 * device-side error flag (MING_E_TIMEOUT). */
int ming_sync(ming_ctx* ctx);
const char* ming_last_error(ming_ctx* ctx);
const char* ming_status_str(int status);

/* MING_FUSED / MING_FUSED_DIT / MING_FUSED_LM (value "0" = off), as
 * enabled()/ditEnabled()/lmEnabled() at src/ming_fused.zig:53-63. */
int ming_fused_enabled(void);
int ming_dit_enabled(void);
int ming_lm_enabled(void);
/* ming-parity's switch (src/ming_fused.zig:49: `force_off`). */
void ming_set_force_off(int off);

/* Device memory for hosts without another allocator (the Zig engine). */
int ming_malloc(ming_ctx* ctx, size_t bytes, void** out);
int ming_free(ming_ctx* ctx, void* p);
int ming_memcpy_htod(ming_ctx* ctx, void* dst, const void* src, size_t bytes);
int ming_memcpy_dtoh(ming_ctx* ctx, void* dst, const void* src, size_t bytes);
int ming_memset(ming_ctx* ctx, void* dst, int value, size_t bytes);

/* ---- MLX-affine quantized linear algebra --------------------------------- */

/* y[N] = global_scale * (W x) with W the MLX-affine matrix [N, K]:
 *   w u32 [N, K*bits/32] (element k of a row in bits [(k%8)*4, +4) of word k/8),
 *   scales/biases bf16 [N, K/group_size], dequantized value s*q + b.
 * x bf16 [K] (or [M, K], M <= 8 rows); y bf16 [N] (or [M, N]), rounded once.
 * Mirrors mlx_quantized_matmul(x, w, scales, biases, transpose_w=true,
 * group_size, bits, "affine") (src/mlx.zig:279); `global_scale` is the
 * parameter the reference's mlx-c patch adds (patches/mlxc-gather-qmm-
 * global-scale.patch:10-18): it multiplies the f32 accumulator, and 1.0 is
 * plain MLX affine.  Supported: bits = 4, group_size = 64, K % 64 == 0. */
int ming_qgemv(ming_ctx* ctx, const ming_tensor* x, const ming_tensor* w, const ming_tensor* scales,
               const ming_tensor* biases, float global_scale, int32_t group_size, int32_t bits, ming_tensor* y);

/* y[N] f32 accumulators (no rounding) of the same product; for logits. */
int ming_qgemv_f32(ming_ctx* ctx, const ming_tensor* x, const ming_tensor* w, const ming_tensor* scales,
                   const ming_tensor* biases, float global_scale, int32_t group_size, int32_t bits,
                   ming_tensor* y);

/* out bf16 [N, K] = bf16(global_scale * (s*q + b)).  Mirrors mlx_dequantize
 * (src/mlx.zig:288). */
int ming_dequantize(ming_ctx* ctx, const ming_tensor* w, const ming_tensor* scales, const ming_tensor* biases,
                    int32_t group_size, int32_t bits, float global_scale, ming_tensor* out);

/* MLX-affine quantization of bf16 [N, K] -> (w, scales, biases).  Mirrors
 * mlx_quantize(w, group_size, bits, "affine") (src/mlx.zig:292). */
int ming_quantize(ming_ctx* ctx, const ming_tensor* w, int32_t group_size, int32_t bits, ming_tensor* wq,
                  ming_tensor* scales, ming_tensor* biases);

/* ---- Qwen2 decode ---------------------------------------------------------- */

enum ming_wkind { MING_W_BF16 = 0, MING_W_AFFINE = 1 };

/* One linear's weights ([out, in], as fused.LmLayer holds them,
 * src/ming_fused.zig:576-589), bf16 or MLX-affine. */
typedef struct {
    int32_t kind;                 /* enum ming_wkind */
    int32_t out_features, in_features;
    int32_t group_size, bits;     /* affine only: 64, 4 */
    float global_scale;           /* affine only; 1.0 = plain affine */
    const void* w;                /* bf16 [out,in] or u32 [out, in*bits/32] */
    const void* scales;           /* bf16 [out, in/group] (affine) */
    const void* biases;           /* bf16 [out, in/group] (affine) */
} ming_linear;

/* Model shape (src/ming_model.zig:497-504; Qwen2-0.5B: 896, 14, 2, 64, 4864,
 * 151936, 24, eps 1e-6, log2(1e6)). */
typedef struct {
    int32_t hidden, heads, kv_heads, head_dim, inter, vocab, n_layers;
    float eps, log2_theta;
} ming_lm_cfg;

/* fused.LmLayer (src/ming_fused.zig:576-589). q/k/v biased; o, gate, up,
 * down not. */
typedef struct {
    const void *ln1, *ln2;        /* bf16 [hidden] */
    ming_linear wq, wk, wv, wo, wg, wu, wd;
    const void *bq, *bk, *bv;     /* bf16 */
} ming_lm_layer_w;

/* KvCache (src/ming_model.zig:638-662), held in place: k/v bf16
 * [n_layers][kv_heads][capacity][head_dim]; `len` cached positions.  The
 * reference grows its cache by concatenation (or the fused copy,
 * src/ming_fused.zig:338-342); here the new row is written at `len`. */
typedef struct {
    void* k;
    void* v;
    int32_t n_layers, kv_heads, head_dim, capacity;
    int32_t len;
} ming_kv;

/* LmOut (src/ming_fused.zig:591): caller-provided bf16 buffers. */
typedef struct {
    void* qkv;   /* [hidden + 2*kv_heads*head_dim]: roped q | roped k | v */
    void* o;     /* [hidden] attention output */
    void* x1;    /* [hidden] x + o_proj */
    void* hh;    /* [inter] swiglu */
    void* x2;    /* [hidden] layer output */
} ming_lm_out;

/* One Qwen2 decode layer on x [hidden] at position `pos` with the cache rows
 * [0, pos) of `layer`; writes the new k/v row at pos.  Replaces
 * lmLayer(l, x, pos, kc, vc, log2_theta, s) (src/ming_fused.zig:597-614).
 * Returns MING_E_CTX_OVER_CAPACITY when pos >= kv->capacity. */
int ming_lm_layer(ming_ctx* ctx, const ming_lm_cfg* cfg, const ming_lm_layer_w* l, const void* x, int32_t pos,
                  ming_kv* kv, int32_t layer, ming_lm_out* out);

/* A prepared decode stack: device-side descriptors of all layers plus the
 * final norm, the tied LM head and the embedding table.  Replaces
 * QStack.fuse (src/ming_model.zig:510-527).  Weights stay caller-owned and
 * must outlive the model. */
typedef struct ming_lm_model ming_lm_model;

int ming_lm_model_create(ming_ctx* ctx, const ming_lm_cfg* cfg, const ming_lm_layer_w* layers,
                         const void* final_norm, const ming_linear* head, const ming_linear* embed,
                         ming_lm_model** out);
int ming_lm_model_destroy(ming_lm_model* m);

/* Execution modes of the decode step. */
enum ming_lm_mode {
    MING_LM_AUTO = 0,        /* fastest available */
    MING_LM_KERNELS = 1,     /* one launch per stage (debug / reference schedule) */
    MING_LM_PERSISTENT = 2,  /* one persistent kernel per token */
    MING_LM_PERSISTENT_DIRECT = 3  /* persistent, every workgroup stages its own inputs (no per-XCD hubs) */
};
int ming_lm_model_set_mode(ming_lm_model* m, int32_t mode);

/* Per-stage timing of the persistent schedule (the reference's MING_PROFILE
 * step timing, src/ming_model.zig:1394-1410, at stage granularity): with a
 * device buffer of u64 [n_stamps][grid] set, every workgroup writes the
 * device wall clock (wall_clock64) at each stage boundary of later steps.
 * NULL turns it off.  ming_lm_model_profile_shape gives the buffer shape. */
int ming_lm_model_profile(ming_lm_model* m, void* stamps_dev);
int ming_lm_model_profile_shape(ming_lm_model* m, int32_t* n_stamps, int32_t* grid);

/* One decode step: QStack.decodeFused (src/ming_model.zig:530-544) plus the
 * tied LM head and greedy argmax.  Input: if `token_dev` is non-NULL, the
 * embedding row of the id it points to (device i32); else x_in (device bf16
 * [hidden]).  Appends one KV position at kv->len and increments kv->len.
 * Outputs (each optional, device): hidden_out bf16 [hidden] (final-normed),
 * logits_out f32 [vocab], argmax_out i32 (argmax of the f32 logits, lowest
 * index on ties). */
int ming_lm_step(ming_ctx* ctx, ming_lm_model* m, const int32_t* token_dev, const void* x_in, ming_kv* kv,
                 void* hidden_out, float* logits_out, int32_t* argmax_out);

/* Per-layer activations of the model's last ming_lm_step, for parity checks
 * (the reference's per-step Trace, src/ming_model.zig:1375-1385): x bf16
 * [n_layers + 1][hidden] (each layer's input, then the stack output), x1 and
 * att [n_layers][hidden], qkv [n_layers][hidden + 2*kv_heads*head_dim] (roped
 * q | roped k | v), hh [n_layers][inter].  Device buffers; NULL skips one.
 * Asynchronous on the context's stream. */
int ming_lm_model_trace(ming_lm_model* m, void* x, void* x1, void* att, void* qkv, void* hh);

/* n greedy steps fed back on the device: token i+1 = argmax of step i.
 * tokens_dev: device i32 [n_steps + 1]; tokens_dev[0] is the input token and
 * tokens_dev[1..n] receive the argmaxes.  No host synchronisation inside. */
int ming_lm_generate(ming_ctx* ctx, ming_lm_model* m, ming_kv* kv, int32_t n_steps, int32_t* tokens_dev);

/* ---- synthetic inputs (host side; benches and tests) -----------------------
 * Counter-based splitmix64 + Box-Muller: element i of stream (seed, name) is
 * a pure function of (seed, fnv1a64(name), i), so any slice can be generated
 * independently and in parallel. */
uint64_t ming_synth_stream(uint64_t seed, const char* name);
/* bf16(mean + std * N(0,1)) into host memory. */
void ming_synth_normal_bf16(uint64_t stream, float mean, float std, uint16_t* out, size_t n, int threads);
/* uniform integers in [0, hi) */
void ming_synth_uniform_i32(uint64_t stream, int32_t hi, int32_t* out, size_t n);

#ifdef __cplusplus
}
#endif
#endif
