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

enum ming_dtype {
    MING_DT_BF16 = 1, MING_DT_F32 = 2, MING_DT_U32 = 3, MING_DT_I32 = 4,
    /* storage dtypes a checkpoint may hold (no compute entry point takes them) */
    MING_DT_F16 = 5, MING_DT_I64 = 6, MING_DT_U8 = 7, MING_DT_F64 = 8, MING_DT_I8 = 9, MING_DT_BOOL = 10,
    MING_DT_I16 = 11, MING_DT_U16 = 12, MING_DT_U64 = 13
};

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
/* Model, batch and weights handles may be destroyed before or after the
 * context they were created on (their destroy calls do not touch it). */
int ming_ctx_destroy(ming_ctx* ctx);
/* Run on a caller-owned hipStream_t, used as given: NULL is HIP's null
 * (default) stream.  A new context runs on a stream of its own until this is
 * called; ming_ctx_use_own_stream() returns to it. */
int ming_ctx_set_stream(ming_ctx* ctx, void* hip_stream);
int ming_ctx_use_own_stream(ming_ctx* ctx);
/* on != 0: the caller promises that nothing else runs on the device while this
 * context's persistent decode step runs, so the step is dispatched as an
 * ordinary launch instead of a cooperative one (about 16 us less per token).
 * Off by default.  A broken promise surfaces as MING_E_TIMEOUT from the
 * bounded waits, never as a hang.  No counterpart in the reference: MLX
 * dispatches per op (src/ming_fused.zig has no persistent step). */
int ming_ctx_set_exclusive(ming_ctx* ctx, int on);
/* Device bytes the context holds in workspaces it grows on demand (the staging
 * of ming_qgemm, the attention partials of ming_lm_layer): 0 on a new context.
 * No counterpart in the reference (MLX owns its allocations); it lets a caller
 * that must not allocate check that its calls did not. */
int ming_ctx_workspace_bytes(const ming_ctx* ctx, int64_t* bytes);
void* ming_ctx_stream(ming_ctx* ctx);
/* The eval point (mlx_eval, src/ming_model.zig:269-274); also reports any
 * device-side error flag raised since the last call: MING_E_TIMEOUT (a
 * bounded wait expired), MING_E_ARG (a gather_qmm index out of range),
 * MING_E_CTX_OVER_CAPACITY (a batched step's position or page id outside its
 * paged cache). */
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

/* Y [M, N] = global_scale * (X W^T) for M = 1..64 activation rows (X bf16
 * [M, K]); y bf16 (rounded once) or f32 (the accumulators).  The batched
 * shape of the same call (mlx_quantized_matmul with M > 1, src/mlx.zig:279),
 * as a server batching M sequences' decode steps issues it: matrix-core
 * GEMM, the weight bytes read once for all M rows.  Same accumulation as
 * ming_qgemv per group of 64; the sum order over groups differs, so results
 * agree with ming_qgemv within f32 rounding, not bit for bit. */
int ming_qgemm(ming_ctx* ctx, const ming_tensor* x, const ming_tensor* w, const ming_tensor* scales,
               const ming_tensor* biases, float global_scale, int32_t group_size, int32_t bits, ming_tensor* y);

/* ming_qgemm without any allocation: no counterpart in the reference.  For
 * callers that cannot allocate device memory (code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc).  Same arguments and
 * the same kernels as ming_qgemm, so the results are bit-identical; the
 * activation staging lives in a fixed per-device array of 1,081,344 bytes
 * (held by every GPU the library runs on until the process ends) instead of
 * the context's growable buffer, which limits a call to M <= 64 rows at
 * K <= 8192 (MING_E_UNSUPPORTED beyond, before anything is launched).
 * Every call on one GPU shares that GPU's array: calls that overlap on one
 * GPU (several streams or host threads) race. */
int ming_qgemm_noalloc(ming_ctx* ctx, const ming_tensor* x, const ming_tensor* w, const ming_tensor* scales,
                       const ming_tensor* biases, float global_scale, int32_t group_size, int32_t bits,
                       ming_tensor* y);

/* Gathered quantized matmul: y[p] = global_scale * (x[lhs[p]] W[rhs[p]]^T)
 * for every index pair p.  Mirrors mlx_gather_qmm(x, w, scales, biases,
 * lhs_indices, rhs_indices, transpose_w, group_size, bits, "affine",
 * sorted_indices) (src/mlx.zig:282) with the global scale MLX 0.32.3 places
 * before sorted_indices, which the reference's mlx-c patch pins to "none"
 * (patches/mlxc-gather-qmm-global-scale.patch:10-18); here it multiplies the
 * f32 accumulator as in ming_qgemv (1.0 = plain affine).
 *   x bf16 [..., M, K] (leading dims = the batch the lhs indices select),
 *   w u32 [..., N, K/8], scales/biases bf16 [..., N, K/64] (leading dims = the
 *     matrices the rhs indices select), lhs/rhs i32 [P] device tensors (lhs
 *     may be NULL: pair p uses x[p], or x[0] when x has one batch entry),
 *   y bf16 or f32 [P, M, N] ([P, N] for M = 1).
 * Each pair's rows equal ming_qgemv of that row and matrix bit for bit.
 * sorted_indices != 0 (rhs non-decreasing) lets a workgroup read a matrix's
 * weights once for a run of pairs that share it; results do not depend on it.
 * Supported: transpose_w = 1, bits 4, group 64, K <= 16384, M <= 8 (fewer at
 * large K).  An index outside its range leaves its pair unwritten and is
 * reported by the next ming_sync as MING_E_ARG. */
int ming_gather_qmm(ming_ctx* ctx, const ming_tensor* x, const ming_tensor* w, const ming_tensor* scales,
                    const ming_tensor* biases, const ming_tensor* lhs_indices, const ming_tensor* rhs_indices,
                    int32_t transpose_w, int32_t group_size, int32_t bits, float global_scale,
                    int32_t sorted_indices, ming_tensor* y);

/* out bf16 [N, K] = bf16(global_scale * (s*q + b)).  Mirrors mlx_dequantize
 * (src/mlx.zig:288). */
int ming_dequantize(ming_ctx* ctx, const ming_tensor* w, const ming_tensor* scales, const ming_tensor* biases,
                    int32_t group_size, int32_t bits, float global_scale, ming_tensor* out);

/* MLX-affine quantization of bf16 [N, K] -> (w, scales, biases).  Mirrors
 * mlx_quantize(w, group_size, bits, "affine", global_scale) (src/mlx.zig:292).
 * The reference leaves the global scale's meaning open (it never quantizes);
 * here each group is quantized as w / global_scale (f32, correctly rounded
 * division), the inverse of ming_dequantize and ming_qgemv, which multiply by
 * it: 1.0 is plain MLX affine, bit for bit.  global_scale must be finite and
 * > 0 (MING_E_ARG otherwise). */
int ming_quantize(ming_ctx* ctx, const ming_tensor* w, int32_t group_size, int32_t bits, float global_scale,
                  ming_tensor* wq, ming_tensor* scales, ming_tensor* biases);

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
    MING_LM_PERSISTENT_DIRECT = 3, /* persistent, every workgroup stages its own inputs (no per-XCD hubs) */
    MING_LM_PERSISTENT_XCD = 4     /* persistent, each kv head's q/k/v, attention and o_proj inside one XCD;
                                      o_proj and down as split-K partials summed by the per-XCD hubs */
};
int ming_lm_model_set_mode(ming_lm_model* m, int32_t mode);

/* Per-stage timing of the persistent schedule (the reference's MING_PROFILE
 * step timing, src/ming_model.zig:1394-1410, at stage granularity): with a
 * device buffer of u64 [n_stamps][grid] set, every workgroup writes the
 * device wall clock (wall_clock64) at each stage boundary of later steps:
 * row 0 its start; for stage s (0 q/k/v, 1 attention, 2 o_proj, 3 gate/up,
 * 4 down) of layer l, row 1 + 2 (5 l + s) when its input has arrived and the
 * next row when it is done; the head takes the two rows after the last
 * layer.  The per-XCD hubs (workgroups 0..7) write the rows of the stages
 * they serve: input arrived (every value of a normalised vector received)
 * and done (the stage image's flag raised).  NULL turns it off.
 * ming_lm_model_profile_shape gives the buffer shape. */
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

/* ---- Multi-request decode over a paged KV cache ------------------------------
 * No counterpart in the reference: its service decodes one request at a
 * time with a contiguous cache per request (src/ming_service.zig:11-14,
 * :175-206).  Here n_seq sequences advance one token per call; each linear is
 * one 4-bit GEMM over the n_seq rows on the matrix cores (ming_qgemm's
 * arithmetic) and attention reads each sequence's pages.  Per sequence the
 * result is the batch-1 step's (ming_lm_step) within f32 summation order.
 *
 * Paged cache: pages of 64 positions, one page id per 64 positions of a
 * sequence for all layers and kv heads; head_dim 64.
 *   k: bf16 [n_layers][n_pages][kv_heads][64 positions][head_dim]
 *   v: bf16 [n_layers][n_pages][kv_heads][head_dim][64 positions]
 *      (each V page stored transposed). */
typedef struct {
    void* k;
    void* v;
    int32_t n_layers, kv_heads, head_dim, page_size, n_pages;
} ming_kv_pages;

/* Workspace for up to max_seqs (<= 512) sequences of up to max_ctx positions
 * on a prepared model (4-bit linears; head_dim 64; hidden and inter
 * multiples of 64).  Holds every layer's activations of the last step.
 * ming_lm_prefill takes a prompt in chunks of max_seqs rows; a step or chunk
 * of more than 64 rows splits each GEMM's K exactly as one of <= 64 rows does,
 * so a row's result does not depend on the number of rows. */
typedef struct ming_lm_batch ming_lm_batch;
int ming_lm_batch_create(ming_ctx* ctx, ming_lm_model* m, int32_t max_seqs, int32_t max_ctx, ming_lm_batch** out);
int ming_lm_batch_destroy(ming_lm_batch* b);

/* One decode step of n_seq sequences.  Input rows: the embeddings of
 * tokens_dev (device i32 [n_seq]) or x_in (device bf16 [n_seq][hidden]).
 * page_table_dev: device i32 [n_seq][pages_per_seq], the pages of sequence i
 * in position order (pages_per_seq * 64 <= max_ctx); pos_dev: device i32
 * [n_seq], the position of each sequence's new row (its cached length); the
 * step writes the new k/v rows there and adds 1 to every pos_dev entry.
 * Outputs (each optional, device): hidden_out bf16 [n_seq][hidden]
 * (final-normed), logits_out f32 [n_seq][vocab], argmax_out i32 [n_seq]
 * (lowest index on ties).  A position at or past pages_per_seq * 64, or a
 * page id outside [0, n_pages), is reported by the next ming_sync as
 * MING_E_CTX_OVER_CAPACITY (that sequence's append and attention are skipped). */
int ming_lm_batch_step(ming_lm_batch* b, int32_t n_seq, const int32_t* tokens_dev, const void* x_in,
                       const ming_kv_pages* kv, const int32_t* page_table_dev, int32_t pages_per_seq, int32_t* pos_dev,
                       void* hidden_out, float* logits_out, int32_t* argmax_out);

/* Multi-token prefill of one sequence (QStack prefill over the prompt,
 * src/ming_model.zig:576-614: every layer over L rows with causal attention):
 * rows [0, L) -- the embeddings of tokens_dev (i32 [L]) or x_in (bf16
 * [L][hidden]) -- at positions pos0 .. pos0 + L - 1 of the sequence whose
 * pages are page_table_dev (i32 [pages_per_seq]).  Row i attends to
 * positions <= pos0 + i; the k/v rows of every position are written into the
 * pages.  Runs as ceil(L / max_seqs) batched steps in which the rows are
 * sequences sharing one page table, so each row's result equals a one-row
 * ming_lm_batch_step at that position bit for bit.  Outputs (optional,
 * device): hidden_out bf16 [L][hidden], logits_out f32 [L][vocab],
 * argmax_out i32 [L].  pos0 + L > pages_per_seq * 64 returns
 * MING_E_CTX_OVER_CAPACITY before anything is launched. */
int ming_lm_prefill(ming_lm_batch* b, int32_t L, const int32_t* tokens_dev, const void* x_in, const ming_kv_pages* kv,
                    const int32_t* page_table_dev, int32_t pages_per_seq, int32_t pos0, void* hidden_out,
                    float* logits_out, int32_t* argmax_out);

/* Per-layer activations of the last ming_lm_batch_step (n_seq rows each), as
 * ming_lm_model_trace lays them out with a sequence axis after the layer
 * axis: x [n_layers + 1][n_seq][hidden], x1 and att [n_layers][n_seq][hidden],
 * qkv [n_layers][n_seq][hidden + 2*kv_heads*head_dim], hh [n_layers][n_seq]
 * [inter].  Device buffers; NULL skips one. */
int ming_lm_batch_trace(ming_lm_batch* b, void* x, void* x1, void* att, void* qkv, void* hh);

/* ---- DiT flow head and aggregator ------------------------------------------
 * The reference's fused DiT path (src/ming_fused.zig:482-573) and its
 * callers DitStack.forward (src/ming_model.zig:770-797), cfmSample (:1143),
 * aggregate (:1154) and stopProb (:1033).  Rows: R = B*L <= 6 (CFM: 2 CFG
 * halves x 3; aggregator 1 x 2); bf16 weights [out, in] with biases. */

/* DiT shape (reference: 1024, 16, 64, 4096, eps 1e-6). */
typedef struct {
    int32_t hidden, heads, head_dim, ff;
    float eps;
} ming_dit_cfg;

/* fused.Block (src/ming_fused.zig:482-500): linears are MING_W_BF16. */
typedef struct {
    const void *norm1, *norm2;                 /* bf16 [hidden] */
    ming_linear wq, wk, wv, wo, w1, w2;
    const void *bq, *bk, *bv, *bo, *b1, *b2;   /* bf16 */
} ming_dit_block_w;

/* BlockOut (src/ming_fused.zig:521): caller buffers, bf16.  qkv [3][R][hidden]
 * (rotated q, rotated k, v), att/x1/x2 [R][hidden], hh [R][ff]. */
typedef struct {
    void *qkv, *att, *x1, *hh, *x2;
} ming_dit_out;

/* Rotary.precompute (src/ming_model.zig:698-704): cos/sin f32 [L][half] =
 * cos/sin(l * inv_freq[i]) from the checkpoint's f32 inv_freq (host). */
int ming_rotary_table(ming_ctx* ctx, const float* inv_freq_host, int32_t half, int32_t L, float* cos_dev,
                      float* sin_dev);

/* fused.block (src/ming_fused.zig:523-539): one DiT block on x [B, L, hidden]
 * with rotary tables [L][head_dim/2]; all five outputs required. */
int ming_dit_block(ming_ctx* ctx, const ming_dit_cfg* cfg, const ming_dit_block_w* w, const void* x, int32_t B,
                   int32_t L, const float* cos_dev, const float* sin_dev, ming_dit_out* out);

/* fused.single (src/ming_fused.zig:542-556): one kernel of a block.  which 0:
 * A (rms + q/k/v + rotary + attention; out = attention [R][hidden], qkv_tmp
 * receives q/k/v); 1: B (out = x + out_proj(in), in = attention); 2: C (out =
 * gelu(ff1(rms(x)))); 3: D (out = x + ff2(in), in = hh). */
int ming_dit_single(ming_ctx* ctx, int32_t which, const ming_dit_cfg* cfg, const ming_dit_block_w* w, const void* x,
                    const void* in, int32_t B, int32_t L, const float* cos_dev, const float* sin_dev, void* qkv_tmp,
                    void* out);

/* fused.embed (src/ming_fused.zig:559-561): CFM input rows h [2][3][hidden] =
 * [te + ce, xh, x_emb(y)] per CFG half; y [latent], te/ce [2][hidden], xh
 * [hidden]. */
int ming_cfm_embed(ming_ctx* ctx, const void* y, const ming_linear* x_emb, const void* bx, const void* te,
                   const void* ce, const void* xh, void* h_out);

/* fused.final (src/ming_fused.zig:565-573): final rms + linear on rows L-1
 * and 2L-1 of h [2L][hidden], CFG combine, Euler step `step` (+ SDE when
 * shift != 0).  dtt/sq bf16 [steps], sde bf16 [steps][latent]. */
int ming_cfm_final(ming_ctx* ctx, const void* h, int32_t L, const void* norm, const ming_linear* wf, const void* bf,
                   const void* y, const void* dtt, const void* sq, const void* sde, int32_t step, float cfg,
                   float shift, void* y_out);

/* Flow head weights (DitStack "flowloss.cfm.model" + embedders + final
 * layer, src/ming_model.zig:955-965). */
typedef struct {
    ming_dit_cfg cfg;
    int32_t n_blocks;
    const ming_dit_block_w* blocks;            /* host array [n_blocks] */
    const float* inv_freq;                     /* host f32 [head_dim/2] (rotary_embed.inv_freq) */
    ming_linear x_emb, c_emb, t_mlp0, t_mlp2, final;
    const void *bx, *bc, *bt0, *bt2, *final_norm, *bf;
} ming_cfm_w;

/* Aggregator weights (DitStack "linear_proj_audio", src/ming_model.zig:966-971). */
typedef struct {
    ming_dit_cfg cfg;
    int32_t n_blocks;
    const ming_dit_block_w* blocks;
    const float* inv_freq;
    ming_linear x_emb, final;
    const void *bx, *cls, *final_norm, *bf;
} ming_agg_w;

typedef struct ming_cfm_model ming_cfm_model;
typedef struct ming_agg_model ming_agg_model;

/* Model.load's flow-head precomputation (src/ming_model.zig:976-1004):
 * rotary table for L = 3, flow schedule, dt, sqrt|dt| and the 10 timestep
 * embeddings; workspace for one sample.  Weights stay caller-owned. */
int ming_cfm_model_create(ming_ctx* ctx, const ming_cfm_w* w, ming_cfm_model** out);
int ming_cfm_model_destroy(ming_cfm_model* m);
/* The model's flow schedule (host copies): t [steps+1], dt [steps], sq
 * [steps], t_emb device pointer [steps][2][hidden]. */
int ming_cfm_model_tables(ming_cfm_model* m, uint16_t* t, uint16_t* dt, uint16_t* sq, const void** t_emb_dev);
/* cfmSample (src/ming_model.zig:1143-1151, :1161-1203): 10 Euler steps of
 * the CFG DiT.  z [lm_hidden], hist/noise [latent], sde [steps][latent] (all
 * device bf16) -> latent_out [latent]; shift = sigma * sqrt(temperature).
 * y_steps (optional, device [steps][latent]) receives each step's latent. */
int ming_cfm_sample(ming_ctx* ctx, ming_cfm_model* m, const void* z, const void* hist, const void* noise,
                    const void* sde, float cfg, float sigma, float temperature, void* latent_out, void* y_steps);

/* Execution modes of ming_cfm_sample (no reference counterpart: the
 * reference dispatches one Metal kernel per fused stage).  PERSISTENT runs
 * the ten Euler steps in one persistent kernel (after the two per-sample
 * projections c_emb(z) and x_emb(hist)), bit-identical to KERNELS (about 42
 * launches per step); it covers hidden 1024, 16 heads of 64, ff 4096, latent
 * 64 and up to 16 blocks on a device with a multiple of 8 CUs, at least 232.  AUTO runs
 * PERSISTENT where it fits (the faster of the two on MI355X), else KERNELS.  Like the persistent
 * LM step, PERSISTENT needs every workgroup resident at once: a cooperative
 * launch, or an ordinary one after ming_ctx_set_exclusive(ctx, 1); a broken
 * promise ends in MING_E_TIMEOUT from ming_sync, not a hang. */
enum ming_cfm_mode {
    MING_CFM_AUTO = 0,
    MING_CFM_KERNELS = 1,
    MING_CFM_PERSISTENT = 2
};
int ming_cfm_model_set_mode(ming_cfm_model* m, int32_t mode);
/* Stage timing of the persistent flow head: with a device buffer of u64
 * [6][steps * n_blocks * 4] set, later persistent samples write device wall
 * clocks (wall_clock64) at index f = (step * n_blocks + block) * 4 + stage
 * (stages: rms1 rows, attention rows, rms2 rows, ff1 rows -- each the input
 * image of one worker stage): row 0, the first worker has published its
 * slice of image f; row 1, it holds the whole image in LDS; row 2, its first
 * compute wave has issued its stage outputs; row 3, it has received the
 * inputs of its slice; row 4 at index step, head 0 done with that step's
 * final layer; row 5, as row 2 for the last worker.  (The first image of
 * each step is published by the heads, so rows 0 and 3 stay unset there.)
 * NULL turns it off. */
int ming_cfm_model_profile(ming_cfm_model* m, void* stamps_dev);

/* cfmSample for n sequences at once (1 <= n <= 64), as a server batching
 * requests runs the flow head once per step (no reference counterpart: the
 * reference samples one request at a time).  Per sequence b the same
 * arithmetic as ming_cfm_sample on row b of each input: z [n][lm_hidden],
 * hist / noise [n][latent], sde [n][steps][latent] (may be NULL when
 * sigma * sqrt(temperature) == 0) -> latents_out [n][latent]; y_steps
 * (optional) [n][steps][latent].  Every DiT linear runs as one matrix-core
 * GEMM over the 6 n rows, so results agree with n ming_cfm_sample calls within
 * f32 summation order, not bit for bit.  hidden, ff, lm_hidden and latent
 * must be multiples of 64. */
int ming_cfm_sample_batch(ming_ctx* ctx, ming_cfm_model* m, int32_t n, const void* z, const void* hist,
                          const void* noise, const void* sde, float cfg, float sigma, float temperature,
                          void* latents_out, void* y_steps);

/* Aggregator precomputation (rotary table for L = 2) and workspace. */
int ming_agg_model_create(ming_ctx* ctx, const ming_agg_w* w, ming_agg_model** out);
int ming_agg_model_destroy(ming_agg_model* m);
/* aggregate (src/ming_model.zig:1042-1053, :1154-1157): latent [latent] ->
 * next LM input row out [lm_hidden]. */
int ming_aggregate(ming_ctx* ctx, ming_agg_model* m, const void* latent, void* out);
/* ming_aggregate with the stack's rows written out as well, for parity checks
 * (the reference's per-step Trace, src/ming_model.zig:1375-1385, at block
 * granularity): rows_out device bf16 [n_blocks + 1][2][hidden] = each
 * block's input rows [cls row, x_emb row], then the stack output; out as
 * ming_aggregate's, bit for bit (the same launches). */
int ming_aggregate_trace(ming_ctx* ctx, ming_agg_model* m, const void* latent, void* rows_out, void* out);

/* stopProb (src/ming_model.zig:1033-1038): p_dev (device f32) =
 * softmax(f32(stop_head(z)))[1]; head [2, lm_hidden] bf16 with bias. */
int ming_stop_prob(ming_ctx* ctx, const ming_linear* head, const void* bias, const void* z, float* p_dev);

/* ---- VAE decoder (the step after the loop) ----------------------------------
 * Model.vaeDecode (src/ming_model.zig:1257-1309): fc1 on the bf16 latents,
 * 4x linear upsample (align_corners=False, :1316-1340), a Qwen2 stack with a
 * causal sliding-window mask (QStack.forward with window 64, :566-636), final
 * norm, the head linear to n_fft + 2 values per frame and the ISTFT head:
 * magnitude min(exp(.), 100), phase, irfft of n_fft points, synthesis
 * window, overlap-add with hop n_fft / 4, division by the window envelope,
 * "same" trim.  As in the reference graph every activation after the
 * upsample is f32 (bf16 or 4-bit weights are widened exactly).  Reference
 * shape: 896, 14 / 2 heads of 64, 4864, 24 layers, eps 1e-6, theta 1e6,
 * window 64, latent 64, patch 4, n_fft 3528, hop 882. */
typedef struct {
    int32_t hidden, heads, kv_heads, head_dim, inter, n_layers;
    float eps, log2_theta;
    int32_t window, latent, patch, n_fft, hop;
} ming_vae_cfg;

typedef struct {
    ming_linear fc1;                  /* [hidden, latent] */
    const void* fc1_bias;             /* bf16 [hidden] or NULL */
    const ming_lm_layer_w* layers;    /* [n_layers]; q/k/v biases may be NULL */
    const void* norm;                 /* bf16 [hidden] */
    ming_linear head;                 /* [n_fft + 2, hidden] */
    const void* head_bias;            /* bf16 [n_fft + 2] or NULL */
    const void* window;               /* f32 [n_fft] (istft.window) */
} ming_vae_w;

typedef struct ming_vae_model ming_vae_model;
/* Builds the irfft basis and the workspace for up to max_latents latents per
 * call; weights stay caller-owned. */
int ming_vae_model_create(ming_ctx* ctx, const ming_vae_cfg* cfg, const ming_vae_w* w, int32_t max_latents,
                          ming_vae_model** out);
int ming_vae_model_destroy(ming_vae_model* m);
/* latents bf16 [T][latent] (device) -> wave_out f32 [T * patch * hop] (device). */
int ming_vae_decode(ming_ctx* ctx, ming_vae_model* m, int32_t T, const void* latents, float* wave_out);
/* The last decode's intermediates (device, f32; NULL skips one): xs
 * [n_layers + 1][F][hidden] the layer inputs (xs[0] = the upsampled rows,
 * xs[n_layers] the stack output before the final norm), head_out
 * [F][n_fft + 2]; F = T * patch. */
int ming_vae_trace(ming_vae_model* m, float* xs, float* head_out);

/* ---- adaLN DiT flow head (config 4) ----------------------------------------
 * No reference implementation exists (the reference DiT conditions by an
 * additive row, src/ming_model.zig:1078-1091); this build defines the variant
 * as the standard adaLN-Zero DiT on the reference block's RMSNorm.  Per CFG half
 * b (uncond: z = 0) and Euler step s: c = bf16(t_emb[s] + c_emb(z)); per block
 * mod = bf16(b_ada + W_ada silu(c)) = [shift_a | scale_a | gate_a | shift_m |
 * scale_m | gate_m] (6 x hidden); modulate(n) = bf16(bf16(n*bf16(1+scale)) +
 * shift) on each rms_norm output; x1 = bf16(x + bf16(gate_a*out_proj(...))),
 * x2 = bf16(x1 + bf16(gate_m*ff2(...))).  Rows are the F patch frames
 * x_emb(y_f) per half (rotary positions 0..F-1); the final layer is
 * modulate(rms(h)) with [shift | scale] = b_fa + W_fa silu(c), a linear to the
 * latent and CFG + Euler (+ SDE) per frame.  shift = scale = 0, gate = 1 gives
 * the reference block exactly. */
typedef struct {
    ming_dit_block_w base;
    ming_linear ada;        /* bf16 [6*hidden, hidden] */
    const void* bada;       /* bf16 [6*hidden] */
} ming_adaln_block_w;

/* One adaLN block on x [B, L, hidden] (B <= 2 CFG halves, B*L <= 8) with
 * mod (device bf16 [B][6*hidden]) and rotary tables [L][head_dim/2]. */
int ming_adaln_block(ming_ctx* ctx, const ming_dit_cfg* cfg, const ming_adaln_block_w* w, const void* mod,
                     const void* x, int32_t B, int32_t L, const float* cos_dev, const float* sin_dev,
                     ming_dit_out* out);

typedef struct {
    ming_dit_cfg cfg;
    int32_t n_blocks, frames;                  /* config 4: 4 blocks, 4 frames */
    const ming_adaln_block_w* blocks;          /* host array [n_blocks] */
    const float* inv_freq;                     /* host f32 [head_dim/2] */
    ming_linear x_emb, c_emb, t_mlp0, t_mlp2, final, final_ada;
    const void *bx, *bc, *bt0, *bt2, *final_norm, *bf, *bfa;
} ming_adaln_w;

typedef struct ming_adaln_model ming_adaln_model;
/* Load-time tables (rotary for L = frames, flow schedule, timestep embeddings)
 * and the workspace of one sample. */
int ming_adaln_model_create(ming_ctx* ctx, const ming_adaln_w* w, ming_adaln_model** out);
int ming_adaln_model_destroy(ming_adaln_model* m);
/* Device tables of the model, the last sample's included: t_emb [10][2][hidden],
 * silu(c) [10][2][hidden], modulations [n_blocks][10*2][6*hidden], final [10*2][2*hidden]. */
int ming_adaln_model_tables(ming_adaln_model* m, const void** t_emb_dev, const void** silu_c_dev,
                            const void** mods_dev, const void** modf_dev);
/* One flow-head sample of a patch: z [lm_hidden], noise [frames][latent], sde
 * [10][frames][latent] (device bf16) -> patch_out [frames][latent]; every
 * modulation of the 10 steps is computed once, up front (its weights are read
 * once per token); y_steps (optional, [10][frames][latent]) = each step's patch. */
int ming_adaln_sample(ming_ctx* ctx, ming_adaln_model* m, const void* z, const void* noise, const void* sde,
                      float cfg, float sigma, float temperature, void* patch_out, void* y_steps);

/* Sizes of a prepared model (out-pointers may be null). */
int ming_lm_model_dims(const ming_lm_model* m, int32_t* hidden, int32_t* vocab);
int ming_cfm_model_dims(const ming_cfm_model* m, int32_t* latent, int32_t* lm_hidden);
int ming_agg_model_dims(const ming_agg_model* m, int32_t* lm_hidden, int32_t* latent);

/* ---- per-token loop ---------------------------------------------------------
 * sampleLatents (src/ming_model.zig:1388-1480) on the handles above. */

/* SampleParams (src/ming_model.zig:1365-1373): defaults 1000, 2.0, 0.25, 0.0. */
typedef struct {
    int32_t max_steps;
    float cfg, sigma, temperature;
} ming_sample_params;

/* Noise replay bank (Noise.replay, src/ming_model.zig:1349-1363): device bf16
 * [steps][11][latent], row 0 the start noise and rows 1..10 the SDE draws of
 * each step, filled from the library's counter-based normal stream (seed,
 * "flow.noise").  MLX's own RNG stream is not reproduced. */
int ming_noise_bank(ming_ctx* ctx, uint64_t seed, int32_t steps, int32_t latent, void* bank_dev);

/* sampleLatents: embeds [L][hidden] (device bf16) are prefilled into kv
 * (appended at kv->len), z = the last row's final-normed hidden.  On an empty
 * cache (kv->len 0) with a model ming_lm_batch_create accepts, the prompt is
 * one multi-row forward (ming_lm_prefill over a page pool of the call's own,
 * then copied into kv; src/ming_model.zig:576-614); otherwise one decode step
 * per row;
 * then for step k < min(max_steps, capacity - len - L): latent_k =
 * cfmSample(z_k, history, bank[k]) into latents_out[k] (device bf16
 * [max_steps][latent]); z_{k+1} = LM(aggregate(latent_k)); stop_k =
 * stopProb(z_k); stop after latent_k when stop_k > 0.5 and k > 3.  history is
 * prompt_latent (device [latent], optional; zeros when null), then latent_{k-1}.
 * Pipelined one step ahead: the LM pass for k+1 is queued before stop_k is
 * read, so on a stop one extra position is appended to kv (the reference
 * discards its cache; here kv->len ends at len + L + n, or len + L + n - 1
 * when the step budget ran out).  Returns after the stream drains; *n_steps_out
 * = latents written; stop_out (host f32 [max_steps], optional) = stop_k;
 * z_trace (device bf16 [max_steps][hidden], optional) = z_k.  The device
 * error flags travel to the host with every stop_k: once one is raised
 * (during the call or before it) the loop ends and the call returns
 * ming_sync's status for it (MING_E_TIMEOUT, MING_E_CTX_OVER_CAPACITY or
 * MING_E_ARG) with *n_steps_out = 0. */
int ming_sample_latents(ming_ctx* ctx, ming_lm_model* lm, ming_cfm_model* cfm, ming_agg_model* agg,
                        const ming_linear* stop_head, const void* stop_bias, const void* embeds, int32_t L,
                        const void* prompt_latent, ming_kv* kv, const void* noise_bank,
                        const ming_sample_params* p, void* latents_out, int32_t* n_steps_out, float* stop_out,
                        void* z_trace);

/* ---- synthetic inputs (host side; benches and tests) -----------------------
 * Counter-based splitmix64 + Box-Muller: element i of stream (seed, name) is
 * a pure function of (seed, fnv1a64(name), i), so any slice can be generated
 * independently and in parallel. */
uint64_t ming_synth_stream(uint64_t seed, const char* name);
/* bf16(mean + std * N(0,1)) into host memory. */
void ming_synth_normal_bf16(uint64_t stream, float mean, float std, uint16_t* out, size_t n, int threads);
/* uniform integers in [0, hi) */
void ming_synth_uniform_i32(uint64_t stream, int32_t hi, int32_t* out, size_t n);

/* ---- Checkpoint loading ------------------------------------------------------
 * Tensors.load (src/ming_model.zig:316-350) reads `model.safetensors` through
 * mlx_load_safetensors; here the container is read natively.  A safetensors
 * file is an 8-byte little-endian header length, a JSON header {name:
 * {dtype, shape, data_offsets}} and the data block. */

/* Host-only index of a safetensors file (no device work): open parses and
 * validates the header (offsets inside the file, sizes matching dtype and
 * shape, unique names); `err` (optional) receives a message on failure.
 * Entry i: name, dtype (enum ming_dtype), ndim <= 8, shape[8], absolute file
 * offset and byte size.  ming_st_find returns an entry index or -1. */
typedef struct ming_st ming_st;
int ming_st_open(const char* path, ming_st** out, char* err, size_t err_cap);
int ming_st_close(ming_st* st);
int32_t ming_st_count(const ming_st* st);
int ming_st_entry(const ming_st* st, int32_t i, const char** name, int32_t* dtype, int32_t* ndim, int64_t* shape,
                  uint64_t* offset, uint64_t* nbytes);
int32_t ming_st_find(const ming_st* st, const char* name);

/* Device copies of a checkpoint's tensors (those whose names start with one
 * of `prefixes`; all when n_prefixes is 0), uploaded through pinned staging
 * buffers on the context's stream; the call returns after the upload.  The
 * handle owns the memory; models built from it borrow it, so it must outlive
 * them.  ming_weights_get fills a borrowed view (ndim > 4 folds into the
 * last kept dimension). */
typedef struct ming_weights ming_weights;
int ming_weights_load(ming_ctx* ctx, const char* path, const char* const* prefixes, int32_t n_prefixes,
                      ming_weights** out);
int ming_weights_destroy(ming_weights* w);
int ming_weights_get(const ming_weights* w, const char* name, ming_tensor* out);

/* The linear `name` [out_features, in_features] (Tensors.lin,
 * src/ming_model.zig:456-466): an MLX 4-bit triplet (`name.weight` u32
 * [out, in/8], `name.scales` and `name.biases` bf16 [out, in/64]) when the
 * checkpoint holds one, else the bf16 `name.weight` -- quantized to MLX
 * affine 4-bit / group 64 on the GPU when quantize != 0 (ming_quantize's
 * arithmetic; the copy is owned by the weights handle). */
int ming_weights_linear(ming_weights* w, const char* name, int32_t out_features, int32_t in_features,
                        int32_t quantize, ming_linear* out);

/* The decode stack of a Ming checkpoint: QStack.load("model.model", 24)
 * (src/ming_model.zig:544-560) with the embedding and tied head
 * `model.model.embed_tokens`, norms, q/k/v biases; the shape comes from cfg
 * and is checked against every tensor.  Linears as ming_weights_linear. */
int ming_lm_model_from_weights(ming_ctx* ctx, ming_weights* w, const ming_lm_cfg* cfg, int32_t quantize,
                               ming_lm_model** out);

/* The flow head (`flowloss.cfm.model`: DitStack.load + embedders + final
 * layer, src/ming_model.zig:941-950, with `rotary_embed.inv_freq` f32) and
 * the aggregator (`linear_proj_audio`, :951-956) of a checkpoint; bf16
 * linears (the fused DiT path's format). */
int ming_cfm_model_from_weights(ming_ctx* ctx, ming_weights* w, const ming_dit_cfg* cfg, int32_t n_blocks,
                                int32_t lm_hidden, int32_t latent, ming_cfm_model** out);
int ming_agg_model_from_weights(ming_ctx* ctx, ming_weights* w, const ming_dit_cfg* cfg, int32_t n_blocks,
                                int32_t lm_hidden, int32_t latent, ming_agg_model** out);
/* The VAE decoder of a checkpoint (Model.load, src/ming_model.zig:963-965,
 * :994-996): `audio.decoder.fc1`, the stack `audio.decoder.decoder`
 * (QStack.load with window 64), `audio.decoder.head.out` and the f32 (or
 * bf16, widened at load) `audio.decoder.head.istft.window`. */
int ming_vae_model_from_weights(ming_ctx* ctx, ming_weights* w, const ming_vae_cfg* cfg, int32_t quantize,
                                int32_t max_latents, ming_vae_model** out);

#ifdef __cplusplus
}
#endif
#endif
