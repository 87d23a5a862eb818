// C ABI glue: contexts, status reporting, argument validation and the decode
// plan.  The kernels live in *.hip; this file only checks shapes and launches.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

#include "internal.h"
#include "args.h"

namespace ming {

hipError_t launch_lm_layer(hipStream_t st, const StepArgs& a, const LayerDev& Ld, int l);
hipError_t launch_lm_step_kernels(hipStream_t st, const StepArgs& a, const LayerDev* host_layers);
hipError_t launch_lm_step_tagged(hipStream_t st, const StepArgs& a, int q4, int grid, bool cooperative);
hipError_t launch_copy_token(hipStream_t st, const int32_t* src, int32_t* dst);
int tagged_grid(int num_cus);
hipError_t launch_lm_step_xcd(hipStream_t st, const StepArgs& a, int q4, int grid, bool cooperative);
bool xcd_fits(int q4, int grid, int H, int heads, int kvh, int hd, int I, int n_layers);
int xcd_slots(int I);
int tagged_split_len(int n);
int tagged_hubs(int grid);
int tagged_img_stride(int H, int I);
int tagged_max_layers();
int tagged_units_per_worker();
int attn_split_len(int n);
size_t attn_part_floats(int kvh, int heads, int hd, int n);

int set_err(ming_ctx* ctx, int status, const std::string& msg) {
    if (ctx) ctx->err = msg;
    return status;
}

int hip_check(ming_ctx* ctx, hipError_t e, const char* what) {
    if (e == hipSuccess) return MING_OK;
    return set_err(ctx, MING_E_HIP, std::string(what) + ": " + hipGetErrorString(e));
}

}  // namespace ming

using namespace ming;

namespace {

bool g_force_off = false;

bool env_off(const char* name) {
    const char* v = std::getenv(name);
    return v && std::strcmp(v, "0") == 0;
}

bool alive(const ming_ctx* c) { return c && c->alive; }

// Stages of the persistent schedule whose inputs the per-XCD hubs stage
// (HUB_* bits).  Measured on MI355X at ctx 2048: the hubs pay off where many
// workgroups read one normalised vector (q/k/v, gate/up, head); o and down
// (64 workgroups each) are faster staging their inputs themselves.
// MING_LM_HUB_STAGES (a decimal bit mask) overrides the choice.
// Attention splits grouped by XCD (StepArgs::att_xl) unless MING_LM_ATT_XL=0.
bool att_xl_enabled() {
    static const bool v = [] {
        const char* e = std::getenv("MING_LM_ATT_XL");
        return !(e && e[0] == '0' && e[1] == '\0');
    }();
    return v;
}

// The XCD-local schedule for MING_LM_AUTO unless MING_LM_XCD=0.
bool xcd_enabled() {
    static const bool on = [] {
        const char* e = std::getenv("MING_LM_XCD");
        return !(e && e[0] == '0');
    }();
    return on;
}

// In the XCD-local schedule, hand-offs inside a slot through plain stores
// (where the slot's workgroups share an XCD) unless MING_LM_XCD_LOCAL=0, read
// at every step (the device-coherent form is what a slot split over XCDs
// runs; tests force it to check that it gives the same bits).
bool xcd_local_enabled() {
    const char* e = std::getenv("MING_LM_XCD_LOCAL");
    return !(e && e[0] == '0');
}

int hub_stages() {
    static const int v = [] {
        const char* e = std::getenv("MING_LM_HUB_STAGES");
        if (e && *e) {
            char* end = nullptr;
            const long x = std::strtol(e, &end, 10);
            if (end && *end == '\0' && x >= 0 && x < 32) return (int)x;
        }
        return (int)(HUB_QKV | HUB_UP | HUB_HEAD);
    }();
    return v;
}

[[maybe_unused]] int64_t numel(const ming_tensor* t) {
    int64_t n = 1;
    for (int i = 0; i < t->ndim; i++) n *= t->shape[i];
    return n;
}

// Rows x cols view of a 1-D or 2-D tensor.
bool as_2d(const ming_tensor* t, int64_t& rows, int64_t& cols) {
    if (!t || !t->data) return false;
    if (t->ndim == 1) {
        rows = 1;
        cols = t->shape[0];
        return true;
    }
    if (t->ndim == 2) {
        rows = t->shape[0];
        cols = t->shape[1];
        return true;
    }
    return false;
}

std::string shape_str(const ming_tensor* t) {
    std::string s = "[";
    for (int i = 0; i < t->ndim; i++) s += (i ? "," : "") + std::to_string(t->shape[i]);
    return s + "]";
}

// Validate an MLX-affine triple (w, scales, biases) -> N, K.
int check_affine(ming_ctx* ctx, const ming_tensor* w, const ming_tensor* s, const ming_tensor* b, int gs, int bits,
                 int64_t& N, int64_t& K) {
    if (bits != 4 || gs != 64)
        return set_err(ctx, MING_E_UNSUPPORTED, "affine: only bits=4, group_size=64 are implemented");
    int64_t wr, wc, sr, sc, br, bc;
    if (!as_2d(w, wr, wc) || !as_2d(s, sr, sc) || !as_2d(b, br, bc))
        return set_err(ctx, MING_E_SHAPE, "affine: w/scales/biases must be 1-D or 2-D device tensors");
    if (w->dtype != MING_DT_U32 || s->dtype != MING_DT_BF16 || b->dtype != MING_DT_BF16)
        return set_err(ctx, MING_E_SHAPE, "affine: w must be u32, scales/biases bf16");
    N = wr;
    K = wc * 8;
    if (sr != N || br != N || sc != K / gs || bc != K / gs || K % 64 != 0)
        return set_err(ctx, MING_E_SHAPE, "affine: scales/biases " + shape_str(s) + " do not match w " +
                                              shape_str(w));
    return MING_OK;
}

LinearDev to_dev(const ming_linear& l) {
    LinearDev d;
    d.kind = l.kind;
    d.N = l.out_features;
    d.K = l.in_features;
    d.gscale = l.kind == MING_W_AFFINE ? l.global_scale : 1.0f;
    d.w = static_cast<const uint32_t*>(l.w);
    d.s = static_cast<const uint16_t*>(l.scales);
    d.b = static_cast<const uint16_t*>(l.biases);
    return d;
}

int check_linear(ming_ctx* ctx, const ming_linear& l, int N, int K, const char* name) {
    if (l.kind != MING_W_BF16 && l.kind != MING_W_AFFINE)
        return set_err(ctx, MING_E_ARG, std::string(name) + ": unknown weight kind");
    if (l.out_features != N || l.in_features != K)
        return set_err(ctx, MING_E_SHAPE, std::string(name) + ": expected [" + std::to_string(N) + "," +
                                              std::to_string(K) + "], got [" + std::to_string(l.out_features) + "," +
                                              std::to_string(l.in_features) + "]");
    if (!l.w) return set_err(ctx, MING_E_ARG, std::string(name) + ": null weight");
    if (l.kind == MING_W_AFFINE) {
        if (l.bits != 4 || l.group_size != 64)
            return set_err(ctx, MING_E_UNSUPPORTED, std::string(name) + ": only 4-bit, group 64 affine");
        if (!l.scales || !l.biases) return set_err(ctx, MING_E_ARG, std::string(name) + ": null scales/biases");
        if (K % 64) return set_err(ctx, MING_E_SHAPE, std::string(name) + ": in_features % 64 != 0");
    } else if (K % 8) {
        return set_err(ctx, MING_E_SHAPE, std::string(name) + ": in_features % 8 != 0");
    }
    return MING_OK;
}

int check_cfg(ming_ctx* ctx, const ming_lm_cfg* c) {
    if (!c) return set_err(ctx, MING_E_ARG, "null cfg");
    if (c->head_dim != 64) return set_err(ctx, MING_E_UNSUPPORTED, "head_dim must be 64");
    if (c->kv_heads < 1 || c->heads % c->kv_heads || c->heads / c->kv_heads > 8)
        return set_err(ctx, MING_E_UNSUPPORTED, "heads / kv_heads must be an integer <= 8");
    if (c->hidden != c->heads * c->head_dim) return set_err(ctx, MING_E_SHAPE, "hidden != heads * head_dim");
    if (c->hidden % 64 || c->hidden > 2048) return set_err(ctx, MING_E_UNSUPPORTED, "hidden must be <= 2048, % 64");
    if (c->inter % 64 || c->inter > 8192) return set_err(ctx, MING_E_UNSUPPORTED, "inter must be <= 8192, % 64");
    if (c->n_layers < 1) return set_err(ctx, MING_E_ARG, "n_layers < 1");
    return MING_OK;
}

int check_layer(ming_ctx* ctx, const ming_lm_cfg* c, const ming_lm_layer_w* l) {
    const int H = c->hidden, kvd = c->kv_heads * c->head_dim, I = c->inter;
    int st;
    if (!l || !l->ln1 || !l->ln2 || !l->bq || !l->bk || !l->bv) return set_err(ctx, MING_E_ARG, "null layer tensor");
    if ((st = check_linear(ctx, l->wq, H, H, "wq")) || (st = check_linear(ctx, l->wk, kvd, H, "wk")) ||
        (st = check_linear(ctx, l->wv, kvd, H, "wv")) || (st = check_linear(ctx, l->wo, H, H, "wo")) ||
        (st = check_linear(ctx, l->wg, I, H, "wg")) || (st = check_linear(ctx, l->wu, I, H, "wu")) ||
        (st = check_linear(ctx, l->wd, H, I, "wd")))
        return st;
    const int k = l->wq.kind;
    if (l->wk.kind != k || l->wv.kind != k || l->wo.kind != k || l->wg.kind != k || l->wu.kind != k ||
        l->wd.kind != k)
        return set_err(ctx, MING_E_UNSUPPORTED, "all linears of a layer must share one weight kind");
    return MING_OK;
}

LayerDev layer_dev(const ming_lm_layer_w* l) {
    LayerDev d;
    d.ln1 = static_cast<const uint16_t*>(l->ln1);
    d.ln2 = static_cast<const uint16_t*>(l->ln2);
    d.q = to_dev(l->wq);
    d.k = to_dev(l->wk);
    d.v = to_dev(l->wv);
    d.o = to_dev(l->wo);
    d.g = to_dev(l->wg);
    d.u = to_dev(l->wu);
    d.d = to_dev(l->wd);
    d.bq = static_cast<const uint16_t*>(l->bq);
    d.bk = static_cast<const uint16_t*>(l->bk);
    d.bv = static_cast<const uint16_t*>(l->bv);
    return d;
}

int check_kv(ming_ctx* ctx, const ming_lm_cfg* c, const ming_kv* kv) {
    if (!kv || !kv->k || !kv->v) return set_err(ctx, MING_E_ARG, "null kv cache");
    if (kv->kv_heads != c->kv_heads || kv->head_dim != c->head_dim || kv->n_layers != c->n_layers ||
        kv->capacity < 1)
        return set_err(ctx, MING_E_SHAPE, "kv cache geometry does not match the model");
    if (kv->len < 0) return set_err(ctx, MING_E_ARG, "kv->len < 0");
    if (kv->len >= kv->capacity)
        return set_err(ctx, MING_E_CTX_OVER_CAPACITY,
                       "kv cache full: len " + std::to_string(kv->len) + " >= capacity " +
                           std::to_string(kv->capacity));
    return MING_OK;
}

}  // namespace

// ---- model --------------------------------------------------------------------

struct ming_lm_model {
    ming_ctx* ctx = nullptr;
    ming_lm_cfg cfg{};
    std::vector<LayerDev> layers;
    LayerDev* d_layers = nullptr;
    LinearDev head{}, embed{};
    const uint16_t* final_norm = nullptr;
    int mode = MING_LM_AUTO;
    int pgrid = 0;
    uint32_t epoch = 0;   // tag of the last persistent step (tags start at 1)
    uint64_t* tstamp = nullptr;  // optional stage-boundary stamps (ming_lm_model_profile)
    // workspace
    DevBuf x, x1, att, qkv, hh, part, hidden, amax_v, amax_i;
    DevBuf tx, tq, ta, tx1, th, counters;  // tagged hand-off buffers, arrival counters
    DevBuf tpo, tpd, tpa;                  // XCD-local schedule: o_proj, down and attention split partials
    bool xcd_ok = false;                   // the XCD-local schedule takes this model
    uint32_t xcd_parity = 0;               // epoch parity of the partials' last writes (0: as zeroed)
    int xnsm = 0;                          // attention split slots per (layer, kv head) in tpa
    DevBuf img, hflag, hubtab;             // per-XCD hub images, their flags, hub XCC ids
    int img_stride = 0, nflag = 0;
};

namespace {

int layer_scratch(ming_ctx* ctx, DevBuf& part, size_t floats) {
    return hip_check(ctx, part.ensure(floats * sizeof(float)), "hipMalloc(attention partials)");
}

}  // namespace

ming::LinearDev ming::linear_dev(const ming_linear& l) { return to_dev(l); }
int ming::check_linear_w(ming_ctx* ctx, const ming_linear& l, int N, int K, const char* name) {
    return check_linear(ctx, l, N, K, name);
}

bool ming::lm_model_view(const ming_lm_model* m, LmView& v) {
    if (!m || !m->ctx) return false;
    v.cfg = m->cfg;
    v.layers = m->layers.data();
    v.head = m->head;
    v.embed = m->embed;
    v.final_norm = m->final_norm;
    return true;
}

extern "C" {

// ---- context ------------------------------------------------------------------

int ming_ctx_create(ming_ctx** out, int device) {
    if (!out) return MING_E_ARG;
    *out = nullptr;
    auto* c = new ming_ctx;
    c->device = device;
    hipError_t e = hipSetDevice(device);
    if (e == hipSuccess) e = hipStreamCreateWithFlags(&c->own_stream, hipStreamNonBlocking);
    if (e == hipSuccess) e = hipMalloc(&c->dev_flags, 64);
    if (e == hipSuccess) e = hipMemset(c->dev_flags, 0, 64);
    // gelu's tanh table in the DiT kernels' device arrays (once per device)
    if (e == hipSuccess) e = tanh_tables_init(device);
    hipDeviceProp_t prop{};
    if (e == hipSuccess) e = hipGetDeviceProperties(&prop, device);
    if (e != hipSuccess) {
        if (c->dev_flags) (void)hipFree(c->dev_flags);
        if (c->own_stream) (void)hipStreamDestroy(c->own_stream);
        delete c;
        return MING_E_HIP;
    }
    c->num_cus = prop.multiProcessorCount;
    c->max_lds = prop.sharedMemPerBlock;
    // this device's fixed scratch (ming_qgemm_noalloc); resolved once per
    // device with the device current.  A failure only disables that entry point.
    if (scratch_init(device) == hipSuccess) c->scratch = scratch_ptr(device);
    c->stream = c->own_stream;
    c->alive = true;
    *out = c;
    return MING_OK;
}

int ming_ctx_destroy(ming_ctx* ctx) {
    if (!alive(ctx)) return MING_E_NOT_INIT;
    (void)hipStreamSynchronize(ctx->stream);
    ctx->part.release();
    ctx->qstage.release();
    if (ctx->dev_flags) (void)hipFree(ctx->dev_flags);
    if (ctx->own_stream) (void)hipStreamDestroy(ctx->own_stream);
    ctx->alive = false;
    delete ctx;
    return MING_OK;
}

int ming_ctx_set_stream(ming_ctx* ctx, void* s) {
    if (!alive(ctx)) return MING_E_NOT_INIT;
    ctx->stream = static_cast<hipStream_t>(s);
    return MING_OK;
}

int ming_ctx_use_own_stream(ming_ctx* ctx) {
    if (!alive(ctx)) return MING_E_NOT_INIT;
    ctx->stream = ctx->own_stream;
    return MING_OK;
}

int ming_ctx_set_exclusive(ming_ctx* ctx, int on) {
    if (!alive(ctx)) return MING_E_NOT_INIT;
    ctx->exclusive = on != 0;
    return MING_OK;
}

int ming_ctx_workspace_bytes(const ming_ctx* ctx, int64_t* bytes) {
    if (!ctx || !ctx->alive) return MING_E_NOT_INIT;
    if (!bytes) return MING_E_ARG;
    *bytes = (int64_t)(ctx->qstage.bytes + ctx->part.bytes);
    return MING_OK;
}

void* ming_ctx_stream(ming_ctx* ctx) { return alive(ctx) ? ctx->stream : nullptr; }

int ming_sync(ming_ctx* ctx) {
    if (!alive(ctx)) return MING_E_NOT_INIT;
    int st = hip_check(ctx, hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
    if (st) return st;
    int32_t flag = 0;
    st = hip_check(ctx, hipMemcpy(&flag, ctx->dev_flags, sizeof(flag), hipMemcpyDeviceToHost), "read error flag");
    if (st) return st;
    if (flag) {
        (void)hipMemset(ctx->dev_flags, 0, sizeof(int32_t));
        ctx->timeout_seen = true;
        return set_err(ctx, MING_E_TIMEOUT, "a device-side wait exceeded its spin limit");
    }
    // [2]: a gather_qmm index outside its range
    st = hip_check(ctx, hipMemcpy(&flag, ctx->dev_flags + 2, sizeof(flag), hipMemcpyDeviceToHost), "read error flag");
    if (st) return st;
    if (flag) {
        (void)hipMemset(ctx->dev_flags + 2, 0, sizeof(int32_t));
        return set_err(ctx, MING_E_ARG, "gather_qmm: an lhs/rhs index outside its range (those pairs left unwritten)");
    }
    // [1]: a batched step met a position or page id outside its paged cache
    st = hip_check(ctx, hipMemcpy(&flag, ctx->dev_flags + 1, sizeof(flag), hipMemcpyDeviceToHost), "read error flag");
    if (st) return st;
    if (flag) {
        (void)hipMemset(ctx->dev_flags + 1, 0, sizeof(int32_t));
        return set_err(ctx, MING_E_CTX_OVER_CAPACITY,
                       "a batched step met a position or page id outside its paged cache (append and attention skipped)");
    }
    return MING_OK;
}

const char* ming_last_error(ming_ctx* ctx) { return alive(ctx) ? ctx->err.c_str() : "context not initialised"; }

const char* ming_status_str(int s) {
    switch (s) {
        case MING_OK: return "ok";
        case MING_E_SHAPE: return "shape";
        case MING_E_CTX_OVER_CAPACITY: return "context over capacity";
        case MING_E_HIP: return "hip error";
        case MING_E_NOT_INIT: return "not initialised";
        case MING_E_ARG: return "invalid argument";
        case MING_E_UNSUPPORTED: return "unsupported";
        case MING_E_TIMEOUT: return "device wait timeout";
    }
    return "unknown";
}

int ming_fused_enabled(void) { return !g_force_off && !env_off("MING_FUSED"); }
int ming_dit_enabled(void) { return ming_fused_enabled() && !env_off("MING_FUSED_DIT"); }
int ming_lm_enabled(void) { return ming_fused_enabled() && !env_off("MING_FUSED_LM"); }
void ming_set_force_off(int off) { g_force_off = off != 0; }

// ---- memory ---------------------------------------------------------------------

int ming_malloc(ming_ctx* ctx, size_t bytes, void** out) {
    if (!alive(ctx)) return MING_E_NOT_INIT;
    if (!out) return set_err(ctx, MING_E_ARG, "null out");
    return hip_check(ctx, hipMalloc(out, bytes ? bytes : 1), "hipMalloc");
}
int ming_free(ming_ctx* ctx, void* p) {
    if (!alive(ctx)) return MING_E_NOT_INIT;
    return hip_check(ctx, hipFree(p), "hipFree");
}
int ming_memcpy_htod(ming_ctx* ctx, void* dst, const void* src, size_t n) {
    if (!alive(ctx)) return MING_E_NOT_INIT;
    return hip_check(ctx, hipMemcpyAsync(dst, src, n, hipMemcpyHostToDevice, ctx->stream), "hipMemcpy H2D");
}
int ming_memcpy_dtoh(ming_ctx* ctx, void* dst, const void* src, size_t n) {
    if (!alive(ctx)) return MING_E_NOT_INIT;
    int st = hip_check(ctx, hipMemcpyAsync(dst, src, n, hipMemcpyDeviceToHost, ctx->stream), "hipMemcpy D2H");
    if (st) return st;
    return hip_check(ctx, hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
}
int ming_memset(ming_ctx* ctx, void* dst, int v, size_t n) {
    if (!alive(ctx)) return MING_E_NOT_INIT;
    return hip_check(ctx, hipMemsetAsync(dst, v, n, ctx->stream), "hipMemset");
}

// ---- quantized linear algebra ---------------------------------------------------

static int qgemv_impl(ming_ctx* ctx, const ming_tensor* x, const ming_tensor* w, const ming_tensor* s,
                      const ming_tensor* b, float g, int32_t gs, int32_t bits, ming_tensor* y, bool f32) {
    if (!alive(ctx)) return MING_E_NOT_INIT;
    int64_t N, K;
    int st = check_affine(ctx, w, s, b, gs, bits, N, K);
    if (st) return st;
    int64_t xm, xk, ym, yn;
    if (!as_2d(x, xm, xk) || !as_2d(y, ym, yn)) return set_err(ctx, MING_E_SHAPE, "qgemv: x/y must be 1-D or 2-D");
    if (x->dtype != MING_DT_BF16) return set_err(ctx, MING_E_SHAPE, "qgemv: x must be bf16");
    if (y->dtype != (f32 ? MING_DT_F32 : MING_DT_BF16))
        return set_err(ctx, MING_E_SHAPE, f32 ? "qgemv_f32: y must be f32" : "qgemv: y must be bf16");
    if (xk != K || ym != xm || yn != N)
        return set_err(ctx, MING_E_SHAPE, "qgemv: x " + shape_str(x) + " / y " + shape_str(y) +
                                              " do not match w [" + std::to_string(N) + "," + std::to_string(K) + "]");
    if (xm < 1 || xm > 8) return set_err(ctx, MING_E_UNSUPPORTED, "qgemv: 1..8 activation rows");
    if (K > 16384) return set_err(ctx, MING_E_UNSUPPORTED, "qgemv: K > 16384");
    if (N > INT32_MAX) return set_err(ctx, MING_E_UNSUPPORTED, "qgemv: N too large");
    return hip_check(ctx,
                     launch_qgemv(ctx->stream, (int)xm, static_cast<const uint16_t*>(x->data),
                                  static_cast<const uint32_t*>(w->data), static_cast<const uint16_t*>(s->data),
                                  static_cast<const uint16_t*>(b->data), (int)N, (int)K, g,
                                  f32 ? nullptr : static_cast<uint16_t*>(y->data),
                                  f32 ? static_cast<float*>(y->data) : nullptr),
                     "qgemv launch");
}

int ming_qgemv(ming_ctx* ctx, const ming_tensor* x, const ming_tensor* w, const ming_tensor* s, const ming_tensor* b,
               float g, int32_t gs, int32_t bits, ming_tensor* y) {
    return qgemv_impl(ctx, x, w, s, b, g, gs, bits, y, false);
}

int ming_qgemv_f32(ming_ctx* ctx, const ming_tensor* x, const ming_tensor* w, const ming_tensor* s,
                   const ming_tensor* b, float g, int32_t gs, int32_t bits, ming_tensor* y) {
    return qgemv_impl(ctx, x, w, s, b, g, gs, bits, y, true);
}

// Batched rows (mlx_quantized_matmul with M > 1, src/mlx.zig:279-282): MFMA GEMM over
// activations staged once per call into the context's growable buffer
// (ming_qgemm) or, with fixed_cap > 0, into `fixed`, the device's fixed
// scratch (ming_qgemm_noalloc: nothing is allocated, and requests that need
// more than fixed_cap bytes are rejected before anything is launched).
static int qgemm_impl(ming_ctx* ctx, const ming_tensor* x, const ming_tensor* w, const ming_tensor* s,
                      const ming_tensor* b, float g, int32_t gs, int32_t bits, ming_tensor* y, void* fixed,
                      size_t fixed_cap, const char* name) {
    if (!alive(ctx)) return MING_E_NOT_INIT;
    const std::string nm(name);
    int64_t N, K;
    int st = check_affine(ctx, w, s, b, gs, bits, N, K);
    if (st) return st;
    int64_t xm, xk, ym, yn;
    if (!as_2d(x, xm, xk) || !as_2d(y, ym, yn)) return set_err(ctx, MING_E_SHAPE, nm + ": x/y must be 1-D or 2-D");
    if (x->dtype != MING_DT_BF16) return set_err(ctx, MING_E_SHAPE, nm + ": x must be bf16");
    if (y->dtype != MING_DT_F32 && y->dtype != MING_DT_BF16) return set_err(ctx, MING_E_SHAPE, nm + ": y must be bf16 or f32");
    if (xk != K || ym != xm || yn != N)
        return set_err(ctx, MING_E_SHAPE, nm + ": x " + shape_str(x) + " / y " + shape_str(y) +
                                              " do not match w [" + std::to_string(N) + "," + std::to_string(K) + "]");
    if (xm < 1 || xm > 64) return set_err(ctx, MING_E_UNSUPPORTED, nm + ": 1..64 activation rows");
    if (N > INT32_MAX / 64 || K > 65536) return set_err(ctx, MING_E_UNSUPPORTED, nm + ": N or K too large");
    const int M = (int)xm, Mp = (M + 15) / 16 * 16;
    const size_t xs_bytes = (size_t)Mp * K * 2, need = xs_bytes + (size_t)Mp * (K / 64) * sizeof(float);
    void* xs = fixed;
    if (fixed_cap) {
        if (!fixed) return set_err(ctx, MING_E_HIP, nm + ": the device's fixed scratch could not be resolved");
        if (need > fixed_cap)
            return set_err(ctx, MING_E_UNSUPPORTED,
                           nm + ": staging " + std::to_string(M) + " x " + std::to_string(K) + " rows needs " +
                               std::to_string(need) + " bytes, over the fixed scratch of " +
                               std::to_string(fixed_cap) + " bytes (at most 64 rows of K <= 8192)");
    } else {
        if ((st = hip_check(ctx, ctx->qstage.ensure(need), "hipMalloc(qgemm staging)"))) return st;
        xs = ctx->qstage.p;
    }
    float* xsum = reinterpret_cast<float*>(static_cast<char*>(xs) + xs_bytes);
    if ((st = hip_check(ctx,
                        launch_stage(ctx->stream, static_cast<const uint16_t*>(x->data), (int)K, M, (int)K, nullptr,
                                     0.0f, xs, xsum, nullptr, nullptr),
                        "qgemm staging launch")))
        return st;
    const bool f32 = y->dtype == MING_DT_F32;
    QgemmArgs a{};
    a.xs = xs;
    a.xsum = xsum;
    a.M = M;
    a.K = (int)K;
    a.nseg = 1;
    a.seg[0] = QSeg{static_cast<const uint32_t*>(w->data), static_cast<const uint16_t*>(s->data),
                    static_cast<const uint16_t*>(b->data), nullptr, (int)N, 0, g};
    a.y = f32 ? nullptr : static_cast<uint16_t*>(y->data);
    a.yf = f32 ? static_cast<float*>(y->data) : nullptr;
    a.ldy = (int)N;
    return hip_check(ctx, launch_qgemm_epi(ctx->stream, a, QE_PLAIN), "qgemm launch");
}

int ming_qgemm(ming_ctx* ctx, const ming_tensor* x, const ming_tensor* w, const ming_tensor* s, const ming_tensor* b,
               float g, int32_t gs, int32_t bits, ming_tensor* y) {
    return qgemm_impl(ctx, x, w, s, b, g, gs, bits, y, nullptr, 0, "qgemm");
}

int ming_qgemm_noalloc(ming_ctx* ctx, const ming_tensor* x, const ming_tensor* w, const ming_tensor* s,
                       const ming_tensor* b, float g, int32_t gs, int32_t bits, ming_tensor* y) {
    if (!alive(ctx)) return MING_E_NOT_INIT;
    return qgemm_impl(ctx, x, w, s, b, g, gs, bits, y, ctx->scratch, scratch_bytes(), "qgemm_noalloc");
}

namespace {

// Leading dims folded into one batch count: t viewed as [batch][rows][cols].
bool as_3d(const ming_tensor* t, int64_t& batch, int64_t& rows, int64_t& cols) {
    if (!t || !t->data || t->ndim < 2 || t->ndim > 4) return false;
    batch = 1;
    for (int i = 0; i < t->ndim - 2; i++) batch *= t->shape[i];
    rows = t->shape[t->ndim - 2];
    cols = t->shape[t->ndim - 1];
    return batch >= 1 && rows >= 1 && cols >= 1;
}

int64_t numel_of(const ming_tensor* t) {
    int64_t n = 1;
    for (int i = 0; i < t->ndim; i++) n *= t->shape[i];
    return n;
}

}  // namespace

// mlx_gather_qmm (src/mlx.zig:282) with the global scale of the mlx-c patch
// (patches/mlxc-gather-qmm-global-scale.patch:10-18).
int ming_gather_qmm(ming_ctx* ctx, const ming_tensor* x, const ming_tensor* w, const ming_tensor* s,
                    const ming_tensor* b, const ming_tensor* lhs, const ming_tensor* rhs, int32_t transpose_w,
                    int32_t gs, int32_t bits, float g, int32_t sorted_indices, ming_tensor* y) {
    if (!alive(ctx)) return MING_E_NOT_INIT;
    if (!transpose_w) return set_err(ctx, MING_E_UNSUPPORTED, "gather_qmm: only transpose_w = true ([N, K] weights)");
    if (bits != 4 || gs != 64)
        return set_err(ctx, MING_E_UNSUPPORTED, "gather_qmm: only bits=4, group_size=64 are implemented");
    int64_t E, N, KW, Es, Ns, G, Eb, Nb, Gb;
    if (!as_3d(w, E, N, KW) || !as_3d(s, Es, Ns, G) || !as_3d(b, Eb, Nb, Gb))
        return set_err(ctx, MING_E_SHAPE, "gather_qmm: w/scales/biases must be [..., N, K/8] / [..., N, K/64] device tensors");
    if (w->dtype != MING_DT_U32 || s->dtype != MING_DT_BF16 || b->dtype != MING_DT_BF16)
        return set_err(ctx, MING_E_SHAPE, "gather_qmm: w must be u32, scales/biases bf16");
    const int64_t K = KW * 8;
    if (Es != E || Eb != E || Ns != N || Nb != N || G != K / 64 || Gb != K / 64 || K % 64)
        return set_err(ctx, MING_E_SHAPE, "gather_qmm: scales/biases " + shape_str(s) + " do not match w " + shape_str(w));
    int64_t Bx, M, xk;
    if (!as_3d(x, Bx, M, xk) || x->dtype != MING_DT_BF16)
        return set_err(ctx, MING_E_SHAPE, "gather_qmm: x must be a bf16 [..., M, K] device tensor");
    if (xk != K) return set_err(ctx, MING_E_SHAPE, "gather_qmm: x " + shape_str(x) + " does not match K " + std::to_string(K));
    if (!rhs || !rhs->data || rhs->dtype != MING_DT_I32)
        return set_err(ctx, MING_E_ARG, "gather_qmm: rhs_indices must be an i32 device tensor");
    const int64_t P = numel_of(rhs);
    const bool has_lhs = lhs && lhs->data;
    if (has_lhs && (lhs->dtype != MING_DT_I32 || numel_of(lhs) != P))
        return set_err(ctx, MING_E_SHAPE, "gather_qmm: lhs_indices must be i32 with as many entries as rhs_indices");
    if (!has_lhs && Bx != 1 && Bx != P)
        return set_err(ctx, MING_E_SHAPE, "gather_qmm: without lhs_indices, x needs one batch entry or one per pair");
    int64_t yp, ym, yn;
    bool yok = as_3d(y, yp, ym, yn) && yp * ym == P * M && yn == N;
    if (yok && y->ndim == 2) yok = M == 1 || yp == 1;  // [P, N] for M = 1 (folded batch 1 otherwise)
    if (!yok || (y->dtype != MING_DT_BF16 && y->dtype != MING_DT_F32))
        return set_err(ctx, MING_E_SHAPE, "gather_qmm: y must be bf16 or f32 [P, M, N] (or [P, N] for M = 1), got " +
                                              (y ? shape_str(y) : std::string("null")));
    if (P < 1) return set_err(ctx, MING_E_ARG, "gather_qmm: no index pairs");
    if (K > 16384 || M > gather_vectors((int)K))
        return set_err(ctx, MING_E_UNSUPPORTED, "gather_qmm: K <= 16384 and M <= " + std::to_string(gather_vectors((int)K)) +
                                                    " rows per pair at this K");
    if (N > INT32_MAX || P > INT32_MAX / 2 || Bx > INT32_MAX || E > INT32_MAX)
        return set_err(ctx, MING_E_UNSUPPORTED, "gather_qmm: sizes too large");
    const bool f32 = y->dtype == MING_DT_F32;
    return hip_check(ctx,
                     launch_gather_qmm(ctx->stream, static_cast<const uint16_t*>(x->data),
                                       static_cast<const uint32_t*>(w->data), static_cast<const uint16_t*>(s->data),
                                       static_cast<const uint16_t*>(b->data),
                                       has_lhs ? static_cast<const int32_t*>(lhs->data) : nullptr,
                                       static_cast<const int32_t*>(rhs->data), (int)P, (int)Bx, (int)E, (int)M, (int)N,
                                       (int)K, g, sorted_indices != 0, ctx->dev_flags,
                                       f32 ? nullptr : static_cast<uint16_t*>(y->data),
                                       f32 ? static_cast<float*>(y->data) : nullptr),
                     "gather_qmm launch");
}

int ming_dequantize(ming_ctx* ctx, const ming_tensor* w, const ming_tensor* s, const ming_tensor* b, int32_t gs,
                    int32_t bits, float g, ming_tensor* out) {
    if (!alive(ctx)) return MING_E_NOT_INIT;
    int64_t N, K, orr, oc;
    int st = check_affine(ctx, w, s, b, gs, bits, N, K);
    if (st) return st;
    if (!as_2d(out, orr, oc) || out->dtype != MING_DT_BF16 || orr != N || oc != K)
        return set_err(ctx, MING_E_SHAPE, "dequantize: out must be bf16 [N, K]");
    return hip_check(ctx,
                     launch_dequantize(ctx->stream, static_cast<const uint32_t*>(w->data),
                                       static_cast<const uint16_t*>(s->data), static_cast<const uint16_t*>(b->data), N,
                                       K, g, static_cast<uint16_t*>(out->data)),
                     "dequantize launch");
}

int ming_quantize(ming_ctx* ctx, const ming_tensor* w, int32_t gs, int32_t bits, float g, ming_tensor* wq,
                  ming_tensor* s, ming_tensor* b) {
    if (!alive(ctx)) return MING_E_NOT_INIT;
    if (!(g > 0.0f) || !std::isfinite(g))
        return set_err(ctx, MING_E_ARG, "quantize: global_scale must be finite and > 0");
    if (bits != 4 || gs != 64)
        return set_err(ctx, MING_E_UNSUPPORTED, "quantize: only bits=4, group_size=64 are implemented");
    int64_t N, K, qn, qk;
    if (!as_2d(w, N, K) || w->dtype != MING_DT_BF16) return set_err(ctx, MING_E_SHAPE, "quantize: w must be bf16 2-D");
    if (K % 64) return set_err(ctx, MING_E_SHAPE, "quantize: K % 64 != 0");
    int64_t sn, sk, bn, bk;
    if (!as_2d(wq, qn, qk) || !as_2d(s, sn, sk) || !as_2d(b, bn, bk) || wq->dtype != MING_DT_U32 ||
        s->dtype != MING_DT_BF16 || b->dtype != MING_DT_BF16 || qn != N || qk != K / 8 || sn != N || bn != N ||
        sk != K / 64 || bk != K / 64)
        return set_err(ctx, MING_E_SHAPE, "quantize: outputs must be u32 [N,K/8], bf16 [N,K/64] x2");
    return hip_check(ctx,
                     launch_quantize(ctx->stream, static_cast<const uint16_t*>(w->data), N, K, g,
                                     static_cast<uint32_t*>(wq->data), static_cast<uint16_t*>(s->data),
                                     static_cast<uint16_t*>(b->data)),
                     "quantize launch");
}

// ---- Qwen2 decode ----------------------------------------------------------------

static StepArgs base_args(const ming_lm_cfg* c) {
    StepArgs a;
    std::memset(&a, 0, sizeof(a));
    a.n_layers = c->n_layers;
    a.H = c->hidden;
    a.heads = c->heads;
    a.kvh = c->kv_heads;
    a.hd = c->head_dim;
    a.I = c->inter;
    a.eps = c->eps;
    a.log2_theta = c->log2_theta;
    return a;
}

int ming_lm_layer(ming_ctx* ctx, const ming_lm_cfg* cfg, const ming_lm_layer_w* l, const void* x, int32_t pos,
                  ming_kv* kv, int32_t layer, ming_lm_out* out) {
    if (!alive(ctx)) return MING_E_NOT_INIT;
    int st;
    if ((st = check_cfg(ctx, cfg)) || (st = check_layer(ctx, cfg, l))) return st;
    if (!x || !out || !out->qkv || !out->o || !out->x1 || !out->hh || !out->x2)
        return set_err(ctx, MING_E_ARG, "lm_layer: null input or output buffer");
    if (!kv || !kv->k || !kv->v || kv->kv_heads != cfg->kv_heads || kv->head_dim != cfg->head_dim)
        return set_err(ctx, MING_E_SHAPE, "lm_layer: kv cache geometry does not match");
    if (layer < 0 || layer >= kv->n_layers) return set_err(ctx, MING_E_ARG, "lm_layer: layer out of range");
    if (pos < 0) return set_err(ctx, MING_E_ARG, "lm_layer: pos < 0");
    if (pos >= kv->capacity)
        return set_err(ctx, MING_E_CTX_OVER_CAPACITY, "lm_layer: pos " + std::to_string(pos) +
                                                          " >= capacity " + std::to_string(kv->capacity));
    StepArgs a = base_args(cfg);
    a.kc = static_cast<uint16_t*>(kv->k);
    a.vc = static_cast<uint16_t*>(kv->v);
    a.cap = kv->capacity;
    a.pos = pos;
    a.x = const_cast<uint16_t*>(static_cast<const uint16_t*>(x));
    a.xo = static_cast<uint16_t*>(out->x2);
    a.x1 = static_cast<uint16_t*>(out->x1);
    a.att = static_cast<uint16_t*>(out->o);
    a.qkv = static_cast<uint16_t*>(out->qkv);
    a.hh = static_cast<uint16_t*>(out->hh);
    a.sx = a.sq = a.sh = 0;
    a.split_len = attn_split_len(pos + 1);
    if ((st = layer_scratch(ctx, ctx->part, attn_part_floats(cfg->kv_heads, cfg->heads, cfg->head_dim, pos + 1))))
        return st;
    a.part = static_cast<float*>(ctx->part.p);
    a.flags = ctx->dev_flags;
    const LayerDev Ld = layer_dev(l);
    return hip_check(ctx, launch_lm_layer(ctx->stream, a, Ld, layer), "lm_layer launch");
}

int ming_lm_model_create(ming_ctx* ctx, const ming_lm_cfg* cfg, const ming_lm_layer_w* layers,
                         const void* final_norm, const ming_linear* head, const ming_linear* embed,
                         ming_lm_model** out) {
    if (!alive(ctx)) return MING_E_NOT_INIT;
    if (!out) return set_err(ctx, MING_E_ARG, "null out");
    *out = nullptr;
    int st;
    if ((st = check_cfg(ctx, cfg))) return st;
    if (!layers || !final_norm || !head || !embed) return set_err(ctx, MING_E_ARG, "lm_model: null argument");
    for (int i = 0; i < cfg->n_layers; i++)
        if ((st = check_layer(ctx, cfg, &layers[i]))) return set_err(ctx, st, "layer " + std::to_string(i) + ": " + ctx->err);
    if ((st = check_linear(ctx, *head, cfg->vocab, cfg->hidden, "head")) ||
        (st = check_linear(ctx, *embed, cfg->vocab, cfg->hidden, "embed")))
        return st;
    for (int i = 0; i < cfg->n_layers; i++)
        if (layers[i].wq.kind != head->kind)
            return set_err(ctx, MING_E_UNSUPPORTED, "the LM head and every layer must share one weight kind");
    auto* m = new ming_lm_model;
    m->ctx = ctx;
    m->cfg = *cfg;
    for (int i = 0; i < cfg->n_layers; i++) m->layers.push_back(layer_dev(&layers[i]));
    m->head = to_dev(*head);
    m->embed = to_dev(*embed);
    m->final_norm = static_cast<const uint16_t*>(final_norm);
    const int H = cfg->hidden, I = cfg->inter, L = cfg->n_layers, nq = H + 2 * cfg->kv_heads * cfg->head_dim;
    hipError_t e = hipMalloc(&m->d_layers, sizeof(LayerDev) * L);
    if (e == hipSuccess)
        e = hipMemcpy(m->d_layers, m->layers.data(), sizeof(LayerDev) * L, hipMemcpyHostToDevice);
    if (e == hipSuccess) e = m->x.ensure(sizeof(uint16_t) * (size_t)(L + 1) * H);
    if (e == hipSuccess) e = m->x1.ensure(sizeof(uint16_t) * (size_t)L * H);
    if (e == hipSuccess) e = m->att.ensure(sizeof(uint16_t) * (size_t)L * H);
    if (e == hipSuccess) e = m->qkv.ensure(sizeof(uint16_t) * (size_t)L * nq);
    if (e == hipSuccess) e = m->hh.ensure(sizeof(uint16_t) * (size_t)L * I);
    if (e == hipSuccess) e = m->hidden.ensure(sizeof(uint16_t) * (size_t)H);
    if (e == hipSuccess) e = m->amax_v.ensure(sizeof(float) * kMaxParts);
    if (e == hipSuccess) e = m->amax_i.ensure(sizeof(int32_t) * kMaxParts);
    if (e == hipSuccess) e = m->tx.ensure(sizeof(uint64_t) * (size_t)(L + 1) * (H / 2));
    if (e == hipSuccess) e = m->tq.ensure(sizeof(uint64_t) * (size_t)L * (nq / 2));
    if (e == hipSuccess) e = m->ta.ensure(sizeof(uint64_t) * (size_t)L * (H / 2));
    if (e == hipSuccess) e = m->tx1.ensure(sizeof(uint64_t) * (size_t)L * (H / 2));
    if (e == hipSuccess) e = m->th.ensure(sizeof(uint64_t) * (size_t)L * (I / 2));
    if (e == hipSuccess) e = m->counters.ensure(sizeof(int32_t) * (size_t)(2 * L * cfg->kv_heads + 1));
    if (e == hipSuccess) e = m->tpo.ensure(sizeof(uint32_t) * (size_t)L * cfg->kv_heads * H);
    if (e == hipSuccess) e = m->tpd.ensure(sizeof(uint32_t) * (size_t)L * kMaxHubs * H);
    m->pgrid = tagged_grid(ctx->num_cus);
    m->xnsm = m->pgrid / kMaxHubs - 1;  // the attention splits of a kv head on one XCD slot's workers
    if (e == hipSuccess && m->xnsm > 0)
        e = m->tpa.ensure(sizeof(uint64_t) * (size_t)L * cfg->kv_heads * m->xnsm * (cfg->heads / cfg->kv_heads) *
                          (cfg->head_dim + 2));
    m->img_stride = tagged_img_stride(H, I);
    m->nflag = (4 * L + 1 + 31) / 32 * 32;  // whole 128-byte lines per hub
    if (e == hipSuccess) e = m->img.ensure(sizeof(uint32_t) * (size_t)kMaxHubs * kImgSlots * m->img_stride);
    if (e == hipSuccess) e = m->hflag.ensure(sizeof(uint32_t) * (size_t)kMaxHubs * m->nflag);
    if (e == hipSuccess) e = m->hubtab.ensure(sizeof(uint64_t) * (kXcdBase + kXcdSlots));
    for (DevBuf* b :
         {&m->tx, &m->tq, &m->ta, &m->tx1, &m->th, &m->counters, &m->img, &m->hflag, &m->hubtab, &m->tpo, &m->tpd,
          &m->tpa})
        if (e == hipSuccess && b->p) e = hipMemset(b->p, 0, b->bytes);
    if (e != hipSuccess) {
        ming_lm_model_destroy(m);
        return hip_check(ctx, e, "lm_model workspace");
    }
    // the XCD-local kernel is instantiated for one weight format throughout (as the first schedule's)
    bool same_kind = true;
    for (const LayerDev& ld : m->layers)
        for (const LinearDev* l : {&ld.q, &ld.k, &ld.v, &ld.o, &ld.g, &ld.u, &ld.d})
            same_kind = same_kind && l->kind == m->head.kind;
    m->xcd_ok = same_kind && m->pgrid > 0 &&
                xcd_fits(m->head.kind == 1, m->pgrid, H, cfg->heads, cfg->kv_heads, cfg->head_dim, I, L);
    *out = m;
    return MING_OK;
}

int ming_lm_model_destroy(ming_lm_model* m) {
    if (!m) return MING_E_NOT_INIT;
    if (m->d_layers) (void)hipFree(m->d_layers);
    for (DevBuf* b : {&m->x, &m->x1, &m->att, &m->qkv, &m->hh, &m->part, &m->hidden, &m->amax_v, &m->amax_i,
                      &m->tx, &m->tq, &m->ta, &m->tx1, &m->th, &m->counters, &m->img, &m->hflag, &m->hubtab,
                      &m->tpo, &m->tpd, &m->tpa})
        b->release();
    delete m;
    return MING_OK;
}

int ming_lm_model_profile(ming_lm_model* m, void* stamps_dev) {
    if (!m) return MING_E_NOT_INIT;
    m->tstamp = static_cast<uint64_t*>(stamps_dev);
    return MING_OK;
}

int ming_lm_model_profile_shape(ming_lm_model* m, int32_t* n_stamps, int32_t* grid) {
    if (!m) return MING_E_NOT_INIT;
    if (n_stamps) *n_stamps = 3 + 10 * m->cfg.n_layers;
    if (grid) *grid = m->pgrid;
    return MING_OK;
}

int ming_lm_model_set_mode(ming_lm_model* m, int32_t mode) {
    if (!m) return MING_E_NOT_INIT;
    if (mode < MING_LM_AUTO || mode > MING_LM_PERSISTENT_XCD) return set_err(m->ctx, MING_E_ARG, "unknown mode");
    m->mode = mode;
    return MING_OK;
}

int ming_lm_model_trace(ming_lm_model* m, void* x, void* x1, void* att, void* qkv, void* hh) {
    if (!m || !alive(m->ctx)) return MING_E_NOT_INIT;
    const ming_lm_cfg* c = &m->cfg;
    const size_t H = c->hidden, L = c->n_layers, nq = H + 2 * c->kv_heads * c->head_dim;
    struct {
        void* dst;
        const DevBuf* src;
        size_t n;
    } cp[] = {{x, &m->x, (L + 1) * H}, {x1, &m->x1, L * H}, {att, &m->att, L * H}, {qkv, &m->qkv, L * nq},
              {hh, &m->hh, L * (size_t)c->inter}};
    for (auto& e : cp) {
        if (!e.dst) continue;
        int st = hip_check(m->ctx, hipMemcpyAsync(e.dst, e.src->p, e.n * sizeof(uint16_t), hipMemcpyDeviceToDevice,
                                                  m->ctx->stream),
                           "trace copy");
        if (st) return st;
    }
    return MING_OK;
}

static int lm_step_impl(ming_ctx* ctx, ming_lm_model* m, const int32_t* token_dev, const void* x_in, ming_kv* kv,
                        void* hidden_out, float* logits_out, int32_t* argmax_out) {
    int st;
    if ((st = check_kv(ctx, &m->cfg, kv))) return st;
    if (!token_dev && !x_in) return set_err(ctx, MING_E_ARG, "lm_step: need a token or an input row");
    const ming_lm_cfg* c = &m->cfg;
    StepArgs a = base_args(c);
    a.layers = m->d_layers;
    a.final_norm = m->final_norm;
    a.head = m->head;
    a.embed = m->embed;
    a.kc = static_cast<uint16_t*>(kv->k);
    a.vc = static_cast<uint16_t*>(kv->v);
    a.cap = kv->capacity;
    a.pos = kv->len;
    a.token_in = token_dev;
    a.argmax_out = argmax_out;
    a.x = static_cast<uint16_t*>(m->x.p);
    a.xo = a.x + c->hidden;
    a.x1 = static_cast<uint16_t*>(m->x1.p);
    a.att = static_cast<uint16_t*>(m->att.p);
    a.qkv = static_cast<uint16_t*>(m->qkv.p);
    a.hh = static_cast<uint16_t*>(m->hh.p);
    a.sx = c->hidden;
    a.sq = c->hidden + 2 * c->kv_heads * c->head_dim;
    a.sh = c->inter;
    a.split_len = attn_split_len(kv->len + 1);
    const size_t pf = attn_part_floats(c->kv_heads, c->heads, c->head_dim, kv->capacity);
    if ((st = hip_check(ctx, m->part.ensure(pf * sizeof(float)), "hipMalloc(attention partials)"))) return st;
    a.part = static_cast<float*>(m->part.p);
    a.hidden = hidden_out ? static_cast<uint16_t*>(hidden_out) : static_cast<uint16_t*>(m->hidden.p);
    a.logits = logits_out;
    a.amax_v = static_cast<float*>(m->amax_v.p);
    a.amax_i = static_cast<int32_t*>(m->amax_i.p);
    a.flags = ctx->dev_flags;
    if (!token_dev && x_in != a.x &&
        (st = hip_check(ctx,
                        hipMemcpyAsync(a.x, x_in, sizeof(uint16_t) * c->hidden, hipMemcpyDeviceToDevice, ctx->stream),
                        "copy x_in")))
        return st;
    // The persistent schedule runs every attention split (a workgroup's
    // LDS-resident K/V rows) on its own workgroup, on workgroups that do not
    // also run q/k/v, o_proj or down (the first ones).
    const int tsl = tagged_split_len(kv->len + 1);
    const int nsplit = (kv->len + 1 + tsl - 1) / tsl;
    const bool want_persistent =
        m->mode == MING_LM_PERSISTENT || m->mode == MING_LM_PERSISTENT_DIRECT || m->mode == MING_LM_AUTO;
    const int nhubs = m->mode == MING_LM_PERSISTENT_DIRECT ? 0 : tagged_hubs(m->pgrid);
    const int workers = m->pgrid - nhubs;
    const int nq = c->hidden + 2 * c->kv_heads * c->head_dim;
    const int upw = tagged_units_per_worker();
    const int front = std::max((nq / 4 + upw - 1) / upw, (c->hidden / 2 + upw - 1) / upw);  // q/k/v, o/down workers
    const bool fits = m->pgrid > 0 && c->head_dim == 64 && c->heads / c->kv_heads <= 8 &&
                      c->kv_heads * nsplit + front <= workers && c->n_layers <= tagged_max_layers();
    const bool persistent = want_persistent && fits;
    if (want_persistent && m->mode != MING_LM_AUTO && !fits)
        return set_err(ctx, MING_E_UNSUPPORTED, "lm_step: context too long for the persistent schedule");
    // The XCD-local schedule: kv head g's splits on ranks 31..32-nsplit of slot 7-g.
    const bool xfits = m->xcd_ok && nsplit <= m->pgrid / kMaxHubs - 1;
    if (m->mode == MING_LM_PERSISTENT_XCD && !xfits)
        return set_err(ctx, MING_E_UNSUPPORTED, "lm_step: shape or context outside the XCD-local schedule");
    if (xfits && (m->mode == MING_LM_PERSISTENT_XCD || (m->mode == MING_LM_AUTO && xcd_enabled()))) {
        if (ctx->timeout_seen) {  // a timed-out step may have left counters raised and partials unwritten
            for (DevBuf* b : {&m->counters, &m->tpo, &m->tpd})
                if ((st = hip_check(ctx, hipMemsetAsync(b->p, 0, b->bytes, ctx->stream), "reset counters")))
                    return st;
            m->xcd_parity = 0;  // the partials now hold parity 0
            ctx->timeout_seen = false;
        }
        a.tx = static_cast<uint64_t*>(m->tx.p);
        a.tq = static_cast<uint64_t*>(m->tq.p);
        a.ta = static_cast<uint64_t*>(m->ta.p);
        a.tx1 = static_cast<uint64_t*>(m->tx1.p);
        a.th = static_cast<uint64_t*>(m->th.p);
        a.tpo = static_cast<uint32_t*>(m->tpo.p);
        a.tpd = static_cast<uint32_t*>(m->tpd.p);
        a.tpa = static_cast<uint64_t*>(m->tpa.p);
        a.xnsm = m->xnsm;
        a.xslots = xcd_slots(c->inter);
        a.counters = static_cast<int32_t*>(m->counters.p);
        a.tstamp = m->tstamp;
        a.nhubs = kMaxHubs;
        a.hub_stages = HUB_QKV | HUB_UP | HUB_HEAD;
        a.img = static_cast<uint32_t*>(m->img.p);
        a.img_stride = m->img_stride;
        a.hflag = static_cast<uint32_t*>(m->hflag.p);
        a.nflag = m->nflag;
        a.hubtab = static_cast<uint64_t*>(m->hubtab.p);
        a.att_xl = 1;
        a.xloc = xcd_local_enabled();
        a.split_len = tsl;
        // the partials were last written with parity xcd_parity: this step takes the other one
        a.epoch = ++m->epoch;
        while (a.epoch == 0 || (a.epoch & 1u) == m->xcd_parity) a.epoch = ++m->epoch;
        st = hip_check(ctx, launch_lm_step_xcd(ctx->stream, a, m->head.kind == 1, m->pgrid, !ctx->exclusive),
                       "lm_step XCD-local launch");
        if (st) return st;
        m->xcd_parity = a.epoch & 1u;
        kv->len += 1;
        return MING_OK;
    }
    if (persistent) {
        if (ctx->timeout_seen) {  // a timed-out step may have left arrival counters raised and partials unwritten
            for (DevBuf* b : {&m->counters, &m->tpo, &m->tpd})
                if ((st = hip_check(ctx, hipMemsetAsync(b->p, 0, b->bytes, ctx->stream), "reset counters")))
                    return st;
            m->xcd_parity = 0;
            ctx->timeout_seen = false;
        }
        a.tx = static_cast<uint64_t*>(m->tx.p);
        a.tq = static_cast<uint64_t*>(m->tq.p);
        a.ta = static_cast<uint64_t*>(m->ta.p);
        a.tx1 = static_cast<uint64_t*>(m->tx1.p);
        a.th = static_cast<uint64_t*>(m->th.p);
        a.counters = static_cast<int32_t*>(m->counters.p);
        a.tstamp = m->tstamp;
        a.nhubs = nhubs;
        a.hub_stages = hub_stages();
        a.img = static_cast<uint32_t*>(m->img.p);
        a.img_stride = m->img_stride;
        a.hflag = static_cast<uint32_t*>(m->hflag.p);
        a.nflag = m->nflag;
        a.hubtab = static_cast<uint64_t*>(m->hubtab.p);
        // XCD-grouped splits: split sp of kv head g on worker W-1-(8 sp + g), clear of the front workers
        a.att_xl = att_xl_enabled() && c->kv_heads <= 8 && 8 * (nsplit - 1) + c->kv_heads <= workers - front &&
                   8 * nsplit <= kAttXlSlots;
        a.split_len = tsl;
        a.epoch = ++m->epoch;
        if (a.epoch == 0) a.epoch = ++m->epoch;
        st = hip_check(ctx, launch_lm_step_tagged(ctx->stream, a, m->head.kind == 1, m->pgrid, !ctx->exclusive),
                       "lm_step persistent launch");
    } else
        st = hip_check(ctx, launch_lm_step_kernels(ctx->stream, a, m->layers.data()), "lm_step launch");
    if (st) return st;
    kv->len += 1;
    return MING_OK;
}

int ming_lm_model_dims(const ming_lm_model* m, int32_t* hidden, int32_t* vocab) {
    if (!m) return MING_E_NOT_INIT;
    if (hidden) *hidden = m->cfg.hidden;
    if (vocab) *vocab = m->cfg.vocab;
    return MING_OK;
}

int ming_lm_step(ming_ctx* ctx, ming_lm_model* m, const int32_t* token_dev, const void* x_in, ming_kv* kv,
                 void* hidden_out, float* logits_out, int32_t* argmax_out) {
    if (!alive(ctx)) return MING_E_NOT_INIT;
    if (!m) return set_err(ctx, MING_E_NOT_INIT, "null model");
    return lm_step_impl(ctx, m, token_dev, x_in, kv, hidden_out, logits_out, argmax_out);
}

int ming_lm_generate(ming_ctx* ctx, ming_lm_model* m, ming_kv* kv, int32_t n_steps, int32_t* tokens_dev) {
    if (!alive(ctx)) return MING_E_NOT_INIT;
    if (!m) return set_err(ctx, MING_E_NOT_INIT, "null model");
    if (!tokens_dev || n_steps < 0) return set_err(ctx, MING_E_ARG, "lm_generate: bad arguments");
    if (kv && kv->len + n_steps > kv->capacity)
        return set_err(ctx, MING_E_CTX_OVER_CAPACITY, "lm_generate: not enough cache capacity for n_steps");
    for (int i = 0; i < n_steps; i++) {
        int st = lm_step_impl(ctx, m, tokens_dev + i, nullptr, kv, nullptr, nullptr, tokens_dev + i + 1);
        if (st) return st;
    }
    return MING_OK;
}

}  // extern "C"

// Layer 0's input row of the model's step (where an input row is copied
// unless the caller wrote it there already, as the TTS loop's aggregator does).
uint16_t* ming::lm_input_row(ming_lm_model* m) { return static_cast<uint16_t*>(m->x.p); }
