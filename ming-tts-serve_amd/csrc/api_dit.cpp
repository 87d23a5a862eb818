// C-ABI glue of the DiT flow head and aggregator (include/ming_hip.h, "DiT
// flow head and aggregator"): argument checks, the load-time tables of
// Model.load (rotary tables, flow schedule, timestep embeddings;
// src/ming_model.zig:976-1004) and the per-call launch sequences of
// cfmSample / aggregate / stopProb (src/ming_model.zig:1033-1053, :1143-1203).
#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <vector>

#include "args.h"
#include "cfmp.h"
#include "internal.h"

namespace ming {
hipError_t launch_dit_stage(hipStream_t st, int which, const DitBlockDev& w, const uint16_t* x, const uint16_t* in,
                            int B, int L, const float* cos_t, const float* sin_t, uint16_t* qkv, uint16_t* out);
hipError_t launch_dit_block(hipStream_t st, const DitBlockDev& w, const uint16_t* x, int B, int L,
                            const float* cos_t, const float* sin_t, uint16_t* qkv, uint16_t* att, uint16_t* x1,
                            uint16_t* hh, uint16_t* x2, bool fuse_attn);
hipError_t launch_dit_linear(hipStream_t st, const uint16_t* x, int64_t xrow0, int64_t xstride, int R,
                             const uint16_t* norm, float eps, const uint16_t* w, int N, int K, const uint16_t* bias,
                             uint16_t* out, bool silu);
hipError_t launch_cfm_embed(hipStream_t st, const uint16_t* y, const uint16_t* wx, const uint16_t* bx, int D,
                            int latent, const uint16_t* te, const uint16_t* ce, const uint16_t* xh, uint16_t* rows);
hipError_t launch_cfm_final(hipStream_t st, const uint16_t* h, int L, int D, const uint16_t* norm, float eps,
                            const uint16_t* wf, const uint16_t* bf, int latent, const uint16_t* y, const uint16_t* dt,
                            const uint16_t* sq, const uint16_t* sde, int step, float cfg, float shift,
                            uint16_t* y_out);
hipError_t launch_stop_prob(hipStream_t st, const uint16_t* z, const uint16_t* w, const uint16_t* b, int K, float* p,
                            const int32_t* flags_in);
bool launch_cfm_pre(hipStream_t st, const uint16_t* z, int H, const uint16_t* wc, const uint16_t* bc, int D,
                    uint16_t* ce, const uint16_t* hist, int lat, const uint16_t* wx, const uint16_t* bx, uint16_t* xh,
                    const uint16_t* ws, const uint16_t* bs, float* p_out, const int32_t* flags_in, hipError_t* err);
hipError_t launch_cfm_persistent(hipStream_t st, const CfmPArgs& a, int grid, bool cooperative);
int cfmp_grid(int num_cus);
hipError_t launch_adaln_block(hipStream_t st, const DitBlockDev& w, const uint16_t* mod, const uint16_t* x, int B,
                              int L, const float* cos_t, const float* sin_t, uint16_t* qkv, uint16_t* att, uint16_t* x1,
                              uint16_t* hh, uint16_t* x2);
hipError_t launch_adaln_cond(hipStream_t st, const uint16_t* te, const uint16_t* ce, int steps, int D, uint16_t* out);
hipError_t launch_adaln_rows(hipStream_t st, const uint16_t* y, int F, const uint16_t* wx, const uint16_t* bx, int D,
                             int latent, uint16_t* rows);
hipError_t launch_adaln_final(hipStream_t st, const uint16_t* h, int F, int D, const uint16_t* norm, float eps,
                              const uint16_t* mod, const uint16_t* wf, const uint16_t* bf, int latent, const uint16_t* y,
                              const uint16_t* dt, const uint16_t* sq, const uint16_t* sde, int step, float cfg,
                              float shift, uint16_t* y_out);
}  // namespace ming

using namespace ming;

namespace {

constexpr int kFlowSteps = 10;  // FLOW_STEPS (src/ming_model.zig:48)
constexpr int kMaxRows = 6;

bool alive(const ming_ctx* c) { return c && c->alive; }

// Host bf16 helpers for the load-time tables (round to nearest even).
uint16_t hbf(float f) {
    uint32_t u;
    std::memcpy(&u, &f, 4);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x0040u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}
float hf(uint16_t h) {
    const uint32_t u = (uint32_t)h << 16;
    float f;
    std::memcpy(&f, &u, 4);
    return f;
}
float hrb(float f) { return hf(hbf(f)); }

int check_cfg(ming_ctx* ctx, const ming_dit_cfg* c) {
    if (!c) return set_err(ctx, MING_E_ARG, "dit: null cfg");
    if (c->hidden <= 0 || c->hidden % 64 != 0 || c->hidden > 4096 || c->ff <= 0 || c->ff % 64 != 0 || c->ff > 4096)
        return set_err(ctx, MING_E_UNSUPPORTED, "dit: hidden and ff must be multiples of 64, at most 4096");
    if (c->head_dim <= 0 || c->head_dim > 64 || c->head_dim % 2 != 0 || c->heads * c->head_dim != c->hidden)
        return set_err(ctx, MING_E_UNSUPPORTED, "dit: heads * head_dim must equal hidden, head_dim even and <= 64");
    return MING_OK;
}

int check_bf16(ming_ctx* ctx, const ming_linear& l, int N, int K, const char* what) {
    if (l.kind != MING_W_BF16 || !l.w)
        return set_err(ctx, MING_E_UNSUPPORTED, std::string(what) + ": DiT linears are bf16 [out, in]");
    if (l.out_features != N || l.in_features != K)
        return set_err(ctx, MING_E_SHAPE, std::string(what) + ": expected [" + std::to_string(N) + ", " +
                                              std::to_string(K) + "], got [" + std::to_string(l.out_features) +
                                              ", " + std::to_string(l.in_features) + "]");
    if (K % 8 != 0) return set_err(ctx, MING_E_UNSUPPORTED, std::string(what) + ": in_features % 8 != 0");
    return MING_OK;
}

int check_block(ming_ctx* ctx, const ming_dit_cfg* c, const ming_dit_block_w* w) {
    if (!w) return set_err(ctx, MING_E_ARG, "dit: null block");
    const int D = c->hidden, F = c->ff;
    int st;
    if ((st = check_bf16(ctx, w->wq, D, D, "wq")) || (st = check_bf16(ctx, w->wk, D, D, "wk")) ||
        (st = check_bf16(ctx, w->wv, D, D, "wv")) || (st = check_bf16(ctx, w->wo, D, D, "wo")) ||
        (st = check_bf16(ctx, w->w1, F, D, "ff1")) || (st = check_bf16(ctx, w->w2, D, F, "ff2")))
        return st;
    if (!w->norm1 || !w->norm2 || !w->bq || !w->bk || !w->bv || !w->bo || !w->b1 || !w->b2)
        return set_err(ctx, MING_E_ARG, "dit: null norm or bias");
    return MING_OK;
}

// B x L rows fit the kernels: R = B*L <= 6, L <= 8.
int check_rows(ming_ctx* ctx, int B, int L, const char* what) {
    if (B <= 0 || L <= 0 || B * L > kMaxRows || L > 8)
        return set_err(ctx, MING_E_SHAPE, std::string(what) + ": B*L must be in [1, 6] and L <= 8");
    return MING_OK;
}

DitBlockDev block_dev(const ming_dit_cfg* c, const ming_dit_block_w* w) {
    auto p = [](const void* v) { return static_cast<const uint16_t*>(v); };
    DitBlockDev d;
    d.D = c->hidden;
    d.F = c->ff;
    d.heads = c->heads;
    d.hd = c->head_dim;
    d.eps = c->eps;
    d.norm1 = p(w->norm1);
    d.norm2 = p(w->norm2);
    d.wq = p(w->wq.w);
    d.wk = p(w->wk.w);
    d.wv = p(w->wv.w);
    d.wo = p(w->wo.w);
    d.w1 = p(w->w1.w);
    d.w2 = p(w->w2.w);
    d.bq = p(w->bq);
    d.bk = p(w->bk);
    d.bv = p(w->bv);
    d.bo = p(w->bo);
    d.b1 = p(w->b1);
    d.b2 = p(w->b2);
    return d;
}

const uint16_t* u16(const void* p) { return static_cast<const uint16_t*>(p); }
uint16_t* u16(void* p) { return static_cast<uint16_t*>(p); }

// Rotary.table in f32 on the host (load time), uploaded.
int rotary_upload(ming_ctx* ctx, const float* inv_freq, int half, int L, float* cos_dev, float* sin_dev) {
    std::vector<float> c((size_t)L * half), s((size_t)L * half);
    for (int l = 0; l < L; l++)
        for (int i = 0; i < half; i++) {
            const float f = (float)l * inv_freq[i];
            c[(size_t)l * half + i] = std::cos(f);
            s[(size_t)l * half + i] = std::sin(f);
        }
    int st;
    if ((st = hip_check(ctx, hipMemcpyAsync(cos_dev, c.data(), c.size() * 4, hipMemcpyHostToDevice, ctx->stream),
                        "rotary cos")))
        return st;
    if ((st = hip_check(ctx, hipMemcpyAsync(sin_dev, s.data(), s.size() * 4, hipMemcpyHostToDevice, ctx->stream),
                        "rotary sin")))
        return st;
    return hip_check(ctx, hipStreamSynchronize(ctx->stream), "rotary table");
}

// Per-block workspace of one DiT stack at R rows.
struct StackBufs {
    DevBuf rows[2], qkv, att, x1, hh;
    hipError_t alloc(int R, int D, int F) {
        hipError_t e = hipSuccess;
        for (DevBuf* b : {&rows[0], &rows[1], &att, &x1})
            if (e == hipSuccess) e = b->ensure(sizeof(uint16_t) * (size_t)R * D);
        if (e == hipSuccess) e = qkv.ensure(sizeof(uint16_t) * (size_t)3 * R * D);
        if (e == hipSuccess) e = hh.ensure(sizeof(uint16_t) * (size_t)R * F);
        return e;
    }
    void release() {
        for (DevBuf* b : {&rows[0], &rows[1], &qkv, &att, &x1, &hh}) b->release();
    }
};

// The blocks of a stack on rows[0] (B x L rows); returns the buffer holding the output.
// The blocks in order on rows ping-ponging between b.rows[0] and [1]; the
// first block reads `first` when given (else b.rows[0]).
hipError_t run_stack(hipStream_t st, const std::vector<DitBlockDev>& blocks, StackBufs& b, int B, int L,
                     const float* cos_t, const float* sin_t, uint16_t** out, uint16_t* first = nullptr) {
    int cur = 0;
    uint16_t* in = first ? first : u16(b.rows[0].p);
    for (const DitBlockDev& w : blocks) {
        hipError_t e = launch_dit_block(st, w, in, B, L, cos_t, sin_t, u16(b.qkv.p), u16(b.att.p), u16(b.x1.p),
                                        u16(b.hh.p), u16(b.rows[cur ^ 1].p), true);
        if (e != hipSuccess) return e;
        cur ^= 1;
        in = u16(b.rows[cur].p);
    }
    *out = in;
    return hipSuccess;
}

// Model.load's flow tables (src/ming_model.zig:976-1004): flowSchedule in
// bf16 (:1207-1215), flow_dt and flow_sq (:995-1002), and the timestep
// embeddings (:976-992, :1064-1076) -- sinusoid rows on the host, the MLP on
// the GPU -- into t_emb [steps][2][D].  Synchronous.
hipError_t flow_tables(hipStream_t s, const ming_linear& mlp0, const void* b0, const ming_linear& mlp2, const void* b2,
                       int D, uint16_t* t, uint16_t* dt, uint16_t* sq, uint16_t* dt_dev, uint16_t* sq_dev,
                       uint16_t* t_emb_dev) {
    static const float sched[kFlowSteps + 1] = {0, 2, 4, 6, 8, 12, 16, 20, 24, 28, 32};
    const float c32 = hrb(1.0f / 32.0f), hpi = hrb((float)(3.14159265358979323846 / 2.0));
    for (int i = 0; i <= kFlowSteps; i++) {
        const float ti = hrb(c32 * hrb(sched[i]));
        const float ct = hrb(std::cos(hrb(hpi * ti)));
        const float sw = hrb(hrb(ct - 1.0f) + ti);
        t[i] = hbf(ti + hrb(-1.0f * sw));
    }
    for (int i = 0; i < kFlowSteps; i++) {
        const float d = hrb(hf(t[i + 1]) - hf(t[i]));
        dt[i] = hbf(d);
        sq[i] = hbf(std::pow(std::fabs(d), hrb(0.5f)));
    }
    std::vector<uint16_t> sc((size_t)kFlowSteps * 2 * 256);
    const float ef = (float)(std::log(10000.0) / 127.0);
    float fr[128];
    for (int k = 0; k < 128; k++) fr[k] = std::exp((float)k * -ef);
    for (int i = 0; i < kFlowSteps; i++) {
        const float ts = hrb(hrb(1000.0f) * hf(t[i]));
        for (int r = 0; r < 2; r++)
            for (int k = 0; k < 128; k++) {
                const float a = ts * fr[k];
                sc[((size_t)i * 2 + r) * 256 + k] = hbf(std::sin(a));
                sc[((size_t)i * 2 + r) * 256 + 128 + k] = hbf(std::cos(a));
            }
    }
    DevBuf scd, tmp;
    hipError_t e = scd.ensure(sizeof(uint16_t) * sc.size());
    if (e == hipSuccess) e = tmp.ensure(sizeof(uint16_t) * 2 * (size_t)D);
    if (e == hipSuccess) e = hipMemcpyAsync(scd.p, sc.data(), sizeof(uint16_t) * sc.size(), hipMemcpyHostToDevice, s);
    if (e == hipSuccess) e = hipMemcpyAsync(dt_dev, dt, sizeof(uint16_t) * kFlowSteps, hipMemcpyHostToDevice, s);
    if (e == hipSuccess) e = hipMemcpyAsync(sq_dev, sq, sizeof(uint16_t) * kFlowSteps, hipMemcpyHostToDevice, s);
    for (int i = 0; i < kFlowSteps && e == hipSuccess; i++) {
        e = launch_dit_linear(s, u16(scd.p) + (size_t)i * 2 * 256, 0, 1, 2, nullptr, 0.0f, u16(mlp0.w), D, 256, u16(b0),
                              u16(tmp.p), true);
        if (e == hipSuccess)
            e = launch_dit_linear(s, u16(tmp.p), 0, 1, 2, nullptr, 0.0f, u16(mlp2.w), D, D, u16(b2),
                                  t_emb_dev + (size_t)i * 2 * D, false);
    }
    const hipError_t es = hipStreamSynchronize(s);  // the host tables above must outlive the copies
    if (e == hipSuccess) e = es;
    scd.release();
    tmp.release();
    return e;
}

}  // namespace

struct ming_cfm_model {
    ming_ctx* ctx = nullptr;
    ming_dit_cfg cfg{};
    std::vector<DitBlockDev> blocks;
    const uint16_t *wx = nullptr, *bx = nullptr, *wc = nullptr, *bc = nullptr, *wf = nullptr, *bf = nullptr,
                   *final_norm = nullptr;
    int latent = 0, lm_hidden = 0;
    uint16_t t[kFlowSteps + 1]{}, dt[kFlowSteps]{}, sq[kFlowSteps]{};
    DevBuf cos, sin, t_emb, dtd, sqd, zc, ce, xh, y;
    StackBufs s;
    // ming_cfm_sample_batch workspace (grown on demand): n sequences, 6 n rows
    DevBuf bce, bxh, bxe, brows[2], bhn, bqkv, batt, bx1, bhh, by[2], bhf, bpart;
    // persistent flow head (cfm_persistent.hip): mode, grid (0: not available
    // for this model / device), launch tag, workspace (allocated zeroed at the
    // first persistent sample), optional stage stamps
    int mode = MING_CFM_AUTO;
    int pgrid = 0;
    uint32_t pepoch = 0;
    DevBuf pblocks, ptq, ptx1, pth, ptxo, pimg, pflg, pxcc;
    uint64_t* pstamps = nullptr;
};

struct ming_adaln_model {
    ming_ctx* ctx = nullptr;
    ming_dit_cfg cfg{};
    int frames = 0, latent = 0, lm_hidden = 0;
    std::vector<DitBlockDev> blocks;
    std::vector<const uint16_t*> ada, bada;
    const uint16_t *wx = nullptr, *bx = nullptr, *wc = nullptr, *bc = nullptr, *wf = nullptr, *bf = nullptr,
                   *final_norm = nullptr, *wfa = nullptr, *bfa = nullptr;
    uint16_t t[kFlowSteps + 1]{}, dt[kFlowSteps]{}, sq[kFlowSteps]{};
    DevBuf cos, sin, t_emb, dtd, sqd, zc, ce, silu_c, mods, modf, y;
    StackBufs s;
};

struct ming_agg_model {
    ming_ctx* ctx = nullptr;
    ming_dit_cfg cfg{};
    std::vector<DitBlockDev> blocks;
    const uint16_t *wx = nullptr, *bx = nullptr, *cls = nullptr, *wf = nullptr, *bf = nullptr,
                   *final_norm = nullptr;
    int latent = 0, lm_hidden = 0;
    DevBuf cos, sin;
    DevBuf in;  // the first block's input rows [cls; x_emb(latent)]: cls written once at creation
    StackBufs s;
};

namespace {

// The persistent flow head's workspace, zeroed (a zero tag never matches a
// launch's epoch, which starts at 1): tagged outputs of every (step, block),
// the hubs' images, flags and XCC table, and the device block table.
hipError_t cfmp_alloc(ming_cfm_model* m) {
    const size_t sb = (size_t)kFlowSteps * m->blocks.size();
    std::vector<CfmPBlock> tab;
    for (const DitBlockDev& d : m->blocks)
        tab.push_back(CfmPBlock{d.norm1, d.norm2, d.wq, d.wk, d.wv, d.wo, d.w1, d.w2, d.bq, d.bk, d.bv, d.bo, d.b1,
                                d.b2});
    hipError_t e = m->pblocks.ensure(sizeof(CfmPBlock) * tab.size());
    if (e == hipSuccess) e = m->ptq.ensure(sizeof(uint64_t) * sb * kPTq);
    if (e == hipSuccess) e = m->ptx1.ensure(sizeof(uint64_t) * sb * kPTx);
    if (e == hipSuccess) e = m->pth.ensure(sizeof(uint64_t) * sb * kPTh);
    if (e == hipSuccess) e = m->ptxo.ensure(sizeof(uint64_t) * sb * kPTx);
    if (e == hipSuccess) e = m->pimg.ensure(sizeof(uint32_t) * (size_t)kPXcds * kPImgWords);
    if (e == hipSuccess) e = m->pflg.ensure(sizeof(uint32_t) * (size_t)kPXcds * 4 * kPFlagLine);
    if (e == hipSuccess) e = m->pxcc.ensure(sizeof(uint64_t) * kPXcds);
    if (e == hipSuccess)
        e = hipMemcpy(m->pblocks.p, tab.data(), sizeof(CfmPBlock) * tab.size(), hipMemcpyHostToDevice);
    for (DevBuf* b : {&m->ptq, &m->ptx1, &m->pth, &m->ptxo, &m->pimg, &m->pflg, &m->pxcc})
        if (e == hipSuccess) e = hipMemset(b->p, 0, b->bytes);
    if (e == hipSuccess) e = hipDeviceSynchronize();
    return e;
}

void cfmp_release(ming_cfm_model* m) {
    for (DevBuf* b : {&m->pblocks, &m->ptq, &m->ptx1, &m->pth, &m->ptxo, &m->pimg, &m->pflg, &m->pxcc})
        b->release();
}

}  // namespace

extern "C" {

int ming_rotary_table(ming_ctx* ctx, const float* inv_freq_host, int32_t half, int32_t L, float* cos_dev,
                      float* sin_dev) {
    if (!alive(ctx)) return MING_E_NOT_INIT;
    if (!inv_freq_host || !cos_dev || !sin_dev || half <= 0 || L <= 0)
        return set_err(ctx, MING_E_ARG, "rotary_table: bad arguments");
    return rotary_upload(ctx, inv_freq_host, half, L, cos_dev, sin_dev);
}

int ming_dit_block(ming_ctx* ctx, const ming_dit_cfg* cfg, const ming_dit_block_w* w, const void* x, int32_t B,
                   int32_t L, const float* cos_dev, const float* sin_dev, ming_dit_out* out) {
    if (!alive(ctx)) return MING_E_NOT_INIT;
    int st;
    if ((st = check_cfg(ctx, cfg)) || (st = check_block(ctx, cfg, w)) || (st = check_rows(ctx, B, L, "dit_block")))
        return st;
    if (!x || !cos_dev || !sin_dev || !out || !out->qkv || !out->att || !out->x1 || !out->hh || !out->x2)
        return set_err(ctx, MING_E_ARG, "dit_block: null buffer");
    const DitBlockDev d = block_dev(cfg, w);
    return hip_check(ctx,
                     launch_dit_block(ctx->stream, d, u16(x), B, L, cos_dev, sin_dev, u16(out->qkv), u16(out->att),
                                      u16(out->x1), u16(out->hh), u16(out->x2), false),
                     "dit_block launch");
}

int ming_dit_single(ming_ctx* ctx, int32_t which, const ming_dit_cfg* cfg, const ming_dit_block_w* w, const void* x,
                    const void* in, int32_t B, int32_t L, const float* cos_dev, const float* sin_dev, void* qkv_tmp,
                    void* out) {
    if (!alive(ctx)) return MING_E_NOT_INIT;
    int st;
    if ((st = check_cfg(ctx, cfg)) || (st = check_block(ctx, cfg, w))) return st;
    if (which < 0 || which > 3) return set_err(ctx, MING_E_ARG, "dit_single: which must be 0..3");
    if ((st = check_rows(ctx, B, L, "dit_single"))) return st;
    if (!x || !out || ((which == 1 || which == 3) && !in) || (which == 0 && (!qkv_tmp || !cos_dev || !sin_dev)))
        return set_err(ctx, MING_E_ARG, "dit_single: null buffer");
    const DitBlockDev d = block_dev(cfg, w);
    return hip_check(ctx,
                     launch_dit_stage(ctx->stream, which, d, u16(x), u16(in), B, L, cos_dev, sin_dev, u16(qkv_tmp),
                                      u16(out)),
                     "dit_single launch");
}

int ming_cfm_embed(ming_ctx* ctx, const void* y, const ming_linear* x_emb, const void* bx, const void* te,
                   const void* ce, const void* xh, void* h_out) {
    if (!alive(ctx)) return MING_E_NOT_INIT;
    if (!x_emb || !y || !bx || !te || !ce || !xh || !h_out) return set_err(ctx, MING_E_ARG, "cfm_embed: null argument");
    int st;
    if ((st = check_bf16(ctx, *x_emb, x_emb->out_features, x_emb->in_features, "x_emb"))) return st;
    if (x_emb->in_features > 4096 || x_emb->out_features % 8 != 0)
        return set_err(ctx, MING_E_UNSUPPORTED, "cfm_embed: x_emb shape");
    return hip_check(ctx,
                     launch_cfm_embed(ctx->stream, u16(y), u16(x_emb->w), u16(bx), x_emb->out_features,
                                      x_emb->in_features, u16(te), u16(ce), u16(xh), u16(h_out)),
                     "cfm_embed launch");
}

int ming_cfm_final(ming_ctx* ctx, const void* h, int32_t L, const void* norm, const ming_linear* wf, const void* bf,
                   const void* y, const void* dtt, const void* sq, const void* sde, int32_t step, float cfg,
                   float shift, void* y_out) {
    if (!alive(ctx)) return MING_E_NOT_INIT;
    if (!h || !norm || !wf || !bf || !y || !dtt || !sq || !y_out || (shift != 0.0f && !sde) || L <= 0 || step < 0)
        return set_err(ctx, MING_E_ARG, "cfm_final: bad arguments");
    int st;
    if ((st = check_bf16(ctx, *wf, wf->out_features, wf->in_features, "final"))) return st;
    if (wf->in_features > 4096) return set_err(ctx, MING_E_UNSUPPORTED, "cfm_final: hidden > 4096");
    return hip_check(ctx,
                     launch_cfm_final(ctx->stream, u16(h), L, wf->in_features, u16(norm), 1e-6f, u16(wf->w), u16(bf),
                                      wf->out_features, u16(y), u16(dtt), u16(sq), u16(sde), step, cfg, shift,
                                      u16(y_out)),
                     "cfm_final launch");
}

// ---- flow head -------------------------------------------------------------------

int ming_cfm_model_create(ming_ctx* ctx, const ming_cfm_w* w, ming_cfm_model** out) {
    if (!alive(ctx)) return MING_E_NOT_INIT;
    if (!w || !out || !w->blocks || w->n_blocks <= 0 || !w->inv_freq)
        return set_err(ctx, MING_E_ARG, "cfm_model_create: bad arguments");
    *out = nullptr;
    const ming_dit_cfg* c = &w->cfg;
    int st;
    if ((st = check_cfg(ctx, c))) return st;
    for (int i = 0; i < w->n_blocks; i++)
        if ((st = check_block(ctx, c, &w->blocks[i]))) return st;
    if ((st = check_rows(ctx, 2, 3, "cfm_model_create"))) return st;
    const int D = c->hidden, latent = w->x_emb.in_features, H = w->c_emb.in_features;
    if ((st = check_bf16(ctx, w->x_emb, D, latent, "x_emb")) || (st = check_bf16(ctx, w->c_emb, D, H, "c_emb")) ||
        (st = check_bf16(ctx, w->t_mlp0, D, 256, "t_mlp0")) || (st = check_bf16(ctx, w->t_mlp2, D, D, "t_mlp2")) ||
        (st = check_bf16(ctx, w->final, latent, D, "final")))
        return st;
    if (H > 4096 || latent > 4096 || latent % 8 != 0)
        return set_err(ctx, MING_E_UNSUPPORTED, "cfm_model_create: latent/LM hidden sizes");
    if (!w->bx || !w->bc || !w->bt0 || !w->bt2 || !w->final_norm || !w->bf)
        return set_err(ctx, MING_E_ARG, "cfm_model_create: null bias or norm");
    auto* m = new ming_cfm_model;
    m->ctx = ctx;
    m->cfg = *c;
    for (int i = 0; i < w->n_blocks; i++) m->blocks.push_back(block_dev(c, &w->blocks[i]));
    m->wx = u16(w->x_emb.w);
    m->bx = u16(w->bx);
    m->wc = u16(w->c_emb.w);
    m->bc = u16(w->bc);
    m->wf = u16(w->final.w);
    m->bf = u16(w->bf);
    m->final_norm = u16(w->final_norm);
    m->latent = latent;
    m->lm_hidden = H;
    const int half = c->head_dim / 2, L = 3;
    hipStream_t s = ctx->stream;
    hipError_t e = m->cos.ensure(sizeof(float) * L * half);
    if (e == hipSuccess) e = m->sin.ensure(sizeof(float) * L * half);
    if (e == hipSuccess) e = m->t_emb.ensure(sizeof(uint16_t) * (size_t)kFlowSteps * 2 * D);
    if (e == hipSuccess) e = m->dtd.ensure(sizeof(uint16_t) * kFlowSteps);
    if (e == hipSuccess) e = m->sqd.ensure(sizeof(uint16_t) * kFlowSteps);
    if (e == hipSuccess) e = m->zc.ensure(sizeof(uint16_t) * 2 * (size_t)H);
    if (e == hipSuccess) e = m->ce.ensure(sizeof(uint16_t) * 2 * (size_t)D);
    if (e == hipSuccess) e = m->xh.ensure(sizeof(uint16_t) * (size_t)D);
    if (e == hipSuccess) e = m->y.ensure(sizeof(uint16_t) * (size_t)latent);
    if (e == hipSuccess) e = m->s.alloc(2 * L, D, c->ff);
    if (e == hipSuccess) e = hipMemsetAsync(m->zc.p, 0, m->zc.bytes, s);
    // c_emb of the unconditional half's zero row, once: row 1 of ce (cfm_sample computes row 0)
    if (e == hipSuccess)
        e = launch_dit_linear(s, u16(m->zc.p) + H, 0, 1, 1, nullptr, c->eps, m->wc, D, H, m->bc, u16(m->ce.p) + D,
                              false);
    if (e != hipSuccess) {
        ming_cfm_model_destroy(m);
        return hip_check(ctx, e, "cfm_model_create");
    }
    if ((st = rotary_upload(ctx, w->inv_freq, half, L, static_cast<float*>(m->cos.p), static_cast<float*>(m->sin.p)))) {
        ming_cfm_model_destroy(m);
        return st;
    }
    e = flow_tables(s, w->t_mlp0, w->bt0, w->t_mlp2, w->bt2, D, m->t, m->dt, m->sq, u16(m->dtd.p), u16(m->sqd.p),
                    u16(m->t_emb.p));
    if (e != hipSuccess) {
        ming_cfm_model_destroy(m);
        return hip_check(ctx, e, "cfm_model_create tables");
    }
    // the persistent flow head, where its fixed shape and grid apply
    if (D == kPD && c->ff == kPF && c->heads == kPHeads && c->head_dim == kPHd && latent == kPLat &&
        w->n_blocks <= kPMaxBlocks) {
        m->pgrid = cfmp_grid(ctx->num_cus);
        if (m->pgrid > 0 && (e = cfmp_alloc(m)) != hipSuccess) {
            ming_cfm_model_destroy(m);
            return hip_check(ctx, e, "cfm_model_create persistent workspace");
        }
    }
    *out = m;
    return MING_OK;
}

int ming_cfm_model_destroy(ming_cfm_model* m) {
    if (!m) return MING_E_NOT_INIT;
    for (DevBuf* b : {&m->cos, &m->sin, &m->t_emb, &m->dtd, &m->sqd, &m->zc, &m->ce, &m->xh, &m->y, &m->bce, &m->bxh,
                      &m->bxe, &m->brows[0], &m->brows[1], &m->bhn, &m->bqkv, &m->batt, &m->bx1, &m->bhh, &m->by[0],
                      &m->by[1], &m->bhf, &m->bpart})
        b->release();
    m->s.release();
    cfmp_release(m);
    delete m;
    return MING_OK;
}

int ming_cfm_model_set_mode(ming_cfm_model* m, int32_t mode) {
    if (!m) return MING_E_NOT_INIT;
    if (mode < MING_CFM_AUTO || mode > MING_CFM_PERSISTENT)
        return set_err(m->ctx, MING_E_ARG, "cfm_model_set_mode: unknown mode");
    if (mode == MING_CFM_PERSISTENT && m->pgrid == 0)
        return set_err(m->ctx, MING_E_UNSUPPORTED,
                       "cfm_model_set_mode: the persistent flow head needs hidden 1024, 16 heads of 64, ff 4096, "
                       "latent 64, at most 16 blocks and one resident workgroup on each of a multiple of 8 CUs, at least 232");
    m->mode = mode;
    return MING_OK;
}

int ming_cfm_model_profile(ming_cfm_model* m, void* stamps_dev) {
    if (!m) return MING_E_NOT_INIT;
    m->pstamps = static_cast<uint64_t*>(stamps_dev);
    return MING_OK;
}

int ming_cfm_model_dims(const ming_cfm_model* m, int32_t* latent, int32_t* lm_hidden) {
    if (!m) return MING_E_NOT_INIT;
    if (latent) *latent = m->latent;
    if (lm_hidden) *lm_hidden = m->lm_hidden;
    return MING_OK;
}

int ming_agg_model_dims(const ming_agg_model* m, int32_t* lm_hidden, int32_t* latent) {
    if (!m) return MING_E_NOT_INIT;
    if (lm_hidden) *lm_hidden = m->lm_hidden;
    if (latent) *latent = m->latent;
    return MING_OK;
}

int ming_cfm_model_tables(ming_cfm_model* m, uint16_t* t, uint16_t* dt, uint16_t* sq, const void** t_emb_dev) {
    if (!m) return MING_E_NOT_INIT;
    if (t) std::memcpy(t, m->t, sizeof(m->t));
    if (dt) std::memcpy(dt, m->dt, sizeof(m->dt));
    if (sq) std::memcpy(sq, m->sq, sizeof(m->sq));
    if (t_emb_dev) *t_emb_dev = m->t_emb.p;
    return MING_OK;
}

int ming_cfm_sample(ming_ctx* ctx, ming_cfm_model* m, const void* z, const void* hist, const void* noise,
                    const void* sde, float cfg, float sigma, float temperature, void* latent_out, void* y_steps) {
    return ming::cfm_sample_impl(ctx, m, z, hist, noise, sde, cfg, sigma, temperature, latent_out, y_steps, false);
}

}  // extern "C"

// cfmSample; pre_done: c_emb(z) and x_emb(hist) are already in the model's rows (cfm_pre).
int ming::cfm_sample_impl(ming_ctx* ctx, ming_cfm_model* m, const void* z, const void* hist, const void* noise,
                          const void* sde, float cfg, float sigma, float temperature, void* latent_out, void* y_steps,
                          bool pre_done) {
    if (!alive(ctx)) return MING_E_NOT_INIT;
    if (!m) return set_err(ctx, MING_E_NOT_INIT, "cfm_sample: null model");
    const float shift = sigma * std::sqrt(temperature);
    if (!z || !hist || !noise || !latent_out || (shift != 0.0f && !sde))
        return set_err(ctx, MING_E_ARG, "cfm_sample: null buffer");
    hipStream_t s = ctx->stream;
    const int D = m->cfg.hidden, H = m->lm_hidden, lat = m->latent, L = 3;
    const float eps = m->cfg.eps;
    // once per sample: c_emb([z, 0]) and x_emb(hist) (:1196-1197).  Row 1 of ce, c_emb of the zero
    // row, is computed at creation; row 0 reads z in place when it is 16-byte aligned (a row's
    // result does not depend on how many rows a launch takes).
    hipError_t e = hipSuccess;
    if (!pre_done) {
        const uint16_t* zin = u16(z);
        if (reinterpret_cast<uintptr_t>(z) % 16 != 0) {
            e = hipMemcpyAsync(m->zc.p, z, sizeof(uint16_t) * H, hipMemcpyDeviceToDevice, s);
            zin = u16(m->zc.p);
        }
        if (e == hipSuccess)
            e = launch_dit_linear(s, zin, 0, 1, 1, nullptr, eps, m->wc, D, H, m->bc, u16(m->ce.p), false);
        if (e == hipSuccess)
            e = launch_dit_linear(s, u16(hist), 0, 1, 1, nullptr, eps, m->wx, D, lat, m->bx, u16(m->xh.p), false);
    }
    // AUTO takes the persistent kernel wherever its shape fits: 1.51 ms per sample against the
    // launch path's 1.92 ms at hidden 1024, 8 blocks
    if (e == hipSuccess && (m->mode == MING_CFM_PERSISTENT || m->mode == MING_CFM_AUTO) && m->pgrid > 0) {
        CfmPArgs a{};
        a.blocks = static_cast<const CfmPBlock*>(m->pblocks.p);
        a.nblk = (int)m->blocks.size();
        a.steps = kFlowSteps;
        a.nflag = kFlowSteps * a.nblk * 4;
        a.eps = eps;
        a.cos_t = static_cast<const float*>(m->cos.p);
        a.sin_t = static_cast<const float*>(m->sin.p);
        a.te = u16(m->t_emb.p);
        a.ce = u16(m->ce.p);
        a.xh = u16(m->xh.p);
        a.wx = m->wx;
        a.bx = m->bx;
        a.fnorm = m->final_norm;
        a.wf = m->wf;
        a.bf = m->bf;
        a.noise = u16(noise);
        a.sde = u16(sde);
        a.dt = u16(m->dtd.p);
        a.sq = u16(m->sqd.p);
        a.cfg = cfg;
        a.shift = shift;
        a.y_out = u16(latent_out);
        a.y_steps = u16(y_steps);
        a.tq = static_cast<uint64_t*>(m->ptq.p);
        a.tx1 = static_cast<uint64_t*>(m->ptx1.p);
        a.th = static_cast<uint64_t*>(m->pth.p);
        a.txo = static_cast<uint64_t*>(m->ptxo.p);
        a.img = static_cast<uint32_t*>(m->pimg.p);
        a.flg = static_cast<uint32_t*>(m->pflg.p);
        a.xcctab = static_cast<uint64_t*>(m->pxcc.p);
        a.tstamp = m->pstamps;
        a.flags = ctx->dev_flags;
        // this launch's tags: pepoch + 1 .. pepoch + nflag (u32); when they
        // would wrap (after about 13 million samples) every tag and flag is
        // cleared and they start again at 1
        if ((uint64_t)m->pepoch + (uint64_t)a.nflag + 1 > 0xffffffffull) {
            for (DevBuf* b : {&m->ptq, &m->ptx1, &m->pth, &m->ptxo, &m->pflg, &m->pxcc})
                if (e == hipSuccess) e = hipMemsetAsync(b->p, 0, b->bytes, s);
            m->pepoch = 0;
        }
        a.epoch = m->pepoch + 1;
        m->pepoch += (uint32_t)a.nflag;
        if (e == hipSuccess) e = launch_cfm_persistent(s, a, m->pgrid, !ctx->exclusive);
        return hip_check(ctx, e, "cfm_sample persistent launch");
    }
    const uint16_t* y = u16(noise);
    for (int i = 0; i < kFlowSteps && e == hipSuccess; i++) {
        e = launch_cfm_embed(s, y, m->wx, m->bx, D, lat, u16(m->t_emb.p) + (size_t)i * 2 * D, u16(m->ce.p),
                             u16(m->xh.p), u16(m->s.rows[0].p));
        uint16_t* h = nullptr;
        if (e == hipSuccess)
            e = run_stack(s, m->blocks, m->s, 2, L, static_cast<const float*>(m->cos.p),
                          static_cast<const float*>(m->sin.p), &h);
        if (e == hipSuccess)
            e = launch_cfm_final(s, h, L, D, m->final_norm, eps, m->wf, m->bf, lat, y, u16(m->dtd.p), u16(m->sqd.p),
                                 u16(sde), i, cfg, shift, u16(m->y.p));
        y = u16(m->y.p);
        if (e == hipSuccess && y_steps)
            e = hipMemcpyAsync(u16(y_steps) + (size_t)i * lat, m->y.p, sizeof(uint16_t) * lat,
                               hipMemcpyDeviceToDevice, s);
    }
    if (e == hipSuccess)
        e = hipMemcpyAsync(latent_out, m->y.p, sizeof(uint16_t) * lat, hipMemcpyDeviceToDevice, s);
    return hip_check(ctx, e, "cfm_sample");
}

// The step's one-row GEMVs before a flow-head sample: c_emb(z) and x_emb(hist)
// into the model's rows (for cfm_sample_impl with pre_done) and the stop head
// on z into p_out[0] with the error flags in p_out[1..3] -- one launch where
// the shapes allow it, else three.
int ming::cfm_pre(ming_ctx* ctx, ming_cfm_model* m, const void* z, const void* hist, const ming_linear* stop_head,
                  const void* stop_bias, float* p_out) {
    if (!alive(ctx)) return MING_E_NOT_INIT;
    if (!m || !z || !hist || !stop_head || !stop_bias || !p_out) return set_err(ctx, MING_E_ARG, "cfm_pre: null argument");
    int st;
    if ((st = check_bf16(ctx, *stop_head, 2, m->lm_hidden, "stop_head"))) return st;
    hipStream_t s = ctx->stream;
    const int D = m->cfg.hidden, H = m->lm_hidden, lat = m->latent;
    hipError_t e = hipSuccess;
    if (launch_cfm_pre(s, u16(z), H, m->wc, m->bc, D, u16(m->ce.p), u16(hist), lat, m->wx, m->bx, u16(m->xh.p),
                       u16(stop_head->w), u16(stop_bias), p_out, ctx->dev_flags, &e))
        return hip_check(ctx, e, "cfm_pre launch");
    if ((st = stop_prob_impl(ctx, stop_head, stop_bias, z, p_out, true))) return st;
    const uint16_t* zin = u16(z);
    if (reinterpret_cast<uintptr_t>(z) % 16 != 0) {
        e = hipMemcpyAsync(m->zc.p, z, sizeof(uint16_t) * H, hipMemcpyDeviceToDevice, s);
        zin = u16(m->zc.p);
    }
    if (e == hipSuccess)
        e = launch_dit_linear(s, zin, 0, 1, 1, nullptr, m->cfg.eps, m->wc, D, H, m->bc, u16(m->ce.p), false);
    if (e == hipSuccess)
        e = launch_dit_linear(s, u16(hist), 0, 1, 1, nullptr, m->cfg.eps, m->wx, D, lat, m->bx, u16(m->xh.p), false);
    return hip_check(ctx, e, "cfm_pre launches");
}

extern "C" {

// cfmSample of n sequences in one pass (the flow head of a batched server
// step): the rows of every sequence go through each DiT linear as one GEMM.
int ming_cfm_sample_batch(ming_ctx* ctx, ming_cfm_model* m, int32_t n, const void* z, const void* hist,
                          const void* noise, const void* sde, float cfg, float sigma, float temperature,
                          void* latents_out, void* y_steps) {
    if (!alive(ctx)) return MING_E_NOT_INIT;
    if (!m) return set_err(ctx, MING_E_NOT_INIT, "cfm_sample_batch: null model");
    const float shift = sigma * std::sqrt(temperature);
    if (n < 1 || n > 64) return set_err(ctx, MING_E_UNSUPPORTED, "cfm_sample_batch: 1..64 sequences");
    if (!z || !hist || !noise || !latents_out || (shift != 0.0f && !sde))
        return set_err(ctx, MING_E_ARG, "cfm_sample_batch: null buffer");
    const int D = m->cfg.hidden, F = m->cfg.ff, H = m->lm_hidden, lat = m->latent, L = 3, R = 6 * n;
    if (D % 64 || F % 64 || H % 64 || lat % 64 || m->cfg.head_dim % 2)
        return set_err(ctx, MING_E_UNSUPPORTED, "cfm_sample_batch: hidden, ff, lm_hidden and latent must be multiples of 64");
    hipStream_t s = ctx->stream;
    const size_t b2 = sizeof(uint16_t);
    hipError_t e = hipSuccess;
    auto grow = [&](DevBuf& d, size_t bytes) {
        if (e == hipSuccess) e = d.ensure(bytes);
    };
    grow(m->bce, (size_t)n * D * b2);
    grow(m->bxh, (size_t)n * D * b2);
    grow(m->bxe, (size_t)n * D * b2);
    grow(m->brows[0], (size_t)R * D * b2);
    grow(m->brows[1], (size_t)R * D * b2);
    grow(m->bhn, (size_t)R * D * b2);
    grow(m->bqkv, (size_t)3 * R * D * b2);
    grow(m->batt, (size_t)R * D * b2);
    grow(m->bx1, (size_t)R * D * b2);
    grow(m->bhh, (size_t)R * F * b2);
    grow(m->by[0], (size_t)n * lat * b2);
    grow(m->by[1], (size_t)n * lat * b2);
    grow(m->bhf, (size_t)2 * n * D * b2);
    grow(m->bpart, (size_t)R * std::max(4 * D, 2 * F) * sizeof(float));  // split-K partials of ff2 / ff1
    if (e != hipSuccess) return hip_check(ctx, e, "cfm_sample_batch workspace");
    const float eps = m->cfg.eps;
    // once per sample: c_emb(z) (the unconditional half is c_emb(0) = bias) and x_emb(hist) (:1196-1197)
    e = launch_dit_linear_gemm(s, u16(z), n, m->wc, D, H, m->bc, u16(m->bce.p));
    if (e == hipSuccess) e = launch_dit_linear_gemm(s, u16(hist), n, m->wx, D, lat, m->bx, u16(m->bxh.p));
    const uint16_t* y = u16(noise);
    int yi = 0;
    for (int i = 0; i < kFlowSteps && e == hipSuccess; i++) {
        e = launch_dit_linear_gemm(s, y, n, m->wx, D, lat, m->bx, u16(m->bxe.p));
        if (e == hipSuccess)
            e = launch_cfm_rows_batch(s, u16(m->t_emb.p) + (size_t)i * 2 * D, u16(m->bce.p), m->bc, u16(m->bxh.p),
                                      u16(m->bxe.p), n, D, u16(m->brows[0].p));
        int cur = 0;
        for (size_t bl = 0; bl < m->blocks.size() && e == hipSuccess; bl++) {
            // each block leaves the next one's rms1 of its output in bhn (fused into its ff2 reduce)
            e = launch_dit_block_gemm(s, m->blocks[bl], u16(m->brows[cur].p), R, L,
                                      static_cast<const float*>(m->cos.p), static_cast<const float*>(m->sin.p),
                                      u16(m->bhn.p), u16(m->bqkv.p), u16(m->batt.p), u16(m->bx1.p), u16(m->bhh.p),
                                      u16(m->brows[cur ^ 1].p), static_cast<float*>(m->bpart.p), bl > 0,
                                      bl + 1 < m->blocks.size() ? &m->blocks[bl + 1] : nullptr);
            cur ^= 1;
        }
        if (e == hipSuccess)
            e = launch_cfm_final_batch(s, u16(m->brows[cur].p), n, L, D, m->final_norm, eps, m->wf, m->bf, lat, y,
                                       u16(m->dtd.p), u16(m->sqd.p), u16(sde), i, kFlowSteps, cfg, shift,
                                       u16(m->bhf.p), u16(m->by[yi].p), u16(y_steps));
        y = u16(m->by[yi].p);
        yi ^= 1;
    }
    if (e == hipSuccess)
        e = hipMemcpyAsync(latents_out, y, (size_t)n * lat * b2, hipMemcpyDeviceToDevice, s);
    return hip_check(ctx, e, "cfm_sample_batch");
}

// ---- aggregator ---------------------------------------------------------------------

int ming_agg_model_create(ming_ctx* ctx, const ming_agg_w* w, ming_agg_model** out) {
    if (!alive(ctx)) return MING_E_NOT_INIT;
    if (!w || !out || !w->blocks || w->n_blocks <= 0 || !w->inv_freq)
        return set_err(ctx, MING_E_ARG, "agg_model_create: bad arguments");
    *out = nullptr;
    const ming_dit_cfg* c = &w->cfg;
    int st;
    if ((st = check_cfg(ctx, c))) return st;
    for (int i = 0; i < w->n_blocks; i++)
        if ((st = check_block(ctx, c, &w->blocks[i]))) return st;
    if ((st = check_rows(ctx, 1, 2, "agg_model_create"))) return st;
    const int D = c->hidden, latent = w->x_emb.in_features, H = w->final.out_features;
    if ((st = check_bf16(ctx, w->x_emb, D, latent, "x_emb")) || (st = check_bf16(ctx, w->final, H, D, "final")))
        return st;
    if (!w->bx || !w->cls || !w->final_norm || !w->bf) return set_err(ctx, MING_E_ARG, "agg_model_create: null bias");
    auto* m = new ming_agg_model;
    m->ctx = ctx;
    m->cfg = *c;
    for (int i = 0; i < w->n_blocks; i++) m->blocks.push_back(block_dev(c, &w->blocks[i]));
    m->wx = u16(w->x_emb.w);
    m->bx = u16(w->bx);
    m->cls = u16(w->cls);
    m->wf = u16(w->final.w);
    m->bf = u16(w->bf);
    m->final_norm = u16(w->final_norm);
    m->latent = latent;
    m->lm_hidden = H;
    const int half = c->head_dim / 2, L = 2;
    hipError_t e = m->cos.ensure(sizeof(float) * L * half);
    if (e == hipSuccess) e = m->sin.ensure(sizeof(float) * L * half);
    if (e == hipSuccess) e = m->s.alloc(L, D, c->ff);
    if (e == hipSuccess) e = m->in.ensure(sizeof(uint16_t) * 2 * (size_t)D);
    if (e == hipSuccess) e = hipMemcpy(m->in.p, m->cls, sizeof(uint16_t) * D, hipMemcpyDeviceToDevice);
    if (e != hipSuccess) {
        ming_agg_model_destroy(m);
        return hip_check(ctx, e, "agg_model_create");
    }
    if ((st = rotary_upload(ctx, w->inv_freq, half, L, static_cast<float*>(m->cos.p), static_cast<float*>(m->sin.p)))) {
        ming_agg_model_destroy(m);
        return st;
    }
    *out = m;
    return MING_OK;
}

int ming_agg_model_destroy(ming_agg_model* m) {
    if (!m) return MING_E_NOT_INIT;
    m->cos.release();
    m->sin.release();
    m->in.release();
    m->s.release();
    delete m;
    return MING_OK;
}

}  // extern "C"

namespace {

// aggregate; with rows_out (device bf16 [n_blocks + 1][2][hidden]) each block's
// input rows and the stack output are copied out as well (the same launches).
int aggregate_impl(ming_ctx* ctx, ming_agg_model* m, const void* latent, void* out, void* rows_out) {
    if (!alive(ctx)) return MING_E_NOT_INIT;
    if (!m) return set_err(ctx, MING_E_NOT_INIT, "aggregate: null model");
    if (!latent || !out) return set_err(ctx, MING_E_ARG, "aggregate: null buffer");
    hipStream_t s = ctx->stream;
    const int D = m->cfg.hidden;
    const size_t rb = sizeof(uint16_t) * 2 * D;
    auto keep = [&](int i, const void* rows) {
        return rows_out ? hipMemcpyAsync(static_cast<char*>(rows_out) + (size_t)i * rb, rows, rb,
                                         hipMemcpyDeviceToDevice, s)
                        : hipSuccess;
    };
    // h = [cls, x_emb(latent)] (:1046-1050): row 0 of m->in holds cls since creation
    uint16_t* in = u16(m->in.p);
    hipError_t e = launch_dit_linear(s, u16(latent), 0, 1, 1, nullptr, 0.0f, m->wx, D, m->latent, m->bx, in + D, false);
    uint16_t* h = nullptr;
    if (e == hipSuccess && !rows_out) {
        e = run_stack(s, m->blocks, m->s, 1, 2, static_cast<const float*>(m->cos.p),
                      static_cast<const float*>(m->sin.p), &h, in);
    } else if (e == hipSuccess) {  // run_stack's launches one block at a time, keeping each input
        int cur = 0;
        h = in;
        for (size_t i = 0; i < m->blocks.size() && e == hipSuccess; i++) {
            e = keep((int)i, h);
            if (e == hipSuccess)
                e = launch_dit_block(s, m->blocks[i], h, 1, 2, static_cast<const float*>(m->cos.p),
                                     static_cast<const float*>(m->sin.p), u16(m->s.qkv.p), u16(m->s.att.p),
                                     u16(m->s.x1.p), u16(m->s.hh.p), u16(m->s.rows[cur ^ 1].p), true);
            cur ^= 1;
            h = u16(m->s.rows[cur].p);
        }
        if (e == hipSuccess) e = keep((int)m->blocks.size(), h);
    }
    // final(rms(h)) on row 0 (:1051-1052)
    if (e == hipSuccess)
        e = launch_dit_linear(s, h, 0, 1, 1, m->final_norm, m->cfg.eps, m->wf, m->lm_hidden, D, m->bf, u16(out),
                              false);
    return hip_check(ctx, e, "aggregate");
}

}  // namespace

extern "C" {

int ming_aggregate(ming_ctx* ctx, ming_agg_model* m, const void* latent, void* out) {
    return aggregate_impl(ctx, m, latent, out, nullptr);
}

int ming_aggregate_trace(ming_ctx* ctx, ming_agg_model* m, const void* latent, void* rows_out, void* out) {
    if (!alive(ctx)) return MING_E_NOT_INIT;
    if (!rows_out) return set_err(ctx, MING_E_ARG, "aggregate_trace: null rows");
    return aggregate_impl(ctx, m, latent, out, rows_out);
}

int ming_stop_prob(ming_ctx* ctx, const ming_linear* head, const void* bias, const void* z, float* p_dev) {
    return stop_prob_impl(ctx, head, bias, z, p_dev, false);
}

}  // extern "C"

// stopProb; with_flags: the context's three error flags follow p in p_dev[1..3]
// (as int32), read after every earlier launch on the stream, so that one copy
// brings both to the host.
int ming::stop_prob_impl(ming_ctx* ctx, const ming_linear* head, const void* bias, const void* z, float* p_dev,
                         bool with_flags) {
    if (!alive(ctx)) return MING_E_NOT_INIT;
    if (!head || !bias || !z || !p_dev) return set_err(ctx, MING_E_ARG, "stop_prob: null argument");
    int st;
    if ((st = check_bf16(ctx, *head, 2, head->in_features, "stop_head"))) return st;
    if (head->in_features > 4096) return set_err(ctx, MING_E_UNSUPPORTED, "stop_prob: hidden > 4096");
    return hip_check(ctx,
                     launch_stop_prob(ctx->stream, u16(z), u16(head->w), u16(bias), head->in_features, p_dev,
                                      with_flags ? ctx->dev_flags : nullptr),
                     "stop_prob launch");
}

// ---- adaLN flow head (config 4) ---------------------------------------------------------

namespace {

int check_adaln_block(ming_ctx* ctx, const ming_dit_cfg* c, const ming_adaln_block_w* w) {
    if (!w) return set_err(ctx, MING_E_ARG, "adaln: null block");
    int st;
    if ((st = check_block(ctx, c, &w->base)) || (st = check_bf16(ctx, w->ada, 6 * c->hidden, c->hidden, "ada")))
        return st;
    if (!w->bada) return set_err(ctx, MING_E_ARG, "adaln: null ada bias");
    return MING_OK;
}

}  // namespace

extern "C" {

int ming_adaln_block(ming_ctx* ctx, const ming_dit_cfg* cfg, const ming_adaln_block_w* w, const void* mod,
                     const void* x, int32_t B, int32_t L, const float* cos_dev, const float* sin_dev,
                     ming_dit_out* out) {
    if (!alive(ctx)) return MING_E_NOT_INIT;
    int st;
    if ((st = check_cfg(ctx, cfg)) || (st = check_adaln_block(ctx, cfg, w))) return st;
    if (B <= 0 || B > 2 || L <= 0 || B * L > 8 || L > 8)
        return set_err(ctx, MING_E_SHAPE, "adaln_block: B must be 1 or 2, B*L <= 8, L <= 8");
    if (!x || !mod || !cos_dev || !sin_dev || !out || !out->qkv || !out->att || !out->x1 || !out->hh || !out->x2)
        return set_err(ctx, MING_E_ARG, "adaln_block: null buffer");
    const DitBlockDev d = block_dev(cfg, &w->base);
    return hip_check(ctx,
                     launch_adaln_block(ctx->stream, d, u16(mod), u16(x), B, L, cos_dev, sin_dev, u16(out->qkv),
                                        u16(out->att), u16(out->x1), u16(out->hh), u16(out->x2)),
                     "adaln_block launch");
}

int ming_adaln_model_create(ming_ctx* ctx, const ming_adaln_w* w, ming_adaln_model** out) {
    if (!alive(ctx)) return MING_E_NOT_INIT;
    if (!w || !out || !w->blocks || w->n_blocks <= 0 || !w->inv_freq)
        return set_err(ctx, MING_E_ARG, "adaln_model_create: bad arguments");
    *out = nullptr;
    const ming_dit_cfg* c = &w->cfg;
    int st;
    if ((st = check_cfg(ctx, c))) return st;
    for (int i = 0; i < w->n_blocks; i++)
        if ((st = check_adaln_block(ctx, c, &w->blocks[i]))) return st;
    const int D = c->hidden, latent = w->x_emb.in_features, H = w->c_emb.in_features, F = w->frames;
    if (F <= 0 || 2 * F > 8) return set_err(ctx, MING_E_SHAPE, "adaln_model_create: frames must be in [1, 4]");
    if ((st = check_bf16(ctx, w->x_emb, D, latent, "x_emb")) || (st = check_bf16(ctx, w->c_emb, D, H, "c_emb")) ||
        (st = check_bf16(ctx, w->t_mlp0, D, 256, "t_mlp0")) || (st = check_bf16(ctx, w->t_mlp2, D, D, "t_mlp2")) ||
        (st = check_bf16(ctx, w->final, latent, D, "final")) ||
        (st = check_bf16(ctx, w->final_ada, 2 * D, D, "final_ada")))
        return st;
    if (H > 4096 || latent > 4096 || latent % 8 != 0)
        return set_err(ctx, MING_E_UNSUPPORTED, "adaln_model_create: latent/LM hidden sizes");
    if (!w->bx || !w->bc || !w->bt0 || !w->bt2 || !w->final_norm || !w->bf || !w->bfa)
        return set_err(ctx, MING_E_ARG, "adaln_model_create: null bias or norm");
    auto* m = new ming_adaln_model;
    m->ctx = ctx;
    m->cfg = *c;
    m->frames = F;
    m->latent = latent;
    m->lm_hidden = H;
    for (int i = 0; i < w->n_blocks; i++) {
        m->blocks.push_back(block_dev(c, &w->blocks[i].base));
        m->ada.push_back(u16(w->blocks[i].ada.w));
        m->bada.push_back(u16(w->blocks[i].bada));
    }
    m->wx = u16(w->x_emb.w);
    m->bx = u16(w->bx);
    m->wc = u16(w->c_emb.w);
    m->bc = u16(w->bc);
    m->wf = u16(w->final.w);
    m->bf = u16(w->bf);
    m->final_norm = u16(w->final_norm);
    m->wfa = u16(w->final_ada.w);
    m->bfa = u16(w->bfa);
    const int half = c->head_dim / 2, rows = 2 * kFlowSteps;
    hipStream_t s = ctx->stream;
    hipError_t e = m->cos.ensure(sizeof(float) * F * half);
    if (e == hipSuccess) e = m->sin.ensure(sizeof(float) * F * half);
    if (e == hipSuccess) e = m->t_emb.ensure(sizeof(uint16_t) * (size_t)kFlowSteps * 2 * D);
    if (e == hipSuccess) e = m->dtd.ensure(sizeof(uint16_t) * kFlowSteps);
    if (e == hipSuccess) e = m->sqd.ensure(sizeof(uint16_t) * kFlowSteps);
    if (e == hipSuccess) e = m->zc.ensure(sizeof(uint16_t) * 2 * (size_t)H);
    if (e == hipSuccess) e = m->ce.ensure(sizeof(uint16_t) * 2 * (size_t)D);
    if (e == hipSuccess) e = m->silu_c.ensure(sizeof(uint16_t) * (size_t)rows * D);
    if (e == hipSuccess) e = m->mods.ensure(sizeof(uint16_t) * (size_t)w->n_blocks * rows * 6 * D);
    if (e == hipSuccess) e = m->modf.ensure(sizeof(uint16_t) * (size_t)rows * 2 * D);
    if (e == hipSuccess) e = m->y.ensure(sizeof(uint16_t) * (size_t)F * latent);
    if (e == hipSuccess) e = m->s.alloc(2 * F, D, c->ff);
    if (e == hipSuccess) e = hipMemsetAsync(m->zc.p, 0, m->zc.bytes, s);
    if (e == hipSuccess)
        e = flow_tables(s, w->t_mlp0, w->bt0, w->t_mlp2, w->bt2, D, m->t, m->dt, m->sq, u16(m->dtd.p), u16(m->sqd.p),
                        u16(m->t_emb.p));
    if (e != hipSuccess) {
        ming_adaln_model_destroy(m);
        return hip_check(ctx, e, "adaln_model_create");
    }
    if ((st = rotary_upload(ctx, w->inv_freq, half, F, static_cast<float*>(m->cos.p), static_cast<float*>(m->sin.p)))) {
        ming_adaln_model_destroy(m);
        return st;
    }
    *out = m;
    return MING_OK;
}

int ming_adaln_model_destroy(ming_adaln_model* m) {
    if (!m) return MING_E_NOT_INIT;
    for (DevBuf* b : {&m->cos, &m->sin, &m->t_emb, &m->dtd, &m->sqd, &m->zc, &m->ce, &m->silu_c, &m->mods, &m->modf,
                      &m->y})
        b->release();
    m->s.release();
    delete m;
    return MING_OK;
}

int ming_adaln_model_tables(ming_adaln_model* m, const void** t_emb_dev, const void** silu_c_dev, const void** mods_dev,
                            const void** modf_dev) {
    if (!m) return MING_E_NOT_INIT;
    if (t_emb_dev) *t_emb_dev = m->t_emb.p;
    if (silu_c_dev) *silu_c_dev = m->silu_c.p;
    if (mods_dev) *mods_dev = m->mods.p;
    if (modf_dev) *modf_dev = m->modf.p;
    return MING_OK;
}

int ming_adaln_sample(ming_ctx* ctx, ming_adaln_model* m, const void* z, const void* noise, const void* sde, float cfg,
                      float sigma, float temperature, void* patch_out, void* y_steps) {
    if (!alive(ctx)) return MING_E_NOT_INIT;
    if (!m) return set_err(ctx, MING_E_NOT_INIT, "adaln_sample: null model");
    const float shift = sigma * std::sqrt(temperature);
    if (!z || !noise || !patch_out || (shift != 0.0f && !sde))
        return set_err(ctx, MING_E_ARG, "adaln_sample: null buffer");
    hipStream_t s = ctx->stream;
    const int D = m->cfg.hidden, H = m->lm_hidden, lat = m->latent, F = m->frames, rows = 2 * kFlowSteps;
    const size_t patch = (size_t)F * lat;
    const float eps = m->cfg.eps;
    // once per token: c_emb([z, 0]), silu(t_emb[s] + c_emb) of every step, and every modulation
    hipError_t e = hipMemcpyAsync(m->zc.p, z, sizeof(uint16_t) * H, hipMemcpyDeviceToDevice, s);
    if (e == hipSuccess)
        e = launch_dit_linear(s, u16(m->zc.p), 0, 1, 2, nullptr, eps, m->wc, D, H, m->bc, u16(m->ce.p), false);
    if (e == hipSuccess) e = launch_adaln_cond(s, u16(m->t_emb.p), u16(m->ce.p), kFlowSteps, D, u16(m->silu_c.p));
    for (size_t k = 0; k < m->blocks.size() && e == hipSuccess; k++)
        e = launch_dit_linear(s, u16(m->silu_c.p), 0, 1, rows, nullptr, eps, m->ada[k], 6 * D, D, m->bada[k],
                              u16(m->mods.p) + k * rows * 6 * D, false);
    if (e == hipSuccess)
        e = launch_dit_linear(s, u16(m->silu_c.p), 0, 1, rows, nullptr, eps, m->wfa, 2 * D, D, m->bfa, u16(m->modf.p),
                              false);
    if (e == hipSuccess) e = hipMemcpyAsync(m->y.p, noise, sizeof(uint16_t) * patch, hipMemcpyDeviceToDevice, s);
    uint16_t* y = u16(m->y.p);
    for (int i = 0; i < kFlowSteps && e == hipSuccess; i++) {
        e = launch_adaln_rows(s, y, F, m->wx, m->bx, D, lat, u16(m->s.rows[0].p));
        int cur = 0;
        for (size_t k = 0; k < m->blocks.size() && e == hipSuccess; k++) {
            const uint16_t* mk = u16(m->mods.p) + (k * rows + 2 * (size_t)i) * 6 * D;
            e = launch_adaln_block(s, m->blocks[k], mk, u16(m->s.rows[cur].p), 2, F, static_cast<const float*>(m->cos.p),
                                   static_cast<const float*>(m->sin.p), u16(m->s.qkv.p), u16(m->s.att.p),
                                   u16(m->s.x1.p), u16(m->s.hh.p), u16(m->s.rows[cur ^ 1].p));
            cur ^= 1;
        }
        if (e == hipSuccess)
            e = launch_adaln_final(s, u16(m->s.rows[cur].p), F, D, m->final_norm, eps,
                                   u16(m->modf.p) + (size_t)2 * i * 2 * D, m->wf, m->bf, lat, y, u16(m->dtd.p),
                                   u16(m->sqd.p), u16(sde), i, cfg, shift, y);
        if (e == hipSuccess && y_steps)
            e = hipMemcpyAsync(u16(y_steps) + (size_t)i * patch, y, sizeof(uint16_t) * patch, hipMemcpyDeviceToDevice,
                               s);
    }
    if (e == hipSuccess) e = hipMemcpyAsync(patch_out, y, sizeof(uint16_t) * patch, hipMemcpyDeviceToDevice, s);
    return hip_check(ctx, e, "adaln_sample");
}

}  // extern "C"
