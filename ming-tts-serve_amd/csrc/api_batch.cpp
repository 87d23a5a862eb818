// C-ABI glue of the multi-request decode (include/ming_hip.h, "Multi-request
// decode over a paged KV cache"): workspace, argument checks and the launch
// sequence of one batched step.  The reference has no counterpart (its
// service decodes one request at a time, src/ming_service.zig:11-14); the
// per-sequence arithmetic is the batch-1 layer's (src/ming_model.zig:566-614).
#include <cstring>
#include <vector>

#include "args.h"
#include "batch.h"
#include "internal.h"

using namespace ming;

struct ming_lm_batch {
    ming_ctx* ctx = nullptr;
    LmView view{};
    std::vector<LayerDev> layers;
    int max_seqs = 0, max_ctx = 0, last_n = 0;
    int H = 0, kvd = 0, nq = 0, I = 0, V = 0, L = 0;
    // every layer's activations, [layer][max_seqs][width]
    DevBuf x, x1, qkv, att, hh;
    DevBuf xs, xsum, part, pmax, pidx, hid, rope;
    DevBuf prows, ppos;  // prefill: page-table rows and positions of one chunk
};

namespace {

bool alive(const ming_ctx* c) { return c && c->alive; }

bool q4(const LinearDev& l) { return l.kind == 1; }

}  // namespace

extern "C" {

int ming_lm_batch_create(ming_ctx* ctx, ming_lm_model* m, int32_t max_seqs, int32_t max_ctx, ming_lm_batch** out) {
    if (!alive(ctx)) return MING_E_NOT_INIT;
    if (!out) return set_err(ctx, MING_E_ARG, "lm_batch_create: null out");
    *out = nullptr;
    LmView v;
    if (!lm_model_view(m, v)) return set_err(ctx, MING_E_NOT_INIT, "lm_batch_create: null model");
    const ming_lm_cfg& c = v.cfg;
    if (max_seqs < 1 || max_seqs > kQgemmMaxRows)
        return set_err(ctx, MING_E_UNSUPPORTED, "lm_batch_create: 1..512 sequences (rows of a prefill chunk)");
    if (max_ctx < 64 || max_ctx % 64) return set_err(ctx, MING_E_ARG, "lm_batch_create: max_ctx must be a positive multiple of 64");
    if (c.head_dim != 64 || c.hidden % 64 || c.inter % 64 || c.heads % c.kv_heads || c.heads / c.kv_heads > 16)
        return set_err(ctx, MING_E_UNSUPPORTED,
                       "lm_batch_create: needs head_dim 64, hidden and inter multiples of 64, <= 16 heads per kv head");
    for (int l = 0; l < c.n_layers; l++) {
        const LayerDev& d = v.layers[l];
        if (!q4(d.q) || !q4(d.k) || !q4(d.v) || !q4(d.o) || !q4(d.g) || !q4(d.u) || !q4(d.d))
            return set_err(ctx, MING_E_UNSUPPORTED, "lm_batch_create: the batched step takes 4-bit linears only");
    }
    if (!q4(v.head)) return set_err(ctx, MING_E_UNSUPPORTED, "lm_batch_create: the batched step takes a 4-bit head only");
    auto* b = new ming_lm_batch();
    b->ctx = ctx;
    b->view = v;
    b->layers.assign(v.layers, v.layers + c.n_layers);
    b->view.layers = b->layers.data();
    b->max_seqs = max_seqs;
    b->max_ctx = max_ctx;
    b->H = c.hidden;
    b->kvd = c.kv_heads * c.head_dim;
    b->nq = b->H + 2 * b->kvd;
    b->I = c.inter;
    b->V = c.vocab;
    b->L = c.n_layers;
    const size_t S = (size_t)max_seqs, L = (size_t)c.n_layers, Mp = (S + 15) / 16 * 16;
    const size_t kmax = (size_t)(b->I > b->H ? b->I : b->H);
    hipError_t e = hipSuccess;
    auto grab = [&](DevBuf& d, size_t bytes) {
        if (e == hipSuccess) e = d.ensure(bytes);
        if (e == hipSuccess) e = hipMemsetAsync(d.p, 0, bytes, ctx->stream);
    };
    grab(b->x, (L + 1) * S * b->H * 2);
    grab(b->x1, L * S * b->H * 2);
    grab(b->att, L * S * b->H * 2);
    grab(b->qkv, L * S * b->nq * 2);
    grab(b->hh, L * S * b->I * 2);
    grab(b->xs, Mp * kmax * 2);
    grab(b->xsum, Mp * (kmax / 64) * 4);
    const size_t nblk = ((size_t)b->V + 31) / 32;  // column blocks of the head GEMM (at most)
    grab(b->pmax, S * nblk * 4);
    grab(b->pidx, S * nblk * 4);
    grab(b->hid, S * b->H * 2);
    grab(b->prows, S * (size_t)(max_ctx / 64) * 4);
    grab(b->ppos, S * 4);
    grab(b->rope, (size_t)max_ctx * 32 * 2 * 4);
    const int max_splits = (max_ctx / 64 + 3) / 4;
    grab(b->part, S * c.kv_heads * max_splits * (c.heads / c.kv_heads) * 68 * 4);
    if (e == hipSuccess)
        e = launch_rope_table(ctx->stream, static_cast<float*>(b->rope.p), max_ctx, 32, c.log2_theta);
    if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
    if (e != hipSuccess) {
        ming_lm_batch_destroy(b);
        return hip_check(ctx, e, "lm_batch_create: workspace");
    }
    *out = b;
    return MING_OK;
}

int ming_lm_batch_destroy(ming_lm_batch* b) {
    if (!b) return MING_OK;
    // the context may already be destroyed: wait for the device, not its stream
    (void)hipDeviceSynchronize();
    for (DevBuf* d : {&b->x, &b->x1, &b->qkv, &b->att, &b->hh, &b->xs, &b->xsum, &b->part, &b->pmax, &b->pidx,
                      &b->hid, &b->rope, &b->prows, &b->ppos})
        d->release();
    delete b;
    return MING_OK;
}

int ming_lm_batch_step(ming_lm_batch* b, int32_t n_seq, const int32_t* tokens_dev, const void* x_in,
                       const ming_kv_pages* kv, const int32_t* page_table_dev, int32_t pages_per_seq, int32_t* pos_dev,
                       void* hidden_out, float* logits_out, int32_t* argmax_out) {
    if (!b || !alive(b->ctx)) return MING_E_NOT_INIT;
    ming_ctx* ctx = b->ctx;
    const ming_lm_cfg& c = b->view.cfg;
    if (n_seq < 1 || n_seq > b->max_seqs)
        return set_err(ctx, MING_E_ARG, "lm_batch_step: n_seq outside [1, max_seqs]");
    if (!tokens_dev && !x_in) return set_err(ctx, MING_E_ARG, "lm_batch_step: need tokens_dev or x_in");
    if (!kv || !kv->k || !kv->v || !page_table_dev || !pos_dev)
        return set_err(ctx, MING_E_ARG, "lm_batch_step: null cache, page table or positions");
    if (kv->n_layers != c.n_layers || kv->kv_heads != c.kv_heads || kv->head_dim != c.head_dim ||
        kv->page_size != 64 || kv->n_pages < 1)
        return set_err(ctx, MING_E_SHAPE, "lm_batch_step: paged cache does not match the model (page_size 64)");
    if (pages_per_seq < 1 || (int64_t)pages_per_seq * 64 > b->max_ctx)
        return set_err(ctx, MING_E_CTX_OVER_CAPACITY, "lm_batch_step: pages_per_seq * 64 exceeds max_ctx");
    hipStream_t st = ctx->stream;
    const int H = b->H, I = b->I, nq = b->nq, S = b->max_seqs;
    const int grp = c.heads / c.kv_heads, max_splits = (pages_per_seq + 3) / 4;
    uint16_t* X = static_cast<uint16_t*>(b->x.p);
    uint16_t* X1 = static_cast<uint16_t*>(b->x1.p);
    uint16_t* QKV = static_cast<uint16_t*>(b->qkv.p);
    uint16_t* ATT = static_cast<uint16_t*>(b->att.p);
    uint16_t* HH = static_cast<uint16_t*>(b->hh.p);
    float* xsum = static_cast<float*>(b->xsum.p);
    int32_t* flags = ctx->dev_flags + 1;
    const size_t page_elems = (size_t)kv->n_pages * c.kv_heads * 64 * 64;
    hipError_t e;
    if (tokens_dev)
        e = launch_embed_rows(st, b->view.embed, tokens_dev, n_seq, X);
    else
        e = hipMemcpyAsync(X, x_in, (size_t)n_seq * H * 2, hipMemcpyDeviceToDevice, st);
    auto gemm = [&](const LinearDev* const* lin, int nseg, const uint16_t* const* bias, int epi, uint16_t* y, int ldy,
                    const uint16_t* res, float* yf, const QPaged* pg) {
        QgemmArgs a{};
        a.xs = b->xs.p;
        a.xsum = xsum;
        a.M = n_seq;
        a.K = lin[0]->K;
        a.nseg = nseg;
        int col = 0;
        for (int i = 0; i < nseg; i++) {
            a.seg[i] = QSeg{lin[i]->w, lin[i]->s, lin[i]->b, bias ? bias[i] : nullptr, lin[i]->N, col, lin[i]->gscale};
            if (epi != QE_SWIGLU) col += lin[i]->N;
        }
        a.y = y;
        a.yf = yf;
        a.ldy = ldy;
        a.res = res;
        a.ldres = ldy;
        if (pg) a.pg = *pg;
        return launch_qgemm_epi(st, a, epi);
    };
    for (int l = 0; l < c.n_layers && e == hipSuccess; l++) {
        const LayerDev& Ld = b->layers[l];
        uint16_t* x = X + (size_t)l * S * H;
        uint16_t* x1 = X1 + (size_t)l * S * H;
        uint16_t* qkv = QKV + (size_t)l * S * nq;
        uint16_t* att = ATT + (size_t)l * S * H;
        uint16_t* hh = HH + (size_t)l * S * I;
        e = launch_stage(st, x, H, n_seq, H, Ld.ln1, c.eps, b->xs.p, xsum, nullptr, nullptr);
        if (e != hipSuccess) break;
        QPaged pg{};
        pg.kp = static_cast<uint16_t*>(kv->k) + (size_t)l * page_elems;
        pg.vp = static_cast<uint16_t*>(kv->v) + (size_t)l * page_elems;
        pg.table = page_table_dev;
        pg.pos = pos_dev;
        pg.rope_cs = static_cast<const float*>(b->rope.p);
        pg.flags = flags;
        pg.pages_per_seq = pages_per_seq;
        pg.n_pages = kv->n_pages;
        pg.kvh = c.kv_heads;
        pg.max_ctx = b->max_ctx;
        const LinearDev* qkvl[3] = {&Ld.q, &Ld.k, &Ld.v};
        const uint16_t* qkvb[3] = {Ld.bq, Ld.bk, Ld.bv};
        e = gemm(qkvl, 3, qkvb, QE_QKV, qkv, nq, nullptr, nullptr, &pg);
        if (e != hipSuccess) break;
        PagedAttnArgs pa{};
        pa.qkv = qkv;
        pa.ldq = nq;
        pa.kp = pg.kp;
        pa.vp = pg.vp;
        pa.table = page_table_dev;
        pa.pos = pos_dev;
        pa.flags = flags;
        pa.part = static_cast<float*>(b->part.p);
        pa.pages_per_seq = pages_per_seq;
        pa.n_pages = kv->n_pages;
        pa.kvh = c.kv_heads;
        pa.grp = grp;
        pa.max_splits = max_splits;
        pa.scale = 0.125f;  // 1/sqrt(64)
        e = launch_paged_attn(st, pa, n_seq);
        if (e != hipSuccess) break;
        MergeArgs ma{pa.part, pos_dev, n_seq, c.heads, c.kv_heads, grp, max_splits, att, b->xs.p, xsum,
                     (n_seq + 15) / 16 * 16};
        e = launch_merge_stage(st, ma);
        if (e != hipSuccess) break;
        const LinearDev* ol[1] = {&Ld.o};
        e = gemm(ol, 1, nullptr, QE_RES, x1, H, x, nullptr, nullptr);
        if (e != hipSuccess) break;
        e = launch_stage(st, x1, H, n_seq, H, Ld.ln2, c.eps, b->xs.p, xsum, nullptr, nullptr);
        if (e != hipSuccess) break;
        const LinearDev* gul[2] = {&Ld.g, &Ld.u};
        e = gemm(gul, 2, nullptr, QE_SWIGLU, hh, I, nullptr, nullptr, nullptr);
        if (e != hipSuccess) break;
        e = launch_stage(st, hh, I, n_seq, I, nullptr, 0.0f, b->xs.p, xsum, nullptr, nullptr);
        if (e != hipSuccess) break;
        const LinearDev* dl[1] = {&Ld.d};
        e = gemm(dl, 1, nullptr, QE_RES, X + (size_t)(l + 1) * S * H, H, x1, nullptr, nullptr);
    }
    if (e == hipSuccess) {
        uint16_t* hout = hidden_out ? static_cast<uint16_t*>(hidden_out) : static_cast<uint16_t*>(b->hid.p);
        e = launch_stage(st, X + (size_t)c.n_layers * S * H, H, n_seq, H, b->view.final_norm, c.eps, b->xs.p, xsum,
                         hout, pos_dev);
    }
    if (e == hipSuccess && (logits_out || argmax_out)) {
        // the head GEMM writes the f32 logits when asked and per-row argmax partials of each column block
        QgemmArgs a{};
        a.xs = b->xs.p;
        a.xsum = xsum;
        a.M = n_seq;
        a.K = H;
        a.nseg = 1;
        const LinearDev& hd = b->view.head;
        a.seg[0] = QSeg{hd.w, hd.s, hd.b, nullptr, hd.N, 0, hd.gscale};
        a.yf = logits_out;
        a.ldy = b->V;
        if (argmax_out) {
            a.pmax = static_cast<float*>(b->pmax.p);
            a.pidx = static_cast<int32_t*>(b->pidx.p);
        }
        e = launch_qgemm_epi(st, a, QE_PLAIN);
        if (e == hipSuccess && argmax_out)
            e = launch_argmax_partials(st, a.pmax, a.pidx, qgemm_argmax_blocks(n_seq, H, b->V), n_seq, argmax_out);
    }
    if (e != hipSuccess) return hip_check(ctx, e, "lm_batch_step launch");
    b->last_n = n_seq;
    return MING_OK;
}

int ming_lm_prefill(ming_lm_batch* b, int32_t L, const int32_t* tokens_dev, const void* x_in, const ming_kv_pages* kv,
                    const int32_t* page_table_dev, int32_t pages_per_seq, int32_t pos0, void* hidden_out,
                    float* logits_out, int32_t* argmax_out) {
    if (!b || !alive(b->ctx)) return MING_E_NOT_INIT;
    ming_ctx* ctx = b->ctx;
    if (L < 1) return set_err(ctx, MING_E_ARG, "lm_prefill: L < 1");
    if (!tokens_dev && !x_in) return set_err(ctx, MING_E_ARG, "lm_prefill: need tokens_dev or x_in");
    if (!page_table_dev) return set_err(ctx, MING_E_ARG, "lm_prefill: null page table");
    if (pages_per_seq < 1 || (int64_t)pages_per_seq * 64 > b->max_ctx)
        return set_err(ctx, MING_E_CTX_OVER_CAPACITY, "lm_prefill: pages_per_seq * 64 exceeds max_ctx");
    if (pos0 < 0 || (int64_t)pos0 + L > (int64_t)pages_per_seq * 64)
        return set_err(ctx, MING_E_CTX_OVER_CAPACITY, "lm_prefill: pos0 + L exceeds the sequence's pages");
    int32_t* rows = static_cast<int32_t*>(b->prows.p);
    int32_t* pos = static_cast<int32_t*>(b->ppos.p);
    const size_t H = (size_t)b->H, V = (size_t)b->V;
    for (int start = 0; start < L; start += b->max_seqs) {
        const int n = L - start < b->max_seqs ? L - start : b->max_seqs;
        int st = hip_check(ctx, launch_prefill_rows(ctx->stream, page_table_dev, pages_per_seq, n, pos0 + start, rows, pos),
                           "lm_prefill rows");
        if (st) return st;
        st = ming_lm_batch_step(
            b, n, tokens_dev ? tokens_dev + start : nullptr,
            x_in ? static_cast<const uint16_t*>(x_in) + (size_t)start * H : nullptr, kv, rows, pages_per_seq, pos,
            hidden_out ? static_cast<uint16_t*>(hidden_out) + (size_t)start * H : nullptr,
            logits_out ? logits_out + (size_t)start * V : nullptr, argmax_out ? argmax_out + start : nullptr);
        if (st) return st;
    }
    return MING_OK;
}

int ming_lm_batch_trace(ming_lm_batch* b, void* x, void* x1, void* att, void* qkv, void* hh) {
    if (!b || !alive(b->ctx)) return MING_E_NOT_INIT;
    ming_ctx* ctx = b->ctx;
    if (b->last_n < 1) return set_err(ctx, MING_E_ARG, "lm_batch_trace: no step yet");
    const size_t n = (size_t)b->last_n, S = (size_t)b->max_seqs, L = (size_t)b->L;
    hipError_t e = hipSuccess;
    auto cp = [&](void* dst, const DevBuf& src, size_t width, size_t layers) {
        if (!dst || e != hipSuccess) return;
        e = hipMemcpy2DAsync(dst, n * width * 2, src.p, S * width * 2, n * width * 2, layers, hipMemcpyDeviceToDevice,
                             ctx->stream);
    };
    cp(x, b->x, b->H, L + 1);
    cp(x1, b->x1, b->H, L);
    cp(att, b->att, b->H, L);
    cp(qkv, b->qkv, b->nq, L);
    cp(hh, b->hh, b->I, L);
    return e == hipSuccess ? MING_OK : hip_check(ctx, e, "lm_batch_trace copy");
}

}  // extern "C"
