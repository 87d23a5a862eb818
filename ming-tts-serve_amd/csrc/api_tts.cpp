// C-ABI glue of the per-token TTS loop (include/ming_hip.h, "per-token
// loop"): sampleLatents (src/ming_model.zig:1388-1480) over the library's own
// handles -- prefill of the prompt rows, then per step the flow head
// (cfmSample), the aggregator and one LM decode step for the next position,
// and the stop head -- pipelined one step ahead like the reference: step k
// enqueues CFM(k) and the LM pass for k+1 before the host reads stop_k, so
// the GPU is never idle while the host decides whether to stop.
#include <cstring>
#include <string>
#include <vector>

#include "batch.h"
#include "internal.h"

using namespace ming;

namespace {

constexpr int kFlowSteps = 10;  // FLOW_STEPS (src/ming_model.zig:48)

bool alive(const ming_ctx* c) { return c && c->alive; }

// What the host reads per step: the stop probability and, copied in the
// same stream order, the context's device error flags ([0] a bounded wait
// expired, [1] a paged position out of range, [2] a gather index out of
// range), so a step whose device waits gave up is seen before its stop value
// is trusted.
struct StopSlot {
    float p;
    int32_t flags[3];
};

// Workspace of one call; released after the stream has drained (an error
// return can leave queued work that still reads it).
struct LoopBufs {
    hipStream_t s = nullptr;
    DevBuf z, xrow, hist;
    StopSlot* host_stop = nullptr;  // pinned [2], written by the stop launch
    hipEvent_t ev[2] = {nullptr, nullptr};
    ~LoopBufs() {
        if (s) (void)hipStreamSynchronize(s);
        for (DevBuf* b : {&z, &xrow, &hist}) b->release();
        if (host_stop) (void)hipHostFree(host_stop);
        for (hipEvent_t& e : ev)
            if (e) (void)hipEventDestroy(e);
    }
};

// Buffers of the batched prompt pass; released after the stream has drained.
struct PrefillBufs {
    hipStream_t s = nullptr;
    ming_lm_batch* batch = nullptr;
    DevBuf kp, vp, table, hid;
    std::vector<int32_t> ids;  // host source of the page table's upload
    ~PrefillBufs() {
        if (s) (void)hipStreamSynchronize(s);
        if (batch) (void)ming_lm_batch_destroy(batch);
        for (DevBuf* b : {&kp, &vp, &table, &hid}) b->release();
    }
};

// The prompt rows as one multi-row forward (QStack.forward over the prompt,
// src/ming_model.zig:576-614): ming_lm_prefill over a page pool of its own
// (pages 0, 1, 2, ... in position order), then the pages copied into kv rows
// [0, L) and z = the last row's final-normed hidden.  Returns
// MING_E_UNSUPPORTED, with the context's error text left as it was, when the
// batched step does not run this model (not 4-bit, head_dim not 64).
int prefill_batched(ming_ctx* ctx, ming_lm_model* lm, const uint16_t* emb, int L, ming_kv* kv, uint16_t* z, int H,
                    PrefillBufs& pb) {
    LmView v;
    if (!lm_model_view(lm, v)) return set_err(ctx, MING_E_NOT_INIT, "sample_latents: null LM model");
    if (!kv->k || !kv->v) return set_err(ctx, MING_E_ARG, "sample_latents: null kv cache");
    if (kv->kv_heads != v.cfg.kv_heads || kv->head_dim != v.cfg.head_dim || kv->n_layers != v.cfg.n_layers)
        return set_err(ctx, MING_E_SHAPE, "sample_latents: kv cache geometry does not match the model");
    hipStream_t s = ctx->stream;
    const int n_pages = (L + 63) / 64;
    const std::string err = ctx->err;
    // the prompt in chunks of up to 512 rows (one GEMM call per linear per chunk)
    int st = ming_lm_batch_create(ctx, lm, L < kQgemmMaxRows ? L : kQgemmMaxRows, n_pages * 64, &pb.batch);
    if (st == MING_E_UNSUPPORTED) {
        ctx->err = err;
        return st;
    }
    if (st) return st;
    pb.s = s;
    const size_t page_bytes = (size_t)kv->n_layers * n_pages * kv->kv_heads * 64 * 64 * sizeof(uint16_t);
    hipError_t e = pb.kp.ensure(page_bytes);
    if (e == hipSuccess) e = pb.vp.ensure(page_bytes);
    if (e == hipSuccess) e = pb.table.ensure(sizeof(int32_t) * n_pages);
    if (e == hipSuccess) e = pb.hid.ensure(sizeof(uint16_t) * (size_t)L * H);
    // unwritten positions of the last page are masked out of attention; zeros keep them finite
    if (e == hipSuccess) e = hipMemsetAsync(pb.kp.p, 0, page_bytes, s);
    if (e == hipSuccess) e = hipMemsetAsync(pb.vp.p, 0, page_bytes, s);
    pb.ids.resize(n_pages);
    for (int i = 0; i < n_pages; i++) pb.ids[i] = i;
    if (e == hipSuccess)
        e = hipMemcpyAsync(pb.table.p, pb.ids.data(), sizeof(int32_t) * n_pages, hipMemcpyHostToDevice, s);
    if ((st = hip_check(ctx, e, "sample_latents prefill buffers"))) return st;
    const ming_kv_pages pages{pb.kp.p, pb.vp.p, kv->n_layers, kv->kv_heads, kv->head_dim, 64, n_pages};
    if ((st = ming_lm_prefill(pb.batch, L, nullptr, emb, &pages, static_cast<const int32_t*>(pb.table.p), n_pages, 0,
                              pb.hid.p, nullptr, nullptr)))
        return st;
    e = launch_pages_to_rows(s, static_cast<const uint16_t*>(pb.kp.p), static_cast<const uint16_t*>(pb.vp.p),
                             kv->n_layers, kv->kv_heads, n_pages, 0, L, static_cast<uint16_t*>(kv->k),
                             static_cast<uint16_t*>(kv->v), kv->capacity);
    if (e == hipSuccess)
        e = hipMemcpyAsync(z, static_cast<const uint16_t*>(pb.hid.p) + (size_t)(L - 1) * H, sizeof(uint16_t) * H,
                           hipMemcpyDeviceToDevice, s);
    if ((st = hip_check(ctx, e, "sample_latents prefill copy"))) return st;
    kv->len = L;
    return MING_OK;
}

}  // namespace

extern "C" {

int ming_noise_bank(ming_ctx* ctx, uint64_t seed, int32_t steps, int32_t latent, void* bank_dev) {
    if (!alive(ctx)) return MING_E_NOT_INIT;
    if (!bank_dev || steps <= 0 || latent <= 0) return set_err(ctx, MING_E_ARG, "noise_bank: bad arguments");
    const size_t n = (size_t)steps * (kFlowSteps + 1) * latent;
    std::vector<uint16_t> h(n);
    ming_synth_normal_bf16(ming_synth_stream(seed, "flow.noise"), 0.0f, 1.0f, h.data(), n, 8);
    int st = hip_check(ctx, hipMemcpyAsync(bank_dev, h.data(), n * 2, hipMemcpyHostToDevice, ctx->stream),
                       "noise_bank upload");
    if (st) return st;
    return hip_check(ctx, hipStreamSynchronize(ctx->stream), "noise_bank");
}

int ming_sample_latents(ming_ctx* ctx, ming_lm_model* lm, ming_cfm_model* cfm, ming_agg_model* agg,
                        const ming_linear* stop_head, const void* stop_bias, const void* embeds, int32_t L,
                        const void* prompt_latent, ming_kv* kv, const void* noise_bank,
                        const ming_sample_params* p, void* latents_out, int32_t* n_steps_out, float* stop_out,
                        void* z_trace) {
    if (!alive(ctx)) return MING_E_NOT_INIT;
    if (!lm || !cfm || !agg) return set_err(ctx, MING_E_NOT_INIT, "sample_latents: null model");
    if (!stop_head || !stop_bias || !embeds || !kv || !noise_bank || !p || !latents_out || !n_steps_out || L <= 0 ||
        p->max_steps <= 0)
        return set_err(ctx, MING_E_ARG, "sample_latents: bad arguments");
    *n_steps_out = 0;
    int H = 0, lat = 0;
    int st;
    if ((st = ming_lm_model_dims(lm, &H, nullptr)) || (st = ming_cfm_model_dims(cfm, &lat, nullptr))) return st;
    int aggH = 0, aggLat = 0;
    if ((st = ming_agg_model_dims(agg, &aggH, &aggLat))) return st;
    if (aggH != H || aggLat != lat || stop_head->in_features != H)
        return set_err(ctx, MING_E_SHAPE, "sample_latents: LM hidden / latent sizes of the models differ");
    // the reference's budget: the prompt plus one position per step (patch size 1)
    const int budget = kv->capacity - kv->len - L;
    if (budget <= 0) return set_err(ctx, MING_E_CTX_OVER_CAPACITY, "sample_latents: prompt does not fit the cache");
    const int steps = p->max_steps < budget ? p->max_steps : budget;
    hipStream_t s = ctx->stream;
    LoopBufs b;
    b.s = s;
    hipError_t e = b.z.ensure(sizeof(uint16_t) * H);
    if (e == hipSuccess) e = b.xrow.ensure(sizeof(uint16_t) * H);
    if (e == hipSuccess) e = b.hist.ensure(sizeof(uint16_t) * lat);
    // coherent pinned memory: the stop launch stores into it directly
    if (e == hipSuccess)
        e = hipHostMalloc(reinterpret_cast<void**>(&b.host_stop), sizeof(StopSlot) * 2,
                          hipHostMallocMapped | hipHostMallocCoherent);
    for (hipEvent_t& ev : b.ev)
        if (e == hipSuccess) e = hipEventCreateWithFlags(&ev, hipEventDisableTiming);
    if ((st = hip_check(ctx, e, "sample_latents workspace"))) return st;
    uint16_t* z = static_cast<uint16_t*>(b.z.p);
    // the aggregator writes the LM step's input row in place
    uint16_t* xrow = lm_input_row(lm) ? lm_input_row(lm) : static_cast<uint16_t*>(b.xrow.p);
    const uint16_t* emb = static_cast<const uint16_t*>(embeds);
    uint16_t* lats = static_cast<uint16_t*>(latents_out);
    const uint16_t* bank = static_cast<const uint16_t*>(noise_bank);
    // prefill; z = the last row's final-normed hidden.  An empty cache takes the
    // prompt in one batched pass where the model allows it; otherwise (or when
    // continuing a cache) one decode step per prompt row.
    PrefillBufs pb;
    st = kv->len == 0 && kv->head_dim == 64 && L > 1 ? prefill_batched(ctx, lm, emb, L, kv, z, H, pb)
                                                     : MING_E_UNSUPPORTED;
    if (st == MING_E_UNSUPPORTED) {
        for (int i = 0; i < L; i++)
            if ((st = ming_lm_step(ctx, lm, nullptr, emb + (size_t)i * H, kv, z, nullptr, nullptr))) return st;
    } else if (st) {
        return st;
    }
    // history: the prompt's last latent, or zeros (history_patch_size 1)
    e = prompt_latent ? hipMemcpyAsync(b.hist.p, prompt_latent, sizeof(uint16_t) * lat, hipMemcpyDeviceToDevice, s)
                      : hipMemsetAsync(b.hist.p, 0, sizeof(uint16_t) * lat, s);
    if ((st = hip_check(ctx, e, "sample_latents history"))) return st;
    const uint16_t* hist = static_cast<const uint16_t*>(b.hist.p);
    // Before each flow-head sample, one launch (cfm_pre) runs its c_emb(z) and x_emb(hist) and the
    // stop head on z, whose probability and the error flags land directly in the pinned host slot
    // k & 1; an event after it tells the host when they are there.
    static_assert(sizeof(StopSlot) == 4 * sizeof(float), "p and three flags");
    auto pre = [&](int slot, const uint16_t* h) {
        int r = cfm_pre(ctx, cfm, z, h, stop_head, stop_bias, reinterpret_cast<float*>(&b.host_stop[slot]));
        if (r) return r;
        return hip_check(ctx, hipEventRecord(b.ev[slot], s), "sample_latents stop event");
    };
    if ((st = pre(0, hist))) return st;
    int n = 0;
    for (int k = 0; k < steps; k++) {
        if (z_trace && (st = hip_check(ctx,
                                       hipMemcpyAsync(static_cast<uint16_t*>(z_trace) + (size_t)k * H, z,
                                                      sizeof(uint16_t) * H, hipMemcpyDeviceToDevice, s),
                                       "sample_latents z trace")))
            return st;
        const uint16_t* noise = bank + (size_t)k * (kFlowSteps + 1) * lat;
        uint16_t* latent = lats + (size_t)k * lat;
        if ((st = cfm_sample_impl(ctx, cfm, z, hist, noise, noise + lat, p->cfg, p->sigma, p->temperature, latent,
                                  nullptr, true)))
            return st;
        const int nxt = (k + 1) & 1;
        if (k + 1 < steps) {  // the next position, queued before the host reads stop_k
            if ((st = ming_aggregate(ctx, agg, latent, xrow)) ||
                (st = ming_lm_step(ctx, lm, nullptr, xrow, kv, z, nullptr, nullptr)) || (st = pre(nxt, latent)))
                return st;
        }
        if ((st = hip_check(ctx, hipEventSynchronize(b.ev[k & 1]), "sample_latents stop wait"))) return st;
        const StopSlot& slot = b.host_stop[k & 1];
        // a raised flag means this step's values (and every later one) are not meaningful:
        // stop here and let ming_sync report it
        if (slot.flags[0] || slot.flags[1] || slot.flags[2]) break;
        const float sp = slot.p;
        if (stop_out) stop_out[k] = sp;
        n = k + 1;
        if (sp > 0.5f && k > 3) break;
        hist = latent;
    }
    // the LM pass queued for a step that did not run is discarded, as in the reference;
    // ming_sync drains the stream and reports (and clears) any device error flag, which also
    // makes the next persistent step reset its arrival counters after a timeout
    if ((st = ming_sync(ctx))) return st;
    *n_steps_out = n;
    return MING_OK;
}

}  // extern "C"
