// C-ABI glue of the per-token TTS loop (include/ming_hip.h, "per-token
// loop"): sampleLatents (src/ming_model.zig:1388-1480) over the library's own
// handles -- prefill of the prompt rows, then per step the flow head
// (cfmSample), the aggregator and one LM decode step for the next position,
// and the stop head -- pipelined one step ahead like the reference: step k
// enqueues CFM(k) and the LM pass for k+1 before the host reads stop_k, so
// the GPU is never idle while the host decides whether to stop.
#include <cstring>
#include <vector>

#include "internal.h"

using namespace ming;

namespace {

constexpr int kFlowSteps = 10;  // FLOW_STEPS (src/ming_model.zig:48)

bool alive(const ming_ctx* c) { return c && c->alive; }

// Workspace of one call; released after the stream has drained (an error
// return can leave queued work that still reads it).
struct LoopBufs {
    hipStream_t s = nullptr;
    DevBuf z, xrow, hist, stop;
    float* host_stop = nullptr;  // pinned [2]
    hipEvent_t ev[2] = {nullptr, nullptr};
    ~LoopBufs() {
        if (s) (void)hipStreamSynchronize(s);
        for (DevBuf* b : {&z, &xrow, &hist, &stop}) b->release();
        if (host_stop) (void)hipHostFree(host_stop);
        for (hipEvent_t& e : ev)
            if (e) (void)hipEventDestroy(e);
    }
};

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
    if (e == hipSuccess) e = b.stop.ensure(sizeof(float) * 2);
    if (e == hipSuccess) e = hipHostMalloc(reinterpret_cast<void**>(&b.host_stop), sizeof(float) * 2);
    for (hipEvent_t& ev : b.ev)
        if (e == hipSuccess) e = hipEventCreateWithFlags(&ev, hipEventDisableTiming);
    if ((st = hip_check(ctx, e, "sample_latents workspace"))) return st;
    uint16_t* z = static_cast<uint16_t*>(b.z.p);
    uint16_t* xrow = static_cast<uint16_t*>(b.xrow.p);
    float* stop_dev = static_cast<float*>(b.stop.p);
    const uint16_t* emb = static_cast<const uint16_t*>(embeds);
    uint16_t* lats = static_cast<uint16_t*>(latents_out);
    const uint16_t* bank = static_cast<const uint16_t*>(noise_bank);
    // prefill: one decode step per prompt row; z = the last row's final-normed hidden
    for (int i = 0; i < L; i++)
        if ((st = ming_lm_step(ctx, lm, nullptr, emb + (size_t)i * H, kv, z, nullptr, nullptr))) return st;
    // history: the prompt's last latent, or zeros (history_patch_size 1)
    e = prompt_latent ? hipMemcpyAsync(b.hist.p, prompt_latent, sizeof(uint16_t) * lat, hipMemcpyDeviceToDevice, s)
                      : hipMemsetAsync(b.hist.p, 0, sizeof(uint16_t) * lat, s);
    if ((st = hip_check(ctx, e, "sample_latents history"))) return st;
    const uint16_t* hist = static_cast<const uint16_t*>(b.hist.p);
    // stop_0 on its way to the host
    if ((st = ming_stop_prob(ctx, stop_head, stop_bias, z, stop_dev))) return st;
    e = hipMemcpyAsync(b.host_stop, stop_dev, sizeof(float), hipMemcpyDeviceToHost, s);
    if (e == hipSuccess) e = hipEventRecord(b.ev[0], s);
    if ((st = hip_check(ctx, e, "sample_latents stop copy"))) return st;
    int n = 0;
    for (int k = 0; k < steps; k++) {
        if (z_trace && (st = hip_check(ctx,
                                       hipMemcpyAsync(static_cast<uint16_t*>(z_trace) + (size_t)k * H, z,
                                                      sizeof(uint16_t) * H, hipMemcpyDeviceToDevice, s),
                                       "sample_latents z trace")))
            return st;
        const uint16_t* noise = bank + (size_t)k * (kFlowSteps + 1) * lat;
        uint16_t* latent = lats + (size_t)k * lat;
        if ((st = ming_cfm_sample(ctx, cfm, z, hist, noise, noise + lat, p->cfg, p->sigma, p->temperature, latent,
                                  nullptr)))
            return st;
        const int nxt = (k + 1) & 1;
        if (k + 1 < steps) {  // the next position, queued before the host reads stop_k
            if ((st = ming_aggregate(ctx, agg, latent, xrow)) ||
                (st = ming_lm_step(ctx, lm, nullptr, xrow, kv, z, nullptr, nullptr)) ||
                (st = ming_stop_prob(ctx, stop_head, stop_bias, z, stop_dev + nxt)))
                return st;
            e = hipMemcpyAsync(b.host_stop + nxt, stop_dev + nxt, sizeof(float), hipMemcpyDeviceToHost, s);
            if (e == hipSuccess) e = hipEventRecord(b.ev[nxt], s);
            if ((st = hip_check(ctx, e, "sample_latents stop copy"))) return st;
        }
        if ((st = hip_check(ctx, hipEventSynchronize(b.ev[k & 1]), "sample_latents stop wait"))) return st;
        const float sp = b.host_stop[k & 1];
        if (stop_out) stop_out[k] = sp;
        n = k + 1;
        if (sp > 0.5f && k > 3) break;
        hist = latent;
    }
    // the LM pass queued for a step that did not run is discarded, as in the reference
    if ((st = hip_check(ctx, hipStreamSynchronize(s), "sample_latents"))) return st;
    *n_steps_out = n;
    return MING_OK;
}

}  // extern "C"
