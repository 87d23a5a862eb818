"""GPU parity of the per-token TTS loop (ming_sample_latents, sampleLatents
src/ming_model.zig:1388-1480) against the oracle, at the reference widths
(LM hidden 896, DiT 1024, latent 64) with 2 LM layers and 2 + 2 DiT blocks.

Each step is recomputed on the oracle from the GPU's own inputs (teacher
forced): z_0 from the prompt prefill, stop_k = stopProb(z_k), latent_k =
cfmSample(z_k, history_k, noise bank row k), aggregate(latent_k) against the
GPU kernel's row, and z_{k+1} = LM(that row) with the oracle's own cache.
Bars: hidden states and aggregator rows 2e-2 + 1e-2 |ref| of the oracle in
its MLX order; stop probabilities 1e-2; the ten-step latent (free running
within the step, as the flow head's own end-to-end test), the aggregator row
and the stop probability bit for bit with the oracle in the kernels'
summation order (and the latent within 6e-2 + 2e-2 |ref| of the MLX-order
oracle); the step count follows the stop
rule (stop after latent_k when stop_k > 0.5 and k > 3) applied to the GPU's
stop values, and the cache grows by the documented number of positions."""
import importlib

import numpy as np
import pytest
import torch

import oracle
from ditkit import AGG, oblock, ocfg, olin, oracle_agg, oracle_cfm
from lmkit import assert_bits, assert_close_bf16, oracle_model, oracle_step

pytestmark = pytest.mark.gpu


def mods():
    return (importlib.import_module("ming-tts-serve_amd"), importlib.import_module("ming-tts-serve_amd.synthetic"))


def dev_u16(a):
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).cuda().view(torch.bfloat16)


def host_u16(t):
    return t.view(torch.int16).cpu().numpy().view(np.uint16)


@pytest.fixture(scope="module")
def models(ctx):
    ming, S = mods()
    spec = S.LmSpec(n_layers=2, vocab=256)
    lm = S.SyntheticLm(ctx, spec, seed=3, quant=True, norm_std=0.1)
    flow = S.SyntheticFlow(ctx, S.DitSpec(cfm_blocks=2, agg_blocks=2), seed=5, norm_std=0.05)
    oracle.set_threads(16)
    with oracle.dit_order(oracle.DIT_ORDER_DEVICE):
        ocfm_dev, oagg_dev = oracle_cfm(flow), oracle_agg(flow)
    return dict(spec=spec, lm=lm, flow=flow, lm_model=lm.model(), cfm=flow.cfm_model(), agg=flow.agg_model(),
                olm=oracle_model(lm), ocfm=oracle_cfm(flow), oagg=oracle_agg(flow), ocfm_dev=ocfm_dev,
                oagg_dev=oagg_dev)


@pytest.mark.parametrize("case,stop_bias,max_steps", [("stops", (0.0, 20.0), 8), ("runs_out", (20.0, 0.0), 6)])
def test_sample_latents_matches_oracle(ming, ctx, models, case, stop_bias, max_steps):
    print(f"[sample_latents] {case} max_steps={max_steps}", flush=True)
    ming, S = mods()
    spec, lm, flow = models["spec"], models["lm"], models["flow"]
    H, lat, L = spec.hidden, flow.spec.latent, 3
    bias = oracle.to_bf16(np.array(stop_bias, np.float32))
    bias_d = dev_u16(bias)
    emb = ming.synth_normal_bf16(71, "loop.embeds", L * H, 0.0, 0.5).reshape(L, H)
    cache = S.KvCache(spec, L + max_steps + 2)
    bank = torch.empty((max_steps, 11, lat), dtype=torch.bfloat16, device="cuda")
    ctx.noise_bank(1234, max_steps, lat, bank)
    lats = torch.zeros((max_steps, lat), dtype=torch.bfloat16, device="cuda")
    ztr = torch.zeros((max_steps, H), dtype=torch.bfloat16, device="cuda")
    params = ming.SampleParams(max_steps, 2.0, 0.25, 0.0)
    n, stops = ctx.sample_latents(models["lm_model"], models["cfm"], models["agg"], flow.lin_w("stop_head"), bias_d,
                                  dev_u16(emb), cache.kv, bank, params, lats, z_trace=ztr)
    g_lat, g_z, g_bank = host_u16(lats), host_u16(ztr), host_u16(bank)
    # the stop rule on the GPU's own stop values
    want_n = max_steps
    for k, sp in enumerate(stops):
        if sp > 0.5 and k > 3:
            want_n = k + 1
            break
    assert n == want_n, (n, stops)
    assert n == (5 if case == "stops" else max_steps)
    assert cache.len == (L + n if n < max_steps or case == "stops" else L + n - 1), cache.len
    cfg, layers, norm, head = models["olm"]
    oc, oa = models["ocfm"], models["oagg"]
    kc = np.zeros((spec.n_layers, spec.kv_heads, L + max_steps + 2, spec.head_dim), np.uint16)
    vc = np.zeros_like(kc)
    for i in range(L):
        _, z_ref, _, _, _ = oracle_step(cfg, layers, norm, head, emb[i], i, kc, vc)
    assert_close_bf16(g_z[0], z_ref, "z_0 (prefill)")
    stop_lin = oracle.Linear(flow.hostw["stop_head.weight"])
    hist = np.zeros(lat, np.uint16)
    for k in range(n):
        assert abs(stops[k] - oracle.stop_prob(stop_lin, bias, g_z[k])) <= 1e-2, (k, stops[k])
        with oracle.dit_order(oracle.DIT_ORDER_DEVICE):
            # the step's ten free-running Euler steps and the stop head: bit for bit with the
            # oracle in the kernels' summation order, on the GPU's own z and history
            assert np.float32(stops[k]) == np.float32(oracle.stop_prob(stop_lin, bias, g_z[k])), k
            ref, _ = oracle.cfm_sample(models["ocfm_dev"], g_z[k], hist, g_bank[k, 0], g_bank[k, 1:], 2.0, 0.0)
        assert_bits(g_lat[k], ref, f"latent {k} (device order)")
        ref_mlx, _ = oracle.cfm_sample(oc, g_z[k], hist, g_bank[k, 0], g_bank[k, 1:], 2.0, 0.0)
        assert_close_bf16(g_lat[k], ref_mlx, f"latent {k} (MLX order)", atol=6e-2, rtol=2e-2)
        hist = g_lat[k]
        if k + 1 < n:
            # the LM input row the loop used: the same aggregate kernel on the same latent
            xd = torch.empty(H, dtype=torch.bfloat16, device="cuda")
            models["agg"].aggregate(dev_u16(g_lat[k]), xd)
            ctx.sync()
            xrow = host_u16(xd)
            assert_close_bf16(xrow, oracle.aggregate(oa, g_lat[k]), f"aggregate {k}")
            with oracle.dit_order(oracle.DIT_ORDER_DEVICE):
                assert_bits(xrow, oracle.aggregate(models["oagg_dev"], g_lat[k]), f"aggregate {k} (device order)")
            _, z_ref, _, _, _ = oracle_step(cfg, layers, norm, head, xrow, L + k, kc, vc)
            assert_close_bf16(g_z[k + 1], z_ref, f"z_{k + 1}")
    assert not np.any(g_lat[n:]), "no latent past the last step"


def test_sample_latents_rejects(ming, ctx, models):
    ming, S = mods()
    spec, flow = models["spec"], models["flow"]
    cache = S.KvCache(spec, 3)
    emb = torch.zeros((3, spec.hidden), dtype=torch.bfloat16, device="cuda")
    bank = torch.zeros((4, 11, 64), dtype=torch.bfloat16, device="cuda")
    lats = torch.zeros((4, 64), dtype=torch.bfloat16, device="cuda")
    with pytest.raises(ming.MingError) as e:  # prompt fills the cache: no step fits
        ctx.sample_latents(models["lm_model"], models["cfm"], models["agg"], flow.lin_w("stop_head"),
                           flow.dev["stop_head.bias"], emb, cache.kv, bank, ming.SampleParams(4, 2.0, 0.25, 0.0),
                           lats)
    assert e.value.status == ming.MING_E_CTX_OVER_CAPACITY
    assert cache.len == 0


def run_loop(ctx, models, emb, cache, max_steps=1):
    ming, S = mods()
    spec, flow = models["spec"], models["flow"]
    H, lat = spec.hidden, flow.spec.latent
    bias_d = dev_u16(oracle.to_bf16(np.array((20.0, 0.0), np.float32)))  # never stops
    bank = torch.empty((max_steps, 11, lat), dtype=torch.bfloat16, device="cuda")
    ctx.noise_bank(99, max_steps, lat, bank)
    lats = torch.zeros((max_steps, lat), dtype=torch.bfloat16, device="cuda")
    ztr = torch.zeros((max_steps, H), dtype=torch.bfloat16, device="cuda")
    n, _ = ctx.sample_latents(models["lm_model"], models["cfm"], models["agg"], flow.lin_w("stop_head"), bias_d,
                              dev_u16(emb), cache.kv, bank, ming.SampleParams(max_steps, 2.0, 0.25, 0.0), lats,
                              z_trace=ztr)
    assert n == max_steps
    return host_u16(ztr)


def test_prompt_prefill_batched_on_empty_cache(ming, ctx, models):
    """A 70-row prompt on an empty cache is one batched prefill (a 64-row and a
    6-row chunk over two pages): the cache rows and z_0 equal ming_lm_prefill's
    own pages and last hidden row bit for bit, and z_0 and the cached rows
    agree with the oracle's one-row-at-a-time prefill."""
    ming, S = mods()
    spec = models["spec"]
    H, L = spec.hidden, 70
    print(f"[sample_latents] batched prompt prefill L={L}", flush=True)
    emb = ming.synth_normal_bf16(72, "loop.embeds.long", L * H, 0.0, 0.5).reshape(L, H)
    cache = S.KvCache(spec, L + 4)
    g_z = run_loop(ctx, models, emb, cache)
    assert cache.len == L
    gk, gv = cache.host()
    b = ming.LmBatch(models["lm_model"], 64, 128)
    pk = S.PagedKv(spec, 1, 2, spare=3, seed=8)
    hid = torch.empty((L, H), dtype=torch.bfloat16, device="cuda")
    b.prefill(pk, pk.table[0].contiguous(), 0, x_in=dev_u16(emb), hidden=hid)
    ctx.sync()
    pk_k, pk_v = pk.gather(0, L)
    assert np.array_equal(gk[:, :, :L], pk_k) and np.array_equal(gv[:, :, :L], pk_v), "cache rows differ from prefill"
    assert np.array_equal(g_z[0], host_u16(hid[L - 1])), "z_0 differs from the prefill's last hidden row"
    b.close()
    cfg, layers, norm, head = models["olm"]
    kc = np.zeros((spec.n_layers, spec.kv_heads, L + 4, spec.head_dim), np.uint16)
    vc = np.zeros_like(kc)
    for i in range(L):
        _, z_ref, _, _, _ = oracle_step(cfg, layers, norm, head, emb[i], i, kc, vc)
    assert_close_bf16(g_z[0], z_ref, "z_0 (batched prefill)")
    assert_close_bf16(gk[:, :, :L], kc[:, :, :L], "cached k")
    assert_close_bf16(gv[:, :, :L], vc[:, :, :L], "cached v")


def test_prompt_prefill_row_by_row_on_filled_cache(ming, ctx, models):
    """A cache that already holds rows takes the prompt one decode step per row:
    z_0 against the oracle over the same cached rows."""
    ming, S = mods()
    spec = models["spec"]
    H, L, pre = spec.hidden, 3, 9
    print(f"[sample_latents] row-by-row prompt prefill after {pre} cached rows", flush=True)
    emb = ming.synth_normal_bf16(73, "loop.embeds.cont", L * H, 0.0, 0.5).reshape(L, H)
    cache = S.KvCache(spec, pre + L + 4)
    cache.fill_random(pre, seed=21)
    kc, vc = (a.copy() for a in cache.host())
    g_z = run_loop(ctx, models, emb, cache)
    assert cache.len == pre + L
    cfg, layers, norm, head = models["olm"]
    for i in range(L):
        _, z_ref, _, _, _ = oracle_step(cfg, layers, norm, head, emb[i], pre + i, kc, vc)
    assert_close_bf16(g_z[0], z_ref, "z_0 (row-by-row prefill)")


def test_sample_latents_reports_a_raised_device_flag(ming, ctx, models):
    """A device error flag raised before the call (here flags[2], from a gather
    whose matrix index is out of range: the gather kernel skips that pair and
    exits normally) ends the loop at the first stop read: the call returns
    ming_sync's status with no step reported, and the next call runs clean."""
    ming, S = mods()
    spec, flow = models["spec"], models["flow"]
    H = spec.hidden
    print("[sample_latents] device flag raised before the call", flush=True)
    wq = torch.zeros((1, 64, 8), dtype=torch.int32, device="cuda")
    sc = torch.zeros((1, 64, 1), dtype=torch.bfloat16, device="cuda")
    y = torch.zeros((1, 1, 64), dtype=torch.float32, device="cuda")
    ctx.gather_qmm(torch.zeros((1, 1, 64), dtype=torch.bfloat16, device="cuda"), wq, sc, sc.clone(), None,
                   torch.tensor([1], dtype=torch.int32, device="cuda"), y)
    emb = ming.synth_normal_bf16(74, "loop.embeds.flag", 3 * H, 0.0, 0.5).reshape(3, H)
    cache = S.KvCache(spec, 10)
    bank = torch.zeros((4, 11, 64), dtype=torch.bfloat16, device="cuda")
    lats = torch.zeros((4, 64), dtype=torch.bfloat16, device="cuda")
    args = (models["lm_model"], models["cfm"], models["agg"], flow.lin_w("stop_head"), flow.dev["stop_head.bias"])
    with pytest.raises(ming.MingError) as e:
        ctx.sample_latents(*args, dev_u16(emb), cache.kv, bank, ming.SampleParams(4, 2.0, 0.25, 0.0), lats)
    assert e.value.status == ming.MING_E_ARG
    cache = S.KvCache(spec, 10)
    n, _ = ctx.sample_latents(*args, dev_u16(emb), cache.kv, bank, ming.SampleParams(2, 2.0, 0.25, 0.0), lats)
    assert n >= 1


# ---- full size: 24-layer 4-bit LM at the Qwen2-0.5B shape, 8 + 8 DiT blocks ----

@pytest.fixture(scope="module")
def full(ctx):
    ming, S = mods()
    spec = S.QWEN2_05B
    print("[sample_latents] building the full-size models: 24-layer 4-bit LM, 8 + 8 DiT blocks", flush=True)
    lm = S.SyntheticLm(ctx, spec, seed=13, quant=True)
    flow = S.SyntheticFlow(ctx, S.MING_DIT, seed=15, norm_std=0.05)
    oracle.set_threads(16)
    d = dict(spec=spec, lm=lm, flow=flow, lm_model=lm.model(), cfm=flow.cfm_model(), agg=flow.agg_model(),
             olm=oracle_model(lm), ocfm=oracle_cfm(flow), oagg=oracle_agg(flow))
    yield d
    for k in ("lm_model", "cfm", "agg"):
        d[k].close()


def check_lm_layers(orc, tr, x_in, pos, kc, vc, new_k, new_v, tag):
    """Every layer of a decode step against the oracle on the GPU's own input to
    that layer and the cache rows [0, pos) the step read; then the final norm."""
    cfg, layers, norm, _ = orc
    assert np.array_equal(tr["x"][0], x_in), f"{tag} input row"
    for l, lay in enumerate(layers):
        k_l, v_l = kc[l].copy(), vc[l].copy()
        x2, t = oracle.lm_layer_step(cfg, lay, tr["x"][l], pos, k_l, v_l, trace=True)
        w = f"{tag} layer {l}"
        assert_close_bf16(tr["qkv"][l], t["qkv"], w + " q|k|v")
        assert_close_bf16(tr["att"][l], t["att"], w + " attention")
        assert_close_bf16(tr["x1"][l], t["x1"], w + " x1")
        assert_close_bf16(tr["hh"][l], t["hh"], w + " swiglu")
        assert_close_bf16(tr["x"][l + 1], x2, w + " output")
        assert_close_bf16(new_k[l, :, pos], k_l[:, pos], w + " appended k")
        assert_close_bf16(new_v[l, :, pos], v_l[:, pos], w + " appended v")
    return oracle.rms_norm(tr["x"][-1], norm, cfg.eps)


def check_aggregate(ctx, agg, flow, latent, tag):
    """ming_aggregate_trace on a latent: the cls and x_emb rows, every block on
    the GPU's own input rows, and the final norm + linear on the GPU's stack
    output, each against the oracle; returns the output row."""
    spec, h = flow.spec, flow.hostw
    D, nb = spec.hidden, spec.agg_blocks
    rows = torch.empty((nb + 1, 2, D), dtype=torch.bfloat16, device="cuda")
    out = torch.empty(spec.lm_hidden, dtype=torch.bfloat16, device="cuda")
    agg.aggregate_trace(dev_u16(latent), rows, out)
    ctx.sync()
    r, o = host_u16(rows), host_u16(out)
    assert np.array_equal(r[0, 0], np.asarray(h[f"{AGG}.word_embedder.weight"]).reshape(-1)[:D]), tag + " cls row"
    assert_close_bf16(r[0, 1], oracle.linear(olin(flow, f"{AGG}.x_embedder"), latent, h[f"{AGG}.x_embedder.bias"]),
                      tag + " x_emb")
    c = ocfg(spec)
    ct, st = oracle.rotary_table(spec.inv_freq(), 2)
    for i in range(nb):
        ref = oracle.dit_block_fwd(c, oblock(flow, AGG, i), r[i], 1, 2, ct, st)
        assert_close_bf16(r[i + 1], ref, f"{tag} block {i} (teacher forced)")
    hn = oracle.rms_norm(r[nb, 0], h[f"{AGG}.final_layer.norm_final.weight"], spec.eps)
    ref = oracle.linear(olin(flow, f"{AGG}.final_layer.linear"), hn, h[f"{AGG}.final_layer.linear.bias"])
    assert_close_bf16(o, ref, tag + " final layer")
    return o


@pytest.mark.parametrize("with_prompt_latent", [False, True])
def test_sample_latents_full_size_equals_its_parts(ming, ctx, full, with_prompt_latent):
    """The loop at full size, with the SDE noise on (temperature 1): every step
    equals the library's own entry points run one at a time on the loop's own
    values, bit for bit -- ming_lm_prefill on the prompt (its rows and last
    hidden row are the loop's prompt rows and z_0), the flow head on (z_k,
    history_k, bank row k), the aggregator on latent_k, the decode step at
    position L + k over the loop's own cache rows (its hidden is z_{k+1}, its
    appended rows are the loop's) -- and each of those is checked against the
    oracle teacher forced: the prefill's last row and every decode step layer
    by layer on the GPU's own inputs, every Euler step from the GPU's previous
    latent, the aggregate row, and stop_k.  With a prompt_latent, that latent
    is the first step's history."""
    ming, S = mods()
    spec, flow = full["spec"], full["flow"]
    lm, cfm, agg = full["lm_model"], full["cfm"], full["agg"]
    H, lat, L, steps = spec.hidden, flow.spec.latent, 12, 5
    cfg_w, sigma, temperature = 2.0, 0.25, 1.0
    print(f"[sample_latents] full size, prompt_latent={with_prompt_latent}", flush=True)
    emb = ming.synth_normal_bf16(81, "loop.full.embeds", L * H, 0.0, 0.5).reshape(L, H)
    pl = ming.synth_normal_bf16(82, "loop.full.prompt_latent", lat) if with_prompt_latent else None
    bias = oracle.to_bf16(np.array((20.0, 0.0), np.float32))  # never stops
    cache = S.KvCache(spec, L + steps + 2)
    bank = torch.empty((steps, 11, lat), dtype=torch.bfloat16, device="cuda")
    ctx.noise_bank(77, steps, lat, bank)
    lats = torch.zeros((steps, lat), dtype=torch.bfloat16, device="cuda")
    ztr = torch.zeros((steps, H), dtype=torch.bfloat16, device="cuda")
    lm.set_mode(ming.LM_AUTO)
    n, stops = ctx.sample_latents(lm, cfm, agg, flow.lin_w("stop_head"), dev_u16(bias), dev_u16(emb), cache.kv, bank,
                                  ming.SampleParams(steps, cfg_w, sigma, temperature), lats,
                                  prompt_latent=dev_u16(pl) if pl is not None else None, z_trace=ztr)
    assert n == steps and cache.len == L + steps - 1, (n, cache.len)
    g_lat, g_z, g_bank = host_u16(lats), host_u16(ztr), host_u16(bank)
    gk, gv = cache.host()
    orc = full["olm"]
    oc = full["ocfm"]
    c = ocfg(flow.spec)
    stop_lin = oracle.Linear(flow.hostw["stop_head.weight"])
    shift = float(np.float32(sigma) * np.sqrt(np.float32(temperature)))
    c2 = S.KvCache(spec, L + steps + 2)

    def decode_on_loop_rows(pos, x):
        c2.k.copy_(cache.k)
        c2.v.copy_(cache.v)
        c2.kv.len = pos
        hid = torch.empty(H, dtype=torch.bfloat16, device="cuda")
        lm.step(c2.kv, x_in=dev_u16(x), hidden=hid)
        ctx.sync()
        tr = {k: host_u16(v) for k, v in lm.trace().items()}
        nk, nv = c2.host()
        return host_u16(hid), tr, nk, nv

    # z_0: the loop's prompt rows and z_0 are ming_lm_prefill's bit for bit, and the prefill's last
    # row is checked layer by layer over the prefill's own rows (24 layers of a random-init stack
    # amplify the prefill's and the decode step's different f32 summation orders past the bf16 bar
    # end to end, so the two are compared layer by layer, each against the oracle)
    b = ming.LmBatch(lm, 64, 128)
    pk = S.PagedKv(spec, 1, 2, spare=3, seed=8)
    hid = torch.empty((L, H), dtype=torch.bfloat16, device="cuda")
    b.prefill(pk, pk.table[0].contiguous(), 0, x_in=dev_u16(emb), hidden=hid)
    ctx.sync()
    pk_k, pk_v = pk.gather(0, L)
    assert np.array_equal(gk[:, :, :L], pk_k) and np.array_equal(gv[:, :, :L], pk_v), "prompt rows differ from prefill"
    assert np.array_equal(g_z[0], host_u16(hid[L - 1])), "z_0 differs from the prefill's last hidden row"
    tr = {k: host_u16(v)[:, L - 1] for k, v in b.trace().items()}
    b.close()
    rz = check_lm_layers(orc, tr, emb[L - 1], L - 1, pk_k, pk_v, pk_k, pk_v, "prefill last row")
    assert_close_bf16(g_z[0], rz, "z_0 (final norm)")
    hist = pl if pl is not None else np.zeros(lat, np.uint16)
    out = torch.empty(lat, dtype=torch.bfloat16, device="cuda")
    ys = torch.empty((10, lat), dtype=torch.bfloat16, device="cuda")
    xd = torch.empty(H, dtype=torch.bfloat16, device="cuda")
    for k in range(n):
        assert abs(stops[k] - oracle.stop_prob(stop_lin, bias, g_z[k])) <= 1e-2, (k, stops[k])
        cfm.sample(dev_u16(g_z[k]), dev_u16(hist), dev_u16(g_bank[k, 0]), dev_u16(g_bank[k, 1:]), cfg_w, sigma,
                   temperature, out, ys)
        ctx.sync()
        assert np.array_equal(host_u16(out), g_lat[k]), f"step {k}: the loop's latent differs from ming_cfm_sample"
        y = host_u16(ys)
        for i in range(10):
            y_in = g_bank[k, 0] if i == 0 else y[i - 1]
            h = oracle.cfm_rows(oc, g_z[k], hist, y_in, i)
            for blk in oc.blocks:
                h = oracle.dit_block_fwd(c, blk, h, 2, 3, oc.keep["cos"], oc.keep["sin"])
            ref = oracle.cfm_final(oc, h, 3, y_in, g_bank[k, 1:], i, cfg_w, shift)
            assert_close_bf16(y[i], ref, f"step {k} Euler step {i} (teacher forced)")
        hist = g_lat[k]
        if k + 1 < n:
            xrow = check_aggregate(ctx, agg, flow, g_lat[k], f"aggregate {k}")
            agg.aggregate(dev_u16(g_lat[k]), xd)
            ctx.sync()
            assert np.array_equal(host_u16(xd), xrow), f"aggregate {k}: traced and plain calls differ"
            z, tr, nk, nv = decode_on_loop_rows(L + k, xrow)
            assert np.array_equal(z, g_z[k + 1]), f"z_{k + 1} differs from ming_lm_step on the loop's rows"
            assert np.array_equal(nk[:, :, L + k], gk[:, :, L + k]) and \
                np.array_equal(nv[:, :, L + k], gv[:, :, L + k]), f"cache row {L + k} differs"
            rz = check_lm_layers(orc, tr, xrow, L + k, gk, gv, nk, nv, f"step {k} LM")
            assert_close_bf16(z, rz, f"z_{k + 1} (final norm)")
    print(f"[sample_latents] full size: {n} steps equal their parts; stops {[round(s, 4) for s in stops]}",
          flush=True)
