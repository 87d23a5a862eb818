"""Models built from safetensors checkpoints (ming_weights_load and the
*_from_weights builders: Tensors.load / QStack.load / DitStack.load under the
reference's key map, src/ming_model.zig:316-350, :544-560, :728-742, :935-956)
against the same models built directly from the synthetic tensors.

Checkpoints are written with the `safetensors` package: an MLX 4-bit one
(`<linear>.weight` u32 + `.scales` + `.biases`), a bf16 one (linears
quantized on the GPU at load, or kept bf16) and the flow head / aggregator /
stop head in bf16 with their f32 `rotary_embed.inv_freq`.  Bar: bit-identical
outputs (the same weights reach the same kernels)."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

SMALL = dict(hidden=128, heads=2, kv_heads=1, head_dim=64, inter=256, vocab=512, n_layers=2)


def syn_mod():
    import importlib

    return importlib.import_module("ming-tts-serve_amd.synthetic")


def save(path, tensors):
    from safetensors.torch import save_file

    save_file({k: v.detach().contiguous().cpu() for k, v in tensors.items()}, str(path))


def lm_tensors(syn):
    out = {}
    for name, t in syn.tensors.items():
        if isinstance(t, dict):
            if "s" in t:
                out[name + ".weight"] = t["w"].view(torch.uint32)
                out[name + ".scales"] = t["s"]
                out[name + ".biases"] = t["b"]
            else:
                out[name + ".weight"] = t["w"]
        else:
            out[name] = t
    return out


def lm_step(ming, ctx, m, spec, ctx_len=70, token=77):
    S = syn_mod()
    cache = S.KvCache(spec, ctx_len + 2)
    cache.fill_random(ctx_len, seed=12)
    tok = torch.tensor([token], dtype=torch.int32, device="cuda")
    hid = torch.empty(spec.hidden, dtype=torch.bfloat16, device="cuda")
    lg = torch.empty(spec.vocab, dtype=torch.float32, device="cuda")
    am = torch.empty(1, dtype=torch.int32, device="cuda")
    m.step(cache.kv, token=tok, hidden=hid, logits=lg, argmax=am)
    ctx.sync()
    return hid, lg, am


def same(a, b):
    return all(torch.equal(x, y) for x, y in zip(a, b))


def test_lm_from_mlx_4bit_checkpoint(ming, ctx, tmp_path):
    S = syn_mod()
    spec = S.LmSpec(**SMALL)
    syn = S.SyntheticLm(ctx, spec, seed=41, quant=True, norm_std=0.1)
    path = tmp_path / "lm4.safetensors"
    save(path, lm_tensors(syn))
    w = ming.Weights(ctx, path)
    m = w.lm_model(spec.cfg())
    ref = syn.model()
    assert same(lm_step(ming, ctx, m, spec), lm_step(ming, ctx, ref, spec))
    m.close()
    ref.close()
    w.close()


def test_lm_from_bf16_checkpoint(ming, ctx, tmp_path):
    S = syn_mod()
    spec = S.LmSpec(**SMALL)
    bf = S.SyntheticLm(ctx, spec, seed=42, quant=False, norm_std=0.1)
    q4 = S.SyntheticLm(ctx, spec, seed=42, quant=True, norm_std=0.1)
    path = tmp_path / "lm16.safetensors"
    save(path, lm_tensors(bf))
    w = ming.Weights(ctx, path)
    for quantize, ref_syn in ((True, q4), (False, bf)):
        m = w.lm_model(spec.cfg(), quantize=quantize)
        ref = ref_syn.model()
        assert same(lm_step(ming, ctx, m, spec), lm_step(ming, ctx, ref, spec)), f"quantize={quantize}"
        m.close()
        ref.close()
    # the quantized copy equals ming_quantize's output bit for bit
    lin = w.linear("model.model.layers.1.mlp.down_proj", spec.hidden, spec.inter, quantize=True)
    n, k = spec.hidden, spec.inter
    import ctypes

    host = np.empty((n, k // 8), np.uint32)
    ctx.check(ming.lib().ming_memcpy_dtoh(ctx.h, host.ctypes.data_as(ctypes.c_void_p), ctypes.c_void_p(lin.w),
                                          host.nbytes))
    assert np.array_equal(host, q4.host("model.model.layers.1.mlp.down_proj")["w"])
    w.close()


def flow_tensors(flow):
    t = {k: v for k, v in flow.dev.items()}
    t["flowloss.cfm.model.rotary_embed.inv_freq"] = torch.from_numpy(flow.inv_freq.copy())
    t["linear_proj_audio.rotary_embed.inv_freq"] = torch.from_numpy(flow.inv_freq.copy())
    return t


def test_flow_head_aggregator_stop_from_checkpoint(ming, ctx, tmp_path):
    S = syn_mod()
    spec = S.DitSpec(hidden=128, heads=2, head_dim=64, ff=256, cfm_blocks=2, agg_blocks=2, latent=64, lm_hidden=128)
    flow = S.SyntheticFlow(ctx, spec, seed=43, norm_std=0.1)
    path = tmp_path / "flow.safetensors"
    save(path, flow_tensors(flow))
    w = ming.Weights(ctx, path, prefixes=["flowloss.", "linear_proj_audio.", "stop_head"])
    cfm = w.cfm_model(spec.cfg(), spec.cfm_blocks, spec.lm_hidden, spec.latent)
    agg = w.agg_model(spec.cfg(), spec.agg_blocks, spec.lm_hidden, spec.latent)
    rcfm, ragg = flow.cfm_model(), flow.agg_model()
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).cuda().view(torch.bfloat16)
    z = dev(ming.synth_normal_bf16(44, "w.z", spec.lm_hidden))
    hist = dev(ming.synth_normal_bf16(45, "w.hist", spec.latent))
    noise = dev(ming.synth_normal_bf16(46, "w.noise", spec.latent))
    sde = dev(ming.synth_normal_bf16(47, "w.sde", 10 * spec.latent))
    outs = []
    for c, a in ((cfm, agg), (rcfm, ragg)):
        lat = torch.empty(spec.latent, dtype=torch.bfloat16, device="cuda")
        c.sample(z, hist, noise, sde, 2.0, 0.25, 1.0, lat)
        zz = torch.empty(spec.lm_hidden, dtype=torch.bfloat16, device="cuda")
        a.aggregate(lat, zz)
        outs.append((lat, zz))
    ps = []
    for head, bias in ((w.linear("stop_head", 2, spec.lm_hidden), w.get("stop_head.bias").data),
                       (flow.lin_w("stop_head"), flow.ptr("stop_head.bias"))):
        p = torch.empty(1, dtype=torch.float32, device="cuda")  # ming_stop_prob writes one f32
        ctx.stop_prob(head, bias, z, p)
        ps.append(p)
    ctx.sync()
    assert same(outs[0], outs[1])
    assert torch.equal(ps[0], ps[1])
    for mdl in (cfm, agg, rcfm, ragg):
        mdl.close()
    w.close()


def test_missing_and_misshapen_weights(ming, ctx, tmp_path):
    S = syn_mod()
    spec = S.LmSpec(**SMALL)
    syn = S.SyntheticLm(ctx, spec, seed=48, quant=True)
    path = tmp_path / "lm.safetensors"
    save(path, lm_tensors(syn))
    w = ming.Weights(ctx, path, prefixes=["model.model.layers.0."])
    with pytest.raises(KeyError):
        w.get("model.model.embed_tokens.weight")
    with pytest.raises(ming.MingError) as e:
        w.lm_model(spec.cfg())
    assert e.value.status == ming.MING_E_ARG
    w.close()
    w = ming.Weights(ctx, path)
    bad = S.LmSpec(**dict(SMALL, inter=512)).cfg()
    with pytest.raises(ming.MingError) as e:
        w.lm_model(bad)
    assert e.value.status == ming.MING_E_SHAPE
    short = S.LmSpec(**dict(SMALL, n_layers=1)).cfg()
    with pytest.raises(ming.MingError) as e:  # the checkpoint holds 2 layers
        w.lm_model(short)
    assert e.value.status == ming.MING_E_SHAPE
    w.close()


def test_handles_outlive_their_context(ming, tmp_path):
    """Weights, models and batches destroyed after their context (as at
    interpreter exit) release their memory without touching the context."""
    S = syn_mod()
    ctx2 = ming.Context(0)
    spec = S.LmSpec(**SMALL)
    syn = S.SyntheticLm(ctx2, spec, seed=49, quant=True)
    path = tmp_path / "lm.safetensors"
    save(path, lm_tensors(syn))
    w = ming.Weights(ctx2, path)
    m = w.lm_model(spec.cfg())
    b = ming.LmBatch(m, 4, 256)
    ctx2.sync()
    ctx2.close()
    b.close()
    m.close()
    w.close()


def test_vae_from_checkpoint(ming, ctx, tmp_path):
    """audio.decoder.* (fc1, decoder stack, head, istft.window stored bf16 and widened at load) ->
    the same waveform bit for bit as the directly built decoder."""
    S = syn_mod()
    spec = S.VaeSpec(hidden=128, heads=2, kv_heads=1, head_dim=64, inter=256, n_layers=2, window=8, latent=64,
                     patch=4, n_fft=64, hop=16)
    syn = S.SyntheticVae(ctx, spec, seed=51, std=0.05, norm_std=0.1)
    t = lm_tensors(syn)
    t["audio.decoder.head.istft.window"] = syn.tensors["audio.decoder.head.istft.window"].to(torch.bfloat16)
    path = tmp_path / "vae.safetensors"
    save(path, t)
    w = ming.Weights(ctx, path, prefixes=["audio.decoder."])
    m = w.vae_model(spec.cfg(), 8)
    ref = syn.model(8)
    # the direct model gets the same bf16-rounded window
    win = syn.tensors["audio.decoder.head.istft.window"].to(torch.bfloat16).float()
    ref.close()
    syn.tensors["audio.decoder.head.istft.window"] = win
    syn._build_views()
    ref = syn.model(8)
    lat = torch.from_numpy(ming.synth_normal_bf16(52, "w.vae", 5 * 64).view(np.int16)).cuda().view(torch.bfloat16)
    outs = []
    for mdl in (m, ref):
        wave = torch.empty(5 * 4 * 16, dtype=torch.float32, device="cuda")
        mdl.decode(5, lat, wave)
        outs.append(wave)
    ctx.sync()
    assert torch.equal(outs[0], outs[1])
    m.close()
    ref.close()
    w.close()
