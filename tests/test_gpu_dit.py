"""GPU parity of the DiT flow head, aggregator and stop head
(ming_dit_block / ming_dit_single, ming_cfm_embed / ming_cfm_final,
ming_cfm_model_* / ming_cfm_sample, ming_aggregate, ming_stop_prob) against
the oracle on the same seeded inputs.

Bars: rotary tables, flow schedule, dt and sqrt|dt| bit-exact; bf16 outputs
(q/k/v, attention, residual stream, gelu, CFM rows, timestep embeddings,
each Euler step's latent, aggregator rows) within |gpu - ref| <= 2e-2 +
1e-2 |ref| of the oracle in its MLX order; the stop probability within 1e-2
absolute.  Each Euler step of the GPU sample is recomputed on the oracle from
the GPU's own previous latent (teacher forced).  With the oracle summing in the
kernels' order (oracle.dit_order(DIT_ORDER_DEVICE): same graph and rounding
points, f32 sums taken as the batch-1 kernels take them) every block stage,
timestep embedding, Euler step and the free-running ten-step latent are equal
bit for bit, and the free-running latent is within 6e-2 + 2e-2 |ref| (mean
|d| <= 2e-2) of the MLX-order oracle: the two f32 orders differ in 1-5 outputs
of a block by one bf16 ulp, which the 8-block, 10-step CFG loop grows."""
import ctypes

import numpy as np
import pytest
import torch

import oracle
from ditkit import CFM, oblock, ocfg, olin, oracle_agg, oracle_cfm
from lmkit import assert_bits, assert_close_bf16

pytestmark = pytest.mark.gpu

REF = dict(hidden=1024, heads=16, head_dim=64, ff=4096)
SMALL = dict(hidden=128, heads=2, head_dim=64, ff=256)


def syn_mod():
    import importlib

    return importlib.import_module("ming-tts-serve_amd.synthetic")


def dev_u16(a):
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).cuda().view(torch.bfloat16)


def host_u16(t):
    return t.view(torch.int16).cpu().numpy().view(np.uint16)


def bf16_empty(*shape):
    return torch.empty(shape, dtype=torch.bfloat16, device="cuda")


def rotary_dev(ctx, spec, L):
    half = spec.head_dim // 2
    cos = torch.empty((L, half), dtype=torch.float32, device="cuda")
    sin = torch.empty((L, half), dtype=torch.float32, device="cuda")
    ctx.rotary_table(spec.inv_freq(), L, cos, sin)
    return cos, sin


# ---- one block ---------------------------------------------------------------------

BLOCK_CASES = [
    # (shape, B, L)
    (SMALL, 1, 1),
    (SMALL, 2, 3),
    (SMALL, 1, 2),
    (REF, 2, 3),
    (REF, 1, 2),
    (dict(hidden=192, heads=6, head_dim=32, ff=320), 2, 3),
]


def test_gelu_epilogue_bit_exact(ming, ctx):
    """Stage C (rms -> ff1 + bias -> gelu_approx) with zero ff1 weights: the
    pre-activation is the bias itself (bf16(0 + b) = b), so each output column
    is gelu_approx of its bias.  Over every bf16 value in [-12, 12] (33,409
    arguments: tanh's argument then crosses the table's end at 9.0625 and its
    saturation) the kernel equals the oracle's gelu_approx bit for bit."""
    S = syn_mod()
    spec = S.DitSpec(hidden=128, heads=2, head_dim=64, ff=4096, cfm_blocks=1)
    syn = S.SyntheticFlow(ctx, spec, seed=13, norm_std=0.1, parts=("cfm",))
    pre = "flowloss.cfm.model.blocks.0.mlp.ff.0.0"
    syn.dev[pre + ".weight"].zero_()
    pos = np.arange(0, 0x4141, dtype=np.uint16)  # +0 .. 12.0
    vals = np.concatenate([pos, pos[1:] | np.uint16(0x8000)])
    R, D, F = 2, spec.hidden, spec.ff
    x = dev_u16(ming.synth_normal_bf16(14, "gelu.x", R * D)).reshape(R, D)
    cos, sin = rotary_dev(ctx, spec, 1)
    got = bf16_empty(R * F)
    w = syn.cfm_blocks[0]
    checked = 0
    for c0 in range(0, vals.size, F):
        b = np.zeros(F, np.uint16)
        chunk = vals[c0:c0 + F]
        b[:chunk.size] = chunk
        syn.dev[pre + ".bias"].copy_(dev_u16(b))
        ctx.dit_single(2, spec.cfg(), w, x, None, R, 1, cos, sin, None, got)
        ctx.sync()
        g = host_u16(got).reshape(R, F)
        ref = oracle.gelu_approx(b)
        for r in range(R):
            bad = np.nonzero(g[r] != ref)[0]
            assert bad.size == 0, f"gelu of bf16 {b[bad[0]]:#06x}: {g[r, bad[0]]:#06x} != {ref[bad[0]]:#06x}"
        checked += chunk.size
    assert checked == vals.size == 33409


@pytest.mark.parametrize("shape,B,L", BLOCK_CASES)
def test_dit_block_matches_oracle(ming, ctx, shape, B, L):
    print(f"[dit_block] {shape} B={B} L={L}", flush=True)
    S = syn_mod()
    spec = S.DitSpec(**shape, cfm_blocks=1)
    syn = S.SyntheticFlow(ctx, spec, seed=11, norm_std=0.1, parts=("cfm",))
    R, D, F = B * L, spec.hidden, spec.ff
    x = ming.synth_normal_bf16(12, "dit.x", R * D, 0.0, 1.0).reshape(R, D)
    cos, sin = rotary_dev(ctx, spec, L)
    ct, st = oracle.rotary_table(spec.inv_freq(), L)
    assert np.array_equal(cos.cpu().numpy(), ct) and np.array_equal(sin.cpu().numpy(), st), "rotary table"
    out = dict(qkv=bf16_empty(3, R, D), att=bf16_empty(R, D), x1=bf16_empty(R, D), hh=bf16_empty(R, F),
               x2=bf16_empty(R, D))
    o = ming.DitOut(*(out[k].data_ptr() for k in ("qkv", "att", "x1", "hh", "x2")))
    xd = dev_u16(x)
    ctx.dit_block(spec.cfg(), syn.cfm_blocks[0], xd, B, L, cos, sin, o)
    ctx.sync()
    blk = oblock(syn, CFM, 0)
    ref, tr = oracle.dit_block_fwd(ocfg(spec), blk, x, B, L, ct, st, trace=True)
    assert_close_bf16(host_u16(out["qkv"]), tr["qkv"], "q|k|v (rotated)")
    assert_close_bf16(host_u16(out["att"]), tr["att"], "attention")
    assert_close_bf16(host_u16(out["x1"]), tr["x1"], "x + out_proj")
    assert_close_bf16(host_u16(out["hh"]), tr["hh"], "gelu(ff1)")
    assert_close_bf16(host_u16(out["x2"]), ref, "block output")
    # the oracle in the kernels' summation order: every stage bit for bit
    with oracle.dit_order(oracle.DIT_ORDER_DEVICE):
        ref_d, tr_d = oracle.dit_block_fwd(ocfg(spec), blk, x, B, L, ct, st, trace=True)
    assert_bits(host_u16(out["qkv"]), tr_d["qkv"], "q|k|v (device order)")
    assert_bits(host_u16(out["att"]), tr_d["att"], "attention (device order)")
    assert_bits(host_u16(out["x1"]), tr_d["x1"], "x + out_proj (device order)")
    assert_bits(host_u16(out["hh"]), tr_d["hh"], "gelu(ff1) (device order)")
    assert_bits(host_u16(out["x2"]), ref_d, "block output (device order)")

    # single stages, teacher forced on the oracle's intermediates
    qkv_tmp = bf16_empty(3, R, D)
    got = bf16_empty(R * max(D, F))  # each stage writes [R][N] row-major
    rows = lambda N: host_u16(got[:R * N]).reshape(R, N)
    w = syn.cfm_blocks[0]
    c = spec.cfg()
    ctx.dit_single(0, c, w, xd, None, B, L, cos, sin, qkv_tmp, got)
    ctx.sync()
    assert np.array_equal(rows(D), host_u16(out["att"])), "stage A == block's attention"
    assert np.array_equal(host_u16(qkv_tmp), host_u16(out["qkv"])), "stage A q/k/v == block's"
    ctx.dit_single(1, c, w, xd, dev_u16(tr["att"]), B, L, cos, sin, None, got)
    ctx.sync()
    assert_close_bf16(rows(D), tr["x1"], "stage B (teacher forced)")
    ctx.dit_single(2, c, w, dev_u16(tr["x1"]), None, B, L, cos, sin, None, got)
    ctx.sync()
    assert_close_bf16(rows(F), tr["hh"], "stage C (teacher forced)")
    ctx.dit_single(3, c, w, dev_u16(tr["x1"]), dev_u16(tr["hh"]), B, L, cos, sin, None, got)
    ctx.sync()
    assert_close_bf16(rows(D), ref, "stage D (teacher forced)")


def test_dit_rejects_bad_shapes(ming, ctx):
    S = syn_mod()
    spec = S.DitSpec(**SMALL, cfm_blocks=1)
    syn = S.SyntheticFlow(ctx, spec, seed=1, parts=("cfm",))
    cos, sin = rotary_dev(ctx, spec, 3)
    x = bf16_empty(8, spec.hidden)
    o = ming.DitOut(*(bf16_empty(3 * 8 * max(spec.hidden, spec.ff)).data_ptr() for _ in range(5)))
    with pytest.raises(ming.MingError) as e:
        ctx.dit_block(spec.cfg(), syn.cfm_blocks[0], x, 2, 4, cos, sin, o)  # 8 rows > 6
    assert e.value.status == ming.MING_E_SHAPE
    bad = S.DitSpec(hidden=128, heads=4, head_dim=64, ff=256).cfg()  # heads * head_dim != hidden
    with pytest.raises(ming.MingError) as e:
        ctx.dit_block(bad, syn.cfm_blocks[0], x, 1, 2, cos, sin, o)
    assert e.value.status == ming.MING_E_UNSUPPORTED
    w = syn.cfm_blocks[0]
    w2 = ming.DitBlockW.from_buffer_copy(w)
    w2.w1 = ming.linear(torch.empty((spec.ff, spec.hidden + 8), dtype=torch.bfloat16, device="cuda"))
    with pytest.raises(ming.MingError) as e:
        ctx.dit_block(spec.cfg(), w2, x, 1, 2, cos, sin, o)
    assert e.value.status == ming.MING_E_SHAPE


# ---- flow head pieces --------------------------------------------------------------

@pytest.fixture(scope="module")
def flow(ming, ctx):
    S = syn_mod()
    syn = S.SyntheticFlow(ctx, S.MING_DIT, seed=21, norm_std=0.05)
    return syn


@pytest.fixture(scope="module")
def flow_oracle(flow):
    oracle.set_threads(16)
    return oracle_cfm(flow), oracle_agg(flow)


@pytest.fixture(scope="module")
def flow_oracle_dev(flow):
    """The same oracle objects built in the kernels' summation order (their load-time
    timestep embeddings included); use them inside oracle.dit_order(DIT_ORDER_DEVICE)."""
    oracle.set_threads(16)
    with oracle.dit_order(oracle.DIT_ORDER_DEVICE):
        return oracle_cfm(flow), oracle_agg(flow)


def test_cfm_tables(ming, ctx, flow, flow_oracle, flow_oracle_dev):
    m = flow.cfm_model()
    t, dt, sq, te_ptr = m.tables()
    rt, rdt, rsq = oracle.flow_schedule()
    assert np.array_equal(t, rt), (t, rt)
    assert np.array_equal(dt, rdt) and np.array_equal(sq, rsq)
    assert t[0] == 0 and t[10] == 0x3F80, "schedule runs from 0 to 1"
    D = flow.spec.hidden
    te = np.empty((10, 2, D), np.uint16)
    ctx.check(ming.lib().ming_memcpy_dtoh(ctx.h, te.ctypes.data_as(ctypes.c_void_p), ctypes.c_void_p(te_ptr),
                                          te.nbytes))
    assert_close_bf16(te, flow_oracle[0].keep["te"], "timestep embeddings")
    assert_bits(te, flow_oracle_dev[0].keep["te"], "timestep embeddings (device order)")
    m.close()


def test_cfm_embed_and_final(ming, ctx, flow, flow_oracle):
    spec, h = flow.spec, flow.hostw
    D, lat = spec.hidden, spec.latent
    oc = flow_oracle[0]
    y = ming.synth_normal_bf16(31, "cfm.y", lat)
    te = ming.synth_normal_bf16(32, "cfm.te", 2 * D).reshape(2, D)
    ce = ming.synth_normal_bf16(33, "cfm.ce", 2 * D).reshape(2, D)
    xh = ming.synth_normal_bf16(34, "cfm.xh", D)
    rows = bf16_empty(6, D)
    ctx.cfm_embed(dev_u16(y), flow.lin_w(f"{CFM}.x_embedder"), flow.dev[f"{CFM}.x_embedder.bias"], dev_u16(te),
                  dev_u16(ce), dev_u16(xh), rows)
    ctx.sync()
    xn = oracle.linear(olin(flow, f"{CFM}.x_embedder"), y, h[f"{CFM}.x_embedder.bias"])
    want = np.stack([oracle.add(te[0], ce[0]), xh, xn, oracle.add(te[1], ce[1]), xh, xn])
    got = host_u16(rows)
    assert np.array_equal(got[[0, 1, 3, 4]], want[[0, 1, 3, 4]]), "t_emb + c_emb and x_emb(hist) rows"
    assert_close_bf16(got, want, "cfm rows")

    hh = ming.synth_normal_bf16(35, "cfm.h", 6 * D).reshape(6, D)
    sde = ming.synth_normal_bf16(36, "cfm.sde", 10 * lat).reshape(10, lat)
    dt_d, sq_d = dev_u16(oc.keep["dt"]), dev_u16(oc.keep["sq"])
    for step, cfg, shift in ((0, 2.0, 0.0), (4, 2.0, 0.25), (9, 1.5, 0.5)):
        yo = bf16_empty(lat)
        ctx.cfm_final(dev_u16(hh), 3, flow.dev[f"{CFM}.final_layer.norm_final.weight"],
                      flow.lin_w(f"{CFM}.final_layer.linear"), flow.dev[f"{CFM}.final_layer.linear.bias"],
                      dev_u16(y), dt_d, sq_d, dev_u16(sde), step, cfg, shift, yo)
        ctx.sync()
        ref = oracle.cfm_final(oc, hh, 3, y, sde, step, cfg, shift)
        assert_close_bf16(host_u16(yo), ref, f"cfm final step {step} cfg {cfg} shift {shift}")


@pytest.mark.parametrize("cfg,sigma,temperature", [(2.0, 0.25, 0.0), (2.0, 0.25, 1.0)])
def test_cfm_sample(ming, ctx, flow, flow_oracle, flow_oracle_dev, cfg, sigma, temperature):
    print(f"[cfm_sample] cfg={cfg} sigma={sigma} temperature={temperature}", flush=True)
    spec = flow.spec
    lat, H = spec.latent, spec.lm_hidden
    oc = flow_oracle[0]
    z = ming.synth_normal_bf16(41, "cfm.z", H)
    hist = ming.synth_normal_bf16(42, "cfm.hist", lat)
    noise = ming.synth_normal_bf16(43, "cfm.noise", lat)
    sde = ming.synth_normal_bf16(44, "cfm.sde", 10 * lat).reshape(10, lat)
    m = flow.cfm_model()
    out = bf16_empty(lat)
    steps = bf16_empty(10, lat)
    m.sample(dev_u16(z), dev_u16(hist), dev_u16(noise), dev_u16(sde), cfg, sigma, temperature, out, steps)
    ctx.sync()
    g_steps = host_u16(steps)
    assert np.array_equal(host_u16(out), g_steps[9]), "latent_out is the last step"
    shift = float(np.float32(sigma) * np.sqrt(np.float32(temperature)))
    c = ocfg(spec)
    # teacher forced: every Euler step from the GPU's previous latent
    for i in range(10):
        y_in = noise if i == 0 else g_steps[i - 1]
        h = oracle.cfm_rows(oc, z, hist, y_in, i)
        for blk in oc.blocks:
            h = oracle.dit_block_fwd(c, blk, h, 2, 3, oc.keep["cos"], oc.keep["sin"])
        ref = oracle.cfm_final(oc, h, 3, y_in, sde, i, cfg, shift)
        assert_close_bf16(g_steps[i], ref, f"Euler step {i} (teacher forced)")
    od = flow_oracle_dev[0]
    with oracle.dit_order(oracle.DIT_ORDER_DEVICE):
        for i in range(10):
            y_in = noise if i == 0 else g_steps[i - 1]
            h = oracle.cfm_rows(od, z, hist, y_in, i)
            for blk in od.blocks:
                h = oracle.dit_block_fwd(c, blk, h, 2, 3, od.keep["cos"], od.keep["sin"])
            assert_bits(g_steps[i], oracle.cfm_final(od, h, 3, y_in, sde, i, cfg, shift),
                        f"Euler step {i} (teacher forced, device order)")
    m.close()


@pytest.mark.parametrize("cfg,sigma,temperature", [(2.0, 0.25, 0.0), (2.0, 0.25, 1.0)])
def test_cfm_sample_end_to_end(ming, ctx, flow, flow_oracle, flow_oracle_dev, cfg, sigma, temperature):
    """The ten steps run free on both sides (the reference's parity replay, src/ming_parity.zig:204-235):
    every step's latent equals the oracle's in the kernels' summation order bit for bit, and the
    final latent is within the order-difference bound of the MLX-order oracle."""
    print(f"[cfm_sample_end_to_end] cfg={cfg} sigma={sigma} temperature={temperature}", flush=True)
    spec = flow.spec
    lat, H = spec.latent, spec.lm_hidden
    z = ming.synth_normal_bf16(41, "cfm.z", H)
    hist = ming.synth_normal_bf16(42, "cfm.hist", lat)
    noise = ming.synth_normal_bf16(43, "cfm.noise", lat)
    sde = ming.synth_normal_bf16(44, "cfm.sde", 10 * lat).reshape(10, lat)
    m = flow.cfm_model()
    out = bf16_empty(lat)
    steps = bf16_empty(10, lat)
    m.sample(dev_u16(z), dev_u16(hist), dev_u16(noise), dev_u16(sde), cfg, sigma, temperature, out, steps)
    ctx.sync()
    m.close()
    shift = float(np.float32(sigma) * np.sqrt(np.float32(temperature)))
    got, g_steps = host_u16(out), host_u16(steps)
    with oracle.dit_order(oracle.DIT_ORDER_DEVICE):
        ref_d, steps_d = oracle.cfm_sample(flow_oracle_dev[0], z, hist, noise, sde, cfg, shift)
    for i in range(10):
        assert_bits(g_steps[i], steps_d[i], f"free-running Euler step {i} (device order)")
    assert_close_bf16(got, ref_d, "sampled latent (end to end, device order)")
    ref_out, _ = oracle.cfm_sample(flow_oracle[0], z, hist, noise, sde, cfg, shift)
    g, r = got.view(np.uint16), ref_out
    gf, rf = (g.astype(np.uint32) << 16).view(np.float32), (r.astype(np.uint32) << 16).view(np.float32)
    assert np.isfinite(gf).all()
    assert_close_bf16(got, ref_out, "sampled latent (end to end, MLX order)", atol=6e-2, rtol=2e-2)
    assert float(np.abs(gf - rf).mean()) <= 2e-2


def test_aggregate(ming, ctx, flow, flow_oracle, flow_oracle_dev):
    spec = flow.spec
    oa = flow_oracle[1]
    m = flow.agg_model()
    for seed in (51, 52):
        latent = ming.synth_normal_bf16(seed, "agg.latent", spec.latent)
        out = bf16_empty(spec.lm_hidden)
        m.aggregate(dev_u16(latent), out)
        ctx.sync()
        assert_close_bf16(host_u16(out), oracle.aggregate(oa, latent), f"aggregate seed {seed}")
        with oracle.dit_order(oracle.DIT_ORDER_DEVICE):
            assert_bits(host_u16(out), oracle.aggregate(flow_oracle_dev[1], latent),
                        f"aggregate seed {seed} (device order)")
    m.close()


def test_aggregate_fused_attention_matches_unfused(ming, ctx, flow):
    """The aggregator's blocks (one sequence of two rows) run attention and out_proj as one launch;
    every block's output rows equal the unfused launches' (ming_dit_block: q/k/v, attention,
    out_proj, ff1, ff2) bit for bit on the same input rows, over consecutive calls."""
    spec = flow.spec
    D, F, nb = spec.hidden, spec.ff, spec.agg_blocks
    m = flow.agg_model()
    cos, sin = rotary_dev(ctx, spec, 2)
    rows = bf16_empty(nb + 1, 2, D)
    out_t, out_a = bf16_empty(spec.lm_hidden), bf16_empty(spec.lm_hidden)
    buf = dict(qkv=bf16_empty(3, 2, D), att=bf16_empty(2, D), x1=bf16_empty(2, D), hh=bf16_empty(2, F),
               x2=bf16_empty(2, D))
    o = ming.DitOut(*(buf[k].data_ptr() for k in ("qkv", "att", "x1", "hh", "x2")))
    for seed in (71, 72, 73):
        latent = dev_u16(ming.synth_normal_bf16(seed, "agg.latent", spec.latent))
        m.aggregate_trace(latent, rows, out_t)
        m.aggregate(latent, out_a)
        ctx.sync()
        assert_bits(host_u16(out_a), host_u16(out_t), f"aggregate vs its trace, seed {seed}")
        for b in range(nb):
            ctx.dit_block(spec.cfg(), flow.agg_blocks[b], rows[b], 1, 2, cos, sin, o)
            ctx.sync()
            assert_bits(host_u16(buf["x2"]), host_u16(rows[b + 1]), f"block {b} output, seed {seed}")
    m.close()


def test_stop_prob(ming, ctx, flow):
    H = flow.spec.lm_hidden
    head = olin(flow, "stop_head")
    p = torch.empty(1, dtype=torch.float32, device="cuda")
    for seed, sd in ((61, 1.0), (62, 8.0), (63, 30.0)):
        z = ming.synth_normal_bf16(seed, "stop.z", H, 0.0, sd)
        ctx.stop_prob(flow.lin_w("stop_head"), flow.dev["stop_head.bias"], dev_u16(z), p)
        ctx.sync()
        ref = oracle.stop_prob(head, flow.hostw["stop_head.bias"], z)
        assert abs(float(p.item()) - ref) <= 1e-2, (seed, float(p.item()), ref)
        with oracle.dit_order(oracle.DIT_ORDER_DEVICE):
            ref_d = oracle.stop_prob(head, flow.hostw["stop_head.bias"], z)
        assert np.float32(p.item()) == np.float32(ref_d), (seed, float(p.item()), ref_d, "device order")
        assert 0.0 <= float(p.item()) <= 1.0


def test_cfm_sample_unaligned_z(ming, ctx, flow):
    """c_emb reads z in place when it is 16-byte aligned and copies it first otherwise: a z two
    bytes off alignment gives the aligned call's latent and Euler steps bit for bit."""
    spec = flow.spec
    lat, H = spec.latent, spec.lm_hidden
    zh = ming.synth_normal_bf16(49, "unaligned.z", H)
    z = dev_u16(zh)
    zbuf = torch.zeros(H + 8, dtype=torch.bfloat16, device="cuda")
    zbuf[1:H + 1].copy_(z)
    zu = zbuf[1:H + 1]
    assert zu.data_ptr() % 16 != 0 and z.data_ptr() % 16 == 0
    hist = dev_u16(ming.synth_normal_bf16(46, "det.hist", lat))
    noise = dev_u16(ming.synth_normal_bf16(47, "det.noise", lat))
    sde = dev_u16(ming.synth_normal_bf16(48, "det.sde", 10 * lat).reshape(10, lat))
    m = flow.cfm_model()
    steps_a, steps_u = bf16_empty(10, lat), bf16_empty(10, lat)
    out_a, out_u = bf16_empty(lat), bf16_empty(lat)
    m.sample(z, hist, noise, sde, 2.0, 0.25, 1.0, out_a, steps_a)
    m.sample(zu, hist, noise, sde, 2.0, 0.25, 1.0, out_u, steps_u)
    ctx.sync()
    assert_bits(host_u16(steps_u), host_u16(steps_a), "Euler steps, unaligned z vs aligned")
    assert_bits(host_u16(out_u), host_u16(out_a), "latent, unaligned z vs aligned")
    m.close()


def test_cfm_sample_deterministic(ming, ctx, flow):
    """30 repeated samples of the same inputs are bit-identical to the first
    (the reference's flow-head determinism check, src/ming_fused_bench.zig:158-169),
    with the SDE term on so that every input of the update is exercised."""
    spec = flow.spec
    lat, H = spec.latent, spec.lm_hidden
    print("[cfm_sample] 30 repeats", flush=True)
    z = dev_u16(ming.synth_normal_bf16(45, "det.z", H))
    hist = dev_u16(ming.synth_normal_bf16(46, "det.hist", lat))
    noise = dev_u16(ming.synth_normal_bf16(47, "det.noise", lat))
    sde = dev_u16(ming.synth_normal_bf16(48, "det.sde", 10 * lat).reshape(10, lat))
    m = flow.cfm_model()
    outs = torch.empty((30, 10, lat), dtype=torch.bfloat16, device="cuda")
    lat_out = bf16_empty(lat)
    for i in range(30):
        m.sample(z, hist, noise, sde, 2.0, 0.25, 1.0, lat_out, outs[i])
    ctx.sync()
    first = host_u16(outs[0])
    for i in range(1, 30):
        assert np.array_equal(host_u16(outs[i]), first), f"repeat {i} differs from the first sample"
    m.close()
