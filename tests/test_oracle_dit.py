"""Pins the DiT half of the oracle (flow head, aggregator, stop head) against
facts that do not come from the oracle's own formulas: closed forms of the
flow schedule and frequency table, float64 torch restatements of the block,
the CFM rows, the CFG/Euler update, the timestep MLP and the aggregator,
complex-number rotation for the interleaved rotary, exact invariants
(identity rotation at position 0, single-key attention returns v, the
unconditional row is t_emb + bias), and a zero-velocity flow whose sampled
latent has a closed form.  Each check is chosen so that a plausible slip
(rotary pairing or sign, attention scale, row selection of the final layer,
CFG sign, dt/sq/sde step index, [sin | cos] order, a dropped bias or norm
weight) fails it.  Every check runs in both of the oracle's summation orders (the MLX
restatement's, and the library kernels' order used for bit-exact GPU comparisons)."""
import importlib
import math

import numpy as np
import pytest
import torch

import oracle
from ditkit import ADA, AGG, CFM, oblock, ocfg, olin, oracle_adaln, oracle_agg, oracle_cfm

S = importlib.import_module("ming-tts-serve_amd.synthetic")

ATOL, RTOL = 2e-2, 1e-2


@pytest.fixture(autouse=True, params=[oracle.DIT_ORDER_MLX, oracle.DIT_ORDER_DEVICE], ids=["mlx_order", "device_order"])
def order(request):
    """Every pin of this module holds in both summation orders of the oracle's DiT functions."""
    with oracle.dit_order(request.param):
        yield request.param


def f64(u16):
    return torch.from_numpy(oracle.to_f32(np.asarray(u16, np.uint16)).astype(np.float64))


def bf16_bits(t):
    return t.to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)


def close(got_u16, want, what, atol=ATOL, rtol=RTOL):
    g = oracle.to_f32(np.asarray(got_u16, np.uint16)).astype(np.float64)
    w = np.asarray(want, np.float64)
    d = np.abs(g - w)
    bad = d > atol + rtol * np.abs(w)
    assert not bad.any(), f"{what}: {bad.sum()}/{bad.size} outside tol, max|d| {d.max():.3e}"


@pytest.fixture(scope="module")
def small():
    spec = S.DitSpec(hidden=128, heads=2, head_dim=64, ff=256, cfm_blocks=2, agg_blocks=2)
    return S.SyntheticFlow(None, spec, seed=7, std=0.1, norm_std=0.1, device="cpu")


# ---- float64 restatements (torch) --------------------------------------------------

def rms64(x, g, eps):
    return x / torch.sqrt((x * x).mean(-1, keepdim=True) + eps) * g


def rotate64(x, L, heads, hd, inv_freq):
    """Interleaved pairs (2i, 2i+1) as complex numbers times e^{i l f_i}."""
    R = x.shape[0]
    xc = torch.view_as_complex(x.reshape(R, heads, hd // 2, 2).contiguous())
    pos = torch.arange(R, dtype=torch.float64) % L
    ang = pos[:, None] * torch.from_numpy(inv_freq.astype(np.float64))[None, :]
    return torch.view_as_real(xc * torch.polar(torch.ones_like(ang), ang)[:, None, :]).reshape(R, heads * hd)


def block64(syn, prefix, i, x, B, L, tf=None):
    """One DiT block in float64.  With tf (the oracle's trace as f64 tensors),
    every stage starts from the oracle's output of the stage before it."""
    sp, h = syn.spec, syn.hostw
    b = f"{prefix}.blocks.{i}"
    W = lambda k: f64(h[f"{b}.{k}.weight"])
    bias = lambda k: f64(h[f"{b}.{k}.bias"])
    lin = lambda k, v: v @ W(k).T + bias(k)
    D, H, hd = sp.hidden, sp.heads, sp.head_dim
    R = B * L
    pick = lambda name, own: own if tf is None else tf[name]
    n1 = rms64(x, f64(h[f"{b}.norm1.weight"]), sp.eps)
    q = rotate64(lin("attn.to_q", n1), L, H, hd, sp.inv_freq())
    k = rotate64(lin("attn.to_k", n1), L, H, hd, sp.inv_freq())
    v = lin("attn.to_v", n1)
    sh = lambda t: t.reshape(B, L, H, hd).transpose(1, 2)
    s = (sh(pick("q", q)) @ sh(pick("k", k)).transpose(-1, -2)) / 8.0
    att = (torch.softmax(s, -1) @ sh(pick("v", v))).transpose(1, 2).reshape(R, D)
    x1 = x + lin("attn.to_out.0", pick("att", att))
    f = lin("mlp.ff.0.0", rms64(pick("x1", x1), f64(h[f"{b}.norm2.weight"]), sp.eps))
    hh = 0.5 * f * (1 + torch.tanh(math.sqrt(2 / math.pi) * (f + 0.044715 * f ** 3)))
    return pick("x1", x1) + lin("mlp.ff.2", pick("hh", hh)), dict(q=q, k=k, v=v, att=att, x1=x1, hh=hh)


# ---- schedule and tables -----------------------------------------------------------

def test_flow_schedule_closed_form():
    t, dt, sq = oracle.flow_schedule()
    s = np.array([0, 2, 4, 6, 8, 12, 16, 20, 24, 28, 32], np.float64) / 32
    want = 1.0 - np.cos(np.pi / 2 * s)  # t - (cos(pi t / 2) - 1 + t)
    tf = oracle.to_f32(t).astype(np.float64)
    # bf16 evaluation cancels near 1 (cos(pi t / 2) - 1 + t holds values of size ~1, rounded
    # at spacing 2^-8): at most three half-ulps at 1 of absolute error
    assert np.all(np.abs(tf - want) <= 3 * 2 ** -9), (tf, want)
    assert tf[0] == 0.0 and tf[10] == 1.0 and np.all(np.diff(tf) > 0)
    dtf = oracle.to_f32(dt).astype(np.float64)
    assert np.all(np.abs(dtf - np.diff(tf)) <= 2 ** -8 * np.diff(tf))
    sqf = oracle.to_f32(sq).astype(np.float64)
    assert np.all(np.abs(sqf - np.sqrt(dtf)) <= 2 ** -8 * np.sqrt(dtf))


def test_t_freq_closed_form():
    f = oracle.t_freq().astype(np.float64)
    want = 10000.0 ** (-np.arange(128) / 127.0)
    assert np.allclose(f, want, rtol=2e-6, atol=0)
    assert f[0] == 1.0


def test_rotary_table_and_rotation():
    inv = S.DitSpec(head_dim=64).inv_freq()
    assert np.allclose(inv.astype(np.float64), 10000.0 ** (-np.arange(0, 64, 2) / 64.0), rtol=1e-6)
    c, s = oracle.rotary_table(inv, 5)
    ang = np.arange(5, dtype=np.float32)[:, None] * inv[None, :]  # f32 product, as the table takes it
    assert np.allclose(c, np.cos(ang.astype(np.float64)), atol=2e-7)
    assert np.allclose(s, np.sin(ang.astype(np.float64)), atol=2e-7)
    rng = np.random.default_rng(3)
    x = bf16_bits(torch.from_numpy(rng.normal(0, 1, (6, 2 * 64)).astype(np.float32)))
    # position 0 (L = 1) is the identity, bit for bit
    assert np.array_equal(oracle.rotary(x, 1, 2, 64, c[:1], s[:1]), x)
    # L = 3: rows are positions 0, 1, 2, 0, 1, 2; complex rotation of pairs (2i, 2i+1)
    got = oracle.rotary(x, 3, 2, 64, c[:3], s[:3])
    close(got, rotate64(f64(x), 3, 2, 64, inv).numpy(), "rotary vs complex rotation", atol=1e-2, rtol=8e-3)


def test_timestep_embed_vs_f64(small):
    h = small.hostw
    m0, m2 = olin(small, f"{CFM}.t_embedder.time_mlp.0"), olin(small, f"{CFM}.t_embedder.time_mlp.2")
    t, _, _ = oracle.flow_schedule()
    for i in (0, 3, 9):
        got = oracle.timestep_embed(m0, h[f"{CFM}.t_embedder.time_mlp.0.bias"], m2,
                                    h[f"{CFM}.t_embedder.time_mlp.2.bias"], t[i])
        ts = (torch.tensor([float(oracle.to_f32(t[i:i + 1])[0])], dtype=torch.bfloat16) * 1000.0).double()
        e = ts * torch.from_numpy(oracle.t_freq().astype(np.float64))
        emb = torch.cat([torch.sin(e), torch.cos(e)])
        a = emb @ f64(h[f"{CFM}.t_embedder.time_mlp.0.weight"]).T + f64(h[f"{CFM}.t_embedder.time_mlp.0.bias"])
        a = a * torch.sigmoid(a)
        want = a @ f64(h[f"{CFM}.t_embedder.time_mlp.2.weight"]).T + f64(h[f"{CFM}.t_embedder.time_mlp.2.bias"])
        assert got.shape == (2, small.spec.hidden) and np.array_equal(got[0], got[1]), "both CFG halves"
        close(got[0], want.numpy(), f"t_emb step {i}")


# ---- block ---------------------------------------------------------------------------

@pytest.mark.parametrize("B,L", [(2, 3), (1, 2), (1, 1)])
def test_dit_block_vs_f64(small, B, L):
    sp = small.spec
    R = B * L
    x = bf16_bits(torch.from_numpy(np.random.default_rng(B * 10 + L).normal(0, 1, (R, sp.hidden))
                                   .astype(np.float32)))
    c, s = oracle.rotary_table(sp.inv_freq(), L)
    out, tr = oracle.dit_block_fwd(ocfg(sp), oblock(small, CFM, 0), x, B, L, c, s, trace=True)
    # each stage from the oracle's previous stage (teacher forced)
    tf = dict(q=f64(tr["qkv"][0]), k=f64(tr["qkv"][1]), v=f64(tr["qkv"][2]), att=f64(tr["att"]),
              x1=f64(tr["x1"]), hh=f64(tr["hh"]))
    want, w = block64(small, CFM, 0, f64(x), B, L, tf)
    close(tr["qkv"][0], w["q"].numpy(), "q rotated")
    close(tr["qkv"][1], w["k"].numpy(), "k rotated")
    close(tr["qkv"][2], w["v"].numpy(), "v")
    close(tr["att"], w["att"].numpy(), "attention")
    close(tr["x1"], w["x1"].numpy(), "x + out_proj")
    close(tr["hh"], w["hh"].numpy(), "gelu(ff1)")
    close(out, want.numpy(), "block output")
    # the whole block from x alone (rounding of four stages accumulates)
    close(out, block64(small, CFM, 0, f64(x), B, L)[0].numpy(), "block output (free running)", atol=6e-2)
    if L == 1:
        assert np.array_equal(tr["att"], tr["qkv"][2]), "one key: attention returns v"


# ---- CFM rows, final, sample ---------------------------------------------------------

def test_cfm_rows_vs_f64(small):
    oc = oracle_cfm(small)
    h, D = small.hostw, small.spec.hidden
    rng = np.random.default_rng(5)
    z = bf16_bits(torch.from_numpy(rng.normal(0, 1, small.spec.lm_hidden).astype(np.float32)))
    hist = bf16_bits(torch.from_numpy(rng.normal(0, 1, 64).astype(np.float32)))
    y = bf16_bits(torch.from_numpy(rng.normal(0, 1, 64).astype(np.float32)))
    rows = oracle.cfm_rows(oc, z, hist, y, 4)
    te = oc.keep["te"][4]
    lin = lambda k, v: v @ f64(h[f"{CFM}.{k}.weight"]).T + f64(h[f"{CFM}.{k}.bias"])
    close(rows[0], (f64(te[0]) + lin("c_embedder.cond_embedder", f64(z))).numpy(), "cond row 0")
    # unconditional half: c_emb(0) is its bias, added to t_emb in bf16
    bc = torch.from_numpy(oracle.to_f32(h[f"{CFM}.c_embedder.cond_embedder.bias"])).to(torch.bfloat16)
    assert np.array_equal(rows[3], bf16_bits(torch.from_numpy(oracle.to_f32(te[1])).to(torch.bfloat16) + bc))
    close(rows[1], lin("x_embedder", f64(hist)).numpy(), "x_emb(hist)")
    close(rows[2], lin("x_embedder", f64(y)).numpy(), "x_emb(y)")
    assert np.array_equal(rows[1], rows[4]) and np.array_equal(rows[2], rows[5])


@pytest.mark.parametrize("step,cfg,shift", [(0, 2.0, 0.0), (6, 2.0, 0.25), (9, 3.0, 0.5)])
def test_cfm_final_vs_f64(small, step, cfg, shift):
    oc = oracle_cfm(small)
    h = small.hostw
    rng = np.random.default_rng(step)
    hh = bf16_bits(torch.from_numpy(rng.normal(0, 1, (6, small.spec.hidden)).astype(np.float32)))
    y = bf16_bits(torch.from_numpy(rng.normal(0, 1, 64).astype(np.float32)))
    sde = bf16_bits(torch.from_numpy(rng.normal(0, 1, (10, 64)).astype(np.float32)))
    got = oracle.cfm_final(oc, hh, 3, y, sde, step, cfg, shift)
    nw = f64(h[f"{CFM}.final_layer.norm_final.weight"])
    lin = lambda v: v @ f64(h[f"{CFM}.final_layer.linear.weight"]).T + f64(h[f"{CFM}.final_layer.linear.bias"])
    pc = lin(rms64(f64(hh[2]), nw, 1e-6))  # last position of the conditional half
    pu = lin(rms64(f64(hh[5]), nw, 1e-6))  # last position of the unconditional half
    dt = f64(oc.keep["dt"])[step]
    sq = f64(oc.keep["sq"])[step]
    want = f64(y) + dt * (pc + (pc - pu) * cfg) + shift * sq * f64(sde[step])
    close(got, want.numpy(), f"Euler step {step}")


def test_zero_velocity_sample_closed_form(small):
    """Final layer weights 0: every step's velocity is the final bias b (cond ==
    uncond), so y_10 = noise + (t_10 - t_0) b + shift * sum_i sq_i sde_i."""
    h = small.hostw
    oc0 = oracle_cfm(small)
    zero = oracle.Linear(np.zeros_like(h[f"{CFM}.final_layer.linear.weight"]))
    k = oc0.keep
    oc = oracle.CfmModel(ocfg(small.spec), oc0.blocks, olin(small, f"{CFM}.x_embedder"), k["bx"],
                         olin(small, f"{CFM}.c_embedder.cond_embedder"), k["bc"], k["fn"], zero, k["bf"], k["te"],
                         k["dt"], k["sq"], k["cos"], k["sin"])
    rng = np.random.default_rng(9)
    mk = lambda *sh: bf16_bits(torch.from_numpy(rng.normal(0, 1, sh).astype(np.float32)))
    z, hist, noise, sde = mk(small.spec.lm_hidden), mk(64), mk(64), mk(10, 64)
    b = f64(k["bf"])
    for shift in (0.0, 0.5):
        out, steps = oracle.cfm_sample(oc, z, hist, noise, sde, 2.0, shift)
        want = f64(noise) + b + shift * (f64(k["sq"])[:, None] * f64(sde)).sum(0)
        close(out, want.numpy(), f"zero-velocity sample shift {shift}", atol=3e-2)
        assert np.array_equal(out, steps[9])


# ---- aggregator and stop head ----------------------------------------------------------

def test_aggregate_vs_f64(small):
    oa = oracle_agg(small)
    h = small.hostw
    lat = bf16_bits(torch.from_numpy(np.random.default_rng(11).normal(0, 1, 64).astype(np.float32)))
    got = oracle.aggregate(oa, lat)
    xe = f64(lat) @ f64(h[f"{AGG}.x_embedder.weight"]).T + f64(h[f"{AGG}.x_embedder.bias"])
    x = torch.stack([f64(h[f"{AGG}.word_embedder.weight"]), xe])
    for i in range(small.spec.agg_blocks):
        x, _ = block64(small, AGG, i, x, 1, 2)
    want = rms64(x[0], f64(h[f"{AGG}.final_layer.norm_final.weight"]), 1e-6) @ \
        f64(h[f"{AGG}.final_layer.linear.weight"]).T + f64(h[f"{AGG}.final_layer.linear.bias"])
    close(got, want.numpy(), "aggregate (cls row)", atol=3e-2, rtol=2e-2)


def test_stop_prob_closed_forms(small):
    head = olin(small, "stop_head")
    bias = small.hostw["stop_head.bias"]
    bb = oracle.to_f32(bias).astype(np.float64)
    zero = np.zeros(small.spec.lm_hidden, np.uint16)
    assert abs(oracle.stop_prob(head, bias, zero) - 1.0 / (1.0 + math.exp(bb[0] - bb[1]))) < 1e-6
    for sd in (1.0, 10.0):
        z = bf16_bits(torch.from_numpy(np.random.default_rng(int(sd)).normal(0, sd, small.spec.lm_hidden)
                                       .astype(np.float32)))
        lg = f64(small.hostw["stop_head.weight"]) @ f64(z) + torch.from_numpy(bb)
        want = float(torch.softmax(lg, 0)[1])
        assert abs(oracle.stop_prob(head, bias, z) - want) < 1e-2


# ---- adaLN flow head (config 4; the build's own definition) -----------------------------

@pytest.fixture(scope="module")
def ada_small():
    spec = S.AdalnSpec(hidden=128, heads=2, head_dim=64, ff=256, cfm_blocks=2, frames=3)
    return S.SyntheticAdaln(None, spec, seed=17, std=0.1, norm_std=0.1, ada_std=0.05, device="cpu")


def zero_mod(B, D):
    m = np.zeros((B, 6 * D), np.uint16)
    m[:, 2 * D:3 * D] = 0x3F80
    m[:, 5 * D:6 * D] = 0x3F80
    return m


def test_adaln_zero_modulation_is_the_reference_block(ada_small):
    sp = ada_small.spec
    x = bf16_bits(torch.from_numpy(np.random.default_rng(2).normal(0, 1, (6, sp.hidden)).astype(np.float32)))
    c, s = oracle.rotary_table(sp.inv_freq(), 3)
    blk = oblock(ada_small, ADA, 0)
    ref, tr = oracle.dit_block_fwd(ocfg(sp), blk, x, 2, 3, c, s, trace=True)
    got, tg = oracle.adaln_block_fwd(ocfg(sp), blk, zero_mod(2, sp.hidden), x, 2, 3, c, s, trace=True)
    assert np.array_equal(oracle.to_f32(got), oracle.to_f32(ref))
    for k in ("qkv", "att", "x1", "hh"):
        assert np.array_equal(oracle.to_f32(tg[k]), oracle.to_f32(tr[k])), k


def test_adaln_block_vs_f64(ada_small):
    sp = ada_small.spec
    B, L, D = 2, 3, sp.hidden
    rng = np.random.default_rng(4)
    x = bf16_bits(torch.from_numpy(rng.normal(0, 1, (B * L, D)).astype(np.float32)))
    mod = bf16_bits(torch.from_numpy(rng.normal(0, 0.3, (B, 6 * D)).astype(np.float32)))
    c, s = oracle.rotary_table(sp.inv_freq(), L)
    out, tr = oracle.adaln_block_fwd(ocfg(sp), oblock(ada_small, ADA, 0), mod, x, B, L, c, s, trace=True)
    h, b = ada_small.hostw, f"{ADA}.blocks.0"
    lin = lambda k, v: v @ f64(h[f"{b}.{k}.weight"]).T + f64(h[f"{b}.{k}.bias"])
    md = f64(mod).reshape(B, 6, D)
    per_row = lambda j: md[:, j, :].repeat_interleave(L, 0)  # [B*L][D]
    modulate = lambda n, j: n * (1 + per_row(j + 1)) + per_row(j)
    # each stage from the oracle's previous stage (teacher forced)
    xf = f64(x)
    n1 = modulate(rms64(xf, f64(h[f"{b}.norm1.weight"]), sp.eps), 0)
    q = rotate64(lin("attn.to_q", n1), L, sp.heads, sp.head_dim, sp.inv_freq())
    close(tr["qkv"][0], q.numpy(), "q (modulated, rotated)")
    close(tr["qkv"][2], lin("attn.to_v", n1).numpy(), "v (modulated)")
    x1 = xf + per_row(2) * lin("attn.to_out.0", f64(tr["att"]))
    close(tr["x1"], x1.numpy(), "x + gate_a * out_proj")
    f = lin("mlp.ff.0.0", modulate(rms64(f64(tr["x1"]), f64(h[f"{b}.norm2.weight"]), sp.eps), 3))
    hh = 0.5 * f * (1 + torch.tanh(math.sqrt(2 / math.pi) * (f + 0.044715 * f ** 3)))
    close(tr["hh"], hh.numpy(), "gelu(ff1(modulated))")
    want = f64(tr["x1"]) + per_row(5) * lin("mlp.ff.2", f64(tr["hh"]))
    close(out, want.numpy(), "block output")


def test_adaln_cond_mods_and_final_vs_f64(ada_small):
    sp, h = ada_small.spec, ada_small.hostw
    om = oracle_adaln(ada_small)
    D = sp.hidden
    z = bf16_bits(torch.from_numpy(np.random.default_rng(6).normal(0, 1, sp.lm_hidden).astype(np.float32)))
    sc = oracle.adaln_cond(om, z)
    ce = torch.stack([f64(z), torch.zeros(sp.lm_hidden, dtype=torch.float64)]) @ \
        f64(h[f"{ADA}.c_embedder.weight"]).T + f64(h[f"{ADA}.c_embedder.bias"])
    te = f64(om.keep["te"])
    cc = te + ce[None]
    close(sc, (cc * torch.sigmoid(cc)).numpy(), "silu(t_emb + c_emb)")
    mods, modf = oracle.adaln_mods(om, sc)
    w0 = f"{ADA}.blocks.1.adaLN_modulation.1"
    want = f64(sc).reshape(20, D) @ f64(h[w0 + ".weight"]).T + f64(h[w0 + ".bias"])
    close(mods[1], want.numpy(), "block 1 modulations")
    # final layer: rows [2F][D], modulation of step 7
    F, step = sp.frames, 7
    rng = np.random.default_rng(8)
    hrow = bf16_bits(torch.from_numpy(rng.normal(0, 1, (2 * F, D)).astype(np.float32)))
    y = bf16_bits(torch.from_numpy(rng.normal(0, 1, (F, 64)).astype(np.float32)))
    sde = bf16_bits(torch.from_numpy(rng.normal(0, 1, (10, F, 64)).astype(np.float32)))
    got = oracle.adaln_final(om, hrow, modf[2 * step:2 * step + 2], y, sde, step, 2.0, 0.5)
    mf = f64(modf[2 * step:2 * step + 2]).reshape(2, 2, D)
    n = rms64(f64(hrow), f64(h[f"{ADA}.final_layer.norm_final.weight"]), sp.eps)
    half = torch.arange(2 * F) // F
    hm = n * (1 + mf[half, 1]) + mf[half, 0]
    o = hm @ f64(h[f"{ADA}.final_layer.linear.weight"]).T + f64(h[f"{ADA}.final_layer.linear.bias"])
    pc, pu = o[:F], o[F:]
    want = f64(y) + f64(om.keep["dt"])[step] * (pc + (pc - pu) * 2.0) + 0.5 * f64(om.keep["sq"])[step] * f64(sde[step])
    close(got, want.numpy(), "final adaLN layer + CFG + Euler (per frame)")


def test_adaln_zero_velocity_closed_form(ada_small):
    """Final linear 0: the velocity of every frame is the final bias b, so
    y_10 = noise + (t_10 - t_0) b + shift * sum_i sq_i sde_i per frame."""
    om0 = oracle_adaln(ada_small)
    h, sp = ada_small.hostw, ada_small.spec
    k = om0.keep
    zero = oracle.Linear(np.zeros_like(h[f"{ADA}.final_layer.linear.weight"]))
    om = oracle.AdalnModel(ocfg(sp), om0.blocks, olin(ada_small, f"{ADA}.x_embedder"), k["bx"],
                           olin(ada_small, f"{ADA}.c_embedder"), k["bc"], k["fn"], zero, k["bf"],
                           olin(ada_small, f"{ADA}.final_layer.adaLN_modulation.1"), k["bfa"], k["te"], k["dt"],
                           k["sq"], k["cos"], k["sin"], sp.frames)
    rng = np.random.default_rng(10)
    mk = lambda *shape: bf16_bits(torch.from_numpy(rng.normal(0, 1, shape).astype(np.float32)))
    z, noise, sde = mk(sp.lm_hidden), mk(sp.frames, 64), mk(10, sp.frames, 64)
    for shift in (0.0, 0.5):
        out, steps = oracle.adaln_sample(om, z, noise, sde, 2.0, shift)
        want = f64(noise) + f64(k["bf"])[None] + shift * (f64(k["sq"])[:, None, None] * f64(sde)).sum(0)
        close(out, want.numpy(), f"adaLN zero-velocity sample shift {shift}", atol=3e-2)
        assert np.array_equal(out, steps[9])
