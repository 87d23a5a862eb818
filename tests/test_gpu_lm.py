"""GPU parity of the Qwen2 decode step (ming_lm_layer, ming_lm_step,
ming_lm_generate) against the oracle on the same seeded inputs.

Bars (bf16 outputs): |gpu - ref| <= 2e-2 + 1e-2 |ref| for q/k/v, attention,
residual stream, swiglu, hidden states and logits; cache rows bit-exact where
the oracle and the kernel round the same value; greedy ids identical at every
step whose oracle top-2 logit margin exceeds 1e-4 (the head's logits on the
same stack output differ from the oracle's by at most ~4e-7, so a 1e-4 margin
leaves more than 200x room), and at the other steps (counted and reported)
the GPU's pick must be within 1e-4 of the oracle's best logit.  Each schedule
(per-stage kernels, persistent kernel) is checked against the oracle and must
reproduce itself bit for bit."""
import numpy as np
import pytest
import torch

import oracle
from lmkit import assert_close_bf16, f32, oracle_model, oracle_step

pytestmark = pytest.mark.gpu

MARGIN = 1e-4


def syn_mod(ming):
    import importlib

    return importlib.import_module("ming-tts-serve_amd.synthetic")


def dev_u16(a):
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).cuda().view(torch.bfloat16)


def host_u16(t):
    return t.view(torch.int16).cpu().numpy().view(np.uint16)


# ---- single layer ------------------------------------------------------------

LAYER_CASES = [
    # (hidden, heads, kv_heads, inter, quant, pos)
    (128, 2, 1, 256, True, 0),
    (128, 2, 1, 256, True, 37),
    (128, 2, 1, 256, False, 37),
    (896, 14, 2, 4864, True, 1),
    (896, 14, 2, 4864, True, 300),
    (896, 14, 2, 4864, False, 300),
    (896, 14, 2, 4864, True, 2047),
    (896, 14, 2, 4864, True, 5000),
]


@pytest.mark.parametrize("H,heads,kvh,I,quant,pos", LAYER_CASES)
def test_lm_layer_matches_oracle(ming, ctx, H, heads, kvh, I, quant, pos):
    print(f"[lm_layer] H={H} heads={heads}/{kvh} I={I} quant={quant} pos={pos}", flush=True)
    S = syn_mod(ming)
    spec = S.LmSpec(hidden=H, heads=heads, kv_heads=kvh, head_dim=64, inter=I, vocab=256, n_layers=1)
    syn = S.SyntheticLm(ctx, spec, seed=3, quant=quant, norm_std=0.1)
    cache = S.KvCache(spec, pos + 8)
    cache.fill_random(pos, seed=4)
    x = ming.synth_normal_bf16(5, "x", H, 0.0, 1.0)
    kvd = kvh * 64
    out = {k: torch.empty(n, dtype=torch.bfloat16, device="cuda")
           for k, n in (("qkv", H + 2 * kvd), ("o", H), ("x1", H), ("hh", I), ("x2", H))}
    lo = ming.LmOut(*(out[k].data_ptr() for k in ("qkv", "o", "x1", "hh", "x2")))
    kc0, vc0 = cache.host()
    ctx.lm_layer(syn.cfg, syn.layers[0], dev_u16(x), pos, cache.kv, 0, lo)
    ctx.sync()
    cfg, layers, _, _ = oracle_model(syn)
    kc, vc = kc0[0].copy(), vc0[0].copy()
    x2, tr = oracle.lm_layer_step(cfg, layers[0], x, pos, kc, vc, trace=True)
    assert_close_bf16(host_u16(out["qkv"]), tr["qkv"], "q|k|v (roped)")
    assert_close_bf16(host_u16(out["o"]), tr["att"], "attention")
    assert_close_bf16(host_u16(out["x1"]), tr["x1"], "x + o_proj")
    assert_close_bf16(host_u16(out["hh"]), tr["hh"], "swiglu")
    assert_close_bf16(host_u16(out["x2"]), x2, "layer output")
    gk, gv = cache.host()
    # the new row is the roped k / v of this token; other rows untouched
    assert_close_bf16(gk[0, :, pos], kc[:, pos], "cache k row")
    assert_close_bf16(gv[0, :, pos], vc[:, pos], "cache v row")
    keep = np.ones(gk.shape[2], bool)
    keep[pos] = False
    assert np.array_equal(gk[0][:, keep], kc0[0][:, keep]) and np.array_equal(gv[0][:, keep], vc0[0][:, keep])


# ---- full model ----------------------------------------------------------------

@pytest.fixture(scope="module")
def q4_model(ming, ctx):
    S = syn_mod(ming)
    print("[lm] building 24-layer 4-bit Qwen2-0.5B-shaped model", flush=True)
    syn = S.SyntheticLm(ctx, S.QWEN2_05B, seed=0, quant=True)
    m = syn.model()
    orc = oracle_model(syn)
    yield syn, m, orc
    m.close()


def run_step(ming, syn, m, cache, token, mode):
    spec = syn.spec
    m.set_mode(mode)
    tok = torch.tensor([token], dtype=torch.int32, device="cuda")
    hid = torch.empty(spec.hidden, dtype=torch.bfloat16, device="cuda")
    lg = torch.empty(spec.vocab, dtype=torch.float32, device="cuda")
    am = torch.empty(1, dtype=torch.int32, device="cuda")
    m.step(cache.kv, token=tok, hidden=hid, logits=lg, argmax=am)
    m.ctx.sync()
    return int(am.item()), host_u16(hid), lg.cpu().numpy()


def check_ids(got, ref_logits, ref_id, margin, what, dlogit=0.0):
    # with every logit within dlogit of the oracle's, a top-2 margin above 2 dlogit fixes the
    # argmax; the bar is 1e-4 unless the measured logit error were ever above half of it
    bar = max(MARGIN, 2.0 * dlogit)
    if margin > bar:
        assert got == ref_id, f"{what}: argmax {got} != {ref_id} (margin {margin:.3e})"
    else:
        assert ref_logits[got] >= ref_logits[ref_id] - bar, f"{what}: low-margin pick too far from the max"


def check_step_teacher_forced(ming, m, cache_before, cache_after, orc, pos, token, am, hid, lg, tag):
    """Every layer of the GPU step against the oracle run on the GPU's own
    input to that layer, then the head/argmax on the GPU's stack output.
    (A random-init 24-layer stack amplifies a one-ulp input change about
    650-fold, so two correct implementations with different f32 summation
    orders drift apart end to end; layer by layer they must agree.)"""
    cfg, layers, norm, head = orc
    tr = {k: host_u16(v) for k, v in m.trace().items()}
    kc, vc = cache_before
    gk, gv = cache_after
    assert np.array_equal(tr["x"][0], oracle.embed(head, token)), "embedding row"
    worst = 0.0
    for l, lay in enumerate(layers):
        k_l, v_l = kc[l].copy(), vc[l].copy()
        x2, t = oracle.lm_layer_step(cfg, lay, tr["x"][l], pos, k_l, v_l, trace=True)
        w = f"{tag} layer {l}"
        assert_close_bf16(tr["qkv"][l], t["qkv"], w + " q|k|v")
        assert_close_bf16(tr["att"][l], t["att"], w + " attention")
        assert_close_bf16(tr["x1"][l], t["x1"], w + " x1")
        assert_close_bf16(tr["hh"][l], t["hh"], w + " swiglu")
        worst = max(worst, assert_close_bf16(tr["x"][l + 1], x2, w + " output"))
        assert_close_bf16(gk[l, :, pos], k_l[:, pos], w + " appended k")
        assert_close_bf16(gv[l, :, pos], v_l[:, pos], w + " appended v")
    ram, rhid, rlg, _, margin = oracle.lm_head(cfg, norm, head, tr["x"][-1])
    assert_close_bf16(hid, rhid, f"{tag} final hidden")
    d = np.abs(lg.astype(np.float64) - rlg)
    assert (d <= 2e-2 + 1e-2 * np.abs(rlg)).all(), f"{tag} logits: max|d| {d.max():.3e}"
    check_ids(am, rlg, ram, margin, tag, float(d.max()))
    return worst, float(d.max()), ram, margin


MODES = {"kernels": "LM_KERNELS", "persistent": "LM_PERSISTENT", "direct": "LM_PERSISTENT_DIRECT",
         "xcd": "LM_PERSISTENT_XCD"}
XCD_MAX_CTX = 31 * 384  # kv head g's attention splits (384 positions each) on the 31 workers of one XCD slot


@pytest.mark.parametrize("mode", ["kernels", "persistent", "direct", "xcd"])
@pytest.mark.parametrize("ctx_len", [0, 1, 63, 64, 512, 2048, 4095, 8192, 11903, 16384])
def test_lm_step_matches_oracle(ming, ctx, q4_model, ctx_len, mode):
    S = syn_mod(ming)
    syn, m, orc = q4_model
    md = getattr(ming, MODES[mode])
    print(f"[lm_step] ctx={ctx_len} mode={mode}", flush=True)
    cache = S.KvCache(syn.spec, ctx_len + 4)
    cache.fill_random(ctx_len, seed=ctx_len)
    before = cache.host()
    token = 1234
    if mode == "xcd" and ctx_len + 1 > XCD_MAX_CTX:
        with pytest.raises(ming.MingError) as e:
            run_step(ming, syn, m, cache, token, md)
        assert e.value.status == ming.MING_E_UNSUPPORTED and cache.len == ctx_len
        return
    am, hid, lg = run_step(ming, syn, m, cache, token, md)
    assert cache.len == ctx_len + 1
    worst, dl, ram, margin = check_step_teacher_forced(ming, m, before, cache.host(), orc, ctx_len, token, am, hid,
                                                       lg, f"ctx {ctx_len} {mode}")
    print(f"[lm_step] ctx={ctx_len} {mode} argmax {am} ref {ram} margin {margin:.3e} worst layer max|d| {worst:.3e} "
          f"max|dlogit| {dl:.3e}", flush=True)


# 4-bit heads at the edges of the matrix-core head (16-row tiles, one MFMA per
# half group, an even number of groups up to 16): all 16 groups in use
# (hidden 1024), two groups (hidden 128), a single group (hidden 64: the
# register ring instead), and vocabularies that leave a partial last tile
HEAD_SHAPES = [  # (hidden, heads, kv_heads, inter, vocab)
    (1024, 16, 2, 512, 1000),
    (128, 2, 1, 256, 300),
    (64, 1, 1, 128, 37),
    (896, 14, 2, 256, 4099),
]


@pytest.mark.parametrize("H,heads,kvh,I,V", HEAD_SHAPES)
@pytest.mark.parametrize("mode", ["kernels", "persistent", "xcd"])
def test_q4_head_shapes_match_oracle(ming, ctx, H, heads, kvh, I, V, mode):
    S = syn_mod(ming)
    print(f"[lm_head] H={H} heads={heads}/{kvh} I={I} V={V} mode={mode}", flush=True)
    spec = S.LmSpec(hidden=H, heads=heads, kv_heads=kvh, head_dim=64, inter=I, vocab=V, n_layers=2)
    syn = S.SyntheticLm(ctx, spec, seed=H + V, quant=True)
    m = syn.model()
    try:
        orc = oracle_model(syn)
        cache = S.KvCache(spec, 40)
        cache.fill_random(33, seed=5)
        before = cache.host()
        am, hid, lg = run_step(ming, syn, m, cache, 7 % V, getattr(ming, MODES[mode]))
        worst, dl, ram, margin = check_step_teacher_forced(ming, m, before, cache.host(), orc, 33, 7 % V, am, hid, lg,
                                                           f"H {H} V {V} {mode}")
        print(f"[lm_head] H={H} V={V} {mode} argmax {am} ref {ram} margin {margin:.3e} max|dlogit| {dl:.3e}",
              flush=True)
    finally:
        m.close()


@pytest.fixture(scope="module")
def bf16_model(ming, ctx):
    S = syn_mod(ming)
    print("[lm] building 4-layer bf16 model at the Qwen2-0.5B layer shape", flush=True)
    syn = S.SyntheticLm(ctx, S.LmSpec(n_layers=4, vocab=8192), seed=12, quant=False)
    m = syn.model()
    yield syn, m, oracle_model(syn)
    m.close()


@pytest.mark.parametrize("mode", ["kernels", "persistent", "direct", "xcd"])
def test_bf16_lm_step_matches_oracle(ming, ctx, bf16_model, mode):
    """bf16 weights (the persistent kernel's second instance, plain bf16 rows
    instead of 4-bit chunks) at hidden 896, 14/2 heads, inter 4864, vocab
    8192, ctx 700: every layer teacher forced, head, logits and argmax."""
    S = syn_mod(ming)
    syn, m, orc = bf16_model
    print(f"[lm_step bf16] mode={mode}", flush=True)
    cache = S.KvCache(syn.spec, 704)
    cache.fill_random(700, seed=70)
    before = cache.host()
    am, hid, lg = run_step(ming, syn, m, cache, 4321, getattr(ming, MODES[mode]))
    assert cache.len == 701
    worst, dl, ram, margin = check_step_teacher_forced(ming, m, before, cache.host(), orc, 700, 4321, am, hid, lg,
                                                       f"bf16 {mode}")
    print(f"[lm_step bf16] {mode} argmax {am} ref {ram} margin {margin:.3e} worst layer max|d| {worst:.3e} "
          f"max|dlogit| {dl:.3e}", flush=True)


def test_schedules_agree_and_deterministic(ming, ctx, q4_model):
    """Each schedule is bit-for-bit reproducible; the persistent kernel gives
    the same bits with and without per-XCD hubs (the stage images are built by
    the same code), and it agrees with the per-stage kernels (which sum in
    different orders) within the bf16 tolerance."""
    S = syn_mod(ming)
    syn, m, _ = q4_model
    outs = {}
    for mode in (ming.LM_KERNELS, ming.LM_PERSISTENT, ming.LM_PERSISTENT_DIRECT, ming.LM_PERSISTENT_XCD):
        for rep in range(3):
            cache = S.KvCache(syn.spec, 1100)
            cache.fill_random(1000, seed=7)
            o = run_step(ming, syn, m, cache, 4321, mode)
            if mode in outs:
                ref = outs[mode]
                assert o[0] == ref[0] and np.array_equal(o[1], ref[1]) and np.array_equal(o[2], ref[2]), \
                    f"mode {mode} not reproducible (repeat {rep})"
            else:
                outs[mode] = o
    k, p, d = outs[ming.LM_KERNELS], outs[ming.LM_PERSISTENT], outs[ming.LM_PERSISTENT_DIRECT]
    assert p[0] == d[0] and np.array_equal(p[1], d[1]) and np.array_equal(p[2], d[2]), "hubs change the result"
    assert_close_bf16(p[1], k[1], "persistent vs kernels hidden", atol=0.2, rtol=0.1)
    x = outs[ming.LM_PERSISTENT_XCD]
    assert_close_bf16(x[1], k[1], "XCD-local vs kernels hidden", atol=0.2, rtol=0.1)


def test_xcd_coherent_handoffs_same_bits(ming, ctx, q4_model, monkeypatch):
    """The XCD-local schedule's hand-offs inside a slot go through that XCD's L2
    (plain stores) where the slot's workgroups share an XCD, else through
    device-coherent stores; MING_LM_XCD_LOCAL=0 forces the second form, which
    must give the same bits (the store kind changes no arithmetic)."""
    S = syn_mod(ming)
    syn, m, _ = q4_model
    outs = []
    for local in ("1", "0"):
        monkeypatch.setenv("MING_LM_XCD_LOCAL", local)
        cache = S.KvCache(syn.spec, 2100)
        cache.fill_random(2048, seed=21)
        outs.append([run_step(ming, syn, m, cache, t, ming.LM_PERSISTENT_XCD) for t in (5, 77777)])
    for a, b in zip(*outs):
        assert a[0] == b[0] and np.array_equal(a[1], b[1]) and np.array_equal(a[2], b[2]), \
            "device-coherent hand-offs change the result"


def test_ordinary_launch_matches_cooperative(ming, ctx, q4_model):
    """With the device held exclusively the persistent step is an ordinary
    launch; the kernel is the same, so the bits are the same, in both the hub
    and the direct schedule, over a few steps that grow the cache."""
    S = syn_mod(ming)
    syn, m, _ = q4_model
    try:
        for mode in (ming.LM_PERSISTENT, ming.LM_PERSISTENT_DIRECT, ming.LM_PERSISTENT_XCD):
            got = {}
            for excl in (False, True):
                ctx.set_exclusive(excl)
                cache = S.KvCache(syn.spec, 600)
                cache.fill_random(500, seed=11)
                got[excl] = [run_step(ming, syn, m, cache, t, mode) for t in (17, 9000, 151000)]
                assert cache.kv.len == 503
            for a, b in zip(got[False], got[True]):
                assert a[0] == b[0] and np.array_equal(a[1], b[1]) and np.array_equal(a[2], b[2]), \
                    f"mode {mode}: ordinary launch differs from cooperative"
    finally:
        ctx.set_exclusive(False)


def test_greedy_generate(ming, ctx, q4_model):
    """A prompt of 8 random ids fed one by one, then 12 greedy steps with the
    token fed back.  Every step is checked teacher-forced (each layer on the
    GPU's own input, the head and argmax on the GPU's own stack output), and
    ming_lm_generate (feedback on the device) must reproduce the ids."""
    S = syn_mod(ming)
    syn, m, orc = q4_model
    spec = syn.spec
    prompt = ming.synth_uniform_i32(0, "prompt", 8, spec.vocab)
    n = 12

    def fresh():
        c = S.KvCache(spec, 64)
        for t in prompt[:-1]:
            m.step(c.kv, token=torch.tensor([int(t)], dtype=torch.int32, device="cuda"))
        return c

    m.set_mode(ming.LM_AUTO)
    cache = fresh()
    ids = [int(prompt[-1])]
    lows = 0
    for i in range(n):
        before = cache.host()
        pos = cache.len
        am, hid, lg = run_step(ming, syn, m, cache, ids[-1], ming.LM_AUTO)
        _, _, ram, margin = check_step_teacher_forced(ming, m, before, cache.host(), orc, pos, ids[-1], am, hid, lg,
                                                      f"greedy step {i}")
        lows += margin <= MARGIN
        ids.append(am)
    cache2 = fresh()
    toks = torch.zeros(n + 1, dtype=torch.int32, device="cuda")
    toks[0] = ids[0]
    m.generate(cache2.kv, n, toks)
    ctx.sync()
    assert toks.cpu().numpy().tolist() == ids, "device-fed greedy ids differ from the step-by-step ids"
    print(f"[greedy] ids {ids} low-margin steps {lows}", flush=True)


def test_capacity_error(ming, ctx, q4_model):
    S = syn_mod(ming)
    syn, m, _ = q4_model
    cache = S.KvCache(syn.spec, 16)
    cache.kv.len = 16
    with pytest.raises(ming.MingError) as e:
        m.step(cache.kv, token=torch.tensor([1], dtype=torch.int32, device="cuda"))
    assert e.value.status == ming.MING_E_CTX_OVER_CAPACITY
