"""GPU parity of the flow head over many sequences (ming_cfm_sample_batch:
cfmSample, src/ming_model.zig:1143-1151, :1161-1203, for n sequences in one
pass, every DiT linear one bf16 matrix-core GEMM over the 6 n rows) against
the oracle, at the reference shape (8 blocks, hidden 1024, 16 x 64 heads,
ff 4096).

Bars (those of the single-sequence flow head): every Euler step of every
sequence, teacher forced on the GPU's own previous latent, within
2e-2 + 1e-2 |ref|; each sequence equal to a one-sequence batch call (bit for
bit: the GEMMs' per-row arithmetic does not depend on n); the free-running
ten-step latent of every sequence finite and within 6e-2 + 2e-2 |ref| (mean
|d| <= 2e-2) of the oracle.  The free-running latent against the per-step
2e-2 + 1e-2 |ref| bar is a separate non-strict expected failure: the matrix
cores' f32 accumulation of a 32-product block is not IEEE sequential, pairwise
or single-rounding (measured with chosen operands: up to a few f32 ulps away
from every such model), so no CPU order reproduces it bit for bit, and the
8-block, 10-step CFG loop grows the bf16 flips this causes past the bar on some
seeds (the batch-1 flow head, whose order the oracle reproduces, is held to
that bar bit for bit in test_gpu_dit.py)."""
import numpy as np
import pytest
import torch

import oracle
from ditkit import ocfg, oracle_cfm
from lmkit import assert_close_bf16

pytestmark = pytest.mark.gpu


def syn_mod():
    import importlib

    return importlib.import_module("ming-tts-serve_amd.synthetic")


def dev_u16(a):
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).cuda().view(torch.bfloat16)


def host_u16(t):
    return t.view(torch.int16).cpu().numpy().view(np.uint16)


@pytest.fixture(scope="module")
def flowb(ming, ctx):
    S = syn_mod()
    syn = S.SyntheticFlow(ctx, S.MING_DIT, seed=61, norm_std=0.05, parts=("cfm",))
    oracle.set_threads(16)
    return syn, syn.cfm_model(), oracle_cfm(syn)


def inputs(ming, spec, n, tag):
    z = ming.synth_normal_bf16(71, f"{tag}.z", n * spec.lm_hidden).reshape(n, spec.lm_hidden)
    hist = ming.synth_normal_bf16(72, f"{tag}.hist", n * spec.latent).reshape(n, spec.latent)
    noise = ming.synth_normal_bf16(73, f"{tag}.noise", n * spec.latent).reshape(n, spec.latent)
    sde = ming.synth_normal_bf16(74, f"{tag}.sde", n * 10 * spec.latent).reshape(n, 10, spec.latent)
    return z, hist, noise, sde


@pytest.mark.parametrize("n,cfg,sigma,temperature", [(5, 2.0, 0.25, 1.0), (16, 2.0, 0.0, 0.0),
                                                     (64, 2.0, 0.25, 1.0)])
def test_cfm_batch_matches_oracle(ming, ctx, flowb, n, cfg, sigma, temperature):
    print(f"[cfm_batch] n={n} cfg={cfg} sigma={sigma} temperature={temperature}", flush=True)
    syn, m, oc = flowb
    spec = syn.spec
    z, hist, noise, sde = inputs(ming, spec, n, f"b{n}")
    out = torch.empty((n, spec.latent), dtype=torch.bfloat16, device="cuda")
    steps = torch.empty((n, 10, spec.latent), dtype=torch.bfloat16, device="cuda")
    m.sample_batch(n, dev_u16(z), dev_u16(hist), dev_u16(noise), dev_u16(sde), cfg, sigma, temperature, out, steps)
    ctx.sync()
    g = host_u16(steps)
    assert np.array_equal(host_u16(out), g[:, 9])
    shift = float(np.float32(sigma) * np.sqrt(np.float32(temperature)))
    c = ocfg(spec)
    check = range(n) if n <= 5 else sorted({0, n // 2, n - 1} | set(range(3, n, max(1, n // 6))))
    for b in check:
        for i in range(10):
            y_in = noise[b] if i == 0 else g[b, i - 1]
            h = oracle.cfm_rows(oc, z[b], hist[b], y_in, i)
            for blk in oc.blocks:
                h = oracle.dit_block_fwd(c, blk, h, 2, 3, oc.keep["cos"], oc.keep["sin"])
            ref = oracle.cfm_final(oc, h, 3, y_in, sde[b], i, cfg, shift)
            assert_close_bf16(g[b, i], ref, f"sequence {b} Euler step {i} (teacher forced)")



def test_cfm_batch_rows_independent_of_n(ming, ctx, flowb):
    syn, m, oc = flowb
    spec = syn.spec
    n = 64
    z, hist, noise, sde = (dev_u16(a) for a in inputs(ming, spec, n, "ind"))
    out = torch.empty((n, spec.latent), dtype=torch.bfloat16, device="cuda")
    m.sample_batch(n, z, hist, noise, sde, 2.0, 0.25, 1.0, out)
    one = torch.empty((1, spec.latent), dtype=torch.bfloat16, device="cuda")
    for b in (0, 7, 19, 40, 63):
        m.sample_batch(1, z[b:b + 1], hist[b:b + 1], noise[b:b + 1], sde[b:b + 1], 2.0, 0.25, 1.0, one)
        ctx.sync()
        assert torch.equal(one[0], out[b]), b


def test_cfm_batch_rejects(ming, ctx, flowb):
    syn, m, oc = flowb
    spec = syn.spec
    buf = torch.empty((65, spec.latent), dtype=torch.bfloat16, device="cuda")
    with pytest.raises(ming.MingError) as e:
        m.sample_batch(65, buf, buf, buf, buf, 2.0, 0.0, 0.0, buf)
    assert e.value.status == ming.MING_E_UNSUPPORTED


def test_cfm_batch_deterministic(ming, ctx, flowb):
    """30 repeated batched samples (split-K GEMMs with their ordered reduce) are
    bit-identical to the first (src/ming_fused_bench.zig:158-169)."""
    syn, m, _ = flowb
    spec, n = syn.spec, 12
    print(f"[cfm_batch] 30 repeats n={n}", flush=True)
    z, hist, noise, sde = (dev_u16(a) for a in inputs(ming, spec, n, "det"))
    outs = torch.empty((30, n, spec.latent), dtype=torch.bfloat16, device="cuda")
    for i in range(30):
        m.sample_batch(n, z, hist, noise, sde, 2.0, 0.25, 1.0, outs[i])
    ctx.sync()
    first = host_u16(outs[0])
    for i in range(1, 30):
        assert np.array_equal(host_u16(outs[i]), first), f"repeat {i} differs from the first batched sample"


def _batch_free_run(ming, ctx, flowb, n, cfg, sigma, temperature):
    syn, m, oc = flowb
    spec = syn.spec
    z, hist, noise, sde = inputs(ming, spec, n, f"b{n}")
    out = torch.empty((n, spec.latent), dtype=torch.bfloat16, device="cuda")
    m.sample_batch(n, dev_u16(z), dev_u16(hist), dev_u16(noise), dev_u16(sde), cfg, sigma, temperature, out)
    ctx.sync()
    shift = float(np.float32(sigma) * np.sqrt(np.float32(temperature)))
    g = host_u16(out)
    refs = [oracle.cfm_sample(oc, z[b], hist[b], noise[b], sde[b], cfg, shift)[0] for b in range(n)]
    return g, refs


@pytest.mark.parametrize("n,cfg,sigma,temperature", [(5, 2.0, 0.25, 1.0), (16, 2.0, 0.0, 0.0)])
def test_cfm_batch_end_to_end_bound(ming, ctx, flowb, n, cfg, sigma, temperature):
    """Free-running latents of every sequence: finite and within the order-difference bound."""
    print(f"[cfm_batch_end_to_end] n={n}", flush=True)
    g, refs = _batch_free_run(ming, ctx, flowb, n, cfg, sigma, temperature)
    for b in range(n):
        gf = (g[b].astype(np.uint32) << 16).view(np.float32)
        rf = (refs[b].astype(np.uint32) << 16).view(np.float32)
        assert np.isfinite(gf).all(), b
        assert_close_bf16(g[b], refs[b], f"sequence {b} latent (end to end)", atol=6e-2, rtol=2e-2)
        assert float(np.abs(gf - rf).mean()) <= 2e-2, b


@pytest.mark.xfail(strict=False, reason="free-running ten-step latent at 2e-2 + 1e-2|ref|: the matrix cores' f32 accumulation is not reproduced by any CPU summation order, and the 8-block, 10-step CFG loop grows the resulting bf16 flips past the bar on some seeds (teacher-forced steps meet it; the batch-1 flow head is bit-exact free-running)")
@pytest.mark.parametrize("n,cfg,sigma,temperature", [(5, 2.0, 0.25, 1.0)])
def test_cfm_batch_end_to_end_strict(ming, ctx, flowb, n, cfg, sigma, temperature):
    g, refs = _batch_free_run(ming, ctx, flowb, n, cfg, sigma, temperature)
    for b in range(n):
        assert_close_bf16(g[b], refs[b], f"sequence {b} latent (end to end)")
