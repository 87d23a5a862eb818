"""GPU parity of the flow head over many sequences (ming_cfm_sample_batch:
cfmSample, src/ming_model.zig:1143-1151, :1161-1203, for n sequences in one
pass, every DiT linear one bf16 matrix-core GEMM over the 6 n rows) against
the oracle, at the reference shape (8 blocks, hidden 1024, 16 x 64 heads,
ff 4096).

Bars: every Euler step of every checked sequence, teacher forced on the GPU's
own previous latent, within 2e-2 + 1e-2 |ref| of the MLX-order oracle and bit
for bit with the oracle in the batched kernels' order
(oracle.dit_order(DIT_ORDER_MFMA): the GEMMs' dot products as the matrix
instruction accumulates them, 8 consecutive k per step, in the kernel's fixed
K slices; or_acc_step is pinned against the device in test_oracle_arith.py and
test_gpu_arith.py); each sequence equal to a one-sequence batch call (bit for
bit: the GEMMs' per-row arithmetic does not depend on n); the free-running
ten-step latent of every sequence bit for bit with that oracle at every step,
and finite and within 6e-2 + 2e-2 |ref| (mean |d| <= 2e-2) of the MLX-order
oracle."""
import numpy as np
import pytest
import torch

import oracle
from ditkit import ocfg, oracle_cfm
from lmkit import assert_bits, assert_close_bf16

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
    with oracle.dit_order(oracle.DIT_ORDER_DEVICE):  # load-time tables as the model builds them
        od = oracle_cfm(syn)
    return syn, syn.cfm_model(), oracle_cfm(syn), od


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
    syn, m, oc, od = flowb
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
    with oracle.dit_order(oracle.DIT_ORDER_MFMA):
        for b in check[:3]:
            for i in range(10):
                y_in = noise[b] if i == 0 else g[b, i - 1]
                h = oracle.cfm_rows(od, z[b], hist[b], y_in, i)
                for blk in od.blocks:
                    h = oracle.dit_block_fwd(c, blk, h, 2, 3, od.keep["cos"], od.keep["sin"])
                assert_bits(g[b, i], oracle.cfm_final(od, h, 3, y_in, sde[b], i, cfg, shift),
                            f"sequence {b} Euler step {i} (teacher forced, batched order)")



def test_cfm_batch_rows_independent_of_n(ming, ctx, flowb):
    syn, m, oc, od = flowb
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
    syn, m, oc, od = flowb
    spec = syn.spec
    buf = torch.empty((65, spec.latent), dtype=torch.bfloat16, device="cuda")
    with pytest.raises(ming.MingError) as e:
        m.sample_batch(65, buf, buf, buf, buf, 2.0, 0.0, 0.0, buf)
    assert e.value.status == ming.MING_E_UNSUPPORTED


def test_cfm_batch_deterministic(ming, ctx, flowb):
    """30 repeated batched samples (split-K GEMMs with their ordered reduce) are
    bit-identical to the first (src/ming_fused_bench.zig:158-169)."""
    syn, m, _, _ = flowb
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
    syn, m, oc, od = flowb
    spec = syn.spec
    z, hist, noise, sde = inputs(ming, spec, n, f"b{n}")
    out = torch.empty((n, spec.latent), dtype=torch.bfloat16, device="cuda")
    steps = torch.empty((n, 10, spec.latent), dtype=torch.bfloat16, device="cuda")
    m.sample_batch(n, dev_u16(z), dev_u16(hist), dev_u16(noise), dev_u16(sde), cfg, sigma, temperature, out, steps)
    ctx.sync()
    shift = float(np.float32(sigma) * np.sqrt(np.float32(temperature)))
    return host_u16(out), host_u16(steps), (z, hist, noise, sde), shift


@pytest.mark.parametrize("n,cfg,sigma,temperature", [(5, 2.0, 0.25, 1.0), (16, 2.0, 0.0, 0.0)])
def test_cfm_batch_end_to_end_bound(ming, ctx, flowb, n, cfg, sigma, temperature):
    """Free-running latents of every sequence: finite and within the order-difference bound of
    the MLX-order oracle."""
    print(f"[cfm_batch_end_to_end] n={n}", flush=True)
    g, _, (z, hist, noise, sde), shift = _batch_free_run(ming, ctx, flowb, n, cfg, sigma, temperature)
    oc = flowb[2]
    for b in range(n):
        ref = oracle.cfm_sample(oc, z[b], hist[b], noise[b], sde[b], cfg, shift)[0]
        gf = (g[b].astype(np.uint32) << 16).view(np.float32)
        rf = (ref.astype(np.uint32) << 16).view(np.float32)
        assert np.isfinite(gf).all(), b
        assert_close_bf16(g[b], ref, f"sequence {b} latent (end to end)", atol=6e-2, rtol=2e-2)
        assert float(np.abs(gf - rf).mean()) <= 2e-2, b


@pytest.mark.parametrize("n,cfg,sigma,temperature", [(5, 2.0, 0.25, 1.0), (16, 2.0, 0.0, 0.0)])
def test_cfm_batch_end_to_end_exact(ming, ctx, flowb, n, cfg, sigma, temperature):
    """The ten steps run free on both sides (src/ming_parity.zig:204-235): every step's latent of
    the checked sequences equals the oracle's in the batched kernels' order bit for bit."""
    print(f"[cfm_batch_end_to_end_exact] n={n}", flush=True)
    g, gs, (z, hist, noise, sde), shift = _batch_free_run(ming, ctx, flowb, n, cfg, sigma, temperature)
    od = flowb[3]
    with oracle.dit_order(oracle.DIT_ORDER_MFMA):
        for b in (range(n) if n <= 5 else (0, 5, 10, 15)):
            ref, rsteps = oracle.cfm_sample(od, z[b], hist[b], noise[b], sde[b], cfg, shift)
            for i in range(10):
                assert_bits(gs[b, i], rsteps[i], f"sequence {b} free-running Euler step {i} (batched order)")
            assert_bits(g[b], ref, f"sequence {b} latent")
