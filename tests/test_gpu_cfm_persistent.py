"""The persistent flow head (one launch per ming_cfm_sample) against the
launch path (MING_CFM_KERNELS, about 42 launches per Euler step, itself held
to the oracle teacher-forced per step in test_gpu_dit.py): every Euler
step's latent bit-identical, for several inputs and CFG / SDE settings, over
repeated and interleaved launches (each launch tags its hand-offs with a
new epoch), at 1, 2, 8 and 16 blocks, plus the stage-stamp profile, the mode checks and AUTO's choice
of the persistent kernel at the reference shape."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

STEPS = 10


def syn_mod():
    import importlib

    return importlib.import_module("ming-tts-serve_amd.synthetic")


def dev_u16(a):
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).cuda().view(torch.bfloat16)


def host_u16(t):
    return t.view(torch.int16).cpu().numpy().view(np.uint16)


@pytest.fixture(scope="module")
def flow(ming, ctx):
    S = syn_mod()
    print("[cfmp] building the 8-block flow head (hidden 1024, ff 4096)", flush=True)
    return S.SyntheticFlow(ctx, S.MING_DIT, seed=21, norm_std=0.05, parts=("cfm",))


def inputs(ming, spec, seed):
    lat, H = spec.latent, spec.lm_hidden
    return (dev_u16(ming.synth_normal_bf16(seed, "cfmp.z", H)),
            dev_u16(ming.synth_normal_bf16(seed, "cfmp.hist", lat)),
            dev_u16(ming.synth_normal_bf16(seed, "cfmp.noise", lat)),
            dev_u16(ming.synth_normal_bf16(seed, "cfmp.sde", STEPS * lat).reshape(STEPS, lat)))


def run(ctx, m, mode, x, cfg, sigma, temperature):
    lat = x[2].shape[0]
    m.set_mode(mode)
    out = torch.empty(lat, dtype=torch.bfloat16, device="cuda")
    steps = torch.empty((STEPS, lat), dtype=torch.bfloat16, device="cuda")
    m.sample(*x, cfg, sigma, temperature, out, steps)
    ctx.sync()
    return host_u16(out), host_u16(steps)


def same(ref, got, what):
    ok = np.array_equal(ref, got)
    if not ok:
        bad = np.argwhere(ref != got)
        s, c = bad[0]
        raise AssertionError(f"{what}: {len(bad)} latent values differ, first at Euler step {s} channel {c} "
                             f"({ref[s, c]:#06x} vs {got[s, c]:#06x})")


@pytest.mark.parametrize("seed,cfg,sigma,temperature", [(71, 2.0, 0.25, 1.0), (72, 2.0, 0.25, 0.0), (73, 1.5, 0.5, 0.5),
                                                        (74, 3.0, 0.0, 1.0)])
def test_persistent_equals_kernels(ming, ctx, flow, seed, cfg, sigma, temperature):
    print(f"[cfmp] seed {seed} cfg {cfg} sigma {sigma} temperature {temperature}", flush=True)
    m = flow.cfm_model()
    x = inputs(ming, flow.spec, seed)
    ko, ks = run(ctx, m, ming.CFM_KERNELS, x, cfg, sigma, temperature)
    po, ps = run(ctx, m, ming.CFM_PERSISTENT, x, cfg, sigma, temperature)
    same(ks, ps, "persistent vs kernels")
    assert np.array_equal(po, ps[STEPS - 1]) and np.array_equal(ko, po), "latent_out is the last step"
    _, as_ = run(ctx, m, ming.CFM_AUTO, x, cfg, sigma, temperature)
    same(ks, as_, "auto vs kernels")
    m.close()


@pytest.mark.parametrize("nblk", [1, 2, 16])
def test_persistent_block_counts(ming, ctx, nblk):
    """AUTO sends every reference-width flow head of 1..16 blocks to the persistent kernel: at 1
    block (the head publishes image A and reads the last block's output in the same step), 2 and
    16 (a full block table and flag range) its latents equal the launch path's bit for bit, and
    AUTO's too."""
    S = syn_mod()
    print(f"[cfmp] {nblk} blocks", flush=True)
    syn = S.SyntheticFlow(ctx, S.DitSpec(cfm_blocks=nblk), seed=90 + nblk, norm_std=0.05, parts=("cfm",))
    m = syn.cfm_model()
    for seed in (91, 92):
        x = inputs(ming, syn.spec, seed)
        ko, ks = run(ctx, m, ming.CFM_KERNELS, x, 2.0, 0.25, 1.0)
        po, ps = run(ctx, m, ming.CFM_PERSISTENT, x, 2.0, 0.25, 1.0)
        same(ks, ps, f"{nblk} blocks: persistent vs kernels")
        _, as_ = run(ctx, m, ming.CFM_AUTO, x, 2.0, 0.25, 1.0)
        same(ks, as_, f"{nblk} blocks: auto vs kernels")
    m.close()
    del syn


def test_persistent_repeated_and_interleaved(ming, ctx, flow):
    """Launch after launch (new epochs over the same hand-off buffers), with
    kernel-path samples of other inputs in between, and without y_steps."""
    m = flow.cfm_model()
    xs = [inputs(ming, flow.spec, 80 + i) for i in range(3)]
    ref = [run(ctx, m, ming.CFM_KERNELS, x, 2.0, 0.25, 1.0) for x in xs]
    for rep in range(4):
        for i, x in enumerate(xs):
            o, s = run(ctx, m, ming.CFM_PERSISTENT, x, 2.0, 0.25, 1.0)
            same(ref[i][1], s, f"repeat {rep} input {i}")
            if i == 1:
                run(ctx, m, ming.CFM_KERNELS, xs[2], 2.0, 0.25, 1.0)
    m.set_mode(ming.CFM_PERSISTENT)
    out = torch.empty(flow.spec.latent, dtype=torch.bfloat16, device="cuda")
    m.sample(*xs[0], 2.0, 0.25, 1.0, out)
    ctx.sync()
    assert np.array_equal(host_u16(out), ref[0][0]), "latent_out without y_steps"
    m.close()


def test_persistent_profile(ming, ctx, flow):
    """Stage stamps of the first worker: it receives its slice's inputs only
    after it issued its own outputs of the stage before, publishes its slice
    after that, holds each image after publishing its own slice of it, issues
    its outputs after that, and the final layer of step s ends after the last
    image of step s."""
    nb = flow.spec.cfm_blocks
    nflag = STEPS * nb * 4
    m = flow.cfm_model()
    x = inputs(ming, flow.spec, 75)
    stamps = torch.zeros((6, nflag), dtype=torch.int64, device="cuda")
    m.profile(stamps)
    run(ctx, m, ming.CFM_PERSISTENT, x, 2.0, 0.25, 1.0)
    m.profile(None)
    st = stamps.cpu().numpy()
    pub, got, sent, recvd, last = st[0], st[1], st[2], st[3], st[5]
    own = np.ones(nflag, bool)
    own[[s * nb * 4 for s in range(STEPS)]] = False  # each step's first rms1 image comes from the heads
    assert (got > 0).all() and (sent > 0).all() and (last > 0).all(), "every image received, every stage issued"
    assert (pub[own] > 0).all() and (recvd[own] > 0).all(), "every owned slice received and published"
    assert (np.diff(got) > 0).all(), "the images arrive in order"
    assert (got[own] >= pub[own]).all(), "no worker holds an image before its own slice of it is out"
    assert (pub[own] >= recvd[own]).all() and (sent >= got).all(), "slice published after its inputs; outputs after the image"
    idx = np.nonzero(own)[0]
    assert (recvd[idx] >= sent[idx - 1]).all(), "a slice's inputs arrive after the worker issued its own share"
    fin = st[4, :STEPS]
    for s in range(STEPS):
        assert fin[s] > got[(s * nb + nb - 1) * 4 + 3], f"final layer of step {s} after its last image"
    ticks = (fin[STEPS - 1] - got[0]) / 100.0  # wall_clock64 runs at 100 MHz
    print(f"[cfmp] first image to last final layer: {ticks:.1f} us", flush=True)
    m.close()


def test_persistent_mode_checks(ming, ctx, flow):
    m = flow.cfm_model()
    with pytest.raises(ming.MingError) as e:
        m.set_mode(7)
    assert e.value.status == ming.MING_E_ARG
    m.close()
    S = syn_mod()
    small = S.DitSpec(hidden=128, heads=2, head_dim=64, ff=256, cfm_blocks=2, agg_blocks=1)
    f2 = S.SyntheticFlow(ctx, small, seed=3, parts=("cfm",))
    m2 = f2.cfm_model()
    with pytest.raises(ming.MingError) as e:
        m2.set_mode(ming.CFM_PERSISTENT)
    assert e.value.status == ming.MING_E_UNSUPPORTED
    m2.set_mode(ming.CFM_AUTO)  # the launch path serves this shape
    x = inputs(ming, small, 76)
    ko, _ = run(ctx, m2, ming.CFM_KERNELS, x, 2.0, 0.25, 1.0)
    ao, _ = run(ctx, m2, ming.CFM_AUTO, x, 2.0, 0.25, 1.0)
    assert np.array_equal(ko, ao)
    m2.close()


def test_persistent_timing(ming, ctx, flow):
    """Informational: host wall time per sample on each path (20 samples queued, then one sync)."""
    import time

    m = flow.cfm_model()
    x = inputs(ming, flow.spec, 77)
    out = torch.empty(flow.spec.latent, dtype=torch.bfloat16, device="cuda")
    res = {}
    for name, mode in (("kernels", ming.CFM_KERNELS), ("persistent", ming.CFM_PERSISTENT)):
        m.set_mode(mode)
        for _ in range(3):
            m.sample(*x, 2.0, 0.25, 1.0, out)
        ctx.sync()
        t0 = time.perf_counter()
        for _ in range(20):
            m.sample(*x, 2.0, 0.25, 1.0, out)
        ctx.sync()
        res[name] = (time.perf_counter() - t0) * 1e3 / 20
    print(f"[cfmp] ms per sample: kernels {res['kernels']:.3f}, persistent {res['persistent']:.3f}", flush=True)
    m.close()


def test_auto_runs_the_persistent_kernel_at_reference_shape(ming, ctx, flow):
    """MING_CFM_AUTO takes the persistent kernel where it fits: only that
    kernel writes the stage stamps, and its latents equal the launch path's."""
    nflag = STEPS * flow.spec.cfm_blocks * 4
    m = flow.cfm_model()
    x = inputs(ming, flow.spec, 78)
    ko, ks = run(ctx, m, ming.CFM_KERNELS, x, 2.0, 0.25, 1.0)
    stamps = torch.zeros((6, nflag), dtype=torch.int64, device="cuda")
    m.profile(stamps)
    ao, as_ = run(ctx, m, ming.CFM_AUTO, x, 2.0, 0.25, 1.0)
    m.profile(None)
    assert (stamps[1].cpu().numpy() > 0).all(), "AUTO ran the launch path at the reference shape"
    same(ks, as_, "auto vs kernels")
    m.close()
