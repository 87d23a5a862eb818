"""The oracle's restatement of gfx950's bf16 dot / matrix accumulation (or_acc_step) against the
device itself, on the full seeded probe inputs (tests/golden/arith_inputs.py; the probe kernels
in tests/golden/arith_probe.hip, built by build()): 2.1 M v_dot2c_f32_bf16 results in eight
categories, 4,096 v_mfma_f32_16x16x32_bf16 tiles (1 M outputs) and 65,536 chains of 128 dot2
steps over DiT-like rows, every result bit for bit, at two seeds of each kind."""
import ctypes
import os
import sys

import numpy as np
import pytest
import torch

import oracle

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "golden"))
import arith_inputs as AI  # noqa: E402


@pytest.fixture(scope="module")
def probe():
    path = os.path.join(HERE, "golden", "libarith_probe.so")
    if not os.path.exists(path):
        pytest.fail("tests/golden/libarith_probe.so is not built (run build())")
    return ctypes.CDLL(path)


def P(t):
    return ctypes.c_void_p(t.data_ptr())


def dev(a):
    a = np.ascontiguousarray(a)
    return torch.from_numpy(a.view({2: np.int16, 4: np.int32}[a.itemsize]) if a.dtype != np.float32 else a).cuda()


def same(got, want, what):
    bad = np.nonzero(got.view(np.uint32) != want.view(np.uint32))[0]
    assert bad.size == 0, f"{what}: {bad.size} results differ, first {[(int(i), float(got.flat[i]), float(want.flat[i])) for i in bad[:4]]}"


@pytest.mark.parametrize("seed", [101, 111])
def test_dot2_matches_oracle(probe, seed):
    print(f"[arith] dot2 seed {seed}", flush=True)
    a, b, c = AI.dot2_inputs(seed, 1 << 18)
    d = torch.empty(c.size, dtype=torch.float32, device="cuda")
    assert probe.arith_dot2(P(dev(a)), P(dev(b)), P(dev(c)), P(d), c.size) == 0
    got = d.cpu().numpy()
    want = oracle.dot2_batch(a, b, c)
    n = 1 << 18
    for ci, cat in enumerate(AI.DOT2_CATS):
        same(got[ci * n:(ci + 1) * n], want[ci * n:(ci + 1) * n], f"dot2 {cat}")


@pytest.mark.parametrize("seed", [102, 112])
def test_mfma_matches_oracle(probe, seed):
    print(f"[arith] mfma seed {seed}", flush=True)
    A, B, C = AI.mfma_inputs(seed, 512)
    D = torch.empty(C.shape, dtype=torch.float32, device="cuda")
    assert probe.arith_mfma(P(dev(A)), P(dev(B)), P(dev(C)), P(D), A.shape[0]) == 0
    got = D.cpu().numpy()
    want = oracle.mfma_batch(A, B, C)
    for ci, cat in enumerate(AI.MFMA_CATS):
        same(got[ci * 512:(ci + 1) * 512], want[ci * 512:(ci + 1) * 512], f"mfma {cat}")


def test_chains_match_oracle(probe):
    print("[arith] dot2 chains", flush=True)
    x, w, c0 = AI.chain_inputs(103, 1 << 16, 128)
    d = torch.empty(c0.size, dtype=torch.float32, device="cuda")
    assert probe.arith_chain(P(dev(x)), P(dev(w)), P(dev(c0)), P(d), x.shape[0], x.shape[1]) == 0
    acc = c0
    for j in range(x.shape[1]):
        acc = oracle.dot2_batch(x[:, j], w[:, j], acc)
    same(d.cpu().numpy(), acc, "dot2 chains")
