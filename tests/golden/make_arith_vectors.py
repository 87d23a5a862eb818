"""Writes tests/golden/arith_gfx950.npz: inputs and the device's results of v_dot2c_f32_bf16 and
v_mfma_f32_16x16x32_bf16 on seeded inputs (tests/golden/arith_inputs.py), selected from the full
probe run -- per category the results that no single rounding of the exact sum gives, plus as
many others.  Run on a machine with the GPU, after `make -C tests/golden`:

    python tests/golden/make_arith_vectors.py OUT.npz

The fixture pins the oracle's or_acc_step (tests/test_oracle_arith.py); tests/test_gpu_arith.py
repeats the whole run on the GPU against the oracle."""
import ctypes
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)
import arith_inputs as AI  # noqa: E402

DOT2_SEED, DOT2_N = 101, 1 << 18
MFMA_SEED, MFMA_PER = 102, 512
KEEP_DOT2, KEEP_MFMA = 512, 4


def run_probe():
    import torch

    lib = ctypes.CDLL(os.path.join(HERE, "libarith_probe.so"))
    P = lambda t: ctypes.c_void_p(t.data_ptr())
    a, b, c = AI.dot2_inputs(DOT2_SEED, DOT2_N)
    ta = torch.from_numpy(a.view(np.int32)).cuda()
    tb = torch.from_numpy(b.view(np.int32)).cuda()
    tc = torch.from_numpy(c).cuda()
    td = torch.empty_like(tc)
    assert lib.arith_dot2(P(ta), P(tb), P(tc), P(td), c.size) == 0
    A, B, C = AI.mfma_inputs(MFMA_SEED, MFMA_PER)
    tA, tB = torch.from_numpy(A.view(np.int16)).cuda(), torch.from_numpy(B.view(np.int16)).cuda()
    tC = torch.from_numpy(C).cuda()
    tD = torch.empty_like(tC)
    assert lib.arith_mfma(P(tA), P(tB), P(tC), P(tD), A.shape[0]) == 0
    return (a, b, c, td.cpu().numpy()), (A, B, C, tD.cpu().numpy())


def single_rounding_dot2(a, b, c):
    lo = lambda w: AI.bf16_to_f32((w & 0xFFFF).astype(np.uint16)).astype(np.float64)
    hi = lambda w: AI.bf16_to_f32((w >> 16).astype(np.uint16)).astype(np.float64)
    return (c.astype(np.float64) + (lo(a) * lo(b) + hi(a) * hi(b))).astype(np.float32)


def main(out):
    (a, b, c, d), (A, B, C, D) = run_probe()
    rng = np.random.default_rng(7)
    ref = single_rounding_dot2(a, b, c)
    keep = []
    for ci in range(len(AI.DOT2_CATS)):
        idx = np.arange(ci * DOT2_N, (ci + 1) * DOT2_N)
        hard = idx[ref[idx].view(np.uint32) != d[idx].view(np.uint32)]
        hard = rng.choice(hard, min(KEEP_DOT2, hard.size), replace=False) if hard.size else hard
        other = rng.choice(idx, KEEP_DOT2, replace=False)
        keep.append(np.union1d(hard, other))
    keep = np.concatenate(keep)
    tests = np.concatenate([np.arange(ci * MFMA_PER, ci * MFMA_PER + KEEP_MFMA) for ci in range(len(AI.MFMA_CATS))])
    np.savez_compressed(out, dot2_a=a[keep], dot2_b=b[keep], dot2_c=c[keep], dot2_d=d[keep],
                        dot2_cat=(keep // DOT2_N).astype(np.int8), mfma_a=A[tests], mfma_b=B[tests],
                        mfma_c=C[tests], mfma_d=D[tests], mfma_cat=(tests // MFMA_PER).astype(np.int8))
    print(f"{out}: {keep.size} dot2 tuples, {tests.size} mfma tiles")


if __name__ == "__main__":
    main(sys.argv[1])
