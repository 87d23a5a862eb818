"""Pins the oracle's bf16 rounding and the synthetic-input generator.

- or_bf16 (round to nearest even) against torch's f32 -> bf16 conversion on
  random values of every magnitude, exact ties, signed zeros, infinities,
  subnormals and NaN.
- ming_synth_normal_bf16 against an independent numpy restatement of its
  published algorithm (splitmix64 counter + Box-Muller), bit for bit, and
  its slice and thread-count independence.
"""
import numpy as np
import torch

import oracle


def torch_bf16(x):
    return torch.from_numpy(np.asarray(x, np.float32)).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)


def test_bf16_matches_torch_random():
    rng = np.random.default_rng(0)
    x = np.concatenate([
        rng.normal(0, 1, 200000), rng.normal(0, 1e-3, 50000), rng.normal(0, 1e4, 50000),
        rng.uniform(-1e-38, 1e-38, 20000), rng.uniform(-3e38, 3e38, 20000)]).astype(np.float32)
    assert np.array_equal(oracle.to_bf16(x), torch_bf16(x))


def test_bf16_ties_and_specials():
    bits = np.array([0x3F808000, 0x3F818000, 0xBF808000, 0x3F80FFFF, 0x3F807FFF, 0x00000001, 0x80000001,
                     0x007FFFFF, 0x7F7FFFFF, 0x7F800000, 0xFF800000, 0x00000000, 0x80000000], np.uint32)
    x = bits.view(np.float32)
    got = oracle.to_bf16(x)
    assert np.array_equal(got, torch_bf16(x))
    assert got[0] == 0x3F80 and got[1] == 0x3F82  # ties to even
    nan = oracle.to_bf16(np.array([np.nan], np.float32))[0]
    assert (nan & 0x7F80) == 0x7F80 and (nan & 0x007F) != 0


def test_f32_of_bf16_exact():
    h = np.arange(0, 65536, dtype=np.uint32).astype(np.uint16)
    f = oracle.to_f32(h)
    finite = np.isfinite(f)
    assert np.array_equal(oracle.to_bf16(f[finite]), h[finite])


# ---- synthetic generator: independent numpy restatement ----

M64 = np.uint64(0xFFFFFFFFFFFFFFFF)


def _mix(z):
    z = np.asarray(z, np.uint64)
    with np.errstate(over="ignore"):
        z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
        z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
    return z ^ (z >> np.uint64(31))


def _stream(seed, name):
    h = 0xcbf29ce484222325
    for ch in name.encode():
        h ^= ch
        h = (h * 0x100000001b3) & 0xFFFFFFFFFFFFFFFF
    return int(_mix(np.uint64(seed ^ h)))


def np_normal_bf16(seed, name, n, mean, std):
    key = np.uint64(_stream(seed, name))
    i = np.arange(n, dtype=np.uint64)
    p = i // np.uint64(2)
    with np.errstate(over="ignore"):
        c1 = key + (np.uint64(2) * p + np.uint64(1)) * np.uint64(0x9E3779B97F4A7C15)
        c2 = key + (np.uint64(2) * p + np.uint64(2)) * np.uint64(0x9E3779B97F4A7C15)
    u1 = ((_mix(c1) >> np.uint64(11)).astype(np.float64) + 0.5) * (1.0 / 9007199254740992.0)
    u2 = ((_mix(c2) >> np.uint64(11)).astype(np.float64) + 0.5) * (1.0 / 9007199254740992.0)
    r = np.sqrt(-2.0 * np.log(u1))
    t = 2.0 * np.pi * u2
    z = np.where(i % np.uint64(2) == 0, r * np.cos(t), r * np.sin(t))
    v = (np.float64(np.float32(mean)) + np.float64(np.float32(std)) * z).astype(np.float32)
    return torch_bf16(v)


def test_synth_matches_numpy_restatement(ming):
    for seed, name, mean, std in [(0, "model.model.embed_tokens.weight", 0.0, 0.02), (7, "kv.k", 0.0, 1.0),
                                  (3, "x", 1.0, 0.1)]:
        got = ming.synth_normal_bf16(seed, name, 20001, mean, std, threads=1)
        ref = np_normal_bf16(seed, name, 20001, mean, std)
        # libm and numpy may differ in the last bit of a double; that can move a
        # bf16 rounding only at an exact tie, which is vanishingly rare
        assert (got != ref).sum() <= 2


def test_synth_slices_and_threads(ming):
    a = ming.synth_normal_bf16(1, "w", 300001, 0.0, 0.02, threads=1)
    b = ming.synth_normal_bf16(1, "w", 300001, 0.0, 0.02, threads=7)
    c = ming.synth_normal_bf16(1, "w", 1000, 0.0, 0.02, threads=1)
    assert np.array_equal(a, b) and np.array_equal(a[:1000], c)
    assert not np.array_equal(a[:1000], ming.synth_normal_bf16(2, "w", 1000, 0.0, 0.02))
    f = oracle.to_f32(a).astype(np.float64)
    assert abs(f.mean()) < 1e-3 and abs(f.std() - 0.02) < 1e-3


def test_synth_uniform(ming):
    ids = ming.synth_uniform_i32(0, "prompt", 100000, 151936)
    assert ids.min() >= 0 and ids.max() < 151936
    assert abs(ids.mean() / 151936 - 0.5) < 0.01
