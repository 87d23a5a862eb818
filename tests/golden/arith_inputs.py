"""Seeded inputs for the arithmetic probe (tests/golden/arith_probe.hip): bf16 pairs and f32
accumulators for v_dot2c_f32_bf16, 16x32 / 32x16 bf16 tiles with 16x16 f32 accumulators for
v_mfma_f32_16x16x32_bf16, and dot-product chains.  numpy's PCG64 stream makes them the same
on every machine, so a test regenerates exactly what the fixture was made from."""
import numpy as np

DOT2_CATS = ("typical", "wide", "dit", "cancel", "acc_dominant", "zeros", "tiny", "cross")
MFMA_CATS = ("typical", "wide", "dit", "zeros", "acc_dominant", "tiny", "cancel", "cross")


def bf16_rand(rng, n, emin, emax):
    """bf16 bit patterns: random sign, exponent uniform in [emin, emax] (unbiased), random mantissa."""
    s = rng.integers(0, 2, n, dtype=np.uint32)
    e = rng.integers(127 + emin, 127 + emax + 1, n).astype(np.uint32)
    m = rng.integers(0, 128, n, dtype=np.uint32)
    return ((s << 15) | (e << 7) | m).astype(np.uint16)


def f32_rand(rng, n, emin, emax):
    s = rng.integers(0, 2, n, dtype=np.uint32)
    e = rng.integers(127 + emin, 127 + emax + 1, n).astype(np.uint32)
    m = rng.integers(0, 1 << 23, n, dtype=np.uint32)
    return ((s << 31) | (e << 23) | m).view(np.float32)


def bf16_normal(rng, n, sd):
    x = (rng.standard_normal(n) * sd).astype(np.float32)
    u = x.view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def bf16_to_f32(h):
    return (np.asarray(h, np.uint16).astype(np.uint32) << 16).view(np.float32)


def _pairs(x):
    x = x.reshape(-1, 2)
    return x[:, 0].astype(np.uint32) | (x[:, 1].astype(np.uint32) << 16)


def _tiny_bf16(rng, n):
    """denormal and smallest-normal bf16 values, with some zeros"""
    s = rng.integers(0, 2, n, dtype=np.uint32)
    e = rng.integers(0, 3, n).astype(np.uint32)
    m = rng.integers(0, 128, n, dtype=np.uint32)
    return ((s << 15) | (e << 7) | m).astype(np.uint16)


def _near_pow2(rng, n, emin, emax):
    """f32 accumulators just above or just below a power of two (random sign): sums with smaller
    products cross the exponent boundary"""
    s = rng.integers(0, 2, n, dtype=np.uint32)
    e = rng.integers(127 + emin, 127 + emax + 1, n).astype(np.uint32)
    t = rng.integers(0, 1 << 12, n, dtype=np.uint32)
    m = np.where(rng.random(n) < 0.5, t, (1 << 23) - 1 - t).astype(np.uint32)
    return ((s << 31) | (e << 23) | m).view(np.float32)


def _below(rng, ec, nprod, dmin, dmax):
    """nprod bf16 (a, b) factor pairs per accumulator whose products lie dmin..dmax binades under
    exponent ec"""
    n = ec.size
    d = rng.integers(dmin, dmax + 1, (n, nprod))
    ea = rng.integers(-4, 5, (n, nprod))
    eb = ec[:, None] - d - ea
    a = ((rng.integers(0, 2, (n, nprod)) << 15) | ((ea + 127) << 7) | rng.integers(0, 128, (n, nprod))).astype(np.uint16)
    b = ((rng.integers(0, 2, (n, nprod)) << 15) | ((eb + 127) << 7) | rng.integers(0, 128, (n, nprod))).astype(np.uint16)
    return a, b


def dot2_inputs(seed, n):
    """n tuples per category (DOT2_CATS order): a, b u32 bf16 pairs (element 0 low), c f32."""
    rng = np.random.default_rng(seed)
    A, B, C = [], [], []
    for cat in DOT2_CATS:
        if cat == "typical":
            a, b, c = bf16_rand(rng, 2 * n, -6, 6), bf16_rand(rng, 2 * n, -6, 6), f32_rand(rng, n, -12, 12)
        elif cat == "wide":
            a, b, c = bf16_rand(rng, 2 * n, -30, 30), bf16_rand(rng, 2 * n, -30, 30), f32_rand(rng, n, -60, 60)
        elif cat == "dit":
            a, b = bf16_normal(rng, 2 * n, 1.0), bf16_normal(rng, 2 * n, 0.03)
            c = (rng.standard_normal(n) * 0.5).astype(np.float32)
        elif cat == "cancel":
            a, b = bf16_rand(rng, 2 * n, -4, 4), bf16_rand(rng, 2 * n, -4, 4)
            p = bf16_to_f32(a).reshape(n, 2).astype(np.float64) * bf16_to_f32(b).reshape(n, 2)
            sel = rng.integers(0, 3, n)
            tgt = np.where(sel == 0, p[:, 0], np.where(sel == 1, p[:, 0] + p[:, 1], p[:, 1]))
            bits = (-tgt).astype(np.float32).view(np.uint32).astype(np.int64) + rng.integers(-64, 65, n)
            c = np.clip(bits, 0, 0xFFFFFFFF).astype(np.uint32).view(np.float32)
            c = np.where(np.isfinite(c), c, np.float32(0)).astype(np.float32)
        elif cat == "acc_dominant":
            a, b = bf16_rand(rng, 2 * n, -6, 6), bf16_rand(rng, 2 * n, -6, 6)
            ef = ((a.astype(np.int32) >> 7) & 0xFF) + ((b.astype(np.int32) >> 7) & 0xFF) - 254
            ep = ef.reshape(n, 2).max(axis=1)
            ec = ep + rng.integers(0, 41, n)
            c = f32_rand(rng, n, 0, 0)
            u = c.view(np.uint32) & np.uint32(0x807FFFFF)
            c = (u | ((ec + 127).astype(np.uint32) << 23)).view(np.float32)
        elif cat == "zeros":
            a, b = bf16_rand(rng, 2 * n, -6, 6), bf16_rand(rng, 2 * n, -6, 6)
            a[rng.random(2 * n) < 0.3] = 0
            b[rng.random(2 * n) < 0.3] = 0x8000
            c = f32_rand(rng, n, -12, 12)
            r = rng.random(n)
            c[r < 0.25] = 0.0
            c[(r >= 0.25) & (r < 0.5)] = -0.0
            # exact cancellation: c = -(p0 + p1) where that is an f32 value
            p = bf16_to_f32(a).reshape(n, 2).astype(np.float64) * bf16_to_f32(b).reshape(n, 2)
            s = p.sum(axis=1)
            ok = (r >= 0.5) & (r < 0.75) & (s.astype(np.float32).astype(np.float64) == s)
            c[ok] = (-s[ok]).astype(np.float32)
        elif cat == "cross":
            c = _near_pow2(rng, n, -10, 10)
            ec = ((c.view(np.uint32) >> 23) & 0xFF).astype(np.int64) - 127
            a, b = _below(rng, ec, 2, 1, 9)
            a, b = a.reshape(-1), b.reshape(-1)
        else:  # tiny
            a, b = _tiny_bf16(rng, 2 * n), bf16_rand(rng, 2 * n, -8, 8)
            swap = rng.random(2 * n) < 0.5
            a, b = np.where(swap, b, a), np.where(swap, a, b)
            c = f32_rand(rng, n, -126, -110)
            r = rng.random(n)
            c[r < 0.3] = (rng.integers(0, 1 << 23, int((r < 0.3).sum()), dtype=np.uint32) |
                          (rng.integers(0, 2, int((r < 0.3).sum()), dtype=np.uint32) << 31)).view(np.float32)
        A.append(_pairs(a))
        B.append(_pairs(b))
        C.append(np.asarray(c, np.float32))
    return np.concatenate(A), np.concatenate(B), np.concatenate(C)


def mfma_inputs(seed, per_cat):
    """per_cat tests per category (MFMA_CATS order): A [t][16][32], B [t][32][16] bf16, C [t][16][16] f32."""
    rng = np.random.default_rng(seed)
    nt = per_cat * len(MFMA_CATS)
    A = np.empty((nt, 16, 32), np.uint16)
    B = np.empty((nt, 32, 16), np.uint16)
    C = np.empty((nt, 16, 16), np.float32)
    for t in range(nt):
        cat = MFMA_CATS[t // per_cat]
        if cat == "typical":
            a, b, c = bf16_rand(rng, 512, -6, 6), bf16_rand(rng, 512, -6, 6), f32_rand(rng, 256, -10, 10)
        elif cat == "wide":
            a, b, c = bf16_rand(rng, 512, -25, 25), bf16_rand(rng, 512, -25, 25), f32_rand(rng, 256, -40, 40)
        elif cat == "dit":
            a, b = bf16_normal(rng, 512, 1.0), bf16_normal(rng, 512, 0.03)
            c = (rng.standard_normal(256) * 0.5).astype(np.float32)
        elif cat == "zeros":
            a, b = bf16_rand(rng, 512, -3, 3), bf16_rand(rng, 512, -3, 3)
            a[rng.random(512) < 0.4] = 0
            c = f32_rand(rng, 256, -4, 4)
            r = rng.random(256)
            c[r < 0.3] = 0.0
            c[(r >= 0.3) & (r < 0.5)] = -0.0
        elif cat == "acc_dominant":
            a, b = bf16_rand(rng, 512, -4, 4), bf16_rand(rng, 512, -4, 4)
            c = f32_rand(rng, 256, 8, 40)
        elif cat == "tiny":
            a, b = _tiny_bf16(rng, 512), bf16_rand(rng, 512, -6, 6)
            c = f32_rand(rng, 256, -126, -115)
        elif cat == "cross":  # one 8-k block (the other k zero): a single step per output
            # row i's accumulators share one exponent e_i; A[i][k] lies 1..9 binades under it and
            # B[k][j] within one binade of 1, so the products land under each accumulator
            e = rng.integers(-10, 11, 16)
            c = _near_pow2(rng, 256, 0, 0).reshape(16, 16)
            u = (c.view(np.uint32) & np.uint32(0x807FFFFF)) | ((e[:, None] + 127).astype(np.uint32) << 23)
            ea = e[:, None] - rng.integers(1, 10, (16, 8))
            A[t] = 0
            B[t] = 0
            A[t, :, :8] = ((rng.integers(0, 2, (16, 8)) << 15) | ((ea + 127) << 7) | rng.integers(0, 128, (16, 8)))
            B[t, :8, :] = ((rng.integers(0, 2, (8, 16)) << 15) | ((rng.integers(-1, 2, (8, 16)) + 127) << 7)
                           | rng.integers(0, 128, (8, 16)))
            C[t] = u.view(np.float32)
            continue
        else:  # cancel: C = -(A B) rounded, perturbed
            a, b = bf16_rand(rng, 512, -3, 3), bf16_rand(rng, 512, -3, 3)
            ab = bf16_to_f32(a).reshape(16, 32).astype(np.float64) @ bf16_to_f32(b).reshape(32, 16)
            bits = (-ab).astype(np.float32).reshape(-1).view(np.uint32).astype(np.int64) + rng.integers(-512, 513, 256)
            c = np.clip(bits, 0, 0xFFFFFFFF).astype(np.uint32).view(np.float32)
            c = np.where(np.isfinite(c), c, np.float32(0)).astype(np.float32)
        A[t] = a.reshape(16, 32)
        B[t] = b.reshape(32, 16)
        C[t] = np.asarray(c, np.float32).reshape(16, 16)
    return A, B, C


def chain_inputs(seed, n, length):
    """n dot-product chains of `length` dot2 steps over DiT-like rows (x ~ N(0, 1), w ~ N(0, 0.02)),
    accumulators starting at 0."""
    rng = np.random.default_rng(seed)
    x = _pairs(bf16_normal(rng, 2 * n * length, 1.0)).reshape(n, length)
    w = _pairs(bf16_normal(rng, 2 * n * length, 0.02)).reshape(n, length)
    return x, w, np.zeros(n, np.float32)
