"""Pins of the VAE decoder's oracle (oracle/oracle_vae.c; Model.vaeDecode,
src/ming_model.zig:1257-1340, QStack.forward with the sliding mask, :566-636).

No reference vectors exist for this path (the reference's parity tool reads
external Python MLX dumps that are not in the tree, src/ming_parity.zig:200),
so each function is pinned by a library routine, a closed form or an
independent float64 construction:
  upsample ........ torch interpolate(mode="linear", align_corners=False)
  ISTFT ........... numpy.fft.irfft per frame, and perfect reconstruction of a
                    signal from its own windowed STFT (any trim, overlap-add part
                    or envelope mistake breaks it)
  window attention  plain causal softmax when the window covers every row; the
                    own row exactly when the window is 1; a float64 band mask
  rope / rms / f32 linears / a whole layer: float64 torch compositions."""
import numpy as np
import pytest
import torch

import oracle


def rng(seed):
    return np.random.default_rng(seed)


def bf16(x):
    return oracle.to_bf16(np.asarray(x, np.float32))


def f32(h):
    return oracle.to_f32(h)


def test_upsample_matches_torch_interpolate():
    for T, C, scale in ((1, 3, 4), (7, 5, 4), (13, 8, 3), (2, 4, 2)):
        x = bf16(rng(T * 10 + C).standard_normal((T, C)))
        got = oracle.linear_upsample(x, scale)
        ref = torch.nn.functional.interpolate(torch.from_numpy(f32(x).astype(np.float64)).T[None], scale_factor=scale,
                                              mode="linear", align_corners=False)[0].T.numpy()
        assert got.shape == (T * scale, C)
        np.testing.assert_allclose(got, ref, rtol=0, atol=2e-6 * max(1.0, np.abs(ref).max()))


def stft_params(n_fft):
    k = np.arange(n_fft)
    return (0.5 - 0.5 * np.cos(2 * np.pi * k / n_fft)).astype(np.float32)  # periodic Hann


@pytest.mark.parametrize("n_fft", [16, 64, 3528])
def test_istft_frames_match_numpy_irfft(n_fft):
    hop = n_fft // 4
    F = 3
    r = rng(n_fft)
    nb = n_fft // 2 + 1
    logmag = (r.standard_normal((F, nb)) * 0.7).astype(np.float32)
    logmag[0, 3] = 6.0  # past log(100): clamped
    phase = r.uniform(-np.pi, np.pi, (F, nb)).astype(np.float32)
    p = np.concatenate([logmag, phase], axis=1)
    win = np.ones(n_fft, np.float32)
    _, frames = oracle.vae_istft(p, n_fft, hop, win, frames=True)
    mag = np.minimum(np.exp(logmag.astype(np.float64)), 100.0)
    ref = np.fft.irfft(mag * np.exp(1j * phase.astype(np.float64)), n=n_fft, axis=1)
    np.testing.assert_allclose(frames, ref, rtol=0, atol=2e-6 * np.abs(ref).max())


@pytest.mark.parametrize("n_fft,F", [(64, 9), (256, 5), (3528, 4)])
def test_istft_reconstructs_its_own_stft(n_fft, F):
    hop, pad = n_fft // 4, (n_fft - n_fft // 4) // 2
    win = stft_params(n_fft)
    r = rng(F + n_fft)
    n = F * hop + n_fft
    x = (r.standard_normal(n) * 0.05).astype(np.float64)
    frames = np.zeros((F, n_fft))
    for t in range(F):
        for j in range(n_fft):
            s = t * hop - pad + j
            frames[t, j] = x[s] if 0 <= s < n else 0.0
    X = np.fft.rfft(frames * win.astype(np.float64), axis=1)
    p = np.concatenate([np.log(np.abs(X)), np.angle(X)], axis=1).astype(np.float32)
    wave = oracle.vae_istft(p, n_fft, hop, win)
    assert wave.shape == (F * hop,)
    np.testing.assert_allclose(wave, x[: F * hop], rtol=0, atol=3e-5 * np.abs(x).max())


def torch_band_attention(q, k, v, window):
    q, k, v = (torch.from_numpy(a.astype(np.float64)) for a in (q, k, v))
    F, heads, hd = q.shape
    grp = heads // k.shape[1]
    k = k.repeat_interleave(grp, dim=1)
    v = v.repeat_interleave(grp, dim=1)
    s = torch.einsum("ihd,jhd->hij", q, k) / np.sqrt(hd)
    i = torch.arange(F)[:, None]
    j = torch.arange(F)[None, :]
    ok = (j <= i) & (j > i - window)
    s = s.masked_fill(~ok, float("-inf"))
    return torch.einsum("hij,jhd->ihd", torch.softmax(s, dim=-1), v).numpy()


@pytest.mark.parametrize("window", [1, 3, 8, 64])
def test_window_attention(window):
    r = rng(window)
    F, heads, kvh, hd = 20, 4, 2, 16
    q = r.standard_normal((F, heads, hd)).astype(np.float32)
    k = r.standard_normal((F, kvh, hd)).astype(np.float32)
    v = r.standard_normal((F, kvh, hd)).astype(np.float32)
    got = oracle.window_attention(q, k, v, window)
    np.testing.assert_allclose(got, torch_band_attention(q, k, v, window), rtol=0, atol=2e-6)
    if window == 1:  # each row sees itself only
        assert np.array_equal(got, np.repeat(v, heads // kvh, axis=1))


def test_rope_f32_rotates_pairs():
    r = rng(5)
    hd, log2b = 64, float(np.log2(np.float32(1e6)))
    x = r.standard_normal((3, hd)).astype(np.float32)
    assert np.array_equal(oracle.rope_f32(x, 0, log2b), x)
    for pos in (1, 17, 1000):
        got = oracle.rope_f32(x, pos, log2b)
        half = hd // 2
        inv = 2.0 ** (-(np.arange(half) / half) * log2b)
        z = (x[:, :half] + 1j * x[:, half:]).astype(np.complex128) * np.exp(1j * pos * inv)
        ref = np.concatenate([z.real, z.imag], axis=1)
        # the angle pos * inv_freq is an f32 product, as in MLX: its rounding (pos * 2^-24
        # relative) bounds the difference; a wrong pair or sign is off by O(|x|)
        np.testing.assert_allclose(got, ref, rtol=0, atol=np.abs(x).max() * (3e-7 + pos * 2.0 ** -22))


def test_rms_and_linear_f32():
    r = rng(6)
    x = r.standard_normal((5, 128)).astype(np.float32)
    w = bf16(1 + 0.1 * r.standard_normal(128))
    ref = x.astype(np.float64) / np.sqrt((x.astype(np.float64) ** 2).mean(1, keepdims=True) + 1e-6) * f32(w)
    np.testing.assert_allclose(oracle.rms_f32(x, w), ref, rtol=2e-6, atol=1e-6)
    wb = bf16(0.05 * r.standard_normal((48, 128)))
    bias = bf16(0.1 * r.standard_normal(48))
    Lb = oracle.Linear(wb)
    ref = x.astype(np.float64) @ f32(wb).astype(np.float64).T + f32(bias)
    np.testing.assert_allclose(oracle.linear_f32(Lb, x, bias), ref, rtol=0, atol=2e-5)
    wq, s, b = oracle.quantize(wb)
    La = oracle.Linear(wq, s, b)
    deq = f32(s).repeat(64, 1) * ((wq[:, :, None] >> (4 * np.arange(8))) & 15).reshape(48, 128) + f32(b).repeat(64, 1)
    ref = x.astype(np.float64) @ deq.astype(np.float64).T
    np.testing.assert_allclose(oracle.linear_f32(La, x), ref, rtol=0, atol=2e-5)


def small_layer(seed, H=64, heads=4, kvh=2, hd=16, I=96):
    r = rng(seed)
    lin = lambda n, k: oracle.Linear(bf16(r.standard_normal((n, k)) * 0.1))
    kvd = kvh * hd
    L = oracle.LmLayer(bf16(1 + 0.1 * r.standard_normal(H)), bf16(1 + 0.1 * r.standard_normal(H)), lin(H, H),
                       lin(kvd, H), lin(kvd, H), lin(H, H), lin(I, H), lin(I, H), lin(H, I),
                       bf16(0.1 * r.standard_normal(H)), bf16(0.1 * r.standard_normal(kvd)),
                       bf16(0.1 * r.standard_normal(kvd)))
    c = oracle.vae_cfg(hidden=H, heads=heads, kv_heads=kvh, head_dim=hd, inter=I, n_layers=1, window=5)
    return c, L


def test_vae_layer_matches_float64_composition():
    c, L = small_layer(7)
    F = 12
    x = rng(8).standard_normal((F, c.hidden)).astype(np.float32)
    got, tr = oracle.vae_layer(c, L, x, trace=True)
    d = lambda a: torch.from_numpy(np.asarray(a, np.float64))
    W = {n: d(f32(L.lin[n].w)) for n in L.lin}
    ln1, ln2, bq, bk, bv = (d(f32(a)) for a in L.keep)
    xt = d(x)
    rms = lambda v, w: v / torch.sqrt((v * v).mean(-1, keepdim=True) + 1e-6) * w
    h = rms(xt, ln1)
    q, k, v = h @ W["q"].T + bq, h @ W["k"].T + bk, h @ W["v"].T + bv
    hd, half = c.head_dim, c.head_dim // 2
    inv = 2.0 ** (-(np.arange(half) / half) * c.log2_theta)

    def rot(t, nh):
        t = t.reshape(F, nh, hd)
        ang = torch.from_numpy(np.arange(F)[:, None] * inv[None, :])[:, None, :]
        a, b = t[..., :half], t[..., half:]
        return torch.cat([a * torch.cos(ang) - b * torch.sin(ang), a * torch.sin(ang) + b * torch.cos(ang)], -1)

    qr, kr = rot(q, c.heads), rot(k, c.kv_heads)
    att = torch_band_attention(qr.numpy(), kr.numpy(), v.reshape(F, c.kv_heads, hd).numpy(), c.window)
    x1 = xt + d(att.reshape(F, c.hidden)) @ W["o"].T
    h2 = rms(x1, ln2)
    g, u = h2 @ W["gate"].T, h2 @ W["up"].T
    out = x1 + (g * torch.sigmoid(g) * u) @ W["down"].T
    np.testing.assert_allclose(tr["x1"], x1.numpy(), rtol=0, atol=5e-5)
    np.testing.assert_allclose(got, out.numpy(), rtol=0, atol=1e-4)


def test_vae_decode_composes_its_stages():
    c, L = small_layer(9)
    c.n_layers, c.latent, c.patch, c.n_fft, c.hop = 2, 8, 4, 64, 16
    L2 = small_layer(10)[1]
    r = rng(11)
    fc1 = oracle.Linear(bf16(r.standard_normal((c.hidden, c.latent)) * 0.2))
    fb = bf16(0.1 * r.standard_normal(c.hidden))
    head = oracle.Linear(bf16(r.standard_normal((c.n_fft + 2, c.hidden)) * 0.05))
    hb = bf16(0.1 * r.standard_normal(c.n_fft + 2))
    norm = bf16(1 + 0.1 * r.standard_normal(c.hidden))
    win = stft_params(c.n_fft)
    m = oracle.VaeModel(c, fc1, fb, [L, L2], norm, head, hb, win)
    T = 6
    lat = bf16(r.standard_normal((T, c.latent)))
    wave, xs, ho = oracle.vae_decode(m, lat, trace=True)
    assert wave.shape == (T * c.patch * c.hop,)
    x0 = oracle.linear_upsample(oracle.linear(fc1, lat, fb), c.patch)
    assert np.array_equal(xs[0], x0)
    x1 = oracle.vae_layer(c, L, x0)
    assert np.array_equal(xs[1], x1)
    x2 = oracle.vae_layer(c, L2, x1)
    assert np.array_equal(xs[2], x2)
    p = oracle.linear_f32(head, oracle.rms_f32(x2, norm), hb)
    assert np.array_equal(ho, p)
    assert np.array_equal(wave, oracle.vae_istft(p, c.n_fft, c.hop, win))
