"""Helpers of the VAE decoder parity tests: mirror a SyntheticVae into the
oracle's VaeModel, compare f32 tensors against a stated tolerance."""
import numpy as np

import oracle
from lmkit import oracle_linear


def oracle_vae(syn):
    """oracle.VaeModel from a SyntheticVae's host copies."""
    spec = syn.spec
    c = oracle.vae_cfg(hidden=spec.hidden, heads=spec.heads, kv_heads=spec.kv_heads, head_dim=spec.head_dim,
                       inter=spec.inter, n_layers=spec.n_layers, eps=spec.eps, theta=spec.theta, window=spec.window,
                       latent=spec.latent, patch=spec.patch, n_fft=spec.n_fft, hop=spec.hop)
    D, P = "audio.decoder", "audio.decoder.decoder"
    layers = []
    for i in range(spec.n_layers):
        L = f"{P}.layers.{i}"
        lin = lambda n: oracle_linear(syn.host(f"{L}.{n}"))
        layers.append(oracle.LmLayer(syn.host(f"{L}.input_layernorm.weight"),
                                     syn.host(f"{L}.post_attention_layernorm.weight"), lin("self_attn.q_proj"),
                                     lin("self_attn.k_proj"), lin("self_attn.v_proj"), lin("self_attn.o_proj"),
                                     lin("mlp.gate_proj"), lin("mlp.up_proj"), lin("mlp.down_proj"),
                                     syn.host(f"{L}.self_attn.q_proj.bias"), syn.host(f"{L}.self_attn.k_proj.bias"),
                                     syn.host(f"{L}.self_attn.v_proj.bias")))
    return oracle.VaeModel(c, oracle_linear(syn.host(f"{D}.fc1")), syn.host(f"{D}.fc1.bias"), layers,
                           syn.host(f"{P}.norm.weight"), oracle_linear(syn.host(f"{D}.head.out")),
                           syn.host(f"{D}.head.out.bias"), syn.host(f"{D}.head.istft.window"))


def assert_close_f32(got, ref, what, rel):
    """|got - ref| <= rel * max|ref| (f32 paths: summation order only)."""
    got, ref = np.asarray(got, np.float64), np.asarray(ref, np.float64)
    scale = max(float(np.abs(ref).max()), 1e-30)
    d = np.abs(got - ref)
    assert d.max() <= rel * scale, (f"{what}: max|d| {d.max():.3e} = {d.max() / scale:.2e} of max|ref| {scale:.3e} "
                                    f"at {np.unravel_index(int(d.argmax()), d.shape)}")
    return float(d.max() / scale)
