"""Helpers shared by the decode parity tests: mirror a synthetic device model
into oracle objects, compare bf16 tensors with the stated tolerance."""
import numpy as np

import oracle

# Tolerance for bf16 floating-point outputs: |gpu - ref| <= ATOL + RTOL * |ref|
ATOL = 2e-2
RTOL = 1e-2


def f32(u16):
    return oracle.to_f32(np.asarray(u16, dtype=np.uint16))


def assert_close_bf16(got_u16, ref_u16, what, atol=ATOL, rtol=RTOL):
    g, r = f32(got_u16).astype(np.float64), f32(ref_u16).astype(np.float64)
    d = np.abs(g - r)
    bad = d > atol + rtol * np.abs(r)
    assert not bad.any(), (f"{what}: {bad.sum()} of {bad.size} outside tol; max|d| {d.max():.3e} at "
                           f"{int(d.argmax())} (ref {r.flat[d.argmax()]:.4f}, got {g.flat[d.argmax()]:.4f})")
    return float(d.max())


def assert_bits(got_u16, ref_u16, what):
    """Bit-for-bit equality of two bf16 arrays, naming the first difference."""
    g = np.ascontiguousarray(got_u16, np.uint16).reshape(-1)
    r = np.ascontiguousarray(ref_u16, np.uint16).reshape(-1)
    assert g.shape == r.shape, (what, g.shape, r.shape)
    bad = np.flatnonzero(g != r)
    assert bad.size == 0, (f"{what}: {bad.size} of {g.size} differ in bits; first at {bad[0]}: "
                           f"{int(g[bad[0]]):#06x} ({float(f32(g[bad[0]:bad[0] + 1])[0]):.6g}) vs {int(r[bad[0]]):#06x} "
                           f"({float(f32(r[bad[0]:bad[0] + 1])[0]):.6g})")


def oracle_linear(host):
    if "s" in host:
        return oracle.Linear(host["w"], host["s"], host["b"])
    return oracle.Linear(host["w"])


def oracle_model(syn):
    """(cfg, [LmLayer], final_norm, head Linear) from a SyntheticLm's host copies."""
    spec = syn.spec
    cfg = oracle.cfg(spec.hidden, spec.heads, spec.kv_heads, spec.head_dim, spec.inter, spec.eps,
                     log2_theta=float(np.log2(np.float32(spec.theta))))
    P = "model.model"
    layers = []
    for i in range(spec.n_layers):
        L = f"{P}.layers.{i}"
        lin = lambda n: oracle_linear(syn.host(f"{L}.{n}"))
        layers.append(oracle.LmLayer(
            syn.host(f"{L}.input_layernorm.weight"), syn.host(f"{L}.post_attention_layernorm.weight"),
            lin("self_attn.q_proj"), lin("self_attn.k_proj"), lin("self_attn.v_proj"), lin("self_attn.o_proj"),
            lin("mlp.gate_proj"), lin("mlp.up_proj"), lin("mlp.down_proj"),
            syn.host(f"{L}.self_attn.q_proj.bias"), syn.host(f"{L}.self_attn.k_proj.bias"),
            syn.host(f"{L}.self_attn.v_proj.bias")))
    head = oracle_linear(syn.host(f"{P}.embed_tokens"))
    return cfg, layers, syn.host(f"{P}.norm.weight"), head


def oracle_step(cfg, layers, norm, head, x, pos, kc, vc):
    """One full decode step on the oracle; kc/vc [L][kvh][cap][hd] updated in place.
    Returns (argmax, hidden, logits f32, margin, per-layer outputs)."""
    xs = [x]
    for i, lay in enumerate(layers):
        k_l, v_l = kc[i], vc[i]
        x = oracle.lm_layer_step(cfg, lay, x, pos, k_l, v_l)
        xs.append(x)
    am, hid, lg, _, margin = oracle.lm_head(cfg, norm, head, x)
    return am, hid, lg, margin, xs
