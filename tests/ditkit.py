"""Helpers of the DiT parity tests: mirror a SyntheticFlow's host copies into
oracle objects (blocks, flow head with the oracle's own load-time tables,
aggregator, stop head)."""
import numpy as np

import oracle

BLOCK_KEYS = (("wq", "attn.to_q"), ("wk", "attn.to_k"), ("wv", "attn.to_v"), ("wo", "attn.to_out.0"),
              ("w1", "mlp.ff.0.0"), ("w2", "mlp.ff.2"))
CFM = "flowloss.cfm.model"
AGG = "linear_proj_audio"


def ocfg(spec):
    return oracle.dit_cfg(spec.hidden, spec.heads, spec.head_dim, spec.ff, spec.eps)


def oblock(syn, prefix, i):
    h = syn.hostw
    b = f"{prefix}.blocks.{i}"
    w = {"norm1": h[f"{b}.norm1.weight"], "norm2": h[f"{b}.norm2.weight"]}
    for k, key in BLOCK_KEYS:
        w[k] = h[f"{b}.{key}.weight"]
        w["b" + k[1:]] = h[f"{b}.{key}.bias"]
    return oracle.DitBlock(w)


def olin(syn, name):
    return oracle.Linear(syn.hostw[name + ".weight"])


def oracle_cfm(syn):
    """The flow head on the oracle, with t_emb / dt / sq from the oracle's own
    schedule and timestep embedding (not the library's tables)."""
    spec, h = syn.spec, syn.hostw
    c = ocfg(spec)
    blocks = [oblock(syn, CFM, i) for i in range(spec.cfm_blocks)]
    t, dt, sq = oracle.flow_schedule()
    m0, m2 = olin(syn, f"{CFM}.t_embedder.time_mlp.0"), olin(syn, f"{CFM}.t_embedder.time_mlp.2")
    te = np.stack([oracle.timestep_embed(m0, h[f"{CFM}.t_embedder.time_mlp.0.bias"], m2,
                                         h[f"{CFM}.t_embedder.time_mlp.2.bias"], t[i]) for i in range(10)])
    cos_t, sin_t = oracle.rotary_table(spec.inv_freq(), 3)
    return oracle.CfmModel(c, blocks, olin(syn, f"{CFM}.x_embedder"), h[f"{CFM}.x_embedder.bias"],
                           olin(syn, f"{CFM}.c_embedder.cond_embedder"), h[f"{CFM}.c_embedder.cond_embedder.bias"],
                           h[f"{CFM}.final_layer.norm_final.weight"], olin(syn, f"{CFM}.final_layer.linear"),
                           h[f"{CFM}.final_layer.linear.bias"], te, dt, sq, cos_t, sin_t)


def oracle_agg(syn):
    spec, h = syn.spec, syn.hostw
    blocks = [oblock(syn, AGG, i) for i in range(spec.agg_blocks)]
    cos_t, sin_t = oracle.rotary_table(spec.inv_freq(), 2)
    return oracle.AggModel(ocfg(spec), blocks, olin(syn, f"{AGG}.x_embedder"), h[f"{AGG}.x_embedder.bias"],
                           h[f"{AGG}.word_embedder.weight"], h[f"{AGG}.final_layer.norm_final.weight"],
                           olin(syn, f"{AGG}.final_layer.linear"), h[f"{AGG}.final_layer.linear.bias"], cos_t,
                           sin_t)


ADA = "adaln"


def oracle_adaln(syn):
    """Config 4's adaLN flow head on the oracle, with its own t_emb / dt / sq."""
    spec, h = syn.spec, syn.hostw
    c = ocfg(spec)
    blocks = [(oblock(syn, ADA, i), olin(syn, f"{ADA}.blocks.{i}.adaLN_modulation.1"),
               h[f"{ADA}.blocks.{i}.adaLN_modulation.1.bias"]) for i in range(spec.cfm_blocks)]
    t, dt, sq = oracle.flow_schedule()
    m0, m2 = olin(syn, f"{ADA}.t_embedder.time_mlp.0"), olin(syn, f"{ADA}.t_embedder.time_mlp.2")
    te = np.stack([oracle.timestep_embed(m0, h[f"{ADA}.t_embedder.time_mlp.0.bias"], m2,
                                         h[f"{ADA}.t_embedder.time_mlp.2.bias"], t[i]) for i in range(10)])
    cos_t, sin_t = oracle.rotary_table(spec.inv_freq(), spec.frames)
    return oracle.AdalnModel(c, blocks, olin(syn, f"{ADA}.x_embedder"), h[f"{ADA}.x_embedder.bias"],
                             olin(syn, f"{ADA}.c_embedder"), h[f"{ADA}.c_embedder.bias"],
                             h[f"{ADA}.final_layer.norm_final.weight"], olin(syn, f"{ADA}.final_layer.linear"),
                             h[f"{ADA}.final_layer.linear.bias"], olin(syn, f"{ADA}.final_layer.adaLN_modulation.1"),
                             h[f"{ADA}.final_layer.adaLN_modulation.1.bias"], te, dt, sq, cos_t, sin_t, spec.frames)
