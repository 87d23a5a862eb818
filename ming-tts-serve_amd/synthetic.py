"""Synthetic random-init Qwen2 decode stacks for benches and tests.

Weights are bf16(N(0, std)) from the library's counter-based generator
(ming_synth_normal_bf16), one stream per tensor name (seed, name), with the
reference checkpoint's key names (src/ming_model.zig:550-561, :938).  RMSNorm
weights are 1.0 + N(0, norm_std) (1.0 exactly when norm_std == 0, the
HF init).  With quant=True every linear is quantized on the GPU to MLX affine
4-bit / group 64 (ming_quantize); the embedding table doubles as the tied LM
head (Qwen2-0.5B convention).
"""
import ctypes
import math
from dataclasses import dataclass

import numpy as np

from . import (Context, Kv, KvPages, Linear, LmCfg, LmLayerW, LmModel, VaeCfg, VaeModel, VaeW, W_AFFINE, W_BF16,
               linear, synth_normal_bf16)


@dataclass
class LmSpec:
    hidden: int = 896
    heads: int = 14
    kv_heads: int = 2
    head_dim: int = 64
    inter: int = 4864
    vocab: int = 151936
    n_layers: int = 24
    eps: float = 1e-6
    theta: float = 1e6

    @property
    def kvd(self):
        return self.kv_heads * self.head_dim

    def cfg(self):
        return LmCfg(self.hidden, self.heads, self.kv_heads, self.head_dim, self.inter, self.vocab, self.n_layers,
                     self.eps, float(np.log2(np.float32(self.theta))))

    def weight_bytes_q4(self):
        """Bytes of all 4-bit linears incl. the tied head (0.5625 B/param)."""
        H, I, kvd = self.hidden, self.inter, self.kvd
        per_layer = H * H * 2 + 2 * kvd * H + 3 * H * I
        return int((per_layer * self.n_layers + self.vocab * H) * 0.5625)


QWEN2_05B = LmSpec()


def _to_dev(arr_u16, shape, device):
    import torch

    t = torch.from_numpy(arr_u16.view(np.int16).reshape(shape))
    return t.to(device).view(torch.bfloat16)


class SyntheticLm:
    """Device weights of a Qwen2 stack plus the C-ABI views of them."""

    def __init__(self, ctx: Context, spec: LmSpec, seed=0, quant=True, std=0.02, norm_std=0.0, device="cuda",
                 threads=None):
        import torch

        self.ctx, self.spec, self.seed, self.quant, self.device = ctx, spec, seed, quant, device
        self.tensors = {}  # name -> dict(w=..., s=..., b=...) or bf16 tensor
        H, I, kvd, V = spec.hidden, spec.inter, spec.kvd, spec.vocab

        def normal(name, shape, mean=0.0, sd=std):
            n = int(np.prod(shape))
            return synth_normal_bf16(seed, name, n, mean, sd, threads)

        def add_linear(name, N, K):
            w = _to_dev(normal(name + ".weight", (N, K)), (N, K), device)
            if not quant:
                self.tensors[name] = dict(w=w)
                return
            wq = torch.empty((N, K // 8), dtype=torch.int32, device=device)
            s = torch.empty((N, K // 64), dtype=torch.bfloat16, device=device)
            b = torch.empty((N, K // 64), dtype=torch.bfloat16, device=device)
            ctx.quantize(w, wq, s, b)
            ctx.sync()
            del w
            self.tensors[name] = dict(w=wq, s=s, b=b)

        def add_vec(name, n, mean=0.0, sd=std):
            self.tensors[name] = _to_dev(normal(name, (n,), mean, sd), (n,), device)

        def add_norm(name, n):
            if norm_std == 0.0:
                self.tensors[name] = torch.ones(n, dtype=torch.bfloat16, device=device)
            else:
                add_vec(name, n, 1.0, norm_std)

        P = "model.model"
        add_linear(f"{P}.embed_tokens", V, H)
        for i in range(spec.n_layers):
            L = f"{P}.layers.{i}"
            add_norm(f"{L}.input_layernorm.weight", H)
            add_norm(f"{L}.post_attention_layernorm.weight", H)
            add_linear(f"{L}.self_attn.q_proj", H, H)
            add_linear(f"{L}.self_attn.k_proj", kvd, H)
            add_linear(f"{L}.self_attn.v_proj", kvd, H)
            add_vec(f"{L}.self_attn.q_proj.bias", H)
            add_vec(f"{L}.self_attn.k_proj.bias", kvd)
            add_vec(f"{L}.self_attn.v_proj.bias", kvd)
            add_linear(f"{L}.self_attn.o_proj", H, H)
            add_linear(f"{L}.mlp.gate_proj", I, H)
            add_linear(f"{L}.mlp.up_proj", I, H)
            add_linear(f"{L}.mlp.down_proj", H, I)
        add_norm(f"{P}.norm.weight", H)
        self._build_views()

    # ---- C-ABI views ----
    def lin(self, name):
        t = self.tensors[name]
        if "s" in t:
            return linear(t["w"], t["s"], t["b"])
        return linear(t["w"])

    def _build_views(self):
        spec, P = self.spec, "model.model"
        self.layers = []
        for i in range(spec.n_layers):
            L = f"{P}.layers.{i}"
            self.layers.append(LmLayerW(
                self.tensors[f"{L}.input_layernorm.weight"].data_ptr(),
                self.tensors[f"{L}.post_attention_layernorm.weight"].data_ptr(),
                self.lin(f"{L}.self_attn.q_proj"), self.lin(f"{L}.self_attn.k_proj"),
                self.lin(f"{L}.self_attn.v_proj"), self.lin(f"{L}.self_attn.o_proj"),
                self.lin(f"{L}.mlp.gate_proj"), self.lin(f"{L}.mlp.up_proj"), self.lin(f"{L}.mlp.down_proj"),
                self.tensors[f"{L}.self_attn.q_proj.bias"].data_ptr(),
                self.tensors[f"{L}.self_attn.k_proj.bias"].data_ptr(),
                self.tensors[f"{L}.self_attn.v_proj.bias"].data_ptr()))
        self.embed = self.lin(f"{P}.embed_tokens")
        self.head = self.embed  # tied
        self.final_norm = self.tensors[f"{P}.norm.weight"]
        self.cfg = spec.cfg()

    def model(self):
        return LmModel(self.ctx, self.cfg, self.layers, self.final_norm, self.head, self.embed)

    # ---- host copies (for the CPU checker) ----
    def host(self, name):
        """numpy copy of a tensor: bf16 -> uint16, packed -> uint32; dict for linears."""
        import torch

        t = self.tensors[name]

        def cpu(x):
            if x.dtype == torch.bfloat16:
                return x.view(torch.int16).cpu().numpy().view(np.uint16)
            return x.cpu().numpy().view(np.uint32)

        if isinstance(t, dict):
            return {k: cpu(v) for k, v in t.items()}
        return cpu(t)


@dataclass
class VaeSpec:
    """The VAE decoder's shape (reference: the LM-shaped Qwen2 stack with a
    window of 64, latent 64, patch 4, n_fft 3528, hop 882)."""
    hidden: int = 896
    heads: int = 14
    kv_heads: int = 2
    head_dim: int = 64
    inter: int = 4864
    n_layers: int = 24
    eps: float = 1e-6
    theta: float = 1e6
    window: int = 64
    latent: int = 64
    patch: int = 4
    n_fft: int = 3528
    hop: int = 882

    @property
    def kvd(self):
        return self.kv_heads * self.head_dim

    def cfg(self):
        return VaeCfg(self.hidden, self.heads, self.kv_heads, self.head_dim, self.inter, self.n_layers, self.eps,
                      float(np.log2(np.float32(self.theta))), self.window, self.latent, self.patch, self.n_fft,
                      self.hop)

    def weight_params(self):
        H, I, kvd = self.hidden, self.inter, self.kvd
        per_layer = H * H * 2 + 2 * kvd * H + 3 * H * I
        return per_layer * self.n_layers + H * self.latent + (self.n_fft + 2) * H


MING_VAE = VaeSpec()


def hann_window(n):
    """Periodic Hann window (torch.hann_window's default), f32."""
    k = np.arange(n)
    return (0.5 - 0.5 * np.cos(2.0 * np.pi * k / n)).astype(np.float32)


class SyntheticVae:
    """Device weights of the VAE decoder under the checkpoint's key names
    (audio.decoder.fc1 / .decoder.layers.* / .decoder.norm / .head.out /
    .head.istft.window): bf16 N(0, std) linears (4-bit when quant), biases on
    fc1, q/k/v and the head, norms 1 + N(0, norm_std), a periodic Hann window."""

    def __init__(self, ctx: Context, spec: VaeSpec = MING_VAE, seed=0, quant=False, std=0.02, norm_std=0.0,
                 device="cuda", threads=None):
        import torch

        self.ctx, self.spec, self.quant = ctx, spec, quant
        self.tensors = {}
        H, I, kvd = spec.hidden, spec.inter, spec.kvd

        def normal(name, n, mean=0.0, sd=std):
            return synth_normal_bf16(seed, name, n, mean, sd, threads)

        def add_linear(name, N, K, sd=std):
            w = _to_dev(normal(name + ".weight", N * K, 0.0, sd), (N, K), device)
            if not quant:
                self.tensors[name] = dict(w=w)
                return
            wq = torch.empty((N, K // 8), dtype=torch.int32, device=device)
            sc = torch.empty((N, K // 64), dtype=torch.bfloat16, device=device)
            bi = torch.empty((N, K // 64), dtype=torch.bfloat16, device=device)
            ctx.quantize(w, wq, sc, bi)
            ctx.sync()
            self.tensors[name] = dict(w=wq, s=sc, b=bi)

        def add_vec(name, n, mean=0.0, sd=std):
            self.tensors[name] = _to_dev(normal(name, n, mean, sd), (n,), device)

        def add_norm(name, n):
            if norm_std == 0.0:
                self.tensors[name] = torch.ones(n, dtype=torch.bfloat16, device=device)
            else:
                add_vec(name, n, 1.0, norm_std)

        D, P = "audio.decoder", "audio.decoder.decoder"
        add_linear(f"{D}.fc1", H, spec.latent, 0.1)
        add_vec(f"{D}.fc1.bias", H)
        for i in range(spec.n_layers):
            L = f"{P}.layers.{i}"
            add_norm(f"{L}.input_layernorm.weight", H)
            add_norm(f"{L}.post_attention_layernorm.weight", H)
            add_linear(f"{L}.self_attn.q_proj", H, H)
            add_linear(f"{L}.self_attn.k_proj", kvd, H)
            add_linear(f"{L}.self_attn.v_proj", kvd, H)
            add_vec(f"{L}.self_attn.q_proj.bias", H)
            add_vec(f"{L}.self_attn.k_proj.bias", kvd)
            add_vec(f"{L}.self_attn.v_proj.bias", kvd)
            add_linear(f"{L}.self_attn.o_proj", H, H)
            add_linear(f"{L}.mlp.gate_proj", I, H)
            add_linear(f"{L}.mlp.up_proj", I, H)
            add_linear(f"{L}.mlp.down_proj", H, I)
        add_norm(f"{P}.norm.weight", H)
        add_linear(f"{D}.head.out", spec.n_fft + 2, H)
        add_vec(f"{D}.head.out.bias", spec.n_fft + 2)
        self.tensors[f"{D}.head.istft.window"] = torch.from_numpy(hann_window(spec.n_fft)).to(device)
        self._build_views()

    def lin(self, name):
        t = self.tensors[name]
        if "s" in t:
            return linear(t["w"], t["s"], t["b"])
        return linear(t["w"])

    def _build_views(self):
        spec, D, P = self.spec, "audio.decoder", "audio.decoder.decoder"
        t = self.tensors
        self.layers = (LmLayerW * spec.n_layers)()
        for i in range(spec.n_layers):
            L = f"{P}.layers.{i}"
            self.layers[i] = LmLayerW(
                t[f"{L}.input_layernorm.weight"].data_ptr(), t[f"{L}.post_attention_layernorm.weight"].data_ptr(),
                self.lin(f"{L}.self_attn.q_proj"), self.lin(f"{L}.self_attn.k_proj"),
                self.lin(f"{L}.self_attn.v_proj"), self.lin(f"{L}.self_attn.o_proj"),
                self.lin(f"{L}.mlp.gate_proj"), self.lin(f"{L}.mlp.up_proj"), self.lin(f"{L}.mlp.down_proj"),
                t[f"{L}.self_attn.q_proj.bias"].data_ptr(), t[f"{L}.self_attn.k_proj.bias"].data_ptr(),
                t[f"{L}.self_attn.v_proj.bias"].data_ptr())
        import ctypes

        self.w = VaeW(self.lin(f"{D}.fc1"), t[f"{D}.fc1.bias"].data_ptr(), ctypes.cast(self.layers, ctypes.c_void_p),
                      t[f"{P}.norm.weight"].data_ptr(), self.lin(f"{D}.head.out"), t[f"{D}.head.out.bias"].data_ptr(),
                      t[f"{D}.head.istft.window"].data_ptr())
        self.cfg = spec.cfg()

    def model(self, max_latents):
        return VaeModel(self.ctx, self.cfg, self.w, max_latents)

    def host(self, name):
        """numpy copy: bf16 -> uint16, packed -> uint32, f32 as is; dict for linears."""
        import torch

        def cpu(x):
            if x.dtype == torch.bfloat16:
                return x.view(torch.int16).cpu().numpy().view(np.uint16)
            if x.dtype == torch.float32:
                return x.cpu().numpy()
            return x.cpu().numpy().view(np.uint32)

        v = self.tensors[name]
        return {k: cpu(x) for k, x in v.items()} if isinstance(v, dict) else cpu(v)


class KvCache:
    """In-place bf16 KV cache [n_layers][kv_heads][capacity][head_dim] on the device."""

    def __init__(self, spec: LmSpec, capacity, device="cuda"):
        import torch

        shape = (spec.n_layers, spec.kv_heads, capacity, spec.head_dim)
        self.k = torch.zeros(shape, dtype=torch.bfloat16, device=device)
        self.v = torch.zeros(shape, dtype=torch.bfloat16, device=device)
        self.kv = Kv(self.k.data_ptr(), self.v.data_ptr(), spec.n_layers, spec.kv_heads, spec.head_dim, capacity, 0)

    @property
    def len(self):
        return self.kv.len

    def fill_random(self, n, seed=0, std=1.0, threads=None):
        """Rows [0, n) of every layer/head ~ bf16(N(0, std)); len = n."""
        import torch

        L, kvh, cap, hd = self.k.shape
        for nm, t in (("kv.k", self.k), ("kv.v", self.v)):
            arr = synth_normal_bf16(seed, nm, L * kvh * n * hd, 0.0, std, threads)
            t[:, :, :n, :] = torch.from_numpy(arr.view(np.int16).reshape(L, kvh, n, hd)).to(t.device).view(
                torch.bfloat16)
        self.kv.len = n

    def host(self):
        import torch

        return (self.k.view(torch.int16).cpu().numpy().view(np.uint16),
                self.v.view(torch.int16).cpu().numpy().view(np.uint16))


class PagedKv:
    """Paged bf16 KV cache of n_seq sequences on the device (ming_kv_pages):
    pages of 64 positions, K [n_layers][n_pages][kv_heads][64][head_dim], V
    [n_layers][n_pages][kv_heads][head_dim][64] (each page transposed).  Each
    sequence owns pages_per_seq pages, drawn from a seeded permutation of the
    pool so that consecutive positions do not sit in consecutive pages."""

    def __init__(self, spec: LmSpec, n_seq, pages_per_seq, spare=0, seed=0, device="cuda"):
        import torch

        self.spec, self.n_seq, self.pps = spec, int(n_seq), int(pages_per_seq)
        self.n_pages = self.n_seq * self.pps + int(spare)
        L, kvh, hd = spec.n_layers, spec.kv_heads, spec.head_dim
        self.k = torch.zeros((L, self.n_pages, kvh, 64, hd), dtype=torch.bfloat16, device=device)
        self.v = torch.zeros((L, self.n_pages, kvh, hd, 64), dtype=torch.bfloat16, device=device)
        perm = np.random.default_rng(seed).permutation(self.n_pages)[: self.n_seq * self.pps]
        self.set_table(perm.reshape(self.n_seq, self.pps))
        self.pos = torch.zeros(self.n_seq, dtype=torch.int32, device=device)
        self.kv = KvPages(self.k.data_ptr(), self.v.data_ptr(), L, kvh, hd, 64, self.n_pages)

    def set_table(self, table):
        import torch

        self.table_host = np.ascontiguousarray(table, dtype=np.int32)
        self.table = torch.from_numpy(self.table_host).to(self.k.device)

    def set_seq(self, i, kc, vc):
        """Rows [0, n) of sequence i from contiguous host u16 [L][kvh][n][hd]; pos[i] = n."""
        import torch

        L, kvh, n, hd = kc.shape
        for p in range((n + 63) // 64):
            m = min(64, n - 64 * p)
            bk = np.zeros((L, kvh, 64, hd), np.uint16)
            bv = np.zeros((L, kvh, 64, hd), np.uint16)
            bk[:, :, :m] = kc[:, :, 64 * p:64 * p + m]
            bv[:, :, :m] = vc[:, :, 64 * p:64 * p + m]
            pid = int(self.table_host[i, p])
            self.k[:, pid] = torch.from_numpy(bk.view(np.int16)).to(self.k.device).view(torch.bfloat16)
            self.v[:, pid] = torch.from_numpy(np.ascontiguousarray(bv.transpose(0, 1, 3, 2)).view(np.int16)).to(
                self.k.device).view(torch.bfloat16)
        self.pos[i] = n

    def fill_random(self, lens, seed=0, std=1.0):
        """Sequence i gets lens[i] rows ~ bf16(N(0, std)) in every layer/head;
        returns the host copies [(kc, vc)] in the contiguous layout."""
        L, kvh, hd = self.spec.n_layers, self.spec.kv_heads, self.spec.head_dim
        host = []
        for i, n in enumerate(lens):
            kc = synth_normal_bf16(seed, f"pkv.k.{i}", L * kvh * n * hd, 0.0, std).reshape(L, kvh, n, hd)
            vc = synth_normal_bf16(seed, f"pkv.v.{i}", L * kvh * n * hd, 0.0, std).reshape(L, kvh, n, hd)
            self.set_seq(i, kc, vc)
            host.append((kc, vc))
        return host

    def fill_device(self, lens, seed=0):
        """Every page ~ bf16(N(0,1)) from a seeded device generator (benchmark
        contents); pos = lens."""
        import torch

        g = torch.Generator(device=self.k.device)
        g.manual_seed(int(seed))
        self.k.normal_(generator=g)
        self.v.normal_(generator=g)
        self.pos.copy_(torch.tensor(lens, dtype=torch.int32))

    def gather(self, i, n):
        """Rows [0, n) of sequence i as contiguous host u16 [L][kvh][n][hd] (k, v)."""
        import torch

        pages = [int(p) for p in self.table_host[i, : (n + 63) // 64]]
        idx = torch.tensor(pages, dtype=torch.long, device=self.k.device)
        k = self.k.index_select(1, idx).permute(0, 2, 1, 3, 4)  # [L][kvh][np][64][hd]
        v = self.v.index_select(1, idx).permute(0, 2, 1, 4, 3)
        L, kvh = k.shape[0], k.shape[1]
        k = k.reshape(L, kvh, -1, k.shape[-1])[:, :, :n]
        v = v.reshape(L, kvh, -1, v.shape[-1])[:, :, :n]
        return (k.contiguous().view(torch.int16).cpu().numpy().view(np.uint16),
                v.contiguous().view(torch.int16).cpu().numpy().view(np.uint16))


def lm_bytes_per_token(spec: LmSpec, ctx_len):
    """Algorithmic HBM bytes of one 4-bit decode token at `ctx_len` cached
    positions: 4-bit linears + tied head (0.5625 B/param), q/k/v biases and
    norm weights, the KV read of ctx_len cached rows and the one-row append."""
    H, kvd, L = spec.hidden, spec.kvd, spec.n_layers
    small = L * (2 * H + (H + 2 * kvd)) * 2 + H * 2
    kv_row = L * 2 * kvd * 2
    return spec.weight_bytes_q4() + small + kv_row * ctx_len + kv_row


# ---- DiT flow head, aggregator and stop head -------------------------------------


@dataclass
class DitSpec:
    """Shapes of the flow head / aggregator (src/ming_model.zig:37-41, :943-956)."""
    hidden: int = 1024
    heads: int = 16
    head_dim: int = 64
    ff: int = 4096
    eps: float = 1e-6
    cfm_blocks: int = 8
    agg_blocks: int = 8
    latent: int = 64
    lm_hidden: int = 896

    def cfg(self):
        from . import DitCfg

        return DitCfg(self.hidden, self.heads, self.head_dim, self.ff, self.eps)

    def inv_freq(self):
        """RotaryEmbedding.inv_freq = 1 / 10000^(2i / head_dim), f32."""
        i = np.arange(0, self.head_dim, 2, dtype=np.float32)
        return (1.0 / (np.float32(10000.0) ** (i / np.float32(self.head_dim)))).astype(np.float32)

    def block_params(self):
        D, F = self.hidden, self.ff
        return 4 * D * D + 2 * D * F + 5 * D + F

    def cfm_weight_bytes(self):
        D, H, lat = self.hidden, self.lm_hidden, self.latent
        return 2 * (self.cfm_blocks * self.block_params() + D * lat + D * H + lat * D + 3 * D + lat)


MING_DIT = DitSpec()

_BLOCK_KEYS = (("wq", "attn.to_q"), ("wk", "attn.to_k"), ("wv", "attn.to_v"), ("wo", "attn.to_out.0"),
               ("w1", "mlp.ff.0.0"), ("w2", "mlp.ff.2"))


class SyntheticFlow:
    """bf16 weights of the flow head ("flowloss.cfm.model"), aggregator
    ("linear_proj_audio") and stop head under the checkpoint's key names
    (src/ming_model.zig:941-956, :728-745), random-init: linears and biases
    bf16(N(0, std)), norm weights 1 + N(0, norm_std).  Host copies (numpy
    uint16) are kept for the CPU checker; device copies feed the C ABI."""

    def __init__(self, ctx, spec: DitSpec = MING_DIT, seed=0, std=0.02, norm_std=0.0, device="cuda", threads=None,
                 parts=("cfm", "agg", "stop")):
        import torch

        from . import AggW, CfmW, DitBlockW

        self.ctx, self.spec, self.device = ctx, spec, device
        self.hostw, self.dev = {}, {}
        D, F, lat, H = spec.hidden, spec.ff, spec.latent, spec.lm_hidden

        def put(name, shape, mean=0.0, sd=std):
            a = synth_normal_bf16(seed, name, int(np.prod(shape)), mean, sd, threads).reshape(shape)
            self.hostw[name] = a
            self.dev[name] = torch.from_numpy(a.view(np.int16)).to(device).view(torch.bfloat16)

        def lin(name, N, K, bias=True):
            put(name + ".weight", (N, K))
            if bias:
                put(name + ".bias", (N,))

        def norm(name, n):
            if norm_std == 0.0:
                a = np.full(n, 0x3F80, np.uint16)
                self.hostw[name] = a
                self.dev[name] = torch.from_numpy(a.view(np.int16)).to(device).view(torch.bfloat16)
            else:
                put(name, (n,), 1.0, norm_std)

        def blocks(prefix, n):
            for i in range(n):
                b = f"{prefix}.blocks.{i}"
                norm(f"{b}.norm1.weight", D)
                norm(f"{b}.norm2.weight", D)
                for k, key in _BLOCK_KEYS:
                    N, K = {"w1": (F, D), "w2": (D, F)}.get(k, (D, D))
                    lin(f"{b}.{key}", N, K)

        self.inv_freq = spec.inv_freq()
        if "cfm" in parts:
            C = "flowloss.cfm.model"
            blocks(C, spec.cfm_blocks)
            lin(f"{C}.t_embedder.time_mlp.0", D, 256)
            lin(f"{C}.t_embedder.time_mlp.2", D, D)
            lin(f"{C}.x_embedder", D, lat)
            lin(f"{C}.c_embedder.cond_embedder", D, H)
            norm(f"{C}.final_layer.norm_final.weight", D)
            lin(f"{C}.final_layer.linear", lat, D)
            self.cfm_blocks = (DitBlockW * spec.cfm_blocks)(*(self.block_w(C, i) for i in range(spec.cfm_blocks)))
            self.cfm_w = CfmW(spec.cfg(), spec.cfm_blocks, ctypes.cast(self.cfm_blocks, ctypes.c_void_p),
                              self.inv_freq.ctypes.data, self.lin_w(f"{C}.x_embedder"),
                              self.lin_w(f"{C}.c_embedder.cond_embedder"), self.lin_w(f"{C}.t_embedder.time_mlp.0"),
                              self.lin_w(f"{C}.t_embedder.time_mlp.2"), self.lin_w(f"{C}.final_layer.linear"),
                              *(self.ptr(f"{C}.{k}") for k in ("x_embedder.bias", "c_embedder.cond_embedder.bias",
                                                                "t_embedder.time_mlp.0.bias",
                                                                "t_embedder.time_mlp.2.bias",
                                                                "final_layer.norm_final.weight",
                                                                "final_layer.linear.bias")))
        if "agg" in parts:
            A = "linear_proj_audio"
            blocks(A, spec.agg_blocks)
            lin(f"{A}.x_embedder", D, lat)
            put(f"{A}.word_embedder.weight", (D,), 0.0, 1.0)
            norm(f"{A}.final_layer.norm_final.weight", D)
            lin(f"{A}.final_layer.linear", H, D)
            self.agg_blocks = (DitBlockW * spec.agg_blocks)(*(self.block_w(A, i) for i in range(spec.agg_blocks)))
            self.agg_w = AggW(spec.cfg(), spec.agg_blocks, ctypes.cast(self.agg_blocks, ctypes.c_void_p),
                              self.inv_freq.ctypes.data, self.lin_w(f"{A}.x_embedder"),
                              self.lin_w(f"{A}.final_layer.linear"),
                              *(self.ptr(f"{A}.{k}") for k in ("x_embedder.bias", "word_embedder.weight",
                                                                "final_layer.norm_final.weight",
                                                                "final_layer.linear.bias")))
        if "stop" in parts:
            lin("stop_head", 2, H)

    # ---- C-ABI views ----
    def ptr(self, name):
        return self.dev[name].data_ptr()

    def lin_w(self, name):
        return linear(self.dev[name + ".weight"])

    def block_w(self, prefix, i):
        from . import DitBlockW

        b = f"{prefix}.blocks.{i}"
        return DitBlockW(self.ptr(f"{b}.norm1.weight"), self.ptr(f"{b}.norm2.weight"),
                         *(self.lin_w(f"{b}.{key}") for _, key in _BLOCK_KEYS),
                         *(self.ptr(f"{b}.{key}.bias") for _, key in _BLOCK_KEYS))

    def cfm_model(self):
        from . import CfmModel

        return CfmModel(self.ctx, self.cfm_w)

    def agg_model(self):
        from . import AggModel

        return AggModel(self.ctx, self.agg_w)


@dataclass
class AdalnSpec(DitSpec):
    """Config 4's adaLN flow head: 4 blocks, hidden 896, 14 heads x 64, ff 4 x 896,
    a patch of 4 frames x 64 (no reference shape; DiT-style adaLN-Zero)."""
    hidden: int = 896
    heads: int = 14
    ff: int = 3584
    cfm_blocks: int = 4
    frames: int = 4

    def ada_params(self):
        return 6 * self.hidden * self.hidden + 6 * self.hidden

    def sample_weight_bytes(self):
        """bf16 bytes one sample reads: the modulation linears once, then per Euler
        step the blocks, x_emb and the final linear; c_emb once."""
        D, H, lat = self.hidden, self.lm_hidden, self.latent
        once = self.cfm_blocks * self.ada_params() + 2 * D * D + 2 * D + D * H + D
        per_step = self.cfm_blocks * self.block_params() + D * lat + D + lat * D + lat + D
        return 2 * (once + 10 * per_step)


MING_ADALN = AdalnSpec()


class SyntheticAdaln:
    """bf16 weights of config 4's adaLN flow head (DiT-style key names under
    "adaln": blocks.{i}.{attn,mlp,norm*,adaLN_modulation.1}, t_embedder,
    x_embedder, c_embedder, final_layer.{norm_final, linear, adaLN_modulation.1}),
    random-init N(0, std); norms 1 + N(0, norm_std).  ada_std scales the
    modulation linears (0 with bias_pattern "zero" gives shift = scale = 0,
    gate = 1: the reference block)."""

    def __init__(self, ctx, spec: AdalnSpec = MING_ADALN, seed=0, std=0.02, norm_std=0.0, ada_std=None,
                 zero_modulation=False, device="cuda", threads=None):
        import torch

        from . import AdalnBlockW, AdalnW

        self.ctx, self.spec, self.device = ctx, spec, device
        self.hostw, self.dev = {}, {}
        D, F, lat, H = spec.hidden, spec.ff, spec.latent, spec.lm_hidden
        ada_std = std if ada_std is None else ada_std

        def store(name, a):
            self.hostw[name] = a
            self.dev[name] = torch.from_numpy(a.view(np.int16)).to(device).view(torch.bfloat16)

        def put(name, shape, mean=0.0, sd=std):
            store(name, synth_normal_bf16(seed, name, int(np.prod(shape)), mean, sd, threads).reshape(shape))

        def lin(name, N, K, bias=True, sd=std):
            put(name + ".weight", (N, K), 0.0, sd)
            if bias:
                put(name + ".bias", (N,), 0.0, sd)

        def norm(name, n):
            if norm_std == 0.0:
                store(name, np.full(n, 0x3F80, np.uint16))
            else:
                put(name, (n,), 1.0, norm_std)

        def zero_ada(name, chunks, gates):
            store(name + ".weight", np.zeros((chunks * D, D), np.uint16))
            b = np.zeros(chunks * D, np.uint16)
            for g in gates:
                b[g * D:(g + 1) * D] = 0x3F80  # 1.0
            store(name + ".bias", b)

        A = "adaln"
        for i in range(spec.cfm_blocks):
            b = f"{A}.blocks.{i}"
            norm(f"{b}.norm1.weight", D)
            norm(f"{b}.norm2.weight", D)
            for k, key in _BLOCK_KEYS:
                N, K = {"w1": (F, D), "w2": (D, F)}.get(k, (D, D))
                lin(f"{b}.{key}", N, K)
            if zero_modulation:
                zero_ada(f"{b}.adaLN_modulation.1", 6, (2, 5))
            else:
                lin(f"{b}.adaLN_modulation.1", 6 * D, D, sd=ada_std)
        lin(f"{A}.t_embedder.time_mlp.0", D, 256)
        lin(f"{A}.t_embedder.time_mlp.2", D, D)
        lin(f"{A}.x_embedder", D, lat)
        lin(f"{A}.c_embedder", D, H)
        norm(f"{A}.final_layer.norm_final.weight", D)
        lin(f"{A}.final_layer.linear", lat, D)
        if zero_modulation:
            zero_ada(f"{A}.final_layer.adaLN_modulation.1", 2, ())
        else:
            lin(f"{A}.final_layer.adaLN_modulation.1", 2 * D, D, sd=ada_std)
        self.inv_freq = spec.inv_freq()
        self.blocks = (AdalnBlockW * spec.cfm_blocks)(*(self.block_w(i) for i in range(spec.cfm_blocks)))
        lw = lambda n: linear(self.dev[n + ".weight"])
        pt = lambda n: self.dev[n].data_ptr()
        self.w = AdalnW(spec.cfg(), spec.cfm_blocks, spec.frames, ctypes.cast(self.blocks, ctypes.c_void_p),
                        self.inv_freq.ctypes.data, lw(f"{A}.x_embedder"), lw(f"{A}.c_embedder"),
                        lw(f"{A}.t_embedder.time_mlp.0"), lw(f"{A}.t_embedder.time_mlp.2"),
                        lw(f"{A}.final_layer.linear"), lw(f"{A}.final_layer.adaLN_modulation.1"),
                        pt(f"{A}.x_embedder.bias"), pt(f"{A}.c_embedder.bias"), pt(f"{A}.t_embedder.time_mlp.0.bias"),
                        pt(f"{A}.t_embedder.time_mlp.2.bias"), pt(f"{A}.final_layer.norm_final.weight"),
                        pt(f"{A}.final_layer.linear.bias"), pt(f"{A}.final_layer.adaLN_modulation.1.bias"))

    def block_w(self, i):
        from . import AdalnBlockW, DitBlockW

        b = f"adaln.blocks.{i}"
        p = lambda n: self.dev[n].data_ptr()
        base = DitBlockW(p(f"{b}.norm1.weight"), p(f"{b}.norm2.weight"),
                         *(linear(self.dev[f"{b}.{key}.weight"]) for _, key in _BLOCK_KEYS),
                         *(p(f"{b}.{key}.bias") for _, key in _BLOCK_KEYS))
        return AdalnBlockW(base, linear(self.dev[f"{b}.adaLN_modulation.1.weight"]),
                           p(f"{b}.adaLN_modulation.1.bias"))

    def model(self):
        from . import AdalnModel

        return AdalnModel(self.ctx, self.w)


__all__ = ["VaeSpec", "MING_VAE", "SyntheticVae", "hann_window", "AdalnSpec", "MING_ADALN", "SyntheticAdaln", "DitSpec", "MING_DIT", "SyntheticFlow", "LmSpec", "QWEN2_05B", "SyntheticLm", "KvCache", "lm_bytes_per_token", "W_AFFINE", "W_BF16",
           "Linear", "math"]
