"""ctypes wrapper of oracle/build/liboracle.so -- TEST INFRASTRUCTURE ONLY.

The CPU restatement of the reference's per-token loop (see oracle.h).  Only
tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use it, as the
checker; the product library never does.

All arrays are numpy: bf16 values travel as uint16 bit patterns, packed
affine weights as uint32.
"""
import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "build", "liboracle.so")

OR_W_BF16, OR_W_AFFINE = 0, 1

c_void_p, c_int, c_i64, c_f32 = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_float


class OrLinear(ctypes.Structure):
    _fields_ = [("kind", c_int), ("N", c_i64), ("K", c_i64), ("w", c_void_p), ("scales", c_void_p),
                ("biases", c_void_p), ("gscale", c_f32), ("group", c_int), ("bits", c_int)]


class OrLmCfg(ctypes.Structure):
    _fields_ = [("hidden", c_int), ("heads", c_int), ("kv_heads", c_int), ("head_dim", c_int), ("inter", c_int),
                ("eps", c_f32), ("log2_theta", c_f32)]


class OrLmLayer(ctypes.Structure):
    _fields_ = [("ln1", c_void_p), ("ln2", c_void_p)] + [
        (n, OrLinear) for n in ("q", "k", "v", "o", "gate", "up", "down")] + [
        ("bq", c_void_p), ("bk", c_void_p), ("bv", c_void_p)]


class OrLmTrace(ctypes.Structure):
    _fields_ = [("h", c_void_p), ("qkv", c_void_p), ("att", c_void_p), ("x1", c_void_p), ("hh", c_void_p)]


class OrDitCfg(ctypes.Structure):
    _fields_ = [("D", c_int), ("heads", c_int), ("head_dim", c_int), ("ff", c_int), ("eps", c_f32)]


class OrDitBlock(ctypes.Structure):
    _fields_ = [("norm1", c_void_p), ("norm2", c_void_p)] + [
        (n, OrLinear) for n in ("q", "k", "v", "o", "ff1", "ff2")] + [
        (n, c_void_p) for n in ("bq", "bk", "bv", "bo", "b1", "b2")]


class OrDitTrace(ctypes.Structure):
    _fields_ = [("qkv", c_void_p), ("att", c_void_p), ("x1", c_void_p), ("hh", c_void_p)]


class OrCfmModel(ctypes.Structure):
    _fields_ = [("c", OrDitCfg), ("n_blocks", c_int), ("blocks", c_void_p), ("x_emb", OrLinear), ("bx", c_void_p),
                ("c_emb", OrLinear), ("bc", c_void_p), ("final_norm", c_void_p), ("final", OrLinear),
                ("bf", c_void_p), ("t_emb", c_void_p), ("dt", c_void_p), ("sq", c_void_p), ("cos_t", c_void_p),
                ("sin_t", c_void_p), ("steps", c_int)]


class OrAdalnBlock(ctypes.Structure):
    _fields_ = [("blk", OrDitBlock), ("ada", OrLinear), ("bada", c_void_p)]


class OrAdalnModel(ctypes.Structure):
    _fields_ = [("c", OrDitCfg), ("n_blocks", c_int), ("blocks", c_void_p), ("x_emb", OrLinear), ("bx", c_void_p),
                ("c_emb", OrLinear), ("bc", c_void_p), ("final_norm", c_void_p), ("final", OrLinear),
                ("bf", c_void_p), ("final_ada", OrLinear), ("bfa", c_void_p), ("t_emb", c_void_p),
                ("dt", c_void_p), ("sq", c_void_p), ("cos_t", c_void_p), ("sin_t", c_void_p), ("steps", c_int),
                ("frames", c_int)]


class OrAggModel(ctypes.Structure):
    _fields_ = [("c", OrDitCfg), ("n_blocks", c_int), ("blocks", c_void_p), ("x_emb", OrLinear), ("bx", c_void_p),
                ("cls", c_void_p), ("final_norm", c_void_p), ("final", OrLinear), ("bf", c_void_p),
                ("cos_t", c_void_p), ("sin_t", c_void_p)]


class OrVaeCfg(ctypes.Structure):
    _fields_ = [("hidden", c_int), ("heads", c_int), ("kv_heads", c_int), ("head_dim", c_int), ("inter", c_int),
                ("n_layers", c_int), ("eps", c_f32), ("log2_theta", c_f32), ("window", c_int), ("latent", c_int),
                ("patch", c_int), ("n_fft", c_int), ("hop", c_int)]


class OrVaeModel(ctypes.Structure):
    _fields_ = [("cfg", OrVaeCfg), ("fc1", OrLinear), ("fc1_bias", c_void_p), ("layers", c_void_p),
                ("norm", c_void_p), ("head", OrLinear), ("head_bias", c_void_p), ("window_fn", c_void_p)]


class OrVaeTrace(ctypes.Structure):
    _fields_ = [("qkv", c_void_p), ("att", c_void_p), ("x1", c_void_p), ("hh", c_void_p)]


_lib = None


def lib():
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise OSError(f"{LIB_PATH} is not built (make -C oracle)")
    L = ctypes.CDLL(LIB_PATH)
    P = ctypes.POINTER
    sig = {
        "or_bf16": (ctypes.c_uint16, [c_f32]),
        "or_f32": (c_f32, [ctypes.c_uint16]),
        "or_rb": (c_f32, [c_f32]),
        "or_to_bf16": (None, [c_void_p, c_void_p, c_i64]),
        "or_quantize": (c_int, [c_void_p, c_i64, c_i64, c_int, c_int, c_f32, c_void_p, c_void_p, c_void_p]),
        "or_dequantize": (c_int, [c_void_p, c_void_p, c_void_p, c_i64, c_i64, c_int, c_int, c_f32, c_void_p]),
        "or_linear_acc": (None, [P(OrLinear), c_void_p, c_i64, c_void_p]),
        "or_linear_fwd": (None, [P(OrLinear), c_void_p, c_i64, c_void_p, c_void_p]),
        "or_rms_norm": (None, [c_void_p, c_void_p, c_i64, c_i64, c_f32, c_void_p]),
        "or_rope": (None, [c_void_p, c_int, c_int, c_int, c_f32]),
        "or_swiglu": (None, [c_void_p, c_void_p, c_i64, c_void_p]),
        "or_gelu_approx": (None, [c_void_p, c_i64, c_void_p]),
        "or_add": (None, [c_void_p, c_void_p, c_i64, c_void_p]),
        "or_attention": (None, [c_void_p, c_void_p, c_void_p, c_int, c_int, c_int, c_int, c_int, c_f32, c_void_p]),
        "or_lm_layer_step": (None, [P(OrLmCfg), P(OrLmLayer), c_void_p, c_int, c_void_p, c_void_p, c_int, c_void_p,
                                    P(OrLmTrace)]),
        "or_lm_head": (c_int, [P(OrLmCfg), c_void_p, P(OrLinear), c_void_p, c_void_p, c_void_p, c_void_p,
                               P(c_f32)]),
        "or_embed": (None, [P(OrLinear), c_int, c_void_p]),
        "or_rotary_table": (None, [c_void_p, c_int, c_int, c_void_p, c_void_p]),
        "or_rotary": (None, [c_void_p, c_int, c_int, c_int, c_int, c_void_p, c_void_p]),
        "or_dit_block_fwd": (None, [P(OrDitCfg), P(OrDitBlock), c_void_p, c_int, c_int, c_void_p, c_void_p,
                                    c_void_p, P(OrDitTrace)]),
        "or_flow_schedule": (None, [c_void_p]),
        "or_flow_steps": (None, [c_void_p, c_void_p, c_void_p]),
        "or_t_freq": (None, [c_void_p]),
        "or_timestep_embed": (None, [P(OrLinear), c_void_p, P(OrLinear), c_void_p, c_void_p, ctypes.c_uint16,
                                     c_void_p]),
        "or_cfm_rows": (None, [P(OrCfmModel), c_void_p, c_void_p, c_void_p, c_int, c_void_p]),
        "or_cfm_final": (None, [P(OrCfmModel), c_void_p, c_int, c_void_p, c_void_p, c_int, c_f32, c_f32, c_void_p]),
        "or_cfm_sample": (None, [P(OrCfmModel), c_void_p, c_void_p, c_void_p, c_void_p, c_f32, c_f32, c_void_p,
                                 c_void_p]),
        "or_aggregate": (None, [P(OrAggModel), c_void_p, c_void_p]),
        "or_stop_prob": (c_f32, [P(OrLinear), c_void_p, c_void_p]),
        "or_adaln_block_fwd": (None, [P(OrDitCfg), P(OrDitBlock), c_void_p, c_void_p, c_int, c_int, c_void_p,
                                      c_void_p, c_void_p, P(OrDitTrace)]),
        "or_adaln_cond": (None, [P(OrAdalnModel), c_void_p, c_void_p]),
        "or_adaln_mods": (None, [P(OrAdalnModel), c_void_p, c_void_p, c_void_p]),
        "or_adaln_rows": (None, [P(OrAdalnModel), c_void_p, c_void_p]),
        "or_adaln_final": (None, [P(OrAdalnModel), c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_f32, c_f32,
                                  c_void_p]),
        "or_adaln_sample": (None, [P(OrAdalnModel), c_void_p, c_void_p, c_void_p, c_f32, c_f32, c_void_p,
                                   c_void_p]),
        "or_linear_f32": (None, [P(OrLinear), c_void_p, c_i64, c_void_p, c_void_p]),
        "or_rms_f32": (None, [c_void_p, c_void_p, c_i64, c_i64, c_f32, c_void_p]),
        "or_rope_f32": (None, [c_void_p, c_int, c_int, c_int, c_f32]),
        "or_linear_upsample": (None, [c_void_p, c_int, c_int, c_int, c_void_p]),
        "or_window_attention": (None, [c_void_p, c_void_p, c_void_p, c_int, c_int, c_int, c_int, c_int, c_f32,
                                       c_void_p]),
        "or_vae_layer": (None, [P(OrVaeCfg), P(OrLmLayer), c_void_p, c_int, c_void_p, P(OrVaeTrace)]),
        "or_vae_istft": (None, [c_void_p, c_int, c_int, c_int, c_void_p, c_void_p, c_void_p]),
        "or_vae_decode": (None, [P(OrVaeModel), c_void_p, c_int, c_void_p, c_void_p, c_void_p]),
        "or_set_dit_order": (None, [c_int]),
        "or_get_dit_order": (c_int, []),
        "or_exp_rep": (c_f32, [c_f32]),
        "or_dot_dev": (c_f32, [c_void_p, c_void_p, c_i64, c_int]),
        "or_acc_step": (c_f32, [c_f32, c_void_p, c_void_p, c_int]),
        "or_dot_mfma": (c_f32, [c_void_p, c_void_p, c_i64, c_int]),
        "or_dot2_batch": (None, [c_void_p, c_void_p, c_void_p, c_void_p, c_i64]),
        "or_mfma_batch": (None, [c_void_p, c_void_p, c_void_p, c_void_p, c_i64]),
        "or_sumsq_dev": (c_f32, [c_void_p, c_i64]),
        "or_set_threads": (None, [c_int]),
        "or_get_threads": (c_int, []),
    }
    for name, (res, args) in sig.items():
        f = getattr(L, name)
        f.restype = res
        f.argtypes = args
    _lib = L
    return L


def _p(a):
    return None if a is None else a.ctypes.data_as(c_void_p)


def _c(a, dtype):
    a = np.ascontiguousarray(a)
    assert a.dtype == dtype, (a.dtype, dtype)
    return a


# ---- bf16 ---------------------------------------------------------------------

def to_bf16(x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, np.uint16)
    lib().or_to_bf16(_p(x), _p(out), x.size)
    return out


def to_f32(h):
    h = np.ascontiguousarray(h, dtype=np.uint16)
    return (h.astype(np.uint32) << 16).view(np.float32)


# ---- affine quantization ----------------------------------------------------

def quantize(w, group=64, bits=4, gscale=1.0):
    w = _c(w, np.uint16)
    N, K = w.shape
    wq = np.empty((N, K * bits // 32), np.uint32)
    s = np.empty((N, K // group), np.uint16)
    b = np.empty((N, K // group), np.uint16)
    assert lib().or_quantize(_p(w), N, K, group, bits, gscale, _p(wq), _p(s), _p(b)) == 0
    return wq, s, b


def dequantize(wq, s, b, group=64, bits=4, gscale=1.0):
    wq, s, b = _c(wq, np.uint32), _c(s, np.uint16), _c(b, np.uint16)
    N = wq.shape[0]
    K = wq.shape[1] * 32 // bits
    out = np.empty((N, K), np.uint16)
    assert lib().or_dequantize(_p(wq), _p(s), _p(b), N, K, group, bits, gscale, _p(out)) == 0
    return out


class Linear:
    """Holds the numpy arrays of one linear and its OrLinear view."""

    def __init__(self, w, scales=None, biases=None, gscale=1.0, group=64, bits=4):
        if scales is None:
            self.w = _c(w, np.uint16)
            N, K = self.w.shape
            self.s = self.b = None
            self.c = OrLinear(OR_W_BF16, N, K, _p(self.w), None, None, 1.0, 0, 0)
        else:
            self.w, self.s, self.b = _c(w, np.uint32), _c(scales, np.uint16), _c(biases, np.uint16)
            N = self.w.shape[0]
            K = self.w.shape[1] * 32 // bits
            self.c = OrLinear(OR_W_AFFINE, N, K, _p(self.w), _p(self.s), _p(self.b), gscale, group, bits)
        self.N, self.K = N, K


def linear_acc(L, x):
    x = _c(x, np.uint16)
    M = x.size // L.K
    y = np.empty((M, L.N), np.float32)
    lib().or_linear_acc(ctypes.byref(L.c), _p(x), M, _p(y))
    return y.reshape(x.shape[:-1] + (L.N,))


def linear(L, x, bias=None):
    x = _c(x, np.uint16)
    M = x.size // L.K
    y = np.empty((M, L.N), np.uint16)
    lib().or_linear_fwd(ctypes.byref(L.c), _p(x), M, _p(None if bias is None else _c(bias, np.uint16)), _p(y))
    return y.reshape(x.shape[:-1] + (L.N,))


# ---- element-wise ------------------------------------------------------------

def rms_norm(x, w, eps=1e-6):
    x, w = _c(x, np.uint16), _c(w, np.uint16)
    n = w.size
    out = np.empty_like(x)
    lib().or_rms_norm(_p(x), _p(w), x.size // n, n, eps, _p(out))
    return out


def rope(x, pos, log2_base):
    x = np.array(x, dtype=np.uint16, copy=True, order="C")
    nh, hd = x.shape
    lib().or_rope(_p(x), nh, hd, int(pos), float(log2_base))
    return x


def swiglu(g, u):
    g, u = _c(g, np.uint16), _c(u, np.uint16)
    out = np.empty_like(g)
    lib().or_swiglu(_p(g), _p(u), g.size, _p(out))
    return out


def gelu_approx(x):
    x = _c(x, np.uint16)
    out = np.empty_like(x)
    lib().or_gelu_approx(_p(x), x.size, _p(out))
    return out


def add(a, b):
    a, b = _c(a, np.uint16), _c(b, np.uint16)
    out = np.empty_like(a)
    lib().or_add(_p(a), _p(b), a.size, _p(out))
    return out


def attention(q, kc, vc, pos, scale=None):
    """q [heads, hd]; kc/vc [kv_heads, cap, hd] (rows 0..pos valid)."""
    q, kc, vc = _c(q, np.uint16), _c(kc, np.uint16), _c(vc, np.uint16)
    heads, hd = q.shape
    kvh, cap, _ = kc.shape
    out = np.empty_like(q)
    lib().or_attention(_p(q), _p(kc), _p(vc), heads, kvh, hd, cap, int(pos),
                       float(scale if scale is not None else 1.0 / np.sqrt(np.float32(hd))), _p(out))
    return out


# ---- Qwen2 decode ------------------------------------------------------------

class LmLayer:
    def __init__(self, ln1, ln2, q, k, v, o, gate, up, down, bq, bk, bv):
        self.keep = [_c(ln1, np.uint16), _c(ln2, np.uint16), _c(bq, np.uint16), _c(bk, np.uint16),
                     _c(bv, np.uint16)]
        self.lin = dict(q=q, k=k, v=v, o=o, gate=gate, up=up, down=down)
        self.c = OrLmLayer(_p(self.keep[0]), _p(self.keep[1]), q.c, k.c, v.c, o.c, gate.c, up.c, down.c,
                           _p(self.keep[2]), _p(self.keep[3]), _p(self.keep[4]))


def cfg(hidden, heads, kv_heads, head_dim, inter, eps=1e-6, log2_theta=None, theta=1e6):
    if log2_theta is None:
        log2_theta = float(np.log2(np.float32(theta)))
    return OrLmCfg(hidden, heads, kv_heads, head_dim, inter, eps, log2_theta)


def lm_layer_step(c, layer, x, pos, kc, vc, trace=False):
    """One layer; kc/vc [kv_heads, cap, hd] uint16 arrays updated in place."""
    x = _c(x, np.uint16)
    assert kc.flags.c_contiguous and vc.flags.c_contiguous and kc.dtype == np.uint16
    cap = kc.shape[1]
    out = np.empty_like(x)
    tr = None
    arrs = {}
    if trace:
        kvd = c.kv_heads * c.head_dim
        arrs = dict(h=np.empty(c.hidden, np.uint16), qkv=np.empty(c.hidden + 2 * kvd, np.uint16),
                    att=np.empty(c.hidden, np.uint16), x1=np.empty(c.hidden, np.uint16),
                    hh=np.empty(c.inter, np.uint16))
        tr = OrLmTrace(*(_p(arrs[k]) for k in ("h", "qkv", "att", "x1", "hh")))
    lib().or_lm_layer_step(ctypes.byref(c), ctypes.byref(layer.c), _p(x), int(pos), _p(kc), _p(vc), cap, _p(out),
                           ctypes.byref(tr) if tr is not None else None)
    return (out, arrs) if trace else out


def lm_head(c, norm, head, x):
    """-> (argmax, hidden bf16, logits f32, logits bf16, top-2 margin)."""
    norm, x = _c(norm, np.uint16), _c(x, np.uint16)
    hid = np.empty(c.hidden, np.uint16)
    lg = np.empty(head.N, np.float32)
    lgb = np.empty(head.N, np.uint16)
    m = c_f32()
    am = lib().or_lm_head(ctypes.byref(c), _p(norm), ctypes.byref(head.c), _p(x), _p(hid), _p(lg), _p(lgb),
                          ctypes.byref(m))
    return am, hid, lg, lgb, m.value


def embed(table, idx):
    out = np.empty(table.K, np.uint16)
    lib().or_embed(ctypes.byref(table.c), int(idx), _p(out))
    return out


def set_threads(n):
    lib().or_set_threads(int(n))


DIT_ORDER_MLX, DIT_ORDER_DEVICE, DIT_ORDER_MFMA = 0, 1, 2


class dit_order:
    """Context manager: the DiT functions (blocks, flow head, aggregator, stop head, adaLN head)
    sum in `mode` inside the block -- DIT_ORDER_DEVICE follows the library's batch-1 DiT kernels
    (team lanes over 16-byte chunks, v_dot2c_f32_bf16 steps as or_acc_step restates them,
    pairwise lane trees, exp_rep); DIT_ORDER_MFMA the batched flow head (its matrix-core GEMM's
    dot products, otherwise the device order)."""

    def __init__(self, mode):
        self.mode = int(mode)

    def __enter__(self):
        self.prev = lib().or_get_dit_order()
        lib().or_set_dit_order(self.mode)
        return self

    def __exit__(self, *exc):
        lib().or_set_dit_order(self.prev)
        return False


def exp_rep(x):
    return float(lib().or_exp_rep(float(x)))


def dot_dev(w, x, team):
    w = np.ascontiguousarray(w, np.uint16)
    x = np.ascontiguousarray(x, np.uint16)
    assert w.shape == x.shape and w.size % 8 == 0
    return float(lib().or_dot_dev(_p(w), _p(x), w.size, int(team)))


def acc_step(acc, a, b):
    """acc + sum a_i b_i (bf16 bit patterns, 1..32 of them) as one accumulation step of the
    device's dot (2 products) or matrix (8 products) instruction."""
    a = np.ascontiguousarray(a, np.uint16)
    b = np.ascontiguousarray(b, np.uint16)
    assert a.shape == b.shape and 1 <= a.size <= 32
    return float(lib().or_acc_step(float(np.float32(acc)), _p(a), _p(b), a.size))


def dot2_batch(a, b, c):
    """or_acc_step over many v_dot2c_f32_bf16 tuples: a, b u32 bf16 pairs, c f32 -> f32."""
    a = np.ascontiguousarray(a, np.uint32)
    b = np.ascontiguousarray(b, np.uint32)
    c = np.ascontiguousarray(c, np.float32)
    d = np.empty_like(c)
    lib().or_dot2_batch(_p(a), _p(b), _p(c), _p(d), c.size)
    return d


def mfma_batch(A, B, C):
    """D = C + A B per 16x32 / 32x16 tile as v_mfma_f32_16x16x32_bf16 accumulates it."""
    A = np.ascontiguousarray(A, np.uint16)
    B = np.ascontiguousarray(B, np.uint16)
    C = np.ascontiguousarray(C, np.float32)
    assert A.shape[1:] == (16, 32) and B.shape[1:] == (32, 16) and C.shape[1:] == (16, 16)
    D = np.empty_like(C)
    lib().or_mfma_batch(_p(A), _p(B), _p(C), _p(D), C.shape[0])
    return D


def dot_mfma(w, x, slices):
    w = np.ascontiguousarray(w, np.uint16)
    x = np.ascontiguousarray(x, np.uint16)
    assert w.shape == x.shape and w.size % (8 * slices) == 0
    return float(lib().or_dot_mfma(_p(w), _p(x), w.size, int(slices)))


def sumsq_dev(x):
    x = np.ascontiguousarray(x, np.uint16)
    assert x.size % 8 == 0 and x.size <= 1024
    return float(lib().or_sumsq_dev(_p(x), x.size))


def get_threads():
    return lib().or_get_threads()


# ---- DiT flow head and aggregator ---------------------------------------------------

def dit_cfg(D=1024, heads=16, head_dim=64, ff=4096, eps=1e-6):
    return OrDitCfg(D, heads, head_dim, ff, eps)


class DitBlock:
    """numpy bf16 weights of one DiT block: dict with norm1, norm2, wq, wk, wv, wo, w1, w2 ([out, in]) and
    bq, bk, bv, bo, b1, b2."""

    def __init__(self, w):
        self.a = {k: _c(v, np.uint16) for k, v in w.items()}
        lin = {n: Linear(self.a[k]) for n, k in (("q", "wq"), ("k", "wk"), ("v", "wv"), ("o", "wo"),
                                                  ("ff1", "w1"), ("ff2", "w2"))}
        self.lin = lin
        self.c = OrDitBlock(_p(self.a["norm1"]), _p(self.a["norm2"]), lin["q"].c, lin["k"].c, lin["v"].c,
                            lin["o"].c, lin["ff1"].c, lin["ff2"].c,
                            *(_p(self.a[k]) for k in ("bq", "bk", "bv", "bo", "b1", "b2")))


def rotary_table(inv_freq, L):
    inv = _c(np.asarray(inv_freq, np.float32), np.float32)
    half = inv.size
    c = np.empty((L, half), np.float32)
    s = np.empty((L, half), np.float32)
    lib().or_rotary_table(_p(inv), half, L, _p(c), _p(s))
    return c, s


def rotary(x, L, heads, hd, cos_t, sin_t):
    x = np.array(x, dtype=np.uint16, copy=True, order="C")
    R = x.shape[0]
    lib().or_rotary(_p(x), R, L, heads, hd, _p(_c(cos_t, np.float32)), _p(_c(sin_t, np.float32)))
    return x


def dit_block_fwd(c, blk, x, B, L, cos_t, sin_t, trace=False):
    x = _c(x, np.uint16)
    R, D = B * L, c.D
    out = np.empty((R, D), np.uint16)
    tr, arrs = None, {}
    if trace:
        arrs = dict(qkv=np.empty((3, R, D), np.uint16), att=np.empty((R, D), np.uint16),
                    x1=np.empty((R, D), np.uint16), hh=np.empty((R, c.ff), np.uint16))
        tr = OrDitTrace(*(_p(arrs[k]) for k in ("qkv", "att", "x1", "hh")))
    lib().or_dit_block_fwd(ctypes.byref(c), ctypes.byref(blk.c), _p(x), B, L, _p(_c(cos_t, np.float32)),
                           _p(_c(sin_t, np.float32)), _p(out), ctypes.byref(tr) if tr is not None else None)
    return (out, arrs) if trace else out


def flow_schedule():
    t = np.empty(11, np.uint16)
    lib().or_flow_schedule(_p(t))
    dt = np.empty(10, np.uint16)
    sq = np.empty(10, np.uint16)
    lib().or_flow_steps(_p(t), _p(dt), _p(sq))
    return t, dt, sq


def t_freq():
    f = np.empty(128, np.float32)
    lib().or_t_freq(_p(f))
    return f


def timestep_embed(mlp0, b0, mlp2, b2, t_bf16):
    D = mlp0.N
    out = np.empty((2, D), np.uint16)
    fr = t_freq()
    lib().or_timestep_embed(ctypes.byref(mlp0.c), _p(_c(b0, np.uint16)), ctypes.byref(mlp2.c), _p(_c(b2, np.uint16)),
                            _p(fr), int(t_bf16), _p(out))
    return out


class CfmModel:
    """The flow head for the oracle: blocks (list of DitBlock), x_emb/c_emb/final (Linear) with biases,
    final_norm, the t_emb table [steps][2][D] and the schedule (dt, sq), rotary tables for L = 3."""

    def __init__(self, c, blocks, x_emb, bx, c_emb, bc, final_norm, final, bf, t_emb, dt, sq, cos_t, sin_t):
        self.keep = dict(bx=_c(bx, np.uint16), bc=_c(bc, np.uint16), fn=_c(final_norm, np.uint16),
                         bf=_c(bf, np.uint16), te=_c(t_emb, np.uint16), dt=_c(dt, np.uint16), sq=_c(sq, np.uint16),
                         cos=_c(cos_t, np.float32), sin=_c(sin_t, np.float32))
        self.blocks = blocks
        self.barr = (OrDitBlock * len(blocks))(*(b.c for b in blocks))
        self.lins = (x_emb, c_emb, final)
        k = self.keep
        self.c = OrCfmModel(c, len(blocks), ctypes.cast(self.barr, c_void_p), x_emb.c, _p(k["bx"]), c_emb.c,
                            _p(k["bc"]), _p(k["fn"]), final.c, _p(k["bf"]), _p(k["te"]), _p(k["dt"]), _p(k["sq"]),
                            _p(k["cos"]), _p(k["sin"]), int(k["dt"].size))
        self.latent = final.N


def cfm_rows(m, z, hist, y, step):
    rows = np.empty((6, m.c.c.D), np.uint16)
    lib().or_cfm_rows(ctypes.byref(m.c), _p(_c(z, np.uint16)), _p(_c(hist, np.uint16)), _p(_c(y, np.uint16)),
                      int(step), _p(rows))
    return rows


def cfm_final(m, h, L, y, sde, step, cfg, shift):
    out = np.empty(m.latent, np.uint16)
    lib().or_cfm_final(ctypes.byref(m.c), _p(_c(h, np.uint16)), L, _p(_c(y, np.uint16)),
                       _p(None if sde is None else _c(sde, np.uint16)), int(step), float(cfg), float(shift), _p(out))
    return out


def cfm_sample(m, z, hist, noise, sde, cfg, shift):
    out = np.empty(m.latent, np.uint16)
    steps = np.empty((m.c.steps, m.latent), np.uint16)
    lib().or_cfm_sample(ctypes.byref(m.c), _p(_c(z, np.uint16)), _p(_c(hist, np.uint16)), _p(_c(noise, np.uint16)),
                        _p(None if sde is None else _c(sde, np.uint16)), float(cfg), float(shift), _p(out),
                        _p(steps))
    return out, steps


class AggModel:
    def __init__(self, c, blocks, x_emb, bx, cls, final_norm, final, bf, cos_t, sin_t):
        self.keep = dict(bx=_c(bx, np.uint16), cls=_c(cls, np.uint16), fn=_c(final_norm, np.uint16),
                         bf=_c(bf, np.uint16), cos=_c(cos_t, np.float32), sin=_c(sin_t, np.float32))
        self.blocks = blocks
        self.barr = (OrDitBlock * len(blocks))(*(b.c for b in blocks))
        self.lins = (x_emb, final)
        k = self.keep
        self.c = OrAggModel(c, len(blocks), ctypes.cast(self.barr, c_void_p), x_emb.c, _p(k["bx"]), _p(k["cls"]),
                            _p(k["fn"]), final.c, _p(k["bf"]), _p(k["cos"]), _p(k["sin"]))
        self.out_dim = final.N


def aggregate(m, latent):
    out = np.empty(m.out_dim, np.uint16)
    lib().or_aggregate(ctypes.byref(m.c), _p(_c(latent, np.uint16)), _p(out))
    return out


def stop_prob(head, bias, z):
    return float(lib().or_stop_prob(ctypes.byref(head.c), _p(_c(bias, np.uint16)), _p(_c(z, np.uint16))))


# ---- adaLN flow head (config 4) ---------------------------------------------------------

def adaln_block_fwd(c, blk, mod, x, B, L, cos_t, sin_t, trace=False):
    """blk: DitBlock; mod [B][6D] bf16 modulation (shift_a, scale_a, gate_a, shift_m, scale_m, gate_m)."""
    x = _c(x, np.uint16)
    R, D = B * L, c.D
    out = np.empty((R, D), np.uint16)
    tr, arrs = None, {}
    if trace:
        arrs = dict(qkv=np.empty((3, R, D), np.uint16), att=np.empty((R, D), np.uint16),
                    x1=np.empty((R, D), np.uint16), hh=np.empty((R, c.ff), np.uint16))
        tr = OrDitTrace(*(_p(arrs[k]) for k in ("qkv", "att", "x1", "hh")))
    lib().or_adaln_block_fwd(ctypes.byref(c), ctypes.byref(blk.c), _p(_c(mod, np.uint16)), _p(x), B, L,
                             _p(_c(cos_t, np.float32)), _p(_c(sin_t, np.float32)), _p(out),
                             ctypes.byref(tr) if tr is not None else None)
    return (out, arrs) if trace else out


class AdalnModel:
    """The adaLN flow head for the oracle: blocks (list of (DitBlock, ada Linear, bada)), embedders, final
    layer with its adaLN linear, t_emb [steps][2][D], schedule, rotary tables for L = frames."""

    def __init__(self, c, blocks, x_emb, bx, c_emb, bc, final_norm, final, bf, final_ada, bfa, t_emb, dt, sq,
                 cos_t, sin_t, frames):
        self.keep = dict(bx=_c(bx, np.uint16), bc=_c(bc, np.uint16), fn=_c(final_norm, np.uint16),
                         bf=_c(bf, np.uint16), bfa=_c(bfa, np.uint16), te=_c(t_emb, np.uint16),
                         dt=_c(dt, np.uint16), sq=_c(sq, np.uint16), cos=_c(cos_t, np.float32),
                         sin=_c(sin_t, np.float32), bada=[_c(b[2], np.uint16) for b in blocks])
        self.blocks = blocks
        self.barr = (OrAdalnBlock * len(blocks))(*(OrAdalnBlock(b[0].c, b[1].c, _p(self.keep["bada"][i]))
                                                  for i, b in enumerate(blocks)))
        self.lins = (x_emb, c_emb, final, final_ada)
        k = self.keep
        self.c = OrAdalnModel(c, len(blocks), ctypes.cast(self.barr, c_void_p), x_emb.c, _p(k["bx"]), c_emb.c,
                              _p(k["bc"]), _p(k["fn"]), final.c, _p(k["bf"]), final_ada.c, _p(k["bfa"]), _p(k["te"]),
                              _p(k["dt"]), _p(k["sq"]), _p(k["cos"]), _p(k["sin"]), int(k["dt"].size), int(frames))
        self.frames, self.latent, self.D = int(frames), final.N, c.D


def adaln_cond(m, z):
    out = np.empty((m.c.steps, 2, m.D), np.uint16)
    lib().or_adaln_cond(ctypes.byref(m.c), _p(_c(z, np.uint16)), _p(out))
    return out


def adaln_mods(m, silu_c):
    rows = 2 * m.c.steps
    mods = np.empty((len(m.blocks), rows, 6 * m.D), np.uint16)
    modf = np.empty((rows, 2 * m.D), np.uint16)
    lib().or_adaln_mods(ctypes.byref(m.c), _p(_c(silu_c, np.uint16)), _p(mods), _p(modf))
    return mods, modf


def adaln_rows(m, y):
    rows = np.empty((2 * m.frames, m.D), np.uint16)
    lib().or_adaln_rows(ctypes.byref(m.c), _p(_c(y, np.uint16)), _p(rows))
    return rows


def adaln_final(m, h, modf_step, y, sde, step, cfg, shift):
    out = np.empty((m.frames, m.latent), np.uint16)
    lib().or_adaln_final(ctypes.byref(m.c), _p(_c(h, np.uint16)), _p(_c(modf_step, np.uint16)), _p(_c(y, np.uint16)),
                         _p(None if sde is None else _c(sde, np.uint16)), int(step), float(cfg), float(shift), _p(out))
    return out


def adaln_sample(m, z, noise, sde, cfg, shift):
    out = np.empty((m.frames, m.latent), np.uint16)
    steps = np.empty((m.c.steps, m.frames, m.latent), np.uint16)
    lib().or_adaln_sample(ctypes.byref(m.c), _p(_c(z, np.uint16)), _p(_c(noise, np.uint16)),
                          _p(None if sde is None else _c(sde, np.uint16)), float(cfg), float(shift), _p(out),
                          _p(steps))
    return out, steps


# ---- VAE decoder (oracle_vae.c) -----------------------------------------------

def vae_cfg(hidden=896, heads=14, kv_heads=2, head_dim=64, inter=4864, n_layers=24, eps=1e-6, theta=1e6,
            window=64, latent=64, patch=4, n_fft=3528, hop=882):
    return OrVaeCfg(hidden, heads, kv_heads, head_dim, inter, n_layers, eps, float(np.log2(np.float32(theta))),
                    window, latent, patch, n_fft, hop)


def linear_f32(L, x, bias=None):
    x = _c(x, np.float32)
    M = x.size // L.K
    y = np.empty((M, L.N), np.float32)
    lib().or_linear_f32(ctypes.byref(L.c), _p(x), M, _p(None if bias is None else _c(bias, np.uint16)), _p(y))
    return y.reshape(x.shape[:-1] + (L.N,))


def rms_f32(x, w, eps=1e-6):
    x, w = _c(x, np.float32), _c(w, np.uint16)
    out = np.empty_like(x)
    lib().or_rms_f32(_p(x), _p(w), x.size // w.size, w.size, eps, _p(out))
    return out


def rope_f32(x, pos, log2_base):
    x = np.array(x, dtype=np.float32, copy=True, order="C")
    nh, hd = x.shape
    lib().or_rope_f32(_p(x), nh, hd, int(pos), float(log2_base))
    return x


def linear_upsample(x, scale):
    """bf16 [T, C] -> f32 [T*scale, C]."""
    x = _c(x, np.uint16)
    T, C = x.shape
    y = np.empty((T * scale, C), np.float32)
    lib().or_linear_upsample(_p(x), T, C, int(scale), _p(y))
    return y


def window_attention(q, k, v, window, scale=None):
    """q [F, heads, hd], k/v [F, kv_heads, hd] f32 -> [F, heads, hd]."""
    q, k, v = _c(q, np.float32), _c(k, np.float32), _c(v, np.float32)
    F, heads, hd = q.shape
    out = np.empty_like(q)
    lib().or_window_attention(_p(q), _p(k), _p(v), F, heads, k.shape[1], hd, int(window),
                              float(scale if scale is not None else 1.0 / np.sqrt(np.float32(hd))), _p(out))
    return out


def vae_layer(c, layer, x, trace=False):
    """One backbone layer over F rows: x f32 [F, hidden] -> f32 [F, hidden]."""
    x = _c(x, np.float32)
    F = x.shape[0]
    out = np.empty_like(x)
    arrs, tr = {}, None
    if trace:
        kvd = c.kv_heads * c.head_dim
        arrs = dict(qkv=np.empty((F, c.hidden + 2 * kvd), np.float32), att=np.empty((F, c.hidden), np.float32),
                    x1=np.empty((F, c.hidden), np.float32), hh=np.empty((F, c.inter), np.float32))
        tr = OrVaeTrace(*(_p(arrs[k]) for k in ("qkv", "att", "x1", "hh")))
    lib().or_vae_layer(ctypes.byref(c), ctypes.byref(layer.c), _p(x), F, _p(out),
                       ctypes.byref(tr) if tr is not None else None)
    return (out, arrs) if trace else out


def vae_istft(p, n_fft, hop, win, frames=False):
    """p f32 [F, n_fft + 2] (log-magnitudes | phases) -> wave f32 [F * hop] (and the windowed frames)."""
    p, win = _c(p, np.float32), _c(win, np.float32)
    F = p.shape[0]
    wave = np.empty(F * hop, np.float32)
    fr = np.empty((F, n_fft), np.float32) if frames else None
    lib().or_vae_istft(_p(p), F, int(n_fft), int(hop), _p(win), _p(wave), _p(fr))
    return (wave, fr) if frames else wave


class VaeModel:
    """The VAE decoder's arrays (fc1, layers as LmLayer, final norm, head, window) and their OrVaeModel view."""

    def __init__(self, c, fc1, fc1_bias, layers, norm, head, head_bias, window_fn):
        self.keep = [None if fc1_bias is None else _c(fc1_bias, np.uint16), _c(norm, np.uint16),
                     None if head_bias is None else _c(head_bias, np.uint16), _c(window_fn, np.float32)]
        self.layers = layers
        self.fc1, self.head = fc1, head
        self.arr = (OrLmLayer * len(layers))(*(l.c for l in layers))
        self.c = OrVaeModel(c, fc1.c, _p(self.keep[0]), ctypes.cast(self.arr, c_void_p), _p(self.keep[1]), head.c,
                            _p(self.keep[2]), _p(self.keep[3]))
        self.cfg = c


def vae_decode(m, latents, trace=False):
    """latents bf16 [T, latent] -> wave f32 [T * patch * hop] (and the layer inputs xs
    [n_layers + 1, F, hidden] and the head output [F, n_fft + 2] when trace)."""
    latents = _c(latents, np.uint16)
    c = m.cfg
    T = latents.shape[0]
    F = T * c.patch
    wave = np.empty(F * c.hop, np.float32)
    xs = np.empty((c.n_layers + 1, F, c.hidden), np.float32) if trace else None
    ho = np.empty((F, c.n_fft + 2), np.float32) if trace else None
    lib().or_vae_decode(ctypes.byref(m.c), _p(latents), T, _p(wave), _p(xs), _p(ho))
    return (wave, xs, ho) if trace else wave
