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
        "or_quantize": (c_int, [c_void_p, c_i64, c_i64, c_int, c_int, c_void_p, c_void_p, c_void_p]),
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

def quantize(w, group=64, bits=4):
    w = _c(w, np.uint16)
    N, K = w.shape
    wq = np.empty((N, K * bits // 32), np.uint32)
    s = np.empty((N, K // group), np.uint16)
    b = np.empty((N, K // group), np.uint16)
    assert lib().or_quantize(_p(w), N, K, group, bits, _p(wq), _p(s), _p(b)) == 0
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


def get_threads():
    return lib().or_get_threads()
