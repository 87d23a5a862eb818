"""ctypes binding of libming_hip.so (include/ming_hip.h) for tests and benches.

The product is the C ABI; this module only declares its structs and
functions and converts torch device tensors into `ming_tensor` views.  It
raises when the library is missing: there is no fallback path.

Mirrors of the reference interface (sbusso/ming-tts-serve):
  Context.lm_layer      <- ming_fused.lmLayer      src/ming_fused.zig:597
  LmModel               <- QStack.fuse/decodeFused src/ming_model.zig:510-544
  Context.qgemv         <- mlx_quantized_matmul    src/mlx.zig:279
  Context.gather_qmm    <- mlx_gather_qmm          src/mlx.zig:282
  Context.quantize      <- mlx_quantize            src/mlx.zig:292
  Context.dequantize    <- mlx_dequantize          src/mlx.zig:288
  Context.dit_block     <- ming_fused.block        src/ming_fused.zig:523
  Context.dit_single    <- ming_fused.single       src/ming_fused.zig:542
  Context.cfm_embed     <- ming_fused.embed        src/ming_fused.zig:559
  Context.cfm_final     <- ming_fused.final        src/ming_fused.zig:565
  Context.stop_prob     <- stopProb                src/ming_model.zig:1033
  CfmModel.sample       <- cfmSample               src/ming_model.zig:1143
  AggModel.aggregate    <- aggregate               src/ming_model.zig:1154
  Context.sample_latents <- sampleLatents          src/ming_model.zig:1388
"""
import atexit
import ctypes
import os
import weakref

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libming_hip.so")

MING_OK = 0
MING_E_SHAPE = 1
MING_E_CTX_OVER_CAPACITY = 2
MING_E_HIP = 3
MING_E_NOT_INIT = 4
MING_E_ARG = 5
MING_E_UNSUPPORTED = 6
MING_E_TIMEOUT = 7

DT_BF16, DT_F32, DT_U32, DT_I32 = 1, 2, 3, 4
W_BF16, W_AFFINE = 0, 1
LM_AUTO, LM_KERNELS, LM_PERSISTENT, LM_PERSISTENT_DIRECT, LM_PERSISTENT_XCD = 0, 1, 2, 3, 4
CFM_AUTO, CFM_KERNELS, CFM_PERSISTENT = 0, 1, 2

c_void_p = ctypes.c_void_p
c_i32 = ctypes.c_int32
c_i64 = ctypes.c_int64
c_f32 = ctypes.c_float


class Tensor(ctypes.Structure):
    _fields_ = [("data", c_void_p), ("dtype", c_i32), ("ndim", c_i32), ("shape", c_i64 * 4)]


class Linear(ctypes.Structure):
    _fields_ = [
        ("kind", c_i32), ("out_features", c_i32), ("in_features", c_i32), ("group_size", c_i32),
        ("bits", c_i32), ("global_scale", c_f32), ("w", c_void_p), ("scales", c_void_p), ("biases", c_void_p),
    ]


class LmCfg(ctypes.Structure):
    _fields_ = [
        ("hidden", c_i32), ("heads", c_i32), ("kv_heads", c_i32), ("head_dim", c_i32), ("inter", c_i32),
        ("vocab", c_i32), ("n_layers", c_i32), ("eps", c_f32), ("log2_theta", c_f32),
    ]


class LmLayerW(ctypes.Structure):
    _fields_ = [("ln1", c_void_p), ("ln2", c_void_p)] + [
        (n, Linear) for n in ("wq", "wk", "wv", "wo", "wg", "wu", "wd")
    ] + [("bq", c_void_p), ("bk", c_void_p), ("bv", c_void_p)]


class Kv(ctypes.Structure):
    _fields_ = [
        ("k", c_void_p), ("v", c_void_p), ("n_layers", c_i32), ("kv_heads", c_i32), ("head_dim", c_i32),
        ("capacity", c_i32), ("len", c_i32),
    ]


class KvPages(ctypes.Structure):
    """ming_kv_pages: paged cache of 64-position pages (V pages transposed)."""
    _fields_ = [
        ("k", c_void_p), ("v", c_void_p), ("n_layers", c_i32), ("kv_heads", c_i32), ("head_dim", c_i32),
        ("page_size", c_i32), ("n_pages", c_i32),
    ]


class LmOut(ctypes.Structure):
    _fields_ = [("qkv", c_void_p), ("o", c_void_p), ("x1", c_void_p), ("hh", c_void_p), ("x2", c_void_p)]


class DitCfg(ctypes.Structure):
    _fields_ = [("hidden", c_i32), ("heads", c_i32), ("head_dim", c_i32), ("ff", c_i32), ("eps", c_f32)]


class DitBlockW(ctypes.Structure):
    _fields_ = [("norm1", c_void_p), ("norm2", c_void_p)] + [
        (n, Linear) for n in ("wq", "wk", "wv", "wo", "w1", "w2")
    ] + [(n, c_void_p) for n in ("bq", "bk", "bv", "bo", "b1", "b2")]


class DitOut(ctypes.Structure):
    _fields_ = [(n, c_void_p) for n in ("qkv", "att", "x1", "hh", "x2")]


class CfmW(ctypes.Structure):
    _fields_ = [("cfg", DitCfg), ("n_blocks", c_i32), ("blocks", c_void_p), ("inv_freq", c_void_p)] + [
        (n, Linear) for n in ("x_emb", "c_emb", "t_mlp0", "t_mlp2", "final")
    ] + [(n, c_void_p) for n in ("bx", "bc", "bt0", "bt2", "final_norm", "bf")]


class AggW(ctypes.Structure):
    _fields_ = [("cfg", DitCfg), ("n_blocks", c_i32), ("blocks", c_void_p), ("inv_freq", c_void_p)] + [
        (n, Linear) for n in ("x_emb", "final")
    ] + [(n, c_void_p) for n in ("bx", "cls", "final_norm", "bf")]


class VaeCfg(ctypes.Structure):
    _fields_ = [(n, c_i32) for n in ("hidden", "heads", "kv_heads", "head_dim", "inter", "n_layers")] + [
        ("eps", c_f32), ("log2_theta", c_f32)] + [(n, c_i32) for n in ("window", "latent", "patch", "n_fft", "hop")]


class VaeW(ctypes.Structure):
    _fields_ = [("fc1", Linear), ("fc1_bias", c_void_p), ("layers", c_void_p), ("norm", c_void_p), ("head", Linear),
                ("head_bias", c_void_p), ("window", c_void_p)]


class AdalnBlockW(ctypes.Structure):
    _fields_ = [("base", DitBlockW), ("ada", Linear), ("bada", c_void_p)]


class AdalnW(ctypes.Structure):
    _fields_ = [("cfg", DitCfg), ("n_blocks", c_i32), ("frames", c_i32), ("blocks", c_void_p),
                ("inv_freq", c_void_p)] + [
        (n, Linear) for n in ("x_emb", "c_emb", "t_mlp0", "t_mlp2", "final", "final_ada")
    ] + [(n, c_void_p) for n in ("bx", "bc", "bt0", "bt2", "final_norm", "bf", "bfa")]


class SampleParams(ctypes.Structure):
    _fields_ = [("max_steps", c_i32), ("cfg", c_f32), ("sigma", c_f32), ("temperature", c_f32)]


_lib = None


def lib():
    """Load libming_hip.so once (raises OSError if it is not built)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise OSError(f"{LIB_PATH} is not built (run __graft_entry__.build())")
    L = ctypes.CDLL(LIB_PATH)
    P = ctypes.POINTER
    sig = {
        "ming_ctx_create": (c_i32, [P(c_void_p), c_i32]),
        "ming_ctx_destroy": (c_i32, [c_void_p]),
        "ming_ctx_set_stream": (c_i32, [c_void_p, c_void_p]),
        "ming_ctx_use_own_stream": (c_i32, [c_void_p]),
        "ming_ctx_set_exclusive": (c_i32, [c_void_p, c_i32]),
        "ming_ctx_workspace_bytes": (c_i32, [c_void_p, P(ctypes.c_int64)]),
        "ming_ctx_stream": (c_void_p, [c_void_p]),
        "ming_sync": (c_i32, [c_void_p]),
        "ming_last_error": (ctypes.c_char_p, [c_void_p]),
        "ming_status_str": (ctypes.c_char_p, [c_i32]),
        "ming_fused_enabled": (c_i32, []),
        "ming_dit_enabled": (c_i32, []),
        "ming_lm_enabled": (c_i32, []),
        "ming_set_force_off": (None, [c_i32]),
        "ming_malloc": (c_i32, [c_void_p, ctypes.c_size_t, P(c_void_p)]),
        "ming_free": (c_i32, [c_void_p, c_void_p]),
        "ming_memcpy_htod": (c_i32, [c_void_p, c_void_p, c_void_p, ctypes.c_size_t]),
        "ming_memcpy_dtoh": (c_i32, [c_void_p, c_void_p, c_void_p, ctypes.c_size_t]),
        "ming_memset": (c_i32, [c_void_p, c_void_p, c_i32, ctypes.c_size_t]),
        "ming_qgemv": (c_i32, [c_void_p, P(Tensor), P(Tensor), P(Tensor), P(Tensor), c_f32, c_i32, c_i32, P(Tensor)]),
        "ming_qgemv_f32": (c_i32, [c_void_p, P(Tensor), P(Tensor), P(Tensor), P(Tensor), c_f32, c_i32, c_i32,
                                   P(Tensor)]),
        "ming_qgemm": (c_i32, [c_void_p, P(Tensor), P(Tensor), P(Tensor), P(Tensor), c_f32, c_i32, c_i32, P(Tensor)]),
        "ming_qgemm_noalloc": (c_i32, [c_void_p, P(Tensor), P(Tensor), P(Tensor), P(Tensor), c_f32, c_i32, c_i32,
                                       P(Tensor)]),
        "ming_gather_qmm": (c_i32, [c_void_p, P(Tensor), P(Tensor), P(Tensor), P(Tensor), P(Tensor), P(Tensor), c_i32,
                                    c_i32, c_i32, c_f32, c_i32, P(Tensor)]),
        "ming_dequantize": (c_i32, [c_void_p, P(Tensor), P(Tensor), P(Tensor), c_i32, c_i32, c_f32, P(Tensor)]),
        "ming_quantize": (c_i32, [c_void_p, P(Tensor), c_i32, c_i32, c_f32, P(Tensor), P(Tensor), P(Tensor)]),
        "ming_lm_layer": (c_i32, [c_void_p, P(LmCfg), P(LmLayerW), c_void_p, c_i32, P(Kv), c_i32, P(LmOut)]),
        "ming_lm_model_create": (c_i32, [c_void_p, P(LmCfg), P(LmLayerW), c_void_p, P(Linear), P(Linear),
                                         P(c_void_p)]),
        "ming_lm_model_destroy": (c_i32, [c_void_p]),
        "ming_lm_model_set_mode": (c_i32, [c_void_p, c_i32]),
        "ming_cfm_model_set_mode": (c_i32, [c_void_p, c_i32]),
        "ming_cfm_model_profile": (c_i32, [c_void_p, c_void_p]),
        "ming_lm_model_profile": (c_i32, [c_void_p, c_void_p]),
        "ming_lm_model_profile_shape": (c_i32, [c_void_p, P(c_i32), P(c_i32)]),
        "ming_lm_step": (c_i32, [c_void_p, c_void_p, c_void_p, c_void_p, P(Kv), c_void_p, c_void_p, c_void_p]),
        "ming_lm_generate": (c_i32, [c_void_p, c_void_p, P(Kv), c_i32, c_void_p]),
        "ming_lm_model_trace": (c_i32, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p]),
        "ming_lm_batch_create": (c_i32, [c_void_p, c_void_p, c_i32, c_i32, P(c_void_p)]),
        "ming_lm_batch_destroy": (c_i32, [c_void_p]),
        "ming_lm_batch_step": (c_i32, [c_void_p, c_i32, c_void_p, c_void_p, P(KvPages), c_void_p, c_i32, c_void_p,
                                       c_void_p, c_void_p, c_void_p]),
        "ming_lm_batch_trace": (c_i32, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p]),
        "ming_st_open": (c_i32, [ctypes.c_char_p, P(c_void_p), ctypes.c_char_p, ctypes.c_size_t]),
        "ming_st_close": (c_i32, [c_void_p]),
        "ming_st_count": (c_i32, [c_void_p]),
        "ming_st_entry": (c_i32, [c_void_p, c_i32, P(ctypes.c_char_p), P(c_i32), P(c_i32), P(ctypes.c_int64),
                                  P(ctypes.c_uint64), P(ctypes.c_uint64)]),
        "ming_st_find": (c_i32, [c_void_p, ctypes.c_char_p]),
        "ming_weights_load": (c_i32, [c_void_p, ctypes.c_char_p, c_void_p, c_i32, P(c_void_p)]),
        "ming_weights_destroy": (c_i32, [c_void_p]),
        "ming_weights_get": (c_i32, [c_void_p, ctypes.c_char_p, P(Tensor)]),
        "ming_weights_linear": (c_i32, [c_void_p, ctypes.c_char_p, c_i32, c_i32, c_i32, P(Linear)]),
        "ming_lm_model_from_weights": (c_i32, [c_void_p, c_void_p, P(LmCfg), c_i32, P(c_void_p)]),
        "ming_cfm_model_from_weights": (c_i32, [c_void_p, c_void_p, P(DitCfg), c_i32, c_i32, c_i32, P(c_void_p)]),
        "ming_agg_model_from_weights": (c_i32, [c_void_p, c_void_p, P(DitCfg), c_i32, c_i32, c_i32, P(c_void_p)]),
        "ming_vae_model_from_weights": (c_i32, [c_void_p, c_void_p, P(VaeCfg), c_i32, c_i32, P(c_void_p)]),
        "ming_vae_model_create": (c_i32, [c_void_p, P(VaeCfg), P(VaeW), c_i32, P(c_void_p)]),
        "ming_vae_model_destroy": (c_i32, [c_void_p]),
        "ming_vae_decode": (c_i32, [c_void_p, c_void_p, c_i32, c_void_p, c_void_p]),
        "ming_vae_trace": (c_i32, [c_void_p, c_void_p, c_void_p]),
        "ming_lm_prefill": (c_i32, [c_void_p, c_i32, c_void_p, c_void_p, P(KvPages), c_void_p, c_i32, c_i32,
                                    c_void_p, c_void_p, c_void_p]),
        "ming_rotary_table": (c_i32, [c_void_p, c_void_p, c_i32, c_i32, c_void_p, c_void_p]),
        "ming_dit_block": (c_i32, [c_void_p, P(DitCfg), P(DitBlockW), c_void_p, c_i32, c_i32, c_void_p, c_void_p,
                                   P(DitOut)]),
        "ming_dit_single": (c_i32, [c_void_p, c_i32, P(DitCfg), P(DitBlockW), c_void_p, c_void_p, c_i32, c_i32,
                                    c_void_p, c_void_p, c_void_p, c_void_p]),
        "ming_cfm_embed": (c_i32, [c_void_p, c_void_p, P(Linear), c_void_p, c_void_p, c_void_p, c_void_p, c_void_p]),
        "ming_cfm_final": (c_i32, [c_void_p, c_void_p, c_i32, c_void_p, P(Linear), c_void_p, c_void_p, c_void_p,
                                   c_void_p, c_void_p, c_i32, c_f32, c_f32, c_void_p]),
        "ming_cfm_model_create": (c_i32, [c_void_p, P(CfmW), P(c_void_p)]),
        "ming_cfm_sample_batch": (c_i32, [c_void_p, c_void_p, c_i32, c_void_p, c_void_p, c_void_p, c_void_p, c_f32, c_f32,
                                          c_f32, c_void_p, c_void_p]),
        "ming_cfm_model_destroy": (c_i32, [c_void_p]),
        "ming_cfm_model_tables": (c_i32, [c_void_p, c_void_p, c_void_p, c_void_p, P(c_void_p)]),
        "ming_cfm_sample": (c_i32, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_f32, c_f32, c_f32,
                                    c_void_p, c_void_p]),
        "ming_agg_model_create": (c_i32, [c_void_p, P(AggW), P(c_void_p)]),
        "ming_agg_model_destroy": (c_i32, [c_void_p]),
        "ming_aggregate": (c_i32, [c_void_p, c_void_p, c_void_p, c_void_p]),
        "ming_aggregate_trace": (c_i32, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p]),
        "ming_stop_prob": (c_i32, [c_void_p, P(Linear), c_void_p, c_void_p, c_void_p]),
        "ming_adaln_block": (c_i32, [c_void_p, P(DitCfg), P(AdalnBlockW), c_void_p, c_void_p, c_i32, c_i32, c_void_p,
                                     c_void_p, P(DitOut)]),
        "ming_adaln_model_create": (c_i32, [c_void_p, P(AdalnW), P(c_void_p)]),
        "ming_adaln_model_destroy": (c_i32, [c_void_p]),
        "ming_adaln_model_tables": (c_i32, [c_void_p, P(c_void_p), P(c_void_p), P(c_void_p), P(c_void_p)]),
        "ming_adaln_sample": (c_i32, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_f32, c_f32, c_f32,
                                      c_void_p, c_void_p]),
        "ming_lm_model_dims": (c_i32, [c_void_p, P(c_i32), P(c_i32)]),
        "ming_cfm_model_dims": (c_i32, [c_void_p, P(c_i32), P(c_i32)]),
        "ming_agg_model_dims": (c_i32, [c_void_p, P(c_i32), P(c_i32)]),
        "ming_noise_bank": (c_i32, [c_void_p, ctypes.c_uint64, c_i32, c_i32, c_void_p]),
        "ming_sample_latents": (c_i32, [c_void_p, c_void_p, c_void_p, c_void_p, P(Linear), c_void_p, c_void_p, c_i32,
                                        c_void_p, P(Kv), c_void_p, P(SampleParams), c_void_p, P(c_i32), c_void_p,
                                        c_void_p]),
        "ming_synth_stream": (ctypes.c_uint64, [ctypes.c_uint64, ctypes.c_char_p]),
        "ming_synth_normal_bf16": (None, [ctypes.c_uint64, c_f32, c_f32, c_void_p, ctypes.c_size_t, c_i32]),
        "ming_synth_uniform_i32": (None, [ctypes.c_uint64, c_i32, c_void_p, ctypes.c_size_t]),
    }
    for name, (res, args) in sig.items():
        f = getattr(L, name)
        f.restype = res
        f.argtypes = args
    _lib = L
    return L


def exported_symbols():
    """Names of every function the ctypes table declares (all must resolve)."""
    lib()
    return [n for n in dir(_lib) if n.startswith("ming_")]


# Handles still open at interpreter exit are destroyed here, newest first
# (models and batches before the context they were created on), while torch
# and the HIP runtime are still whole -- not by __del__ during finalization.
_open_handles = []


def _track(obj):
    _open_handles.append(weakref.ref(obj))


@atexit.register
def _close_open_handles():
    while _open_handles:
        obj = _open_handles.pop()()
        if obj is not None:
            try:
                obj.close()
            except Exception:
                pass


class MingError(RuntimeError):
    def __init__(self, status, msg):
        super().__init__(f"{lib().ming_status_str(status).decode()} ({status}): {msg}")
        self.status = status


# ---- torch helpers ----------------------------------------------------------


def _torch():
    import torch

    return torch


def tensor(t, dtype=None):
    """ming_tensor view of a contiguous torch tensor (u32 data travel as int32)."""
    torch = _torch()
    assert t.is_contiguous(), "ming tensors are row-major contiguous"
    if dtype is None:
        dtype = {torch.bfloat16: DT_BF16, torch.float32: DT_F32, torch.int32: DT_I32}[t.dtype]
    shape = list(t.shape)
    assert len(shape) <= 4
    return Tensor(t.data_ptr(), dtype, len(shape), (c_i64 * 4)(*(shape + [0] * (4 - len(shape)))))


def ptr(t):
    """Device address of a torch tensor (or an address given as an int)."""
    if t is None:
        return None
    return ctypes.c_void_p(t if isinstance(t, int) else t.data_ptr())


def linear(w, scales=None, biases=None, global_scale=1.0, out_features=None, in_features=None):
    """ming_linear from torch tensors: bf16 [N,K] or affine (int32 [N,K/8], bf16 scales/biases)."""
    if scales is None:
        n, k = w.shape
        return Linear(W_BF16, n, k, 0, 0, 1.0, w.data_ptr(), None, None)
    n = w.shape[0]
    k = w.shape[1] * 8
    return Linear(W_AFFINE, out_features or n, in_features or k, 64, 4, float(global_scale), w.data_ptr(),
                  scales.data_ptr(), biases.data_ptr())


class Context:
    """A ming_ctx bound to torch's current stream on `device`."""

    def __init__(self, device=0, use_torch_stream=True):
        L = lib()
        h = c_void_p()
        st = L.ming_ctx_create(ctypes.byref(h), device)
        if st:
            raise MingError(st, "ming_ctx_create failed")
        self.h = h
        self.L = L
        _track(self)
        if use_torch_stream:
            torch = _torch()
            self.set_stream(torch.cuda.current_stream(device).cuda_stream)

    def close(self):
        if self.h:
            self.L.ming_ctx_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def check(self, st):
        if st:
            raise MingError(st, self.L.ming_last_error(self.h).decode())

    def set_stream(self, s):
        self.check(self.L.ming_ctx_set_stream(self.h, c_void_p(s)))

    def set_exclusive(self, on=True):
        self.check(self.L.ming_ctx_set_exclusive(self.h, int(bool(on))))

    def workspace_bytes(self):
        """Device bytes of the context's on-demand workspaces (0 on a new context)."""
        v = ctypes.c_int64(0)
        self.check(self.L.ming_ctx_workspace_bytes(self.h, ctypes.byref(v)))
        return int(v.value)

    def sync(self):
        self.check(self.L.ming_sync(self.h))

    # ---- MLX-affine linear algebra ----
    def qgemv(self, x, w, scales, biases, y, global_scale=1.0, f32=False):
        f = self.L.ming_qgemv_f32 if f32 else self.L.ming_qgemv
        tx, tw, ts, tb, ty = tensor(x), tensor(w, DT_U32), tensor(scales), tensor(biases), tensor(y)
        self.check(f(self.h, ctypes.byref(tx), ctypes.byref(tw), ctypes.byref(ts), ctypes.byref(tb),
                     float(global_scale), 64, 4, ctypes.byref(ty)))

    def qgemm(self, x, w, scales, biases, y, global_scale=1.0):
        """Y [M, N] = g * X W^T on the matrix cores (M = 1..64); y bf16 or f32."""
        tx, tw, ts, tb, ty = tensor(x), tensor(w, DT_U32), tensor(scales), tensor(biases), tensor(y)
        self.check(self.L.ming_qgemm(self.h, ctypes.byref(tx), ctypes.byref(tw), ctypes.byref(ts), ctypes.byref(tb),
                                     float(global_scale), 64, 4, ctypes.byref(ty)))

    def qgemm_noalloc(self, x, w, scales, biases, y, global_scale=1.0):
        """ming_qgemm through the device's fixed scratch (no allocation; M <= 64, K <= 8192)."""
        tx, tw, ts, tb, ty = tensor(x), tensor(w, DT_U32), tensor(scales), tensor(biases), tensor(y)
        self.check(self.L.ming_qgemm_noalloc(self.h, ctypes.byref(tx), ctypes.byref(tw), ctypes.byref(ts),
                                             ctypes.byref(tb), float(global_scale), 64, 4, ctypes.byref(ty)))

    def gather_qmm(self, x, w, scales, biases, lhs, rhs, y, global_scale=1.0, sorted_indices=False):
        """mlx_gather_qmm: y[p] = g * x[lhs[p]] W[rhs[p]]^T (lhs may be None)."""
        tx, tw, ts, tb, ty = tensor(x), tensor(w, DT_U32), tensor(scales), tensor(biases), tensor(y)
        tr = tensor(rhs)
        tl = tensor(lhs) if lhs is not None else None
        self.check(self.L.ming_gather_qmm(self.h, ctypes.byref(tx), ctypes.byref(tw), ctypes.byref(ts),
                                          ctypes.byref(tb), ctypes.byref(tl) if tl is not None else None,
                                          ctypes.byref(tr), 1, 64, 4, float(global_scale), int(bool(sorted_indices)),
                                          ctypes.byref(ty)))

    def quantize(self, w, wq, scales, biases, global_scale=1.0):
        tw, tq, ts, tb = tensor(w), tensor(wq, DT_U32), tensor(scales), tensor(biases)
        self.check(self.L.ming_quantize(self.h, ctypes.byref(tw), 64, 4, float(global_scale), ctypes.byref(tq),
                                        ctypes.byref(ts), ctypes.byref(tb)))

    def dequantize(self, wq, scales, biases, out, global_scale=1.0):
        tq, ts, tb, to = tensor(wq, DT_U32), tensor(scales), tensor(biases), tensor(out)
        self.check(self.L.ming_dequantize(self.h, ctypes.byref(tq), ctypes.byref(ts), ctypes.byref(tb), 64, 4,
                                          float(global_scale), ctypes.byref(to)))

    # ---- Qwen2 decode ----
    def lm_layer(self, cfg, layer_w, x, pos, kv, layer, out):
        self.check(self.L.ming_lm_layer(self.h, ctypes.byref(cfg), ctypes.byref(layer_w), ptr(x), int(pos),
                                        ctypes.byref(kv), int(layer), ctypes.byref(out)))


    # ---- DiT flow head / aggregator pieces ----
    def rotary_table(self, inv_freq, L, cos, sin):
        """inv_freq: numpy f32 [half]; cos/sin: device f32 [L, half]."""
        import numpy as np

        inv = np.ascontiguousarray(inv_freq, dtype=np.float32)
        self.check(self.L.ming_rotary_table(self.h, inv.ctypes.data_as(c_void_p), inv.size, int(L), ptr(cos),
                                            ptr(sin)))

    def dit_block(self, cfg, w, x, B, L, cos, sin, out):
        self.check(self.L.ming_dit_block(self.h, ctypes.byref(cfg), ctypes.byref(w), ptr(x), int(B), int(L),
                                         ptr(cos), ptr(sin), ctypes.byref(out)))

    def dit_single(self, which, cfg, w, x, inp, B, L, cos, sin, qkv_tmp, out):
        self.check(self.L.ming_dit_single(self.h, int(which), ctypes.byref(cfg), ctypes.byref(w), ptr(x), ptr(inp),
                                          int(B), int(L), ptr(cos), ptr(sin), ptr(qkv_tmp), ptr(out)))

    def cfm_embed(self, y, x_emb, bx, te, ce, xh, h_out):
        self.check(self.L.ming_cfm_embed(self.h, ptr(y), ctypes.byref(x_emb), ptr(bx), ptr(te), ptr(ce), ptr(xh),
                                         ptr(h_out)))

    def cfm_final(self, h, L, norm, wf, bf, y, dt, sq, sde, step, cfg, shift, y_out):
        self.check(self.L.ming_cfm_final(self.h, ptr(h), int(L), ptr(norm), ctypes.byref(wf), ptr(bf), ptr(y),
                                         ptr(dt), ptr(sq), ptr(sde), int(step), float(cfg), float(shift),
                                         ptr(y_out)))

    def adaln_block(self, cfg, w, mod, x, B, L, cos, sin, out):
        self.check(self.L.ming_adaln_block(self.h, ctypes.byref(cfg), ctypes.byref(w), ptr(mod), ptr(x), int(B),
                                           int(L), ptr(cos), ptr(sin), ctypes.byref(out)))

    def stop_prob(self, head, bias, z, p):
        self.check(self.L.ming_stop_prob(self.h, ctypes.byref(head), ptr(bias), ptr(z), ptr(p)))


    # ---- per-token loop ----
    def noise_bank(self, seed, steps, latent, bank):
        self.check(self.L.ming_noise_bank(self.h, int(seed), int(steps), int(latent), ptr(bank)))

    def sample_latents(self, lm, cfm, agg, stop_head, stop_bias, embeds, kv, bank, params, latents_out,
                       prompt_latent=None, z_trace=None):
        """sampleLatents; returns (n_steps, [stop_k]).  embeds: device bf16 [L, hidden]."""
        n = c_i32()
        stops = (c_f32 * int(params.max_steps))()
        self.check(self.L.ming_sample_latents(self.h, lm.h, cfm.h, agg.h, ctypes.byref(stop_head), ptr(stop_bias),
                                              ptr(embeds), int(embeds.shape[0]), ptr(prompt_latent),
                                              ctypes.byref(kv), ptr(bank), ctypes.byref(params), ptr(latents_out),
                                              ctypes.byref(n), stops, ptr(z_trace)))
        return n.value, [stops[i] for i in range(n.value)]


class CfmModel:
    """ming_cfm_model: the flow head's load-time tables plus one sample's workspace."""

    @classmethod
    def wrap(cls, ctx, h, keep=None):
        """A model created by another entry point (the *_from_weights loaders)."""
        m = cls.__new__(cls)
        m.ctx, m.w, m.h = ctx, keep, h
        _track(m)
        return m

    def __init__(self, ctx, w):
        self.ctx, self.w = ctx, w  # w: CfmW (its blocks array and inv_freq must stay alive)
        h = c_void_p()
        ctx.check(ctx.L.ming_cfm_model_create(ctx.h, ctypes.byref(w), ctypes.byref(h)))
        self.h = h
        _track(self)

    def close(self):
        if self.h:
            self.ctx.L.ming_cfm_model_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def tables(self):
        """(t [11], dt [10], sq [10]) as numpy uint16 bf16 bits, and the t_emb device pointer."""
        import numpy as np

        t = np.empty(11, np.uint16)
        dt = np.empty(10, np.uint16)
        sq = np.empty(10, np.uint16)
        te = c_void_p()
        self.ctx.check(self.ctx.L.ming_cfm_model_tables(self.h, t.ctypes.data_as(c_void_p),
                                                        dt.ctypes.data_as(c_void_p), sq.ctypes.data_as(c_void_p),
                                                        ctypes.byref(te)))
        return t, dt, sq, te.value

    def sample_batch(self, n, z, hist, noise, sde, cfg, sigma, temperature, latents_out, y_steps=None):
        """ming_cfm_sample_batch: n sequences' flow head in one pass."""
        self.ctx.check(self.ctx.L.ming_cfm_sample_batch(self.ctx.h, self.h, int(n), ptr(z), ptr(hist), ptr(noise),
                                                        ptr(sde), float(cfg), float(sigma), float(temperature),
                                                        ptr(latents_out), ptr(y_steps)))

    def set_mode(self, mode):
        """ming_cfm_model_set_mode: CFM_AUTO, CFM_KERNELS or CFM_PERSISTENT."""
        self.ctx.check(self.ctx.L.ming_cfm_model_set_mode(self.h, int(mode)))

    def profile(self, stamps):
        """ming_cfm_model_profile: a device u64 tensor [4][steps * n_blocks * 4], or None."""
        self.ctx.check(self.ctx.L.ming_cfm_model_profile(self.h, ptr(stamps)))

    def sample(self, z, hist, noise, sde, cfg, sigma, temperature, latent_out, y_steps=None):
        self.ctx.check(self.ctx.L.ming_cfm_sample(self.ctx.h, self.h, ptr(z), ptr(hist), ptr(noise), ptr(sde),
                                                  float(cfg), float(sigma), float(temperature), ptr(latent_out),
                                                  ptr(y_steps)))


class AdalnModel:
    """ming_adaln_model: the adaLN flow head (config 4)."""

    def __init__(self, ctx, w):
        self.ctx, self.w = ctx, w
        h = c_void_p()
        ctx.check(ctx.L.ming_adaln_model_create(ctx.h, ctypes.byref(w), ctypes.byref(h)))
        self.h = h
        _track(self)

    def close(self):
        if self.h:
            self.ctx.L.ming_adaln_model_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def tables(self):
        """Device pointers: t_emb, silu(c), block modulations, final modulations."""
        ps = [c_void_p() for _ in range(4)]
        self.ctx.check(self.ctx.L.ming_adaln_model_tables(self.h, *(ctypes.byref(p) for p in ps)))
        return [p.value for p in ps]

    def sample(self, z, noise, sde, cfg, sigma, temperature, patch_out, y_steps=None):
        self.ctx.check(self.ctx.L.ming_adaln_sample(self.ctx.h, self.h, ptr(z), ptr(noise), ptr(sde), float(cfg),
                                                    float(sigma), float(temperature), ptr(patch_out), ptr(y_steps)))


class AggModel:
    """ming_agg_model: the aggregator's rotary table and workspace."""

    @classmethod
    def wrap(cls, ctx, h, keep=None):
        """A model created by another entry point (the *_from_weights loaders)."""
        m = cls.__new__(cls)
        m.ctx, m.w, m.h = ctx, keep, h
        _track(m)
        return m

    def __init__(self, ctx, w):
        self.ctx, self.w = ctx, w
        h = c_void_p()
        ctx.check(ctx.L.ming_agg_model_create(ctx.h, ctypes.byref(w), ctypes.byref(h)))
        self.h = h
        _track(self)

    def close(self):
        if self.h:
            self.ctx.L.ming_agg_model_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def aggregate(self, latent, out):
        self.ctx.check(self.ctx.L.ming_aggregate(self.ctx.h, self.h, ptr(latent), ptr(out)))

    def aggregate_trace(self, latent, rows_out, out):
        """aggregate, with rows_out (device bf16 [n_blocks + 1][2][hidden]) = each block's input rows
        and the stack output."""
        self.ctx.check(self.ctx.L.ming_aggregate_trace(self.ctx.h, self.h, ptr(latent), ptr(rows_out), ptr(out)))


class VaeModel:
    """ming_vae_model: the VAE decoder's irfft basis and workspace (up to max_latents per decode)."""

    @classmethod
    def wrap(cls, ctx, cfg, h, keep=None):
        m = cls.__new__(cls)
        m.ctx, m.cfg, m.w, m.h = ctx, cfg, keep, h
        _track(m)
        return m

    def __init__(self, ctx, cfg, w, max_latents):
        self.ctx, self.cfg, self.w = ctx, cfg, w
        h = c_void_p()
        ctx.check(ctx.L.ming_vae_model_create(ctx.h, ctypes.byref(cfg), ctypes.byref(w), int(max_latents),
                                              ctypes.byref(h)))
        self.h = h
        _track(self)

    def close(self):
        if self.h:
            self.ctx.L.ming_vae_model_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def decode(self, T, latents, wave):
        self.ctx.check(self.ctx.L.ming_vae_decode(self.ctx.h, self.h, int(T), ptr(latents), ptr(wave)))

    def trace(self, xs=None, head_out=None):
        self.ctx.check(self.ctx.L.ming_vae_trace(self.h, ptr(xs) if xs is not None else None,
                                                 ptr(head_out) if head_out is not None else None))


class LmModel:
    """ming_lm_model: prepared decode stack (QStack.fuse)."""

    @classmethod
    def wrap(cls, ctx, cfg, h):
        """A model created by another entry point (ming_lm_model_from_weights)."""
        m = cls.__new__(cls)
        m.ctx, m.cfg, m.h = ctx, cfg, h
        _track(m)
        return m

    def __init__(self, ctx, cfg, layers, final_norm, head, embed):
        self.ctx = ctx
        self.cfg = cfg
        self._layers = (LmLayerW * len(layers))(*layers)
        self._head = head
        self._embed = embed
        h = c_void_p()
        ctx.check(ctx.L.ming_lm_model_create(ctx.h, ctypes.byref(cfg), self._layers, ptr(final_norm),
                                             ctypes.byref(head), ctypes.byref(embed), ctypes.byref(h)))
        self.h = h
        _track(self)

    def close(self):
        if self.h:
            self.ctx.L.ming_lm_model_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def set_mode(self, mode):
        self.ctx.check(self.ctx.L.ming_lm_model_set_mode(self.h, int(mode)))

    def step(self, kv, token=None, x_in=None, hidden=None, logits=None, argmax=None):
        self.ctx.check(self.ctx.L.ming_lm_step(self.ctx.h, self.h, ptr(token), ptr(x_in), ctypes.byref(kv),
                                               ptr(hidden), ptr(logits), ptr(argmax)))

    def trace(self):
        """dict of per-layer activations of the last step (torch bf16 device tensors)."""
        torch = _torch()
        c = self.cfg
        H, L, nq = c.hidden, c.n_layers, c.hidden + 2 * c.kv_heads * c.head_dim
        t = dict(x=torch.empty((L + 1, H), dtype=torch.bfloat16, device="cuda"),
                 x1=torch.empty((L, H), dtype=torch.bfloat16, device="cuda"),
                 att=torch.empty((L, H), dtype=torch.bfloat16, device="cuda"),
                 qkv=torch.empty((L, nq), dtype=torch.bfloat16, device="cuda"),
                 hh=torch.empty((L, c.inter), dtype=torch.bfloat16, device="cuda"))
        self.ctx.check(self.ctx.L.ming_lm_model_trace(self.h, *(ptr(t[k]) for k in ("x", "x1", "att", "qkv", "hh"))))
        return t

    def generate(self, kv, n_steps, tokens):
        self.ctx.check(self.ctx.L.ming_lm_generate(self.ctx.h, self.h, ctypes.byref(kv), int(n_steps), ptr(tokens)))


class LmBatch:
    """ming_lm_batch: workspace of the multi-request decode step of an LmModel."""

    def __init__(self, model, max_seqs, max_ctx):
        self.ctx = model.ctx
        self.model = model
        self.max_seqs = int(max_seqs)
        h = c_void_p()
        self.ctx.check(self.ctx.L.ming_lm_batch_create(self.ctx.h, model.h, int(max_seqs), int(max_ctx),
                                                       ctypes.byref(h)))
        self.h = h
        _track(self)
        self.n = 0

    def close(self):
        if self.h:
            self.ctx.L.ming_lm_batch_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def step(self, pages, table, pos, tokens=None, x_in=None, hidden=None, logits=None, argmax=None):
        """One step of n = len(pos) sequences; table: device i32 [n][pages_per_seq]."""
        n, pps = int(table.shape[0]), int(table.shape[1])
        self.ctx.check(self.ctx.L.ming_lm_batch_step(self.h, n, ptr(tokens), ptr(x_in), ctypes.byref(pages.kv),
                                                     ptr(table), pps, ptr(pos), ptr(hidden), ptr(logits),
                                                     ptr(argmax)))
        self.n = n

    def prefill(self, pages, table_row, pos0, tokens=None, x_in=None, hidden=None, logits=None, argmax=None, L=None):
        """Causal prefill of one sequence: rows at positions pos0.. over its pages
        (table_row: device i32 [pages_per_seq])."""
        n = int(L if L is not None else (tokens.shape[0] if tokens is not None else x_in.shape[0]))
        self.ctx.check(self.ctx.L.ming_lm_prefill(self.h, n, ptr(tokens), ptr(x_in), ctypes.byref(pages.kv),
                                                  ptr(table_row), int(table_row.shape[-1]), int(pos0), ptr(hidden),
                                                  ptr(logits), ptr(argmax)))
        self.n = min(n, self.max_seqs) if n <= self.max_seqs else n - (n - 1) // self.max_seqs * self.max_seqs

    def trace(self):
        """dict of per-layer activations [layer][seq][...] of the last step (device bf16)."""
        torch = _torch()
        c, n = self.model.cfg, self.n
        H, L, nq = c.hidden, c.n_layers, c.hidden + 2 * c.kv_heads * c.head_dim
        t = dict(x=torch.empty((L + 1, n, H), dtype=torch.bfloat16, device="cuda"),
                 x1=torch.empty((L, n, H), dtype=torch.bfloat16, device="cuda"),
                 att=torch.empty((L, n, H), dtype=torch.bfloat16, device="cuda"),
                 qkv=torch.empty((L, n, nq), dtype=torch.bfloat16, device="cuda"),
                 hh=torch.empty((L, n, c.inter), dtype=torch.bfloat16, device="cuda"))
        self.ctx.check(self.ctx.L.ming_lm_batch_trace(self.h, *(ptr(t[k]) for k in ("x", "x1", "att", "qkv", "hh"))))
        return t


# ---- checkpoints ----------------------------------------------------------------

DTYPE_NAMES = {1: "BF16", 2: "F32", 3: "U32", 4: "I32", 5: "F16", 6: "I64", 7: "U8", 8: "F64", 9: "I8", 10: "BOOL",
               11: "I16", 12: "U16", 13: "U64"}


def st_index(path):
    """ming_st_*: the parsed header of a safetensors file as a list of dicts
    (name, dtype name, shape, absolute offset, nbytes); MingError on a bad file."""
    L = lib()
    h = c_void_p()
    err = ctypes.create_string_buffer(512)
    st = L.ming_st_open(str(path).encode(), ctypes.byref(h), err, len(err))
    if st:
        raise MingError(st, err.value.decode(errors="replace"))
    try:
        out = []
        for i in range(L.ming_st_count(h)):
            name, dt, nd = ctypes.c_char_p(), c_i32(), c_i32()
            shape = (ctypes.c_int64 * 8)()
            off, nb = ctypes.c_uint64(), ctypes.c_uint64()
            L.ming_st_entry(h, i, ctypes.byref(name), ctypes.byref(dt), ctypes.byref(nd), shape, ctypes.byref(off),
                            ctypes.byref(nb))
            out.append(dict(name=name.value.decode(), dtype=DTYPE_NAMES.get(dt.value, "?"),
                            shape=[shape[k] for k in range(nd.value)], offset=off.value, nbytes=nb.value))
        return out
    finally:
        L.ming_st_close(h)


class Weights:
    """ming_weights: a checkpoint's tensors on the device (Tensors.load)."""

    def __init__(self, ctx, path, prefixes=None):
        self.ctx = ctx
        h = c_void_p()
        pre = [p.encode() for p in (prefixes or [])]
        arr = (ctypes.c_char_p * max(1, len(pre)))(*pre)
        ctx.check(ctx.L.ming_weights_load(ctx.h, str(path).encode(), arr if pre else None, len(pre), ctypes.byref(h)))
        self.h = h
        _track(self)

    def close(self):
        if self.h:
            self.ctx.L.ming_weights_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def get(self, name):
        t = Tensor()
        if self.ctx.L.ming_weights_get(self.h, name.encode(), ctypes.byref(t)):
            raise KeyError(name)
        return t

    def linear(self, name, out_features, in_features, quantize=False):
        w = Linear()
        self.ctx.check(self.ctx.L.ming_weights_linear(self.h, name.encode(), int(out_features), int(in_features),
                                                      int(quantize), ctypes.byref(w)))
        return w

    def lm_model(self, cfg, quantize=True):
        h = c_void_p()
        self.ctx.check(self.ctx.L.ming_lm_model_from_weights(self.ctx.h, self.h, ctypes.byref(cfg), int(quantize),
                                                             ctypes.byref(h)))
        return LmModel.wrap(self.ctx, cfg, h)

    def cfm_model(self, cfg, n_blocks, lm_hidden, latent):
        h = c_void_p()
        self.ctx.check(self.ctx.L.ming_cfm_model_from_weights(self.ctx.h, self.h, ctypes.byref(cfg), int(n_blocks),
                                                              int(lm_hidden), int(latent), ctypes.byref(h)))
        return CfmModel.wrap(self.ctx, h, keep=self)

    def agg_model(self, cfg, n_blocks, lm_hidden, latent):
        h = c_void_p()
        self.ctx.check(self.ctx.L.ming_agg_model_from_weights(self.ctx.h, self.h, ctypes.byref(cfg), int(n_blocks),
                                                              int(lm_hidden), int(latent), ctypes.byref(h)))
        return AggModel.wrap(self.ctx, h, keep=self)

    def vae_model(self, cfg, max_latents, quantize=False):
        h = c_void_p()
        self.ctx.check(self.ctx.L.ming_vae_model_from_weights(self.ctx.h, self.h, ctypes.byref(cfg), int(quantize),
                                                              int(max_latents), ctypes.byref(h)))
        return VaeModel.wrap(self.ctx, cfg, h, keep=self)


# ---- synthetic inputs ---------------------------------------------------------


def synth_stream(seed, name):
    return lib().ming_synth_stream(int(seed), name.encode())


def synth_normal_bf16(seed, name, n, mean=0.0, std=1.0, threads=None):
    """numpy uint16 (bf16 bits) [n] of bf16(mean + std * N(0,1))."""
    import numpy as np

    out = np.empty(int(n), dtype=np.uint16)
    lib().ming_synth_normal_bf16(synth_stream(seed, name), float(mean), float(std),
                                 out.ctypes.data_as(c_void_p), out.size, int(threads or min(16, os.cpu_count() or 1)))
    return out


def synth_uniform_i32(seed, name, n, hi):
    import numpy as np

    out = np.empty(int(n), dtype=np.int32)
    lib().ming_synth_uniform_i32(synth_stream(seed, name), int(hi), out.ctypes.data_as(c_void_p), out.size)
    return out
