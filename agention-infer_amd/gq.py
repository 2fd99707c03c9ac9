"""Python mirror of gguf-rs's Backend boundary over libgq.so (ctypes).

Mirrors:
  trait Backend { fn name(&self); fn matmul_dequant(dtype, w, x, out) }
      src/ops/mod.rs:93-106                      -> HipBackend.name / .matmul_dequant
  WgpuBackend::upload_weight                      src/ops/wgpu_backend/mod.rs:61-92
      -> HipBackend.upload_weight -> GpuWeightHandle
  matmul_dequant_preloaded / _qkv / _multi / _ffn  wgpu_backend/mod.rs:642-854
  launch_only / launch_only_f32out / _batch        wgpu_backend/resident.rs:13-104
  GpuWeightHandle::shape / out_dim                 wgpu_backend/mod.rs:914-922
  create_backend(BackendPreference::Hip)           ops/backend_select.rs:60-108

Errors surface as GqError (the GgufError::BackendError channel).  There is no
CPU fallback: if libgq.so is missing or no gfx950 is present, calls raise.
Device buffers are torch tensors on `cuda` (PyTorch is plumbing here: it
owns device memory and streams; all compute runs in libgq.so).
"""
import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.environ.get("GQ_LIBRARY") or os.path.join(_HERE, "libgq.so")

GQ_GEMM_BF16 = 0
GQ_GEMM_INT8 = 1

# GgmlType ids (src/types.rs:9-46)
Q8_0, Q4_K, Q5_K, Q6_K, IQ3_XXS = 8, 12, 13, 14, 18
GPU_DEQUANT_DTYPES = (Q8_0, Q4_K, Q5_K, Q6_K)  # src/ops/mod.rs:27-28

# Every entry point declared in include/gq.h, with its ctypes signature.
_P, _I, _SZ = ctypes.c_void_p, ctypes.c_int, ctypes.c_size_t
SIGNATURES = {
    "gq_init": (_I, [_I]),
    "gq_backend_name": (ctypes.c_char_p, []),
    "gq_last_error": (ctypes.c_char_p, []),
    "gq_type_size": (_SZ, [_I, _SZ]),
    "gq_upload": (_I, [_I, _P, _SZ, _I, _I, ctypes.POINTER(_P)]),
    "gq_upload_device": (_I, [_I, _P, _SZ, _I, _I, ctypes.POINTER(_P)]),
    "gq_weight_free": (_I, [_P]),
    "gq_weight_shape": (_I, [_P, ctypes.POINTER(_I), ctypes.POINTER(_I), ctypes.POINTER(_I)]),
    "gq_weight_bytes": (_SZ, [_P]),
    "gq_matvec": (_I, [_P, _P, _P, _P]),
    "gq_matvec_multi": (_I, [ctypes.POINTER(_P), _I, _P, ctypes.POINTER(_P), _P]),
    "gq_matmul_dequant_preloaded": (_I, [_P, _P, _P]),
    "gq_matmul_dequant_host": (_I, [_I, _P, _SZ, _P, _SZ, _P, _SZ]),
    "gq_dequant_rows": (_I, [_P, _I, _I, _P, _P]),
    "gq_gemm": (_I, [_P, _P, _I, _P, _I, _P]),
    "gq_quantize_q8_32": (_I, [_P, _I, _P, _P, _P]),
    "gq_set_iq3xxs_grid": (_I, [_P]),
    "gq_get_iq3xxs_grid": (_I, [_P]),
    "gq_sync": (_I, [_P]),
    "gq_upload_experts": (_I, [_I, _P, _SZ, _I, _I, _I, ctypes.POINTER(_P)]),
    "gq_model_create": (_I, [_P, ctypes.POINTER(_P)]),
    "gq_model_free": (_I, [_P]),
    "gq_model_kv_upload": (_I, [_P, _I, _P, _P, _I]),
    "gq_model_kv_download": (_I, [_P, _I, _P, _P, _I]),
    "gq_model_decode": (_I, [_P, _I, _I, _P, ctypes.POINTER(_I)]),
    "gq_model_generate": (_I, [_P, _I, _I, _I, _P, _P]),
    "gq_moe_ffn": (_I, [_P, _P, _P, _I, _P, _I, _I, _P, _P, _P, _P, _P]),
}


class GqError(RuntimeError):
    def __init__(self, code, msg):
        super().__init__(f"gq error {code}: {msg}")
        self.code = code


_lib = None


def lib():
    """Load libgq.so (built by agention-infer_amd/build.py).  Raises if absent."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise GqError(-6, f"{LIB_PATH} not built; run __graft_entry__.build()")
        # Load torch (and with it torch's HIP runtime) first, so that libgq
        # binds to the same libamdhip64 instance instead of loading a second
        # HIP runtime into the process.
        import torch  # noqa: F401
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _lib = L
    return _lib


def _check(rc):
    if rc != 0:
        raise GqError(rc, lib().gq_last_error().decode())


def _ptr(a):
    """Device pointer of a torch tensor, or host pointer of a numpy array."""
    if a is None:
        return None
    if hasattr(a, "data_ptr"):
        return ctypes.c_void_p(a.data_ptr())
    return ctypes.c_void_p(a.ctypes.data)


def _stream(stream):
    if stream is None:
        import torch
        return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    return ctypes.c_void_p(stream)


def type_size(dtype, n):
    return lib().gq_type_size(dtype, n)


class GpuWeightHandle:
    """A weight tensor resident on the GPU (GpuWeightHandle)."""

    def __init__(self, handle, dtype, in_dim, out_dim):
        self._h = ctypes.c_void_p(handle)
        self.dtype, self.in_dim, self._out_dim = dtype, in_dim, out_dim

    def __del__(self):
        if getattr(self, "_h", None) is not None and _lib is not None:
            _lib.gq_weight_free(self._h)
            self._h = None

    def shape(self):
        return (self.dtype, self.in_dim)

    def out_dim(self):
        return self._out_dim

    def nbytes(self):
        return lib().gq_weight_bytes(self._h)

    # launch_only / launch_only_f32out: device in, device out, async
    def launch_only(self, x_dev, y_dev=None, stream=None):
        import torch
        if y_dev is None:
            y_dev = torch.empty(self._out_dim, dtype=torch.float32, device=x_dev.device)
        _check(lib().gq_matvec(self._h, _ptr(x_dev), _ptr(y_dev), _stream(stream)))
        return y_dev

    launch_only_f32out = launch_only

    def dequant_rows(self, row0, nrows, out_dev=None, stream=None):
        import torch
        if out_dev is None:
            out_dev = torch.empty((nrows, self.in_dim), dtype=torch.float32, device="cuda")
        _check(lib().gq_dequant_rows(self._h, row0, nrows, _ptr(out_dev), _stream(stream)))
        return out_dev

    # launch_only_batch: X [n][in_dim] -> Y [n][out_dim]
    def launch_only_batch(self, X_dev, mode=GQ_GEMM_BF16, Y_dev=None, stream=None):
        import torch
        n = X_dev.shape[0]
        if Y_dev is None:
            Y_dev = torch.empty((n, self._out_dim), dtype=torch.float32, device=X_dev.device)
        _check(lib().gq_gemm(self._h, _ptr(X_dev), n, _ptr(Y_dev), mode, _stream(stream)))
        return Y_dev


class HipBackend:
    """The HIP arm of AnyBackend (src/ops/backend_select.rs:25-56)."""

    def __init__(self, device=0):
        _check(lib().gq_init(device))

    def name(self):
        return lib().gq_backend_name().decode()

    def matmul_dequant(self, dtype, w, x, out):
        """Backend::matmul_dequant: w = whole tensor bytes (numpy uint8),
        x = float32[in_dim], out = float32[out_dim] (overwritten)."""
        w = np.ascontiguousarray(w, dtype=np.uint8)
        x = np.ascontiguousarray(x, dtype=np.float32)
        assert out.dtype == np.float32 and out.flags.c_contiguous
        _check(lib().gq_matmul_dequant_host(dtype, _ptr(w), w.nbytes, _ptr(x), x.size,
                                            _ptr(out), out.size))

    def upload_weight(self, dtype, w, in_dim, out_dim=None):
        """upload_weight: w is numpy uint8 (host) or a torch uint8 cuda tensor."""
        rb = type_size(dtype, in_dim)
        if out_dim is None:
            out_dim = (w.nbytes if hasattr(w, "nbytes") else w.numel()) // rb if rb else 0
        h = ctypes.c_void_p()
        if hasattr(w, "data_ptr"):
            _check(lib().gq_upload_device(dtype, _ptr(w), w.numel() * w.element_size(), in_dim,
                                          out_dim, ctypes.byref(h)))
        else:
            w = np.ascontiguousarray(w, dtype=np.uint8)
            _check(lib().gq_upload(dtype, _ptr(w), w.nbytes, in_dim, out_dim, ctypes.byref(h)))
        return GpuWeightHandle(h.value, dtype, in_dim, out_dim)

    def matmul_dequant_preloaded(self, handle, x, out):
        x = np.ascontiguousarray(x, dtype=np.float32)
        _check(lib().gq_matmul_dequant_preloaded(handle._h, _ptr(x), _ptr(out)))

    def matmul_dequant_multi(self, handles, x_dev, outs=None, stream=None):
        """_qkv / _multi / _ffn: weights sharing x, one launch (device in/out)."""
        import torch
        if outs is None:
            outs = [torch.empty(h.out_dim(), dtype=torch.float32, device=x_dev.device)
                    for h in handles]
        hs = (ctypes.c_void_p * len(handles))(*[h._h.value for h in handles])
        ys = (ctypes.c_void_p * len(outs))(*[o.data_ptr() for o in outs])
        _check(lib().gq_matvec_multi(hs, len(handles), _ptr(x_dev), ys, _stream(stream)))
        return outs

    matmul_dequant_qkv = matmul_dequant_multi
    matmul_dequant_ffn = matmul_dequant_multi

    def quantize_q8_32(self, x_dev, stream=None):
        import torch
        n = x_dev.numel()
        scale = torch.empty(n // 32, dtype=torch.int16, device=x_dev.device)
        q = torch.empty(n, dtype=torch.int8, device=x_dev.device)
        _check(lib().gq_quantize_q8_32(_ptr(x_dev), n, _ptr(scale), _ptr(q), _stream(stream)))
        return scale, q

    def upload_experts(self, dtype, w, in_dim, rows_per_expert, n_experts):
        """A stacked expert tensor [n_experts][rows_per_expert][in_dim]."""
        w = np.ascontiguousarray(w, dtype=np.uint8)
        h = ctypes.c_void_p()
        _check(lib().gq_upload_experts(dtype, _ptr(w), w.nbytes, in_dim, rows_per_expert,
                                       n_experts, ctypes.byref(h)))
        return GpuWeightHandle(h.value, dtype, in_dim, rows_per_expert * n_experts)

    def moe_ffn(self, gate, up, down, n_experts, logits_dev, x_dev, top_k, out_dev=None,
                want_routing=False, stream=None):
        """MoE expert FFN for T tokens; returns out [T][h] (and ids, w)."""
        import torch
        T, h = x_dev.shape
        if out_dev is None:
            out_dev = torch.empty((T, h), dtype=torch.float32, device=x_dev.device)
        ids = torch.empty((T, top_k), dtype=torch.int32, device=x_dev.device) if want_routing else None
        w = torch.empty((T, top_k), dtype=torch.float32, device=x_dev.device) if want_routing else None
        _check(lib().gq_moe_ffn(gate._h, up._h, down._h, n_experts, _ptr(logits_dev), T, top_k,
                                _ptr(x_dev), _ptr(out_dev), _ptr(ids), _ptr(w), _stream(stream)))
        return (out_dev, ids, w) if want_routing else out_dev

    def set_iq3xxs_grid(self, grid=None):
        if grid is None:
            _check(lib().gq_set_iq3xxs_grid(None))
        else:
            g = np.ascontiguousarray(grid, dtype=np.uint32)
            assert g.size == 256
            _check(lib().gq_set_iq3xxs_grid(_ptr(g)))

    def get_iq3xxs_grid(self):
        g = np.zeros(256, np.uint32)
        _check(lib().gq_get_iq3xxs_grid(_ptr(g)))
        return g

    def sync(self, stream=None):
        _check(lib().gq_sync(_stream(stream)))


class _ModelDesc(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int) for n in ("n_layers", "hidden", "n_heads", "n_kv_heads",
                                             "head_dim", "ffn", "vocab", "ctx", "max_tokens")] + \
        [("eps", ctypes.c_float), ("theta", ctypes.c_float)] + \
        [(n, ctypes.c_void_p) for n in ("wq", "wk", "wv", "wo", "wgate", "wup", "wdown",
                                         "lm_head", "attn_norm", "ffn_norm", "output_norm",
                                         "embd")]


class DecodeModel:
    """GPU-resident dense decoder (run_gpu_resident, gpu_resident.rs:427-697).

    weights: dict with per-layer lists of GpuWeightHandle ("wq", "wk", "wv",
    "wo", "wgate", "wup", "wdown"), "lm_head", host float32 arrays
    "attn_norm"/"ffn_norm" ([n_layers][hidden]), "output_norm", "embd".
    """

    def __init__(self, cfg, weights):
        self._keep = []
        d = _ModelDesc()
        for k in ("n_layers", "hidden", "n_heads", "n_kv_heads", "head_dim", "ffn", "vocab",
                  "ctx"):
            setattr(d, k, int(cfg[k]))
        d.max_tokens = int(cfg.get("max_tokens", 4096))
        d.eps, d.theta = float(cfg["eps"]), float(cfg["theta"])
        L = cfg["n_layers"]
        for k in ("wq", "wk", "wv", "wo", "wgate", "wup", "wdown"):
            arr = (ctypes.c_void_p * L)(*[h._h.value for h in weights[k]])
            self._keep.append(arr)
            setattr(d, k, ctypes.cast(arr, ctypes.c_void_p))
        d.lm_head = weights["lm_head"]._h.value
        for k in ("attn_norm", "ffn_norm"):
            rows = [np.ascontiguousarray(r, np.float32) for r in weights[k]]
            self._keep.extend(rows)
            arr = (ctypes.c_void_p * L)(*[r.ctypes.data for r in rows])
            self._keep.append(arr)
            setattr(d, k, ctypes.cast(arr, ctypes.c_void_p))
        for k in ("output_norm", "embd"):
            a = np.ascontiguousarray(weights[k], np.float32)
            self._keep.append(a)
            setattr(d, k, a.ctypes.data)
        self._weights = weights  # handles must outlive the model
        self.cfg = cfg
        h = ctypes.c_void_p()
        _check(lib().gq_model_create(ctypes.byref(d), ctypes.byref(h)))
        self._h = h
        self._keep = None  # the library copied norms and embedding

    def __del__(self):
        if getattr(self, "_h", None) is not None and _lib is not None:
            _lib.gq_model_free(self._h)
            self._h = None

    def kv_upload(self, layer, k_f16, v_f16):
        k = np.ascontiguousarray(k_f16, np.uint16)
        v = np.ascontiguousarray(v_f16, np.uint16)
        _check(lib().gq_model_kv_upload(self._h, layer, _ptr(k), _ptr(v), k.shape[0]))

    def kv_download(self, layer, n_pos):
        kvd = self.cfg["n_kv_heads"] * self.cfg["head_dim"]
        k = np.zeros((n_pos, kvd), np.uint16)
        v = np.zeros((n_pos, kvd), np.uint16)
        _check(lib().gq_model_kv_download(self._h, layer, _ptr(k), _ptr(v), n_pos))
        return k, v

    def decode(self, token, pos, want_logits=True):
        """One step (Model::forward): returns (next_token, logits or None)."""
        logits = np.zeros(self.cfg["vocab"], np.float32) if want_logits else None
        nxt = ctypes.c_int()
        _check(lib().gq_model_decode(self._h, token, pos, _ptr(logits), ctypes.byref(nxt)))
        return nxt.value, logits

    def generate(self, token, pos, n_steps, stream=None):
        """n_steps greedy steps (one HIP graph replay each); returns the tokens."""
        out = np.zeros(n_steps, np.int32)
        _check(lib().gq_model_generate(self._h, token, pos, n_steps, _ptr(out), _stream(stream)))
        return out


def create_backend(preference="hip", device=0):
    """create_backend: only the HIP arm lives here (no silent CPU fallback)."""
    if preference not in ("hip", "auto"):
        raise GqError(-2, f"backend {preference!r} is not provided by libgq")
    return HipBackend(device)
