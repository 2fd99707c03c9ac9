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
    "gq_dequant_rows_host": (_I, [_P, _I, _I, _P]),
    "gq_gemm": (_I, [_P, _P, _I, _P, _I, _P]),
    "gq_quantize_q8_32": (_I, [_P, _I, _P, _P, _P]),
    "gq_quantize_row_q8k": (_I, [_P, _I, _P, _P, _P, _P]),
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
    "gq_model_prefill": (_I, [_P, _P, _I, _I, _P, ctypes.POINTER(_I), _P]),
    "gq_moe_ffn": (_I, [_P, _P, _P, _I, _P, _I, _I, _P, _P, _P, _P, _P]),
    "gq_moe_ffn_noalloc": (_I, [_P, _P, _P, _I, _P, _I, _I, _P, _P, _P, _P, _P]),
}


# Every entry point of include/gq_host.h (libgq_host.so: GGUF files, uploads).
_U32, _U64, _I64 = ctypes.c_uint32, ctypes.c_uint64, ctypes.c_int64
_PP = ctypes.POINTER(_P)
HOST_SIGNATURES = {
    "gqh_last_error": (ctypes.c_char_p, []),
    "gqh_gguf_open": (_I, [ctypes.c_char_p, _PP]),
    "gqh_gguf_parse": (_I, [_P, _SZ, _PP]),
    "gqh_gguf_close": (_I, [_P]),
    "gqh_gguf_header": (_I, [_P, ctypes.POINTER(_U32), ctypes.POINTER(_U64), ctypes.POINTER(_U64),
                             ctypes.POINTER(_U64)]),
    "gqh_gguf_tensor": (_I, [_P, _U64, ctypes.POINTER(ctypes.c_char_p), ctypes.POINTER(_U32),
                             ctypes.POINTER(_U64), ctypes.POINTER(_U32), ctypes.POINTER(_U64),
                             ctypes.POINTER(_U64)]),
    "gqh_gguf_find_tensor": (_I, [_P, ctypes.c_char_p, ctypes.POINTER(_U64)]),
    "gqh_gguf_tensor_data": (_I, [_P, _U64, _PP, ctypes.POINTER(_SZ)]),
    "gqh_gguf_meta_type": (_I, [_P, ctypes.c_char_p, ctypes.POINTER(_U32)]),
    "gqh_gguf_meta_u64": (_I, [_P, ctypes.c_char_p, ctypes.POINTER(_U64)]),
    "gqh_gguf_meta_i64": (_I, [_P, ctypes.c_char_p, ctypes.POINTER(_I64)]),
    "gqh_gguf_meta_f32": (_I, [_P, ctypes.c_char_p, ctypes.POINTER(ctypes.c_float)]),
    "gqh_gguf_meta_bool": (_I, [_P, ctypes.c_char_p, ctypes.POINTER(_I)]),
    "gqh_gguf_meta_str": (_I, [_P, ctypes.c_char_p, _PP, ctypes.POINTER(_SZ)]),
    "gqh_gguf_meta_array": (_I, [_P, ctypes.c_char_p, ctypes.POINTER(_U32), ctypes.POINTER(_U64)]),
    "gqh_gguf_meta_array_i64": (_I, [_P, ctypes.c_char_p, _U64, ctypes.POINTER(_I64)]),
    "gqh_gguf_meta_array_str": (_I, [_P, ctypes.c_char_p, _U64, _PP, ctypes.POINTER(_SZ)]),
    "gqh_parse_split_index": (_I, [ctypes.c_char_p, ctypes.POINTER(_U64), ctypes.POINTER(_U64)]),
    "gqh_gguf_upload": (_I, [_P, ctypes.c_char_p, _PP]),
    "gqh_model_load": (_I, [_P, _I, _I, _PP]),
    "gqh_model_free": (_I, [_P]),
    "gqh_model_config_get": (_I, [_P, _P]),
    "gqh_model_handle": (_I, [_P, _PP]),
}


class _HostModelConfig(ctypes.Structure):
    _fields_ = [(n, _U64) for n in ("context_length", "embedding_length", "block_count",
                                     "head_count", "head_count_kv", "head_dim",
                                     "feed_forward_length", "vocab_size")] + \
        [("rope_freq_base", ctypes.c_float), ("layer_norm_rms_epsilon", ctypes.c_float),
         ("ctx", ctypes.c_int), ("architecture", ctypes.c_char * 64)]
HOST_LIB_PATH = os.environ.get("GQ_HOST_LIBRARY") or os.path.join(_HERE, "libgq_host.so")


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


_host = None


def host_lib():
    """Load libgq_host.so (the C++ host library: GGUF files, uploads)."""
    global _host
    if _host is None:
        lib()  # libgq.so (and torch's HIP runtime) first
        if not os.path.exists(HOST_LIB_PATH):
            raise GqError(-6, f"{HOST_LIB_PATH} not built; run __graft_entry__.build()")
        L = ctypes.CDLL(HOST_LIB_PATH)
        for name, (res, args) in HOST_SIGNATURES.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _host = L
    return _host


class GgufError(GqError):
    """A GGUF parse / load failure; .code is the GQH_E* kind (gq_host.h)."""


def _hcheck(rc):
    if rc != 0:
        raise GgufError(rc, host_lib().gqh_last_error().decode())


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

    def quantize_row_q8_k(self, x_dev, stream=None):
        """quantize_row_q8_k (q8_k.rs:49-91): (d f32[nb], qs int8[nb*256],
        bsums int16[nb*16]) on the device."""
        import torch
        n = x_dev.numel()
        nb = (n + 255) // 256
        d = torch.empty(nb, dtype=torch.float32, device=x_dev.device)
        qs = torch.empty(nb * 256, dtype=torch.int8, device=x_dev.device)
        bs = torch.empty(nb * 16, dtype=torch.int16, device=x_dev.device)
        _check(lib().gq_quantize_row_q8k(_ptr(x_dev), n, _ptr(d), _ptr(qs), _ptr(bs),
                                         _stream(stream)))
        return d, qs, bs

    def upload_experts(self, dtype, w, in_dim, rows_per_expert, n_experts):
        """A stacked expert tensor [n_experts][rows_per_expert][in_dim]."""
        w = np.ascontiguousarray(w, dtype=np.uint8)
        h = ctypes.c_void_p()
        _check(lib().gq_upload_experts(dtype, _ptr(w), w.nbytes, in_dim, rows_per_expert,
                                       n_experts, ctypes.byref(h)))
        return GpuWeightHandle(h.value, dtype, in_dim, rows_per_expert * n_experts)

    def moe_ffn(self, gate, up, down, n_experts, logits_dev, x_dev, top_k, out_dev=None,
                want_routing=False, stream=None, noalloc=False):
        """MoE expert FFN for T tokens; returns out [T][h] (and ids, w).
        noalloc: gq_moe_ffn_noalloc (workspace in the library's static device
        scratch, no allocation)."""
        import torch
        T, h = x_dev.shape
        if out_dev is None:
            out_dev = torch.empty((T, h), dtype=torch.float32, device=x_dev.device)
        ids = torch.empty((T, top_k), dtype=torch.int32, device=x_dev.device) if want_routing else None
        w = torch.empty((T, top_k), dtype=torch.float32, device=x_dev.device) if want_routing else None
        fn = lib().gq_moe_ffn_noalloc if noalloc else lib().gq_moe_ffn
        _check(fn(gate._h, up._h, down._h, n_experts, _ptr(logits_dev), T, top_k,
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
                                         "embd")] + \
        [("kv_dtype", ctypes.c_int)]


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
        # KvDtype::parse (model/mod.rs:540-547): "f16" (default) or "q8_0"
        self.kv_q8 = str(cfg.get("kv_dtype", "f16")).lower() in ("q8_0", "q8")
        d.kv_dtype = Q8_0 if self.kv_q8 else 0
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

    def _kv_row(self):
        kvd = self.cfg["n_kv_heads"] * self.cfg["head_dim"]
        return (kvd // 32 * 34, np.uint8) if self.kv_q8 else (kvd, np.uint16)

    def kv_upload(self, layer, k_rows, v_rows):
        """Rows [n_pos][...] in the cache's KvDtype format: f16 bits
        (uint16) or Q8_0 blocks (uint8, kv_dim/32 * 34 bytes per row)."""
        width, dt = self._kv_row()
        k = np.ascontiguousarray(k_rows, dt)
        v = np.ascontiguousarray(v_rows, dt)
        if k.shape != v.shape or k.ndim != 2 or k.shape[1] != width:
            raise ValueError(f"KV rows must be [n_pos][{width}] {np.dtype(dt).name}")
        _check(lib().gq_model_kv_upload(self._h, layer, _ptr(k), _ptr(v), k.shape[0]))

    def kv_download(self, layer, n_pos):
        width, dt = self._kv_row()
        k = np.zeros((n_pos, width), dt)
        v = np.zeros((n_pos, width), dt)
        _check(lib().gq_model_kv_download(self._h, layer, _ptr(k), _ptr(v), n_pos))
        return k, v

    def decode(self, token, pos, want_logits=True):
        """One step (Model::forward): returns (next_token, logits or None)."""
        logits = np.zeros(self.cfg["vocab"], np.float32) if want_logits else None
        nxt = ctypes.c_int()
        _check(lib().gq_model_decode(self._h, token, pos, _ptr(logits), ctypes.byref(nxt)))
        return nxt.value, logits

    def prefill(self, tokens, pos, want_logits=True, stream=None):
        """LlamaModel::run_batch: the prompt tokens at positions pos .. through
        every layer at once; returns (greedy next token, last-position logits
        or None)."""
        toks = np.ascontiguousarray(tokens, np.int32)
        logits = np.zeros(self.cfg["vocab"], np.float32) if want_logits else None
        nxt = ctypes.c_int()
        _check(lib().gq_model_prefill(self._h, _ptr(toks), toks.size, pos, _ptr(logits),
                                      ctypes.byref(nxt), _stream(stream)))
        return nxt.value, logits

    def generate(self, token, pos, n_steps, stream=None):
        """n_steps greedy steps (one HIP graph replay each); returns the tokens."""
        out = np.zeros(n_steps, np.int32)
        _check(lib().gq_model_generate(self._h, token, pos, n_steps, _ptr(out), _stream(stream)))
        return out


class TensorInfo:
    """TensorInfo (src/types.rs): name, dims (dims[0] fastest), GGML type id,
    byte offset from the data section, byte size."""

    def __init__(self, name, dims, ggml_type, byte_offset, nbytes):
        self.name, self.dims, self.ggml_type = name, dims, ggml_type
        self.byte_offset, self.nbytes = byte_offset, nbytes

    def n_elements(self):
        n = 1
        for d in self.dims:
            n *= d
        return n

    def __repr__(self):
        return f"TensorInfo({self.name!r}, {self.dims}, type {self.ggml_type})"


class GgufFile:
    """A GGUF file parsed and mapped once by libgq_host (loader::load; a
    "-00001-of-0000N.gguf" name opens all N parts), or parsed from bytes
    (parser::parse).  Metadata via .get(key) / get_u64 / get_f32 /
    get_string / get_bool / get_i64_array / get_str_array; tensor bytes are
    read from the mapping; .upload(name) puts a weight on the GPU once."""

    def __init__(self, path=None, data=None):
        h = ctypes.c_void_p()
        if path is not None:
            _hcheck(host_lib().gqh_gguf_open(os.fsencode(path), ctypes.byref(h)))
        else:
            buf = bytes(data)
            _hcheck(host_lib().gqh_gguf_parse(buf, len(buf), ctypes.byref(h)))
        self._h = h
        v, tc, mc, do = _U32(), _U64(), _U64(), _U64()
        _hcheck(host_lib().gqh_gguf_header(h, ctypes.byref(v), ctypes.byref(tc), ctypes.byref(mc),
                                           ctypes.byref(do)))
        self.version, self.tensor_count = v.value, tc.value
        self.metadata_count, self.data_offset = mc.value, do.value
        self.tensors = [self._tensor(i) for i in range(self.tensor_count)]

    def close(self):
        if getattr(self, "_h", None) is not None and _host is not None:
            _host.gqh_gguf_close(self._h)
            self._h = None

    __del__ = close

    def _tensor(self, i):
        name, nd, ty = ctypes.c_char_p(), _U32(), _U32()
        dims, off, nb = (_U64 * 8)(), _U64(), _U64()
        _hcheck(host_lib().gqh_gguf_tensor(self._h, i, ctypes.byref(name), ctypes.byref(nd), dims,
                                           ctypes.byref(ty), ctypes.byref(off), ctypes.byref(nb)))
        return TensorInfo(name.value.decode(), [dims[k] for k in range(min(nd.value, 8))],
                          ty.value, off.value, nb.value)

    def find(self, name):
        for t in self.tensors:
            if t.name == name:
                return t
        return None

    def tensor_bytes(self, name):
        """The tensor's bytes (a numpy uint8 copy out of the mapping)."""
        idx = _U64()
        _hcheck(host_lib().gqh_gguf_find_tensor(self._h, name.encode(), ctypes.byref(idx)))
        p, n = ctypes.c_void_p(), _SZ()
        _hcheck(host_lib().gqh_gguf_tensor_data(self._h, idx.value, ctypes.byref(p), ctypes.byref(n)))
        return np.ctypeslib.as_array((ctypes.c_uint8 * n.value).from_address(p.value)).copy()

    # metadata (GgufFile::get_* in src/types.rs); None when absent
    def _meta(self, fn, key, out):
        rc = fn(self._h, key.encode(), ctypes.byref(out))
        if rc == -107:  # GQH_EMISSING
            return None
        _hcheck(rc)
        return out.value

    def get_u64(self, key):
        return self._meta(host_lib().gqh_gguf_meta_u64, key, _U64())

    def get_i64(self, key):
        return self._meta(host_lib().gqh_gguf_meta_i64, key, _I64())

    def get_f32(self, key):
        return self._meta(host_lib().gqh_gguf_meta_f32, key, ctypes.c_float())

    def get_bool(self, key):
        v = self._meta(host_lib().gqh_gguf_meta_bool, key, _I())
        return None if v is None else bool(v)

    def get_string(self, key):
        p, n = ctypes.c_void_p(), _SZ()
        rc = host_lib().gqh_gguf_meta_str(self._h, key.encode(), ctypes.byref(p), ctypes.byref(n))
        if rc == -107:
            return None
        _hcheck(rc)
        return ctypes.string_at(p.value, n.value).decode()

    def _array(self, key):
        et, cnt = _U32(), _U64()
        rc = host_lib().gqh_gguf_meta_array(self._h, key.encode(), ctypes.byref(et), ctypes.byref(cnt))
        if rc == -107:
            return None, 0
        _hcheck(rc)
        return et.value, cnt.value

    def get_i64_array(self, key):
        et, cnt = self._array(key)
        if et is None:
            return None
        out, v = [], _I64()
        for k in range(cnt):
            _hcheck(host_lib().gqh_gguf_meta_array_i64(self._h, key.encode(), k, ctypes.byref(v)))
            out.append(v.value)
        return out

    def get_str_array(self, key):
        et, cnt = self._array(key)
        if et is None:
            return None
        out, p, n = [], ctypes.c_void_p(), _SZ()
        for k in range(cnt):
            _hcheck(host_lib().gqh_gguf_meta_array_str(self._h, key.encode(), k, ctypes.byref(p),
                                                       ctypes.byref(n)))
            out.append(ctypes.string_at(p.value, n.value).decode())
        return out

    def meta_type(self, key):
        t = _U32()
        rc = host_lib().gqh_gguf_meta_type(self._h, key.encode(), ctypes.byref(t))
        if rc == -107:
            return None
        _hcheck(rc)
        return t.value

    def get(self, key):
        """The value of any kind (arrays as lists), or None."""
        t = self.meta_type(key)
        if t is None:
            return None
        if t in (0, 2, 4, 10):
            return self.get_u64(key)
        if t in (1, 3, 5, 11):
            return self.get_i64(key)
        if t in (6, 12):
            return self.get_f32(key)
        if t == 7:
            return self.get_bool(key)
        if t == 8:
            return self.get_string(key)
        et, _ = self._array(key)
        return self.get_str_array(key) if et == 8 else self.get_i64_array(key)

    def architecture(self):
        return self.get_string("general.architecture")

    def upload(self, name):
        """HipBackend::upload_tensor: a 2-D weight tensor, resident once."""
        t = self.find(name)
        h = ctypes.c_void_p()
        _hcheck(host_lib().gqh_gguf_upload(self._h, name.encode(), ctypes.byref(h)))
        return GpuWeightHandle(h.value, t.ggml_type, t.dims[0], t.dims[1])


    def load_model(self, ctx=0, max_tokens=4096):
        """LlamaModel::new + pre_upload_gpu: the whole decoder on the GPU."""
        return GgufModel(self, ctx, max_tokens)


class GgufModel(DecodeModel):
    """A dense decoder loaded from a GGUF file by libgq_host (gqh_model_load);
    decode / generate / kv_upload / kv_download as DecodeModel.  .config is
    ModelConfig::from_gguf (architecture, embedding_length, ...)."""

    def __init__(self, gguf, ctx=0, max_tokens=4096):
        h = ctypes.c_void_p()
        _hcheck(host_lib().gqh_model_load(gguf._h, int(ctx), int(max_tokens), ctypes.byref(h)))
        self._owner = h
        c = _HostModelConfig()
        _hcheck(host_lib().gqh_model_config_get(h, ctypes.byref(c)))
        self.config = {k: getattr(c, k) for k, _ in _HostModelConfig._fields_}
        self.config["architecture"] = c.architecture.decode()
        self.cfg = dict(n_layers=c.block_count, hidden=c.embedding_length, n_heads=c.head_count,
                        n_kv_heads=c.head_count_kv, head_dim=c.head_dim, vocab=c.vocab_size,
                        ctx=c.ctx, eps=c.layer_norm_rms_epsilon, theta=c.rope_freq_base)
        self.kv_q8 = False  # gqh_model_load builds an f16 KV cache (KvDtype::F16)
        m = ctypes.c_void_p()
        _hcheck(host_lib().gqh_model_handle(h, ctypes.byref(m)))
        self._h = m

    def __del__(self):
        if getattr(self, "_owner", None) is not None and _host is not None:
            _host.gqh_model_free(self._owner)
            self._owner = self._h = None


def parse_split_index(file_name):
    """loader::parse_split_index: "x-00002-of-00005.gguf" -> (2, 5), else None."""
    i, t = _U64(), _U64()
    rc = host_lib().gqh_parse_split_index(file_name.encode(), ctypes.byref(i), ctypes.byref(t))
    return None if rc != 0 else (i.value, t.value)


def create_backend(preference="hip", device=0):
    """create_backend: only the HIP arm lives here (no silent CPU fallback)."""
    if preference not in ("hip", "auto"):
        raise GqError(-2, f"backend {preference!r} is not provided by libgq")
    return HipBackend(device)
