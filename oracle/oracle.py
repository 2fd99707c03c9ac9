"""ctypes wrapper of liboracle.so -- TEST INFRASTRUCTURE ONLY.

The CPU restatement of gguf-rs's quant path (gq_oracle.c).  Only tests/,
__graft_entry__.smoke() and bench.py's cpu_baseline leg use it, always as
the checker or the timed CPU baseline, never as the product path.
"""
import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None

_P, _I, _SZ = ctypes.c_void_p, ctypes.c_int, ctypes.c_size_t


def build():
    subprocess.run(["make", "-B", "-C", _HERE, "liboracle.so"], check=True,
                   capture_output=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = ctypes.CDLL(LIB_PATH)
        sig = {
            "gqo_type_size": (_SZ, [_I, _SZ]),
            "gqo_f16_to_f32": (ctypes.c_float, [ctypes.c_uint16]),
            "gqo_f32_to_f16": (ctypes.c_uint16, [ctypes.c_float]),
            "gqo_dequant": (_I, [_I, _P, _SZ, _SZ, _P]),
            "gqo_dot_row": (_I, [_I, _P, _SZ, _P, _SZ, _P]),
            "gqo_get_scale_min_k4": (None, [_I, _P, _P, _P]),
            "gqo_quantize_row_q8_k": (None, [_P, _SZ, _P, _P, _P]),
            "gqo_dot_q5_k_q8k": (_I, [_P, _SZ, _SZ, _P, _P, _P, _P]),
            "gqo_quantize_q8_32": (None, [_P, _SZ, _P, _P]),
            "gqo_set_iq3xxs_grid": (None, [_P]),
            "gqo_get_iq3xxs_grid": (None, [_P]),
            "gqo_matmul_into": (_I, [_I, _P, _SZ, _P, _SZ, _P, _SZ, _I]),
            "gqo_matmul_rows": (_I, [_I, _P, _SZ, _P, _SZ, _P, _SZ, _I]),
            "gqo_matmul_dequant": (_I, [_I, _P, _SZ, _P, _SZ, _P, _SZ]),
            "gqo_matmul_batch_into": (_I, [_I, _P, _SZ, _P, _SZ, _SZ, _P, _SZ, _I]),
            "gqo_argmax": (_SZ, [_P, _SZ]),
            "gqo_moe_route": (None, [_P, _I, _I, _I, _P, _P]),
            "gqo_decode_step": (_I, [_P, _I, _I, _P, _I]),
            "gqo_moe_ffn": (_I, [_I, _P, _P, _P, _I, _I, _I, _P, _I, _I, _P, _P, _P, _I]),
        }
        for n, (r, a) in sig.items():
            f = getattr(L, n)
            f.restype = r
            f.argtypes = a
        _lib = L
    return _lib


class OracleError(RuntimeError):
    pass


def _p(a):
    return ctypes.c_void_p(a.ctypes.data)


def _chk(rc):
    if rc != 0:
        raise OracleError({-1: "short buffer", -2: "unsupported dtype", -3: "row range"}.get(rc, rc))


def f16_to_f32(bits):
    return lib().gqo_f16_to_f32(int(bits))


def f32_to_f16(v):
    return lib().gqo_f32_to_f16(float(v))


def type_size(dtype, n):
    return lib().gqo_type_size(dtype, n)


def dequant(dtype, data, n):
    data = np.ascontiguousarray(data, np.uint8)
    out = np.empty(n, np.float32)
    _chk(lib().gqo_dequant(dtype, _p(data), data.nbytes, n, _p(out)))
    return out


def dequant_rows(dtype, w2d, in_dim):
    return np.stack([dequant(dtype, w2d[r], in_dim) for r in range(w2d.shape[0])]) \
        if w2d.shape[0] else np.zeros((0, in_dim), np.float32)


def dot_row(dtype, data, x):
    data = np.ascontiguousarray(data, np.uint8)
    x = np.ascontiguousarray(x, np.float32)
    r = np.zeros(1, np.float32)
    _chk(lib().gqo_dot_row(dtype, _p(data), data.nbytes, _p(x), x.size, _p(r)))
    return float(r[0])


def get_scale_min_k4(j, scales):
    s = np.ascontiguousarray(scales, np.uint8)
    sc = np.zeros(1, np.uint8)
    m = np.zeros(1, np.uint8)
    lib().gqo_get_scale_min_k4(j, _p(s), _p(sc), _p(m))
    return int(sc[0]), int(m[0])


def quantize_row_q8_k(x):
    x = np.ascontiguousarray(x, np.float32)
    nb = (x.size + 255) // 256
    d = np.zeros(nb, np.float32)
    qs = np.zeros(nb * 256, np.int8)
    bs = np.zeros(nb * 16, np.int16)
    lib().gqo_quantize_row_q8_k(_p(x), x.size, _p(d), _p(qs), _p(bs))
    return d, qs, bs


def dot_q5_k_q8k(data, n, d, qs, bs):
    data = np.ascontiguousarray(data, np.uint8)
    r = np.zeros(1, np.float32)
    _chk(lib().gqo_dot_q5_k_q8k(_p(data), data.nbytes, n, _p(d), _p(qs), _p(bs), _p(r)))
    return float(r[0])


def quantize_q8_32(x):
    x = np.ascontiguousarray(x, np.float32)
    nb = (x.size + 31) // 32
    sc = np.zeros(nb, np.uint16)
    q = np.zeros(nb * 32, np.int8)
    lib().gqo_quantize_q8_32(_p(x), x.size, _p(sc), _p(q))
    return sc, q[: x.size]


def set_iq3xxs_grid(grid=None):
    if grid is None:
        lib().gqo_set_iq3xxs_grid(None)
    else:
        g = np.ascontiguousarray(grid, np.uint32)
        lib().gqo_set_iq3xxs_grid(_p(g))


def get_iq3xxs_grid():
    g = np.zeros(256, np.uint32)
    lib().gqo_get_iq3xxs_grid(_p(g))
    return g


def matmul_into(dtype, w, x, out_dim, nthreads=0):
    """WeightMap::matmul_into: threaded row-parallel fused dot (Q5_K: x to
    Q8_K once, then dot_q5_k_q8k per row, model/mod.rs:381-394)."""
    w = np.ascontiguousarray(w, np.uint8)
    x = np.ascontiguousarray(x, np.float32)
    out = np.zeros(out_dim, np.float32)
    _chk(lib().gqo_matmul_into(dtype, _p(w), w.nbytes, _p(x), x.size, _p(out), out_dim, nthreads))
    return out


def matmul_rows(dtype, w, x, out_dim, nthreads=0):
    """quant::dot_row per row for every type (ffn_gate_up's float dots; for
    Q5_K this differs from matmul_into, which takes the Q8_K int dot)."""
    w = np.ascontiguousarray(w, np.uint8)
    x = np.ascontiguousarray(x, np.float32)
    out = np.zeros(out_dim, np.float32)
    _chk(lib().gqo_matmul_rows(dtype, _p(w), w.nbytes, _p(x), x.size, _p(out), out_dim, nthreads))
    return out


def matmul_dequant(dtype, w, x, out_dim):
    """CpuBackend::matmul_dequant: serial rows."""
    w = np.ascontiguousarray(w, np.uint8)
    x = np.ascontiguousarray(x, np.float32)
    out = np.zeros(out_dim, np.float32)
    _chk(lib().gqo_matmul_dequant(dtype, _p(w), w.nbytes, _p(x), x.size, _p(out), out_dim))
    return out


def matmul_batch_into(dtype, w, X, out_dim, nthreads=0):
    """WeightMap::matmul_batch_into: X [batch][in_dim] -> [batch][out_dim]."""
    w = np.ascontiguousarray(w, np.uint8)
    X = np.ascontiguousarray(X, np.float32)
    batch, in_dim = X.shape
    out = np.zeros((batch, out_dim), np.float32)
    _chk(lib().gqo_matmul_batch_into(dtype, _p(w), w.nbytes, _p(X), in_dim, batch, _p(out),
                                     out_dim, nthreads))
    return out


def moe_route(logits, k):
    logits = np.ascontiguousarray(logits, np.float32)
    T, E = logits.shape
    ids = np.zeros((T, k), np.int32)
    w = np.zeros((T, k), np.float32)
    lib().gqo_moe_route(_p(logits), T, E, k, _p(ids), _p(w))
    return ids, w


def moe_ffn(dtype, gate, up, down, E, H, F, x, ids, w, nthreads=0):
    gate, up, down = (np.ascontiguousarray(a, np.uint8) for a in (gate, up, down))
    x = np.ascontiguousarray(x, np.float32)
    ids = np.ascontiguousarray(ids, np.int32)
    w = np.ascontiguousarray(w, np.float32)
    T, k = ids.shape
    out = np.zeros((T, H), np.float32)
    _chk(lib().gqo_moe_ffn(dtype, _p(gate), _p(up), _p(down), E, H, F, _p(x), T, k, _p(ids),
                           _p(w), _p(out), nthreads))
    return out


class _Model(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int) for n in ("n_layers", "hidden", "n_heads", "n_kv_heads",
                                             "head_dim", "ffn", "vocab", "ctx")] + \
        [("eps", ctypes.c_float), ("theta", ctypes.c_float)] + \
        [(n, ctypes.c_int) for n in ("attn_type", "gate_up_type", "down_type", "head_type")] + \
        [(n, ctypes.c_void_p) for n in ("embd", "output_norm", "lm_head", "attn_norm",
                                         "ffn_norm", "wq", "wk", "wv", "wo", "wgate", "wup",
                                         "wdown", "kcache", "vcache", "layer_types")] + \
        [("kv_q8", ctypes.c_int)]


class DecoderModel:
    """LlamaModel::run restated on the CPU (gqo_decode_step) with its own KV
    cache: f16 [layer][ctx][kv_dim] (kv_dtype "f16"), or the reference's
    Q8_0 blocks [layer][ctx][kv_dim/32 * 34] bytes (kv_dtype "q8_0")."""

    def __init__(self, cfg, w, kv_init=None, kv_dtype="f16"):
        self.cfg = cfg
        self.keep = []
        m = _Model()
        for k in ("n_layers", "hidden", "n_heads", "n_kv_heads", "head_dim", "ffn", "vocab", "ctx"):
            setattr(m, k, int(cfg[k]))
        m.eps, m.theta = float(cfg["eps"]), float(cfg["theta"])
        m.attn_type, m.gate_up_type = cfg["attn_type"], cfg["gate_up_type"]
        m.down_type, m.head_type = cfg["down_type"], cfg["head_type"]

        def ptr_array(arrs):
            arrs = [np.ascontiguousarray(a) for a in arrs]
            self.keep.extend(arrs)
            pa = (ctypes.c_void_p * len(arrs))(*[a.ctypes.data for a in arrs])
            self.keep.append(pa)
            return ctypes.cast(pa, ctypes.c_void_p)

        for k in ("embd", "output_norm", "lm_head"):
            a = np.ascontiguousarray(w[k])
            self.keep.append(a)
            setattr(m, k, a.ctypes.data)
        for k in ("attn_norm", "ffn_norm", "wq", "wk", "wv", "wo", "wgate", "wup", "wdown"):
            setattr(m, k, ptr_array(w[k]))
        L, ctx = cfg["n_layers"], cfg["ctx"]
        kvd = cfg["n_kv_heads"] * cfg["head_dim"]
        if kv_dtype == "q8_0":
            m.kv_q8 = 1
            self.kc = np.zeros((L, ctx, kvd // 32 * 34), np.uint8)
        else:
            self.kc = np.zeros((L, ctx, kvd), np.uint16)
        self.vc = np.zeros_like(self.kc)
        if kv_init is not None:
            kk, vv = kv_init
            self.kc[:, :kk.shape[1]] = kk
            self.vc[:, :vv.shape[1]] = vv
        if "layer_types" in w:  # [n_layers][7] per-tensor types (wq .. wdown)
            lt = np.ascontiguousarray(w["layer_types"], np.int32).reshape(L, 7)
            self.keep.append(lt)
            m.layer_types = lt.ctypes.data
        m.kcache = ptr_array([self.kc[l] for l in range(L)])
        m.vcache = ptr_array([self.vc[l] for l in range(L)])
        self.m = m

    def step(self, token, pos, nthreads=0, want_logits=True):
        """One decode step; want_logits=False skips the output head (the
        KV rows are still written) and returns None."""
        if not want_logits:
            _chk(lib().gqo_decode_step(ctypes.byref(self.m), token, pos, None, nthreads))
            return None
        logits = np.zeros(self.cfg["vocab"], np.float32)
        _chk(lib().gqo_decode_step(ctypes.byref(self.m), token, pos, _p(logits), nthreads))
        return logits


def argmax(xs):
    xs = np.ascontiguousarray(xs, np.float32)
    return int(lib().gqo_argmax(_p(xs), xs.size))
