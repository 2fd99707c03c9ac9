"""Seeded synthetic GGUF weight blocks with the benchmark distributions.

Produces raw tensors in ggml block order (what a GGUF file holds and what
gq_upload takes), so the CPU oracle and the GPU see identical bytes.

Distributions (per block):
  Q8_0    d = f16(|N(0,1)|*0.01), 32 int8 quants uniform in [-127, 127]
  Q4_K    d, dmin = f16(|N(0,1)|*0.01); 8 six-bit scales and 8 six-bit mins
          uniform in [0, 63], packed the way get_scale_min_k4
          (src/quant/q4_k.rs:26-35) unpacks them; 128 qs bytes uniform
          (both nibbles uniform in [0, 15])
  Q5_K    as Q4_K plus 32 uniform qh bytes
  Q6_K    128 ql and 64 qh bytes uniform, 16 int8 scales uniform in
          [-32, 31], d = f16(|N(0,1)|*0.01) (stored last, bytes 208..209)
  IQ3_XXS d = f16(|N(0,1)|*0.01), 64 grid-index bytes and 32 sign/scale
          bytes uniform
"""
import numpy as np

Q8_0, Q4_K, Q5_K, Q6_K, IQ3_XXS = 8, 12, 13, 14, 18
BLOCK_ELEMS = {Q8_0: 32, Q4_K: 256, Q5_K: 256, Q6_K: 256, IQ3_XXS: 256}
BLOCK_BYTES = {Q8_0: 34, Q4_K: 144, Q5_K: 176, Q6_K: 210, IQ3_XXS: 98}
NAMES = {Q8_0: "Q8_0", Q4_K: "Q4_K", Q5_K: "Q5_K", Q6_K: "Q6_K", IQ3_XXS: "IQ3_XXS"}


def type_size(dtype, n):
    be = BLOCK_ELEMS[dtype]
    return (n + be - 1) // be * BLOCK_BYTES[dtype]


def _f16_scale(rng, shape):
    return (np.abs(rng.standard_normal(shape, dtype=np.float32)) * np.float32(0.01)).astype(
        np.float16).view(np.uint16)


def pack_scale_min_k4(sc, m):
    """Inverse of get_scale_min_k4: sc, m uint8 [..., 8] in [0, 63] -> [..., 12]."""
    sc = sc.astype(np.uint8)
    m = m.astype(np.uint8)
    out = np.zeros(sc.shape[:-1] + (12,), np.uint8)
    for j in range(4):
        out[..., j] = (sc[..., j] & 63) | ((sc[..., j + 4] >> 4) << 6)
        out[..., j + 4] = (m[..., j] & 63) | ((m[..., j + 4] >> 4) << 6)
        out[..., j + 8] = (sc[..., j + 4] & 0xF) | ((m[..., j + 4] & 0xF) << 4)
    return out


def make_blocks(dtype, rows, in_dim, seed=0, zero=False, centered=False):
    """Return a uint8 array [rows, type_size(in_dim)] in ggml block order.

    centered=True (Q4_K only) draws the same d, scales and quants but sets
    dmin = f16(7.5 d) and every min equal to its scale, so each element is
    d*sc*(q - 7.5) up to the f16 rounding of dmin: zero-mean rows, as in a
    trained model, instead of the per-block positive bias of independent
    mins."""
    nb = (in_dim + BLOCK_ELEMS[dtype] - 1) // BLOCK_ELEMS[dtype]
    bb = BLOCK_BYTES[dtype]
    if zero:
        return np.zeros((rows, nb * bb), np.uint8)
    rng = np.random.default_rng(seed)
    blk = np.empty((rows, nb, bb), np.uint8)
    if dtype == Q8_0:
        blk[..., 0:2] = _f16_scale(rng, (rows, nb))[..., None].view(np.uint8)
        blk[..., 2:] = rng.integers(-127, 128, (rows, nb, 32), dtype=np.int8).view(np.uint8)
    elif dtype in (Q4_K, Q5_K):
        blk[..., 0:2] = _f16_scale(rng, (rows, nb))[..., None].view(np.uint8)
        blk[..., 2:4] = _f16_scale(rng, (rows, nb))[..., None].view(np.uint8)
        sc = rng.integers(0, 64, (rows, nb, 8), dtype=np.uint8)
        m = rng.integers(0, 64, (rows, nb, 8), dtype=np.uint8)
        if centered:
            if dtype != Q4_K:
                raise ValueError("centered blocks are defined for Q4_K only")
            d = blk[..., 0:2].copy().view(np.float16).astype(np.float32)
            blk[..., 2:4] = (d * np.float32(7.5)).astype(np.float16).view(np.uint8)
            m = sc
        blk[..., 4:16] = pack_scale_min_k4(sc, m)
        blk[..., 16:] = rng.integers(0, 256, (rows, nb, bb - 16), dtype=np.uint8)
    elif dtype == Q6_K:
        blk[..., 0:192] = rng.integers(0, 256, (rows, nb, 192), dtype=np.uint8)
        blk[..., 192:208] = rng.integers(-32, 32, (rows, nb, 16), dtype=np.int8).view(np.uint8)
        blk[..., 208:210] = _f16_scale(rng, (rows, nb))[..., None].view(np.uint8)
    elif dtype == IQ3_XXS:
        blk[..., 0:2] = _f16_scale(rng, (rows, nb))[..., None].view(np.uint8)
        blk[..., 2:] = rng.integers(0, 256, (rows, nb, 96), dtype=np.uint8)
    else:
        raise ValueError(f"unsupported dtype {dtype}")
    return blk.reshape(rows, nb * bb)


def make_x(n, seed=1, batch=None):
    rng = np.random.default_rng(seed)
    shape = (n,) if batch is None else (batch, n)
    return rng.standard_normal(shape, dtype=np.float32)


# ------------------------------------------------------------ dense decoder
QWEN25_7B = dict(n_layers=28, hidden=3584, n_heads=28, n_kv_heads=4, head_dim=128, ffn=18944,
                 vocab=152064, eps=1e-6, theta=1e6, attn_type=Q4_K, gate_up_type=Q4_K,
                 down_type=Q6_K, head_type=Q6_K)


def make_decoder(cfg, seed=0, embd_scale=1.0, centered=False):
    """Random-init weights of a dense decoder in ggml block order (the
    Q4_K_M layout of the benchmark: Q4_K attention/gate/up, Q6_K down/head),
    RMSNorm weights ~ N(1, 0.1), f32 embedding ~ N(0, 1) * embd_scale.

    With the benchmark's block distributions every row carries a large
    per-block bias, so the layer outputs dwarf an N(0, 1) embedding and the
    greedy token stops depending on the input token; tests raise
    embd_scale to keep the token path live.  centered=True draws the Q4_K
    tensors zero-mean (make_blocks), so that every layer's attention and
    FFN output stays a visible part of the residual stream."""
    rng = np.random.default_rng(seed)
    L, H, F = cfg["n_layers"], cfg["hidden"], cfg["ffn"]
    qd, kvd = cfg["n_heads"] * cfg["head_dim"], cfg["n_kv_heads"] * cfg["head_dim"]
    w = {k: [] for k in ("wq", "wk", "wv", "wo", "wgate", "wup", "wdown", "attn_norm", "ffn_norm")}
    s = seed * 1000

    def cq(kind):
        return centered and cfg[kind] == Q4_K

    for l in range(L):
        s += 10
        w["wq"].append(make_blocks(cfg["attn_type"], qd, H, seed=s + 1, centered=cq("attn_type")))
        w["wk"].append(make_blocks(cfg["attn_type"], kvd, H, seed=s + 2, centered=cq("attn_type")))
        w["wv"].append(make_blocks(cfg["attn_type"], kvd, H, seed=s + 3, centered=cq("attn_type")))
        w["wo"].append(make_blocks(cfg["attn_type"], H, qd, seed=s + 4, centered=cq("attn_type")))
        w["wgate"].append(make_blocks(cfg["gate_up_type"], F, H, seed=s + 5, centered=cq("gate_up_type")))
        w["wup"].append(make_blocks(cfg["gate_up_type"], F, H, seed=s + 6, centered=cq("gate_up_type")))
        w["wdown"].append(make_blocks(cfg["down_type"], H, F, seed=s + 7))
        w["attn_norm"].append((1.0 + 0.1 * rng.standard_normal(H)).astype(np.float32))
        w["ffn_norm"].append((1.0 + 0.1 * rng.standard_normal(H)).astype(np.float32))
    w["lm_head"] = make_blocks(cfg["head_type"], cfg["vocab"], H, seed=s + 100)
    w["output_norm"] = (1.0 + 0.1 * rng.standard_normal(H)).astype(np.float32)
    w["embd"] = rng.standard_normal((cfg["vocab"], H), dtype=np.float32)
    if embd_scale != 1.0:
        w["embd"] *= np.float32(embd_scale)
    return w


def make_kv(cfg, n_pos, seed=0):
    """Prefilled f16 KV cache ~ N(0, 1): [n_layers][n_pos][kv_dim] bits."""
    rng = np.random.default_rng(seed)
    kvd = cfg["n_kv_heads"] * cfg["head_dim"]
    shape = (cfg["n_layers"], n_pos, kvd)
    k = rng.standard_normal(shape, dtype=np.float32).astype(np.float16).view(np.uint16)
    v = rng.standard_normal(shape, dtype=np.float32).astype(np.float16).view(np.uint16)
    return k, v


def upload_decoder(backend, cfg, w):
    """Upload every weight matrix once (pre_upload_gpu, gpu_resident.rs:69-229)."""
    H, F = cfg["hidden"], cfg["ffn"]
    qd, kvd = cfg["n_heads"] * cfg["head_dim"], cfg["n_kv_heads"] * cfg["head_dim"]
    dims = dict(wq=(qd, H), wk=(kvd, H), wv=(kvd, H), wo=(H, qd), wgate=(F, H), wup=(F, H),
                wdown=(H, F))
    types = dict(wq="attn_type", wk="attn_type", wv="attn_type", wo="attn_type",
                 wgate="gate_up_type", wup="gate_up_type", wdown="down_type")
    hw = {}
    for k, (rows, cols) in dims.items():
        hw[k] = [backend.upload_weight(cfg[types[k]], a, cols, rows) for a in w[k]]
    hw["lm_head"] = backend.upload_weight(cfg["head_type"], w["lm_head"], H, cfg["vocab"])
    for k in ("attn_norm", "ffn_norm", "output_norm", "embd"):
        hw[k] = w[k]
    return hw
