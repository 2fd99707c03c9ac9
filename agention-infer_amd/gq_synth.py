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


def make_blocks(dtype, rows, in_dim, seed=0, zero=False):
    """Return a uint8 array [rows, type_size(in_dim)] in ggml block order."""
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
