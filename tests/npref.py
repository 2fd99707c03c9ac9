"""Independent numpy restatements of the ggml block formats (test helpers).

Written from the block layouts (float32 arithmetic, one rounding per
operation, no FMA), not from the C oracle, so that a mistake in either one
shows up as a mismatch.  Used to pin the oracle and, on the GPU, as a second
opinion on dequant.
"""
import numpy as np


def f16(u16):
    return np.asarray(u16, np.uint16).view(np.float16).astype(np.float32)


def round_half_away(v):
    v = np.asarray(v, np.float64)
    return np.sign(v) * np.floor(np.abs(v) + 0.5)


def unpack_k4_scales(s):
    """s: uint8 [..., 12] -> (sc, m) uint8 [..., 8]; ggml's 6-bit packing."""
    s = s.astype(np.uint8)
    sc = np.empty(s.shape[:-1] + (8,), np.uint8)
    m = np.empty_like(sc)
    sc[..., :4] = s[..., 0:4] & 63
    m[..., :4] = s[..., 4:8] & 63
    sc[..., 4:] = (s[..., 8:12] & 0x0F) | ((s[..., 0:4] >> 6) << 4)
    m[..., 4:] = (s[..., 8:12] >> 4) | ((s[..., 4:8] >> 6) << 4)
    return sc, m


def dequant_q8_0(data, n):
    nb = (n + 31) // 32
    b = np.asarray(data, np.uint8)[: nb * 34].reshape(nb, 34)
    d = f16(b[:, 0:2].copy().view(np.uint16)[:, 0])
    q = b[:, 2:].view(np.int8).astype(np.float32)
    return (d[:, None] * q).reshape(-1)[:n]


def dequant_k4(data, n, q5=False):
    bb = 176 if q5 else 144
    nb = (n + 255) // 256
    b = np.asarray(data, np.uint8)[: nb * bb].reshape(nb, bb)
    d = f16(b[:, 0:2].copy().view(np.uint16)[:, 0])
    dmin = f16(b[:, 2:4].copy().view(np.uint16)[:, 0])
    sc, m = unpack_k4_scales(b[:, 4:16])
    qs = b[:, 48:176] if q5 else b[:, 16:144]
    qh = b[:, 16:48] if q5 else None
    y = np.empty((nb, 256), np.float32)
    for g in range(4):                      # 64-element groups
        byte = qs[:, 32 * g:32 * g + 32]
        for half in range(2):               # low nibbles, then high nibbles
            sub = 2 * g + half
            q = (byte >> 4) if half else (byte & 0x0F)
            if q5:
                q = q | (((qh >> sub) & 1) << 4)
            scale = d * sc[:, sub].astype(np.float32)
            mn = dmin * m[:, sub].astype(np.float32)
            y[:, 64 * g + 32 * half:64 * g + 32 * half + 32] = \
                scale[:, None] * q.astype(np.float32) - mn[:, None]
    return y.reshape(-1)[:n]


def dequant_q6_k(data, n):
    nb = (n + 255) // 256
    b = np.asarray(data, np.uint8)[: nb * 210].reshape(nb, 210)
    ql, qh = b[:, 0:128], b[:, 128:192]
    sc = b[:, 192:208].view(np.int8).astype(np.float32)
    d = f16(b[:, 208:210].copy().view(np.uint16)[:, 0])
    y = np.empty((nb, 256), np.float32)
    for half in range(2):
        for quarter in range(4):            # 32-element run within the half
            low = ql[:, 64 * half + 32 * (quarter & 1): 64 * half + 32 * (quarter & 1) + 32]
            low = (low >> 4) if quarter >= 2 else (low & 0x0F)
            high = (qh[:, 32 * half:32 * half + 32] >> (2 * quarter)) & 3
            q = (low | (high << 4)).astype(np.int32) - 32
            for sixteen in range(2):
                s = sc[:, 8 * half + 2 * quarter + sixteen]
                lo = 16 * sixteen
                y[:, 128 * half + 32 * quarter + lo:128 * half + 32 * quarter + lo + 16] = \
                    (d * s)[:, None] * q[:, lo:lo + 16].astype(np.float32)
    return y.reshape(-1)[:n]


def ksigns():
    i = np.arange(128, dtype=np.uint32)
    par = np.array([bin(v).count("1") & 1 for v in range(128)], np.uint32)
    return (i | (par << 7)).astype(np.uint8)


def dequant_iq3_xxs(data, n, grid):
    nb = (n + 255) // 256
    b = np.asarray(data, np.uint8)[: nb * 98].reshape(nb, 98)
    d = f16(b[:, 0:2].copy().view(np.uint16)[:, 0])
    qs = b[:, 2:66]
    aux = b[:, 66:98].copy().view(np.uint32)          # [nb, 8]
    mags = np.asarray(grid, np.uint32)[qs.astype(np.int64)]  # [nb, 64]
    mag_bytes = mags.view(np.uint8).reshape(nb, 64, 4).astype(np.float32)  # 4 per index
    ks = ksigns()
    y = np.empty((nb, 256), np.float32)
    for ib in range(8):
        a = aux[:, ib]
        db = d * (np.float32(0.5) + (a >> 28).astype(np.float32)) * np.float32(0.5)
        for l in range(4):
            sg = ks[(a >> (7 * l)) & 127]
            for j in range(8):
                mag = mag_bytes[:, 8 * ib + 2 * l + j // 4, j % 4]
                sign = np.where((sg >> j) & 1, np.float32(-1), np.float32(1))
                y[:, 32 * ib + 8 * l + j] = (db * mag) * sign
    return y.reshape(-1)[:n]


def dequant(dtype, data, n, grid=None):
    if dtype == 8:
        return dequant_q8_0(data, n)
    if dtype == 12:
        return dequant_k4(data, n)
    if dtype == 13:
        return dequant_k4(data, n, q5=True)
    if dtype == 14:
        return dequant_q6_k(data, n)
    if dtype == 18:
        return dequant_iq3_xxs(data, n, grid)
    raise ValueError(dtype)


def quantize_q8_32(x):
    """KvDtype::Q8_0::pack (src/model/mod.rs:574-583)."""
    x = np.asarray(x, np.float32).reshape(-1, 32)
    amax = np.abs(x).max(axis=1)
    scale = np.where(amax > 0, amax / np.float32(127.0), np.float32(1.0)).astype(np.float32)
    q = round_half_away((x / scale[:, None]).astype(np.float32))
    q = np.clip(q, -127, 127).astype(np.int8)
    return scale.astype(np.float16).view(np.uint16), q.reshape(-1)


def pack_q8_0_rows(x):
    """One KV row as KvDtype::Q8_0 bytes (model/mod.rs:574-583): per 32
    values an f16 scale (little endian) then 32 int8."""
    sc, q = quantize_q8_32(np.asarray(x, np.float32))
    nb = sc.size
    out = np.empty((nb, 34), np.uint8)
    out[:, 0] = sc & 0xFF
    out[:, 1] = sc >> 8
    out[:, 2:] = q.view(np.uint8).reshape(nb, 32)
    return out.reshape(-1)


def unpack_q8_0_rows(rows):
    """KvDtype::Q8_0::unpack (model/mod.rs:595-602): rows [n][nb*34] ->
    float64 [n][nb*32]."""
    r = np.asarray(rows, np.uint8)
    n = r.shape[0]
    b = r.reshape(n, -1, 34)
    sc = f16((b[:, :, 0].astype(np.uint16) | (b[:, :, 1].astype(np.uint16) << 8))).astype(np.float64)
    q = b[:, :, 2:].view(np.int8).astype(np.float64)
    return (q * sc[:, :, None]).reshape(n, -1)


def quantize_row_q8_k(x):
    """quantize_row_q8_k (src/quant/q8_k.rs:49-91)."""
    x = np.asarray(x, np.float32)
    n = x.size
    nb = (n + 255) // 256
    xp = np.zeros(nb * 256, np.float32)
    xp[:n] = x
    xb = xp.reshape(nb, 256)
    d = np.zeros(nb, np.float32)
    qs = np.zeros((nb, 256), np.int8)
    for b in range(nb):
        v = xb[b, : min(256, n - 256 * b)]
        i = int(np.argmax(np.abs(v)))        # first index of the max |v|
        if np.abs(v[i]) > 0:
            iscale = np.float32(-127.0) / v[i]
            r = round_half_away((iscale * v).astype(np.float32))
            qs[b, : v.size] = np.minimum(r, 127).astype(np.int8)
            d[b] = np.float32(1.0) / iscale
    bs = qs.reshape(nb, 16, 16).astype(np.int16).sum(axis=2).reshape(-1)
    return d, qs.reshape(-1), bs.astype(np.int16)


def rope_angles(pos, theta, hd):
    """RoPE angles as cpu_path.rs:99-133 forms them, in f32: pos as f32
    divided by powf(theta, 2i/hd) (so at large positions they carry the f32
    rounding of pos / den, ~1e-3 rad at 20000); the sin / cos that follow
    are taken in float64.  pos: int or int array; returns float64 [..., hd/2]."""
    i = np.arange(hd // 2, dtype=np.float32)
    den = np.power(np.float32(theta), (np.float32(2.0) * i) / np.float32(hd)).astype(np.float32)
    p = np.asarray(pos, np.float32)[..., None]
    return (p / den).astype(np.float32).astype(np.float64)


def decode_step(cfg, w, kc, vc, token, pos):
    """One decode step of a dense Llama/Qwen2 decoder in float64, written
    from the model's definition (RMSNorm, NEOX RoPE with theta^(2i/hd) and
    f32 angles (rope_angles),
    causal softmax attention with grouped KV heads, SwiGLU FFN, residual
    adds), with the weights dequantized by the numpy block decoders above.
    kc / vc: float16 bit arrays [n_layers][ctx][kv_dim], updated at pos
    with k / v rounded to f16; or (uint8) KvDtype::Q8_0 rows
    [n_layers][ctx][kv_dim/32 * 34], packed with quantize_q8_32 from the
    fp32 values and read back as q * f16(scale).  Returns the logits
    (float64)."""
    H, hd = cfg["hidden"], cfg["head_dim"]
    nh, nkv, F = cfg["n_heads"], cfg["n_kv_heads"], cfg["ffn"]
    half, group = hd // 2, nh // nkv

    def mat(dtype, blob, rows, cols):
        return np.stack([dequant(dtype, blob[r], cols) for r in range(rows)]).astype(np.float64)

    def norm(x, g):
        return g * x / np.sqrt(np.mean(x * x) + cfg["eps"])

    i = np.arange(half)
    ang = rope_angles(pos, cfg["theta"], hd)
    cs, sn = np.cos(ang), np.sin(ang)

    def rope(v):  # v [heads, hd]
        a, b = v[:, :half].copy(), v[:, half:].copy()
        return np.concatenate([a * cs - b * sn, a * sn + b * cs], axis=1)

    x = w["embd"][token].astype(np.float64)
    for L in range(cfg["n_layers"]):
        xn = norm(x, w["attn_norm"][L].astype(np.float64))
        q = mat(cfg["attn_type"], w["wq"][L], nh * hd, H) @ xn
        k = mat(cfg["attn_type"], w["wk"][L], nkv * hd, H) @ xn
        v = mat(cfg["attn_type"], w["wv"][L], nkv * hd, H) @ xn
        q = rope(q.reshape(nh, hd))
        k = rope(k.reshape(nkv, hd)).reshape(-1)
        if kc.dtype == np.uint8:
            kc[L, pos] = pack_q8_0_rows(k)
            vc[L, pos] = pack_q8_0_rows(v)
            K = unpack_q8_0_rows(kc[L, :pos + 1]).reshape(pos + 1, nkv, hd)
            V = unpack_q8_0_rows(vc[L, :pos + 1]).reshape(pos + 1, nkv, hd)
        else:
            kc[L, pos] = k.astype(np.float16).view(np.uint16)
            vc[L, pos] = v.astype(np.float16).view(np.uint16)
            K = kc[L, :pos + 1].view(np.float16).astype(np.float64).reshape(pos + 1, nkv, hd)
            V = vc[L, :pos + 1].view(np.float16).astype(np.float64).reshape(pos + 1, nkv, hd)
        att = np.empty((nh, hd))
        for h in range(nh):
            s = K[:, h // group, :] @ q[h] / np.sqrt(hd)
            p = np.exp(s - s.max())
            att[h] = (p / p.sum()) @ V[:, h // group, :]
        x = x + mat(cfg["attn_type"], w["wo"][L], H, nh * hd) @ att.reshape(-1)
        xn = norm(x, w["ffn_norm"][L].astype(np.float64))
        g = mat(cfg["gate_up_type"], w["wgate"][L], F, H) @ xn
        u = mat(cfg["gate_up_type"], w["wup"][L], F, H) @ xn
        with np.errstate(over="ignore"):  # exp(-g) = inf gives silu(g) = -0
            act = g / (1.0 + np.exp(-g)) * u
        x = x + mat(cfg["down_type"], w["wdown"][L], H, F) @ act
    xn = norm(x, w["output_norm"].astype(np.float64))
    return mat(cfg["head_type"], w["lm_head"], cfg["vocab"], H) @ xn


def bf16(a):
    """Round float32 values to bfloat16 (nearest even), returned as float64."""
    u = np.ascontiguousarray(a, np.float32).view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
    return r.astype(np.uint32).view(np.float32).astype(np.float64)


def prefill_bf16(cfg, w, kc, vc, tokens, pos0, kv="f16"):
    """Batched prefill (run_batch: every layer over all prompt tokens at
    once) in float64 with the GPU prefill's operand rounding at each
    projection: weights rounded to bf16 from their fp32 dequant, the
    activations entering a projection (normed x, attention output,
    silu(g) * u) rounded to fp32 and then to bf16.  RoPE (f32 angles, rope_angles), the f16 K/V cache,
    the causal softmax and the residual adds stay float64; the output head
    is unrounded (the GPU runs it on the matvec).  kc / vc are updated.
    kv="q8_0": kc / vc hold KvDtype::Q8_0 rows ([layer][ctx][kv_dim/32*34]
    bytes); the new rows are packed from their fp32 values and every row is
    read back as f16(code * scale), the GPU's attention operands.
    Returns the logits of the last token."""
    H, hd = cfg["hidden"], cfg["head_dim"]
    nh, nkv, F = cfg["n_heads"], cfg["n_kv_heads"], cfg["ffn"]
    half, group = hd // 2, nh // nkv
    n = len(tokens)

    def mat32(dtype, blob, rows, cols):
        if cols % 256 == 0:  # whole blocks per row: the rows dequantize as one run
            return dequant(dtype, np.ascontiguousarray(blob).reshape(-1), rows * cols).reshape(rows, cols)
        return np.stack([dequant(dtype, blob[r], cols) for r in range(rows)])

    def matb(dtype, blob, rows, cols):
        return bf16(mat32(dtype, blob, rows, cols))

    def mat(dtype, blob, rows, cols):
        return mat32(dtype, blob, rows, cols).astype(np.float64)

    def norm(x, g):  # rows of x
        return g * x / np.sqrt(np.mean(x * x, axis=1, keepdims=True) + cfg["eps"])

    pos = pos0 + np.arange(n)
    i = np.arange(half)
    ang = rope_angles(pos, cfg["theta"], hd)
    cs, sn = np.cos(ang)[:, None, :], np.sin(ang)[:, None, :]

    def rope(v):  # v [n, heads, hd]
        a, b = v[..., :half].copy(), v[..., half:].copy()
        return np.concatenate([a * cs - b * sn, a * sn + b * cs], axis=2)

    x = w["embd"][np.asarray(tokens)].astype(np.float64)
    for L in range(cfg["n_layers"]):
        xn = bf16(norm(x, w["attn_norm"][L].astype(np.float64)))
        q = xn @ matb(cfg["attn_type"], w["wq"][L], nh * hd, H).T
        k = xn @ matb(cfg["attn_type"], w["wk"][L], nkv * hd, H).T
        v = xn @ matb(cfg["attn_type"], w["wv"][L], nkv * hd, H).T
        q = rope(q.reshape(n, nh, hd))
        k = rope(k.reshape(n, nkv, hd)).reshape(n, -1)
        if kv == "q8_0":
            for t in range(n):
                kc[L, pos0 + t] = pack_q8_0_rows(k[t].astype(np.float32))
                vc[L, pos0 + t] = pack_q8_0_rows(v[t].astype(np.float32))
            K = unpack_q8_0_rows(kc[L, :pos0 + n]).astype(np.float16).astype(np.float64)
            V = unpack_q8_0_rows(vc[L, :pos0 + n]).astype(np.float16).astype(np.float64)
            K, V = K.reshape(pos0 + n, nkv, hd), V.reshape(pos0 + n, nkv, hd)
        else:
            kc[L, pos0:pos0 + n] = k.astype(np.float16).view(np.uint16)
            vc[L, pos0:pos0 + n] = v.astype(np.float16).view(np.uint16)
            K = kc[L, :pos0 + n].view(np.float16).astype(np.float64).reshape(pos0 + n, nkv, hd)
            V = vc[L, :pos0 + n].view(np.float16).astype(np.float64).reshape(pos0 + n, nkv, hd)
        att = np.empty((n, nh, hd))
        for h in range(nh):
            s = q[:, h, :] @ K[:, h // group, :].T / np.sqrt(hd)  # [n, pos0 + n]
            s[np.arange(pos0 + n)[None, :] > pos[:, None]] = -np.inf
            p = np.exp(s - s.max(axis=1, keepdims=True))
            att[:, h, :] = (p / p.sum(axis=1, keepdims=True)) @ V[:, h // group, :]
        x = x + bf16(att.reshape(n, -1)) @ matb(cfg["attn_type"], w["wo"][L], H, nh * hd).T
        xn = bf16(norm(x, w["ffn_norm"][L].astype(np.float64)))
        g = xn @ matb(cfg["gate_up_type"], w["wgate"][L], F, H).T
        u = xn @ matb(cfg["gate_up_type"], w["wup"][L], F, H).T
        with np.errstate(over="ignore"):
            act = g / (1.0 + np.exp(-g)) * u
        x = x + bf16(act) @ matb(cfg["down_type"], w["wdown"][L], H, F).T
    xn = norm(x[-1:], w["output_norm"].astype(np.float64))[0]
    return mat(cfg["head_type"], w["lm_head"], cfg["vocab"], H) @ xn
