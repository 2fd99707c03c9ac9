"""Pin the CPU oracle (oracle/gq_oracle.c) before trusting it as the checker.

Sources of truth, in order: the reference's own unit-test vectors
(src/quant/q8_0.rs:109-170, q4_k.rs:228-259, q6_k.rs:147-164,
q8_k.rs:97-138), closed forms written independently in numpy (npref.py),
exhaustive enumeration (f16, 6-bit scale packing), and fp64 brute force.
"""
import numpy as np
import pytest

import gq_synth as syn
import npref

Q8_0, Q4_K, Q5_K, Q6_K, IQ3 = 8, 12, 13, 14, 18


def f16b(v):
    return np.array([v], np.float16).view(np.uint16)[0]


# ----------------------------------------------------------------- formats
def test_type_sizes(orc):
    # src/types.rs:126-168
    assert orc.type_size(Q8_0, 2048) == 2176
    assert orc.type_size(Q4_K, 3584) == 2016
    assert orc.type_size(Q6_K, 18944) == 15540
    assert orc.type_size(Q6_K, 3584) == 2940
    assert orc.type_size(IQ3, 3072) == 1176
    assert orc.type_size(IQ3, 1536) == 588
    assert orc.type_size(Q8_0, 33) == 68
    assert orc.type_size(Q5_K, 256) == 176


def test_f16_to_f32_exhaustive(orc):
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    ref = bits.view(np.float16).astype(np.float32)
    got = np.array([orc.f16_to_f32(b) for b in bits], np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))


def test_f32_to_f16_rne(orc):
    rng = np.random.default_rng(3)
    vals = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * np.float32(0.01),
        rng.standard_normal(20000).astype(np.float32) * np.float32(1000),
        np.float32([0.0, -0.0, 65504, 65520, 65519.99, 1e-8, 6e-8, 2.98e-8, 3e-8, 1e-5, 6.1e-5,
                    np.inf, -np.inf]),
        # exact ties between two f16 values (RNE must pick the even one)
        (np.arange(1024, 2048, dtype=np.float32) + np.float32(0.5)),
    ])
    got = np.array([orc.f32_to_f16(v) for v in vals], np.uint16)
    ref = vals.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, ref)


# -------------------------------------------------------------------- Q8_0
def q8_block(scale_bits, values):
    b = np.zeros(34, np.uint8)
    b[0:2] = np.array([scale_bits], np.uint16).view(np.uint8)
    b[2:2 + len(values)] = np.array(values, np.int8).view(np.uint8)
    return b


def test_q8_0_single_block(orc):
    # q8_0.rs:109-126
    vals = [(i % 5) - 2 for i in range(32)]
    y = orc.dequant(Q8_0, q8_block(f16b(2.0), vals), 32)
    assert np.all(np.abs(y - 2.0 * np.array(vals, np.float32)) < 1e-6)


def test_q8_0_partial_block(orc):
    # q8_0.rs:129-148
    data = np.concatenate([q8_block(f16b(1.0), list(range(32))), q8_block(f16b(1.0), [42])])
    y = orc.dequant(Q8_0, data, 33)
    assert y.shape == (33,) and y[32] == 42.0


def test_q8_0_dot_matches_dequant(orc):
    # q8_0.rs:151-170
    data = np.concatenate([q8_block(f16b(0.75), [((i + b) % 7) - 3 for i in range(32)])
                           for b in range(3)])
    n = 70
    x = (np.arange(n, dtype=np.float32) * np.float32(0.1) - np.float32(3.0)).astype(np.float32)
    row = orc.dequant(Q8_0, data, n)
    assert abs(orc.dot_row(Q8_0, data, x) - float(np.sum(row * x, dtype=np.float32))) < 1e-3


# -------------------------------------------------------------------- Q4_K
def test_get_scale_min_k4_known_answers(orc):
    # q4_k.rs:228-241
    s = np.array([10, 20, 30, 40, 50, 60, 70, 80, 0, 0, 0, 0], np.uint8)
    assert orc.get_scale_min_k4(0, s) == (10, 50)
    assert orc.get_scale_min_k4(1, s) == (20, 60)
    assert orc.get_scale_min_k4(2, s) == (30, 6)
    assert orc.get_scale_min_k4(3, s) == (40, 16)
    s = np.array([0xC0, 0x80, 0x40, 0, 0, 0, 0, 0, 0x3F, 0x2F, 0x1F, 0x0F], np.uint8)
    assert orc.get_scale_min_k4(4, s) == (0x3F, 3)
    assert orc.get_scale_min_k4(5, s) == (0x2F, 2)


def test_scale_min_pack_roundtrip_all_pairs(orc):
    # every (sc, m) in 64 x 64 in every sub-block slot round-trips through
    # the generator's packing and the oracle's unpacking
    sc = np.arange(64 * 64, dtype=np.uint32) // 64
    m = np.arange(64 * 64, dtype=np.uint32) % 64
    for j in range(8):
        scs = np.zeros((4096, 8), np.uint8)
        ms = np.zeros((4096, 8), np.uint8)
        scs[:, j] = sc
        ms[:, j] = m
        packed = syn.pack_scale_min_k4(scs, ms)
        usc, um = npref.unpack_k4_scales(packed)
        assert np.array_equal(usc[:, j], sc) and np.array_equal(um[:, j], m)
        for i in range(0, 4096, 257):
            assert orc.get_scale_min_k4(j, packed[i]) == (int(sc[i]), int(m[i]))


def test_q4_k_dot_matches_dequant(orc):
    # q4_k.rs:243-259
    b = np.zeros(144, np.uint8)
    b[0:2] = np.array([f16b(0.05)], np.uint16).view(np.uint8)
    b[2:4] = np.array([f16b(-0.01)], np.uint16).view(np.uint8)
    b[4:16] = [10, 20, 30, 40, 50, 60, 70, 80, 0x3F, 0x2F, 0x1F, 0x0F]
    b[16:] = (np.arange(128) * 13) % 256
    x = (np.arange(256, dtype=np.float32) * np.float32(0.01) - np.float32(1.0)).astype(np.float32)
    row = orc.dequant(Q4_K, b, 256)
    assert abs(orc.dot_row(Q4_K, b, x) - float(np.sum(row * x, dtype=np.float32))) < 1e-3


# -------------------------------------------------------------------- Q6_K
def test_q6_k_dot_matches_dequant(orc):
    # q6_k.rs:147-164
    b = np.zeros(210, np.uint8)
    b[0:128] = (np.arange(128) * 37) % 256
    b[128:192] = (np.arange(64) * 53 + 1) % 256
    b[192:208] = (np.arange(16) - 6).astype(np.int8).view(np.uint8)
    b[208:210] = np.array([f16b(0.02)], np.uint16).view(np.uint8)
    x = (np.arange(256, dtype=np.float32) * np.float32(0.005) - np.float32(0.6)).astype(np.float32)
    row = orc.dequant(Q6_K, b, 256)
    assert abs(orc.dot_row(Q6_K, b, x) - float(np.sum(row * x, dtype=np.float32))) < 1e-2


def test_q6_k_every_code_and_scale(orc):
    # one-hot blocks: each 6-bit code at each element position with a
    # scale/sign pattern; the decoded value must be d*sc*(code-32)
    d = 0.5
    for e in range(0, 256, 7):
        for code in (0, 1, 31, 32, 33, 63):
            b = np.zeros(210, np.uint8)
            h, t, l = e // 128, (e % 128) // 32, e % 32
            qi = 64 * h + l + (32 if t & 1 else 0)
            lo = code & 0xF
            b[qi] = (lo << 4) if t >= 2 else lo
            b[128 + 32 * h + l] = ((code >> 4) & 3) << (2 * t)
            s = np.arange(16, dtype=np.int8) - 8
            b[192:208] = s.view(np.uint8)
            b[208:210] = np.array([f16b(d)], np.uint16).view(np.uint8)
            y = orc.dequant(Q6_K, b, 256)
            sidx = 8 * h + l // 16 + 2 * t
            assert y[e] == np.float32(d) * np.float32(s[sidx]) * np.float32(code - 32)


# ------------------------------------------------ closed forms vs the oracle
@pytest.mark.parametrize("dtype", [Q8_0, Q4_K, Q5_K, Q6_K, IQ3])
@pytest.mark.parametrize("n", [256, 512, 70, 300])
def test_dequant_bit_exact_vs_numpy(orc, dtype, n):
    if dtype != Q8_0 and n % 256 and n < 256:
        pytest.skip("K-quant rows shorter than a block are not a GGUF shape")
    w = syn.make_blocks(dtype, 7, n, seed=n + dtype)
    grid = orc.get_iq3xxs_grid()
    for r in range(7):
        got = orc.dequant(dtype, w[r], n)
        ref = npref.dequant(dtype, w[r], n, grid)
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), (dtype, r)


@pytest.mark.parametrize("dtype", [Q8_0, Q4_K, Q5_K, Q6_K, IQ3])
def test_dot_vs_fp64_brute_force(orc, dtype):
    n = 1024
    w = syn.make_blocks(dtype, 16, n, seed=11)
    x = syn.make_x(n, seed=12)
    grid = orc.get_iq3xxs_grid()
    for r in range(16):
        ref = float(np.dot(npref.dequant(dtype, w[r], n, grid).astype(np.float64),
                           x.astype(np.float64)))
        got = orc.dot_row(dtype, w[r], x)
        scale = float(np.sum(np.abs(npref.dequant(dtype, w[r], n, grid) * x)))
        assert abs(got - ref) <= 1e-5 * scale + 1e-30


def test_q4_k_dot_lane_order_matters(orc):
    # The oracle follows dot_q4_k_group's 8-lane accumulation (q4_k.rs:152-203);
    # a plain sequential sum differs in the last bits on random data, which
    # shows the restated order is actually exercised.
    w = syn.make_blocks(Q4_K, 64, 2048, seed=5)
    x = syn.make_x(2048, seed=6)
    diff = 0
    for r in range(64):
        row = orc.dequant(Q4_K, w[r], 2048)
        seq = np.float32(0)
        for v in (row * x):
            seq = np.float32(seq + v)
        diff += orc.dot_row(Q4_K, w[r], x) != seq
    assert diff > 0


def test_matmul_into_equals_rows(orc):
    w = syn.make_blocks(Q4_K, 33, 512, seed=2)
    x = syn.make_x(512, seed=3)
    y = orc.matmul_into(Q4_K, w, x, 33, nthreads=4)
    y1 = orc.matmul_dequant(Q4_K, w, x, 33)
    assert np.array_equal(y, y1)
    assert np.array_equal(y, np.array([orc.dot_row(Q4_K, w[r], x) for r in range(33)], np.float32))


def test_matmul_batch_into(orc):
    w = syn.make_blocks(Q6_K, 20, 512, seed=4)
    X = syn.make_x(512, seed=5, batch=3)
    Y = orc.matmul_batch_into(Q6_K, w, X, 20, nthreads=3)
    W = np.stack([npref.dequant_q6_k(w[r], 512) for r in range(20)]).astype(np.float64)
    ref = X.astype(np.float64) @ W.T
    assert np.max(np.abs(Y - ref)) <= 1e-5 * np.max(np.abs(ref))


def test_errors(orc):
    w = syn.make_blocks(Q4_K, 1, 512, seed=1)
    with pytest.raises(orc.OracleError):
        orc.dot_row(Q4_K, w[0][:200], syn.make_x(512))
    with pytest.raises(orc.OracleError):
        orc.matmul_into(0, w, syn.make_x(512), 1)
    # all-zero weights (warmup) succeed and give zeros
    z = syn.make_blocks(Q6_K, 4, 256, zero=True)
    assert np.all(orc.matmul_into(Q6_K, z, syn.make_x(256), 4) == 0)


# -------------------------------------------------------------------- Q8_K
def test_q8_k_roundtrip_bsums_zero_partial(orc):
    # q8_k.rs:97-138
    x = ((np.arange(256, dtype=np.float32) - 128) * np.float32(0.1)).astype(np.float32)
    d, qs, bs = orc.quantize_row_q8_k(x)
    assert d.size == 1
    assert np.all(np.abs(d[0] * qs.astype(np.float32) - x) < 0.15)
    x = (((np.arange(256) % 7) - 3) * 0.3).astype(np.float32)
    d, qs, bs = orc.quantize_row_q8_k(x)
    assert np.array_equal(bs, qs.reshape(16, 16).astype(np.int16).sum(1))
    d, qs, bs = orc.quantize_row_q8_k(np.zeros(256, np.float32))
    assert d[0] == 0 and np.all(qs == 0)
    d, qs, bs = orc.quantize_row_q8_k((np.arange(100) * 0.01).astype(np.float32))
    assert d.size == 1 and qs.size == 256 and bs.size == 16


def test_q8_k_vs_numpy(orc):
    x = syn.make_x(1000, seed=8)
    d, qs, bs = orc.quantize_row_q8_k(x)
    d2, qs2, bs2 = npref.quantize_row_q8_k(x)
    assert np.array_equal(d, d2) and np.array_equal(qs, qs2) and np.array_equal(bs, bs2)


def test_dot_q5_k_q8k_close_to_float(orc):
    n = 512
    w = syn.make_blocks(Q5_K, 4, n, seed=9)
    x = syn.make_x(n, seed=10)
    d, qs, bs = orc.quantize_row_q8_k(x)
    xq = (np.repeat(d, 256) * qs.astype(np.float32))[:n]
    for r in range(4):
        ref = float(np.dot(npref.dequant_k4(w[r], n, q5=True).astype(np.float64), xq))
        got = orc.dot_q5_k_q8k(w[r], n, d, qs, bs)
        assert abs(got - ref) <= 1e-5 * max(1.0, abs(ref))


# ------------------------------------------------------ per-32 Q8 pack
def test_quantize_q8_32_vs_numpy(orc):
    x = syn.make_x(4096, seed=13)
    x[64:96] = 0  # all-zero block -> scale 1.0, q = 0
    sc, q = orc.quantize_q8_32(x)
    sc2, q2 = npref.quantize_q8_32(x)
    assert np.array_equal(sc, sc2) and np.array_equal(q, q2)
    assert sc[2] == f16b(1.0) and np.all(q[64:96] == 0)
    assert np.all(np.abs(q.astype(np.int32)) <= 127)


# ---------------------------------------------------------------- IQ3_XXS
def test_iq3_signs_have_even_parity():
    ks = npref.ksigns()
    assert all(bin(int(v)).count("1") % 2 == 0 for v in ks)
    assert np.array_equal(ks & 127, np.arange(128))


def test_iq3_grid_install(orc):
    g0 = orc.get_iq3xxs_grid()
    mags = {4, 12, 20, 28, 36, 44, 52, 62}
    assert all(b in mags for b in g0.view(np.uint8))
    custom = np.arange(256, dtype=np.uint32) * 0x01010101
    orc.set_iq3xxs_grid(custom)
    try:
        w = syn.make_blocks(IQ3, 1, 256, seed=1)
        assert np.array_equal(orc.dequant(IQ3, w[0], 256),
                              npref.dequant_iq3_xxs(w[0], 256, custom))
    finally:
        orc.set_iq3xxs_grid(None)
    assert np.array_equal(orc.get_iq3xxs_grid(), g0)


def test_iq3_one_hot_fields(orc):
    """Scale nibbles, sign indices and grid slots of the oracle's IQ3_XXS
    dequant against closed forms (tests/iq3_onehot.py)."""
    import iq3_onehot as oh
    g0 = orc.get_iq3xxs_grid()
    orc.set_iq3xxs_grid(oh.IDENT_GRID)
    try:
        b, exp = oh.scale_blocks(oh.IDENT_GRID)
        y = orc.dequant(IQ3, b.reshape(-1), 16 * 256).reshape(16, 256)
        assert np.array_equal(y.astype(np.float64), exp)
        b, mags, idx = oh.sign_blocks(oh.IDENT_GRID)
        oh.check_signs(orc.dequant(IQ3, b.reshape(-1), 4 * 256).reshape(4, 256), mags, idx)
        b, exp = oh.grid_blocks(oh.IDENT_GRID)
        y = orc.dequant(IQ3, b.reshape(-1), 4 * 256).reshape(4, 256)
        assert np.array_equal(y.astype(np.float64), exp)
    finally:
        orc.set_iq3xxs_grid(g0)


def test_matmul_into_q5_k_takes_the_q8_k_route(orc):
    """model/mod.rs:381-394: for Q5_K, matmul_into quantizes x to Q8_K once
    and runs dot_q5_k_q8k per row; CpuBackend::matmul_dequant and
    ffn_gate_up run the float dot_row.  The two routes differ by the Q8_K
    rounding of x (about 1/254 of a block's max per element)."""
    rows, n = 40, 1024
    w = syn.make_blocks(Q5_K, rows, n, seed=31)
    x = syn.make_x(n, seed=32)
    y = orc.matmul_into(Q5_K, w, x, rows, nthreads=3)
    d, qs, bs = orc.quantize_row_q8_k(x)
    assert np.array_equal(y, np.array([orc.dot_q5_k_q8k(w[r], n, d, qs, bs) for r in range(rows)],
                                      np.float32))
    yf = orc.matmul_rows(Q5_K, w, x, rows)
    assert np.array_equal(yf, orc.matmul_dequant(Q5_K, w, x, rows))
    assert np.array_equal(yf, np.array([orc.dot_row(Q5_K, w[r], x) for r in range(rows)], np.float32))
    gap = np.abs(y - yf).max() / np.abs(yf).max()
    assert 1e-4 < gap < 2e-2, gap
    # Q8_K x against the exact float dot: the quantized-x product in fp64
    xq = (np.repeat(d, 256) * qs.astype(np.float32)).astype(np.float64)[:n]
    W = np.stack([npref.dequant_k4(w[r], n, q5=True) for r in range(rows)]).astype(np.float64)
    ref = W @ xq
    assert np.abs(y - ref).max() <= 1e-5 * np.abs(ref).max()
    # the other types: matmul_into == matmul_rows
    w4 = syn.make_blocks(Q4_K, 8, 512, seed=2)
    x4 = syn.make_x(512, seed=3)
    assert np.array_equal(orc.matmul_into(Q4_K, w4, x4, 8), orc.matmul_rows(Q4_K, w4, x4, 8))


def test_argmax_first_max_wins(orc):
    # sampler.rs:120-131
    assert orc.argmax(np.array([1, 3, 3, 2], np.float32)) == 1
    assert orc.argmax(np.array([-np.inf, -np.inf], np.float32)) == 0


# -------------------------------------------------------------------- MoE
def test_moe_route_vs_numpy(orc):
    rng = np.random.default_rng(5)
    logits = rng.standard_normal((7, 256), dtype=np.float32)
    logits[3, 10] = logits[3, 20] = 9.0  # a tie: lower index first
    ids, w = orc.moe_route(logits, 8)
    for t in range(7):
        order = sorted(range(256), key=lambda e: (-logits[t, e], e))[:8]
        assert list(ids[t]) == order
        p = np.exp(logits[t].astype(np.float64) - logits[t].max())
        p /= p.sum()
        assert np.allclose(w[t], p[order], rtol=1e-5)
    assert ids[3, 0] == 10 and ids[3, 1] == 20


def test_moe_ffn_vs_numpy(orc):
    E, H, F, T, k = 6, 256, 512, 3, 2
    gate = syn.make_blocks(18, E * F, H, seed=1)
    up = syn.make_blocks(18, E * F, H, seed=2)
    down = syn.make_blocks(18, E * H, F, seed=3)
    x = syn.make_x(H, seed=4, batch=T)
    logits = np.random.default_rng(6).standard_normal((T, E), dtype=np.float32)
    ids, w = orc.moe_route(logits, k)
    out = orc.moe_ffn(18, gate, up, down, E, H, F, x, ids, w, nthreads=4)
    grid = orc.get_iq3xxs_grid()
    Wg = np.stack([npref.dequant_iq3_xxs(gate[r], H, grid) for r in range(E * F)]).astype(np.float64)
    Wu = np.stack([npref.dequant_iq3_xxs(up[r], H, grid) for r in range(E * F)]).astype(np.float64)
    Wd = np.stack([npref.dequant_iq3_xxs(down[r], F, grid) for r in range(E * H)]).astype(np.float64)
    for t in range(T):
        ref = np.zeros(H)
        for s in range(k):
            e = ids[t, s]
            g = Wg[e * F:(e + 1) * F] @ x[t]
            u = Wu[e * F:(e + 1) * F] @ x[t]
            hmid = g / (1 + np.exp(-g)) * u
            ref += w[t, s] * (Wd[e * H:(e + 1) * H] @ hmid)
        assert np.max(np.abs(out[t] - ref)) <= 1e-4 * np.max(np.abs(ref))


TINY_MODEL = dict(n_layers=2, hidden=256, n_heads=4, n_kv_heads=2, head_dim=64, ffn=512,
                  vocab=300, ctx=24, eps=1e-6, theta=1e6, attn_type=Q4_K, gate_up_type=Q4_K,
                  down_type=Q6_K, head_type=Q6_K)


def test_decode_step_vs_numpy(orc):
    """gqo_decode_step (cpu_path.rs:695-818) against an independent float64
    restatement: same logits to fp32 accumulation error, same KV rows up to
    one f16 rounding step.  An embedding scaled by 1e4 keeps every term of
    the residual stream visible in the logits."""
    cfg = TINY_MODEL
    w = syn.make_decoder(cfg, 21, embd_scale=1e4)
    kv = syn.make_kv(cfg, 16, 22)
    om = orc.DecoderModel(cfg, w, kv)
    kc = np.zeros_like(om.kc)
    vc = np.zeros_like(om.vc)
    kc[:, :16], vc[:, :16] = kv
    for pos, tok in ((16, 7), (17, 250), (18, 0)):
        got = om.step(tok, pos)
        ref = npref.decode_step(cfg, w, kc, vc, tok, pos)
        assert np.abs(got - ref).max() <= 1e-4 * np.abs(ref).max(), pos
        assert orc.argmax(got) == int(np.argmax(ref))
    for arr_o, arr_r in ((om.kc, kc), (om.vc, vc)):
        a = arr_o[:, :19].view(np.float16).astype(np.float64)
        b = arr_r[:, :19].view(np.float16).astype(np.float64)
        assert np.allclose(a, b, rtol=2e-3, atol=1e-3)


def test_decode_step_q8_0_kv_vs_numpy(orc):
    """The Q8_0 KV cache (KvDtype::Q8_0, model/mod.rs:540-603) in the
    oracle's decode step against the float64 restatement packing with
    npref.quantize_q8_32: same logits to fp32 error, and every stored value
    within one quantization step (inputs that differ in the last fp32 bits
    may round to neighbouring int8 codes)."""
    cfg = TINY_MODEL
    w = syn.make_decoder(cfg, 25, embd_scale=1e4)
    om = orc.DecoderModel(cfg, w, kv_dtype="q8_0")
    kc = np.zeros_like(om.kc)
    vc = np.zeros_like(om.vc)
    assert kc.dtype == np.uint8 and kc.shape[2] == cfg["n_kv_heads"] * cfg["head_dim"] // 32 * 34
    for pos, tok in enumerate((7, 250, 0, 33)):
        got = om.step(tok, pos)
        ref = npref.decode_step(cfg, w, kc, vc, tok, pos)
        assert np.abs(got - ref).max() <= 1e-4 * np.abs(ref).max(), pos
    for arr_o, arr_r in ((om.kc, kc), (om.vc, vc)):
        for l in range(cfg["n_layers"]):
            a = npref.unpack_q8_0_rows(arr_o[l, :4])
            b = npref.unpack_q8_0_rows(arr_r[l, :4])
            step = np.repeat(np.abs(b).reshape(4, -1, 32).max(axis=2) / 127.0, 32, axis=1)
            assert np.all(np.abs(a - b) <= 1.01 * step + 1e-30)


def test_decode_step_first_position(orc):
    """At position 0 RoPE is the identity and attention over one position
    returns v itself: the oracle's step equals the numpy step there too."""
    cfg = dict(TINY_MODEL, n_layers=1)
    w = syn.make_decoder(cfg, 23, embd_scale=1e4)
    om = orc.DecoderModel(cfg, w)
    kc = np.zeros_like(om.kc)
    vc = np.zeros_like(om.vc)
    got = om.step(3, 0)
    ref = npref.decode_step(cfg, w, kc, vc, 3, 0)
    assert np.abs(got - ref).max() <= 1e-4 * np.abs(ref).max()
    a = om.vc[0, 0].view(np.float16).astype(np.float64)
    b = vc[0, 0].view(np.float16).astype(np.float64)
    assert np.allclose(a, b, rtol=2e-3, atol=1e-3)
