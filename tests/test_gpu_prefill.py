"""GPU batched prefill (gq_model_prefill) against two CPU references.

1. npref.prefill_bf16: run_batch (src/model/llama/cpu_path.rs:834-991)
   restated in float64 with the GPU prefill's operand rounding at each
   projection (weights: bf16 of the exact fp32 dequant; activations: fp32
   then bf16).  Same operands up to rounding ties: an activation whose fp32
   value lies within an fp32 ulp of a bf16 (or f16 K/V) rounding tie may
   round the other way (a 2^-9 step in one GEMM input).  The K/V rows of
   the first layer agree to a few f16 ulps; later layers inherit the ties'
   steps, so the median row agrees to <= 1e-4 of max|value| (observed 0)
   and the worst row to 1e-2 (observed <= 6e-3 at 600 tokens); the logits
   to <= 2e-3 * max|ref| (observed 2e-7 .. 8e-4).
2. The oracle's sequential fp32 path (LlamaModel::run, cpu_path.rs:695-818;
   prefilling a prompt is, token by token, the same arithmetic).  The bf16
   operands (2^-9 relative each) set the distance: logits <= 2e-2 * max|ref|,
   and the greedy token is compared where the top-2 margin exceeds the error.
The synthetic decoders' activations are large (attention scores ~ 1e4, a
near-argmax softmax): keys within an fp32 rounding of a tie swap between
any two summation orders, and after the first layer a few tokens' K/V rows
move by percents.  The same-rounding checks therefore scale the attention
norm weights down (scores ~ 10); the fp32-path check uses the model as is.
"""
import numpy as np
import pytest

import gq_synth as syn
import npref
import oracle

pytestmark = pytest.mark.gpu

SMALL = dict(n_layers=2, hidden=256, n_heads=4, n_kv_heads=2, head_dim=64, ffn=512, vocab=1000,
             ctx=1400, eps=1e-6, theta=1e6, attn_type=syn.Q4_K, gate_up_type=syn.Q4_K,
             down_type=syn.Q6_K, head_type=syn.Q6_K)
HD128 = dict(SMALL, hidden=512, n_heads=4, n_kv_heads=1, head_dim=128, ffn=768)

TOL_SAME = 2e-3   # vs the same-rounding reference (logits)
# A Q8_0 KV cache: a rounding tie flips a code, 1/127 of its block's max
# (16x an f16 ulp), and later layers inherit it.
TOL_SAME_Q8KV = 1e-2
KV_SAME = 1e-2    # K/V rows vs the same-rounding reference (worst row), of max|value|
KV_MEDIAN = 1e-4  # ... and the median row (rounding ties are rare: observed 0)
TOL_FP32 = 2e-2   # vs the fp32 CPU path (bf16 operands)
ATTN_SCALE = 0.05  # attention-norm scale of the same-rounding models


def say(*a):
    print(*a, flush=True)


def _build(backend, cfg, seed, n_ctx, embd_scale=1.0, attn_scale=1.0):
    import gq
    w = syn.make_decoder(cfg, seed, embd_scale=embd_scale)
    if attn_scale != 1.0:  # smaller q, k, v: a well-conditioned softmax
        w["attn_norm"] = [np.float32(attn_scale) * a for a in w["attn_norm"]]
    kv = syn.make_kv(cfg, n_ctx, seed + 1) if n_ctx else None
    hw = syn.upload_decoder(backend, cfg, w)
    gm = gq.DecodeModel(dict(cfg, max_tokens=1024), hw)
    kvd = cfg["n_kv_heads"] * cfg["head_dim"]
    kc = np.zeros((cfg["n_layers"], cfg["ctx"], kvd), np.uint16)
    vc = kc.copy()
    if kv is not None:
        for l in range(cfg["n_layers"]):
            gm.kv_upload(l, kv[0][l], kv[1][l])
            kc[l, :n_ctx], vc[l, :n_ctx] = kv[0][l], kv[1][l]
    return gm, w, kv, kc, vc


def _f16(a):
    return a.view(np.float16).astype(np.float32)


# Projection-type mixes beyond Q4_K_M: an all-Q8_0 model (the Llama-3.2-1B
# Q8_0 file type of BASELINE configs[0]) and a Q5_K_M-like one.
MIXES = {"Q4_K_M": {}, "Q8_0": dict(attn_type=syn.Q8_0, gate_up_type=syn.Q8_0, down_type=syn.Q8_0,
                                    head_type=syn.Q8_0),
         "Q5_K_M": dict(attn_type=syn.Q5_K, gate_up_type=syn.Q5_K, down_type=syn.Q6_K)}


CASES = [("SMALL", 0, 37, "Q4_K_M"), ("SMALL", 100, 64, "Q4_K_M"), ("HD128", 70, 130, "Q4_K_M"),
         ("SMALL", 5, 600, "Q4_K_M"), ("HD128", 0, 300, "Q4_K_M"), ("SMALL", 100, 64, "Q8_0"),
         ("SMALL", 5, 600, "Q8_0"), ("HD128", 70, 300, "Q8_0"), ("SMALL", 30, 200, "Q5_K_M"),
         ("HD128", 0, 130, "Q5_K_M"), ("SMALL", 20000, 64, "Q4_K_M"), ("HD128", 9000, 130, "Q4_K_M")]
# Embedding scale of the same-rounding models.  The all-Q8_0 decoders (zero-
# mean rows, no per-block bias to dominate the residual) are ill-conditioned
# at an N(0, 1) embedding: a 1e-7 relative change of the embedding moves the
# same-rounding reference's own logits by 2e-3 to 4e-3 of their max after
# two layers, so no two roundings agree to TOL_SAME.  A x100 embedding (the
# token drives the residual) brings that to <= 4e-5.
MIX_EMBD = {"Q4_K_M": 1.0, "Q5_K_M": 1.0, "Q8_0": 100.0}


@pytest.mark.parametrize("cfg_name,n_ctx,n,mix", CASES)
def test_prefill_same_rounding(backend, cfg_name, n_ctx, n, mix):
    """Logits and every K/V row written against npref.prefill_bf16; the
    rows before the prompt are untouched.  n = 600 takes two passes; 20000
    and 9000 cached positions run the attention over long key ranges."""
    cfg = dict({"SMALL": SMALL, "HD128": HD128}[cfg_name], **MIXES[mix])
    cfg["ctx"] = max(cfg["ctx"], n_ctx + n + 8)
    say(f"prefill {cfg_name} ({mix}) n_ctx={n_ctx} n={n}")
    gm, w, kv, kc, vc = _build(backend, cfg, seed=11 + n, n_ctx=n_ctx, attn_scale=ATTN_SCALE,
                               embd_scale=MIX_EMBD[mix])
    toks = np.random.default_rng(n).integers(0, cfg["vocab"], n).astype(np.int32)
    nxt, got = gm.prefill(toks, n_ctx)
    ref = npref.prefill_bf16(cfg, w, kc, vc, toks, n_ctx)
    err = float(np.abs(got - ref).max())
    say(f"  logits max|err| {err:.3g} of {float(np.abs(ref).max()):.3g}")
    assert nxt == int(np.argmax(got))
    for l in range(cfg["n_layers"]):
        k, v = gm.kv_download(l, n_ctx + n)
        if n_ctx:
            np.testing.assert_array_equal(k[:n_ctx], kv[0][l])
            np.testing.assert_array_equal(v[:n_ctx], kv[1][l])
        for nm, got_rows, ref_rows in (("K", k, kc[l]), ("V", v, vc[l])):
            g, r = _f16(got_rows[n_ctx:]), _f16(ref_rows[n_ctx:n_ctx + n])
            rows = np.abs(g - r).max(axis=1)
            top = float(np.abs(r).max())
            say(f"  layer {l} {nm} max|err| {rows.max():.3g} median {np.median(rows):.3g} of {top:.3g}")
            assert rows.max() <= KV_SAME * top
            assert np.median(rows) <= KV_MEDIAN * top
    assert err <= TOL_SAME * float(np.abs(ref).max())


# (The all-Q8_0 model is checked against the same-rounding reference only:
# its zero-mean rows make logits of order 10, and the near-argmax softmax of
# the unscaled model moves them by percents between any two roundings.)
@pytest.mark.parametrize("cfg_name,n_ctx,n,mix", [("SMALL", 100, 64, "Q4_K_M"), ("HD128", 70, 130, "Q4_K_M"),
                                                  ("SMALL", 30, 200, "Q5_K_M"), ("HD128", 0, 130, "Q5_K_M")])
def test_prefill_vs_fp32_oracle(backend, cfg_name, n_ctx, n, mix):
    cfg = dict({"SMALL": SMALL, "HD128": HD128}[cfg_name], **MIXES[mix])
    gm, w, kv, _, _ = _build(backend, cfg, seed=11 + n, n_ctx=n_ctx)
    om = oracle.DecoderModel(cfg, w, kv)
    toks = np.random.default_rng(n).integers(0, cfg["vocab"], n).astype(np.int32)
    nxt, got = gm.prefill(toks, n_ctx)
    for i, t in enumerate(toks):
        ref = om.step(int(t), n_ctx + i)
    err = float(np.abs(got - ref).max())
    say(f"fp32 path ({mix}): logits max|err| {err:.3g} of {float(np.abs(ref).max()):.3g}")
    assert err <= TOL_FP32 * float(np.abs(ref).max())
    top = np.sort(ref)[-2:]
    if top[1] - top[0] > 2 * err:
        assert nxt == oracle.argmax(ref)


def test_prefill_then_generate(backend):
    """A token-driven model (large embedding): the prompt through prefill,
    then greedy decode on the GPU, against the oracle stepping the prompt
    and decoding."""
    cfg = SMALL
    gm, w, kv, _, _ = _build(backend, cfg, seed=21, n_ctx=40, embd_scale=1e5)
    om = oracle.DecoderModel(cfg, w, kv)
    toks = np.random.default_rng(7).integers(0, cfg["vocab"], 50).astype(np.int32)
    nxt, _ = gm.prefill(toks, 40, want_logits=False)
    for i, t in enumerate(toks):
        ref = om.step(int(t), 40 + i)
    assert nxt == oracle.argmax(ref)
    got = gm.generate(nxt, 90, 16)
    exp = []
    tok = nxt
    for i in range(16):
        tok = oracle.argmax(om.step(tok, 90 + i))
        exp.append(tok)
    np.testing.assert_array_equal(got, np.array(exp, np.int32))


def test_prefill_errors(backend):
    import gq
    gm = _build(backend, SMALL, seed=3, n_ctx=0)[0]
    with pytest.raises(gq.GqError, match="out of range"):
        gm.prefill(np.array([1, SMALL["vocab"]], np.int32), 0)
    with pytest.raises(gq.GqError, match="exceed the context"):
        gm.prefill(np.zeros(10, np.int32), SMALL["ctx"] - 5)
    with pytest.raises(gq.GqError, match="at least one token"):
        gm.prefill(np.zeros(0, np.int32), 0)
    iq3 = dict(SMALL, gate_up_type=syn.IQ3_XXS)
    giq = _build(backend, iq3, seed=4, n_ctx=0)[0]
    with pytest.raises(gq.GqError, match="Q4_K, Q5_K, Q6_K or Q8_0"):
        giq.prefill(np.zeros(4, np.int32), 0)


def test_prefill_next_token_skips_nan(backend):
    """A NaN logit at index 0 (the head's row 0 has a NaN scale) never wins
    the greedy pick: prefill's next token, decode's and the sampler's
    first-maximum rule from -inf (sampler.rs:120-131) agree."""
    import gq
    cfg = SMALL
    w = syn.make_decoder(cfg, 41, embd_scale=1e4)
    head = w["lm_head"].copy()
    head[0, 208:210] = np.array([0x7E00], np.uint16).view(np.uint8)  # Q6_K d of row 0, block 0
    w["lm_head"] = head
    hw = syn.upload_decoder(backend, cfg, w)
    gm = gq.DecodeModel(dict(cfg, max_tokens=64), hw)
    toks = np.array([3, 14, 15, 92], np.int32)
    nxt, lg = gm.prefill(toks, 0)
    assert np.isnan(lg[0]) and not np.isnan(lg[1:]).any()
    assert nxt == int(np.nanargmax(lg)) == oracle.argmax(lg)
    gm2 = gq.DecodeModel(dict(cfg, max_tokens=64), hw)
    for pos, t in enumerate(toks[:-1]):
        gm2.decode(int(t), pos, want_logits=False)
    nxt2, lg2 = gm2.decode(int(toks[-1]), len(toks) - 1)
    assert np.isnan(lg2[0]) and nxt2 == oracle.argmax(lg2)


@pytest.mark.parametrize("cfg_name,n_ctx,n,mix", [("SMALL", 100, 64, "Q4_K_M"), ("HD128", 70, 130, "Q4_K_M"),
                                                  ("SMALL", 5, 600, "Q4_K_M"), ("HD128", 40, 100, "Q8_0")])
def test_prefill_q8_0_kv(backend, cfg_name, n_ctx, n, mix):
    """Prefill into a Q8_0 KV cache (KvDtype::Q8_0, src/model/mod.rs:536-603):
    run_batch writes each prompt row packed and attends over the unpacked
    rows (cpu_path.rs:904-906).  Against npref.prefill_bf16 with the same
    cache type (the new rows packed from their fp32 values, every row read
    as f16(code * scale)): logits to TOL_SAME_Q8KV; the packed prompt rows' codes
    equal but for rounding ties (a value within an fp32 ulp of a code
    boundary, and what later layers inherit of them: at most 1% of the
    codes, and the unpacked rows to KV_SAME of the layer's max); the uploaded
    rows untouched; every block with a nonzero scale holds a code of
    magnitude 127 (the scale is f16(max|x| / 127)).  Then the oracle
    (LlamaModel::run with the Q8_0 cache) takes the GPU's rows and both
    decode greedily: the same tokens."""
    import gq
    cfg = dict({"SMALL": SMALL, "HD128": HD128}[cfg_name], **MIXES[mix], kv_dtype="q8_0")
    w = syn.make_decoder(cfg, 51 + n, embd_scale=1e4)
    w["attn_norm"] = [np.float32(ATTN_SCALE) * a for a in w["attn_norm"]]
    L, kvd = cfg["n_layers"], cfg["n_kv_heads"] * cfg["head_dim"]
    rng = np.random.default_rng(n)
    kv = [np.stack([np.stack([npref.pack_q8_0_rows(rng.standard_normal(kvd).astype(np.float32))
                              for _ in range(n_ctx)]) for _ in range(L)]) if n_ctx else
          np.zeros((L, 0, kvd // 32 * 34), np.uint8) for _ in range(2)]
    hw = syn.upload_decoder(backend, cfg, w)
    gm = gq.DecodeModel(dict(cfg, max_tokens=64), hw)
    if n_ctx:
        for l in range(L):
            gm.kv_upload(l, kv[0][l], kv[1][l])
    kc = np.zeros((L, cfg["ctx"], kvd // 32 * 34), np.uint8)
    vc = kc.copy()
    kc[:, :n_ctx], vc[:, :n_ctx] = kv[0], kv[1]
    toks = np.random.default_rng(n + 1).integers(0, cfg["vocab"], n).astype(np.int32)
    nxt, got = gm.prefill(toks, n_ctx)
    ref = npref.prefill_bf16(cfg, w, kc, vc, toks, n_ctx, kv="q8_0")
    err = float(np.abs(got - ref).max())
    say(f"q8_0 prefill {cfg_name} ({mix}): logits max|err| {err:.3g} of {float(np.abs(ref).max()):.3g}")
    assert nxt == int(np.argmax(got))
    om = oracle.DecoderModel(cfg, w, kv, kv_dtype="q8_0")
    for l in range(L):
        k, v = gm.kv_download(l, n_ctx + n)
        np.testing.assert_array_equal(k[:n_ctx], kv[0][l])
        np.testing.assert_array_equal(v[:n_ctx], kv[1][l])
        for nm, got_rows, ref_rows in (("K", k, kc[l]), ("V", v, vc[l])):
            blk = got_rows[n_ctx:].reshape(n, -1, 34)
            codes = blk[:, :, 2:].view(np.int8).astype(np.int32)
            scale = blk[:, :, 0].astype(np.uint16) | (blk[:, :, 1].astype(np.uint16) << 8)
            assert np.all(np.abs(codes).max(axis=2)[scale != 0x3C00] == 127), (nm, l)
            rcodes = ref_rows[n_ctx:n_ctx + n].reshape(n, -1, 34)[:, :, 2:].view(np.int8).astype(np.int32)
            frac = float(np.mean(codes != rcodes))
            g = npref.unpack_q8_0_rows(got_rows[n_ctx:])
            r = npref.unpack_q8_0_rows(ref_rows[n_ctx:n_ctx + n])
            top = float(np.abs(r).max())
            say(f"  layer {l} {nm}: codes differing {frac:.3g}, max|err| {np.abs(g - r).max():.3g} of {top:.3g}")
            assert frac <= 1e-2
            assert np.abs(g - r).max() <= KV_SAME * top
        om.kc[l, :n_ctx + n] = k
        om.vc[l, :n_ctx + n] = v
    assert err <= TOL_SAME_Q8KV * float(np.abs(ref).max())
    exp, tok = [], nxt
    for i in range(12):
        tok = oracle.argmax(om.step(tok, n_ctx + n + i))
        exp.append(tok)
    np.testing.assert_array_equal(gm.generate(nxt, n_ctx + n, 12), np.array(exp, np.int32))


def test_prefill_same_rounding_7b_width(backend):
    """The same-rounding check at the 7B shapes of the GEMMs and the
    attention (hidden 3584, 28 / 4 heads of 128, ffn 18944; Q4_K_M types),
    two layers and a 1000-token vocabulary so that the float64 reference
    fits: 100 uploaded rows, a 300-token prompt.  At this width the bf16
    operand roundings make the reference itself sensitive: with attention
    norms x0.01 and FFN norms x0.006, scaling the embedding by 1 + 1e-6
    moves its logits by 2e-3 of their maximum and its layer-1 K rows by
    1e-3 (rms).  With zero-mean Q4_K rows, attention norms x0.001, FFN norms
    x0.002, embedding x100 and cached V ~ N(0, 30^2), that perturbation
    moves the logits by 2e-4 and the layer-1 K/V by 3e-4 (rms), while
    zeroing layer 0's FFN down / attention output moves the logits by 6e-2
    / 0.48 and the layer-1 K by 6e-2 / 0.9 (rms).  Logits to TOL_SAME;
    layer 0's K/V rows as in test_prefill_same_rounding; later layers'
    rows to KV_SAME (worst) and KV_RMS_7B (rms over all values)."""
    import gq
    KV_RMS_7B = 2e-3
    cfg = dict(syn.QWEN25_7B, n_layers=2, vocab=1000, ctx=512)
    n_ctx, n = 100, 300
    w = syn.make_decoder(cfg, 61, embd_scale=100.0, centered=True)
    w["attn_norm"] = [np.float32(0.001) * a for a in w["attn_norm"]]
    w["ffn_norm"] = [np.float32(0.002) * a for a in w["ffn_norm"]]
    k0, v0 = syn.make_kv(cfg, n_ctx, 62)
    v0 = (v0.view(np.float16) * np.float16(30.0)).view(np.uint16)
    hw = syn.upload_decoder(backend, cfg, w)
    gm = gq.DecodeModel(dict(cfg, max_tokens=64), hw)
    kvd = cfg["n_kv_heads"] * cfg["head_dim"]
    kc = np.zeros((cfg["n_layers"], cfg["ctx"], kvd), np.uint16)
    vc = kc.copy()
    for l in range(cfg["n_layers"]):
        gm.kv_upload(l, k0[l], v0[l])
        kc[l, :n_ctx], vc[l, :n_ctx] = k0[l], v0[l]
    toks = np.random.default_rng(63).integers(0, cfg["vocab"], n).astype(np.int32)
    nxt, got = gm.prefill(toks, n_ctx)
    ref = npref.prefill_bf16(cfg, w, kc, vc, toks, n_ctx)
    err = float(np.abs(got - ref).max())
    say(f"7b width: logits max|err| {err:.3g} of {float(np.abs(ref).max()):.3g}")
    for l in range(cfg["n_layers"]):
        k, v = gm.kv_download(l, n_ctx + n)
        for nm, got_rows, ref_rows in (("K", k, kc[l]), ("V", v, vc[l])):
            g = _f16(got_rows[n_ctx:]).astype(np.float64)
            r = _f16(ref_rows[n_ctx:n_ctx + n]).astype(np.float64)
            rows = np.abs(g - r).max(axis=1)
            top = float(np.abs(r).max())
            rms = float(np.sqrt(np.mean((g - r) ** 2) / np.mean(r * r)))
            say(f"  layer {l} {nm} max|err| {rows.max():.3g} median {np.median(rows):.3g} "
                f"of {top:.3g}; rms {rms:.3g}")
            assert rows.max() <= KV_SAME * top
            if l == 0:
                assert np.median(rows) <= KV_MEDIAN * top
            else:
                assert rms <= KV_RMS_7B
    assert err <= TOL_SAME * float(np.abs(ref).max())
    assert nxt == int(np.argmax(got))
