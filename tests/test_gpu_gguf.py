"""A decoder written as a GGUF file, loaded by libgq_host (gqh_model_load:
ModelConfig::from_gguf, LlamaModel::new's tensor discovery, pre_upload_gpu)
and decoded on the GPU, against the CPU oracle's decode step on the same
weights (LlamaModel::run, src/model/llama/cpu_path.rs:695-818).  Also
single tensors uploaded from a file (HipBackend::upload_tensor) against the
oracle's matvec.  The tolerance and the greedy-token criterion are those of
the GPU-resident decode tests."""
import numpy as np
import pytest

import gguf_write as gw
import gq
import gq_synth as syn
import oracle

pytestmark = pytest.mark.gpu

CFG = dict(n_layers=2, hidden=256, n_heads=4, n_kv_heads=2, head_dim=64, ffn=512, vocab=1000,
           ctx=320, eps=1e-6, theta=1e6, attn_type=syn.Q4_K, gate_up_type=syn.Q4_K,
           down_type=syn.Q6_K, head_type=syn.Q6_K)
LOGIT_TOL = 1e-4
Q4K, Q6K, Q8 = syn.Q4_K, syn.Q6_K, syn.Q8_0


def _weights(cfg, layer_types, seed):
    """make_decoder's weights, re-drawn where a tensor's type differs."""
    w = syn.make_decoder(cfg, seed, embd_scale=1e4)
    H, F = cfg["hidden"], cfg["ffn"]
    qd, kvd = cfg["n_heads"] * cfg["head_dim"], cfg["n_kv_heads"] * cfg["head_dim"]
    rows = dict(wq=(qd, H), wk=(kvd, H), wv=(kvd, H), wo=(H, qd), wgate=(F, H), wup=(F, H),
                wdown=(H, F))
    uniform = [cfg["attn_type"]] * 4 + [cfg["gate_up_type"]] * 2 + [cfg["down_type"]]
    for l, types in enumerate(layer_types):
        for i, (k, t) in enumerate(zip(gw.ORDER, types)):
            if t != uniform[i]:
                w[k][l] = syn.make_blocks(t, rows[k][0], rows[k][1], seed=seed * 77 + 7 * l + i)
    w["layer_types"] = np.asarray(layer_types, np.int32)
    return w


def _load(tmp_path, cfg, w, layer_types, embd=None, head_type=Q6K, norm_f16=False, ctx=0):
    path = str(tmp_path / "model.gguf")
    gw.write(path, gw.decoder_metadata(cfg, context_length=cfg["ctx"]),
             gw.decoder_tensors(cfg, w, layer_types, embd, head_type, norm_f16))
    f = gq.GgufFile(path)
    m = f.load_model(ctx=ctx, max_tokens=64)
    f.close()  # the model keeps what it needs
    return m


def _check_steps(gm, om, cfg, tokens, pos0):
    for i, tok in enumerate(tokens):
        ref = om.step(int(tok), pos0 + i)
        nxt, got = gm.decode(int(tok), pos0 + i)
        err = np.abs(got - ref).max()
        assert err <= LOGIT_TOL * np.abs(ref).max(), (pos0 + i, err)
        assert nxt == oracle.argmax(ref)


def test_gguf_model_config_and_decode(backend, tmp_path):
    types = [[Q4K] * 6 + [Q6K]] * CFG["n_layers"]
    w = _weights(CFG, types, seed=11)
    gm = _load(tmp_path, CFG, w, types)
    c = gm.config
    assert c["architecture"] == "qwen2" and c["block_count"] == 2 and c["head_dim"] == 64
    assert c["vocab_size"] == 1000 and c["ctx"] == CFG["ctx"] and c["feed_forward_length"] == 512
    om = oracle.DecoderModel(CFG, w)
    _check_steps(gm, om, CFG, np.random.default_rng(1).integers(0, 1000, 4), 0)


def test_gguf_mixed_types_q4_k_m(backend, tmp_path):
    """Per-tensor types as a Q4_K_M file has them: attn_v and ffn_down in
    Q6_K on some layers only, Q4_K elsewhere (q/k/v then run as two
    launches), F16 norm weights."""
    types = [[Q4K, Q4K, Q6K, Q4K, Q4K, Q4K, Q6K],
             [Q4K, Q4K, Q4K, Q4K, Q4K, Q4K, Q4K]]
    w = _weights(CFG, types, seed=12)
    for k in ("attn_norm", "ffn_norm"):  # what the F16 file holds
        w[k] = [a.astype(np.float16).astype(np.float32) for a in w[k]]
    w["output_norm"] = w["output_norm"].astype(np.float16).astype(np.float32)
    gm = _load(tmp_path, CFG, w, types, norm_f16=True)
    om = oracle.DecoderModel(CFG, w)
    _check_steps(gm, om, CFG, np.random.default_rng(2).integers(0, 1000, 3), 0)
    got = gm.generate(7, 3, 16)
    ref, tok = [], 7
    for i in range(16):
        tok = oracle.argmax(om.step(tok, 3 + i))
        ref.append(tok)
    np.testing.assert_array_equal(got, ref)


def test_gguf_tied_quantized_embedding(backend, tmp_path):
    """No output.weight: lm_head is token_embd (Q8_0 here), and the
    embedding rows come from the GPU dequant of the same tensor, which is
    bit-identical to the CPU dequant."""
    cfg = dict(CFG, head_type=Q8)
    types = [[Q4K] * 6 + [Q6K]] * cfg["n_layers"]
    w = _weights(cfg, types, seed=13)
    emb = syn.make_blocks(Q8, cfg["vocab"], cfg["hidden"], seed=1313)
    w["lm_head"] = emb
    w["embd"] = oracle.dequant(Q8, emb, cfg["vocab"] * cfg["hidden"]).reshape(cfg["vocab"], -1)
    gm = _load(tmp_path, cfg, w, types, embd=(Q8, bytes(emb)), head_type=None, ctx=128)
    assert gm.config["ctx"] == 128
    om = oracle.DecoderModel(dict(cfg, ctx=128), w)
    _check_steps(gm, om, cfg, [5, 999, 0], 0)


@pytest.mark.parametrize("dtype", [Q8, Q4K, Q6K, syn.Q5_K])
def test_gguf_upload_tensor_matvec(backend, tmp_path, dtype):
    rows, cols = 300, 512
    wb = syn.make_blocks(dtype, rows, cols, seed=dtype)
    path = str(tmp_path / "w.gguf")
    gw.write(path, [("general.architecture", gw.STRING, "llama")],
             [("norm", [cols], gw.GGML_F32, np.ones(cols, np.float32).tobytes()),
              ("w", [cols, rows], dtype, bytes(wb))])
    f = gq.GgufFile(path)
    h = f.upload("w")
    assert h.shape() == (dtype, cols) and h.out_dim() == rows
    x = np.random.default_rng(dtype).standard_normal(cols).astype(np.float32)
    out = np.zeros(rows, np.float32)
    # Backend::matmul_dequant_preloaded: the float dot of every type
    backend.matmul_dequant_preloaded(h, x, out)
    ref = oracle.matmul_dequant(dtype, wb, x, rows)
    assert np.abs(out - ref).max() <= 1e-4 * np.abs(ref).max()
    # launch_only follows matmul_into (Q5_K: the Q8_K route)
    import torch
    y = h.launch_only(torch.from_numpy(x).cuda()).cpu().numpy()
    ref = oracle.matmul_into(dtype, wb, x, rows)
    assert np.abs(y - ref).max() <= 1e-4 * np.abs(ref).max()
    with pytest.raises(gq.GgufError):
        f.upload("norm")  # 1-D F32: not a weight the backend multiplies


def test_gguf_q8_0_model_prefill_and_generate(backend, tmp_path):
    """An all-Q8_0 file (the file type of BASELINE configs[0]'s Llama-3.2-1B
    Q8_0 model; here a small decoder with a Q8_0 head): gq_model_prefill of
    a 40-token prompt (LlamaModel::run_batch, cpu_path.rs:834-991) against
    the oracle stepping the same tokens (logits to the bf16-operand bound
    2e-2 of their max), then, on the GPU's prompt K/V rows, 16 greedy steps
    equal to the oracle's."""
    cfg = dict(CFG, attn_type=Q8, gate_up_type=Q8, down_type=Q8, head_type=Q8)
    types = [[Q8] * 7] * cfg["n_layers"]
    w = _weights(cfg, types, seed=14)
    gm = _load(tmp_path, cfg, w, types, head_type=Q8)
    om = oracle.DecoderModel(cfg, w)
    toks = np.random.default_rng(14).integers(0, cfg["vocab"], 40).astype(np.int32)
    nxt, got = gm.prefill(toks, 0)
    for i, t in enumerate(toks):
        ref = om.step(int(t), i)
    err = float(np.abs(got - ref).max())
    assert err <= 2e-2 * float(np.abs(ref).max()), err
    top = np.sort(ref)[-2:]
    if top[1] - top[0] > 2 * err:
        assert nxt == oracle.argmax(ref)
    for l in range(cfg["n_layers"]):
        k, v = gm.kv_download(l, 40)
        om.kc[l, :40], om.vc[l, :40] = k, v
    exp, tok = [], nxt
    for i in range(16):
        tok = oracle.argmax(om.step(tok, 40 + i))
        exp.append(tok)
    np.testing.assert_array_equal(gm.generate(nxt, 40, 16), np.array(exp, np.int32))
