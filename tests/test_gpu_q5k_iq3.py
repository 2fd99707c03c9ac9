"""GPU parity for the Q5_K -> Q8_K route and the IQ3_XXS codebook guard.

Q5_K: WeightMap::matmul_into quantizes x to Q8_K once and runs
dot_q5_k_q8k per row (src/model/mod.rs:381-394, q8_k.rs:49-91,
q5_k.rs:126-184); CpuBackend::matmul_dequant and ffn_gate_up run the float
dot.  gq_quantize_row_q8k must be bit-identical to quantize_row_q8_k, and
gq_matvec must follow matmul_into (each 256-element block's term is the
reference's integer-exact one; only the order of the per-block sums
differs), gq_matmul_dequant_* the float dot.

IQ3_XXS: the library refuses IQ3_XXS uploads until a codebook is
installed, and the dequant / matvec of one-hot blocks match closed forms
(tests/iq3_onehot.py) for every scale nibble, sign index and grid slot.
"""
import os
import subprocess
import sys

import numpy as np
import pytest

import gq_synth as syn
import iq3_onehot as oh

pytestmark = pytest.mark.gpu

Q5_K, IQ3 = 13, 18
ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def say(*a):
    print(*a, flush=True)


def cuda(a):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _special_x(n, seed):
    x = syn.make_x(n, seed=seed)
    if n >= 512:
        x[256:512] = 0.0                              # an all-zero block
        x[3], x[10] = 2.5e3, -2.5e3                   # tie: the first one is the pivot
    if n >= 768:
        x[512:768] *= np.float32(1e-30)               # tiny block
        x[600] = -7.0                                 # negative pivot
    return x


@pytest.mark.parametrize("n", [256, 100, 257, 1000, 3584, 18944])
def test_quantize_row_q8k_bit_exact(backend, orc, n):
    import torch
    say(f"quantize_row_q8k n={n}")
    x = _special_x(n, seed=n)
    d, qs, bs = backend.quantize_row_q8_k(cuda(x))
    torch.cuda.synchronize()
    d_ref, qs_ref, bs_ref = orc.quantize_row_q8_k(x)
    assert np.array_equal(d.cpu().numpy().view(np.uint32), d_ref.view(np.uint32))
    assert np.array_equal(qs.cpu().numpy(), qs_ref)
    assert np.array_equal(bs.cpu().numpy(), bs_ref)


@pytest.mark.parametrize("rows,k", [(3584, 3584), (512, 18944), (77, 1024), (5, 300)])
def test_matvec_q5k_follows_matmul_into(backend, orc, rows, k):
    import torch
    say(f"q5k matvec rows={rows} k={k}")
    w = syn.make_blocks(Q5_K, rows, k, seed=rows + k)
    x = _special_x(k, seed=k + 1)
    h = backend.upload_weight(Q5_K, w, k, rows)
    y = h.launch_only(cuda(x)).cpu().numpy().astype(np.float64)
    torch.cuda.synchronize()
    ref = orc.matmul_into(Q5_K, w, x, rows).astype(np.float64)
    flt = orc.matmul_dequant(Q5_K, w, x, rows).astype(np.float64)
    scale = np.abs(ref).max()
    err = np.abs(y - ref).max()
    # per-block terms are exact; the sum order of ~k/256 terms differs
    assert err <= 1e-5 * scale, err / scale
    # and the route is the Q8_K one, not the float dot
    assert np.abs(y - flt).max() > 10 * max(err, 1e-30)
    # matmul_dequant_preloaded (the Backend::matmul_dequant family) keeps
    # the float dot
    out = np.zeros(rows, np.float32)
    backend.matmul_dequant_preloaded(h, x, out)
    assert np.abs(out - flt).max() <= 1e-4 * np.abs(flt).max()


def test_decode_q5k_layers(backend):
    """A decoder whose projections are all Q5_K: q/k/v, o, down and the
    head take matmul_into's Q8_K route, gate/up the float dot
    (ffn_gate_up), as in LlamaModel::run.  The normalised inputs come from
    a different summation order than the CPU's, so an input can sit on the
    other side of a Q8_K rounding boundary (one code, ~1/254 of the block's
    max): logits agree to 1e-3 of the max, greedy tokens exactly."""
    import gq
    import oracle
    cfg = dict(n_layers=2, hidden=512, n_heads=4, n_kv_heads=2, head_dim=128, ffn=768,
               vocab=1000, ctx=256, eps=1e-6, theta=1e6, attn_type=Q5_K, gate_up_type=Q5_K,
               down_type=Q5_K, head_type=Q5_K)
    w = syn.make_decoder(cfg, 17, embd_scale=1e4)
    hw = syn.upload_decoder(backend, cfg, w)
    gm = gq.DecodeModel(dict(cfg, max_tokens=64), hw)
    om = oracle.DecoderModel(cfg, w)
    worst = 0.0
    for pos, tok in enumerate([7, 901, 33, 450]):
        ref = om.step(tok, pos)
        nxt, got = gm.decode(tok, pos)
        worst = max(worst, float(np.abs(got - ref).max() / np.abs(ref).max()))
        assert nxt == oracle.argmax(ref)
    say(f"q5k decode worst rel err {worst:.3g}")
    assert worst <= 1e-3
    got = gm.generate(5, 4, 12)
    exp, tok = [], 5
    for i in range(12):
        tok = oracle.argmax(om.step(tok, 4 + i))
        exp.append(tok)
    np.testing.assert_array_equal(got, np.array(exp, np.int32))


def test_iq3_refused_until_a_codebook_is_installed():
    """A fresh process: IQ3_XXS uploads fail with GQ_EDTYPE before
    gq_set_iq3xxs_grid, and succeed after it."""
    code = (
        "import sys; sys.path[:0] = [%r, %r]\n"
        "import gq, gq_synth as syn\n"
        "be = gq.create_backend('hip')\n"
        "w = syn.make_blocks(18, 4, 256, seed=1)\n"
        "try:\n"
        "    be.upload_weight(18, w, 256, 4)\n"
        "    raise SystemExit('IQ3_XXS upload accepted without a codebook')\n"
        "except gq.GqError as e:\n"
        "    assert e.code == -2 and 'codebook' in str(e), e\n"
        "be.set_iq3xxs_grid(None)\n"
        "be.upload_weight(18, w, 256, 4)\n"
        "print('ok')\n" % (ROOT, os.path.join(ROOT, "agention-infer_amd")))
    r = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0 and r.stdout.strip().endswith("ok"), r.stdout + r.stderr


def test_iq3_one_hot_fields(backend):
    """Every scale nibble, sign index and grid slot against closed forms,
    through the GPU dequant and the GPU matvec (x = one-hot columns)."""
    import torch
    g0 = backend.get_iq3xxs_grid()
    backend.set_iq3xxs_grid(oh.IDENT_GRID)
    try:
        cases = [("scales", *oh.scale_blocks(oh.IDENT_GRID)), ("grid", *oh.grid_blocks(oh.IDENT_GRID))]
        for name, b, exp in cases:
            say(f"iq3 one-hot {name}")
            rows = b.shape[0]
            h = backend.upload_weight(IQ3, b, 256, rows)
            y = h.dequant_rows(0, rows).cpu().numpy().astype(np.float64)
            assert np.array_equal(y, exp), name
            # matvec against e_j for a few columns j: y = column j exactly
            for j in (0, 5, 127, 200, 255):
                x = np.zeros(256, np.float32)
                x[j] = 1.0
                col = h.launch_only(cuda(x)).cpu().numpy().astype(np.float64)
                np.testing.assert_allclose(col, exp[:, j], rtol=1e-6, atol=0)
        say("iq3 one-hot signs")
        b, mags, idx = oh.sign_blocks(oh.IDENT_GRID)
        h = backend.upload_weight(IQ3, b, 256, 4)
        oh.check_signs(h.dequant_rows(0, 4).cpu().numpy(), mags, idx)
        torch.cuda.synchronize()
    finally:
        backend.set_iq3xxs_grid(g0)
