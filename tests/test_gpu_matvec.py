"""GPU parity: libgq.so (through its C ABI) against the CPU oracle.

Bars (from the task's north star):
  * dequantized weights bit-exact;
  * matvec outputs max|err| <= 1e-4 * max|y_ref| (fp32 accumulation);
  * the per-32 Q8 activation pack bit-exact.
"""
import sys

import numpy as np
import pytest

import gq_synth as syn
import npref

pytestmark = pytest.mark.gpu

Q8_0, Q4_K, Q5_K, Q6_K, IQ3 = 8, 12, 13, 14, 18
TOL = 1e-4


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def cuda(a):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def run_matvec(backend, dtype, rows, k, seed, x=None):
    import torch
    w = syn.make_blocks(dtype, rows, k, seed=seed)
    if x is None:
        x = syn.make_x(k, seed=seed + 1)
    h = backend.upload_weight(dtype, w, k, rows)
    y = h.launch_only(cuda(x))
    torch.cuda.synchronize()
    return w, x, y.cpu().numpy()


def check_close(y, ref, what):
    err = float(np.max(np.abs(y.astype(np.float64) - ref))) if ref.size else 0.0
    bound = TOL * float(np.max(np.abs(ref))) if ref.size else 0.0
    assert err <= bound, f"{what}: max|err| {err:.3g} > {bound:.3g}"


# ---------------------------------------------------------------- dequant
@pytest.mark.parametrize("dtype,rows,k", [
    (Q8_0, 37, 2048), (Q8_0, 5, 70), (Q4_K, 37, 3584), (Q4_K, 3, 300), (Q5_K, 19, 1024),
    (Q6_K, 37, 3584), (Q6_K, 4, 18944), (IQ3, 23, 3072), (IQ3, 3, 1536)])
def test_dequant_bit_exact(backend, orc, dtype, rows, k):
    import torch
    say(f"dequant dtype={dtype} rows={rows} k={k}")
    w = syn.make_blocks(dtype, rows, k, seed=rows * 7 + k)
    h = backend.upload_weight(dtype, w, k, rows)
    got = h.dequant_rows(0, rows).cpu().numpy()
    ref = orc.dequant_rows(dtype, w, k)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))
    # a row window
    got2 = h.dequant_rows(rows // 2, rows - rows // 2).cpu().numpy()
    assert np.array_equal(got2.view(np.uint32), ref[rows // 2:].view(np.uint32))
    torch.cuda.synchronize()


@pytest.mark.parametrize("dtype,E,f,k", [(IQ3, 5, 32, 512), (Q4_K, 3, 48, 256), (IQ3, 3, 24, 256)])
def test_dequant_experts_bit_exact(backend, orc, dtype, E, f, k):
    # stacked experts: rows per expert a multiple of 16 (quad layout, experts
    # back to back) or not (wave-tiled, one tile per expert)
    say(f"dequant experts dtype={dtype} E={E} f={f} k={k}")
    w = syn.make_blocks(dtype, E * f, k, seed=E * f + k)
    h = backend.upload_experts(dtype, w, k, f, E)
    got = h.dequant_rows(0, E * f).cpu().numpy()
    ref = orc.dequant_rows(dtype, w, k)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


def test_dequant_f16_scale_every_pattern(backend, orc):
    # Q8_0 blocks whose scale runs through all 65536 f16 bit patterns (incl.
    # subnormals, inf, nan) with q = 1: pins the device f16 decode exactly.
    say("dequant f16 exhaustive")
    blk = np.zeros((65536, 34), np.uint8)
    blk[:, 0:2] = np.arange(65536, dtype=np.uint32).astype(np.uint16)[:, None].view(np.uint8)
    blk[:, 2] = 1
    blk[:, 3] = 0xFF  # -1
    w = blk.reshape(2048, 32 * 34)
    h = backend.upload_weight(Q8_0, w, 1024, 2048)
    got = h.dequant_rows(0, 2048).cpu().numpy().reshape(65536, 32)
    ref = np.arange(65536, dtype=np.uint32).astype(np.uint16).view(np.float16).astype(np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(got[~nan, 0].view(np.uint32), ref[~nan].view(np.uint32))
    assert np.array_equal(got[~nan, 1].view(np.uint32), (-ref[~nan]).view(np.uint32))
    assert np.all(np.isnan(got[nan, 0]))


def test_dequant_rows_range_error(backend):
    import gq
    w = syn.make_blocks(Q4_K, 4, 256, seed=1)
    h = backend.upload_weight(Q4_K, w, 256, 4)
    with pytest.raises(gq.GqError):
        h.dequant_rows(3, 2)


# ----------------------------------------------------------------- matvec
SHAPES = [
    # (dtype, rows, in_dim): the benchmark configs plus ragged / tiny cases
    (Q8_0, 8192, 2048),                      # config 0: Llama-3.2-1B FFN-up
    (Q4_K, 3584, 3584), (Q4_K, 512, 3584),   # Wq/Wo, Wk/Wv
    (Q4_K, 18944, 3584),                     # Wgate/Wup
    (Q6_K, 3584, 18944),                     # Wdown
    (Q5_K, 1000, 2048),
    (IQ3, 1536, 3072), (IQ3, 3072, 1536),    # MoE expert gate/up, down
    (Q8_0, 3, 70), (Q8_0, 1, 32), (Q4_K, 7, 300), (Q4_K, 1, 256), (Q6_K, 5, 512),
    (Q6_K, 33, 600), (Q5_K, 9, 256), (IQ3, 13, 512), (Q4_K, 1001, 7168),
]


@pytest.mark.parametrize("dtype,rows,k", SHAPES)
def test_matvec_parity(backend, orc, dtype, rows, k):
    say(f"matvec dtype={dtype} rows={rows} k={k}")
    w, x, y = run_matvec(backend, dtype, rows, k, seed=rows + k + dtype)
    ref = orc.matmul_into(dtype, w, x, rows)
    check_close(y, ref, f"{dtype} {rows}x{k}")


def test_matvec_output_head(backend, orc):
    # config 1: Q6_K output head 152064 x 3584 (447 MB of weights)
    say("matvec Q6_K head 152064x3584")
    w, x, y = run_matvec(backend, Q6_K, 152064, 3584, seed=77)
    ref = orc.matmul_into(Q6_K, w, x, 152064)
    check_close(y, ref, "head")


def test_matvec_zero_weights(backend):
    # warmup path (backend_select.rs:133-139): all-zero blocks give zeros
    import torch
    for dtype in (Q8_0, Q4_K, Q5_K, Q6_K, IQ3):
        say(f"zero weights dtype={dtype}")
        k = 512
        w = syn.make_blocks(dtype, 9, k, zero=True)
        h = backend.upload_weight(dtype, w, k, 9)
        y = h.launch_only(cuda(syn.make_x(k)))
        torch.cuda.synchronize()
        assert np.all(y.cpu().numpy() == 0)


def test_matvec_multi_qkv(backend, orc):
    import torch
    say("matvec multi qkv")
    k = 3584
    ws = [syn.make_blocks(Q4_K, r, k, seed=s) for r, s in ((3584, 1), (512, 2), (512, 3))]
    hs = [backend.upload_weight(Q4_K, w, k) for w in ws]
    x = syn.make_x(k, seed=9)
    ys = backend.matmul_dequant_qkv(hs, cuda(x))
    torch.cuda.synchronize()
    for w, y in zip(ws, ys):
        check_close(y.cpu().numpy(), orc.matmul_into(Q4_K, w, x, w.shape[0]), "qkv")
    # five weights: more than one launch segment table
    ws5 = [syn.make_blocks(Q6_K, 100 + 17 * i, 512, seed=i) for i in range(5)]
    hs5 = [backend.upload_weight(Q6_K, w, 512) for w in ws5]
    x5 = syn.make_x(512, seed=4)
    ys5 = backend.matmul_dequant_multi(hs5, cuda(x5))
    torch.cuda.synchronize()
    for w, y in zip(ws5, ys5):
        check_close(y.cpu().numpy(), orc.matmul_into(Q6_K, w, x5, w.shape[0]), "multi5")


def test_matmul_dequant_host_mirror(backend, orc):
    # Backend::matmul_dequant: host bytes in, host floats out
    for dtype in (Q8_0, Q4_K, Q5_K, Q6_K):
        say(f"matmul_dequant host dtype={dtype}")
        k, rows = 1024, 77
        w = syn.make_blocks(dtype, rows, k, seed=dtype)
        x = syn.make_x(k, seed=3)
        out = np.full(rows, np.nan, np.float32)
        backend.matmul_dequant(dtype, w, x, out)
        check_close(out, orc.matmul_dequant(dtype, w, x, rows), f"host {dtype}")
        h = backend.upload_weight(dtype, w, k)
        out2 = np.zeros(rows, np.float32)
        backend.matmul_dequant_preloaded(h, x, out2)
        assert np.array_equal(out, out2)
        assert h.shape() == (dtype, k) and h.out_dim() == rows and h.nbytes() == w.nbytes


def test_matmul_dequant_errors(backend):
    import gq
    w = syn.make_blocks(Q4_K, 4, 512, seed=1)
    out = np.zeros(4, np.float32)
    with pytest.raises(gq.GqError, match="need"):
        backend.matmul_dequant(Q4_K, w.reshape(-1)[:1000], syn.make_x(512), out)
    with pytest.raises(gq.GqError, match="unsupported dtype"):
        backend.matmul_dequant(0, w, syn.make_x(512), out)
    with pytest.raises(gq.GqError, match="unsupported dtype"):
        backend.matmul_dequant(IQ3, w, syn.make_x(512), out)
    # out_dim 0 is a no-op
    backend.matmul_dequant(Q4_K, w, syn.make_x(512), np.zeros(0, np.float32))


def test_iq3_custom_grid(backend, orc):
    import torch
    say("iq3 custom grid")
    grid = (np.arange(256, dtype=np.uint64) * 2654435761 % (1 << 32)).astype(np.uint32)
    grid = ((grid & 0x3F3F3F3F) | 0x01010101).astype(np.uint32)  # magnitudes 1..63
    backend.set_iq3xxs_grid(grid)
    orc.set_iq3xxs_grid(grid)
    try:
        w = syn.make_blocks(IQ3, 64, 1024, seed=3)
        h = backend.upload_weight(IQ3, w, 1024)
        got = h.dequant_rows(0, 64).cpu().numpy()
        assert np.array_equal(got.view(np.uint32), orc.dequant_rows(IQ3, w, 1024).view(np.uint32))
        x = syn.make_x(1024, seed=4)
        y = h.launch_only(cuda(x))
        torch.cuda.synchronize()
        check_close(y.cpu().numpy(), orc.matmul_into(IQ3, w, x, 64), "iq3 grid")
    finally:
        backend.set_iq3xxs_grid(None)
        orc.set_iq3xxs_grid(None)
    assert np.array_equal(backend.get_iq3xxs_grid(), orc.get_iq3xxs_grid())
    import gq
    bad = grid.copy()
    bad[3] &= 0xFFFFFF00  # a zero magnitude
    with pytest.raises(gq.GqError, match="1..127"):
        backend.set_iq3xxs_grid(bad)
    bad = grid.copy()
    bad[5] |= 0x80
    with pytest.raises(gq.GqError, match="1..127"):
        backend.set_iq3xxs_grid(bad)


def test_quantize_q8_32_bit_exact(backend, orc):
    import torch
    say("quantize q8_32")
    x = syn.make_x(512 * 64, seed=21)
    x[32:64] = 0
    x[96:128] *= 1e-30
    sc, q = backend.quantize_q8_32(cuda(x))
    torch.cuda.synchronize()
    sc_ref, q_ref = orc.quantize_q8_32(x)
    assert np.array_equal(sc.cpu().numpy().view(np.uint16), sc_ref)
    assert np.array_equal(q.cpu().numpy(), q_ref)
