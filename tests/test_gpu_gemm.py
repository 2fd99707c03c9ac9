"""GPU parity for the batched prefill GEMM (gq_gemm) against CPU references.

Both modes change the operands' precision by definition, so each is
compared against a CPU matmul of the *same* operands (tolerance
max|err| <= 1e-4 * max|y_ref|, fp64 reference):
  * GQ_GEMM_BF16: W = bf16(dequant(W)) (round to nearest even of the
    bit-exact fp32 dequant), X = bf16(X).
  * GQ_GEMM_INT8: W = dequant(W) exactly, X = per-32 Q8 pack of X
    (KvDtype::Q8_0::pack, src/model/mod.rs:574-583), i.e. q * f16(scale).
The distance to the fp32 CPU path (WeightMap::matmul_batch_into,
src/model/mod.rs:414-464) is also checked, with a tolerance that reflects
the operand rounding (bf16: 2^-9 relative per operand).
"""
import sys

import numpy as np
import pytest

import gq_synth as syn

pytestmark = pytest.mark.gpu

Q4_K = 12
TOL = 1e-4


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def bf16_round(a):
    u = np.ascontiguousarray(a, np.float32).view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
    return r.astype(np.uint32).view(np.float32)


def run(backend, orc, rows, k, n, mode, seed, dtype=Q4_K):
    import torch
    import gq
    w = syn.make_blocks(dtype, rows, k, seed=seed)
    X = syn.make_x(k, seed=seed + 1, batch=n)
    h = backend.upload_weight(dtype, w, k, rows)
    Y = h.launch_only_batch(torch.from_numpy(X).cuda(), mode=mode)
    torch.cuda.synchronize()
    Wf = orc.dequant(dtype, w.reshape(-1), rows * k).reshape(rows, k) if k % 256 == 0 else \
        orc.dequant_rows(dtype, w, k)
    return w, X, Wf, Y.cpu().numpy()


def check(y, ref, what, tol=TOL):
    err = float(np.max(np.abs(y.astype(np.float64) - ref)))
    bound = tol * float(np.max(np.abs(ref)))
    say(f"{what}: max|err| {err:.3g} bound {bound:.3g}")
    assert err <= bound, f"{what}: max|err| {err:.3g} > {bound:.3g}"


SHAPES = [(331, 512, 37), (1024, 3584, 64), (160, 256, 256), (7, 300, 5), (2000, 1024, 300)]
Q6_K = 14
# Q6_K (the ffn_down / attn_v type of Q4_K_M files): narrow and wide token
# tiles, K splits (few row tiles), a partial last unit.
Q6_SHAPES = [(331, 512, 37), (512, 2048, 300), (100, 768, 20), (3584, 2048, 512), (40, 300, 3)]


@pytest.mark.parametrize("rows,k,n", Q6_SHAPES)
def test_gemm_bf16_q6k(backend, orc, rows, k, n):
    import gq
    say(f"gemm bf16 Q6_K rows={rows} k={k} n={n}")
    w, X, Wf, Y = run(backend, orc, rows, k, n, gq.GQ_GEMM_BF16, seed=rows + 7 * k, dtype=Q6_K)
    ref = bf16_round(X).astype(np.float64) @ bf16_round(Wf).astype(np.float64).T
    check(Y, ref, "bf16 Q6_K vs same-operand fp64")


@pytest.mark.parametrize("rows,k,n", SHAPES)
def test_gemm_bf16(backend, orc, rows, k, n):
    import gq
    say(f"gemm bf16 rows={rows} k={k} n={n}")
    w, X, Wf, Y = run(backend, orc, rows, k, n, gq.GQ_GEMM_BF16, seed=rows + k)
    ref = bf16_round(X).astype(np.float64) @ bf16_round(Wf).astype(np.float64).T
    check(Y, ref, "bf16 vs same-operand fp64")
    ref32 = orc.matmul_batch_into(Q4_K, w, X, rows)
    check(Y, ref32, "bf16 vs fp32 CPU path", tol=1e-2)


@pytest.mark.parametrize("dtype,rows,k,n", [(Q4_K,) + sh for sh in SHAPES] + [(Q6_K,) + sh for sh in Q6_SHAPES]
                         + [(Q6_K, 3584, 18944, 512)])
def test_gemm_int8(backend, orc, dtype, rows, k, n):
    """GQ_GEMM_INT8 for Q4_K and Q6_K weights (Q4_K_M files keep ffn_down and
    attn_v in Q6_K; 3584 x 18944 is the 7B down projection) against the
    same-operand fp64 product and the fp32 CPU path."""
    import gq
    say(f"gemm int8 dtype={dtype} rows={rows} k={k} n={n}")
    w, X, Wf, Y = run(backend, orc, rows, k, n, gq.GQ_GEMM_INT8, seed=rows + k + 1, dtype=dtype)
    kp = (k + 31) // 32 * 32
    Xq = np.zeros((n, k), np.float64)
    for t in range(n):
        sc, q = orc.quantize_q8_32(X[t])
        s = np.repeat(sc.view(np.float16).astype(np.float64), 32)[:kp]
        Xq[t] = (q.astype(np.float64) * s[: q.size])[:k]
    ref = Xq @ Wf.astype(np.float64).T
    check(Y, ref, "int8 vs same-operand fp64")
    sub = np.arange(0, n, max(1, n // 16))
    ref32 = orc.matmul_batch_into(dtype, w, X[sub], rows)
    check(Y[sub], ref32, "int8 vs fp32 CPU path", tol=3e-2)


def test_gemm_full_config(backend, orc):
    """config 2: Q4_K 18944 x 3584 times 512 tokens, both modes."""
    import gq
    import torch
    rows, k, n = 18944, 3584, 512
    say("gemm full config 18944x3584x512")
    w = syn.make_blocks(Q4_K, rows, k, seed=42)
    X = syn.make_x(k, seed=43, batch=n)
    h = backend.upload_weight(Q4_K, w, k, rows)
    Xd = torch.from_numpy(X).cuda()
    Yb = h.launch_only_batch(Xd, mode=gq.GQ_GEMM_BF16).cpu().numpy()
    Yi = h.launch_only_batch(Xd, mode=gq.GQ_GEMM_INT8).cpu().numpy()
    torch.cuda.synchronize()
    Wf = orc.dequant(Q4_K, w.reshape(-1), rows * k).reshape(rows, k).astype(np.float64)
    ref = bf16_round(X).astype(np.float64) @ bf16_round(Wf.astype(np.float32)).astype(np.float64).T
    check(Yb, ref, "full bf16 vs same-operand fp64")
    Xq = np.zeros((n, k), np.float64)
    for t in range(n):
        sc, q = orc.quantize_q8_32(X[t])
        Xq[t] = q.astype(np.float64) * np.repeat(sc.view(np.float16).astype(np.float64), 32)
    check(Yi, Xq @ Wf.T, "full int8 vs same-operand fp64")
    # the fp32 CPU path (WeightMap::matmul_batch_into) on 16 of the 512
    # tokens: the distance is the operands' rounding (bf16 2^-9 each; per-32
    # Q8 activations 2^-8)
    sub = np.arange(0, n, n // 16)
    ref32 = orc.matmul_batch_into(Q4_K, w, X[sub], rows)
    check(Yb[sub], ref32, "full bf16 vs fp32 CPU path (16 tokens)", tol=1e-2)
    check(Yi[sub], ref32, "full int8 vs fp32 CPU path (16 tokens)", tol=3e-2)


Q8_0, Q5_K = 8, 13
# Q8_0 and Q5_K (bf16 mode only): token counts on both sides of the ring /
# direct kernel boundary (both run the direct kernel), a ragged last unit
# (Q8_0 k = 288), K splits.
OTHER_SHAPES = [(Q8_0, 331, 512, 37), (Q8_0, 1024, 2048, 300), (Q8_0, 100, 288, 20),
                (Q8_0, 8192, 2048, 512), (Q5_K, 331, 512, 37), (Q5_K, 512, 3584, 300),
                (Q5_K, 40, 768, 3)]


@pytest.mark.parametrize("dtype,rows,k,n", OTHER_SHAPES)
def test_gemm_bf16_q8_0_q5k(backend, orc, dtype, rows, k, n):
    """WeightMap::matmul_batch_into (src/model/mod.rs:414-464) dequantizes
    every dtype with dequant_row; the bf16 GEMM of Q8_0 and Q5_K weights
    against the same-operand fp64 product (1e-4) and the fp32 CPU path
    (1e-2, bf16 operands).  (8192 x 2048 is BASELINE configs[0]'s Q8_0 FFN-up
    matrix, here over 512 prompt tokens.)"""
    import gq
    say(f"gemm bf16 dtype={dtype} rows={rows} k={k} n={n}")
    w, X, Wf, Y = run(backend, orc, rows, k, n, gq.GQ_GEMM_BF16, seed=rows + 3 * k + dtype, dtype=dtype)
    ref = bf16_round(X).astype(np.float64) @ bf16_round(Wf).astype(np.float64).T
    check(Y, ref, f"bf16 dtype {dtype} vs same-operand fp64")
    sub = np.arange(0, n, max(1, n // 16))
    ref32 = orc.matmul_batch_into(dtype, w, X[sub], rows)
    check(Y[sub], ref32, f"bf16 dtype {dtype} vs fp32 CPU path", tol=1e-2)


def test_gemm_errors_and_edges(backend):
    import gq
    import torch
    w = syn.make_blocks(13, 4, 256, seed=1)  # Q5_K: bf16 only
    h = backend.upload_weight(13, w, 256, 4)
    with pytest.raises(gq.GqError, match="not supported"):
        h.launch_only_batch(torch.zeros((2, 256), device="cuda"), mode=gq.GQ_GEMM_INT8)
    w8 = syn.make_blocks(8, 4, 256, seed=1)  # Q8_0: bf16 only
    h8 = backend.upload_weight(8, w8, 256, 4)
    with pytest.raises(gq.GqError, match="not supported"):
        h8.launch_only_batch(torch.zeros((2, 256), device="cuda"), mode=gq.GQ_GEMM_INT8)
    w4 = syn.make_blocks(Q4_K, 4, 256, seed=1)
    h4 = backend.upload_weight(Q4_K, w4, 256, 4)
    with pytest.raises(gq.GqError, match="mode"):
        h4.launch_only_batch(torch.zeros((2, 256), device="cuda"), mode=7)
    # n = 0 is a no-op; zero weights give zeros
    h4.launch_only_batch(torch.zeros((0, 256), device="cuda"))
    z = backend.upload_weight(Q4_K, syn.make_blocks(Q4_K, 9, 512, zero=True), 512, 9)
    for mode in (gq.GQ_GEMM_BF16, gq.GQ_GEMM_INT8):
        y = z.launch_only_batch(torch.randn((3, 512), device="cuda"), mode=mode)
        torch.cuda.synchronize()
        assert torch.all(y == 0)


def test_gemm_capture_survives_workspace_growth(backend):
    """A HIP graph captured around gq_gemm keeps its workspace: a later,
    larger call on the same stream grows the stream's workspace without
    freeing the captured one, and every replay (with eager work between)
    reproduces the eager result.  Under capture, growing the workspace and
    the first call on a weight (which builds its GEMM records) fail with
    GqError instead of allocating."""
    import torch
    import gq
    rows, k = 1024, 3584
    w = syn.make_blocks(Q4_K, rows, k, seed=61)
    h = backend.upload_weight(Q4_K, w, k, rows)
    h_new = backend.upload_weight(Q4_K, syn.make_blocks(Q4_K, 256, k, seed=64), k, 256)
    s = torch.cuda.Stream()
    Xs = torch.from_numpy(syn.make_x(k, seed=62, batch=64)).cuda()
    Xl = torch.from_numpy(syn.make_x(k, seed=63, batch=512)).cuda()
    Ys = torch.zeros((64, rows), device="cuda")
    Yl = torch.zeros((512, rows), device="cuda")
    Yn = torch.zeros((64, 256), device="cuda")
    torch.cuda.synchronize()
    h.launch_only_batch(Xs, Y_dev=Ys, stream=s.cuda_stream)
    s.synchronize()
    ref = Ys.clone()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        h.launch_only_batch(Xs, Y_dev=Ys, stream=s.cuda_stream)
    for bad, Xb, Yb in ((h, Xl, Yl), (h_new, Xs, Yn)):
        g_bad = torch.cuda.CUDAGraph()
        with pytest.raises(gq.GqError, match="capture"):
            with torch.cuda.graph(g_bad, stream=s):
                bad.launch_only_batch(Xb, Y_dev=Yb, stream=s.cuda_stream)
        torch.cuda.synchronize()
    # the larger call grows the workspace (eager)
    h.launch_only_batch(Xl, Y_dev=Yl, stream=s.cuda_stream)
    s.synchronize()
    ref_l = Yl.clone()
    for i in range(3):
        Ys.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(Ys, ref), f"replay {i}"
        h.launch_only_batch(Xl, Y_dev=Yl, stream=s.cuda_stream)
        s.synchronize()
        assert torch.equal(Yl, ref_l)
