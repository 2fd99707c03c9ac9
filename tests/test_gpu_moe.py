"""GPU parity for the IQ3_XXS MoE expert FFN (gq_moe_ffn) against the CPU
oracle (routing bit-identical, output max|err| <= 1e-4 * max|out_ref|).

IQ3_XXS arithmetic is "parity unpinned" against the reference (it has no
IQ3_XXS implementation); both sides use the same codebook.
"""
import sys

import numpy as np
import pytest

import gq_synth as syn

pytestmark = pytest.mark.gpu
IQ3 = 18
TOL = 1e-4


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def make(E, H, F, seed):
    gate = syn.make_blocks(IQ3, E * F, H, seed=seed)
    up = syn.make_blocks(IQ3, E * F, H, seed=seed + 1)
    down = syn.make_blocks(IQ3, E * H, F, seed=seed + 2)
    return gate, up, down


def run(backend, orc, E, H, F, T, k, seed, check_tokens=None, weights=None):
    import torch
    gate, up, down = weights if weights else make(E, H, F, seed)
    hg = backend.upload_experts(IQ3, gate, H, F, E)
    hu = backend.upload_experts(IQ3, up, H, F, E)
    hd = backend.upload_experts(IQ3, down, F, H, E)
    rng = np.random.default_rng(seed + 10)
    logits = rng.standard_normal((T, E), dtype=np.float32)
    x = syn.make_x(H, seed=seed + 11, batch=T)
    out, ids, w = backend.moe_ffn(hg, hu, hd, E, torch.from_numpy(logits).cuda(),
                                  torch.from_numpy(x).cuda(), k, want_routing=True)
    torch.cuda.synchronize()
    out, ids, w = out.cpu().numpy(), ids.cpu().numpy(), w.cpu().numpy()
    rids, rw = orc.moe_route(logits, k)
    assert np.array_equal(ids, rids), "routing differs"
    assert np.allclose(w, rw, rtol=2e-6, atol=0)
    toks = range(T) if check_tokens is None else check_tokens
    sel = list(toks)
    ref = orc.moe_ffn(IQ3, gate, up, down, E, H, F, x[sel], rids[sel], rw[sel])
    got = out[sel]
    err = float(np.max(np.abs(got.astype(np.float64) - ref)))
    bound = TOL * float(np.max(np.abs(ref)))
    say(f"moe E={E} H={H} F={F} T={T} k={k}: max|err| {err:.3g} bound {bound:.3g}")
    assert err <= bound
    return ids


# Expert row counts that are multiples of 16 (F for gate/up, H for down)
# take the quad layout and the MFMA kernels, others the wave-tiled layout
# and the v_dot4 kernels; the last three shapes mix the two.
@pytest.mark.parametrize("E,H,F,T,k", [(16, 512, 256, 3, 4), (8, 256, 768, 5, 2), (4, 1024, 512, 1, 4),
                                       (4, 200, 40, 2, 2), (4, 208, 40, 3, 2), (4, 200, 48, 2, 3),
                                       (64, 512, 256, 48, 8), (1100, 256, 32, 6, 4)])
def test_moe_small(backend, orc, E, H, F, T, k):
    """(The last two: 384 (token, slot) pairs, more than one block each
    would fill the GPU with; 1100 experts, routed by the router kernel.)"""
    say(f"moe small E={E} H={H} F={F} T={T} k={k}")
    run(backend, orc, E, H, F, T, k, seed=E + H + T)


def test_moe_full_config(backend, orc):
    """config 4: 256 experts, hidden 3072, expert intermediate 1536, top-8,
    T = 1, 4, 16, every token's output and routing checked."""
    E, H, F, k = 256, 3072, 1536, 8
    say("moe full config: generating 1.39 GB of IQ3_XXS experts")
    weights = make(E, H, F, seed=100)
    for T, toks in ((1, None), (4, None), (16, None)):
        say(f"moe full T={T}")
        run(backend, orc, E, H, F, T, k, seed=200 + T, check_tokens=toks, weights=weights)


def test_moe_errors(backend):
    import gq
    import torch
    gate, up, down = make(4, 256, 256, seed=1)
    hg = backend.upload_experts(IQ3, gate, 256, 256, 4)
    hu = backend.upload_experts(IQ3, up, 256, 256, 4)
    hd = backend.upload_experts(IQ3, down, 256, 256, 4)
    x = torch.zeros((2, 256), device="cuda")
    lg = torch.zeros((2, 4), device="cuda")
    with pytest.raises(gq.GqError):
        backend.moe_ffn(hg, hu, hd, 4, lg, x, 5)       # top_k > experts
    with pytest.raises(gq.GqError):
        backend.moe_ffn(hg, hu, hd, 3, lg, x, 2)       # wrong expert count
    hq = backend.upload_experts(12, syn.make_blocks(12, 4 * 256, 256, seed=2), 256, 256, 4)
    with pytest.raises(gq.GqError):
        backend.moe_ffn(hq, hu, hd, 4, lg, x, 2)       # mixed dtypes
    # top_k <= 64 even when there are more experts
    g2, u2, d2 = make(66, 256, 256, seed=3)
    hg2 = backend.upload_experts(IQ3, g2, 256, 256, 66)
    hu2 = backend.upload_experts(IQ3, u2, 256, 256, 66)
    hd2 = backend.upload_experts(IQ3, d2, 256, 256, 66)
    lg2 = torch.zeros((2, 66), device="cuda")
    backend.moe_ffn(hg2, hu2, hd2, 66, lg2, x, 8)
    with pytest.raises(gq.GqError, match="top_k=65"):
        backend.moe_ffn(hg2, hu2, hd2, 66, lg2, x, 65)


def test_moe_routing_ties(backend, orc):
    """Tied logits go to the lower expert index, -0.0 ties +0.0, and -inf
    logits rank like any other value (both routing kernels: in-kernel for
    few experts, the router kernel past 1024)."""
    import torch
    for E, H, F in ((16, 256, 32), (1100, 256, 16)):
        k = 4
        gate, up, down = make(E, H, F, seed=5)
        hg = backend.upload_experts(IQ3, gate, H, F, E)
        hu = backend.upload_experts(IQ3, up, H, F, E)
        hd = backend.upload_experts(IQ3, down, F, H, E)
        rng = np.random.default_rng(6)
        lg = np.zeros((4, E), np.float32)
        lg[0, ::2] = -0.0                                 # all ties, mixed signs of zero
        lg[1] = rng.integers(0, 3, E).astype(np.float32)  # many ties
        lg[2] = -np.inf
        lg[2, E // 2] = 1.0
        lg[3] = rng.integers(-2, 2, E).astype(np.float32) * 0.5
        x = syn.make_x(H, seed=7, batch=4)
        say(f"routing ties E={E}")
        _, ids, w = backend.moe_ffn(hg, hu, hd, E, torch.from_numpy(lg).cuda(),
                                    torch.from_numpy(x).cuda(), k, want_routing=True)
        torch.cuda.synchronize()
        rids, rw = orc.moe_route(lg, k)
        assert np.array_equal(ids.cpu().numpy(), rids)
        # softmax sums over E terms in another order: a few ulps per term
        assert np.allclose(w.cpu().numpy(), rw, rtol=1e-5, atol=0)


@pytest.mark.parametrize("dtype", [8, 12, 13, 14])
@pytest.mark.parametrize("E,H,F,T,k", [(6, 512, 48, 3, 2), (5, 256, 40, 2, 2)])
def test_moe_other_formats(backend, orc, dtype, E, H, F, T, k):
    """Q8_0 / Q4_K / Q5_K / Q6_K experts: the quad-layout MFMA stages (F and H
    multiples of 16) and the wave-tiled v_dot4 gate/up (F = 40)."""
    import torch
    say(f"moe dtype={dtype} E={E} H={H} F={F} T={T} k={k}")
    gate = syn.make_blocks(dtype, E * F, H, seed=dtype + F)
    up = syn.make_blocks(dtype, E * F, H, seed=dtype + F + 1)
    down = syn.make_blocks(dtype, E * H, F, seed=dtype + F + 2)
    hg = backend.upload_experts(dtype, gate, H, F, E)
    hu = backend.upload_experts(dtype, up, H, F, E)
    hd = backend.upload_experts(dtype, down, F, H, E)
    rng = np.random.default_rng(dtype + 7)
    logits = rng.standard_normal((T, E), dtype=np.float32)
    x = syn.make_x(H, seed=dtype + 8, batch=T)
    out, ids, w = backend.moe_ffn(hg, hu, hd, E, torch.from_numpy(logits).cuda(),
                                  torch.from_numpy(x).cuda(), k, want_routing=True)
    torch.cuda.synchronize()
    out, ids, w = out.cpu().numpy(), ids.cpu().numpy(), w.cpu().numpy()
    rids, rw = orc.moe_route(logits, k)
    assert np.array_equal(ids, rids)
    ref = orc.moe_ffn(dtype, gate, up, down, E, H, F, x, rids, rw)
    err = float(np.max(np.abs(out.astype(np.float64) - ref)))
    bound = TOL * float(np.max(np.abs(ref)))
    say(f"  max|err| {err:.3g} bound {bound:.3g}")
    assert err <= bound


def test_moe_capture_survives_workspace_growth(backend):
    """gq_moe_ffn captured in a HIP graph after an eager call of the same
    size: a later, larger eager call grows the stream's workspace without
    freeing the captured one, every replay (eager work between) reproduces
    the eager output, and a call that would grow the workspace under
    capture fails with GqError instead of allocating."""
    import gq
    import torch
    E, H, F, k = 16, 512, 256, 4
    gate, up, down = make(E, H, F, seed=71)
    hg = backend.upload_experts(IQ3, gate, H, F, E)
    hu = backend.upload_experts(IQ3, up, H, F, E)
    hd = backend.upload_experts(IQ3, down, F, H, E)
    s = torch.cuda.Stream()
    lg2 = torch.from_numpy(syn.make_x(E, seed=72, batch=2)).cuda()
    x2 = torch.from_numpy(syn.make_x(H, seed=73, batch=2)).cuda()
    lg8 = torch.from_numpy(syn.make_x(E, seed=74, batch=8)).cuda()
    x8 = torch.from_numpy(syn.make_x(H, seed=75, batch=8)).cuda()
    y2 = torch.zeros((2, H), device="cuda")
    y8 = torch.zeros((8, H), device="cuda")
    torch.cuda.synchronize()
    backend.moe_ffn(hg, hu, hd, E, lg2, x2, k, out_dev=y2, stream=s.cuda_stream)
    s.synchronize()
    ref2 = y2.clone()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        backend.moe_ffn(hg, hu, hd, E, lg2, x2, k, out_dev=y2, stream=s.cuda_stream)
    g_bad = torch.cuda.CUDAGraph()
    with pytest.raises(gq.GqError, match="capture"):
        with torch.cuda.graph(g_bad, stream=s):
            backend.moe_ffn(hg, hu, hd, E, lg8, x8, k, out_dev=y8, stream=s.cuda_stream)
    torch.cuda.synchronize()
    backend.moe_ffn(hg, hu, hd, E, lg8, x8, k, out_dev=y8, stream=s.cuda_stream)
    s.synchronize()
    ref8 = y8.clone()
    for i in range(3):
        y2.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(y2, ref2), f"replay {i}"
        backend.moe_ffn(hg, hu, hd, E, lg8, x8, k, out_dev=y8, stream=s.cuda_stream)
        s.synchronize()
        assert torch.equal(y8, ref8)
