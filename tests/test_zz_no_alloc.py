"""gq_moe_ffn_noalloc (the entry point that allocates nothing: its workspace
is the library's static device scratch) against gq_moe_ffn on the same
inputs: two calls in a row, the second smaller, each bit-identical to the
allocating entry point (same kernels, fixed summation order); shapes whose
workspace exceeds the scratch are refused."""
import numpy as np
import pytest

import gq_synth as syn

pytestmark = pytest.mark.gpu
IQ3 = 18


def test_moe_ffn_noalloc_matches_moe_ffn(backend):
    import gq
    import torch
    E, H, F, k = 16, 512, 768, 4
    gate = syn.make_blocks(IQ3, E * F, H, seed=71)
    up = syn.make_blocks(IQ3, E * F, H, seed=72)
    down = syn.make_blocks(IQ3, E * H, F, seed=73)
    hg = backend.upload_experts(IQ3, gate, H, F, E)
    hu = backend.upload_experts(IQ3, up, H, F, E)
    hd = backend.upload_experts(IQ3, down, F, H, E)
    rng = np.random.default_rng(74)
    for T in (16, 3):  # the second call smaller: stale scratch must not leak in
        print(f"noalloc moe T={T}", flush=True)
        logits = torch.from_numpy(rng.standard_normal((T, E), dtype=np.float32)).cuda()
        x = torch.from_numpy(syn.make_x(H, seed=75 + T, batch=T)).cuda()
        ref, rids, rw = backend.moe_ffn(hg, hu, hd, E, logits, x, k, want_routing=True)
        got, gids, gw = backend.moe_ffn(hg, hu, hd, E, logits, x, k, want_routing=True, noalloc=True)
        got2 = backend.moe_ffn(hg, hu, hd, E, logits, x, k, noalloc=True)  # ids/w in the scratch
        torch.cuda.synchronize()
        assert torch.equal(rids, gids) and torch.equal(rw, gw)
        assert torch.equal(ref, got) and torch.equal(ref, got2)
    # a workspace past GQ_MOE_NOALLOC_MAX_BYTES (4 MiB) is refused
    T = 512
    logits = torch.zeros((T, E), device="cuda")
    x = torch.zeros((T, H), device="cuda")
    with pytest.raises(gq.GqError, match="exceeds"):
        backend.moe_ffn(hg, hu, hd, E, logits, x, k, noalloc=True)
