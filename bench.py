"""Benchmark: Qwen2.5-7B-shaped Q4_K_M decode-layer matvecs on one MI355X.

One step = one batch-1 pass over the decode matvecs of one layer plus the
output head, with weights resident in HBM (5 launches: qkv, o, gate+up,
down, head -- same-input weights share a launch as in the reference's
resident path):
    Wq 3584x3584, Wk 512x3584, Wv 512x3584, Wo 3584x3584,
    Wgate 18944x3584, Wup 18944x3584          (Q4_K)
    Wdown 3584x18944, head 152064x3584        (Q6_K)
value = algorithmic bytes per step (weights + x + y) / step time, in GB/s.
Every timed launch reads its weights cold from HBM (two device copies per
matrix, alternated; a step streams ~0.6 GB, more than twice the 256 MB
Infinity Cache).  Each step is one captured HIP graph of the 8 launches.

Prints ONE JSON line (rank 0).  --gpus above 1 exits: this build uses one GPU.
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "agention-infer_amd"))

HBM_PEAK_GBS = 8000.0

Q4_K, Q6_K = 12, 14
HID, KV, FFN, VOCAB = 3584, 512, 18944, 152064
MATS = [  # name, dtype, out_dim, in_dim
    ("Wq", Q4_K, HID, HID), ("Wk", Q4_K, KV, HID), ("Wv", Q4_K, KV, HID),
    ("Wo", Q4_K, HID, HID), ("Wgate", Q4_K, FFN, HID), ("Wup", Q4_K, FFN, HID),
    ("Wdown", Q6_K, HID, FFN), ("head", Q6_K, VOCAB, HID),
]
# Two device copies of every matrix, alternated step to step: between two
# uses of a copy the step streams > 1 GB (the head alone is 447 MB), far
# more than the 256 MB Infinity Cache, so every launch reads cold HBM.
NCOPY = 2


def measured_traffic():
    """HBM bytes per head launch from the committed rocprof summary, or None."""
    path = os.path.join(ROOT, "profiles", "matvec_q6k_head_and_q4k_layer.md")
    try:
        for line in open(path):
            if line.startswith("traffic_bytes_per_launch:"):
                return int(line.split(":")[1])
    except OSError:
        pass
    return None


def algo_bytes(gq, dtype, out_dim, in_dim):
    return gq.type_size(dtype, in_dim) * out_dim + 4 * in_dim + 4 * out_dim


def cpu_baseline(mats, host, xs, nthreads, budget_s=15.0):
    """The oracle's WeightMap::matmul_into restatement on the host cores."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle
    total_bytes = sum(b for *_, b in mats)
    oracle.matmul_into(Q4_K, host["Wq"], xs[HID], HID, nthreads)  # warm
    steps, t0 = 0, time.perf_counter()
    while True:
        for name, dtype, out_dim, in_dim, _ in mats:
            oracle.matmul_into(dtype, host[name], xs[in_dim], out_dim, nthreads)
        steps += 1
        el = time.perf_counter() - t0
        if el > budget_s or steps >= 50:
            break
    return {"value": round(total_bytes * steps / el / 1e9, 3), "unit": "GB/s",
            "cores": nthreads, "kind": "port",
            "sample": f"{steps} full steps (all 8 matvecs, {total_bytes / 1e6:.0f} MB each) "
                      f"through oracle matmul_into, {el:.1f} s"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--cpu-seconds", type=float, default=15.0)
    ap.add_argument("--calib-copy", action="store_true",
                    help="also run a plain 256 MiB device copy (HBM counter calibration)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU only (asked for --gpus {args.gpus}); "
              "see DESIGN.md for how the path would shard.", file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch

    import gq
    import gq_synth as syn

    be = gq.create_backend("hip", 0)
    stream = torch.cuda.current_stream()

    host, xs, mats, copies = {}, {}, [], {}
    for i, (name, dtype, out_dim, in_dim) in enumerate(MATS):
        w = syn.make_blocks(dtype, out_dim, in_dim, seed=100 + i)
        host[name] = w
        nb = algo_bytes(gq, dtype, out_dim, in_dim)
        mats.append((name, dtype, out_dim, in_dim, nb))
        dev = torch.from_numpy(w.reshape(-1)).cuda()
        copies[name] = [be.upload_weight(dtype, dev, in_dim, out_dim) for _ in range(NCOPY)]
        del dev
    for d in (HID, FFN):
        xs[d] = syn.make_x(d, seed=d)
    xd = {d: torch.from_numpy(v).cuda() for d, v in xs.items()}
    yd = {name: torch.empty(out_dim, dtype=torch.float32, device="cuda")
          for name, _, out_dim, _, _ in mats}
    torch.cuda.synchronize()

    # The decode layer launches matvecs the way the reference's resident path
    # groups them: same-input weights share one launch
    # (matmul_dequant_qkv / _ffn, src/ops/wgpu_backend/mod.rs:702-854).
    GROUPS = [("Wq", "Wk", "Wv"), ("Wo",), ("Wgate", "Wup"), ("Wdown",), ("head",)]
    dims = {name: in_dim for name, _, _, in_dim, _ in mats}
    nbytes = {name: nb for name, *_, nb in mats}

    def group_bytes(grp):  # weights + y of every member, x once
        return sum(nbytes[n] - 4 * dims[n] for n in grp) + 4 * dims[grp[0]]
    step_bytes = sum(group_bytes(g) for g in GROUPS)

    def step(s):
        for grp in GROUPS:
            hs = [copies[n][s % NCOPY] for n in grp]
            if len(grp) == 1:
                hs[0].launch_only(xd[dims[grp[0]]], yd[grp[0]])
            else:
                be.matmul_dequant_multi(hs, xd[dims[grp[0]]], [yd[n] for n in grp])

    # Warm up (also compiles nothing: kernels are prebuilt), then capture one
    # HIP graph per copy parity so the timed loop is launch-overhead free.
    for s in range(args.warmup):
        step(s)
    torch.cuda.synchronize()
    graphs = []
    for r in range(NCOPY):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            step(r)
        graphs.append(g)
    for g in graphs:
        g.replay()
    torch.cuda.synchronize()

    t_start, t_end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    wall0 = time.perf_counter()
    t_start.record()
    for s in range(args.steps):
        graphs[s % NCOPY].replay()
    t_end.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - wall0
    ms_total = t_start.elapsed_time(t_end)
    ms_step = ms_total / args.steps
    value = step_bytes / (ms_step * 1e-3) / 1e9

    # Per-launch kernel time: a graph of REPS launches of one group,
    # alternating the copies, bracketed by events on the replay stream.
    per = {}
    REPS = 20
    for grp in GROUPS:
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            for r in range(REPS):
                hs = [copies[n][r % NCOPY] for n in grp]
                if len(grp) == 1:
                    hs[0].launch_only(xd[dims[grp[0]]], yd[grp[0]])
                else:
                    be.matmul_dequant_multi(hs, xd[dims[grp[0]]], [yd[n] for n in grp])
        g.replay()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        g.replay()
        e1.record()
        torch.cuda.synchronize()
        us = e0.elapsed_time(e1) * 1e3 / REPS
        nb = group_bytes(grp)
        per["+".join(grp)] = {"us": round(us, 2), "GB/s": round(nb / (us * 1e-6) / 1e9, 1)}
    head_bytes = [b for n, *_, b in mats if n == "head"][0]
    head_us = per["head"]["us"]
    achieved = head_bytes / (head_us * 1e-6) / 1e9

    out = {
        "metric": "Q4_K/Q6_K matvec HBM GB/s (% of peak); 7B-shape Q4_K_M decode tok/s",
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded ggml blocks with the BASELINE distributions)",
        "config": {"workload": "Qwen2.5-7B-shaped Q4_K_M decode-layer matvecs, batch 1 "
                               "(Wq,Wk,Wv,Wo,Wgate,Wup Q4_K; Wdown,head Q6_K), cold HBM",
                   "step_bytes": step_bytes, "timing": "HIP graph per step", "pct_of_hbm_peak": round(100 * value / HBM_PEAK_GBS, 1),
                   "wall_s": round(wall, 4)},
        "roofline": {"bound": "hbm", "kernel": "k_matvec<Q6_K> (output head 152064x3584)",
                     "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": measured_traffic(),
                     "launch_us": head_us, "algo_bytes": head_bytes},
        "per_kernel": per,
    }
    if args.calib_copy:
        src = torch.ones(64 * 1024 * 1024, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
    if not args.no_cpu:
        nthreads = min(len(os.sched_getaffinity(0)), 16)
        out["cpu_baseline"] = cpu_baseline(mats, host, xs, nthreads, args.cpu_seconds)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
