#!/usr/bin/env python
"""Selective-scan fwd+bwd throughput on one MI355X (BASELINE.json metric).

Workload: the custom-VJP selective scan of a
SelectiveSSM block, B=8, L=8192, D_inner=2048, N=16, fp32, loss = sum(y * g).
One step = ssm_fwd (with the checkpoints the backward needs) + ssm_bwd over one
batch of synthetic inputs already resident in HBM.  value = B*L*steps / time.

The JSON line also carries
  roofline      for the dominant launch (ssm_bwd): algorithmic bytes per launch
                / its mean duration from HIP events on the launch stream,
                against MI355X's 8 TB/s; `traffic` = HBM bytes per launch from
                rocprofv3 FETCH_SIZE/WRITE_SIZE (profiles/traffic_c1.txt), or null
  cpu_baseline  the CPU restatement of the reference's custom-VJP path
                (oracle/ssm_oracle.c), timed on this host's cores on a sample
                of the same workload
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, REPO)

HBM_PEAK_GBS = 8000.0

# BASELINE.json configs at the op level (the scan's own shapes: D = D_inner).
# --config 1 is the bench line; the others are extra measurements.
CONFIGS = {
    1: dict(batch=8, seqlen=8192, dim=2048, dstate=16, io="f32", directions=1,
            workload="SelectiveSSM custom_vjp_scan selective scan fwd+bwd (configs[1])"),
    2: dict(batch=4, seqlen=131072, dim=512, dstate=16, io="f32", directions=2,
            workload="BidirectionalMamba scans fwd+bwd, forward and reverse+complement directions (configs[2])"),
    3: dict(batch=1, seqlen=1 << 20, dim=1024, dstate=16, io="f32", directions=1,
            workload="SelectiveSSM recursive_scan selective scan fwd+bwd, long sequence (configs[3])"),
    4: dict(batch=16, seqlen=4096, dim=5120, dstate=16, io="bf16", directions=1,
            workload="SelectiveSSM selective scan fwd+bwd, bf16 I/O, fp32 state (configs[4])"),
}
CONFIG = CONFIGS[1]


def alg_bytes(B, L, D, N, w=4, gate=False):
    """Compulsory op-boundary bytes: every input read once, every output written once."""
    fwd = (3 * B * L * D + 2 * B * L * N) * w + 4 * D * N            # u, dt, y; B, C; A
    bwd = (5 * B * L * D + 4 * B * L * N) * w + 8 * D * N            # u, dt, dy, du, ddt; B, C, dB, dC; A, dA
    if gate:
        fwd += B * L * D * w                                          # z
        bwd += 2 * B * L * D * w                                      # z, dz
    return fwd, bwd


def read_traffic(path):
    """HBM bytes per ssm_bwd launch from a rocprofv3 PMC summary, or None."""
    if not os.path.exists(path):
        return None
    vals = {}
    with open(path) as f:
        for line in f:
            if ":" in line and not line.startswith("#"):
                k, v = line.split(":", 1)
                vals[k.strip()] = v.strip()
    try:
        return float(vals["traffic_bytes_per_launch"])
    except (KeyError, ValueError):
        return None


def cpu_baseline(B, L, D, N, tensors):
    """Time the C port of the reference's custom-VJP path on a sample: half the batch
    rows of the very arrays the GPU ran (``tensors``: u, dt, A, B, C, g on the GPU)."""
    import numpy as np
    from oracle import c_oracle

    cores = len(os.sched_getaffinity(0))
    sb = min(4, B)  # 4 of the 8 batch rows: about 3 s per run on 16 cores, 10-15 s in all
    inp = {k: (t if k == "A" else t[:sb]).float().cpu().numpy() for k, t in tensors.items()}
    args = (inp["u"], inp["dt"], inp["A"], inp["B"], inp["C"])
    times = []
    for rep in range(4):  # first run is the warmup
        t0 = time.perf_counter()
        c_oracle.scan_fwd(*args, nthreads=cores)
        c_oracle.scan_bwd(*args, inp["g"], nthreads=cores)
        times.append(time.perf_counter() - t0)
    t = float(np.median(times[1:]))
    return {
        "value": sb * L / t,
        "unit": "tokens/s",
        "cores": cores,
        "kind": "port",
        "sample": f"fwd+bwd of batch rows 0..{sb - 1} of {B} of the GPU run's inputs (L={L}, D={D}, N={N}, "
                  f"fp32), recursive custom-VJP "
                  f"algorithm (min_recursion_length=2, recursive_split=2), median of 3 after 1 warmup, "
                  f"{t:.2f} s per run",
    }


MODULES = {
    1: ("SelectiveSSM(hidden_features=16, shift_conv_size=4, custom_vjp_scan=True) on x (8, 8192, 2048)",
        dict(kind="ssm", B=8, L=8192, D=2048, kw=dict(custom_vjp_scan=True))),
    2: ("BidirectionalMamba(hidden_features=16, expansion_factor=2, complement, tie_in_proj, tie_gate, concat), "
        "d_model 256, on one-hot DNA (4, 131072) embedded by Linear(4, 256)",
        dict(kind="mamba", B=4, L=131072, D=256)),
    3: ("SelectiveSSM(hidden_features=16, shift_conv_size=4, recursive_scan=True) on x (1, 1048576, 1024)",
        dict(kind="ssm", B=1, L=1 << 20, D=1024, kw=dict(recursive_scan=True))),
    4: ("SelectiveSSM(hidden_features=16, shift_conv_size=4) on bf16 x (16, 4096, 5120)",
        dict(kind="ssm", B=16, L=4096, D=5120, kw=dict(), bf16=True)),
}


def module_bench(args):
    """fwd+bwd of the config's whole module (BASELINE.json configs[1..4] module shapes)."""
    import torch
    from selectssm_amd import BidirectionalMamba, SelectiveSSM

    desc, m = MODULES[args.config]
    B, L, D = m["B"], m["L"], m["D"]
    g = torch.Generator(device="cuda").manual_seed(0)
    if m["kind"] == "ssm":
        model = SelectiveSSM(hidden_features=16, shift_conv_size=4, features=D, device="cuda", generator=g, **m["kw"])
        dtype = torch.bfloat16 if m.get("bf16") else torch.float32
        x = torch.randn(B, L, D, device="cuda", generator=g).to(dtype)
        embed = None
    else:
        model = BidirectionalMamba(hidden_features=16, expansion_factor=2.0, complement=True, tie_in_proj=True,
                                   tie_gate=True, concatenate_fwd_rev=True, ssm_args=dict(shift_conv_size=4),
                                   features=D, device="cuda", generator=g)
        ids = torch.randint(0, 4, (B, L), device="cuda", generator=g)
        x = torch.nn.functional.one_hot(ids, 4).float()
        embed = torch.nn.Linear(4, D, device="cuda")
    params = list(model.parameters()) + (list(embed.parameters()) if embed is not None else [])

    def step():
        for p in params:
            p.grad = None
        x.grad = None  # the input's gradient is produced every step, not accumulated over steps
        h = embed(x) if embed is not None else x.requires_grad_(True)
        y = model(h)
        grad = torch.ones_like(y) if args.config != 2 else torch.randn_like(y, generator=g)
        y.backward(grad)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    torch.cuda.reset_peak_memory_stats()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    return {
        "metric": "module fwd+bwd tokens/s on 1 MI355X",
        "value": B * L * args.steps / wall,
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": wall * 1e3 / args.steps,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16 I/O, f32 state" if m.get("bf16") else "f32",
        "data": "synthetic (torch generator, seed 0), random-init parameters",
        "config": {"workload": desc, "batch": B, "seqlen": L, "d_model" if m["kind"] == "mamba" else "d_inner": D},
        "peak_hbm_bytes": torch.cuda.max_memory_allocated(),
    }


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--config", type=int, default=1, choices=sorted(CONFIGS),
                    help="BASELINE.json config to run (1 is the bench line)")
    ap.add_argument("--gate", action="store_true", help="fuse the silu(z) gate (BidirectionalMamba epilogue)")
    ap.add_argument("--module", action="store_true",
                    help="time the whole module of the config (SelectiveSSM / BidirectionalMamba fwd+bwd, "
                         "with its projections) instead of the scan op")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="only run a plain 1 GiB device copy (known HBM bytes) to scale rocprofv3 "
                         "FETCH_SIZE / WRITE_SIZE counters")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (asked for --gpus {args.gpus}); the scan's multi-GPU "
              "sharding is a design note, not a measured path", file=sys.stderr)
        sys.exit(2)

    import torch

    if args.calibrate_copy:
        n = (1 << 30) // 4
        src = torch.ones(n, dtype=torch.float32, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(max(args.steps, 1)):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"calibrate_copy_bytes_read": 4 * n, "calibrate_copy_bytes_written": 4 * n,
                          "launches": max(args.steps, 1)}))
        return

    if args.module:
        print(json.dumps(module_bench(args)), flush=True)
        return

    from selectssm_amd.scan import scan_bwd, scan_bwd_pair, scan_fwd, scan_fwd_pair
    from selectssm_amd.synthetic import make_inputs_gpu

    cfg = CONFIGS[args.config]
    B, L, D, N = cfg["batch"], cfg["seqlen"], cfg["dim"], cfg["dstate"]
    io = torch.bfloat16 if cfg["io"] == "bf16" else torch.float32
    w = 2 if cfg["io"] == "bf16" else 4
    x = make_inputs_gpu(B, L, D, N, seed=0)
    u, dt, Bc, Cc, g = (x[k].to(io).contiguous() for k in ("u", "dt", "B", "C", "g"))
    A = x["A"]
    z = x["z"].to(io).contiguous() if args.gate else None
    del x
    # direction 2 is the reverse + complement scan with its own A
    dirs = [dict(A=A, reverse=False, complement=False)]
    if cfg["directions"] == 2:
        dirs.append(dict(A=(A * 0.5).contiguous(), reverse=True, complement=True))

    def call(dr):
        return dict(u=u, delta=dt, A=dr["A"], B=Bc, C=Cc, z=z, reverse=dr["reverse"], complement=dr["complement"])

    # one direction: ssm_fwd then ssm_bwd; two: ssm_fwd_pair then
    # ssm_bwd_pair, whose time-split aggregate passes cover both directions
    def fwd():
        if len(dirs) == 2:
            return [ck for _, ck in scan_fwd_pair([call(dr) for dr in dirs])]
        return [scan_fwd(u, dt, A, Bc, Cc, None, z)[1]]

    def bwd(cks):
        if len(dirs) == 2:
            return scan_bwd_pair([dict(call(dr), ckpt=ck, dy=g) for dr, ck in zip(dirs, cks)])
        return scan_bwd(u, dt, A, Bc, Cc, None, z, cks[0], g)

    for _ in range(args.warmup):
        bwd(fwd())
    torch.cuda.synchronize()
    torch.cuda.reset_peak_memory_stats()

    K = args.steps
    nd = len(dirs)
    # events: one at the start, then one after each forward and one after each
    # backward; a step's forward is timed from the previous step's last event
    # (each recorded event costs the stream a few microseconds, so none is
    # recorded twice at one point)
    start = torch.cuda.Event(enable_timing=True)
    ev = [[torch.cuda.Event(enable_timing=True) for _ in range(2)] for _ in range(K)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    start.record()
    for k in range(K):
        cks = fwd()
        ev[k][0].record()
        bwd(cks)
        ev[k][1].record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0

    # per direction (a pair call's time split evenly between its two scans)
    fwd_ms = sum((start if k == 0 else ev[k - 1][1]).elapsed_time(ev[k][0]) for k in range(K)) / (K * nd)
    bwd_ms = sum(e[0].elapsed_time(e[1]) for e in ev) / (K * nd)
    fwd_b, bwd_b = alg_bytes(B, L, D, N, w, gate=args.gate)
    tokens = B * L * K
    achieved = bwd_b / (bwd_ms * 1e-3) / 1e9
    traffic = read_traffic(os.path.join(REPO, "profiles", "traffic_c1.txt")) if args.config == 1 and not args.gate \
        else None

    config = {"workload": cfg["workload"] + (" with the silu(z) gate fused" if args.gate else ""),
              "batch": B, "seqlen": L, "d_inner": D, "d_state": N, "io": cfg["io"]}
    if nd == 2:
        config["directions"] = 2
    line = {
        "metric": "selective-scan fwd+bwd tokens/s and % of HBM roofline on 1 MI355X",
        "value": tokens / wall,
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": K,
        "warmup": args.warmup,
        "ms_per_step": wall * 1e3 / K,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32" if cfg["io"] == "f32" else "bf16 I/O, f32 state",
        "data": f"synthetic (BASELINE.json configs[{args.config}] distributions, torch generator, seed 0)",
        "config": config,
        "roofline": {
            "bound": "hbm",
            "kernel": "ssm_bwd (ssm_bwd_kernel + partial-sum reductions)",
            "achieved": achieved,
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": achieved / HBM_PEAK_GBS,
            "traffic": traffic,
            "alg_bytes_per_launch": bwd_b,
            "mean_launch_ms": bwd_ms,
        },
        "step_roofline_frac": nd * (fwd_b + bwd_b) / (wall / K) / 1e9 / HBM_PEAK_GBS,
        "fwd": {"mean_launch_ms": fwd_ms, "alg_bytes_per_launch": fwd_b,
                "achieved_GBs": fwd_b / (fwd_ms * 1e-3) / 1e9},
        "peak_hbm_bytes": torch.cuda.max_memory_allocated(),
    }
    if not args.no_cpu_baseline and args.config == 1 and not args.gate:
        line["cpu_baseline"] = cpu_baseline(B, L, D, N, dict(u=u, dt=dt, A=A, B=Bc, C=Cc, g=g))
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
