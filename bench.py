"""Benchmark of the CPAB hot path on one MI355X (BASELINE.json metric).

Workload ("C2"): 2D tessellation [20, 20] on [0,1]^2,
zero_boundary=True, fp32, batch 16, 125,000 points uniform in [0,1]^2 (seed 21);
theta ~ N(0,1) * 0.5 in basis coordinates (seed 22); loss = MSE against a second
seeded theta's (seed 23) warped points.  One step = transform_grid forward +
MSE + backward w.r.t. theta (the Cpab API path: A = B theta, expm, fixed-step
forward kernel, fused replay/adjoint kernel, projection), inputs resident in HBM.

Prints ONE JSON line.  Besides the step throughput it reports
  roofline      the dominant kernel's algorithmic fp32 FLOPs per launch over its
                average duration, timed with HIP events recorded by the library on
                the launch stream during the timed steps;
  cpu_baseline  the reference-semantics CPU restatement (oracle/, OpenMP) timed on
                this host on a bounded sample of the same workload.
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.realpath(__file__))
sys.path.insert(0, os.path.join(ROOT, "fg-cpab_amd"))
sys.path.insert(0, ROOT)

# Algorithmic fp32 FLOPs per trajectory and step (FMA = 2), from the reference
# kernels: forward Trels step 15 (lookup 7 + affine apply 8); backward = midpoint
# replay 31 (lookup 7 + 2 affine evals 16 + 4 fma 8) + adjoint/moments 52.
FLOPS_FWD_STEP_2D = 15
FLOPS_BWD_STEP_2D = 31 + 52
PEAK_FP32_TFLOPS = 157.3   # MI355X fp32 vector peak (packed); non-packed issue tops out at half
PEAK_HBM_GBS = 8000.0


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--cpu-seconds", type=float, default=15.0,
                    help="approximate CPU time budget of the cpu_baseline sample")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--nstep", type=int, default=50)
    ap.add_argument("--calibrate-copy", type=int, default=0, metavar="MIB",
                    help="only run 3 device-to-device copies of MIB MiB (scales the "
                         "rocprofv3 FETCH_SIZE / WRITE_SIZE counters) and exit")
    return ap.parse_args()


def calibrate_copy(mib):
    """Plain copy kernel of known size: reads and writes mib MiB per launch."""
    import torch
    n = mib * (1 << 20) // 4
    src = torch.rand(n, device="cuda:0")
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_bytes_per_launch": n * 4, "launches": 3}))


def make_inputs(T, nP, B, seed_pts=21, seed_theta=22, seed_target=23):
    import numpy as np
    pts = np.random.default_rng(seed_pts).random((2, nP)).astype(np.float32)
    theta = (np.random.default_rng(seed_theta).standard_normal((B, T.params.d)) * 0.5).astype(np.float32)
    theta_t = (np.random.default_rng(seed_target).standard_normal((B, T.params.d)) * 0.5).astype(np.float32)
    return pts, theta, theta_t


def gpu_bench(args):
    import numpy as np
    import torch
    from cpab import Cpab
    from cpab.pytorch import _native

    dev = torch.device("cuda:0")
    T = Cpab([20, 20])
    T.set_solver_params(nstepsolver=args.nstep)
    nP, B = 125_000, 16
    pts, theta, theta_t = make_inputs(T, nP, B)
    x = torch.tensor(pts, device=dev)
    th0 = torch.tensor(theta, device=dev)
    with torch.no_grad():
        target = T.transform_grid(x, torch.tensor(theta_t, device=dev))

    def step():
        th = th0.detach().requires_grad_(True)
        out = T.transform_grid(x, th)
        loss = torch.mean((out - target) ** 2)
        loss.backward()
        return th.grad

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    _native.profile_read("forward")
    _native.profile_read("backward")
    _native.profile_enable(True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        g = step()
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    _native.profile_enable(False)
    fwd_ms, fwd_n = _native.profile_read("forward")
    bwd_ms, bwd_n = _native.profile_read("backward")
    assert torch.isfinite(g).all()

    ms_step = (t1 - t0) * 1e3 / args.steps
    traj = nP * B
    kern = {
        "forward": (fwd_ms / max(fwd_n, 1), FLOPS_FWD_STEP_2D * args.nstep * traj),
        "backward": (bwd_ms / max(bwd_n, 1), FLOPS_BWD_STEP_2D * args.nstep * traj),
    }
    dom = max(kern, key=lambda k: kern[k][0])
    dom_ms, dom_flops = kern[dom]
    achieved = dom_flops / (dom_ms * 1e-3) / 1e12
    total_flops = (FLOPS_FWD_STEP_2D + FLOPS_BWD_STEP_2D) * args.nstep * traj
    return {
        "ms_per_step": ms_step,
        "value": traj / (ms_step * 1e-3),
        "kernels": {k: {"avg_ms": round(v[0], 5), "gflop": round(v[1] / 1e9, 4),
                        "tflops": round(v[1] / (v[0] * 1e-3) / 1e12, 3)} for k, v in kern.items()},
        "dominant": dom,
        "roofline": {"bound": "valu", "kernel": dom, "achieved": round(achieved, 3),
                     "peak": PEAK_FP32_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(achieved / PEAK_FP32_TFLOPS, 4), "traffic": None},
        "step_tflops": round(total_flops / (ms_step * 1e-3) / 1e12, 3),
    }


def cpu_baseline(args):
    """Oracle (C, OpenMP) on a sample of the same workload: forward + MSE grad + backward."""
    import numpy as np
    cores = len(os.sched_getaffinity(0))
    os.environ.setdefault("OMP_NUM_THREADS", str(cores))
    cores = int(os.environ["OMP_NUM_THREADS"])
    from cpab import Cpab
    from oracle import oracle as orc

    T = Cpab([20, 20])
    B = 16
    pts_all, theta, theta_t = make_inputs(T, 125_000, B)
    nstep = args.nstep

    def run(n):
        pts = pts_all[:, :n]
        As = orc.affine(theta, T.params.basis).reshape(B, -1, 2, 3)
        At = orc.affine(theta_t, T.params.basis).reshape(B, -1, 2, 3)
        tgt = orc.forward_trels(pts, orc.expm(2, At, 1.0 / nstep), At, [20, 20], nstep)
        t0 = time.perf_counter()
        As = orc.affine(theta, T.params.basis).reshape(B, -1, 2, 3)
        out = orc.forward_trels(pts, orc.expm(2, As, 1.0 / nstep), As, [20, 20], nstep)
        g = (2.0 / out.size) * (out - tgt)
        mom, gp = orc.backward(pts, As, g.astype(np.float32), [20, 20], nstep)
        orc.project(mom.reshape(B, -1).astype(np.float32), T.params.basis)
        return time.perf_counter() - t0

    n = 2000
    dt = run(n)
    # grow the sample to ~cpu_seconds of work (capped at the full 125k points)
    while dt < args.cpu_seconds / 4 and n < 125_000:
        n = min(125_000, int(n * min(8.0, max(2.0, args.cpu_seconds / 4 / max(dt, 1e-3)))))
        dt = run(n)
    reps, tot = 0, 0.0
    while tot < args.cpu_seconds / 2 or reps < 2:
        tot += run(n)
        reps += 1
        if reps >= 20:
            break
    per = tot / reps
    return {"value": round(n * B / per, 1), "unit": "points/s", "cores": cores, "kind": "port",
            "sample": f"{n} of the 125000 points x 16 thetas, fwd+MSE+grad, mean of "
                      f"{reps} runs ({per:.3f} s each), OpenMP C restatement (oracle/)"}


def main():
    args = parse()
    if args.calibrate_copy:
        calibrate_copy(args.calibrate_copy)
        return
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only; --gpus {args.gpus} is not supported "
              "(the CPAB path has no multi-GPU component here)", file=sys.stderr)
        sys.exit(2)
    r = gpu_bench(args)
    cpu = None if args.no_cpu else cpu_baseline(args)
    line = {
        "metric": "points/sec (fwd+grad), 2D 20x20 tess, 125k pts, B=16; % fp32 VALU peak",
        "value": round(r["value"], 1),
        "unit": "points/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(r["ms_per_step"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded uniform points, N(0,1)*0.5 thetas)",
        "config": {"workload": "C2: 2D CPAB transform_grid fwd+MSE+backward, tess [20,20], "
                               "zero_boundary, 125000 uniform points, batch 16, nstepsolver 50",
                   "global_batch": 16, "points": 125000, "parallelism": "single-gpu"},
        "roofline": r["roofline"],
        "cpu_baseline": cpu,
        "kernels": r["kernels"],
        "step_tflops": r["step_tflops"],
        "pct_fp32_valu_peak_step": round(100 * r["step_tflops"] / PEAK_FP32_TFLOPS, 2),
    }
    print(json.dumps(line))


if __name__ == "__main__":
    main()
