"""Benchmark of the CPAB hot path on one MI355X (BASELINE.json metric and configs).

Default (the driver's line) = BASELINE.json configs[1], "C2": 2D tessellation
[20, 20] on [0,1]^2, zero_boundary=True, fp32, batch 16, 125,000 points uniform
in [0,1]^2 (seed 21); theta ~ N(0,1) * 0.5 in basis coordinates (seed 22);
loss = MSE (torch.nn.functional.mse_loss, mean) against a second seeded theta's (seed 23) warped points.  One step =
Cpab.transform_grid forward + MSE + backward w.r.t. theta, inputs resident in
HBM (A = B theta, expm, fixed-step forward kernel, fused replay/adjoint kernel,
projection).  --config c1|c3|c4|c5|all measures the other BASELINE.json
configs the same way (not the driver's line).

Prints one JSON line per config with, besides the throughput,
  roofline      the dominant kernel: algorithmic work per launch (fp32 FLOPs, or
                bytes for the resampling kernels) over its average duration,
                timed with HIP events that the library records on the launch
                stream around every launch, in a separate run of the same
                number of steps (the timed steps run uninstrumented, last,
                after the other measurements have kept the GPU busy);
  cpu_baseline  the reference-semantics CPU restatement (oracle/, C + OpenMP)
                timed on this host on a bounded sample of the same workload
                (default config only).
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.realpath(__file__))
sys.path.insert(0, os.path.join(ROOT, "fg-cpab_amd"))
sys.path.insert(0, ROOT)

# Algorithmic fp32 FLOPs per trajectory and integration step (FMA = 2), counted
# from the reference kernels (cpab_ops_{1d,2d,3d}.cu):
#   forward  = lookup + Trels apply                  2D 7+8,  3D 25+18
#   backward = midpoint replay + adjoint/moments     2D 31+52, 3D 73+114, 1D 9+18
# The 1D forward is the closed form (~15 flops + 9 per crossing; 15 counted).
FLOPS = {1: {"forward": None, "backward": 27}, 2: {"forward": 15, "backward": 83},
         3: {"forward": 43, "backward": 187}}
FLOPS_1D_FWD = 15
PEAK_FP32_TFLOPS = 157.3   # MI355X fp32 vector peak (packed); non-packed issue tops out at half
PEAK_HBM_GBS = 8000.0
METRIC = "points/sec (fwd+grad), 2D 20x20 tess, 125k pts, B=16; % fp32 VALU peak"


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--config", default="c2",
                    choices=["c1", "c2", "c3", "c4", "c5", "c2_t16", "c2_t30", "all"])
    ap.add_argument("--cpu-seconds", type=float, default=15.0,
                    help="approximate CPU time budget of the cpu_baseline sample")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--nstep", type=int, default=50)
    ap.add_argument("--calibrate-copy", type=int, default=0, metavar="MIB",
                    help="only run 3 device-to-device copies of MIB MiB (scales the "
                         "rocprofv3 FETCH_SIZE / WRITE_SIZE counters) and exit")
    return ap.parse_args()


def calibrate_copy(mib):
    """Plain copies of known size for scaling the rocprofv3 FETCH_SIZE / WRITE_SIZE
    counters: a runtime device-to-device copy and an elementwise kernel (x * 1),
    each reading and writing ``mib`` MiB per launch, 3 launches each."""
    import torch
    n = mib * (1 << 20) // 4
    src = torch.rand(n, device="cuda:0")
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    for _ in range(3):
        dst.copy_(src)
    for _ in range(3):
        torch.mul(src, 1.0, out=dst)
    torch.cuda.synchronize()
    print(json.dumps({"copy_bytes_per_launch": n * 4, "launches": 3,
                      "kernels": ["device copy", "elementwise mul"]}))


def _theta(T, n, scale, seed):
    import numpy as np
    return (np.random.default_rng(seed).standard_normal((n, T.params.d)) * scale).astype(np.float32)


def _blur_noise(shape, sigma, seed):
    import numpy as np
    from scipy.ndimage import gaussian_filter
    x = np.random.default_rng(seed).random(shape).astype(np.float32)
    nsp = len(shape) - 2
    return gaussian_filter(x, sigma=[0, 0] + [sigma] * nsp, mode="reflect",
                           truncate=4.0).astype(np.float32)


def make_c2_inputs(T, nP=125_000, B=16):
    import numpy as np
    pts = np.random.default_rng(21).random((2, nP)).astype(np.float32)
    return pts, _theta(T, B, 0.5, 22), _theta(T, B, 0.5, 23)


def setup(cfg, nstep, dev):
    """Returns (step_fn, info) for one config; step_fn runs one fwd+grad step."""
    import numpy as np
    import torch
    from cpab import Cpab

    if cfg in ("c1", "c2", "c2_t16", "c2_t30"):
        if cfg == "c1":
            T = Cpab([50])
            pts = np.linspace(0, 1, 10_000, dtype=np.float32)[None]
            theta, theta_t = _theta(T, 16, 0.5, 11), _theta(T, 16, 0.5, 12)
            desc = ("C1: 1D CPAB transform_grid fwd+MSE+backward, tess [50], zero_boundary, "
                    "10000 grid points, batch 16, nstepsolver %d" % nstep)
        else:
            n = {"c2": 20, "c2_t16": 16, "c2_t30": 30}[cfg]
            T = Cpab([n, n])
            pts, theta, theta_t = make_c2_inputs(T)
            label = "C2" if cfg == "c2" else f"C2 shape at N_tess {n}"
            desc = (f"{label}: 2D CPAB transform_grid fwd+MSE+backward, tess [{n},{n}], "
                    "zero_boundary, 125000 uniform points, batch 16, nstepsolver %d" % nstep)
        T.set_solver_params(nstepsolver=nstep)
        x = torch.tensor(pts, device=dev)
        th0 = torch.tensor(theta, device=dev)
        with torch.no_grad():
            target = T.transform_grid(x, torch.tensor(theta_t, device=dev))

        def step():
            th = th0.detach().requires_grad_(True)
            out = T.transform_grid(x, th)
            torch.nn.functional.mse_loss(out, target).backward()
            return th.grad

        traj = pts.shape[1] * theta.shape[0]
        info = {"ndim": T.params.ndim, "traj": traj, "desc": desc,
                "global_batch": theta.shape[0], "points": pts.shape[1], "params": T.params}
        if cfg != "c1":
            info["ref_latency"] = lambda: reference_latency(T, x, th0)
        return step, info

    if cfg in ("c3", "c4"):
        if cfg == "c3":
            T = Cpab([30, 30])
            B, size, sigma, seeds = 16, [512, 512], 4.0, (31, 32, 33)
            desc = ("C3: 2D CPAB transform_data fwd+MSE+backward, tess [30,30], zero_boundary, "
                    "16x1x512x512 blurred noise, bilinear, nstepsolver %d" % nstep)
        else:
            T = Cpab([10, 10, 10])
            B, size, sigma, seeds = 1, [128, 128, 128], 3.0, (41, 42, 43)
            desc = ("C4: 3D CPAB transform_data fwd+MSE+backward, tess [10,10,10], zero_boundary, "
                    "1x1x128^3 blurred noise, trilinear, nstepsolver %d" % nstep)
        T.set_solver_params(nstepsolver=nstep)
        data = torch.tensor(_blur_noise((B, 1, *size), sigma, seeds[0]), device=dev)
        target = torch.tensor(_blur_noise((B, 1, *size), sigma, seeds[1]), device=dev)
        th0 = torch.tensor(_theta(T, B, 0.5, seeds[2]), device=dev)

        def step():
            th = th0.detach().requires_grad_(True)
            out = T.transform_data(data, th, size)
            torch.nn.functional.mse_loss(out, target).backward()
            return th.grad

        # The resampling alone (Cpab.interpolate at the warped grid of this
        # workload, forward + backward to the grid): measured separately, since
        # transform_data runs it inside the fused kernels.
        with torch.no_grad():
            grid_t = T.transform_grid(T.uniform_meshgrid(size), th0)
        gout_i = torch.ones((B, 1, *size), device=dev)

        def interp_step():
            gt = grid_t.detach().requires_grad_(True)
            T.interpolate(data, gt, size).backward(gout_i)
            return gt.grad

        nP = int(np.prod(size))
        nd = len(size)
        # Algorithmic HBM bytes of the resampling (data not requiring grad):
        # fwd reads grid_t + image and writes out; bwd reads grad_out, grid_t and
        # image and writes grad_grid.
        img = B * nP * 4
        grid_b = B * nd * nP * 4
        interp_bytes = {"interp_forward": grid_b + img + img,
                        "interp_backward": img + grid_b + img + grid_b}
        return step, {"ndim": nd, "traj": B * nP, "desc": desc, "global_batch": B, "params": T.params,
                      "points": nP, "interp_bytes": interp_bytes, "interp_step": interp_step}

    # c5: chain of 8 stages on a 512x512 meshgrid
    T = Cpab([16, 16])
    T.set_solver_params(nstepsolver=nstep)
    K = 8
    grid = T.uniform_meshgrid([512, 512])
    chain0 = torch.tensor((np.random.default_rng(51).standard_normal((K, T.params.d)) * 0.3)
                          .astype(np.float32), device=dev)
    chain_t = torch.tensor((np.random.default_rng(52).standard_normal((K, T.params.d)) * 0.3)
                           .astype(np.float32), device=dev)
    with torch.no_grad():
        target = T.transform_grid_chain(grid, chain_t, scale_by_dt=True)

    def step():
        ch = chain0.detach().requires_grad_(True)
        out = T.transform_grid_chain(grid, ch, scale_by_dt=True)
        torch.nn.functional.mse_loss(out, target).backward()
        return ch.grad

    nP = 512 * 512
    return step, {"ndim": 2, "traj": nP * K, "points_per_step": nP, "desc":
                  "C5: 2D CPAB transform_grid_chain fwd+MSE+backward, tess [16,16], 8 stages, "
                  "scale_by_dt, 262144 grid points, nstepsolver %d" % nstep,
                  "global_batch": 1, "points": nP, "params": T.params}


def reference_latency(T, x, th0, n_warmup=10, n_iter=100):
    """Forward and backward latency measured the way the reference's benchmark
    does (benchmarks/benchmark_transformer.py:71-128): the forward is timed from
    one synchronisation to the next around ``transform_grid``; the backward is
    ``output.sum().backward()`` alone, the forward run untimed before it.  Mean
    milliseconds over ``n_iter`` runs, comparable with the published figure's
    N_tess points (docs/assets/fgcpab-scaling-2d.svg:518,734)."""
    import numpy as np
    import torch

    def fwd():
        return T.transform_grid(x, th0.detach().requires_grad_(True))

    for _ in range(n_warmup):
        fwd().sum().backward()
    torch.cuda.synchronize()
    tf, tb = [], []
    for _ in range(n_iter):
        torch.cuda.synchronize()
        a = time.perf_counter()
        out = fwd()
        torch.cuda.synchronize()
        tf.append(time.perf_counter() - a)
    for _ in range(n_iter):
        loss = fwd().sum()
        torch.cuda.synchronize()
        a = time.perf_counter()
        loss.backward()
        torch.cuda.synchronize()
        tb.append(time.perf_counter() - a)
    del out
    # Peak device memory of that backward above what is allocated just before it
    # (the output, the saved tensors and the inputs already resident).
    loss = fwd().sum()
    torch.cuda.synchronize()
    base = torch.cuda.memory_allocated()
    torch.cuda.reset_peak_memory_stats()
    loss.backward()
    torch.cuda.synchronize()
    bwd_mib = (torch.cuda.max_memory_allocated() - base) / 2**20
    return {"forward_ms": round(float(np.mean(tf)) * 1e3, 4),
            "backward_ms": round(float(np.mean(tb)) * 1e3, 4),
            "backward_peak_MiB": round(bwd_mib, 2),
            "method": "benchmarks/benchmark_transformer.py:71-128 (sync-to-sync mean of 100, "
                      "backward = sum().backward() alone; backward_peak_MiB = allocator peak during "
                      "that backward above the memory allocated before it)"}


def deterministic_timing(step, params, steps, warmup):
    """The same step with ``Cpab.set_solver_params(deterministic_grad=True)``:
    uninstrumented ms per step, and whether two steps' theta gradients are the
    same bit for bit (they are not in the default mode's float-atomic sums)."""
    import torch

    params.deterministic_grad = True
    try:
        for _ in range(warmup):
            step()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps):
            step()
        torch.cuda.synchronize()
        t1 = time.perf_counter()
        a, b = step().clone(), step().clone()
        return {"ms_per_step": round((t1 - t0) * 1e3 / steps, 4),
                "repeat_bitwise_equal": bool(torch.equal(a, b))}
    finally:
        params.deterministic_grad = False


def step_memory(step):
    """Device memory of one step beyond what is resident before it (inputs, target,
    parameters): the peak of torch's caching allocator during the step, in MiB."""
    import torch
    torch.cuda.synchronize()
    base = torch.cuda.memory_allocated()
    torch.cuda.reset_peak_memory_stats()
    step()
    torch.cuda.synchronize()
    peak = torch.cuda.max_memory_allocated()
    return {"step_peak_MiB": round((peak - base) / 2**20, 2),
            "resident_before_step_MiB": round(base / 2**20, 2)}


NAMES = ["forward", "backward", "image_forward", "image_backward", "interp_forward",
         "interp_backward"]
# fused transform_data kernels carry the integrator's work
FLOP_KIND = {"forward": "forward", "backward": "backward", "image_forward": "forward",
             "image_backward": "backward"}


def kernel_timing(step, steps, warmup):
    """{kernel: (total ms, launches)} over ``steps`` steps run after ``warmup``
    ones with the library's HIP-event timing on.  Those events leave the GPU
    idle for a few microseconds between kernels (about 5.5 us per timed kernel
    on MI355X), so the wall time comes from separate, uninstrumented steps
    (wall_time)."""
    import torch
    from cpab.pytorch import _native

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    for n in NAMES:
        _native.profile_read(n)
    _native.profile_enable(True)
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    _native.profile_enable(False)
    return {n: _native.profile_read(n) for n in NAMES}


def wall_time(step, steps, warmup):
    """Seconds for exactly ``steps`` uninstrumented steps after ``warmup``
    untimed ones, bracketed by device synchronisations."""
    import torch

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        g = step()
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    assert torch.isfinite(g).all()
    return t1 - t0


def gpu_bench(cfg, args):
    import torch

    dev = torch.device("cuda:0")
    step, info = setup(cfg, args.nstep, dev)
    # The bench's other measurements first, the kernel timing and the timed
    # steps last: the GPU then comes to them busy, at its sustained clocks (from
    # a cold start the first few tens of steps run ~5 % slower).
    extras = {"memory": step_memory(step),
              "deterministic": deterministic_timing(step, info["params"], args.steps,
                                                    args.warmup)}
    if "ref_latency" in info:
        extras["reference_style_latency"] = info["ref_latency"]()
    if "interp_step" in info:
        # HBM roofline of the standalone resampling kernels on this workload's shapes
        itiming = kernel_timing(info["interp_step"], args.steps, args.warmup)
        for n, nbytes in info["interp_bytes"].items():
            ms, cnt = itiming[n]
            if cnt:
                rate = nbytes / (ms / cnt * 1e-3) / 1e9
                extras.setdefault("interp_roofline", {})[n] = {
                    "avg_ms": round(ms / cnt, 5), "achieved_GBs": round(rate, 1),
                    "peak_GBs": PEAK_HBM_GBS, "frac": round(rate / PEAK_HBM_GBS, 4),
                    "algorithmic_bytes": nbytes, "traffic": profiled_traffic(cfg, n)}
    timing = kernel_timing(step, args.steps, args.warmup)
    secs = wall_time(step, args.steps, args.warmup)
    ms_step = secs * 1e3 / args.steps
    nd, traj, T = info["ndim"], info["traj"], args.nstep
    kern = {}
    for n, kind in FLOP_KIND.items():
        ms, cnt = timing[n]
        if cnt == 0:
            continue
        per_step = cnt / args.steps
        per_launch_traj = traj / per_step
        f_step = FLOPS[nd][kind]
        flops = (FLOPS_1D_FWD if f_step is None else f_step * T) * per_launch_traj
        kern[n] = {"avg_ms": ms / cnt, "work": flops, "unit": "TFLOP/s",
                   "rate": flops / (ms / cnt * 1e-3) / 1e12, "per_step": per_step}
    # dominant kernel = largest share of the step's kernel time
    dom = max(kern, key=lambda k: kern[k]["avg_ms"] * kern[k]["per_step"])
    d = kern[dom]
    roof = {"bound": "valu", "kernel": dom, "achieved": round(d["rate"], 3),
            "peak": PEAK_FP32_TFLOPS, "unit": d["unit"],
            "frac": round(d["rate"] / PEAK_FP32_TFLOPS, 4), "traffic": profiled_traffic(cfg, dom)}
    pts_per_step = info.get("points_per_step", traj)
    out = {"ms_per_step": ms_step, "value": pts_per_step / (ms_step * 1e-3), "roofline": roof,
           "info": info,
           "kernels": {k: {"avg_ms": round(v["avg_ms"], 5), "launches_per_step": v["per_step"],
                           v["unit"]: round(v["rate"], 3)} for k, v in kern.items()}}
    total = sum(v["work"] * v["per_step"] for v in kern.values())
    out["integrator_tflops_per_step"] = round(total / (ms_step * 1e-3) / 1e12, 3)
    out.update(extras)
    return out


KERNEL_PREFIX = {"forward": ("fwd2d_kernel", "fwd3d_kernel", "fwd1d_closed_kernel"),
                 "backward": ("backward_kernel",),
                 "image_forward": ("image_forward_kernel",),
                 "image_backward": ("image_backward_kernel",),
                 "interp_forward": ("interp_fwd_kernel", "interp1d_fwd_kernel"),
                 "interp_backward": ("interp_bwd_kernel", "interp1d_bwd_kernel")}


def profiled_traffic(cfg, kernel):
    """HBM bytes per launch of ``kernel`` for ``cfg`` as measured by the committed
    rocprofv3 FETCH_SIZE / WRITE_SIZE runs (profiles/traffic.json, each counter
    scaled by its plain-copy factor), or None when no such measurement exists."""
    try:
        with open(os.path.join(ROOT, "profiles", "traffic.json")) as f:
            t = json.load(f)
    except (OSError, ValueError):
        return None
    for name, v in t.get("configs", {}).get(cfg, {}).items():
        if name.startswith(KERNEL_PREFIX.get(kernel, ())):
            return v["bytes"]
    return None


def cpu_model():
    """The host CPU's model name (/proc/cpuinfo), or the platform's processor string."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.lower().startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    import platform
    return platform.processor() or "unknown"


def cpu_baseline(args):
    """Oracle (C, OpenMP) on a sample of the C2 workload: forward + MSE grad + backward."""
    import numpy as np
    cores = len(os.sched_getaffinity(0))
    os.environ.setdefault("OMP_NUM_THREADS", str(cores))
    cores = int(os.environ["OMP_NUM_THREADS"])
    from cpab import Cpab
    from oracle import oracle as orc

    T = Cpab([20, 20])
    B = 16
    pts_all, theta, theta_t = make_c2_inputs(T)
    nstep = args.nstep

    def run(n):
        pts = pts_all[:, :n]
        At = orc.affine(theta_t, T.params.basis).reshape(B, -1, 2, 3)
        tgt = orc.forward_trels(pts, orc.expm(2, At, 1.0 / nstep), At, [20, 20], nstep)
        t0 = time.perf_counter()
        As = orc.affine(theta, T.params.basis).reshape(B, -1, 2, 3)
        out = orc.forward_trels(pts, orc.expm(2, As, 1.0 / nstep), As, [20, 20], nstep)
        g = (2.0 / out.size) * (out - tgt)
        orc.backward(pts, As, g.astype(np.float32), [20, 20], nstep)
        return time.perf_counter() - t0

    n = 2000
    dt = run(n)
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
    pps = n * B / per
    return {"value": round(pps, 1), "unit": "points/s", "cores": cores, "kind": "port",
            "cpu_model": cpu_model(),
            "gflops": round(pps * (FLOPS[2]["forward"] + FLOPS[2]["backward"]) * nstep / 1e9, 3),
            "gflops_note": "algorithmic fp32 FLOPs of fwd+grad, 98 per trajectory-step (the count "
                           "the GPU roofline uses)",
            "sample": f"{n} of the 125000 points x 16 thetas, fwd+MSE+grad, mean of "
                      f"{reps} runs ({per:.3f} s each), C/OpenMP restatement of the reference "
                      f"kernels (oracle/)"}


def line_for(cfg, r, args, cpu):
    info = r["info"]
    line = {
        "metric": METRIC if cfg == "c2" else f"points/sec (fwd+grad), {info['desc'].split(':')[0]}",
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
        "data": "synthetic (seeded inputs as in BASELINE.json configs)",
        "config": {"workload": info["desc"], "global_batch": info["global_batch"],
                   "points": info["points"], "parallelism": "single-gpu"},
        "roofline": r["roofline"],
        "cpu_baseline": cpu,
        "kernels": r["kernels"],
        "integrator_tflops_per_step": r["integrator_tflops_per_step"],
        "memory": r["memory"],
        "deterministic": r["deterministic"],
    }
    if "reference_style_latency" in r:
        line["reference_style_latency"] = r["reference_style_latency"]
    if "interp_roofline" in r:
        line["interp_roofline"] = r["interp_roofline"]
    if cfg == "c2":
        line["pct_fp32_valu_peak_step"] = round(100 * r["integrator_tflops_per_step"]
                                                / PEAK_FP32_TFLOPS, 2)
    return line


def main():
    args = parse()
    if args.calibrate_copy:
        calibrate_copy(args.calibrate_copy)
        return
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only; --gpus {args.gpus} is not supported "
              "(the CPAB path has no multi-GPU component here)", file=sys.stderr)
        sys.exit(2)
    cfgs = (["c1", "c2", "c3", "c4", "c5", "c2_t16", "c2_t30"] if args.config == "all"
            else [args.config])
    for cfg in cfgs:
        r = gpu_bench(cfg, args)
        cpu = None if (args.no_cpu or cfg != "c2") else cpu_baseline(args)
        print(json.dumps(line_for(cfg, r, args, cpu)), flush=True)


if __name__ == "__main__":
    main()
