"""Benchmark of the LTC fused ODE-solver path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu-baseline] [--no-large]

Headline workload (BASELINE.json metric, config 1's shape run on the GPU):
one TrueLiquidTimeConstant layer, B=24 T=8 D=128 H=64, 6 unfolds, dt=1/30,
Bernoulli(0.5) masks, seeded init (torch.manual_seed(42)), x ~ N(0,1),
loss = sum(out). A step is module forward (LayerNorm, affine, softplus
transforms, fused HIP loop) plus loss.backward(), as the reference's
bench_ltc.py:62-96 times it.

Printed: one JSON line with the contract fields, plus
  roofline      dominant kernel of the step: algorithmic FLOP per launch over
                its mean launch time from HIP events recorded by the library on
                its launch stream, against the 157.3 TFLOP/s FP32 peak;
  cpu_baseline  the CPU oracle's TorchScript restatement of the reference path,
                same module and shapes, timed on this host's cores;
  large_configs BASELINE configs 2-5 at full size on the GPU (kernel times).

Only rank 0 at N=1 runs; more GPUs are not part of this build.
"""

from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "ltc-cuda_amd"))
sys.path.insert(0, ROOT)

import torch  # noqa: E402

METRIC = "fwd+bwd ms/step & synapse-updates/s (B24 T8 D128 H64, 6 unfolds)"
PEAK_FP32_TFLOPS = 157.3          # MI355X FP32 (vector and matrix)
LANE_SLOTS_PER_S = 256 * 64 * 2.4e9  # 256 CUs x 64 lanes x 2.4 GHz
PEAK_HBM_GBS = 8000.0
# Published fwd+bwd of the reference CUDA kernels at this config, GTX 1080 (README.md:13).
REF_GTX1080_MS = 12.7

C1 = dict(B=24, T=8, D=128, H=64, U=6, sparsity=0.5, loss="sum", x="randn")
LARGE = {
    "C2": dict(B=32, T=16, D=128, H=128, U=6, sparsity=0.5, loss="sum", x="randn"),
    "C3": dict(B=256, T=64, D=256, H=256, U=6, sparsity=0.5, loss="mse", x="randn"),
    "C4": dict(B=128, T=32, D=512, H=512, U=6, sparsity=1.0, loss="sum", x="uniform3"),
    "C5": dict(B=4096, T=4, D=64, H=64, U=6, sparsity=0.5, loss=None, x="strided"),
}


def n_syn(c):
    return c["B"] * c["T"] * (c["D"] * c["H"] + c["U"] * c["H"] ** 2)


def kernel_flops(c):
    """Algorithmic FLOP per launch of each kernel, per synapse (evaluation):
    forward 10 (z 2, sigmoid 4, two products 2, two sums 2), chain 14 per
    recurrent synapse-unfold (sigmoid recompute 6, sigmoid' 2, delta 4, dv 2),
    8 for the four recurrent parameter sums, 22 per sensory synapse backward.
    Per-neuron, LayerNorm and finalize work is not counted."""
    rec = c["B"] * c["T"] * c["U"] * c["H"] ** 2
    sens = c["B"] * c["T"] * c["D"] * c["H"]
    return {
        "ltc_sens_fwd": 10 * sens,
        "ltc_ode_fwd": 10 * rec,
        "ltc_ode_bwd": 14 * rec,
        "ltc_rec_grad": 8 * rec,
        "ltc_sens_bwd": 22 * sens,
        "ltc_prep": 0,
        "ltc_ln_bwd": 0,
        "ltc_finalize": 0,
    }


def make_inputs(c, device, seed=42):
    import ltc

    torch.manual_seed(seed)
    m = ltc.TrueLiquidTimeConstant(c["D"], c["H"], dt=1.0 / 30.0, ode_unfolds=c["U"],
                                   sparsity=c["sparsity"], sensory_sparsity=c["sparsity"])
    if c["x"] == "uniform3":
        x = torch.rand(c["B"], c["T"], c["D"]) * 6.0 - 3.0
    elif c["x"] == "strided":
        x = torch.randn(c["B"], c["T"], 2 * c["D"])
    else:
        x = torch.randn(c["B"], c["T"], c["D"])
    target = torch.randn(c["B"], c["T"], c["H"]) if c["loss"] == "mse" else None
    m = m.to(device)
    x = x.to(device)
    if c["x"] == "strided":
        x = x[:, :, 0::2]
    if target is not None:
        target = target.to(device)
    return m, x, target


def loss_of(out, target):
    if target is None:
        return out.sum()
    return torch.nn.functional.mse_loss(out, target)


def sync():
    torch.cuda.synchronize()
    if torch.distributed.is_available() and torch.distributed.is_initialized():
        torch.distributed.barrier()


def step(m, x, target):
    out, _ = m(x)
    loss_of(out, target).backward()
    m.zero_grad(set_to_none=True)


def time_split(m, x, target, iters):
    """Median fwd (inside f+b), total and fwd-only (no_grad), torch.cuda.Event timed."""
    fwd, tot, inf = [], [], []
    for _ in range(iters):
        s, f, e = (torch.cuda.Event(enable_timing=True) for _ in range(3))
        s.record()
        out, _ = m(x)
        f.record()
        loss_of(out, target).backward()
        e.record()
        torch.cuda.synchronize()
        m.zero_grad(set_to_none=True)
        fwd.append(s.elapsed_time(f))
        tot.append(s.elapsed_time(e))
    for _ in range(iters):
        s, e = (torch.cuda.Event(enable_timing=True) for _ in range(2))
        s.record()
        with torch.no_grad():
            m(x)
        e.record()
        torch.cuda.synchronize()
        inf.append(s.elapsed_time(e))
    return statistics.median(fwd), statistics.median(tot), statistics.median(inf)


class _GraphStep(torch.nn.Module):
    """Layer forward returning plain tensors, for torch.cuda.make_graphed_callables."""

    def __init__(self, inner):
        super().__init__()
        self.inner = inner

    def forward(self, x):
        out, (h, _) = self.inner(x)
        return out, h


def graphed_step_ms(m, x, target, steps, warmup):
    """Same step with the layer's fwd and bwd captured into HIP graphs (replayed)."""
    g = torch.cuda.make_graphed_callables(_GraphStep(m), (x,))

    def one():
        out, _ = g(x)
        loss_of(out, target).backward()
        m.zero_grad(set_to_none=True)

    for _ in range(warmup):
        one()
    sync()
    t0 = time.perf_counter()
    for _ in range(steps):
        one()
    sync()
    return (time.perf_counter() - t0) * 1e3 / steps


def kernel_times(capi, fn, iters):
    """Mean per-launch duration of each library kernel over `iters` calls of fn."""
    capi.timing_enable(True)
    for _ in range(iters):
        fn()
    torch.cuda.synchronize()
    t = capi.timing_read()
    capi.timing_enable(False)
    return {k: (ms / n, n // iters) for k, (ms, n) in t.items() if n > 0}


def roofline(c, ktimes, traffic=None):
    fl = kernel_flops(c)
    per_step = {k: avg * per for k, (avg, per) in ktimes.items()}
    dom = max(per_step, key=per_step.get)
    avg_ms = ktimes[dom][0]
    achieved = fl[dom] / (avg_ms * 1e-3) / 1e12
    r = {"bound": "valu", "kernel": dom, "achieved": round(achieved, 4),
         "peak": PEAK_FP32_TFLOPS, "unit": "TFLOP/s",
         "frac": round(achieved / PEAK_FP32_TFLOPS, 5),
         "traffic": None if traffic is None else traffic.get(dom),
         "avg_launch_ms": round(avg_ms, 5)}
    return r


R_TRANS = 2.0  # measured on gfx950: v_exp_f32 / v_rcp_f32 cost 2 lane-slots (probes/issue_rate)


def issue_fraction(c, t_ms, which, r=R_TRANS):
    """Mix-aware VALU bound over measured time.

    Minimum lane-slots per synapse: forward 4 FMA-class + 2 transcendental,
    backward 12 + 2; a transcendental costs r lane-slots.
    """
    per = {"fwd": 4 + 2 * r, "fwdbwd": 16 + 4 * r}[which]
    return n_syn(c) * per / LANE_SLOTS_PER_S / (t_ms * 1e-3)


def cpu_baseline(c, budget_s=15.0):
    """CPU oracle (TorchScript restatement of ltc.py:19-106, 249-326) on host cores."""
    from oracle import ltc_oracle as O

    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    torch.manual_seed(42)
    p = O.init_params(c["D"], c["H"], c["sparsity"], c["sparsity"])
    x = torch.randn(c["B"], c["T"], c["D"])
    leaves = {k: v.clone().requires_grad_(k not in ("sparsity_mask", "sensory_sparsity_mask"))
              for k, v in p.items()}

    def one():
        out, _ = O.module_forward(leaves, x, None, dt=1.0 / 30.0, ode_unfolds=c["U"],
                                  scripted=True)
        out.sum().backward()
        for v in leaves.values():
            v.grad = None

    for _ in range(2):
        one()
    times = []
    t_start = time.perf_counter()
    while time.perf_counter() - t_start < budget_s or len(times) < 5:
        t0 = time.perf_counter()
        one()
        times.append(time.perf_counter() - t0)
    med = statistics.median(times)
    cpu = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    cpu = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"value": n_syn(c) / med, "unit": "synapse-updates/s", "cores": torch.get_num_threads(),
            "kind": "port", "ms_per_step": round(med * 1e3, 3),
            "sample": f"{len(times)} fwd+bwd steps of the C1 workload (median), "
                      f"TorchScript oracle, fp32, {threads} threads, {cpu}"}


def load_traffic(workload):
    path = os.path.join(ROOT, "profiles", "traffic.json")
    try:
        with open(path) as f:
            data = json.load(f)
        return data.get(workload)
    except (OSError, ValueError):
        return None


def measure_large(name, c, capi):
    import ltc_cuda

    m, x, target = make_inputs(c, "cuda:0")
    rec = {"shape": {k: c[k] for k in ("B", "T", "D", "H", "U")}, "n_syn": n_syn(c)}
    if c["loss"] is None:
        def fn():
            with torch.no_grad():
                m(x)
    else:
        def fn():
            step(m, x, target)
    for _ in range(2):
        fn()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    iters = 3
    for _ in range(iters):
        fn()
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / iters
    kt = kernel_times(capi, fn, 2)
    rec["ms_per_step"] = round(ms, 4)
    rec["synapse_updates_per_s"] = n_syn(c) / (ms * 1e-3)
    rec["kernels_ms"] = {k: round(v[0], 5) for k, v in kt.items()}
    rec["roofline"] = roofline(c, kt, load_traffic(name))
    which = "fwd" if c["loss"] is None else "fwdbwd"
    ksum = sum(v[0] * v[1] for v in kt.values())
    rec["kernel_ms_sum"] = round(ksum, 4)
    rec["issue_frac_kernels"] = round(issue_fraction(c, ksum, which), 4)
    rec["issue_frac_kernels_r4"] = round(issue_fraction(c, ksum, which, 4.0), 4)
    rec["flop_frac_kernels"] = round(
        n_syn(c) * (10 if which == "fwd" else 32) / (ksum * 1e-3) / 1e12 / PEAK_FP32_TFLOPS, 4)
    del m, x, target
    torch.cuda.empty_cache()
    _ = ltc_cuda
    return rec


COPY_BYTES = 64 << 20


def profile_pass(name):
    """Known-size copy, then a few steps of one config (run under rocprofv3 --pmc)."""
    src = torch.ones(COPY_BYTES // 4, device="cuda:0")
    dst = torch.empty_like(src)
    dst.copy_(src)
    torch.cuda.synchronize()
    c = C1 if name == "C1" else LARGE[name]
    m, x, target = make_inputs(c, "cuda:0")
    for _ in range(3):
        if c["loss"] is None:
            with torch.no_grad():
                m(x)
        else:
            step(m, x, target)
    torch.cuda.synchronize()
    print(f"profile pass {name} done", flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-large", action="store_true")
    ap.add_argument("--profile-pass", choices=["C1", "C2", "C3", "C4", "C5"], default=None,
                    help="for rocprofv3 --pmc: a 64 MiB device copy (calibrates the byte "
                         "counters), then 3 steps of the named config; prints nothing else")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print(f"bench.py: this build measures one GPU only (asked for --gpus {args.gpus}); "
              "multi-GPU runs are not part of it.", file=sys.stderr)
        sys.exit(2)
    rank = int(os.environ.get("RANK", "0"))

    import ltc_cuda

    if not torch.cuda.is_available():
        print("bench.py needs a HIP device", file=sys.stderr)
        sys.exit(1)
    capi = ltc_cuda.require_kernels().capi
    if args.profile_pass:
        profile_pass(args.profile_pass)
        return
    c = C1
    m, x, target = make_inputs(c, "cuda:0")

    for _ in range(args.warmup):
        step(m, x, target)
    sync()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step(m, x, target)
    sync()
    ms = (time.perf_counter() - t0) * 1e3 / args.steps

    fwd_ms, tot_ms, inf_ms = time_split(m, x, target, max(10, args.steps // 2))
    graphed_ms = graphed_step_ms(m, x, target, args.steps, args.warmup)
    kt = kernel_times(capi, lambda: step(m, x, target), max(10, args.steps // 2))
    ksum = sum(v[0] * v[1] for v in kt.values())
    line = {
        "metric": METRIC,
        "value": n_syn(c) / (ms * 1e-3),
        "unit": "synapse-updates/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp32",
        "data": "synthetic (x ~ N(0,1), seeded module init; no dataset)",
        "config": {"workload": "C1: one LTC layer fwd+bwd, B=24 T=8 D=128 H=64, 6 unfolds, "
                               "dt=1/30, sparsity 0.5/0.5, loss=sum(out)",
                   "B": 24, "T": 8, "D": 128, "H": 64, "ode_unfolds": 6,
                   "parallelism": "single GPU"},
        "fwd_ms": round(fwd_ms, 5),
        "bwd_ms": round(tot_ms - fwd_ms, 5),
        "fwd_bwd_event_ms": round(tot_ms, 5),
        "fwd_only_nograd_ms": round(inf_ms, 5),
        "graphed_ms_per_step": round(graphed_ms, 5),
        "graphed_synapse_updates_per_s": n_syn(c) / (graphed_ms * 1e-3),
        "kernels_ms": {k: round(v[0], 5) for k, v in kt.items()},
        "kernel_ms_sum": round(ksum, 5),
        "issue_frac_step": round(issue_fraction(c, ms, "fwdbwd"), 5),
        "issue_frac_kernels": round(issue_fraction(c, ksum, "fwdbwd"), 5),
        "issue_frac_kernels_r4": round(issue_fraction(c, ksum, "fwdbwd", 4.0), 5),
        "roofline": roofline(c, kt, load_traffic("C1")),
        "vs_reference_gtx1080_published": round(REF_GTX1080_MS / ms, 3),
    }
    del m, x, target
    torch.cuda.empty_cache()
    if not args.no_large:
        line["large_configs"] = {name: measure_large(name, cfg, capi)
                                 for name, cfg in LARGE.items()}
    if not args.no_cpu_baseline and rank == 0:
        line["cpu_baseline"] = cpu_baseline(c)
    else:
        line["cpu_baseline"] = None
    if rank == 0:
        print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
