"""Benchmark of the LTC fused ODE-solver path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu-baseline] [--no-large]
    python bench.py --build-probe        (compile issue_rate_probe.hip; no GPU needed)

Headline workload (BASELINE.json metric, config C1's shape run on the GPU):
one TrueLiquidTimeConstant layer, B=24 T=8 D=128 H=64, 6 unfolds, dt=1/30,
Bernoulli(0.5) masks, seeded init (torch.manual_seed(42)), x ~ N(0,1),
loss = sum(out). A step is the module forward (LayerNorm, affine, softplus
transforms, the fused HIP time loop), the loss and loss.backward(), as the
reference's bench_ltc.py:62-96 times it. The headline step is that whole step
captured as one HIP graph and replayed (ltc_cuda.CapturedStep), after a check
that its outputs and gradients equal an eager step's bit for bit; the eager
step is timed beside it.

Printed: one JSON line with the contract fields, plus
  roofline       dominant kernel of the C1 step: algorithmic FLOP per launch
                 over its mean launch time (HIP events the library records on
                 its launch stream), against the 157.3 TFLOP/s FP32 peak;
                 traffic = measured HBM bytes per launch (profiles/traffic.json);
  cpu_baseline   the CPU oracle's TorchScript restatement of the reference
                 path, same module and shapes, timed on this host's cores;
  fwd/bwd split  median fwd (inside fwd+bwd), fwd+bwd and no-grad fwd from
                 torch.cuda.Event, as bench_ltc.py:62-96 and :258-289;
  peak memory and kernel launches, as bench_ltc.py:99-134;
  issue_rate     the probe's measured FMA / exp / rcp issue rates, which set
                 the mix-aware VALU bound (valu_mix_bound_ms, mix_frac_*);
  large_configs  BASELINE configs C2-C5 at full size on the GPU, each with
                 the same split, kernel times, roofline and a CPU baseline
                 (C3/C4: a batch slice, scaled in B; rows are independent).

Only rank 0 at N=1 runs; more GPUs are not part of this build.
"""

from __future__ import annotations

import argparse
import json
import os
import statistics
import subprocess
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "ltc-cuda_amd"))
sys.path.insert(0, ROOT)

import torch  # noqa: E402
import torch.nn.functional as F  # noqa: E402

METRIC = "fwd+bwd ms/step & synapse-updates/s (B24 T8 D128 H64, 6 unfolds)"
PEAK_FP32_TFLOPS = 157.3             # MI355X FP32 vector peak (packed FP32)
PEAK_HBM_GBS = 8000.0
# Published fwd+bwd of the reference CUDA kernels at this config, GTX 1080 (README.md:13).
REF_GTX1080_MS = 12.7
# Issue rates (lane-ops per CU per clock) used when the probe is not built:
# one FMA per lane per clock, transcendentals at half rate.
RATES = {"fma": 64.0, "exp": 32.0, "rcp": 32.0, "cus": 256, "clk_hz": 2.4e9}
PROBE_SRC = os.path.join(ROOT, "issue_rate_probe.hip")
PROBE_BIN = os.path.join(ROOT, "issue_rate_probe")

C1 = dict(B=24, T=8, D=128, H=64, U=6, sparsity=0.5, loss="sum", x="randn")
LARGE = {
    "C2": dict(B=32, T=16, D=128, H=128, U=6, sparsity=0.5, loss="sum", x="randn"),
    "C3": dict(B=256, T=64, D=256, H=256, U=6, sparsity=0.5, loss="mse", x="randn"),
    "C4": dict(B=128, T=32, D=512, H=512, U=6, sparsity=1.0, loss="sum", x="uniform3"),
    "C5": dict(B=4096, T=4, D=64, H=64, U=6, sparsity=0.5, loss=None, x="strided"),
}
# CPU baseline sample per config: batch rows timed (scaled to B when fewer),
# minimum runs and time budget in seconds.
CPU_SAMPLE = {"C1": (24, 5, 10.0), "C2": (32, 5, 5.0), "C3": (4, 3, 4.0), "C4": (4, 3, 4.0),
              "C5": (512, 5, 3.0)}


def n_syn(c, B=None):
    B = c["B"] if B is None else B
    return B * c["T"] * (c["D"] * c["H"] + c["U"] * c["H"] ** 2)


def kernel_flops(c, fused_chain, counts=None):
    """Algorithmic FLOP per launch of each kernel: per sensory synapse, the
    forward counts 10 (z 2, sigmoid 4, two products 2, two sums 2) and the
    backward 22; per recurrent synapse-unfold, the forward 10 and the chain 14
    (sigmoid recompute 6, sigmoid' 2, delta 4, dv 2), plus the 8 of the four
    parameter-gradient sums, which the fused chain does itself (22) and
    rec_grad does otherwise. Without `counts` every synapse counts, masked or
    not (the unit's dense work); with `counts` (syn_counts) synapses count as
    the kernels evaluate them (the compacted kernels skip masked ones).
    Per-neuron, LayerNorm and finalize work is not counted."""
    counts = counts or syn_counts(c)
    rec = c["B"] * c["T"] * c["U"] * c["H"] ** 2
    return {
        "ltc_sens_fwd": 10 * counts["sens_fwd"],
        "ltc_ode_fwd": 10 * counts["rec_fwd"],
        "ltc_ode_bwd": 22 * counts["rec_bwd"] if fused_chain else 14 * counts.get("rec_dv", rec),
        "ltc_rec_grad": 8 * counts["rec_bwd"],
        "ltc_sens_bwd": 22 * counts["sens_bwd"],
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
    return F.mse_loss(out, target)


def sync():
    torch.cuda.synchronize()
    if torch.distributed.is_available() and torch.distributed.is_initialized():
        torch.distributed.barrier()


def step(m, x, target):
    out, _ = m(x)
    loss_of(out, target).backward()
    m.zero_grad(set_to_none=True)


def time_split(m, x, target, iters, train=True):
    """Median fwd (inside fwd+bwd), fwd+bwd, and no-grad fwd, torch.cuda.Event timed
    around whole module calls (bench_ltc.py:62-96)."""
    fwd, tot, inf = [], [], []
    if train:
        for _ in range(iters):
            s, f, e = (torch.cuda.Event(enable_timing=True) for _ in range(3))
            s.record()
            out, _ = m(x)
            f.record()
            loss_of(out, target).backward()
            e.record()
            torch.cuda.synchronize()
            m.zero_grad(set_to_none=True)
            del out
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
    med = statistics.median
    r = {"fwd_nograd_ms": round(med(inf), 5)}
    if train:
        r.update({"fwd_ms": round(med(fwd), 5), "bwd_ms": round(med(tot) - med(fwd), 5),
                  "fwd_bwd_ms": round(med(tot), 5)})
    return r


def kernel_times(capi, fn, iters):
    """Mean per-launch duration (HIP events on the launch stream) and launches per
    call of each library kernel over `iters` calls of fn."""
    capi.timing_enable(True)
    for _ in range(iters):
        fn()
    torch.cuda.synchronize()
    t = capi.timing_read()
    capi.timing_enable(False)
    return {k: (ms / n, n // iters) for k, (ms, n) in t.items() if n > 0}


def _kernel_flops_by_launch(c, plan, ktimes, counts=None):
    fl = kernel_flops(c, bool(plan["fuse"]), counts)
    if ((plan.get("module_row_bwd_fused") or plan.get("module_row128_rec_fused"))
            and "ltc_sens_bwd" not in ktimes):
        # the chain launch also runs the sensory backward (its companions)
        fl["ltc_ode_bwd"] += fl["ltc_sens_bwd"]
    if plan.get("module_row128_rec_fused") and "ltc_rec_grad" not in ktimes:
        # the Hp = 128 chain launch also forms the recurrent parameter-gradient sums
        fl["ltc_ode_bwd"] += fl["ltc_rec_grad"]
    if plan.get("module_sens_in_prep") and "ltc_sens_fwd" not in ktimes:
        # the prep launch forms the sensory sums of the module forward
        fl["ltc_prep"] += fl["ltc_sens_fwd"]
    return fl


def roofline(c, ktimes, plan, traffic=None, counts=None):
    """Dominant kernel of the step against the FP32 peak. `frac` prices the
    unit's dense work (every synapse, masked or not: SURVEY's FLOP_fwd = 10 and
    FLOP_bwd = 22 per synapse); `frac_evaluated` the synapses the kernels
    actually evaluate (the compacted kernels skip masked ones)."""
    fl = _kernel_flops_by_launch(c, plan, ktimes)
    fle = _kernel_flops_by_launch(c, plan, ktimes, counts)
    per_step = {k: avg * per for k, (avg, per) in ktimes.items()}
    dom = max(per_step, key=per_step.get)
    avg_ms = ktimes[dom][0]
    achieved = fl[dom] / (avg_ms * 1e-3) / 1e12
    achieved_e = fle[dom] / (avg_ms * 1e-3) / 1e12
    return {"bound": "valu", "kernel": dom, "achieved": round(achieved, 4),
            "peak": PEAK_FP32_TFLOPS, "unit": "TFLOP/s",
            "frac": round(achieved / PEAK_FP32_TFLOPS, 5),
            "traffic": None if traffic is None else traffic.get(dom),
            "avg_launch_ms": round(avg_ms, 5),
            "flop_per_launch": fl[dom],
            "achieved_evaluated": round(achieved_e, 4),
            "frac_evaluated": round(achieved_e / PEAK_FP32_TFLOPS, 5),
            "flop_per_launch_evaluated": fle[dom]}


# Minimum instruction mix per synapse evaluation: (FMA-class, v_exp_f32, v_rcp_f32).
# Forward: gate argument, 1 + e, two accumulations; backward adds the recompute
# (argument, 1 + e), sigmoid' (2), delta (4), dv (2) and the four parameter sums
# (4) plus one exp and one rcp.
MIX = {"fwd": (4, 1, 1), "fwdbwd": (16, 2, 2)}


def mask_density(m):
    """Fractions of nonzero entries in the recurrent and sensory masks."""
    return (float((m.sparsity_mask != 0).float().mean()),
            float((m.sensory_sparsity_mask != 0).float().mean()))


def syn_counts(c, plan=None, density=(1.0, 1.0)):
    """Synapse evaluations per step as the kernels run them, and the layer's
    active-only count (both masks' densities):
    - sens_fwd: the compacted sensory launch skips masked sensory synapses
      (every sensory launch; the dense form only when the module forward forms
      the sums in its parameter-image launch: plan field module_sens_in_prep);
    - sens_bwd: the module path's sensory backward launch skips masked
      sensory synapses; the companions of the fused row backward (plan field
      module_row_bwd_fused, and module_row128_rec_fused with D <= 128)
      evaluate every one;
    - rec_fwd / rec_dv: the compacted forward and chain skip masked recurrent
      synapses (plan fields cmp_fwd / cmp_bwd);
    - rec_bwd: the parameter-gradient sums, skipped with the chain only when
      the chain forms them itself (fuse); an unfused chain's rec_grad pass
      evaluates every synapse."""
    rho_r, rho_s = density
    sens = c["B"] * c["T"] * c["D"] * c["H"]
    rec = c["B"] * c["T"] * c["U"] * c["H"] ** 2
    plan = plan or {}
    skip_bwd = plan.get("cmp_bwd") and plan.get("fuse")
    sens_cmp = bool(plan) and not plan.get("module_sens_in_prep")
    sens_bwd_dense = (not plan or plan.get("module_row_bwd_fused")
                      or (plan.get("module_row128_rec_fused") and plan.get("Dp", 0) <= 128))
    return {"sens_fwd": sens * (rho_s if sens_cmp else 1.0),
            "sens_bwd": sens * (1.0 if sens_bwd_dense else rho_s),
            "rec_fwd": rec * (rho_r if plan.get("cmp_fwd") else 1.0),
            "rec_bwd": rec * (rho_r if skip_bwd else 1.0),
            "rec_dv": rec * (rho_r if plan.get("cmp_bwd") else 1.0),
            "active": sens * rho_s + rec * rho_r}


def mix_bound_ms(c, which, counts=None, clock_scale=1.0):
    """Mix-aware VALU bound: the minimum mix of every synapse evaluation, each
    instruction class at the issue rate the probe measured on this GPU
    (lane-ops per CU per clock), issued one after another (the probe's synapse
    kernel confirms the classes do not overlap). Without `counts` every synapse
    is priced (the unit's dense work); with `counts` (syn_counts) synapses are
    priced as the kernels evaluate them: the forward part (4, 1, 1) for each
    forward evaluation, the backward's (12, 1, 1) for each backward one.
    `clock_scale` = (engine clock while the probe ran) / (engine clock while
    the priced kernels ran): the probe's rates hold per clock, so a slower
    clock during the kernels stretches the bound by that ratio."""
    def clk(mix):
        f, e, r = mix
        return f / RATES["fma"] + e / RATES["exp"] + r / RATES["rcp"]
    bwd_part = tuple(a - b for a, b in zip(MIX["fwdbwd"], MIX["fwd"]))
    if counts is None:
        work = n_syn(c) * clk(MIX[which])
    elif which == "fwd":
        work = (counts["sens_fwd"] + counts["rec_fwd"]) * clk(MIX["fwd"])
    else:
        work = ((counts["sens_fwd"] + counts["rec_fwd"]) * clk(MIX["fwd"]) +
                (counts["sens_bwd"] + counts["rec_bwd"]) * clk(bwd_part))
    return work / (RATES["cus"] * RATES["clk_hz"]) * 1e3 * clock_scale


def flop_count(c, which, counts):
    """Algorithmic FLOP per step over the evaluated synapses (10 per forward
    evaluation; sensory backward 22, chain 22 with its parameter sums)."""
    fwd = 10 * (counts["sens_fwd"] + counts["rec_fwd"])
    if which == "fwd":
        return fwd
    return fwd + 22 * (counts["sens_bwd"] + counts["rec_bwd"])


# --------------------------------------------------------------------------- clock

class ClockSampler:
    """Engine clock, board power and temperature while a region runs, read
    from the amdgpu sysfs files by a thread (as bench_ltc.py:221-234 polls
    nvidia-smi beside its timings). The clock is the current level of
    pp_dpm_sclk; reading sysfs does not touch the GPU's queues. Samples at or
    below the lowest DPM level (500 MHz on MI355X: idle or deep sleep) are
    counted apart, so that a region with idle gaps reports the clock while
    busy."""

    def __init__(self, period_s=0.004, floor_mhz=500.0):
        import glob
        self.period = period_s
        self.floor = floor_mhz
        cards = sorted(glob.glob("/sys/class/drm/card*/device/pp_dpm_sclk"))
        self.reason = None
        if not cards:
            self.reason = "no readable pp_dpm_sclk"
        elif len(cards) > 1:
            self.reason = f"{len(cards)} cards visible; the bench GPU is ambiguous"
        self.sclk = cards[0] if len(cards) == 1 else None
        dev = os.path.dirname(self.sclk) if self.sclk else None
        self.power = (sorted(glob.glob(os.path.join(dev, "hwmon", "hwmon*", "power1_input")))
                      if dev else [])
        self.temps = (sorted(glob.glob(os.path.join(dev, "hwmon", "hwmon*", "temp*_input")))
                      if dev else [])
        self.mhz, self.watts, self.celsius = [], [], []
        self._stop = None
        self._thread = None

    @staticmethod
    def _read(path):
        try:
            with open(path) as f:
                return f.read()
        except OSError:
            return None

    def _sample(self):
        txt = self._read(self.sclk)
        if txt:
            for line in txt.splitlines():
                if line.rstrip().endswith("*"):
                    num = "".join(ch for ch in line.split(":", 1)[-1] if ch.isdigit() or ch == ".")
                    if num:
                        self.mhz.append(float(num))
        if self.power:
            v = self._read(self.power[0])
            if v and v.strip().isdigit():
                self.watts.append(int(v) / 1e6)
        for tp in self.temps:
            v = self._read(tp)
            if v and v.strip().lstrip("-").isdigit():
                self.celsius.append(int(v) / 1e3)

    def _run(self):
        while not self._stop.is_set():
            self._sample()
            self._stop.wait(self.period)

    def __enter__(self):
        import threading
        if self.sclk is not None:
            self._stop = threading.Event()
            self._thread = threading.Thread(target=self._run, daemon=True)
            self._thread.start()
        return self

    def __exit__(self, *exc):
        if self._thread is not None:
            self._stop.set()
            self._thread.join()
        return False

    def stats(self):
        if self.sclk is None:
            return {"source": None, "reason": self.reason}
        busy = sorted(m for m in self.mhz if m > self.floor)
        rec = {"source": self.sclk, "samples": len(self.mhz), "busy_samples": len(busy),
               "mhz_busy_median": statistics.median(busy) if busy else None,
               "mhz_busy_min": busy[0] if busy else None,
               "mhz_busy_max": busy[-1] if busy else None,
               "power_w_median": round(statistics.median(self.watts), 1) if self.watts else None,
               "temp_c_max": max(self.celsius) if self.celsius else None}
        return rec


def clock_window(fn, seconds):
    """Runs fn back to back for about `seconds` under a ClockSampler; returns
    the clock statistics and the mean ms per call over the window."""
    torch.cuda.synchronize()
    n = 0
    with ClockSampler() as cs:
        t0 = time.perf_counter()
        while time.perf_counter() - t0 < seconds:
            fn()
            n += 1
            if n % 8 == 0:
                torch.cuda.synchronize()
        torch.cuda.synchronize()
        ms = (time.perf_counter() - t0) * 1e3 / n
    return {"calls": n, "ms_per_call": round(ms, 5), **cs.stats()}


def clock_scale(probe, window):
    """(the clock the bound is priced at, RATES clk_hz) / (engine clock in the
    window), or None when the window's clock is unknown. The probe's rates
    are per engine clock (it measures the clock each kernel ran at), so the
    bound at the window's clock is the bound at clk_hz times this ratio."""
    wm = (window or {}).get("mhz_busy_median")
    if not wm or not probe or "clock_mhz_measured" not in probe:
        return None
    return RATES["clk_hz"] / 1e6 / wm


# --------------------------------------------------------------------------- probe

def build_probe() -> str:
    """hipcc the issue-rate probe into ./issue_rate_probe (no GPU needed)."""
    import shutil
    hipcc = os.environ.get("HIPCC") or "/opt/rocm/bin/hipcc"
    if not os.path.isfile(hipcc):
        hipcc = shutil.which("hipcc") or hipcc
    cmd = [hipcc, "--offload-arch=gfx950", "-O3", "-std=c++17",
           "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
           "-Wno-unused-command-line-argument", "-o", PROBE_BIN + ".tmp", PROBE_SRC]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError("hipcc failed on issue_rate_probe.hip:\n" + proc.stderr)
    os.replace(PROBE_BIN + ".tmp", PROBE_BIN)
    return PROBE_BIN


def run_probe():
    """Run the probe as a child process (before this process touches the GPU);
    its rates replace the defaults in RATES."""
    if not os.path.isfile(PROBE_BIN):
        return {"source": "defaults (probe not built)", **RATES}
    try:
        proc = subprocess.run([PROBE_BIN], capture_output=True, text=True, timeout=120)
        rec = json.loads(proc.stdout.strip().splitlines()[-1])
    except (OSError, ValueError, IndexError, subprocess.TimeoutExpired) as exc:
        return {"source": f"defaults (probe failed: {exc})", **RATES}
    if "error" in rec:
        return {"source": f"defaults (probe: {rec['error']})", **RATES}
    RATES.update(fma=rec["fma_per_cu_clk"], exp=rec["exp_per_cu_clk"],
                 rcp=rec["rcp_per_cu_clk"], cus=rec["cus"], clk_hz=rec["clock_mhz"] * 1e6)
    rec["source"] = "issue_rate_probe (measured in this run)"
    return rec


# --------------------------------------------------------------------------- CPU baseline

def _cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(name, c):
    """The oracle's TorchScript restatement of the reference path (ltc.py:19-106,
    249-326) on this host's cores, fp32: fwd+bwd (or fwd only for C5) on a batch
    slice of the config, scaled to the full batch (rows are independent)."""
    from oracle import ltc_oracle as O

    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    bs, min_runs, budget = CPU_SAMPLE[name]
    bs = min(bs, c["B"])
    torch.manual_seed(42)
    p = O.init_params(c["D"], c["H"], c["sparsity"], c["sparsity"])
    x = torch.randn(bs, c["T"], 2 * c["D"] if c["x"] == "strided" else c["D"])
    if c["x"] == "strided":
        x = x[:, :, 0::2]
    elif c["x"] == "uniform3":
        x = x.uniform_(-3.0, 3.0)
    target = torch.randn(bs, c["T"], c["H"]) if c["loss"] == "mse" else None
    leaves = {k: v.clone().requires_grad_(k not in ("sparsity_mask", "sensory_sparsity_mask"))
              for k, v in p.items()}
    train = c["loss"] is not None

    def one():
        if not train:
            with torch.no_grad():
                O.module_forward(leaves, x, None, dt=1.0 / 30.0, ode_unfolds=c["U"], scripted=True)
            return
        out, _ = O.module_forward(leaves, x, None, dt=1.0 / 30.0, ode_unfolds=c["U"],
                                  scripted=True)
        loss_of(out, target).backward()
        for v in leaves.values():
            v.grad = None

    for _ in range(2):
        one()
    times = []
    t_start = time.perf_counter()
    while time.perf_counter() - t_start < budget or len(times) < min_runs:
        t0 = time.perf_counter()
        one()
        times.append(time.perf_counter() - t0)
    med = statistics.median(times)
    scale = c["B"] / bs
    what = "fwd+bwd" if train else "no-grad fwd"
    return {"value": n_syn(c) / (med * scale), "unit": "synapse-updates/s",
            "cores": torch.get_num_threads(), "kind": "port",
            "ms_per_step": round(med * scale * 1e3, 3),
            "scaled": scale != 1.0,
            "sample": f"{len(times)} {what} steps (median) of {name} on {bs} of its {c['B']} "
                      f"batch rows{', scaled x%g in B' % scale if scale != 1.0 else ''}; "
                      f"TorchScript oracle, fp32, {threads} threads, {_cpu_model()}"}


# Rows of each config whose output and input gradient the oracle checks
# (every row where the oracle finishes in seconds).
AGREE_ROWS = {"C1": None, "C2": None, "C3": (0, 255), "C4": (0, 127), "C5": (0, 1, 4095)}


def oracle_agreement(name, c):
    """The GPU path against the float64 oracle on the bench's own inputs, outside
    every timed region, as bench_ltc.py:137-218 checks its CUDA path against
    TorchScript before reporting. Rows are independent, so the output and
    dL/dx of sampled rows are checked in a full-batch run; with every row
    sampled, so are all parameter gradients. Loss sum(out); the bars are the
    reference's (forward max-abs 1e-3; gradients allclose rtol 5e-2 /
    atol 1e-2), plus max error <= 2e-3 of each gradient's largest entry."""
    from oracle import ltc_oracle as O

    m, x, _ = make_inputs(c, "cuda:0")
    train = c["loss"] is not None
    rows = AGREE_ROWS[name]
    idx = list(range(c["B"])) if rows is None else list(rows)
    # (C5 reads its strided view in place, as the timed forward does)
    xg = x.detach().requires_grad_(True) if train else x
    if train:
        out, _ = m(xg)
        out.sum().backward()
    else:
        with torch.no_grad():
            out, _ = m(xg)
    torch.cuda.synchronize()
    leaves = {k: v.detach().cpu().double().clone() for k, v in m.state_dict().items()}
    pnames = [n for n, _ in m.named_parameters()]
    for k in pnames:
        leaves[k].requires_grad_(train)
    xr = x.detach()[idx].cpu().double().requires_grad_(train)
    if train:
        r_out, _ = O.module_forward(leaves, xr, None, dt=m.dt, ode_unfolds=m.ode_unfolds,
                                    epsilon=m.epsilon)
        r_out.sum().backward()
    else:
        with torch.no_grad():
            r_out, _ = O.module_forward(leaves, xr, None, dt=m.dt, ode_unfolds=m.ode_unfolds,
                                        epsilon=m.epsilon)
    got = out.detach()[idx].cpu().double()
    rec = {"rows": "all" if rows is None else idx,
           "out_max_abs": (got - r_out.detach()).abs().max().item()}
    ok = rec["out_max_abs"] <= 1e-3

    def grad_err(a, r):
        err = (a - r).abs().max().item()
        passed = (torch.allclose(a, r, rtol=5e-2, atol=1e-2) and
                  err <= 2e-3 * r.abs().max().item() + 1e-6)
        return err / max(r.abs().max().item(), 1e-30), passed

    if train:
        rel, passed = grad_err(xg.grad[idx].cpu().double(), xr.grad)
        rec["dx_max_rel"] = rel
        ok = ok and passed
        if rows is None:
            worst = 0.0
            for n, prm in m.named_parameters():
                rel, passed = grad_err(prm.grad.cpu().double(), leaves[n].grad)
                worst = max(worst, rel)
                ok = ok and passed
            rec["param_grads_max_rel"] = worst
    rec["pass"] = bool(ok)
    rec["loss"] = "sum(out)" if train else "none (forward only)"
    del m, x, xg, out
    torch.cuda.empty_cache()
    return rec


# --------------------------------------------------------------------------- memory, launches

def peak_memory_mb(m, x, target, train):
    """Peak allocated GPU memory of one step (bench_ltc.py:118-134)."""
    torch.cuda.synchronize()
    torch.cuda.reset_peak_memory_stats()
    base = torch.cuda.memory_allocated()
    if train:
        out, _ = m(x)
        loss_of(out, target).backward()
        del out
        m.zero_grad(set_to_none=True)
    else:
        with torch.no_grad():
            m(x)
    torch.cuda.synchronize()
    peak = torch.cuda.max_memory_allocated()
    return {"peak_mb": round(peak / 2 ** 20, 3), "peak_above_inputs_mb": round((peak - base) / 2 ** 20, 3)}


def kernel_launches(fn):
    """Device kernels of one call of fn, counted with torch.profiler as
    bench_ltc.py:99-115 counts them."""
    try:
        from torch.profiler import ProfilerActivity, profile
        with profile(activities=[ProfilerActivity.CPU, ProfilerActivity.CUDA]) as prof:
            fn()
            torch.cuda.synchronize()
        n = 0
        for evt in prof.events():
            if evt.device_type == torch.autograd.DeviceType.CUDA:
                n += 1
        return n
    except Exception as exc:  # the profiler is optional here
        return f"unavailable: {exc}"


# --------------------------------------------------------------------------- configs

def measure_config(name, c, capi, cpu, probe=None):
    import ltc_cuda

    m, x, target = make_inputs(c, "cuda:0")
    train = c["loss"] is not None
    plan = capi.plan(c["B"], c["T"], c["D"], c["H"], c["U"])
    dens = mask_density(m)
    counts = syn_counts(c, plan, dens)
    rec = {"shape": {k: c[k] for k in ("B", "T", "D", "H", "U")}, "n_syn": n_syn(c),
           "loss": c["loss"], "x": c["x"]}
    rec.update(sparsity_record(plan, dens, counts))

    if train:
        def fn():
            step(m, x, target)
    else:
        def fn():
            with torch.no_grad():
                m(x)
    for _ in range(2):
        fn()
    torch.cuda.synchronize()
    # about 50 ms of timed steps (5 to 200), so that a short step is not one
    # host hiccup away from twice its time
    t0 = time.perf_counter()
    fn()
    torch.cuda.synchronize()
    one_ms = (time.perf_counter() - t0) * 1e3
    iters = max(5, min(200, int(50.0 / max(one_ms, 1e-3))))
    t0 = time.perf_counter()
    for _ in range(iters):
        fn()
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / iters
    rec["ms_per_step"] = round(ms, 4)
    rec["synapse_updates_per_s"] = n_syn(c) / (ms * 1e-3)
    rec["active_synapse_updates_per_s"] = counts["active"] / (ms * 1e-3)
    rec.update(time_split(m, x, target, 5, train=train))
    kt = kernel_times(capi, fn, 2)
    rec["kernels_ms"] = {k: round(v[0], 5) for k, v in kt.items()}
    rec["launches_per_step_library"] = sum(v[1] for v in kt.values())
    rec["roofline"] = roofline(c, kt, plan, load_traffic(name), counts)
    which = "fwdbwd" if train else "fwd"
    ksum = sum(v[0] * v[1] for v in kt.values())
    rec["kernel_ms_sum"] = round(ksum, 4)
    rec["valu_mix_bound_ms"] = round(mix_bound_ms(c, which, counts), 4)
    rec["mix_frac_kernels"] = round(mix_bound_ms(c, which, counts) / ksum, 4)
    rec["flop_frac_kernels"] = round(
        flop_count(c, which, counts) / (ksum * 1e-3) / 1e12 / PEAK_FP32_TFLOPS, 4)
    # the same against the dense, mask-inclusive work of the unit (every
    # synapse evaluated, as the reference does): what skipping buys
    rec["valu_mix_bound_dense_ms"] = round(mix_bound_ms(c, which), 4)
    rec["mix_frac_kernels_dense"] = round(mix_bound_ms(c, which) / ksum, 4)
    # the engine clock while the config's steps run back to back, and the
    # bound priced at that clock
    win = clock_window(fn, 1.0 if name in ("C3", "C4") else 0.5)
    rec["clock_window"] = win
    scale = clock_scale(probe, win)
    if scale is not None:
        rec["valu_mix_bound_at_clock_ms"] = round(mix_bound_ms(c, which, counts, scale), 4)
        rec["mix_frac_kernels_at_clock"] = round(mix_bound_ms(c, which, counts, scale) / ksum, 4)
    rec["memory"] = peak_memory_mb(m, x, target, train)
    del m, x, target
    torch.cuda.empty_cache()
    if cpu:
        rec["cpu_baseline"] = cpu_baseline(name, c)
        gpu_ms = rec["fwd_bwd_ms"] if train else rec["fwd_nograd_ms"]
        rec["gpu_vs_cpu"] = round(rec["cpu_baseline"]["ms_per_step"] / gpu_ms, 1)
        rec["oracle_agreement"] = oracle_agreement(name, c)
    _ = ltc_cuda
    return rec


def sparsity_record(plan, dens, counts):
    """What the kernels skip, and the active-only count beside the dense one."""
    return {"mask_density": {"recurrent": round(dens[0], 5), "sensory": round(dens[1], 5)},
            "skips_masked_recurrent": {"forward": bool(plan.get("cmp_fwd")),
                                       "chain": bool(plan.get("cmp_bwd"))},
            "n_syn_active": int(round(counts["active"])),
            "n_syn_evaluated_fwd": int(round(counts["sens_fwd"] + counts["rec_fwd"])),
            "n_syn_evaluated_bwd": int(round(counts["sens_bwd"] + counts["rec_bwd"]))}


def load_traffic(workload):
    path = os.path.join(ROOT, "profiles", "traffic.json")
    try:
        with open(path) as f:
            data = json.load(f)
        return data.get(workload)
    except (OSError, ValueError):
        return None


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


def graphed_c1(m, x, target, steps, warmup):
    """The C1 step captured whole (forward, loss, backward) and replayed; returns
    (ms per replayed step, bitwise equal to an eager step)."""
    import ltc_cuda

    def eager_result():
        m.zero_grad(set_to_none=True)
        out, _ = m(x)
        loss_of(out, target).backward()
        res = [out.detach().clone()] + [p.grad.detach().clone() for p in m.parameters()]
        m.zero_grad(set_to_none=True)
        return res

    ref = eager_result()
    torch.cuda.synchronize()
    cap = ltc_cuda.CapturedStep(m, (x,), lambda o: loss_of(o[0], target))
    cap.replay()
    torch.cuda.synchronize()
    got = [cap.outputs[0]] + [p.grad for p in m.parameters()]
    equal = len(got) == len(ref) and all(torch.equal(a, b) for a, b in zip(got, ref))
    for _ in range(warmup):
        cap.replay()
    sync()
    t0 = time.perf_counter()
    for _ in range(steps):
        cap.replay()
    sync()
    ms = (time.perf_counter() - t0) * 1e3 / steps
    del cap
    m.zero_grad(set_to_none=True)
    return ms, equal


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-large", action="store_true")
    ap.add_argument("--no-graph", action="store_true",
                    help="report the eager step as the headline (no HIP-graph capture)")
    ap.add_argument("--build-probe", action="store_true",
                    help="compile issue_rate_probe.hip into ./issue_rate_probe and exit")
    ap.add_argument("--profile-pass", choices=["C1", "C2", "C3", "C4", "C5"], default=None,
                    help="for rocprofv3 --pmc: a 64 MiB device copy (calibrates the byte "
                         "counters), then 3 steps of the named config; prints nothing else")
    args = ap.parse_args()
    if args.build_probe:
        print(build_probe())
        return
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print(f"bench.py: this build measures one GPU only (asked for --gpus {args.gpus}); "
              "multi-GPU runs are not part of it.", file=sys.stderr)
        sys.exit(2)
    rank = int(os.environ.get("RANK", "0"))

    probe = None if args.profile_pass else run_probe()  # before this process uses the GPU

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
    plan = capi.plan(c["B"], c["T"], c["D"], c["H"], c["U"])
    dens = mask_density(m)
    counts = syn_counts(c, plan, dens)

    for _ in range(max(args.warmup, 200)):
        step(m, x, target)
    sync()
    # the eager step is host-bound at this size: time enough of them (about
    # 0.3 s) that one host hiccup does not move the mean
    n_eager = max(args.steps, 2000)
    t0 = time.perf_counter()
    for _ in range(n_eager):
        step(m, x, target)
    sync()
    eager_ms = (time.perf_counter() - t0) * 1e3 / n_eager

    split = time_split(m, x, target, max(10, args.steps // 2))
    kt = kernel_times(capi, lambda: step(m, x, target), max(10, args.steps // 2))
    ksum = sum(v[0] * v[1] for v in kt.values())
    mem = peak_memory_mb(m, x, torch.randn(c["B"], c["T"], c["H"], device="cuda:0"), True)
    with torch.no_grad():
        launches_fwd = kernel_launches(lambda: m(x))
    launches_step = kernel_launches(lambda: step(m, x, target))
    win = clock_window(lambda: step(m, x, target), 0.5)
    scale = clock_scale(probe, win)
    graph_ms, graph_equal = (None, None)
    if not args.no_graph:
        graph_ms, graph_equal = graphed_c1(m, x, target, args.steps, args.warmup)
    use_graph = graph_ms is not None and graph_equal
    ms = graph_ms if use_graph else eager_ms
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
                   "parallelism": "single GPU",
                   "step": "whole step replayed as one HIP graph" if use_graph
                           else "eager module forward + loss.backward()"},
        "active_synapse_updates_per_s": counts["active"] / (ms * 1e-3),
        **sparsity_record(plan, dens, counts),
        "eager_ms_per_step": round(eager_ms, 5),
        "eager_synapse_updates_per_s": n_syn(c) / (eager_ms * 1e-3),
        "graphed_ms_per_step": None if graph_ms is None else round(graph_ms, 5),
        "graph_replay_bitwise_equal_to_eager": graph_equal,
        **split,
        "kernels_ms": {k: round(v[0], 5) for k, v in kt.items()},
        "kernel_ms_sum": round(ksum, 5),
        "launches": {"library_per_step": sum(v[1] for v in kt.values()),
                     "device_kernels_fwd_nograd": launches_fwd,
                     "device_kernels_step": launches_step},
        "memory_fwd_bwd_mse": mem,
        "issue_rate": probe,
        "valu_mix_bound_ms": round(mix_bound_ms(c, "fwdbwd", counts), 5),
        "mix_frac_step": round(mix_bound_ms(c, "fwdbwd", counts) / ms, 5),
        "clock_window": win,
        "mix_frac_step_at_clock": (None if scale is None else
                                   round(mix_bound_ms(c, "fwdbwd", counts, scale) / ms, 5)),
        "roofline": roofline(c, kt, plan, load_traffic("C1"), counts),
        "vs_reference_gtx1080_published": round(REF_GTX1080_MS / ms, 3),
    }
    del m, x, target
    torch.cuda.empty_cache()
    cpu = not args.no_cpu_baseline and rank == 0
    if not args.no_large:
        line["large_configs"] = {}
        for name, cfg in LARGE.items():
            line["large_configs"][name] = measure_config(name, cfg, capi, cpu, probe)
            print(f"bench: {name} done", file=sys.stderr, flush=True)
    line["cpu_baseline"] = cpu_baseline("C1", c) if cpu else None
    if cpu:
        line["oracle_agreement"] = oracle_agreement("C1", c)
    if rank == 0:
        print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
