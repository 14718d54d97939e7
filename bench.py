#!/usr/bin/env python3
"""Benchmark of the KLA scan hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload NAME]

A step is one forward + backward pass of the Moebius precision scan and of the
affine information scan over one batch of synthetic inputs already resident in
HBM (BASELINE metric "KLA scan fwd+bwd tokens/s + achieved HBM GB/s, B=8 T=4096
fp32, 1 GPU"; workload: Moebius + affine, batch 8, 4096 steps, 2048 lanes =
heads * d_state, fp32). Prints one JSON line with tokens/s (value), the achieved
HBM bandwidth, a roofline entry for the dominant kernel (HIP-event timing on the
launch stream) and a CPU baseline: the reference's pure-PyTorch CPU algorithm
(restated in oracle/torch_ref.py) timed on a bounded sample on this host.

Inputs are drawn on the CPU with torch.Generator(seed 0) in a fixed order and
copied to the GPU, so the CPU and GPU sides see the same bytes.

After the headline the same JSON line carries ``configs``: every other BASELINE
config (``--configs``, default all), each with its GPU time and rate, a roofline
for what bounds it and a bounded CPU baseline of the reference's algorithm on
this host: c1 the KLALayer(512) forward, c3 the standalone affine scan at
(8, 8192, 2048) fp32 and bf16 I/O, c4 the KLALayer(1024) training step (its fused
scan kernels timed inside the step and priced on VALU issue), c5 the
SequenceModel prefill (fp32 matrix flops) and one-token decode (weight bytes).

``--layer c1|c4|c5`` measures one layer-level BASELINE config instead of the
headline (its own JSON line; ``--backend`` picks the kla backend): c1 is a
KLALayer(512, d_state=16) forward on x (2, 1024, 512), timed on the GPU and, on
backend "torch", on this host's CPU; c4 is a
KLALayer(1024, d_state=16) training step on x (4, 4096, 1024) under bf16
autocast, loss = mean(out^2); c5 is SequenceModel(vocab 50304, d_model 512,
6 layers) stateful prefill of (16, 2048) random ids, then 256 one-token decode
steps (prefill tokens/s and decode ms/token).

``--layer scan --shape B,L,M,S`` times kla_scan alone (fwd + bwd) on ``--backend``
(the d_state > 64 fused kernels against the composed path).

``--workload affine_b8_t8192_l2048[_bf16]`` is BASELINE config 3: the standalone
affine scan alone, fp32 or bf16 I/O.

``--only KERNEL`` runs just one kernel K times (for rocprofv3 counter runs);
``--only copy`` runs a 1 GiB device-to-device copy, the calibration kernel for
the FETCH_SIZE / WRITE_SIZE counters; ``--only all`` runs the copy and then every
scan kernel, so one counter pass covers them all.
"""

from __future__ import annotations

import argparse
import gc
import json
import os
import platform
import statistics
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(REPO, "kalman-linear-attention_amd"))

import torch  # noqa: E402
import torch.nn.functional as F  # noqa: E402

METRIC = "KLA scan fwd+bwd tokens/s + achieved HBM GB/s, B=8 T=4096 fp32, 1 GPU"
PEAK_HBM_GBPS = 8000.0

WORKLOADS = {
    # name: (batch, steps, lanes, affine I/O dtype, scans in a step)
    "mobius_affine_b8_t4096_l2048": (8, 4096, 2048, torch.float32, "mobius+affine"),
    "mobius_affine_b8_t8192_l2048": (8, 8192, 2048, torch.float32, "mobius+affine"),
    "mobius_affine_b8_t4096_l2048_bf16affine": (8, 4096, 2048, torch.bfloat16, "mobius+affine"),
    "small_b2_t1024_l512": (2, 1024, 512, torch.float32, "mobius+affine"),
    # the standalone affine scan, fp32 and bf16 I/O.
    "affine_b8_t8192_l2048": (8, 8192, 2048, torch.float32, "affine"),
    "affine_b8_t8192_l2048_bf16": (8, 8192, 2048, torch.bfloat16, "affine"),
}
DEFAULT_WORKLOAD = "mobius_affine_b8_t4096_l2048"

# Compulsory HBM bytes per element of the reference's algorithm (each input read
# once, each output written once). Moebius with D == 1: fwd reads A, B, C and
# writes lam; bwd reads dlam, A, B, C, lam and writes dA, dB, dC. Affine: fwd
# reads g, u and writes h; bwd reads dh, g, h and writes dg, du. [batch, lanes]
# state tensors are excluded. The roofline's `achieved` is priced on these.
def alg_bytes_per_elem(kernel: str, affine_dtype: torch.dtype) -> int:
    e = 2 if affine_dtype == torch.bfloat16 else 4
    return {"mobius_fwd": 16, "mobius_bwd": 32, "affine_fwd": 3 * e, "affine_bwd": 5 * e}[kernel]


# Bytes per element the kernels themselves must move: the same, except that the
# Moebius backward reads the saved lam once per thread's run of steps (24, the
# backward tile's steps per wave) and recomputes the rest from A, B, C (so
# 28 + 4/24 instead of 32).
MOBIUS_BWD_STEPS = 24


def kernel_bytes_per_elem(kernel: str, affine_dtype: torch.dtype) -> float:
    if kernel == "mobius_bwd":
        return 28 + 4 / MOBIUS_BWD_STEPS
    return float(alg_bytes_per_elem(kernel, affine_dtype))


# ------------------------------------------------------------------ inputs


def mobius_inputs(batch, steps, lanes, seed=0):
    """A = exp(-softplus(z1)), B = softplus(z2), C = softplus(z3), D = 1 (implicit),
    lam0 = softplus(N(0,1)), dlam ~ N(0,1); z ~ N(0,1). CPU tensors."""
    g = torch.Generator().manual_seed(seed)
    z1 = torch.randn(batch, steps, lanes, generator=g)
    z2 = torch.randn(batch, steps, lanes, generator=g)
    z3 = torch.randn(batch, steps, lanes, generator=g)
    A = torch.exp(-F.softplus(z1))
    B = F.softplus(z2)
    C = F.softplus(z3)
    lam0 = F.softplus(torch.randn(batch, lanes, generator=g))
    dlam = torch.randn(batch, steps, lanes, generator=g)
    return A, B, C, lam0, dlam


def affine_inputs(batch, steps, lanes, seed=1, dtype=torch.float32):
    """g = sigmoid(N(0,1)), u ~ N(0,1), h0 = 0, dh ~ N(0,1); bf16 by round-to-nearest-even."""
    gen = torch.Generator().manual_seed(seed)
    g = torch.sigmoid(torch.randn(batch, steps, lanes, generator=gen))
    u = torch.randn(batch, steps, lanes, generator=gen)
    dh = torch.randn(batch, steps, lanes, generator=gen)
    return g.to(dtype), u.to(dtype), dh.to(dtype)


# --------------------------------------------------------------- CPU baseline


def cpu_model_name() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


def _median_time(fn, budget_s: float, max_reps: int = 60):
    """Warm up once, then repeat ``fn`` to fill about ``budget_s`` seconds; (median s, reps)."""
    t0 = time.perf_counter()
    fn()
    reps = int(min(max_reps, max(3, budget_s / max(time.perf_counter() - t0, 1e-3))))
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return statistics.median(times), reps


def cpu_baseline(lanes_full: int, ops: str = "mobius+affine", budget_s: float = 15.0,
                 seq_budget_s: float = 5.0) -> dict:
    """The reference's pure-PyTorch CPU scan (oracle.torch_ref: doubling scans of the
    trace-normalised Moebius combine and the affine combine, backward by autograd),
    fp32, on a bounded sample: batch 1, 4096 steps, all lanes; repeated to fill
    about ``budget_s`` seconds, median reported. The reference widens bf16 to fp32
    (kla_ops.py:126-137), so the CPU side is fp32 for every workload.

    Beside it, ``sequential``: the step-by-step form (oracle.scans, the per-step
    recurrences of lane_mobius_scan.metal / tiled_mobius_scan.py's backward, the
    shape of kla_scan_reference) in numpy fp32 on one thread, same sample."""
    import numpy as np

    from oracle import scans as oscans
    from oracle import torch_ref

    with_mobius = ops == "mobius+affine"
    sb, st, sl = 1, 4096, lanes_full
    A, B, C, lam0, dlam = mobius_inputs(sb, st, sl, seed=0)
    g, u, dh = affine_inputs(sb, st, sl, seed=1)

    def one():
        if with_mobius:
            Ar, Br, Cr, lr = (t.clone().requires_grad_(True) for t in (A, B, C, lam0))
            lam = torch_ref.mobius_scan(Ar, Br, Cr, None, lr)
            torch.autograd.backward(lam, dlam)
        gr, ur = g.clone().requires_grad_(True), u.clone().requires_grad_(True)
        h = torch_ref.affine_scan(gr, ur)
        torch.autograd.backward(h, dh)

    med, reps = _median_time(one, budget_s)

    na = [t.numpy() for t in (A, B, C, lam0, dlam, g, u, dh)]

    def one_seq():
        An, Bn, Cn, l0, dl, gn, un, dhn = na
        if with_mobius:
            lam = oscans.mobius_scan_fwd(An, Bn, Cn, None, l0, dtype=np.float32)
            oscans.mobius_scan_bwd(dl, An, Bn, Cn, None, l0, lam, dtype=np.float32)
        h = oscans.affine_scan_fwd(gn, un, dtype=np.float32)
        oscans.affine_scan_bwd(dhn, gn, h, dtype=np.float32)

    seq_med, seq_reps = _median_time(one_seq, seq_budget_s)
    full_width_tokens = sb * st * sl / lanes_full
    what = "Moebius+affine" if with_mobius else "affine"
    return {
        "value": full_width_tokens / med,
        "unit": "tokens/s",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": (f"oracle/torch_ref (reference kla_ops.py doubling scans, autograd) {what} fwd+bwd fp32 "
                   f"on batch {sb} x {st} steps x {sl} of {lanes_full} lanes; median of {reps} reps = "
                   f"{med:.3f} s"),
        "sequential": {"value": full_width_tokens / seq_med, "unit": "tokens/s", "cores": 1, "kind": "port",
                       "sample": (f"oracle/scans per-step recurrences, numpy fp32, {what} fwd+bwd, same sample; "
                                  f"median of {seq_reps} reps = {seq_med:.3f} s")},
        "host": {"cpu": cpu_model_name(), "affinity_cores": len(os.sched_getaffinity(0)),
                 "torch_threads": torch.get_num_threads()},
    }


# ----------------------------------------------------------------- GPU side


def build_step(batch, steps, lanes, adt, device, ops="mobius+affine", streams=1):
    """(step, kernels): one fwd + bwd of the workload's scans, and each kernel alone.
    With ``streams`` 2 the affine chain runs on a second stream beside the Moebius
    chain (the two scans are independent); the same kernels, overlapped."""
    from kla.ops.hip import scans as hs

    if ops == "mobius+affine":
        A, B, C, lam0, dlam = (t.to(device) for t in mobius_inputs(batch, steps, lanes))
    g, u, dh = (t.to(device) for t in affine_inputs(batch, steps, lanes, dtype=adt))
    state = {}

    def mobius_fwd():
        state["lam"] = hs._mobius_scan_op(A, B, C, None, lam0)

    def mobius_bwd():
        state["dm"] = hs._mobius_scan_bwd_op(dlam, A, B, C, None, lam0, state["lam"])

    def affine_fwd():
        state["h"] = hs._affine_scan_op(g, u, None)

    def affine_bwd():
        state["da"] = hs._affine_scan_bwd_op(dh, g, state["h"], None)

    kernels = {"mobius_fwd": mobius_fwd, "mobius_bwd": mobius_bwd, "affine_fwd": affine_fwd,
               "affine_bwd": affine_bwd}
    if ops == "affine":
        del kernels["mobius_fwd"], kernels["mobius_bwd"]
    order = list(kernels.values())

    def step():
        for fn in order:
            fn()

    if streams == 2 and ops == "mobius+affine":
        main = torch.cuda.current_stream(device)
        side = torch.cuda.Stream(device)

        def step():  # noqa: F811
            side.wait_stream(main)
            mobius_fwd()
            mobius_bwd()
            with torch.cuda.stream(side):
                affine_fwd()
                affine_bwd()
            main.wait_stream(side)

    return step, kernels


def time_kernels_in_step(kernels, steps, stream):
    """Average duration of each kernel where it runs in the step: ``steps`` more steps,
    each kernel bracketed by HIP events on the launch stream.

    Timing a kernel inside the step, not repeated on its own, matters here: run
    back to back on the same inputs a backward scan is 6-12% faster than after
    the other kernels of the step (the caches and the DRAM write queue hold what
    the previous kernel left behind)."""
    ev = {name: [] for name in kernels}
    for _ in range(steps):
        for name, fn in kernels.items():
            s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            s.record(stream)
            fn()
            e.record(stream)
            ev[name].append((s, e))
    torch.cuda.synchronize()
    return {name: statistics.mean(s.elapsed_time(e) for s, e in pairs) for name, pairs in ev.items()}


class _NoGC:
    """Python's cyclic garbage collector off for the warmup and the timed region
    (collected just before the warmup).

    A generation-2 collection is a host-side pause of tens of milliseconds (81 ms
    measured in the C4 step's process) during which no kernel is launched and the
    GPU runs dry; the step's kernels are the same either way. The collection comes
    before the warmup, not between the warmup's synchronize and the first timed
    launch: after such a pause the steps that follow run slower while the GPU
    comes back from idle (C1's forward over 20 steps: 0.236-0.247 ms with no
    gap, 0.25-0.27 after a 50 ms sleep, 0.268-0.276 after gc.collect())."""

    def __enter__(self):
        gc.collect()
        self.was = gc.isenabled()
        gc.disable()

    def __exit__(self, *exc):
        if self.was:
            gc.enable()


def _timed(fn, steps, warmup, stream):
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    with _NoGC():
        for _ in range(warmup):
            fn()
        torch.cuda.synchronize()
        start.record(stream)
        for _ in range(steps):
            fn()
        end.record(stream)
        torch.cuda.synchronize()
    return start.elapsed_time(end) / steps


def bench_scan(args, device, stream) -> dict:
    """The KLA scan alone (kla_scan fwd + bwd: y, y_var, every input gradient; or
    with ``--scan-pass fwd`` the forward under no_grad, where small grids take the
    time-split forward) at ``--shape B,L,M,S`` on the chosen backend: the d_state
    > 64 case of the fused kernels (hip_fused) against the composed path
    (hip_composed)."""
    from kla.ops import kla_scan

    B, L, M, S = (int(x) for x in args.shape.split(","))
    g = torch.Generator().manual_seed(0)
    ins = [torch.randn(B, L, M, generator=g), torch.rand(B, L, M, generator=g) + 0.5,
           torch.randn(B, L, S, generator=g) * 0.3, torch.randn(B, L, S, generator=g) * 0.3,
           torch.rand(M, S, generator=g) * 0.5 + 0.45, torch.rand(M, S, generator=g) * 0.05 + 0.01]
    dy, dyv = torch.randn(B, L, M, generator=g).to(device), torch.randn(B, L, M, generator=g).to(device)
    fwd_only = args.scan_pass == "fwd"
    xs = [t.to(device).requires_grad_(not fwd_only) for t in ins]

    def step():
        y, y_var, _ = kla_scan(*xs, backend=args.backend)
        torch.autograd.backward((y, y_var), (dy, dyv))
        for x in xs:
            x.grad = None

    @torch.no_grad()
    def forward():
        kla_scan(*xs, backend=args.backend)

    ms = _timed(forward if fwd_only else step, args.steps, args.warmup, stream)
    what = "forward (no_grad)" if fwd_only else "fwd+bwd"
    return {"metric": f"kla_scan {what} tokens/s, (B, L, M, S) = ({B}, {L}, {M}, {S}), fp32",
            "value": B * L / (ms * 1e-3), "unit": "tokens/s", "ms_per_step": round(ms, 4),
            "lane_steps_per_s": B * L * M * S / (ms * 1e-3), "backend": args.backend,
            "steps": args.steps, "warmup": args.warmup,
            "peak_mem_GiB": round(torch.cuda.max_memory_allocated(device) / 2**30, 2)}


# ------------------------------------------------------- BASELINE configs 1-5
#
# Each config entry carries the GPU time and rate, a roofline for what bounds it
# and a CPU baseline: the same workload's reference algorithm (the kla package's
# restated torch backend, reference kla_ops.py:188-290 and the layer and model
# around it) on a bounded sample on this host.

PEAK_FP32_MATRIX_TFLOPS = 157.3
# VALU issue: 256 CUs x 4 SIMDs, one wave64 VALU instruction per SIMD every 4
# cycles (16 lanes wide) at 2.4 GHz = 614.4 G wave-instructions/s. SQ_INSTS_VALU
# counts wave-instructions; transcendentals issue at a quarter of this rate, so
# the fraction of a kernel that uses them is a lower bound on its issue use.
VALU_ISSUE_PEAK_G = 256 * 4 * 2.4 / 4


def linear_flops_per_token(module) -> int:
    """Multiply-add flops per token of every nn.Linear in ``module`` (2 in out)."""
    import torch.nn as nn

    return sum(2 * m.in_features * m.out_features for m in module.modules() if isinstance(m, nn.Linear))


def _mfma_roofline(what: str, flops: float, ms: float) -> dict:
    tflops = flops / (ms * 1e-3) / 1e12
    return {"kernel": what, "bound": "mfma", "achieved": round(tflops, 2), "peak": PEAK_FP32_MATRIX_TFLOPS,
            "unit": "TFLOP/s", "frac": round(tflops / PEAK_FP32_MATRIX_TFLOPS, 4), "traffic": None,
            "flops": int(flops)}


def _hbm_roofline(what: str, nbytes: float, ms: float, traffic=None, traffic_source=None) -> dict:
    gbps = nbytes / (ms * 1e-3) / 1e9
    return {"kernel": what, "bound": "hbm", "achieved": round(gbps, 1), "peak": PEAK_HBM_GBPS, "unit": "GB/s",
            "frac": round(gbps / PEAK_HBM_GBPS, 4), "traffic": traffic, "traffic_source": traffic_source,
            "alg_bytes": int(nbytes)}


def _host() -> dict:
    return {"cpu": cpu_model_name(), "affinity_cores": len(os.sched_getaffinity(0)),
            "torch_threads": torch.get_num_threads()}


def _cpu_once(fn, warm=None):
    """One untimed call of ``warm`` (or ``fn``), then one timed call of ``fn``; seconds."""
    (warm or fn)()
    t0 = time.perf_counter()
    fn()
    return time.perf_counter() - t0


def config_c1(device, stream, steps, warmup, backend="hip", cpu=True) -> dict:
    """KLALayer(512, d_state=16) forward, x (2, 1024, 512) fp32."""
    from kla import KLAConfig, KLALayer

    torch.manual_seed(0)
    layer = KLALayer(512, KLAConfig(d_state=16, backend=backend))
    x_cpu = torch.randn(2, 1024, 512, generator=torch.Generator().manual_seed(0))
    out = {}
    # The GPU first: CPU worker threads still spinning after a large CPU run slow
    # the thread that launches the GPU kernels.
    with torch.no_grad():
        layer.to(device)
        x = x_cpu.to(device)
        ms = _timed(lambda: layer(x), steps, warmup, stream)
        y = layer(x).float().cpu()
        layer.cpu()
        layer.config.backend = "torch"
        y_cpu = layer(x_cpu)
        if cpu:
            cpu_s, reps = _median_time(lambda: layer(x_cpu), 6.0, max_reps=5)
            out["cpu_baseline"] = {
                "value": 2 * 1024 / cpu_s, "unit": "tokens/s", "cores": torch.get_num_threads(), "kind": "port",
                "sample": (f"the whole config (same layer and input) on backend 'torch' on the host CPU (reference "
                           f"kla_scan_torch, doubling scan under no_grad); median of {reps} reps = {cpu_s:.2f} s"),
                "host": _host()}
        layer.config.backend = backend
    err = ((y - y_cpu).abs().max() / (y_cpu.abs().max() + 1e-12)).item()
    flops = linear_flops_per_token(layer) * 2 * 1024
    out.update({"metric": "KLALayer(512, d_state=16) forward tokens/s, x (2,1024,512) fp32",
                "value": 2 * 1024 / (ms * 1e-3), "unit": "tokens/s", "ms": round(ms, 4), "backend": backend,
                "dtype": "f32", "max_rel_err_vs_cpu": err,
                "roofline": _mfma_roofline("whole forward: fp32 projections (hipBLASLt) + HIP scan and glue, "
                                           "priced on the projections' flops", flops, ms)})
    return out


def config_c3(device, stream, steps, warmup, adt, cpu=True) -> dict:
    """the standalone affine scan fwd + bwd at (8, 8192, 2048), fp32 or bf16 I/O."""
    name = "affine_b8_t8192_l2048" + ("_bf16" if adt == torch.bfloat16 else "")
    batch, steps_t, lanes, _, ops = WORKLOADS[name]
    elems = batch * steps_t * lanes
    step, kernels = build_step(batch, steps_t, lanes, adt, device, ops)
    ms = _timed(step, steps, warmup, stream)
    per = time_kernels_in_step(kernels, steps, stream)
    kern = {}
    for k, kms in per.items():
        nbytes = alg_bytes_per_elem(k, adt) * elems
        kern[k] = {"ms": round(kms, 4), "alg_bytes": nbytes, "GBps": round(nbytes / (kms * 1e-3) / 1e9, 1)}
    dom = max(kern, key=lambda k: kern[k]["ms"])
    traffic, src = None, None
    tfile = os.path.join(REPO, "profiles", f"traffic_{name}.json")
    if os.path.exists(tfile):
        with open(tfile) as f:
            traffic, src = json.load(f).get(dom), os.path.relpath(tfile, REPO)
    step_bytes = sum(v["alg_bytes"] for v in kern.values())
    out = {"metric": f"Affine scan fwd+bwd tokens/s, B=8 T=8192 L=2048 {'bf16 I/O' if adt == torch.bfloat16 else 'fp32'}",
           "value": batch * steps_t / (ms * 1e-3), "unit": "tokens/s", "ms": round(ms, 4),
           "dtype": "f32" if adt == torch.float32 else "bf16 I/O, f32 arithmetic",
           "achieved_GBps": round(step_bytes / (ms * 1e-3) / 1e9, 1), "alg_bytes_per_step": step_bytes,
           "roofline": _hbm_roofline(dom, kern[dom]["alg_bytes"], kern[dom]["ms"], traffic, src),
           "kernels": kern, "workload": name}
    del step, kernels
    torch.cuda.empty_cache()
    if cpu:
        cb = cpu_baseline(lanes, "affine", budget_s=5.0, seq_budget_s=3.0)
        cb["sample"] += " (the reference widens bf16 to fp32, so the CPU side is fp32)" if adt == torch.bfloat16 else ""
        out["cpu_baseline"] = cb
    return out


def _fused_kernel_bytes(B, L, M, S, sensor_bytes, var=False):
    """Bytes the fused scan kernels of a KLALayer training step must move: the
    forward reads v and log sigma^2 (sensor dtype), k, q and writes y (and y_var)
    and the (lam, eta) checkpoints every 16 steps; the backward reads dy (and
    dy_var), v, log sigma^2, k, q, the checkpoints and writes dv, d log sigma^2
    (sensor dtype) and the per-channel-group dk, dq partials ([B, L, M / (256 /
    S), S] fp32, which the backward's fixed-order reductions then sum: the one
    part of these bytes that the reference algorithm does not move)."""
    seq, st = B * L * M, B * L * S
    ck = 2 * B * -(-L // 16) * M * S * 4
    groups = -(-M // (256 // S))
    fwd = 2 * seq * sensor_bytes + 2 * st * 4 + seq * 4 * (2 if var else 1) + ck
    bwd = seq * 4 * (2 if var else 1) + 2 * seq * sensor_bytes + 2 * st * 4 + ck + 2 * seq * sensor_bytes \
        + 2 * B * L * groups * S * 4
    return {"fused_fwd": fwd, "fused_bwd": bwd}


def config_c4(device, stream, steps, warmup, backend="hip", cpu=True) -> dict:
    """KLALayer(1024, d_state=16) training step, x (4, 4096, 1024),
    bf16 autocast, loss = mean(out^2). The fused scan kernels are timed inside the
    step with HIP events that the library records around each launch
    (kla_set_kernel_events) and priced on their VALU issue (SQ_INSTS_VALU of a
    committed rocprofv3 counter run) and on their compulsory HBM bytes."""
    from kla import KLAConfig, KLALayer

    torch.cuda.reset_peak_memory_stats(device)   # peak_mem_GiB: this config's own
    torch.manual_seed(0)
    layer = KLALayer(1024, KLAConfig(d_state=16, backend=backend))
    out = {}
    layer.to(device)
    x = torch.randn(4, 4096, 1024, generator=torch.Generator().manual_seed(0)).to(device)

    def step():
        with torch.autocast("cuda", dtype=torch.bfloat16):
            y = layer(x)
        y.float().square().mean().backward()
        layer.zero_grad(set_to_none=True)

    ms = _timed(step, steps, warmup, stream)
    out.update({"metric": "KLALayer(1024, d_state=16) train step tokens/s, x (4,4096,1024), bf16 autocast",
                "value": 4 * 4096 / (ms * 1e-3), "unit": "tokens/s", "ms": round(ms, 4), "backend": backend,
                "dtype": "bf16 activations, f32 scan state",
                "peak_mem_GiB": round(torch.cuda.max_memory_allocated(device) / 2**30, 2)})
    if backend.startswith("hip"):
        out.update(_c4_kernel_rooflines(layer, step, steps, device))
    if cpu:
        layer.cpu()
        torch.cuda.empty_cache()
        out["cpu_baseline"] = _c4_cpu_baseline(layer, backend)
    return out


def _c4_kernel_rooflines(layer, step, steps, device) -> dict:
    """The fused scan kernels of the C4 step, timed inside it (HIP events the
    library records around each launch) and priced on VALU issue and bytes."""
    from kla.ops.hip import _lib

    with _lib.KernelTimer(_lib.KLA_KERNEL_FUSED_FWD, device) as tf, \
            _lib.KernelTimer(_lib.KLA_KERNEL_FUSED_BWD, device) as tb:
        for _ in range(steps):
            tf.arm()
            tb.arm()
            step()
    kms = {"fused_fwd": statistics.mean(tf.times_ms()), "fused_bwd": statistics.mean(tb.times_ms())}
    kb = _fused_kernel_bytes(4, 4096, layer.d_inner, 16, sensor_bytes=2)
    valu = {}
    vfile = os.path.join(REPO, "profiles", "valu_fused_kla_c4_layer_train_step.json")
    if os.path.exists(vfile):
        with open(vfile) as f:
            valu = json.load(f)
    kern = {}
    for k in ("fused_fwd", "fused_bwd"):
        e = {"ms": round(kms[k], 4), "kernel_bytes": kb[k], "GBps": round(kb[k] / (kms[k] * 1e-3) / 1e9, 1)}
        if k in valu:
            rate = valu[k]["SQ_INSTS_VALU"] / (kms[k] * 1e-3) / 1e9
            e.update({"valu_wave_instructions": valu[k]["SQ_INSTS_VALU"], "valu_G_per_s": round(rate, 1),
                      "valu_frac": round(rate / VALU_ISSUE_PEAK_G, 4)})
        kern[k] = e
    bwd = kern["fused_bwd"]
    out = {"kernels": kern}
    out["roofline"] = {"kernel": "fused_kla_bwd_kernel<16, false, true, false>", "bound": "valu",
                       "achieved": bwd.get("valu_G_per_s"), "peak": VALU_ISSUE_PEAK_G,
                       "unit": "G VALU wave-instructions/s", "frac": bwd.get("valu_frac"), "traffic": None,
                       "valu_source": os.path.relpath(vfile, REPO) if valu else None,
                       "hbm_GBps": bwd["GBps"], "hbm_frac": round(bwd["GBps"] / PEAK_HBM_GBPS, 4)}
    return out


def _c4_cpu_baseline(layer, backend) -> dict:
    """The same layer's training step on backend 'torch' on the host CPU."""
    L = 1024

    def cpu_step(x):
        with torch.autocast("cpu", dtype=torch.bfloat16):
            y = layer(x)
        y.float().square().mean().backward()
        layer.zero_grad(set_to_none=True)

    layer.config.backend = "torch"
    xs = torch.randn(1, L, 1024, generator=torch.Generator().manual_seed(1))
    cpu_s = _cpu_once(lambda: cpu_step(xs), warm=lambda: cpu_step(xs[:, :16]))
    layer.config.backend = backend
    return {
        "value": L / cpu_s, "unit": "tokens/s", "cores": torch.get_num_threads(), "kind": "port",
        "sample": (f"the same layer's training step on backend 'torch' on the host CPU under bf16 autocast, "
                   f"x (1, {L}, 1024) (the reference's associative scan under grad; its cost grows faster than "
                   f"linearly in L, so the full 4096-step rate is lower); one rep after a 16-step warm-up = "
                   f"{cpu_s:.2f} s"),
        "host": _host()}


def config_c5(device, stream, steps, backend="hip", nb=16, phases=("prefill", "decode"), cpu=True) -> dict:
    """SequenceModel(vocab 50304, d_model 512, 6 layers) stateful
    prefill of (nb, 2048) random ids, then 256 greedy one-token decode steps."""
    from kla import KLAConfig, ModelConfig, SequenceModel

    torch.cuda.reset_peak_memory_stats(device)   # peak_mem_GiB: this config's own
    torch.manual_seed(0)
    model = SequenceModel(ModelConfig(vocab_size=50304, d_model=512, n_layers=6),
                          KLAConfig(backend=backend)).eval()
    weight_bytes = sum(p.numel() * p.element_size() for n, p in model.named_parameters() if n != "embedding.weight")
    flops_tok = linear_flops_per_token(model)
    out = {}
    model.to(device)
    ids = torch.randint(0, 50304, (nb, 2048), generator=torch.Generator().manual_seed(0)).to(device)
    state = {}

    @torch.no_grad()
    def prefill():
        st = model.init_state(nb)
        logits, st = model(ids, state=st)
        state["s"], state["tok"] = st, model._sample(logits[:, -1], 0.0, None)   # greedy

    pre_ms = _timed(prefill, max(1, steps), 1, stream)
    out["prefill"] = {"metric": f"SequenceModel(d=512, 6 layers) stateful prefill tokens/s ({nb}x2048)",
                      "value": nb * 2048 / (pre_ms * 1e-3), "unit": "prefill tokens/s", "ms": round(pre_ms, 3),
                      "backend": backend, "dtype": "f32",
                      "roofline": _mfma_roofline("whole prefill: fp32 projections and LM head (hipBLASLt) + HIP "
                                                 "scan and glue, priced on the projections' flops",
                                                 flops_tok * nb * 2048, pre_ms),
                      "cpu_baseline": None}
    if "decode" not in phases:
        return _c5_finish(out, model, backend, nb, cpu)

    @torch.no_grad()
    def decode256():
        st, tok = state["s"], state["tok"]
        for _ in range(256):
            logits, st = model(tok, state=st)
            tok = model._sample(logits[:, -1], 0.0, None)

    eager_ms = _timed(decode256, 1, 1, stream) / 256
    dec = {"metric": f"SequenceModel(d=512, 6 layers) one-token decode ms/token (batch {nb}, 256 greedy steps)",
           "unit": "ms/token", "higher_is_better": False, "eager_ms": round(eager_ms, 4), "backend": backend,
           "dtype": "f32", "weight_bytes_per_token": weight_bytes, "cpu_baseline": None}
    graph_ms = None
    if backend.startswith("hip"):
        from kla.models.decode_graph import DecodeGraph

        graph = DecodeGraph(model, state["s"])

        @torch.no_grad()
        def decode256_graph():
            tok = state["tok"]
            for _ in range(256):
                tok = model._sample(graph.step(tok)[:, -1], 0.0, None)

        graph_ms = _timed(decode256_graph, 1, 1, stream) / 256
        dec["graph_ms"] = round(graph_ms, 4)
    best = graph_ms if graph_ms is not None else eager_ms
    dec["value"] = round(best, 4)
    dec["ms"] = round(best, 4)
    dec["roofline"] = _hbm_roofline("one decode step (every weight but the embedding table streamed once)",
                                    weight_bytes, best)
    out["decode"] = dec
    out["peak_mem_GiB"] = round(torch.cuda.max_memory_allocated(device) / 2**30, 2)
    return _c5_finish(out, model, backend, nb, cpu)


def _c5_finish(out, model, backend, nb, cpu) -> dict:
    """The CPU baselines, after the GPU timings (GPU first: CPU worker threads
    still spinning after a large CPU run slow the thread that launches kernels)."""
    if cpu:
        model.cpu()
        torch.cuda.empty_cache()
        pre, dec = _c5_cpu_baselines(model, backend, nb)
        out["prefill"]["cpu_baseline"] = pre
        if "decode" in out:
            out["decode"]["cpu_baseline"] = dec
    return out


def _c5_cpu_baselines(model, backend, nb) -> tuple:
    """The same model on backend 'torch' on the host CPU: prefill and one-token decode."""
    for blk in model.blocks:
        blk.mixer.config.backend = "torch"
    Lp = 1024
    ids_c = torch.randint(0, 50304, (1, Lp), generator=torch.Generator().manual_seed(1))
    with torch.no_grad():
        pre_s = _cpu_once(lambda: model(ids_c, state=model.init_state(1)), warm=lambda: model(ids_c[:, :8]))
        ids16 = torch.randint(0, 50304, (nb, 16), generator=torch.Generator().manual_seed(2))
        lg, st = model(ids16, state=model.init_state(nb))
        tok = lg[:, -1].argmax(-1, keepdim=True)
        t0 = time.perf_counter()
        for _ in range(16):
            lg, st = model(tok, state=st)
            tok = lg[:, -1].argmax(-1, keepdim=True)
        dec_s = (time.perf_counter() - t0) / 16
    for blk in model.blocks:
        blk.mixer.config.backend = backend
    pre = {"value": Lp / pre_s, "unit": "prefill tokens/s", "cores": torch.get_num_threads(), "kind": "port",
           "sample": (f"the same model on backend 'torch' on the host CPU, stateful prefill of (1, {Lp}) ids; "
                      f"one rep after a warm-up = {pre_s:.2f} s"), "host": _host()}
    dec = {"value": dec_s * 1e3, "unit": "ms/token", "cores": torch.get_num_threads(), "kind": "port",
           "sample": (f"the same model on backend 'torch' on the host CPU: 16 one-token decode steps at batch "
                      f"{nb} after a 16-token prefill; mean {dec_s * 1e3:.1f} ms per step"), "host": _host()}
    return pre, dec


CONFIG_NAMES = ("c1", "c3_fp32", "c3_bf16", "c4", "c5")


def run_configs(names, device, stream, steps, warmup, cpu=True) -> dict:
    """The BASELINE configs named in ``names``, each in its own entry."""
    out = {}
    for name in names:
        print(f"[bench] config {name}", file=sys.stderr, flush=True)
        time.sleep(0.5)   # let the CPU worker threads of the previous config's CPU baseline go idle
        t0 = time.perf_counter()
        if name == "c1":
            out["c1_layer_forward"] = config_c1(device, stream, steps, warmup, cpu=cpu)
        elif name == "c3_fp32":
            out["c3_affine_fp32"] = config_c3(device, stream, steps, warmup, torch.float32, cpu=cpu)
        elif name == "c3_bf16":
            out["c3_affine_bf16"] = config_c3(device, stream, steps, warmup, torch.bfloat16, cpu=cpu)
        elif name == "c4":
            out["c4_layer_train_step"] = config_c4(device, stream, steps, max(3, warmup // 4), cpu=cpu)
        elif name == "c5":
            c5 = config_c5(device, stream, max(1, steps // 4), cpu=cpu)
            out["c5_prefill"] = c5["prefill"]
            out["c5_decode"] = c5["decode"]
        gc.collect()
        torch.cuda.empty_cache()
        print(f"[bench] config {name} done in {time.perf_counter() - t0:.1f} s", file=sys.stderr, flush=True)
    return out


def bench_layer(args, device, stream) -> dict:
    """One layer-level BASELINE config (c1 / c4 / c5) on the chosen kla backend, on its own line."""
    cpu = not args.no_cpu_baseline
    if args.layer == "c1":
        return config_c1(device, stream, args.steps, args.warmup, args.backend, cpu=cpu)
    if args.layer == "c4":
        return config_c4(device, stream, args.steps, args.warmup, args.backend, cpu=cpu)
    phases = ("prefill",) if args.c5_phase == "prefill" else ("prefill", "decode")
    return config_c5(device, stream, max(1, args.steps // 4), args.backend, args.c5_batch, phases, cpu=cpu)


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--workload", default=DEFAULT_WORKLOAD, choices=sorted(WORKLOADS))
    ap.add_argument("--only", default=None,
                    choices=["mobius_fwd", "mobius_bwd", "affine_fwd", "affine_bwd", "copy", "all"])
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--streams", type=int, default=1, choices=[1, 2],
                    help="2: run the affine chain on a second stream beside the Moebius chain (the timed step "
                         "only; the per-kernel timings and the roofline stay those of the serial step)")
    ap.add_argument("--layer", default=None, choices=["c1", "c4", "c5", "scan"],
                    help="measure a layer-level config instead of the headline scan step "
                         "(scan: kla_scan alone at --shape)")
    ap.add_argument("--shape", default="2,2048,512,128", help="B,L,M,S for --layer scan")
    ap.add_argument("--scan-pass", default="fwd+bwd", choices=["fwd+bwd", "fwd"],
                    help="--layer scan: forward and backward, or the inference forward alone")
    ap.add_argument("--c5-batch", type=int, default=16,
                    help="--layer c5: sequences per prefill / decode batch (16 is the C5 config)")
    ap.add_argument("--c5-phase", default="all", choices=["all", "prefill"],
                    help="--layer c5: time the prefill and the decode (all) or the prefill only")
    ap.add_argument("--backend", default="hip", help="kla backend for --layer (hip, hip_composed, torch)")
    ap.add_argument("--configs-only", action="store_true",
                    help="skip the headline step: print the configs alone (for per-config rocprofv3 runs)")
    ap.add_argument("--configs", default="all",
                    help="BASELINE configs measured after the headline, in the same JSON line's 'configs': 'all', "
                         "'none' or a comma list of " + ", ".join(CONFIG_NAMES))
    args = ap.parse_args(argv)
    if args.configs == "all":
        config_names = list(CONFIG_NAMES)
    elif args.configs == "none":
        config_names = []
    else:
        config_names = [c for c in args.configs.split(",") if c]
        bad = [c for c in config_names if c not in CONFIG_NAMES]
        if bad:
            ap.error(f"unknown config(s) {bad}; choose from {', '.join(CONFIG_NAMES)}")

    if args.gpus != 1:
        print(f"bench.py: --gpus {args.gpus} is not supported: this build runs the scan on one GPU "
              "(the multi-GPU sharding of the path is a design note only); use --gpus 1.", file=sys.stderr)
        return 2
    if not torch.cuda.is_available():
        print("bench.py: no GPU visible", file=sys.stderr)
        return 1

    device = torch.device("cuda", 0)
    stream = torch.cuda.current_stream(device)
    if args.layer == "scan":
        print(json.dumps(bench_scan(args, device, stream)), flush=True)
        return 0
    if args.layer:
        print(json.dumps(bench_layer(args, device, stream)), flush=True)
        return 0
    if args.configs_only:
        print(json.dumps({"configs": run_configs(config_names, device, stream, args.steps, args.warmup,
                                                 cpu=not args.no_cpu_baseline)}), flush=True)
        return 0
    batch, steps, lanes, adt, ops = WORKLOADS[args.workload]
    elems = batch * steps * lanes

    if args.only in ("copy", "all"):
        # Calibration kernel for the HBM byte counters: 1 GiB read + 1 GiB written per launch.
        a = torch.ones(1 << 28, device=device)
        b = torch.empty_like(a)
        for _ in range(args.warmup + args.steps):
            b.copy_(a)
        torch.cuda.synchronize()
        print(json.dumps({"only": "copy", "bytes_read": a.numel() * 4, "bytes_written": b.numel() * 4,
                          "launches": args.warmup + args.steps}), flush=True)
        del a, b
        if args.only == "copy":
            return 0

    print(f"[bench] building inputs for {args.workload} ({batch}x{steps}x{lanes})", file=sys.stderr, flush=True)
    step, kernels = build_step(batch, steps, lanes, adt, device, ops, args.streams)

    if args.only:
        names = list(kernels) if args.only == "all" else [args.only]
        if any(n not in kernels for n in names):
            print(f"bench.py: workload {args.workload} has no {args.only} kernel", file=sys.stderr)
            return 2
        for name in ("mobius_fwd", "affine_fwd"):  # the backward kernels read the forward outputs
            if name in kernels:
                kernels[name]()
        for _ in range(args.warmup + args.steps):
            for name in names:
                kernels[name]()
        torch.cuda.synchronize()
        print(json.dumps({"only": args.only, "launches": args.warmup + args.steps, "workload": args.workload}),
              flush=True)
        return 0

    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    with _NoGC():
        for _ in range(args.warmup):
            step()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        start.record(stream)
        for _ in range(args.steps):
            step()
        end.record(stream)
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
    ms_per_step = start.elapsed_time(end) / args.steps

    from kla.ops.hip import _lib

    failures = _lib.workspace_failures_all(device)
    per_kernel_ms = time_kernels_in_step(kernels, args.steps, stream)
    per_kernel = {}
    for name, ms in per_kernel_ms.items():
        kdt = adt if name.startswith("affine") else torch.float32
        nbytes = alg_bytes_per_elem(name, kdt) * elems
        own = int(kernel_bytes_per_elem(name, kdt) * elems)
        per_kernel[name] = {"ms": round(ms, 4), "alg_bytes": nbytes, "GBps": round(nbytes / (ms * 1e-3) / 1e9, 1),
                            "kernel_bytes": own, "kernel_GBps": round(own / (ms * 1e-3) / 1e9, 1)}
    dom = max(per_kernel, key=lambda k: per_kernel[k]["ms"])
    step_bytes = sum(v["alg_bytes"] for v in per_kernel.values())
    tokens = batch * steps
    achieved_step = step_bytes / (ms_per_step * 1e-3) / 1e9

    traffic = None
    tfile = os.path.join(REPO, "profiles", f"traffic_{args.workload}.json")
    if os.path.exists(tfile):
        with open(tfile) as f:
            traffic = json.load(f).get(dom)

    if ops == "affine":
        metric = (f"Affine scan fwd+bwd tokens/s + achieved HBM GB/s, B={batch} T={steps} "
                  f"{'bf16 I/O' if adt == torch.bfloat16 else 'fp32'}, 1 GPU")
        ops_desc = "affine fwd+bwd" + (" (bf16 I/O, f32 state)" if adt == torch.bfloat16 else "")
        dtype = "f32" if adt == torch.float32 else "bf16 I/O, f32 arithmetic"
    else:
        metric = METRIC
        ops_desc = "Moebius fwd+bwd (D=1) + affine fwd+bwd"
        dtype = "f32" if adt == torch.float32 else "f32 (Moebius), bf16 I/O with f32 state (affine)"
    result = {
        "metric": metric,
        "value": tokens / (ms_per_step * 1e-3),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": dtype,
        "data": "synthetic",
        "config": {"workload": args.workload, "batch": batch, "steps": steps, "lanes": lanes,
                   "schedule": "one stream" if args.streams == 1 or ops != "mobius+affine" else
                   "Moebius and affine chains on two streams",
                   "ops": ops_desc, "parallelism": "single GPU"},
        "achieved_GBps": round(achieved_step, 1),
        "alg_bytes_per_step": step_bytes,
        "roofline": {
            "kernel": dom,
            "bound": "hbm",
            "achieved": per_kernel[dom]["GBps"],
            "peak": PEAK_HBM_GBPS,
            "unit": "GB/s",
            "frac": round(per_kernel[dom]["GBps"] / PEAK_HBM_GBPS, 4),
            "traffic": traffic,
            # traffic is not counted in this run: it is the calibrated FETCH_SIZE +
            # WRITE_SIZE bytes per launch from a rocprofv3 --pmc run of this workload.
            "traffic_source": (os.path.relpath(tfile, REPO) if traffic is not None else None),
            # The same launch priced on the bytes the kernel itself must move.
            "kernel_bytes": per_kernel[dom]["kernel_bytes"],
            "kernel_GBps": per_kernel[dom]["kernel_GBps"],
            "kernel_frac": round(per_kernel[dom]["kernel_GBps"] / PEAK_HBM_GBPS, 4),
        },
        "kernels": per_kernel,
        "wall_s": round(wall, 4),
        "lookback_failures": failures,
    }
    if not args.no_cpu_baseline:
        print("[bench] timing the CPU baseline", file=sys.stderr, flush=True)
        result["cpu_baseline"] = cpu_baseline(lanes, ops)
    if config_names and args.workload == DEFAULT_WORKLOAD:
        del step, kernels
        gc.collect()
        torch.cuda.empty_cache()
        result["configs"] = run_configs(config_names, device, stream, args.steps, args.warmup,
                                        cpu=not args.no_cpu_baseline)
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
