#!/usr/bin/env python
"""Benchmark of the gfx950 hot path on one MI355X.

Default workload (BASELINE.json metric "Pairformer layer ms @N=1024 bf16;
tri-attn/mult % of MFMA/HBM roofline"): one Boltz-2 PairformerLayer forward
at N=1024 (configs[3], one of the 64 trunk blocks): tri_mul_out, tri_mul_in,
tri_att_start, tri_att_end, transition_z on the fp32 pair stream with the bf16
gfx950 kernels, then the fp32 sequence stack.  Inputs (z [1,N,N,128],
s [1,N,384], masks all ones) and random-init weights (seed 0, N(0, 0.08),
norm weights N(1, 0.08)) are resident in HBM before timing.

The default line also carries ``dropin``: the same layer (weights, inputs)
timed through ``install()`` as a Boltz user runs it (guards, dropout draws,
per-call allocation), with its ratio to the headline.

Other workloads (--workload), each on one BASELINE config:
  dropin           configs[3]: the installed PairformerLayer alone (its own line)
  trimul           configs[2]: TriangleMultiplication out and in, N=768, 5% of tokens masked
  triattn          configs[1]: TriangleAttention start and end, N=512, last 51 tokens masked
  trunk            configs[3]: the 64-block PairformerModule at N=1024
  diffusion-step   configs[4]: 20 consecutive denoiser steps of the score model's transformer
                   stacks (atom encoder / decoder 3 + 3 blocks at 5 x 8192 atoms, token
                   transformer 24 blocks at 5 x 1024 tokens), fp32 as the reference runs them
  token-attention, diffusion   single diffusion modules at configs[4] shapes

Prints one JSON line.  ``roofline`` covers the kernel with the largest share
of the step, timed with HIP events on the launch stream; its ``bound`` is
whichever of flop time (at the MFMA peak) and byte time (at 8 TB/s) is larger.
``modules`` gives each triangle module's time against its roofline T* =
max(F / 2.5 PFLOP/s, B / 8 TB/s), F the module's algorithmic flops and B its
compulsory HBM bytes (``tri_module_cost``).  ``cpu_baseline`` times the fp32
CPU oracle on the host cores: a reported baseline, not the target.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import statistics
import sys
import time

PEAK_BF16_TFLOPS = 2500.0
PEAK_FP32_TFLOPS = 157.3
PEAK_HBM_GBS = 8000.0
# Transcendental issue rate: one 64-lane v_exp_f32 per 8 cycles per SIMD
# (probe on the box), 256 CUs x 4 SIMDs at 2.4 GHz.
EXP_PER_SIMD_CYCLE, SIMDS, CLOCK_HZ = 64 / 8, 1024, 2.4e9
ROOT = os.path.dirname(os.path.abspath(__file__))
WORKLOADS = ("pairformer", "dropin", "trunk", "trimul", "triattn", "diffusion-step", "token-attention", "diffusion")


def parse():
    p = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=None, help="timed steps (default depends on the workload)")
    p.add_argument("--warmup", type=int, default=3)
    p.add_argument("--n", type=int, default=None, help="token count (default: the workload's config)")
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--kernel-reps", type=int, default=3, help="repetitions of the per-kernel timing pass")
    p.add_argument("--calibrate-copy", action="store_true",
                   help="first copy 1 GiB device-to-device (a kernel of known traffic for scaling PMC byte counters)")
    p.add_argument("--workload", choices=WORKLOADS, default="pairformer")
    return p.parse_args()


def init_weights(module, seed: int):
    """Every parameter N(0, 0.08), norm weights N(1, 0.08) (the reference
    tests' convention, tests/test_operator_additions.py:43-47)."""
    import torch

    g = torch.Generator().manual_seed(seed)
    with torch.no_grad():
        for name, p in module.named_parameters():
            mean = 1.0 if "norm" in name and name.endswith("weight") else 0.0
            p.copy_(torch.randn(p.shape, generator=g) * 0.08 + mean)
    return module


def fan_in_weights(module, seed: int):
    """Weights N(0, 1 / fan_in), norm weights N(1, 0.08), vectors N(0, 0.08):
    keeps 24 residual blocks of width 768 bounded (the 0.08 convention
    amplifies each such block's output about a hundredfold)."""
    import torch

    g = torch.Generator().manual_seed(seed)
    with torch.no_grad():
        for name, p in module.named_parameters():
            if "norm" in name and name.endswith("weight"):
                p.copy_(1 + 0.08 * torch.randn(p.shape, generator=g))
            elif p.dim() == 2:
                p.copy_(torch.randn(p.shape, generator=g) / math.sqrt(p.shape[1]))
            else:
                p.copy_(0.08 * torch.randn(p.shape, generator=g))
    return module


# ----------------------------------------------------------------- rooflines


def tri_module_cost(kind: str, n: int):
    """(F flops, B compulsory bytes) of one triangle module direction:
    tri-attention F = 512 N^3 + 164864 N^2,
    tri-multiplication F = 256 N^3 + 196608 N^2; B = N^2 (128*4 + 4 + 128*2)
    (fp32 z and mask in, bf16 out)."""
    n2, n3 = float(n) ** 2, float(n) ** 3
    f = 512 * n3 + 164864 * n2 if kind == "triattn" else 256 * n3 + 196608 * n2
    return f, n2 * (128 * 4 + 4 + 128 * 2)


def t_star_ms(flops, nbytes, peak_tflops=PEAK_BF16_TFLOPS):
    return max(flops / (peak_tflops * 1e12), nbytes / (PEAK_HBM_GBS * 1e9)) * 1e3


def kernel_table(n: int):
    """Algorithmic flops and compulsory HBM bytes per launch, per kernel."""
    n2, n3 = float(n) ** 2, float(n) ** 3
    return {
        "trimul_proj": (2 * n2 * 128 * 512, n2 * (512 + 4 + 2 * 256)),
        "trimul_contract": (2 * 128 * n3, n2 * 128 * 2 * 3),
        "trimul_out": (2 * n2 * 128 * 256, n2 * (256 + 512 + 512)),
        "triattn_proj": (2 * n2 * 128 * 388, n2 * (512 + 4 + 3 * 256 + 16)),
        "triattn_core": (4 * 4 * 32 * n3, n2 * 4 * 3 * 64 + n2 * 256),
        "triattn_out": (2 * n2 * 128 * 256, n2 * (512 + 256 + 512)),
        "pair_transition": (2 * n2 * 128 * (1536 + 16), n2 * (1024 + 64)),  # + the fused pair bias
    }


def roofline_of(flops, nbytes, ms, peak_tflops=PEAK_BF16_TFLOPS):
    """Bound, achieved rate and fraction of peak of one launch; the bound is
    whichever of flop time and byte time is larger."""
    mfma = flops / (peak_tflops * 1e12) >= nbytes / (PEAK_HBM_GBS * 1e9)
    if mfma:
        achieved, peak, unit = flops / (ms * 1e-3) / 1e12, peak_tflops, "TFLOP/s"
    else:
        achieved, peak, unit = nbytes / (ms * 1e-3) / 1e9, PEAK_HBM_GBS, "GB/s"
    return {"bound": "mfma" if mfma else "hbm", "achieved": round(achieved, 2), "peak": peak, "unit": unit,
            "frac": round(achieved / peak, 4)}


def measured_traffic(kernel: str, n: int):
    """HBM bytes per launch of ``kernel`` from the committed rocprofv3 counter
    summary (FETCH_SIZE / WRITE_SIZE scaled by a 1 GiB copy), when it was
    taken at this N; None otherwise."""
    path = os.path.join(ROOT, "profiles", f"hbm_traffic_n{n}.json")
    try:
        with open(path) as f:
            data = json.load(f)
    except (OSError, ValueError):
        return None
    return data.get("bytes_per_launch", {}).get(kernel) if data.get("n") == n else None


def exp_co_bound(n, core_ms):
    """Exp co-bound of the attention core (H N^3 exponentials per direction at
    the measured v_exp_f32 issue rate) and its MFMA+exp issue floor."""
    exps = 4.0 * n ** 3
    exp_ms = exps / (EXP_PER_SIMD_CYCLE * SIMDS * CLOCK_HZ) * 1e3
    mfma_ms = 4 * 4 * 32 * float(n) ** 3 / (PEAK_BF16_TFLOPS * 1e12) * 1e3
    return {"exp_ms": round(exp_ms, 4), "mfma_ms": round(mfma_ms, 4), "issue_floor_ms": round(exp_ms + mfma_ms, 4),
            "issue_floor_frac": round((exp_ms + mfma_ms) / core_ms, 4)}


class no_gc:
    """Run the cyclic garbage collector, then pause it for the block (a full
    collection stalls the launching thread for 50-60 ms, measured)."""

    def __enter__(self):
        import gc

        gc.collect()
        self.was_enabled = gc.isenabled()
        gc.disable()

    def __exit__(self, *exc):
        import gc

        if self.was_enabled:
            gc.enable()
        return False


def event_timer():
    import torch

    class Timer:
        def __init__(self):
            self.spans = []

        def run(self, name, fn, k=1):
            """k consecutive calls of fn between one event pair (time per call)."""
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            for _ in range(k):
                fn()
            e1.record()
            self.spans.append((name, e0, e1, k))

        def averages(self):
            torch.cuda.synchronize()
            tot, cnt = {}, {}
            for name, e0, e1, k in self.spans:
                tot[name] = tot.get(name, 0.0) + e0.elapsed_time(e1) / k
                cnt[name] = cnt.get(name, 0) + 1
            return {k: tot[k] / cnt[k] for k in tot}, cnt

    return Timer()


def timed_loop(fn, steps, warmup, warm_s=0.25):
    """ms per call of ``fn`` over ``steps`` calls after ``warmup`` untimed ones
    (continued until ``warm_s`` seconds have passed, so that the GPU has left
    its idle clocks on the measured work itself), between device
    synchronisations, by HIP events on the current stream.  Python's cyclic
    garbage collector is run before and paused during the timed calls: a full
    collection stalls the launching thread for 50-60 ms (measured), which
    would leave the GPU idle for ten layers' worth of work."""
    import torch

    t0 = time.perf_counter()
    done = 0
    while done < warmup or (warmup and time.perf_counter() - t0 < warm_s):
        fn()
        done += 1
        if done >= warmup:
            torch.cuda.synchronize()
    torch.cuda.synchronize()
    with no_gc():
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        wall0 = time.perf_counter()
        e0.record()
        for _ in range(steps):
            fn()
        e1.record()
        torch.cuda.synchronize()
        wall = time.perf_counter() - wall0
    return e0.elapsed_time(e1) / steps, wall


def first_call_ms(fn):
    """HIP-event and wall time (ms) of a first call of ``fn``, made cold: the
    weight packs are built and the kernels' code objects loaded inside it."""
    import torch

    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record()
    fn()
    e1.record()
    torch.cuda.synchronize()
    return {"gpu_ms": round(e0.elapsed_time(e1), 3), "wall_ms": round((time.perf_counter() - t0) * 1e3, 3)}


def line(metric, value, unit, args, steps, dtype, data, config, higher_is_better=False, **extra):
    out = {"metric": metric, "value": round(value, 4), "unit": unit, "n_gpus": 1, "steps": steps,
           "warmup": args.warmup, "ms_per_step": round(value, 4) if unit == "ms" else None,
           "higher_is_better": higher_is_better, "scaling": "weak", "vs_baseline": None, "dtype": dtype,
           "data": data, "config": config}
    out.update(extra)
    return out


# ------------------------------------------------------------ CPU baselines


def _cpu_setup():
    import torch

    if ROOT not in sys.path:
        sys.path.insert(0, ROOT)
    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    return cores


def _median_ms(fn, reps, warm=None):
    if warm is not None:
        warm()
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        fn()
        times.append((time.perf_counter() - t0) * 1e3)
    return statistics.median(times), times


def cpu_pairformer(n_layer=1024, n_small=128):
    """CPU baseline of configs[0] and configs[3]: one PairformerLayer of the
    fp32 oracle at N=128 (2 warm-ups, median of 10) and at N=1024 (one
    warm-up at N=256, median of 2; x64 reported as the extrapolated trunk)."""
    import torch

    cores = _cpu_setup()
    from oracle import boltz_ref as R  # the checker, timed as the reference CPU path

    layer = init_weights(R.PairformerLayer(), 0).eval()
    g = torch.Generator().manual_seed(0)

    def inputs(n):
        return (torch.randn(1, n, 384, generator=g), torch.randn(1, n, n, 128, generator=g), torch.ones(1, n),
                torch.ones(1, n, n))

    with torch.inference_mode():
        small = inputs(n_small)
        run_small = lambda: layer(*small, chunk_size_tri_attn=64)
        cfg1, _ = _median_ms(run_small, 10, warm=lambda: (run_small(), run_small()))
        big = inputs(n_layer)
        warm = inputs(256)
        cfg4, times = _median_ms(lambda: layer(*big, chunk_size_tri_attn=64), 2,
                                 warm=lambda: layer(*warm, chunk_size_tri_attn=64))
    flops1 = 2.22e10
    return {"value": round(cfg4, 1), "unit": "ms per layer", "cores": cores, "kind": "port",
            "sample": f"fp32 CPU oracle (oracle/boltz_ref.py) PairformerLayer at N={n_layer}, median of 2 after a "
                      f"warm-up at N=256, tri-attention chunked 64 rows, {cores} threads",
            "runs_ms": [round(t, 1) for t in times],
            "trunk_64_ms_extrapolated": round(64 * cfg4, 1),
            "config1_n128_ms": round(cfg1, 2), "config1_gflops": round(flops1 / (cfg1 * 1e-3) / 1e9, 1)}


# ----------------------------------------------------------- the workloads


def pairformer(args):
    import torch
    from boltz_lumi_amd import layers, ops

    dev = torch.device("cuda:0")
    n = args.n or 1024
    steps = args.steps or 20
    if args.calibrate_copy:
        src = torch.ones(1 << 28, device=dev)  # 1 GiB of fp32
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    layer = init_weights(layers.PairformerLayer(), 0).to(dev).eval()
    g = torch.Generator().manual_seed(0)
    z = torch.randn(1, n, n, 128, generator=g).to(dev)
    s = torch.randn(1, n, 384, generator=g).to(dev)
    mask = torch.ones(1, n, device=dev)
    pair_mask = torch.ones(1, n, n, device=dev)
    ws = ops.new_workspace(n, dev)
    z_out = torch.empty_like(z)
    with torch.inference_mode():
        first = first_call_ms(lambda: layer(s, z, mask, pair_mask, z_out=z_out, workspace=ws))
        ms, wall = timed_loop(lambda: layer(s, z, mask, pair_mask, z_out=z_out, workspace=ws), steps, args.warmup)
        kt, modules_ms = per_kernel_times(layer, s, z, mask, pair_mask, z_out, ws, args.kernel_reps)
    del ws, z_out
    dropin = dropin_layer_ms(layer, s, z, mask, pair_mask, steps, args.warmup)
    dropin["vs_headline"] = round(dropin["ms"] / ms, 4)
    table = kernel_table(n)
    breakdown = {}
    for name, (avg_ms, launches) in kt.items():
        entry = {"ms": round(avg_ms, 4), "launches_per_layer": launches}
        if name in table:
            flops, nbytes = table[name]
            entry.update(roofline_of(flops, nbytes, avg_ms))
        breakdown[name] = entry
    dominant = max((k for k in breakdown if k in table),
                   key=lambda k: breakdown[k]["ms"] * breakdown[k]["launches_per_layer"])
    d = breakdown[dominant]
    roofline = {"kernel": dominant, **{k: d[k] for k in ("bound", "achieved", "peak", "unit", "frac")},
                "traffic": measured_traffic(dominant, n), "kernel_ms": d["ms"]}
    if dominant == "triattn_core":
        roofline["co_bound"] = exp_co_bound(n, d["ms"])
    modules = {}
    for name, mod_ms in modules_ms.items():
        f, b = tri_module_cost("triattn" if name.startswith("triattn") else "trimul", n)
        ts = t_star_ms(f, b)
        modules[name] = {"ms": round(mod_ms, 4), "t_star_ms": round(ts, 4), "frac": round(ts / mod_ms, 4)}
    layer_f = 2.831e12 * (n / 1024) ** 3  # algorithmic flops of one layer at N=1024 (dominated by the N^3 terms)
    modules["layer"] = {"ms": round(ms, 4), "t_star_ms": round(t_star_ms(layer_f, 0), 4),
                        "frac": round(t_star_ms(layer_f, 0) / ms, 4)}
    out = line("Pairformer layer ms @N=1024 bf16", ms, "ms", args, steps, "bf16",
               "synthetic (z, s ~ N(0,1); masks ones; random-init weights seed 0)",
               {"workload": f"PairformerLayer forward, N={n}, c_z=128, c_s=384, tri-att 4x32, tri-mult 128, "
                            f"transition x4, single attention 16 heads (BASELINE configs[3], one of 64 blocks)",
                "n_tokens": n, "batch": 1},
               wall_s=round(wall, 3), first_call=first,
               caches="value is warm: the bf16 weight packs are built on the first call (first_call) and reused "
                      "while the parameters keep their identity and version; z_out and the workspace are "
                      "preallocated (the dropin path takes them from torch's caching allocator every call)",
               roofline=roofline, modules=modules, breakdown=breakdown, dropin=dropin)
    if not args.no_cpu_baseline:
        out["cpu_baseline"] = cpu_pairformer(n)
    print(json.dumps(out), flush=True)


def dropin_layer_ms(layer, s, z, mask, pair_mask, steps, warmup):
    """The same layer as a Boltz user runs it: ``install`` on a model holding a
    PairformerLayer (Boltz's class and module names), called as upstream's
    PairformerModule calls it under bf16 autocast, with upstream's chunk size
    (128 above 384 tokens).  The patched forward checks its guards, draws the
    four dropout masks as upstream does, allocates its output z and workspace
    from torch's caching allocator, and runs the fused composition."""
    import copy

    import torch
    from boltz_lumi_amd import adapters

    host = torch.nn.Module()
    host.pairformer_module = torch.nn.Module()
    host.pairformer_module.layers = torch.nn.ModuleList([copy.deepcopy(layer)])
    patched = adapters.install(host, require_boltz2=False)
    installed = host.pairformer_module.layers[0]
    if "forward" not in vars(installed):
        raise RuntimeError("install() did not patch the PairformerLayer")
    chunk = 128 if z.shape[1] > 384 else 512
    with torch.inference_mode(), torch.autocast("cuda", dtype=torch.bfloat16):
        first = first_call_ms(lambda: installed(s, z, mask, pair_mask, chunk))
        ms, wall = timed_loop(lambda: installed(s, z, mask, pair_mask, chunk), steps, warmup)
    adapters.uninstall(host)
    return {"ms": round(ms, 4), "wall_s": round(wall, 3), "first_call": first, "patched_modules": patched,
            "path": "install(model) -> pairformer.pairformer_layer_forward under bf16 autocast"}


def dropin(args):
    """``--workload dropin``: the installed PairformerLayer alone (the headline
    layer's weights and inputs), one JSON line."""
    import torch
    from boltz_lumi_amd import layers

    dev = torch.device("cuda:0")
    n = args.n or 1024
    steps = args.steps or 20
    layer = init_weights(layers.PairformerLayer(), 0).to(dev).eval()
    g = torch.Generator().manual_seed(0)
    z = torch.randn(1, n, n, 128, generator=g).to(dev)
    s = torch.randn(1, n, 384, generator=g).to(dev)
    mask = torch.ones(1, n, device=dev)
    pair_mask = torch.ones(1, n, n, device=dev)
    d = dropin_layer_ms(layer, s, z, mask, pair_mask, steps, args.warmup)
    layer_f = 2.831e12 * (n / 1024) ** 3
    out = line("Pairformer layer ms @N=1024 bf16 (installed drop-in path)", d["ms"], "ms", args, steps, "bf16",
               "synthetic (z, s ~ N(0,1); masks ones; random-init weights seed 0)",
               {"workload": f"PairformerLayer forward through install() under bf16 autocast, N={n} (BASELINE "
                            f"configs[3], one of 64 blocks)", "n_tokens": n, "batch": 1},
               wall_s=d["wall_s"], path=d["path"], patched_modules=d["patched_modules"],
               modules={"layer": {"ms": d["ms"], "t_star_ms": round(t_star_ms(layer_f, 0), 4),
                                  "frac": round(t_star_ms(layer_f, 0) / d["ms"], 4)}})
    if not args.no_cpu_baseline:
        out["cpu_baseline"] = cpu_pairformer(n)
    print(json.dumps(out), flush=True)


def per_kernel_times(layer, s, z, mask, pair_mask, z_out, ws, reps):
    """Average ms per launch of every kernel of the layer (each stage launched
    on its own) and per module (stages 1|2|4 in one call), from HIP events on
    torch's current stream (the stream the kernels launch on)."""
    import torch
    from boltz_lumi_amd import ops

    zi, zo, mb = z[0], z_out[0], pair_mask[0].float().contiguous()
    plan = []
    modules = []
    for mod, outgoing, first, mname in ((layer.tri_mul_out, True, True, "trimul_out"),
                                        (layer.tri_mul_in, False, False, "trimul_in")):
        mode = ops.OUT_RESIDUAL if first else ops.OUT_ACCUMULATE
        src = zi if first else zo
        for stage, name in ((1, "trimul_proj"), (2, "trimul_contract"), (4, "trimul_out")):
            plan.append((name, lambda m=mod, o=outgoing, md=mode, x=src, st=stage:
                         ops.trimul(m, x, mb, o, md, zo, ws, stages=st)))
        modules.append((mname, lambda m=mod, o=outgoing, md=mode, x=src: ops.trimul(m, x, mb, o, md, zo, ws)))
    for mod, starting, mname in ((layer.tri_att_start, True, "triattn_start"),
                                 (layer.tri_att_end, False, "triattn_end")):
        for stage, name in ((1, "triattn_proj"), (2, "triattn_core"), (4, "triattn_out")):
            plan.append((name, lambda m=mod, st_=starting, st=stage:
                         ops.triattn(m, zo, mb, st_, ops.OUT_ACCUMULATE, zo, ws, stages=st)))
        modules.append((mname, lambda m=mod, st_=starting: ops.triattn(m, zo, mb, st_, ops.OUT_ACCUMULATE, zo, ws)))
    # the transition's epilogue also writes the sequence stack's pair bias, as in PairformerLayer.forward
    bias = torch.empty((1, 16) + zo.shape[:2], device=zo.device)
    pb = (layer.attention.proj_z[0], layer.attention.proj_z[1], bias[0])
    plan.append(("pair_transition", lambda: ops.pair_transition(layer.transition_z, zo, ops.OUT_ACCUMULATE, zo,
                                                                pair_bias=pb)))
    plan.append(("sequence_stack", lambda: layer.sequence_stack(s, z_out, mask, pair_bias=bias)))
    # untimed passes first, until the GPU has left the clocks it dropped to in the
    # synchronisation before this call (as timed_loop does): otherwise the first
    # timed launches run up to 40% slower; the first entry rewrites zo from zi, so
    # every pass sees the same inputs
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < 0.25:
        for _, fn in plan + modules:
            fn()
        torch.cuda.synchronize()  # host time then measures GPU time
    # each kernel timed over 4 consecutive launches: an event pair around a single
    # launch adds about 0.1 ms to the attention core (its per-layer sum then
    # exceeds the measured layer by 8%), while 4 launches agree with a kernel
    # trace's durations to 1%
    timer = event_timer()
    with no_gc():
        for _ in range(reps):
            for name, fn in plan:
                timer.run(name, fn, k=4)
            for name, fn in modules:
                timer.run("module:" + name, fn, k=4)
        avg, cnt = timer.averages()
    kernels = {k: (v, cnt[k] // reps) for k, v in avg.items() if not k.startswith("module:")}
    mods = {k[len("module:"):]: v for k, v in avg.items() if k.startswith("module:")}
    return kernels, mods


def trunk(args):
    """configs[3] in full: the 64-block PairformerModule at N=1024, layer l's
    weights from seed l; ping-pong pair buffers and one workspace."""
    import torch
    from boltz_lumi_amd import layers

    dev = torch.device("cuda:0")
    n = args.n or 1024
    steps = args.steps or 3
    module = layers.PairformerModule(num_blocks=64)
    for idx, layer in enumerate(module.layers):
        init_weights(layer, idx)
    module = module.to(dev).eval()
    g = torch.Generator().manual_seed(0)
    z = torch.randn(1, n, n, 128, generator=g).to(dev)
    s = torch.randn(1, n, 384, generator=g).to(dev)
    mask = torch.ones(1, n, device=dev)
    pair_mask = torch.ones(1, n, n, device=dev)
    with torch.inference_mode():
        ms, wall = timed_loop(lambda: module(s, z, mask, pair_mask), steps, min(args.warmup, 1))
        s_out, z_out = module(s, z, mask, pair_mask)
        finite = bool(torch.isfinite(z_out).all()) and bool(torch.isfinite(s_out).all())
    layer_f = 2.831e12 * (n / 1024) ** 3
    ts = 64 * t_star_ms(layer_f, 0)
    out = line("Pairformer trunk (64 blocks) ms @N=1024 bf16", ms, "ms", args, steps, "bf16",
               "synthetic (z, s ~ N(0,1); masks ones; random-init weights, layer l from seed l)",
               {"workload": f"PairformerModule, 64 PairformerLayers, N={n} (BASELINE configs[3] in full)",
                "n_tokens": n, "blocks": 64, "ms_per_layer": round(ms / 64, 4), "outputs_finite": finite},
               wall_s=round(wall, 3),
               modules={"trunk": {"ms": round(ms, 3), "t_star_ms": round(ts, 3), "frac": round(ts / ms, 4)}})
    if not args.no_cpu_baseline:
        out["cpu_baseline"] = cpu_pairformer(n)
    print(json.dumps(out), flush=True)


def token_mask_config(n, masked_tokens, seed=0):
    """Token mask with ``masked_tokens`` tokens set to 0: the last ones
    (``last``) or a random choice (``random``, randperm seed 0)."""
    import torch

    kind, count = masked_tokens
    m = torch.ones(n)
    if kind == "last":
        m[n - count:] = 0
    else:
        m[torch.randperm(n, generator=torch.Generator().manual_seed(seed))[:count]] = 0
    return m


def isolated_module(args, kind):
    """configs[1] (triattn: N=512, last 51 tokens masked) or configs[2]
    (trimul: N=768, 38 random tokens (5%) masked): both directions of the
    module under bf16 autocast on an fp32 z (the upstream bf16-mixed call),
    through the Boltz-compatible modules."""
    import torch
    from boltz_lumi_amd import layers, ops

    dev = torch.device("cuda:0")
    if kind == "triattn":
        n = args.n or 512
        masked = ("last", 51 * n // 512)
        mods = {"start": layers.TriangleAttention(), "end": layers.TriangleAttentionEndingNode()}
        core = "triattn_core"
    else:
        n = args.n or 768
        masked = ("random", round(0.05 * n))
        mods = {"out": layers.TriangleMultiplicationOutgoing(), "in": layers.TriangleMultiplicationIncoming()}
        core = "trimul_contract"
    steps = args.steps or 20
    for i, m in enumerate(mods.values()):
        init_weights(m, i)
    mods = {k: m.to(dev).eval() for k, m in mods.items()}
    g = torch.Generator().manual_seed(0)
    z = torch.randn(1, n, n, 128, generator=g)
    tok = token_mask_config(n, masked)
    pm = (tok[:, None] * tok[None, :])[None]
    zd, pmd = z.to(dev), pm.to(dev)
    ws = ops.new_workspace(n, dev)
    times, kernel_ms = {}, {}
    with torch.inference_mode(), torch.autocast("cuda", dtype=torch.bfloat16):
        for name, m in mods.items():
            fn = (lambda m=m: m(zd, pmd, workspace=ws)) if kind == "trimul" else \
                (lambda m=m: m(zd, pmd, workspace=ws))
            times[name], _ = timed_loop(fn, steps, args.warmup)
            # the dominant kernel alone (stage 2), after a full call filled the workspace
            x = zd[0].contiguous()
            mb = pmd[0].contiguous()
            if kind == "trimul":
                kfn = lambda m=m, nm=name: ops.trimul(m, x, mb, nm == "out", ops.OUT_BF16, None, ws, stages=2)
            else:
                kfn = lambda m=m, nm=name: ops.triattn(m, x, mb, nm == "start", ops.OUT_BF16, None, ws, stages=2)
            kfn()
            kernel_ms[name], _ = timed_loop(kfn, steps, 1)
    fp32_ms = {}
    if kind == "triattn":  # fp32 mode (autocast off): fp32 LN and GEMMs, fused fp32-MFMA attention
        with torch.inference_mode():
            for name, m in mods.items():
                fp32_ms[name], _ = timed_loop(lambda m=m, nm=name: ops.triattn_fp32(m, zd[0], pmd[0], nm == "start"),
                                              max(3, steps // 4), 1)
    f, b = tri_module_cost(kind, n)
    ts = t_star_ms(f, b)
    modules = {f"{kind}_{k}": {"ms": round(v, 4), "t_star_ms": round(ts, 4), "frac": round(ts / v, 4)}
               for k, v in times.items()}
    for k, v in fp32_ms.items():
        modules[f"{kind}_{k}_fp32_mode"] = {"ms": round(v, 4), "t_star_ms": round(ts, 4), "frac": round(ts / v, 4),
                                            "note": "fp32 mode, against the bf16 MFMA T*"}
    kf, kb = kernel_table(n)[core]
    kms = statistics.mean(kernel_ms.values())
    roofline = {"kernel": core, **roofline_of(kf, kb, kms), "traffic": measured_traffic(core, n),
                "kernel_ms": round(kms, 4), "kernel_ms_per_direction": {k: round(v, 4) for k, v in kernel_ms.items()}}
    if kind == "triattn":
        roofline["co_bound"] = exp_co_bound(n, kms)
    value = statistics.mean(times.values())
    title = {"triattn": "TriangleAttention (start, end) ms per direction @N=512, 10% padded, bf16",
             "trimul": "TriangleMultiplication (out, in) ms per direction @N=768, 5% masked, bf16"}[kind]
    desc = {"triattn": f"isolated TriangleAttention starting and ending node, N={n}, 4 heads x 32, last "
                       f"{masked[1]} tokens masked (BASELINE configs[1])",
            "trimul": f"isolated TriangleMultiplication outgoing and incoming, N={n}, {masked[1]} random tokens "
                      f"masked (BASELINE configs[2])"}[kind]
    out = line(title, value, "ms", args, steps, "bf16",
               "synthetic (z ~ N(0,1); random-init weights; token mask as stated)",
               {"workload": desc, "n_tokens": n, "masked_tokens": masked[1]},
               roofline=roofline, modules=modules)
    if not args.no_cpu_baseline:
        out["cpu_baseline"] = cpu_isolated(kind, n, masked)
    print(json.dumps(out), flush=True)


def cpu_isolated(kind, n, masked):
    """CPU baseline of configs[1] and configs[2]: the fp32 oracle module per
    direction, one warm-up at a quarter of N, median of 3."""
    import torch

    cores = _cpu_setup()
    from oracle import boltz_ref as R

    if kind == "triattn":
        mods = {"start": R.TriangleAttention(128, 32, 4), "end": R.TriangleAttentionEndingNode(128, 32, 4)}
    else:
        mods = {"out": R.TriangleMultiplicationOutgoing(128), "in": R.TriangleMultiplicationIncoming(128)}
    for i, m in enumerate(mods.values()):
        init_weights(m, i)
    g = torch.Generator().manual_seed(0)
    z = torch.randn(1, n, n, 128, generator=g)
    tok = token_mask_config(n, masked)
    pm = (tok[:, None] * tok[None, :])[None]
    small = n // 4
    per = {}
    with torch.inference_mode():
        for name, m in mods.items():
            kw = {"chunk_size": 64} if kind == "triattn" else {}
            per[name], _ = _median_ms(lambda m=m: m(z, pm, **kw), 3,
                                      warm=lambda m=m: m(z[:, :small, :small], pm[:, :small, :small], **kw))
    f, _ = tri_module_cost(kind, n)
    value = statistics.mean(per.values())
    return {"value": round(value, 1), "unit": "ms per direction", "cores": cores, "kind": "port",
            "sample": f"fp32 CPU oracle (oracle/boltz_ref.py) {kind} at N={n} with the same mask, each direction "
                      f"median of 3 after a warm-up at N={small}, {cores} threads",
            "per_direction_ms": {k: round(v, 1) for k, v in per.items()},
            "gflops": round(f / (value * 1e-3) / 1e9, 1)}


def diffusion_step(args):
    """``--steps`` (default 20) consecutive denoiser steps of the
    score model's transformer stacks (oracle.boltz_ref.DiffusionStacks at
    their Boltz module paths, the native forwards installed by
    ``install``): atom encoder and decoder (3 blocks each, 4 heads, 128
    channels, windows of 32 queries over 128 keys, 5 x 8192 atoms) and the
    token transformer (24 blocks, 16 heads x 48, 5 x 1024 tokens, one
    prepacked bias shared by the samples), fp32 with autocast off as the
    reference runs the score model (diffusion.py:37-49).  Each step feeds
    the coordinate update back into the coordinates."""
    import torch
    from torch import nn
    from boltz_lumi_amd import adapters, ops
    from boltz_lumi_amd.pair_bias import prepare_token_bias, prepare_window_bias

    if ROOT not in sys.path:
        sys.path.insert(0, ROOT)
    from oracle import boltz_ref as R  # the stacks' module structure (upstream Boltz classes, restated)

    dev = torch.device("cuda:0")
    samples, tokens, atoms, w, h = 5, args.n or 1024, 8192, 32, 128
    nw = atoms // w
    steps = args.steps or 20
    host = nn.Module()
    host.structure_module = nn.Module()
    host.structure_module.score_model = fan_in_weights(R.DiffusionStacks(), 0).to(dev).eval()
    stacks = host.structure_module.score_model
    patched = adapters.install(host, require_boltz2=False)
    g = torch.Generator().manual_seed(0)
    t = dict(r=torch.randn(samples, atoms, 3, generator=g) * 160.0, q=torch.randn(samples, atoms, 128, generator=g),
             c=torch.randn(samples, atoms, 128, generator=g), atom_mask=torch.ones(samples, atoms),
             enc_bias=torch.randn(1, nw, w, h, 12, generator=g), dec_bias=torch.randn(1, nw, w, h, 12, generator=g),
             a=torch.randn(samples, tokens, 768, generator=g), s=torch.randn(samples, tokens, 768, generator=g),
             token_bias=torch.randn(1, tokens, tokens, 24 * 16, generator=g), token_mask=torch.ones(samples, tokens))
    t = {k: v.to(dev) for k, v in t.items()}
    index = R.get_indexing_matrix(nw, w, h, device=dev)
    packed = prepare_token_bias(t["token_bias"])
    # the window biases as optimized_sample hands them to the atom transformers (channel-major)
    t["enc_bias"], t["dec_bias"] = prepare_window_bias(t["enc_bias"]), prepare_window_bias(t["dec_bias"])

    def to_keys(x):
        return R.single_to_keys(x, index, w, h)

    state = {"r": t["r"]}

    def step():
        upd, _, _ = stacks(state["r"], t["q"], t["c"], t["atom_mask"], t["enc_bias"], t["dec_bias"], to_keys, t["a"],
                           t["s"], packed, t["token_mask"], multiplicity=samples)
        state["r"] = state["r"] + 0.1 * upd

    with torch.inference_mode():
        ms, wall = timed_loop(step, steps, args.warmup)
        # per-stack times and the fused kernels of one step, by HIP events
        timer = event_timer()
        enc, dec = stacks.atom_attention_encoder.atom_encoder, stacks.atom_attention_decoder.atom_decoder
        for _ in range(3):
            timer.run("atom_encoder", lambda: enc(t["q"], t["c"], t["enc_bias"], to_keys, t["atom_mask"], samples))
            timer.run("token_transformer", lambda: stacks.token_transformer(t["a"], t["s"], packed, t["token_mask"],
                                                                            multiplicity=samples))
            timer.run("atom_decoder", lambda: dec(t["q"], t["c"], t["dec_bias"], to_keys, t["atom_mask"], samples))
        block_ms, _ = timer.averages()
        kernels = diffusion_kernel_times(stacks, t, packed, samples, tokens)
    dominant = max(kernels, key=lambda k: kernels[k]["ms"] * kernels[k]["launches_per_step"])
    d = kernels[dominant]
    roofline = {"kernel": dominant, **{k: d[k] for k in ("bound", "achieved", "peak", "unit", "frac")},
                "traffic": None, "kernel_ms": d["ms"]}
    out = line("diffusion denoiser step ms (configs[4]: 5 samples, 24 token + 3 + 3 atom blocks)", ms, "ms", args,
               steps, "f32", "synthetic (coords ~ N(0, 160^2), activations / conditioning / biases ~ N(0,1); "
                              "weights N(0, 1/fan_in))",
               {"workload": f"score-model transformer stacks, {steps} consecutive steps: atom encoder + token "
                            f"transformer + atom decoder, {samples} samples, {tokens} tokens x 768 (16 heads), "
                            f"{atoms} atoms x 128 (4 heads, windows 32 x 128), fp32 as the reference runs them "
                            f"(BASELINE configs[4])",
                "host_model": "stand-in for Boltz's score model: oracle/boltz_ref.py DiffusionStacks (the three "
                              "stacks' upstream module structure, restated) with install() applied; every "
                              "transformer layer, stack and attention runs the patched native forwards, while the "
                              "container's glue (r_to_q and pos_update linears, the stack calls) is the stand-in's "
                              "own torch code and is inside the timed region",
                "samples": samples, "n_tokens": tokens, "n_atoms": atoms, "patched_modules": patched,
                "ms_for_all_steps": round(ms * steps, 2),
                "stack_ms": {k: round(v, 4) for k, v in block_ms.items()}},
               wall_s=round(wall, 3), roofline=roofline, kernels=kernels)
    if not args.no_cpu_baseline:
        out["cpu_baseline"] = cpu_diffusion_step(tokens, steps)
    print(json.dumps(out), flush=True)


def elementwise_kernel_rates(m, d, di, g, dev, reps_min=10):
    """The fused diffusion elementwise kernels at M rows: bmx_adaln (width D),
    bmx_diffusion_epilogue GATED_SWIGLU (width Di) and GATE (width D), each
    launched through the C ABI on preallocated outputs, cycling through input
    sets larger than the 256 MB Infinity Cache, and timed by HIP events.  The
    Python wrappers allocate the output and check the arguments on every call
    (host time longer than these 10-20 us kernels), so they are not in the
    loop.  Bytes per launch: AdaLN 16 M D, GATED_SWIGLU 16 M Di, GATE 12 M D."""
    import torch
    from boltz_lumi_amd import _native as N, ops

    sets = 1 + (768 << 20) // (16 * m * d)
    st = torch.cuda.current_stream().cuda_stream

    def rnd(*shape):
        return torch.randn(*shape, generator=g).to(dev)

    bufs = [{"a": rnd(m, d), "scale": rnd(m, d), "shift": rnd(m, d), "u": rnd(m, 2 * di), "b": rnd(m, di),
             "g": rnd(m, d), "y": rnd(m, d), "out": torch.empty(m, d, device=dev),
             "out_i": torch.empty(m, di, device=dev)} for _ in range(sets)]
    reps = sets * max(1, reps_min // sets + 1)
    # entry point, per-set argument tuples (pointers taken once), bytes per launch
    launches = {
        "adaln": ("bmx_adaln", [(t["a"].data_ptr(), t["scale"].data_ptr(), t["shift"].data_ptr(),
                                 t["out"].data_ptr(), 0, m, d, 1e-5, st) for t in bufs], 16 * m * d),
        "gated_swiglu": ("bmx_diffusion_epilogue", [(ops.GATED_SWIGLU, t["u"].data_ptr(), t["b"].data_ptr(), None,
                                                     t["out_i"].data_ptr(), 0, m, di, st) for t in bufs],
                         16 * m * di),
        "gate": ("bmx_diffusion_epilogue", [(ops.GATE, t["g"].data_ptr(), t["y"].data_ptr(), None,
                                             t["out"].data_ptr(), 0, m, d, st) for t in bufs], 12 * m * d)}
    out = {}
    for name, (entry, arg_sets, nbytes) in launches.items():
        fn = getattr(N.lib(), entry)
        turn = [0]

        def step(fn=fn, arg_sets=arg_sets, entry=entry):
            if fn(*arg_sets[turn[0]]) != 0:
                raise RuntimeError(f"{entry} failed: {N.last_error()}")
            turn[0] = (turn[0] + 1) % sets

        ms, _ = timed_loop(step, reps, sets)
        out[name] = {"ms": round(ms, 4), "bytes": nbytes, "input_sets": sets,
                     **roofline_of(0, nbytes, ms, PEAK_BF16_TFLOPS)}
    return out


def token_attention_launch(q, k, v, bias, mask, g, samples, inf=1e6):
    """The token transformer's attention over `samples` elements sharing one
    bias (bmx_seq_attention_x3_batched_fwd: the K / V split pre-pass and the
    split-bf16 attention) as a step function launching through the C ABI on a
    preallocated output and workspace: the Python wrapper's argument checks and
    allocations are host time that the stacks overlap with earlier kernels.
    Checked once, bit for bit, against the wrapper."""
    import torch
    from boltz_lumi_amd import _native as N, ops

    b, nq, width = q.shape
    nk, heads = k.shape[1], bias.shape[1]
    hd = width // heads
    out = torch.empty(b, nq, width, device=q.device)
    nbytes = N.lib().bmx_seq_attention_x3_workspace_bytes(b, nk, heads, hd)
    ws = torch.empty(nbytes, dtype=torch.uint8, device=q.device)
    args = (q.data_ptr(), k.data_ptr(), v.data_ptr(), bias.data_ptr(), mask.data_ptr(), g.data_ptr(), b, nq, nk,
            q.stride(1), k.stride(1), q.stride(0), k.stride(0), bias.stride(0), mask.stride(0), samples, heads, hd,
            float(inf), out.data_ptr(), ws.data_ptr(), nbytes, torch.cuda.current_stream().cuda_stream)
    fn = N.lib().bmx_seq_attention_x3_batched_fwd

    def step(keep=(out, ws)):
        if fn(*args) != 0:
            raise RuntimeError(f"bmx_seq_attention_x3_batched_fwd failed: {N.last_error()}")

    step()
    if not torch.equal(out, ops.seq_attention_batched(q, k, v, bias, mask, g, inf, bias_div=samples, split=True)):
        raise RuntimeError("C-ABI launch of the token attention differs from the wrapper's")
    return step


def diffusion_kernel_times(stacks, t, packed, samples, tokens):
    """Each fused kernel of one step at the step's shapes, timed alone:
    the token attention (split-bf16 MFMA, 16 x 48), the windowed atom attention
    (4 x 32), AdaLN and the conditioned-transition epilogues at the token
    shape; launches per step count every layer."""
    import torch
    from boltz_lumi_amd import _native as N, ops
    from boltz_lumi_amd.pair_bias import prepare_window_bias

    dev = t["a"].device
    g = torch.Generator().manual_seed(1)
    out = {}

    def rate(name, fn, flops, nbytes, launches, peak=PEAK_FP32_TFLOPS):
        ms, _ = timed_loop(fn, 10, 2)
        out[name] = {"ms": round(ms, 4), "launches_per_step": launches, **roofline_of(flops, nbytes, ms, peak)}

    m, d = samples * tokens, 768
    q = torch.randn(samples, tokens, 4 * d, generator=g).to(dev)
    qq, kk, vv, gg = q.split(d, dim=-1)
    bias = packed[..., :16].movedim(-1, 1)
    mask = torch.ones(samples, tokens, device=dev)
    # split-bf16 by default (the K / V split pre-pass included): 3 bf16 MFMA
    # products per fp32 product, so the executed flops against the bf16 peak
    rate("seq_attention (token, 16 x 48, split-bf16)", token_attention_launch(qq, kk, vv, bias, mask, gg, samples),
         3 * 4.0 * 16 * 48 * tokens * tokens * samples, samples * tokens * d * 16 + 16 * tokens * tokens * 4, 24,
         PEAK_BF16_TFLOPS)
    # the atom transformer's attention as the installed stacks run it: q | k | v | g of the atom rows,
    # each window's 128 keys read by address (keys past a sample's ends absent), and one layer's 4
    # heads of the [1, 256, 32, 128, 12] window bias in place, shared by the samples; HBM bytes:
    # q, k, v, g and out once per atom, the bias slice once
    nw = 8192 // 32
    proj = torch.randn(samples * 8192, 4 * 128, generator=g).to(dev)
    pq, pk, pv, pg = proj.split(128, dim=-1)
    ab = prepare_window_bias(torch.randn(1, nw, 32, 128, 12, generator=g).to(dev))[..., 4:8]
    am = torch.ones(samples * 8192, device=dev)
    # the wrapper's one C-ABI launch (its output, the only buffer it allocates, kept alive) replayed
    calls = []
    real_call = N.call
    N.call = lambda name, *a: (calls.append((name, a)), real_call(name, *a))[1]
    try:
        win_out = ops.seq_attention_windowed(pq.view(samples * nw, 32, 128), pk, pv, ab, am,
                                             pg.view(samples * nw, 32, 128), 1e6, windows=nw, key_offset=-48,
                                             bias_group=samples * nw)
    finally:
        N.call = real_call
    if [c[0] for c in calls] != ["bmx_seq_attention_windowed_fwd"]:
        raise RuntimeError(f"unexpected launches {[c[0] for c in calls]}")
    win_fn, win_args = getattr(N.lib(), calls[0][0]), calls[0][1]

    def win_step(keep=win_out):
        if win_fn(*win_args) != 0:
            raise RuntimeError(f"bmx_seq_attention_windowed_fwd failed: {N.last_error()}")

    rate("seq_attention (atom windows, 4 x 32)", win_step,
         4.0 * 4 * 32 * 32 * 128 * samples * nw, samples * 8192 * 5 * 128 * 4 + nw * 32 * 128 * 4 * 4, 6)
    per_step = {"adaln": 48, "gated_swiglu": 24, "gate": 24}
    for name, rec in elementwise_kernel_rates(m, d, 2 * d, g, dev).items():
        out[f"{name} (token)"] = {"ms": rec["ms"], "launches_per_step": per_step[name],
                                  **{k: rec[k] for k in ("bound", "achieved", "peak", "unit", "frac")}}
    return out


def cpu_diffusion_step(tokens, steps):
    """CPU baseline of configs[4]: one denoiser step of the fp32 oracle
    stacks for one of the 5 samples (x5), reported x``steps`` as
    extrapolated."""
    import torch

    cores = _cpu_setup()
    from oracle import boltz_ref as R

    atoms, w, h = 8192, 32, 128
    nw = atoms // w
    stacks = fan_in_weights(R.DiffusionStacks(), 0).eval()
    g = torch.Generator().manual_seed(0)
    index = R.get_indexing_matrix(nw, w, h)
    args = (torch.randn(1, atoms, 3, generator=g) * 160.0, torch.randn(1, atoms, 128, generator=g),
            torch.randn(1, atoms, 128, generator=g), torch.ones(1, atoms), torch.randn(1, nw, w, h, 12, generator=g),
            torch.randn(1, nw, w, h, 12, generator=g), lambda x: R.single_to_keys(x, index, w, h),
            torch.randn(1, tokens, 768, generator=g), torch.randn(1, tokens, 768, generator=g),
            torch.randn(1, tokens, tokens, 384, generator=g), torch.ones(1, tokens))
    with torch.inference_mode():
        one, _ = _median_ms(lambda: stacks(*args), 1)
    step_ms = 5 * one
    return {"value": round(step_ms, 1), "unit": "ms per step, 5 samples (1 sample timed, x5)", "cores": cores,
            "kind": "port",
            "sample": f"fp32 CPU oracle (oracle/boltz_ref.py DiffusionStacks) one step for one sample at {tokens} "
                      f"tokens / {atoms} atoms, x5 samples, {cores} threads",
            f"{steps}_steps_ms_extrapolated": round(steps * step_ms, 1)}


# ------------------------------------------ single-module diffusion lines


def token_attention(args):
    """One token-transformer AttentionPairBias forward (c_s 768, 16 heads x 48)
    over 5 samples of N tokens sharing one prepacked [1, N, N, 24 * 16] bias
    (BASELINE configs[4] shape, one of the 24 layers), through the drop-in
    ``prepared_forward``.  The roofline covers the fused attention the
    forward runs, the split-bf16 kernel with its K / V pre-pass over the 5
    samples: 3 x 4 * 16 * 48 * N^2 bf16 MFMA flops executed per sample."""
    import torch
    from boltz_lumi_amd import layers, ops
    from boltz_lumi_amd.pair_bias import prepare_token_bias, prepared_forward

    dev = torch.device("cuda:0")
    n, samples, heads, width = args.n or 1024, 5, 16, 768
    steps = args.steps or 10
    module = init_weights(layers.AttentionPairBias(width, num_heads=heads, compute_pair_bias=False), 0).to(dev).eval()
    g = torch.Generator().manual_seed(0)
    s = torch.randn(samples, n, width, generator=g).to(dev)
    bias = prepare_token_bias(torch.randn(1, n, n, 24 * heads, generator=g).to(dev))[..., :heads]
    mask = torch.ones(samples, n, device=dev)
    with torch.inference_mode():
        ms, _ = timed_loop(lambda: prepared_forward(module, s, bias, mask, s, multiplicity=samples), steps,
                           args.warmup)
        proj = torch.randn(samples, n, 4 * width, generator=g).to(dev)
        q, k, v, gl = proj.split(width, dim=-1)
        kms, _ = timed_loop(token_attention_launch(q, k, v, bias.movedim(-1, 1), mask, gl, samples, module.inf),
                            max(steps, 10), 1)
    flops = 3 * 4.0 * heads * 48 * n * n * samples
    out_line = line("token-transformer AttentionPairBias ms @N=1024, 5 samples", ms, "ms", args, steps, "f32",
                    "synthetic (s ~ N(0,1), bias ~ N(0,1) prepacked, masks ones; weights seed 0)",
                    {"workload": f"diffusion token-transformer AttentionPairBias forward (prepared_forward), "
                                 f"c_s=768, 16 heads x 48, {samples} samples x N={n} (BASELINE configs[4] shape)",
                     "n_tokens": n, "samples": samples},
                    roofline={"kernel": "seq_attention_x3 (with its K / V split pre-pass)",
                              **roofline_of(flops, samples * n * width * 16 + n * n * heads * 4, kms,
                                            PEAK_BF16_TFLOPS),
                              "traffic": None, "kernel_ms": round(kms, 4)})
    if not args.no_cpu_baseline:
        out_line["cpu_baseline"] = token_attention_cpu(n)
    print(json.dumps(out_line), flush=True)


def token_attention_cpu(n: int):
    import torch

    cores = _cpu_setup()
    from oracle import boltz_ref as R  # the checker, timed as the reference CPU path

    module = init_weights(R.AttentionPairBias(768, num_heads=16, compute_pair_bias=False), 0).eval()
    g = torch.Generator().manual_seed(0)
    s = torch.randn(1, n, 768, generator=g)
    bias = torch.randn(1, n, n, 16, generator=g)
    mask = torch.ones(1, n)
    with torch.inference_mode():
        one, _ = _median_ms(lambda: module(s, bias, mask, s), 3, warm=lambda: module(s[:, :32], bias[:, :32, :32],
                                                                                        mask[:, :32], s[:, :32]))
    return {"value": round(one * 5, 1), "unit": "ms per 5-sample forward (1 sample timed, x5)", "cores": cores,
            "kind": "port",
            "sample": f"one sample of the fp32 CPU oracle AttentionPairBias at N={n} (oracle/boltz_ref.py), "
                      f"median of 3, {cores} threads, scaled x5"}


def diffusion(args):
    """One token-transformer layer and one atom-transformer layer of the
    score model (AdaLN, AttentionPairBias through prepared_forward,
    ConditionedTransitionBlock) at configs[4] shapes, fp32, plus the fused
    elementwise kernels alone against the 8 TB/s roofline (input sets larger
    than the 256 MB Infinity Cache).  Bytes per launch: AdaLN 16 M D,
    GATED_SWIGLU 16 M Di, GATE 12 M D."""
    import torch
    from boltz_lumi_amd import layers, ops
    from boltz_lumi_amd.pair_bias import prepare_token_bias, prepared_forward

    dev = torch.device("cuda:0")
    samples, n = 5, args.n or 1024
    steps = args.steps or 10
    shapes = {"token": (samples * n, 768, 768), "atom": (samples * 8192, 128, 128)}
    g = torch.Generator().manual_seed(0)
    kernels, blocks = {}, {}
    heads = {"token": 16, "atom": 4}
    modules = {name: (init_weights(layers.AdaLN(d, dc), 0).to(dev).eval(),
                      init_weights(layers.AttentionPairBias(d, num_heads=heads[name], compute_pair_bias=False), 2)
                      .to(dev).eval(),
                      init_weights(layers.ConditionedTransitionBlock(d, dc), 1).to(dev).eval())
               for name, (m, d, dc) in shapes.items()}
    with torch.inference_mode():
        for name, (m, d, dc) in shapes.items():
            di = 2 * d
            adaln, apb, ctb = modules[name]
            a = torch.randn(m, d, generator=g).to(dev)
            c = torch.randn(m, dc, generator=g).to(dev)
            if name == "token":  # 5 samples sharing one prepacked layer bias
                qs = a.view(samples, n, d)
                ks, mult = qs, samples
                z = prepare_token_bias(torch.randn(1, n, n, heads[name], generator=g).to(dev))
                kmask = torch.ones(samples, n, device=dev)
                index = None
            else:  # windows of 32 atoms over 128 keys centred on them (clamped at the ends)
                nw, w, h = 8192 // 32, 32, 128
                index = torch.stack([torch.clamp(torch.arange(h) + w * i - (h - w) // 2, 0, 8191)
                                     for i in range(nw)]).to(dev)
                qs = a.view(samples * nw, w, d)
                ks, mult = a.view(samples, 8192, d)[:, index].reshape(samples * nw, h, d), 1
                z = torch.randn(samples * nw, heads[name], w, h, generator=g).to(dev).movedim(1, -1)
                kmask = torch.ones(samples * nw, h, device=dev)
            gate = init_weights(torch.nn.Linear(dc, d), 3).to(dev)

            def layer(a=a, c=c, qs=qs, z=z, kmask=kmask, mult=mult, index=index, name=name, d=d):
                b = adaln(a, c)
                bq = b.view(qs.shape)
                k_in = bq if name == "token" else b.view(samples, 8192, d)[:, index].reshape(qs.shape[0], 128, d)
                o = prepared_forward(apb, bq, z, kmask, k_in, mult).reshape(a.shape)
                x = a + torch.sigmoid(ops.linear_fp32(c, gate)) * o
                return x + ctb(x, c)

            blocks[name], _ = timed_loop(layer, steps, args.warmup)
            blocks[name + "_attention"], _ = timed_loop(lambda: prepared_forward(apb, qs, z, kmask, ks, mult), steps, 1)
            for kname, rec in elementwise_kernel_rates(m, d, di, g, dev, max(steps, 10)).items():
                kernels[f"{kname}_{name}"] = {"ms": rec["ms"], "bytes": rec["bytes"], "gbs": rec["achieved"],
                                              "frac": rec["frac"], "input_sets": rec["input_sets"]}
    ms = blocks["token"] + blocks["atom"]
    dom = kernels["gated_swiglu_token"]
    out_line = line("diffusion score-model modules (AdaLN + AttentionPairBias + ConditionedTransitionBlock) ms per "
                    "token + atom layer, 5 samples", ms, "ms", args, steps, "f32",
                    "synthetic (activations and conditioning ~ N(0,1); weights seeds 0 and 1)",
                    {"workload": f"one token layer ({samples} x {n} x 768, 16 heads, one shared bias) + one atom "
                                 f"layer ({samples} x 8192 x 128, 4 heads, windows of 32 queries x 128 keys), "
                                 f"BASELINE configs[4] shapes",
                     "n_tokens": n, "n_atoms": 8192, "samples": samples,
                     "block_ms": {k: round(v, 4) for k, v in blocks.items()}},
                    roofline={"kernel": "gated_swiglu (token)", "bound": "hbm", "achieved": dom["gbs"],
                              "peak": PEAK_HBM_GBS, "unit": "GB/s", "frac": dom["frac"], "traffic": None,
                              "kernels": kernels})
    print(json.dumps(out_line), flush=True)


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU only; --gpus must be 1 "
                                   "(multi-GPU sharding of the pair stack is a design note, not built)"}))
        sys.exit(2)
    {"pairformer": pairformer, "dropin": dropin, "trunk": trunk, "trimul": lambda a: isolated_module(a, "trimul"),
     "triattn": lambda a: isolated_module(a, "triattn"), "diffusion-step": diffusion_step,
     "token-attention": token_attention, "diffusion": diffusion}[args.workload](args)


if __name__ == "__main__":
    main()
