#!/usr/bin/env python
"""Benchmark: one Boltz-2 PairformerLayer forward at N=1024 on one MI355X.

Metric: "Pairformer layer ms @N=1024 bf16; tri-attn/mult % of
MFMA/HBM roofline".  A step is one full PairformerLayer forward (v2, eval):
tri_mul_out, tri_mul_in, tri_att_start, tri_att_end, transition_z on the fp32
pair stream with the bf16 gfx950 kernels, then the fp32 sequence stack.  Inputs
(z [1,N,N,128], s [1,N,384], masks all ones) and random-init weights (seed 0,
N(0, 0.08), norm weights N(1, 0.08)) are resident in HBM before timing.

Prints one JSON line.  ``roofline`` covers the kernel with the largest share
of the layer, timed with HIP events on the launch stream; ``breakdown`` lists
every kernel.  ``cpu_baseline`` times the CPU oracle on the host cores for one
layer at --cpu-n (default: the benchmark N) -- a reported baseline only.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

PEAK_BF16_TFLOPS = 2500.0
PEAK_HBM_GBS = 8000.0
# Transcendental issue rate: one 64-lane v_exp_f32 per 8 cycles per SIMD
# (probe on the box), 256 CUs x 4 SIMDs at 2.4 GHz.
EXP_PER_SIMD_CYCLE, SIMDS, CLOCK_HZ = 64 / 8, 1024, 2.4e9


def parse():
    p = argparse.ArgumentParser(description=__doc__)
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=10)
    p.add_argument("--warmup", type=int, default=3)
    p.add_argument("--n", type=int, default=1024)
    p.add_argument("--cpu-n", type=int, default=None, help="token count of the CPU sample (default: --n)")
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--kernel-reps", type=int, default=3, help="repetitions of the per-kernel timing pass")
    p.add_argument("--calibrate-copy", action="store_true",
                   help="first copy 1 GiB device-to-device (a kernel of known traffic for scaling PMC byte counters)")
    p.add_argument("--workload", choices=("pairformer", "token-attention", "diffusion"), default="pairformer",
                   help="pairformer: the headline PairformerLayer line (default); token-attention: the diffusion "
                        "token transformer's AttentionPairBias (16 x 48 heads, 5 samples, prepacked bias); "
                        "diffusion: the score model's AdaLN / ConditionedTransitionBlock forwards and their fused "
                        "kernels at the token and atom transformer shapes")
    return p.parse_args()


def init_weights(module, seed: int):
    import torch

    g = torch.Generator().manual_seed(seed)
    with torch.no_grad():
        for name, p in module.named_parameters():
            mean = 1.0 if "norm" in name and name.endswith("weight") else 0.0
            p.copy_(torch.randn(p.shape, generator=g) * 0.08 + mean)
    return module


def kernel_table(n: int):
    """Algorithmic flops and compulsory HBM bytes per launch, per kernel."""
    n2, n3 = float(n) ** 2, float(n) ** 3
    return {
        # name: (flops, bytes, bound)
        "trimul_proj": (2 * n2 * 128 * 512, n2 * (512 + 4 + 2 * 256), "hbm"),
        "trimul_contract": (2 * 128 * n3, n2 * 128 * 2 * 3, "mfma"),
        "trimul_out": (2 * n2 * 128 * 256, n2 * (256 + 512 + 512), "hbm"),
        "triattn_proj": (2 * n2 * 128 * 388, n2 * (512 + 4 + 3 * 256 + 16), "hbm"),
        "triattn_core": (4 * 4 * 32 * n3, n2 * 4 * 3 * 64 + n2 * 256, "mfma"),
        "triattn_out": (2 * n2 * 128 * 256, n2 * (512 + 256 + 512), "hbm"),
        "pair_transition": (2 * n2 * 128 * (1536 + 16), n2 * (1024 + 64), "hbm"),  # + the fused pair bias
    }


def measured_traffic(kernel: str, n: int):
    """HBM bytes per launch of ``kernel`` from the committed rocprofv3 counter
    summary (FETCH_SIZE / WRITE_SIZE scaled by a 1 GiB copy), when it was
    taken at this N; None otherwise."""
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", f"hbm_traffic_n{n}.json")
    try:
        with open(path) as f:
            data = json.load(f)
    except (OSError, ValueError):
        return None
    return data.get("bytes_per_launch", {}).get(kernel) if data.get("n") == n else None


def per_kernel_times(layer, s, z, mask, pair_mask, z_out, ws, reps):
    """Average ms per launch of every kernel of the layer, from HIP events
    recorded on torch's current stream (the stream the kernels launch on)."""
    import torch
    from boltz_lumi_amd import ops

    zi, zo, mb = z[0], z_out[0], pair_mask[0].float().contiguous()
    plan = []
    for mod, outgoing, first in ((layer.tri_mul_out, True, True), (layer.tri_mul_in, False, False)):
        mode = ops.OUT_RESIDUAL if first else ops.OUT_ACCUMULATE
        src = zi if first else zo
        for stage, name in ((1, "trimul_proj"), (2, "trimul_contract"), (4, "trimul_out")):
            plan.append((name, lambda m=mod, o=outgoing, md=mode, x=src, st=stage:
                         ops.trimul(m, x, mb, o, md, zo, ws, stages=st)))
    for mod, starting in ((layer.tri_att_start, True), (layer.tri_att_end, False)):
        for stage, name in ((1, "triattn_proj"), (2, "triattn_core"), (4, "triattn_out")):
            plan.append((name, lambda m=mod, st_=starting, st=stage:
                         ops.triattn(m, zo, mb, st_, ops.OUT_ACCUMULATE, zo, ws, stages=st)))
    # the transition's epilogue also writes the sequence stack's pair bias, as in PairformerLayer.forward
    bias = torch.empty((1, 16) + zo.shape[:2], device=zo.device)
    pb = (layer.attention.proj_z[0], layer.attention.proj_z[1], bias[0])
    plan.append(("pair_transition", lambda: ops.pair_transition(layer.transition_z, zo, ops.OUT_ACCUMULATE, zo,
                                                                pair_bias=pb)))
    plan.append(("sequence_stack", lambda: layer.sequence_stack(s, z_out, mask, pair_bias=bias)))
    totals = {}
    counts = {}
    for _ in range(reps):
        events = []
        for name, fn in plan:
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            fn()
            e1.record()
            events.append((name, e0, e1))
        torch.cuda.synchronize()
        for name, e0, e1 in events:
            totals[name] = totals.get(name, 0.0) + e0.elapsed_time(e1)
            counts[name] = counts.get(name, 0) + 1
    return {k: (totals[k] / counts[k], counts[k] // reps) for k in totals}


def cpu_baseline(n: int, seed: int):
    import torch

    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
    from oracle import boltz_ref as R  # the checker, timed as the reference CPU path

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    layer = init_weights(R.PairformerLayer(), seed).eval()
    g = torch.Generator().manual_seed(seed)
    z = torch.randn(1, n, n, 128, generator=g)
    s = torch.randn(1, n, 384, generator=g)
    mask, pm = torch.ones(1, n), torch.ones(1, n, n)
    with torch.inference_mode():
        layer(s[:, :32], z[:, :32, :32], mask[:, :32], pm[:, :32, :32], chunk_size_tri_attn=32)  # thread warm-up
        t0 = time.perf_counter()
        layer(s, z, mask, pm, chunk_size_tri_attn=64)
        dt = time.perf_counter() - t0
    return dt * 1e3, cores


PEAK_FP32_TFLOPS = 157.3


def token_attention(args):
    """One token-transformer AttentionPairBias forward (c_s 768, 16 heads x 48)
    over 5 samples of N tokens sharing one prepacked [1, N, N, 24 * 16] bias
    (BASELINE configs[4] shape, one of the 24 layers), through the drop-in
    ``prepared_forward``.  The roofline covers the fused attention kernel: fp32
    MFMA flops 4 * 16 * 48 * N^2 per sample."""
    import torch
    from boltz_lumi_amd import layers, ops
    from boltz_lumi_amd.pair_bias import prepare_token_bias, prepared_forward

    dev = torch.device("cuda:0")
    n, samples, heads, width = args.n, 5, 16, 768
    module = init_weights(layers.AttentionPairBias(width, num_heads=heads, compute_pair_bias=False), 0).to(dev).eval()
    g = torch.Generator().manual_seed(0)
    s = torch.randn(samples, n, width, generator=g).to(dev)
    bias = prepare_token_bias(torch.randn(1, n, n, 24 * heads, generator=g).to(dev))[..., :heads]
    mask = torch.ones(samples, n, device=dev)

    def step():
        prepared_forward(module, s, bias, mask, s, multiplicity=samples)

    with torch.inference_mode():
        for _ in range(args.warmup):
            step()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(args.steps):
            step()
        e1.record()
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / args.steps
        # the attention kernel alone, on the same inputs
        proj = torch.randn(n, 4 * width, generator=g).to(dev)
        q, k, v, gl = proj.split(width, dim=-1)
        b0, m0 = bias[0].movedim(-1, 0), mask[0]
        out = torch.empty(n, width, device=dev)
        reps = max(args.steps, 10) * samples
        ops.seq_attention(q, k, v, b0, m0, gl, module.inf, out=out)
        e0.record()
        for _ in range(reps):
            ops.seq_attention(q, k, v, b0, m0, gl, module.inf, out=out)
        e1.record()
        torch.cuda.synchronize()
        kms = e0.elapsed_time(e1) / reps
    flops = 4.0 * heads * 48 * n * n
    achieved = flops / (kms * 1e-3) / 1e12
    out_line = {
        "metric": "token-transformer AttentionPairBias ms @N=1024, 5 samples",
        "value": round(ms, 4), "unit": "ms", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(ms, 4), "higher_is_better": False, "scaling": "weak", "vs_baseline": None,
        "dtype": "f32", "data": "synthetic (s ~ N(0,1), bias ~ N(0,1) prepacked, masks ones; weights seed 0)",
        "config": {"workload": f"diffusion token-transformer AttentionPairBias forward (prepared_forward), "
                               f"c_s=768, 16 heads x 48, {samples} samples x N={n} (BASELINE configs[4] shape)",
                   "n_tokens": n, "samples": samples},
        "roofline": {"kernel": "seq_attention", "bound": "mfma", "achieved": round(achieved, 2),
                     "peak": PEAK_FP32_TFLOPS, "unit": "TFLOP/s", "frac": round(achieved / PEAK_FP32_TFLOPS, 4),
                     "traffic": None, "kernel_ms_per_sample": round(kms, 4)},
    }
    if not args.no_cpu_baseline:
        out_line["cpu_baseline"] = token_attention_cpu(min(n, args.cpu_n or n))
    print(json.dumps(out_line), flush=True)


def token_attention_cpu(n: int):
    import torch

    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
    from oracle import boltz_ref as R  # the checker, timed as the reference CPU path

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    module = init_weights(R.AttentionPairBias(768, num_heads=16, compute_pair_bias=False), 0).eval()
    g = torch.Generator().manual_seed(0)
    s = torch.randn(1, n, 768, generator=g)
    bias = torch.randn(1, n, n, 16, generator=g)
    mask = torch.ones(1, n)
    with torch.inference_mode():
        module(s[:, :32], bias[:, :32, :32], mask[:, :32], s[:, :32])
        t0 = time.perf_counter()
        module(s, bias, mask, s)
        dt = time.perf_counter() - t0
    return {"value": round(dt * 1e3 * 5, 1), "unit": "ms per 5-sample forward (1 sample timed, x5)",
            "cores": cores, "kind": "port",
            "sample": f"one sample of the fp32 CPU oracle AttentionPairBias at N={n} (oracle/boltz_ref.py), "
                      f"{cores} threads, scaled x5"}


def diffusion(args):
    """The diffusion score model's per-layer modules at BASELINE configs[4]
    shapes (5 samples; token transformer 1024 tokens x 768 with 16 heads,
    atom transformer 8192 atoms x 128 with 4 heads in windows of 32 queries
    over 128 keys): the AdaLN, AttentionPairBias (prepared_forward, the fused
    batched attention) and ConditionedTransitionBlock forwards of one layer of
    each transformer, fp32 as the reference runs them (diffusion.py:37-68,
    pair_bias.py:15-36), plus the fused elementwise kernels alone (bmx_adaln,
    the GATED_SWIGLU and GATE epilogues) against the 8 TB/s HBM roofline.
    Bytes per launch: AdaLN 16 M D (a, scale, shift in, out), GATED_SWIGLU
    16 M Di (u [M, 2 Di] and b in, out), GATE 12 M D."""
    import torch
    from boltz_lumi_amd import layers, ops
    from boltz_lumi_amd.pair_bias import prepare_token_bias, prepared_forward

    dev = torch.device("cuda:0")
    samples = 5
    shapes = {"token": (samples * args.n, 768, 768), "atom": (samples * 8192, 128, 128)}
    g = torch.Generator().manual_seed(0)

    def timed(fn, reps):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        fn()
        torch.cuda.synchronize()
        e0.record()
        for _ in range(reps):
            fn()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / reps

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
                qs = a.view(samples, args.n, d)
                ks, mult = qs, samples
                z = prepare_token_bias(torch.randn(1, args.n, args.n, heads[name], generator=g).to(dev))
                kmask = torch.ones(samples, args.n, device=dev)
            else:  # windows of 32 atoms over the 128 atoms centred on them (to_keys)
                nw, w, h = 8192 // 32, 32, 128
                index = torch.stack([torch.clamp(torch.arange(h) + w * i - (h - w) // 2, 0, 8191)
                                     for i in range(nw)]).to(dev)
                qs = a.view(samples * nw, w, d)
                ks, mult = a.view(samples, 8192, d)[:, index].reshape(samples * nw, h, d), 1
                z = torch.randn(samples * nw, heads[name], w, h, generator=g).to(dev).movedim(1, -1)
                kmask = torch.ones(samples * nw, h, device=dev)

            gate = init_weights(torch.nn.Linear(dc, d), 3).to(dev)

            def layer():  # upstream DiffusionTransformerLayer.forward
                b = adaln(a, c)
                bq = b.view(qs.shape)
                if name == "token":
                    k_in = bq
                else:
                    k_in = b.view(samples, 8192, d)[:, index].reshape(samples * nw, h, d)
                o = prepared_forward(apb, bq, z, kmask, k_in, mult).reshape(a.shape)
                x = a + torch.sigmoid(ops.linear_fp32(c, gate)) * o
                return x + ctb(x, c)

            for _ in range(args.warmup):
                layer()
            torch.cuda.synchronize()
            blocks[name] = timed(layer, args.steps)
            blocks[name + "_attention"] = timed(lambda: prepared_forward(apb, qs, z, kmask, ks, mult), args.steps)
            # Each kernel cycles over enough input sets that successive launches
            # do not find their operands in the 256 MB Infinity Cache.
            sets = 1 + (768 << 20) // (16 * m * d)
            bufs = [{"a": torch.randn(m, d, generator=g).to(dev), "scale": torch.randn(m, d, generator=g).to(dev),
                     "shift": torch.randn(m, d, generator=g).to(dev), "u": torch.randn(m, 2 * di, generator=g).to(dev),
                     "b": torch.randn(m, di, generator=g).to(dev), "g": torch.randn(m, d, generator=g).to(dev),
                     "y": torch.randn(m, d, generator=g).to(dev)} for _ in range(sets)]
            reps = sets * max(1, max(args.steps, 10) // sets)
            turn = [0]

            def nxt():
                turn[0] = (turn[0] + 1) % sets
                return bufs[turn[0]]

            for kname, fn, nbytes in (
                    ("adaln", lambda: (lambda t: ops.adaln_modulate(t["a"], t["scale"], t["shift"], 1e-5))(nxt()),
                     16 * m * d),
                    ("gated_swiglu", lambda: (lambda t: ops.epilogue(t["u"], t["b"], None, ops.GATED_SWIGLU))(nxt()),
                     16 * m * di),
                    ("gate", lambda: (lambda t: ops.epilogue(t["g"], t["y"], None, ops.GATE))(nxt()), 12 * m * d)):
                ms = timed(fn, reps)
                gbs = nbytes / (ms * 1e-3) / 1e9
                kernels[f"{kname}_{name}"] = {"ms": round(ms, 4), "bytes": nbytes, "gbs": round(gbs, 1),
                                              "frac": round(gbs / PEAK_HBM_GBS, 4), "input_sets": sets}
            del bufs
    ms = blocks["token"] + blocks["atom"]
    dom = kernels["gated_swiglu_token"]
    out_line = {
        "metric": "diffusion score-model modules (AdaLN + AttentionPairBias + ConditionedTransitionBlock) ms per "
                  "token + atom layer, 5 samples; AdaLN/gating kernels % of HBM roofline",
        "value": round(ms, 4), "unit": "ms", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(ms, 4), "higher_is_better": False, "scaling": "weak", "vs_baseline": None,
        "dtype": "f32", "data": "synthetic (activations and conditioning ~ N(0,1); weights seeds 0 and 1)",
        "config": {"workload": f"diffusion score-model AdaLN + AttentionPairBias + ConditionedTransitionBlock "
                               f"forwards, token layer ({samples} x {args.n} x 768, 16 heads, one shared bias) + "
                               f"atom layer ({samples} x 8192 x 128, 4 heads, windows of 32 queries x 128 keys), "
                               f"BASELINE configs[4] shapes",
                   "n_tokens": args.n, "n_atoms": 8192, "samples": samples,
                   "block_ms": {k: round(v, 4) for k, v in blocks.items()}},
        "roofline": {"kernel": "gated_swiglu (token)", "bound": "hbm", "achieved": dom["gbs"], "peak": PEAK_HBM_GBS,
                     "unit": "GB/s", "frac": dom["frac"], "traffic": None, "kernels": kernels},
    }
    if not args.no_cpu_baseline:
        out_line["cpu_baseline"] = diffusion_cpu(args.n)
    print(json.dumps(out_line), flush=True)


def diffusion_cpu(n: int):
    import torch

    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
    from oracle import boltz_ref as R  # the checker, timed as the reference CPU path

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    g = torch.Generator().manual_seed(0)
    total = 0.0
    with torch.inference_mode():
        for m, d, heads in ((n, 768, 16), (8192, 128, 4)):
            layer = init_weights(R.DiffusionTransformerLayer(heads, d, d), 0).eval()
            a, c = torch.randn(1, m, d, generator=g), torch.randn(1, m, d, generator=g)
            if d == 768:
                z, mask, to_keys, a, c = torch.randn(1, m, m, heads, generator=g), torch.ones(1, m), None, a, c
            else:  # windows of 32 atoms over the 128 atoms centred on them
                nw, w, h = m // 32, 32, 128
                index = torch.stack([torch.clamp(torch.arange(h) + w * i - (h - w) // 2, 0, m - 1) for i in range(nw)])
                to_keys = lambda x: x.view(1, m, -1)[:, index].reshape(nw, h, -1)
                z, mask = torch.randn(nw, w, h, heads, generator=g), torch.ones(nw, w)
                a, c = a.view(nw, w, d), c.view(nw, w, d)
            t0 = time.perf_counter()
            layer(a, c, bias=z, mask=mask, to_keys=to_keys)
            total += time.perf_counter() - t0
    return {"value": round(total * 1e3 * 5, 1), "unit": "ms per token + atom layer, 5 samples (1 sample timed, x5)",
            "cores": cores, "kind": "port",
            "sample": f"one sample of the fp32 CPU oracle DiffusionTransformerLayer (oracle/boltz_ref.py) at {n} "
                      f"tokens x 768 (16 heads) and 8192 atoms x 128 (4 heads, 32 x 128 windows), {cores} threads, "
                      f"scaled x5"}


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU only; --gpus must be 1 "
                                   "(multi-GPU sharding of the pair stack is a design note, not built)"}))
        sys.exit(2)
    if args.workload == "token-attention":
        return token_attention(args)
    if args.workload == "diffusion":
        return diffusion(args)
    import torch
    from boltz_lumi_amd import layers, ops

    dev = torch.device("cuda:0")
    n = args.n
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

    def step():
        layer(s, z, mask, pair_mask, z_out=z_out, workspace=ws)

    with torch.inference_mode():
        for _ in range(args.warmup):
            step()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        wall0 = time.perf_counter()
        e0.record()
        for _ in range(args.steps):
            step()
        e1.record()
        torch.cuda.synchronize()
        wall = time.perf_counter() - wall0
        ms = e0.elapsed_time(e1) / args.steps
        kt = per_kernel_times(layer, s, z, mask, pair_mask, z_out, ws, args.kernel_reps)

    table = kernel_table(n)
    breakdown = {}
    for name, (avg_ms, launches) in kt.items():
        entry = {"ms": round(avg_ms, 4), "launches_per_layer": launches}
        if name in table:
            flops, nbytes, bound = table[name]
            entry["tflops"] = round(flops / (avg_ms * 1e-3) / 1e12, 2)
            entry["gbs"] = round(nbytes / (avg_ms * 1e-3) / 1e9, 1)
            entry["bound"] = bound
            entry["frac"] = round(entry["tflops"] / PEAK_BF16_TFLOPS if bound == "mfma"
                                  else entry["gbs"] / PEAK_HBM_GBS, 4)
        breakdown[name] = entry
    dominant = max((k for k in breakdown if k in table),
                   key=lambda k: breakdown[k]["ms"] * breakdown[k]["launches_per_layer"])
    d = breakdown[dominant]
    roofline = {
        "kernel": dominant,
        "bound": d["bound"],
        "achieved": d["tflops"] if d["bound"] == "mfma" else d["gbs"],
        "peak": PEAK_BF16_TFLOPS if d["bound"] == "mfma" else PEAK_HBM_GBS,
        "unit": "TFLOP/s" if d["bound"] == "mfma" else "GB/s",
        "frac": d["frac"],
        "traffic": measured_traffic(dominant, n),
    }
    if dominant == "triattn_core":
        # Exp co-bound (H N^3 exponentials per direction): v_exp_f32 issues one
        # wave instruction per 8 cycles per SIMD (measured on the box), and MFMA
        # and VALU issue overlap little, so the core's issue floor is the sum.
        exps = 4.0 * n ** 3
        exp_ms = exps / (EXP_PER_SIMD_CYCLE * SIMDS * CLOCK_HZ) * 1e3
        mfma_ms = table[dominant][0] / (PEAK_BF16_TFLOPS * 1e12) * 1e3
        roofline["co_bound"] = {"exp_ms": round(exp_ms, 4), "mfma_ms": round(mfma_ms, 4),
                                "issue_floor_ms": round(exp_ms + mfma_ms, 4),
                                "issue_floor_frac": round((exp_ms + mfma_ms) / d["ms"], 4)}
    out = {
        "metric": "Pairformer layer ms @N=1024 bf16",
        "value": round(ms, 4),
        "unit": "ms",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (z, s ~ N(0,1); masks ones; random-init weights seed 0)",
        "config": {"workload": f"PairformerLayer forward, N={n}, c_z=128, c_s=384, tri-att 4x32, "
                               f"tri-mult 128, transition x4, single attention 16 heads (BASELINE configs[3], "
                               f"one of 64 blocks)", "n_tokens": n, "batch": 1},
        "wall_s": round(wall, 3),
        "roofline": roofline,
        "breakdown": breakdown,
    }
    if not args.no_cpu_baseline:
        cpu_n = args.cpu_n or n
        cpu_ms, cores = cpu_baseline(cpu_n, 0)
        out["cpu_baseline"] = {
            "value": round(cpu_ms, 1),
            "unit": "ms per layer",
            "cores": cores,
            "kind": "port",
            "sample": f"one PairformerLayer forward at N={cpu_n}, fp32 CPU oracle (oracle/boltz_ref.py), "
                      f"tri-attention chunked 64 rows, {cores} threads",
        }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
