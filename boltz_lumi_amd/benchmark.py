"""A/B harness: upstream forwards against the native ones, same inputs, same seeds.

Reference: src/boltz_lumi/benchmark.py.  The model-independent part is
:class:`ABRecorder` (per-call timing with GPU-event stage timers, peak memory,
finiteness and the comparison of every output with the first upstream call
of the same candidate, the ``timings.json`` report), driven either by
:func:`ab_benchmark` (any model and step callable) or by :func:`main`, which
binds it to Boltz's ``predict`` CLI as the reference does
(benchmark.py:273-325; Boltz 2.2.1 and pytorch_lightning required).

Report schema (reference benchmark.py:56-150, 197-214): the run settings,
``torch`` / ``hip`` / ``gpu``, ``model_calls`` (recipe, iteration, first,
profiled, candidate, model_s, peak_allocated_bytes, stages_s), ``rounds``
(recipe, iteration, candidates, round_s), ``errors`` (recipe, iteration,
candidate, field, max_absolute_error, relative_l2_error, atol, rtol,
failing_values), ``upstream_warm_mean_s`` / ``optimized_warm_mean_s``,
``saved_s``, ``saved_percent`` and ``status`` (running / complete /
numerical_difference / failed, with ``error``).

One difference on purpose: the native kernels compute in bf16 with their own
summation order, so an output counts as failing where
``|x - upstream| > atol + rtol * |upstream|`` (default 1e-2 each, the
end-to-end bar of the port); the reference counts every value that is not
bit-identical (atol = rtol = 0, which ``--atol 0 --rtol 0`` restores).
"""

from __future__ import annotations

import argparse
import json
import math
import os
import random
import statistics
import time
from contextlib import ExitStack, contextmanager
from pathlib import Path
from unittest.mock import patch

import numpy as np
import torch

from .adapters import install

RECIPES = ("upstream", "optimized")
ATOL = 1e-2
RTOL = 1e-2

# Module paths timed as stages, plus the structure module's ``sample``
# (reference benchmark.py:36-52).
STAGES = (
    "input_embedder",
    "template_module",
    "msa_module",
    "pairformer_module",
    "diffusion_conditioning",
    "confidence_module",
)

# Prediction outputs compared between the recipes (reference benchmark.py:108-127).
FIELDS = (
    "coords",
    "plddt",
    "confidence_score",
    "ptm",
    "iptm",
    "complex_plddt",
    "ligand_iptm",
    "protein_iptm",
    "affinity_pred_value",
    "affinity_probability_binary",
    "affinity_pred_value1",
    "affinity_pred_value2",
    "affinity_probability_binary1",
    "affinity_probability_binary2",
)

# Fields of a confidence summary file (reference benchmark.py:243-246).
CONFIDENCE_FIELDS = (
    "confidence_score", "ptm", "iptm", "ligand_iptm", "protein_iptm",
    "complex_plddt", "complex_iplddt", "complex_pde", "complex_ipde",
)


def seed_all(seed: int) -> None:
    """Seed Python, NumPy and torch (all devices) with one value."""
    random.seed(seed)
    np.random.seed(seed % 2**32)
    torch.manual_seed(seed)


@contextmanager
def stage_timers(model, events: list):
    """Time the stage modules' forwards and ``structure_module.sample`` with GPU
    events on the current stream; each call appends ``(name, start, end)`` to
    ``events``.  The wrappers are removed on exit (instance attributes that
    existed before, such as an installed ``sample``, are restored)."""

    def wrap(original, name):
        def timed(*args, **kwargs):
            start = torch.cuda.Event(enable_timing=True)
            end = torch.cuda.Event(enable_timing=True)
            start.record()
            try:
                with torch.profiler.record_function(name):
                    return original(*args, **kwargs)
            finally:
                end.record()
                events.append((name, start, end))

        return timed

    with ExitStack() as stack:
        for name, module in model.named_modules():
            if name in STAGES:
                stack.enter_context(patch.object(module, "forward", wrap(module.forward, name)))
        sampler = getattr(model, "structure_module", None)
        if sampler is not None and hasattr(sampler, "sample"):
            stack.enter_context(patch.object(sampler, "sample", wrap(sampler.sample, "diffusion_sample")))
        yield


def compare(value: torch.Tensor, expected: torch.Tensor, atol: float, rtol: float) -> dict:
    """Error record of one output field against its upstream value."""
    value, expected = value.double(), expected.double()
    delta = value - expected
    denominator = expected.norm().item()
    failing = ~(delta.abs() <= atol + rtol * expected.abs())
    return dict(
        max_absolute_error=delta.abs().max().item() if delta.numel() else 0.0,
        relative_l2_error=delta.norm().item() / denominator if denominator else None,
        atol=atol,
        rtol=rtol,
        failing_values=int(failing.sum()),
    )


class ABRecorder:
    """Accumulates the report of one A/B run (reference benchmark.py:56-150)."""

    def __init__(self, model, *, seed: int, atol: float = ATOL, rtol: float = RTOL, fields=FIELDS,
                 settings=None, output: Path | None = None):
        self.model = model
        self.seed = seed
        self.atol, self.rtol = atol, rtol
        self.fields = tuple(fields)
        self.output = None if output is None else Path(output)
        self.report = dict(
            settings or {},
            seed=seed,
            torch=torch.__version__,
            hip=torch.version.hip,
            gpu=torch.cuda.get_device_name(0) if torch.cuda.is_available() else None,
            slurm_job=os.environ.get("SLURM_JOB_ID"),
            model_calls=[],
            rounds=[],
            errors=[],
            status="running",
        )
        self.references = {}
        self.events = []
        self.current = {}

    def save(self) -> None:
        if self.output is not None:
            self.output.mkdir(parents=True, exist_ok=True)
            (self.output / "timings.json").write_text(json.dumps(self.report, indent=2) + "\n")

    def measured_call(self, candidate: str, call, *args, **kwargs):
        """Run one model call with the seed reset, time it and compare its
        outputs with the first upstream call of ``candidate``."""
        seed_all(self.seed)
        self.events.clear()
        torch.cuda.synchronize()
        torch.cuda.reset_peak_memory_stats()
        begin = time.perf_counter()
        output = call(*args, **kwargs)
        torch.cuda.synchronize()
        elapsed = time.perf_counter() - begin
        if output.get("exception"):
            raise RuntimeError("Prediction failed; inspect the preceding log")
        stages = {}
        for name, start, end in self.events:
            stages[name] = stages.get(name, 0.0) + start.elapsed_time(end) / 1000
        self.report["model_calls"].append(dict(
            self.current,
            candidate=candidate,
            model_s=elapsed,
            peak_allocated_bytes=torch.cuda.max_memory_allocated(),
            stages_s=stages,
        ))
        values = {k: output[k].detach().cpu() for k in self.fields if k in output}
        bad = [k for k, v in values.items() if not torch.isfinite(v).all()]
        if bad:
            raise RuntimeError(f"Nonfinite prediction: {', '.join(bad)}")
        expected = self.references.setdefault(candidate, values)
        if expected.keys() != values.keys():
            raise RuntimeError(f"Output fields changed for {candidate}")
        for key, value in values.items():
            if value.shape != expected[key].shape:
                raise RuntimeError(f"Output shape of {key} changed for {candidate}")
            self.report["errors"].append(dict(
                self.current, candidate=candidate, field=key,
                **compare(value, expected[key], self.atol, self.rtol)))
        return output

    def run_round(self, recipe: str, iteration: int, body, candidates, profiled: bool = False):
        """Run ``body()`` (which makes the model calls of one round) and check
        that it called every candidate once, in order."""
        self.current.update(recipe=recipe, iteration=iteration, first=iteration == 0, profiled=profiled)
        seed_all(self.seed)
        before = len(self.report["model_calls"])
        torch.cuda.synchronize()
        begin = time.perf_counter()
        result = body()
        torch.cuda.synchronize()
        elapsed = time.perf_counter() - begin
        called = [c["candidate"] for c in self.report["model_calls"][before:]]
        if called != list(candidates):
            raise RuntimeError("Missing or reordered prediction calls")
        self.report["rounds"].append(dict(self.current, candidates=list(candidates), round_s=elapsed))
        self.save()
        return result

    def finish(self) -> dict:
        """Warm means, savings and status; raises when outputs differ beyond
        the tolerance (the report is saved first)."""
        report = self.report
        for recipe in RECIPES:
            warm = [c["model_s"] for c in report["model_calls"]
                    if c["recipe"] == recipe and not c["first"] and not c["profiled"]]
            if warm:
                report[recipe + "_warm_mean_s"] = statistics.mean(warm)
        upstream = report.get("upstream_warm_mean_s")
        optimized = report.get("optimized_warm_mean_s")
        if upstream and optimized is not None:
            report.update(saved_s=upstream - optimized, saved_percent=100 * (upstream - optimized) / upstream)
        differs = any(e["failing_values"] for e in report["errors"])
        report["status"] = "numerical_difference" if differs else "complete"
        self.save()
        if differs:
            raise RuntimeError("Predictions differ; see timings.json for absolute and relative errors")
        return report

    def fail(self, error: BaseException) -> None:
        self.report.update(status="failed", error=str(error))
        self.save()


def profile_round(run, output: Path | None):
    """One profiled round under ``torch.profiler``: a Chrome trace and the 20
    entries with the most GPU self time (reference benchmark.py:180-196)."""
    activities = [torch.profiler.ProfilerActivity.CPU, torch.profiler.ProfilerActivity.CUDA]
    with torch.profiler.profile(activities=activities) as profiler:
        run()
    if output is None:
        return
    profiler.export_chrome_trace(str(output / "trace.json"))
    entries = sorted(profiler.key_averages(), key=lambda e: e.self_device_time_total, reverse=True)
    lines = ["Operator or kernel                         GPU self seconds    Calls"]
    lines += [f"{e.key[:42]:42} {e.self_device_time_total / 1e6:15.6f} {e.count:8}" for e in entries[:20]]
    (output / "profile.txt").write_text("\n".join(lines) + "\n")


def ab_benchmark(model, step, candidates, *, repeats: int = 3, seed: int = 42, atol: float = ATOL,
                 rtol: float = RTOL, fields=FIELDS, output=None, profile: bool = False, settings=None,
                 install_kwargs=None) -> dict:
    """Upstream rounds, then ``install(model)`` and optimized rounds, each of
    ``repeats`` warm rounds after one first round, over ``candidates`` (pairs
    of ``(id, batch)``); ``step(model, batch)`` makes one model call and
    returns a dict of output tensors.  Returns the report (also written to
    ``output/timings.json`` when ``output`` is given)."""
    if repeats < 1:
        raise ValueError("Use at least one warm repeat")
    candidates = list(candidates)
    ids = [c for c, _ in candidates]
    if len(set(ids)) != len(ids):
        raise ValueError("Candidate ids must be unique")
    recorder = ABRecorder(model, seed=seed, atol=atol, rtol=rtol, fields=fields, settings=settings,
                          output=output)

    def body():
        for candidate, batch in candidates:
            recorder.measured_call(candidate, step, model, batch)

    try:
        for recipe in RECIPES:
            if recipe == "optimized":
                install(model, **(install_kwargs or {}))
            with stage_timers(model, recorder.events):
                for iteration in range(repeats + 1):
                    recorder.run_round(recipe, iteration, body, ids)
        if profile:
            with stage_timers(model, recorder.events):
                profile_round(lambda: recorder.run_round(RECIPES[-1], repeats + 1, body, ids, True),
                              recorder.output)
        return recorder.finish()
    except BaseException as error:
        if recorder.report["status"] == "running":
            recorder.fail(error)
        raise


def validate_outputs(directory, candidates, samples, output_format="mmcif", affinity=False):
    """Every candidate has its structure files and finite confidence (or
    affinity) summaries (reference benchmark.py:249-270)."""
    directory = Path(directory)
    if not candidates:
        raise RuntimeError("No inputs were predicted")
    suffix = ".pdb" if output_format == "pdb" else ".cif"
    for candidate in candidates:
        for rank in range(1 if affinity else samples):
            stem = f"{candidate}_model_{rank}"
            if affinity:
                summary = directory / candidate / f"affinity_{candidate}.json"
                fields = ("affinity_pred_value", "affinity_probability_binary")
            else:
                structure = directory / candidate / (stem + suffix)
                if not structure.is_file() or structure.stat().st_size == 0:
                    raise RuntimeError(f"Missing output for {stem}")
                summary = directory / candidate / f"confidence_{stem}.json"
                fields = CONFIDENCE_FIELDS
            if not summary.is_file():
                raise RuntimeError(f"Missing output for {stem}")
            values = json.loads(summary.read_text())
            for key in fields:
                value = values.get(key)
                if isinstance(value, bool) or not isinstance(value, (int, float)) or not math.isfinite(value):
                    raise RuntimeError(f"Invalid confidence summary for {stem}")


def _boltz_predict(args, settings_base):
    """``Trainer.predict`` replacement that runs the A/B rounds over Boltz's
    own preprocessed batches (reference benchmark.py:55-240, 300-320)."""
    from boltz.data.write.writer import BoltzAffinityWriter, BoltzWriter
    from torch.utils.data import DataLoader

    from .__main__ import InferenceAdapter

    def predict(original, trainer, model, *positional, **keywords):
        writers = [c for c in trainer.callbacks if isinstance(c, (BoltzWriter, BoltzAffinityWriter))]
        if len(writers) != 1:
            raise RuntimeError("Expected one Boltz prediction writer")
        writer = writers[0]
        phase = "affinity" if isinstance(writer, BoltzAffinityWriter) else "structure"
        output = writer.output_dir.parent / "benchmark" / phase
        output.mkdir(parents=True)
        samples = model.predict_args["diffusion_samples"]
        settings = dict(settings_base, phase=phase, prediction_settings=model.predict_args)
        recorder = ABRecorder(model, seed=args.seed, atol=args.atol, rtol=args.rtol, settings=settings,
                              output=output)
        datamodule = keywords["datamodule"]
        started = time.perf_counter()
        batches = list(datamodule.predict_dataloader())  # the same features for every round
        ids = [record.id for batch in batches for record in batch["record"]]
        if ids != [r.id for r in datamodule.manifest.records]:
            raise RuntimeError("Prediction loader changed candidate identity or order")
        recorder.report["feature_load_s"] = time.perf_counter() - started
        step = model.predict_step
        normal_output = writer.output_dir
        adapter = InferenceAdapter(optimize=False)  # --no_kernels and failure checks only
        trainer.callbacks.append(adapter)

        def measured_step(batch, *a, **kw):
            if len(batch["record"]) != 1:
                raise RuntimeError("Only one input per model call is supported")
            return recorder.measured_call(batch["record"][0].id, step, batch, *a, **kw)

        def one_round(recipe, iteration, profiled=False):
            final = recipe == "optimized" and iteration == args.repeats and not profiled
            # The last optimized round writes where Boltz's affinity stage reads.
            writer.output_dir = normal_output if final else (
                output / recipe / ("profile" if profiled else f"round-{iteration:02}"))
            writer.output_dir.mkdir(parents=True, exist_ok=True)

            def body():
                return original(trainer, model, *positional, **keywords)

            result = recorder.run_round(recipe, iteration, body, ids, profiled)
            validate_outputs(writer.output_dir, ids, samples,
                             output_format=getattr(writer, "output_format", "mmcif"),
                             affinity=phase == "affinity")
            return result

        result = None
        try:
            with patch.object(datamodule, "predict_dataloader",
                              lambda: DataLoader(batches, batch_size=None, num_workers=0)), \
                    patch.object(model, "predict_step", measured_step):
                for recipe in RECIPES:
                    if recipe == "optimized":
                        install(model)
                    with stage_timers(model, recorder.events):
                        for iteration in range(args.repeats + 1):
                            result = one_round(recipe, iteration)
                if args.profile:
                    with stage_timers(model, recorder.events):
                        profile_round(lambda: one_round(RECIPES[-1], args.repeats + 1, True), output)
            recorder.finish()
        except BaseException as error:
            if recorder.report["status"] == "running":
                recorder.fail(error)
            raise
        finally:
            writer.output_dir = normal_output
            trainer.callbacks.remove(adapter)
        print(output / "timings.json")
        return result

    return predict


def main(arguments=None):
    """``python -m boltz_lumi_amd.benchmark predict input.yaml [Boltz options]
    [--repeats R] [--profile] [--atol A] [--rtol R]``."""
    from .__main__ import require_boltz

    parser = argparse.ArgumentParser(description=__doc__.splitlines()[0], allow_abbrev=False)
    parser.add_argument("--repeats", type=int, default=3)
    parser.add_argument("--profile", action="store_true")
    parser.add_argument("--atol", type=float, default=ATOL)
    parser.add_argument("--rtol", type=float, default=RTOL)
    args, rest = parser.parse_known_args(arguments)
    if args.repeats < 1:
        parser.error("Use at least one warm repeat")
    found = require_boltz()
    if torch.cuda.device_count() != 1:
        raise RuntimeError("Run the comparison with one visible GPU")
    from boltz.main import cli
    from pytorch_lightning import Trainer

    if rest[:1] == ["predict"]:
        rest.pop(0)
    with cli.commands["predict"].make_context("predict", list(rest)) as context:
        options = context.params
    args.seed = options["seed"] if options["seed"] is not None else 42
    rest += ["--seed", str(args.seed), "--no_kernels"]
    settings = dict(boltz=found, input=str(options["data"]), seed=args.seed)
    ab = _boltz_predict(args, settings)
    original = Trainer.predict

    def predict(trainer, model, *positional, **keywords):
        return ab(original, trainer, model, *positional, **keywords)

    with patch.object(Trainer, "predict", predict):
        cli(["predict", *rest], standalone_mode=False)


if __name__ == "__main__":
    main()
