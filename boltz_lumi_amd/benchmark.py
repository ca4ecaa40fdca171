"""A/B timing of Boltz inference: upstream forwards against this package's.

Reference: src/boltz_lumi/benchmark.py (the ``timings.json`` report and the
``python -m ... benchmark predict ...`` entry).  The design here:

* :class:`StageClock` times the top-level stages of a Boltz-2 model with GPU
  events, attached as forward hooks (and a wrapper of
  ``structure_module.sample``), detached again on exit;
* :class:`Tolerance` turns an output field and its upstream value into one
  error record;
* :class:`Report` is the ``timings.json`` document: it collects call, round
  and error records and works out the warm means, the saving and the status;
* :class:`ABSession` runs the recipes, upstream first and then with the native
  forwards installed, over one fixed list of candidates with the seed reset
  before every round and every call;
* :func:`ab_benchmark` drives a session with any model and step callable,
  :func:`main` with Boltz's ``predict`` CLI (Boltz 2.2.1 and
  pytorch_lightning required).

``timings.json`` keys (the reference's schema, kept so that its readers work):
the run settings, ``torch`` / ``hip`` / ``gpu`` / ``slurm_job``,
``model_calls`` (recipe, iteration, first, profiled, candidate, model_s,
peak_allocated_bytes, stages_s), ``rounds`` (recipe, iteration, first,
profiled, candidates, round_s), ``errors`` (recipe, iteration, first,
profiled, candidate, field, max_absolute_error, relative_l2_error, atol, rtol,
failing_values), ``feature_load_s`` (CLI runs), ``upstream_warm_mean_s``,
``optimized_warm_mean_s``, ``saved_s``, ``saved_percent`` and ``status``
(running, complete, numerical_difference or failed with ``error``).

Outputs count as different where ``|x - upstream| > atol + rtol * |upstream|``
(default 1e-2 each): the native kernels round in bf16 in their own order.
The reference counts every value that is not bit-identical; ``--atol 0
--rtol 0`` asks for that.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import random
import statistics
import time
from contextlib import contextmanager
from dataclasses import dataclass
from pathlib import Path

import numpy as np
import torch

from .adapters import install

RECIPES = ("upstream", "optimized")
ATOL = 1e-2
RTOL = 1e-2

# Top-level modules of a Boltz-2 model timed as stages; ``diffusion_sample``
# is the structure module's ``sample`` method.
STAGES = (
    "input_embedder",
    "template_module",
    "msa_module",
    "pairformer_module",
    "diffusion_conditioning",
    "confidence_module",
)
SAMPLE_STAGE = "diffusion_sample"

# Prediction outputs compared between the recipes, where present.
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

# Scalars every confidence summary of a structure prediction must hold.
CONFIDENCE_FIELDS = (
    "confidence_score", "ptm", "iptm", "ligand_iptm", "protein_iptm",
    "complex_plddt", "complex_iplddt", "complex_pde", "complex_ipde",
)
AFFINITY_FIELDS = ("affinity_pred_value", "affinity_probability_binary")


def seed_all(seed: int) -> None:
    """One seed for Python's, NumPy's and torch's generators (all devices)."""
    random.seed(seed)
    np.random.seed(seed % 2**32)
    torch.manual_seed(seed)


# ------------------------------------------------------------- stage timing


class StageClock:
    """GPU-event timing of a model's stages.

    While active, every call of a stage module (by ``named_modules`` name, in
    :data:`STAGES`) and of ``structure_module.sample`` appends
    ``(stage, start_event, end_event)`` to :attr:`spans`; :meth:`seconds`
    sums them per stage once the work has finished.  Modules are timed by
    forward pre- and post-hooks, the sampler by an instance attribute that
    shadows the method; both are removed on exit, restoring any instance
    attribute that was there before."""

    def __init__(self, model):
        self.model = model
        self.spans = []
        self._open = {}
        self._handles = []
        self._sampler = None

    def _start(self, stage):
        event = torch.cuda.Event(enable_timing=True)
        event.record()
        self._open.setdefault(stage, []).append(event)

    def _stop(self, stage):
        pending = self._open.get(stage)
        if pending:
            end = torch.cuda.Event(enable_timing=True)
            end.record()
            self.spans.append((stage, pending.pop(), end))

    def __enter__(self):
        for name, module in self.model.named_modules():
            if name in STAGES:
                self._handles.append(module.register_forward_pre_hook(lambda m, a, s=name: self._start(s)))
                self._handles.append(module.register_forward_hook(lambda m, a, o, s=name: self._stop(s)))
        sampler = getattr(self.model, "structure_module", None)
        if sampler is not None and callable(getattr(sampler, "sample", None)):
            previous = vars(sampler).get("sample")
            inner = sampler.sample

            def timed_sample(*args, **kwargs):
                self._start(SAMPLE_STAGE)
                try:
                    with torch.profiler.record_function(SAMPLE_STAGE):
                        return inner(*args, **kwargs)
                finally:
                    self._stop(SAMPLE_STAGE)

            sampler.sample = timed_sample
            self._sampler = (sampler, previous)
        return self

    def __exit__(self, *exc):
        for handle in self._handles:
            handle.remove()
        self._handles.clear()
        if self._sampler is not None:
            sampler, previous = self._sampler
            if previous is None:
                del sampler.sample
            else:
                sampler.sample = previous
            self._sampler = None
        self._open.clear()
        return False

    def reset(self):
        self.spans.clear()
        self._open.clear()

    def seconds(self) -> dict:
        totals = {}
        for stage, start, end in self.spans:
            totals[stage] = totals.get(stage, 0.0) + start.elapsed_time(end) / 1e3
        return totals


# ------------------------------------------------------------ comparisons


@dataclass(frozen=True)
class Tolerance:
    """Elementwise bar ``|x - expected| <= atol + rtol |expected|``."""

    atol: float = ATOL
    rtol: float = RTOL

    def record(self, value: torch.Tensor, expected: torch.Tensor) -> dict:
        """Error record of ``value`` against ``expected`` (NaN counts as failing)."""
        x, e = value.detach().double(), expected.detach().double()
        diff = (x - e).abs()
        within = diff <= self.atol + self.rtol * e.abs()
        norm = e.norm().item()
        return {
            "max_absolute_error": diff.max().item() if diff.numel() else 0.0,
            "relative_l2_error": (x - e).norm().item() / norm if norm else None,
            "atol": self.atol,
            "rtol": self.rtol,
            "failing_values": int(diff.numel() - within.sum().item()),
        }


def compare(value: torch.Tensor, expected: torch.Tensor, atol: float, rtol: float) -> dict:
    """Error record of one output field against its upstream value."""
    return Tolerance(atol, rtol).record(value, expected)


# ------------------------------------------------------------------ report


class Report(dict):
    """The ``timings.json`` document of one A/B run."""

    def __init__(self, settings=None, path: Path | None = None):
        super().__init__(settings or {})
        self.update(
            torch=torch.__version__,
            hip=torch.version.hip,
            gpu=torch.cuda.get_device_name(0) if torch.cuda.is_available() else None,
            slurm_job=os.environ.get("SLURM_JOB_ID"),
            model_calls=[],
            rounds=[],
            errors=[],
            status="running",
        )
        self.path = None if path is None else Path(path)

    def write(self) -> None:
        if self.path is not None:
            self.path.mkdir(parents=True, exist_ok=True)
            (self.path / "timings.json").write_text(json.dumps(self, indent=2) + "\n")

    def warm_times(self, recipe: str):
        return [c["model_s"] for c in self["model_calls"]
                if c["recipe"] == recipe and not c["first"] and not c["profiled"]]

    def conclude(self) -> bool:
        """Fill in the warm means, the saving and the status; True when no
        output field failed its tolerance."""
        for recipe in RECIPES:
            warm = self.warm_times(recipe)
            if warm:
                self[f"{recipe}_warm_mean_s"] = statistics.mean(warm)
        base, new = self.get("upstream_warm_mean_s"), self.get("optimized_warm_mean_s")
        if base and new is not None:
            self["saved_s"] = base - new
            self["saved_percent"] = 100.0 * (base - new) / base
        agree = not any(e["failing_values"] for e in self["errors"])
        self["status"] = "complete" if agree else "numerical_difference"
        self.write()
        return agree

    def failed(self, error: BaseException) -> None:
        if self["status"] == "running":
            self["status"] = "failed"
            self["error"] = str(error)
            self.write()


# ----------------------------------------------------------------- session


class ABSession:
    """Rounds of model calls under the two recipes.

    A round is one pass over the candidates (ids in a fixed order).  Every
    round and every call starts from ``seed``; a call's outputs (``fields``
    present in its result dict) are compared with the first upstream call of
    the same candidate."""

    def __init__(self, model, *, seed: int, tolerance: Tolerance = Tolerance(), fields=FIELDS, settings=None,
                 output=None):
        self.model = model
        self.seed = seed
        self.tolerance = tolerance
        self.fields = tuple(fields)
        self.report = Report(dict(settings or {}, seed=seed), output)
        self.clock = StageClock(model)
        self.baseline = {}
        self.tags = {}

    # one model call -------------------------------------------------------
    def call(self, candidate: str, fn, *args, **kwargs):
        seed_all(self.seed)
        self.clock.reset()
        torch.cuda.synchronize()
        torch.cuda.reset_peak_memory_stats()
        t0 = time.perf_counter()
        result = fn(*args, **kwargs)
        torch.cuda.synchronize()
        seconds = time.perf_counter() - t0
        if result.get("exception"):
            raise RuntimeError(f"the model call for {candidate} reported an exception (see the log above)")
        self.report["model_calls"].append(dict(
            self.tags, candidate=candidate, model_s=seconds,
            peak_allocated_bytes=torch.cuda.max_memory_allocated(), stages_s=self.clock.seconds()))
        self._check(candidate, result)
        return result

    def _check(self, candidate, result):
        values = {key: result[key].detach().cpu() for key in self.fields if key in result}
        broken = [key for key, v in values.items() if not torch.isfinite(v).all()]
        if broken:
            raise RuntimeError(f"non-finite output field(s) for {candidate}: {', '.join(broken)}")
        baseline = self.baseline.setdefault(candidate, values)
        if set(baseline) != set(values):
            raise RuntimeError(f"{candidate} returned fields {sorted(values)}, the first call {sorted(baseline)}")
        for key, value in values.items():
            if value.shape != baseline[key].shape:
                raise RuntimeError(f"{candidate}: {key} changed shape from {tuple(baseline[key].shape)} "
                                   f"to {tuple(value.shape)}")
            self.report["errors"].append(dict(self.tags, candidate=candidate, field=key,
                                              **self.tolerance.record(value, baseline[key])))

    # one round --------------------------------------------------------------
    def round(self, recipe: str, iteration: int, run, candidates, profiled: bool = False):
        """``run()`` makes the round's model calls (through :meth:`call`); it
        must call every candidate exactly once, in order."""
        self.tags = dict(recipe=recipe, iteration=iteration, first=iteration == 0, profiled=profiled)
        seed_all(self.seed)
        done = len(self.report["model_calls"])
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        result = run()
        torch.cuda.synchronize()
        seconds = time.perf_counter() - t0
        seen = [c["candidate"] for c in self.report["model_calls"][done:]]
        if seen != list(candidates):
            raise RuntimeError(f"round {recipe}/{iteration} called {seen}, expected {list(candidates)}")
        self.report["rounds"].append(dict(self.tags, candidates=list(candidates), round_s=seconds))
        self.report.write()
        return result

    def run(self, candidates, one_round, repeats: int, profile: bool = False, install_kwargs=None):
        """Upstream rounds 0..repeats, ``install``, optimized rounds
        0..repeats, then an optional profiled optimized round.  Raises when
        outputs differ beyond the tolerance (the report is written first)."""
        if repeats < 1:
            raise ValueError("at least one warm repeat is needed")
        result = None
        try:
            for recipe in RECIPES:
                if recipe == "optimized":
                    install(self.model, **(install_kwargs or {}))
                with self.clock:  # entered after install, which rebinds structure_module.sample
                    for iteration in range(repeats + 1):
                        result = self.round(recipe, iteration, lambda: one_round(recipe, iteration, False),
                                            candidates)
            if profile:
                with self.clock:
                    profiled_round(lambda: self.round(RECIPES[-1], repeats + 1,
                                                      lambda: one_round(RECIPES[-1], repeats + 1, True),
                                                      candidates, profiled=True), self.report.path)
            agree = self.report.conclude()
        except BaseException as error:
            self.report.failed(error)
            raise
        if not agree:
            raise RuntimeError("optimized outputs differ from upstream beyond the tolerance; the error records "
                               "are in timings.json")
        return result


def profiled_round(run, directory: Path | None):
    """``run()`` under torch.profiler; writes ``trace.json`` (Chrome trace)
    and ``profile.txt`` (the 20 entries with the most GPU self time)."""
    kinds = [torch.profiler.ProfilerActivity.CPU, torch.profiler.ProfilerActivity.CUDA]
    with torch.profiler.profile(activities=kinds) as prof:
        run()
    if directory is None:
        return
    prof.export_chrome_trace(str(directory / "trace.json"))
    top = sorted(prof.key_averages(), key=lambda e: e.self_device_time_total, reverse=True)[:20]
    rows = [f"{'Operator or kernel':42} {'GPU self seconds':>16} {'Calls':>8}"]
    rows += [f"{e.key[:42]:42} {e.self_device_time_total / 1e6:16.6f} {e.count:8d}" for e in top]
    (directory / "profile.txt").write_text("\n".join(rows) + "\n")


def ab_benchmark(model, step, candidates, *, repeats: int = 3, seed: int = 42, atol: float = ATOL,
                 rtol: float = RTOL, fields=FIELDS, output=None, profile: bool = False, settings=None,
                 install_kwargs=None) -> dict:
    """A/B run of ``step(model, batch)`` (one model call returning a dict of
    output tensors) over ``candidates``, pairs ``(id, batch)`` with unique
    ids.  Returns the report, also written to ``output/timings.json`` when
    ``output`` is given."""
    candidates = list(candidates)
    ids = [cid for cid, _ in candidates]
    if len(set(ids)) != len(ids):
        raise ValueError("candidate ids must be unique")
    session = ABSession(model, seed=seed, tolerance=Tolerance(atol, rtol), fields=fields, settings=settings,
                        output=output)

    def one_round(recipe, iteration, profiled):
        for cid, batch in candidates:
            session.call(cid, step, model, batch)

    session.run(ids, one_round, repeats, profile=profile, install_kwargs=install_kwargs)
    return session.report


# ------------------------------------------------------ output validation


def _expected_outputs(directory: Path, candidate: str, samples: int, output_format: str, affinity: bool):
    """(structure file or None, summary file, required fields, label) per
    output Boltz writes for one candidate."""
    folder = directory / candidate
    if affinity:
        yield None, folder / f"affinity_{candidate}.json", AFFINITY_FIELDS, f"{candidate} affinity"
        return
    ext = ".pdb" if output_format == "pdb" else ".cif"
    for rank in range(samples):
        stem = f"{candidate}_model_{rank}"
        yield folder / f"{stem}{ext}", folder / f"confidence_{stem}.json", CONFIDENCE_FIELDS, stem


def _finite_number(value) -> bool:
    return isinstance(value, (int, float)) and not isinstance(value, bool) and math.isfinite(value)


def validate_outputs(directory, candidates, samples, output_format="mmcif", affinity=False):
    """Check that Boltz wrote every output of every candidate: a non-empty
    structure file per sample (mmCIF, or PDB when ``output_format == "pdb"``)
    with a confidence summary of finite scalars, or one affinity summary per
    candidate when ``affinity``."""
    candidates = list(candidates)
    if not candidates:
        raise RuntimeError("no candidate was predicted")
    directory = Path(directory)
    for candidate in candidates:
        for structure, summary, fields, label in _expected_outputs(directory, candidate, samples, output_format,
                                                                    affinity):
            if structure is not None and (not structure.is_file() or structure.stat().st_size == 0):
                raise RuntimeError(f"prediction output missing or empty: {structure.name} ({label})")
            if not summary.is_file():
                raise RuntimeError(f"prediction output missing: {summary.name} ({label})")
            data = json.loads(summary.read_text())
            bad = [key for key in fields if not _finite_number(data.get(key))]
            if bad:
                raise RuntimeError(f"summary {summary.name} ({label}) lacks finite values for {', '.join(bad)}")


# --------------------------------------------------------------- Boltz CLI


def _option(arguments, name, default=None):
    """Value of ``--name value`` / ``--name=value`` in a Boltz argument list."""
    for index, arg in enumerate(arguments):
        if arg == name and index + 1 < len(arguments):
            return arguments[index + 1]
        if arg.startswith(name + "="):
            return arg.split("=", 1)[1]
    return default


class _BoltzAB:
    """``Trainer.predict`` stand-in that runs the A/B session over the
    batches Boltz's own data module prepared (loaded once, so every round
    sees the same features)."""

    def __init__(self, args, settings, original_predict):
        self.args = args
        self.settings = settings
        self.original = original_predict

    def __call__(self, trainer, model, *positional, **keywords):
        from boltz.data.write.writer import BoltzAffinityWriter, BoltzWriter
        from torch.utils.data import DataLoader

        from .__main__ import InferenceAdapter

        writers = [cb for cb in trainer.callbacks if isinstance(cb, (BoltzWriter, BoltzAffinityWriter))]
        if len(writers) != 1:
            raise RuntimeError(f"expected exactly one Boltz writer callback, found {len(writers)}")
        writer = writers[0]
        phase = "affinity" if isinstance(writer, BoltzAffinityWriter) else "structure"
        out_dir = writer.output_dir.parent / "benchmark" / phase
        out_dir.mkdir(parents=True)
        session = ABSession(model, seed=self.args.seed, tolerance=Tolerance(self.args.atol, self.args.rtol),
                            settings=dict(self.settings, phase=phase, prediction_settings=model.predict_args),
                            output=out_dir)
        data = keywords["datamodule"]
        t0 = time.perf_counter()
        batches = list(data.predict_dataloader())
        ids = [record.id for batch in batches for record in batch["record"]]
        if ids != [record.id for record in data.manifest.records]:
            raise RuntimeError("the prediction loader reordered or dropped candidates")
        session.report["feature_load_s"] = time.perf_counter() - t0
        final_dir = writer.output_dir
        raw_step = model.predict_step

        def step(batch, *a, **kw):
            if len(batch["record"]) != 1:
                raise RuntimeError("the A/B run needs one candidate per model call (batch size 1)")
            return session.call(batch["record"][0].id, raw_step, batch, *a, **kw)

        def one_round(recipe, iteration, profiled):
            last = recipe == RECIPES[-1] and iteration == self.args.repeats and not profiled
            # the last optimized round writes where Boltz's next stage reads
            writer.output_dir = final_dir if last else out_dir / recipe / (
                "profile" if profiled else f"round-{iteration:02}")
            writer.output_dir.mkdir(parents=True, exist_ok=True)
            result = self.original(trainer, model, *positional, **keywords)
            validate_outputs(writer.output_dir, ids, model.predict_args["diffusion_samples"],
                             output_format=getattr(writer, "output_format", "mmcif"), affinity=phase == "affinity")
            return result

        checks = InferenceAdapter(optimize=False)  # --no_kernels on the model and the failure checks
        trainer.callbacks.append(checks)
        try:
            with _shadowed(data, "predict_dataloader", lambda: DataLoader(batches, batch_size=None, num_workers=0)), \
                    _shadowed(model, "predict_step", step):
                result = session.run(ids, one_round, self.args.repeats, profile=self.args.profile)
        finally:
            writer.output_dir = final_dir
            trainer.callbacks.remove(checks)
        print(out_dir / "timings.json")
        return result


@contextmanager
def _shadowed(obj, name, value):
    """``obj.name = value`` as an instance attribute for the duration, then
    whatever instance attribute (or none) was there before."""
    missing = object()
    before = vars(obj).get(name, missing)
    setattr(obj, name, value)
    try:
        yield
    finally:
        if before is missing:
            delattr(obj, name)
        else:
            setattr(obj, name, before)


def main(arguments=None):
    """``python -m boltz_lumi_amd.benchmark predict input.yaml [Boltz options]
    [--repeats R] [--profile] [--atol A] [--rtol R]``."""
    from .__main__ import require_boltz

    parser = argparse.ArgumentParser(description=__doc__.splitlines()[0], allow_abbrev=False)
    parser.add_argument("--repeats", type=int, default=3, help="warm rounds per recipe (after one first round)")
    parser.add_argument("--profile", action="store_true", help="add one optimized round under torch.profiler")
    parser.add_argument("--atol", type=float, default=ATOL)
    parser.add_argument("--rtol", type=float, default=RTOL)
    args, boltz_args = parser.parse_known_args(arguments)
    if args.repeats < 1:
        parser.error("--repeats must be at least 1")
    boltz_version = require_boltz()
    if torch.cuda.device_count() != 1:
        raise RuntimeError(f"the A/B run needs exactly one visible GPU, found {torch.cuda.device_count()}")
    from boltz.main import cli
    from pytorch_lightning import Trainer

    if boltz_args[:1] == ["predict"]:
        boltz_args = boltz_args[1:]
    data = boltz_args[0] if boltz_args and not boltz_args[0].startswith("-") else None
    args.seed = int(_option(boltz_args, "--seed", 42))
    if _option(boltz_args, "--seed") is None:
        boltz_args += ["--seed", str(args.seed)]  # the upstream and optimized runs share it
    if "--no_kernels" not in boltz_args:
        boltz_args.append("--no_kernels")
    ab = _BoltzAB(args, dict(boltz=boltz_version, input=data, seed=args.seed), Trainer.predict)
    with _shadowed(Trainer, "predict", lambda trainer, model, *p, **k: ab(trainer, model, *p, **k)):
        cli(["predict", *boltz_args], standalone_mode=False)


if __name__ == "__main__":
    main()
