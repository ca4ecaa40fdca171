"""GPU tests of the A/B harness (reference benchmark.py) on a stand-in Boltz-2
trunk: upstream rounds, then ``install`` and optimized rounds over the same
candidates and seeds; the report holds every call with its stage timings,
the error records against the first upstream call, the warm means and the
status, and is written as ``timings.json``.  The optimized recipe runs the
native kernels (counted), and a planted difference or a non-finite output
ends the run with the matching status."""

import json

import pytest
import torch
from torch import nn

from boltz_lumi_amd import adapters, ops
from boltz_lumi_amd.benchmark import RECIPES, ab_benchmark
from oracle import boltz_ref as R

pytestmark = pytest.mark.gpu

FIELDS = ("plddt", "confidence_score")


class Trunk(nn.Module):
    def __init__(self):
        super().__init__()
        self.layers = nn.ModuleList([R.PairformerLayer()])

    def forward(self, s, z, mask, pair_mask):
        for layer in self.layers:
            s, z = layer(s, z, mask, pair_mask)
        return s, z


class Boltz2(nn.Module):
    def __init__(self):
        super().__init__()
        self.pairformer_module = Trunk()


def step(model, batch):
    s, z, mask = batch
    with torch.inference_mode(), torch.autocast("cuda", dtype=torch.bfloat16):
        _, z = model.pairformer_module(s, z, mask, mask[:, :, None] * mask[:, None, :])
    z = z.float()
    return {"plddt": z.mean(dim=(2, 3)), "confidence_score": z.square().mean().reshape(1), "unused": z}


@pytest.fixture()
def model(gpu):
    torch.manual_seed(4410)
    m = R.randomize(Boltz2()).to(gpu).eval()
    yield m
    adapters.uninstall(m)


def candidates(gpu):
    out = []
    for name, n, masked in (("first", 48, 0), ("second", 70, 6)):
        mask = torch.ones(1, n, device=gpu)
        if masked:
            mask[:, -masked:] = 0
        out.append((name, (torch.randn(1, n, 384, device=gpu), torch.randn(1, n, n, 128, device=gpu) * 0.5, mask)))
    return out


def test_ab_benchmark_report(model, gpu, tmp_path, monkeypatch):
    native = []
    original = ops.triattn
    monkeypatch.setattr(ops, "triattn", lambda *a, **k: native.append(1) or original(*a, **k))
    report = ab_benchmark(model, step, candidates(gpu), repeats=1, seed=7, fields=FIELDS, output=tmp_path,
                          settings=dict(input="stand-in"))
    assert report["status"] == "complete"
    assert json.loads((tmp_path / "timings.json").read_text()) == json.loads(json.dumps(report))
    assert report["input"] == "stand-in" and report["hip"] == torch.version.hip
    calls = report["model_calls"]
    assert [(c["recipe"], c["iteration"], c["candidate"]) for c in calls] == [
        (r, i, c) for r in RECIPES for i in range(2) for c in ("first", "second")]
    assert all(c["stages_s"]["pairformer_module"] > 0 for c in calls)
    assert all(c["stages_s"]["pairformer_module"] <= c["model_s"] for c in calls)
    assert all(c["first"] == (c["iteration"] == 0) and not c["profiled"] for c in calls)
    assert len(native) == 2 * 2 * 2  # optimized rounds only: 2 rounds x 2 candidates x 2 triangle attentions
    assert [(r["recipe"], r["iteration"]) for r in report["rounds"]] == [(r, i) for r in RECIPES for i in range(2)]
    errors = report["errors"]
    assert len(errors) == len(calls) * len(FIELDS)
    for e in errors:
        assert e["failing_values"] == 0 and e["atol"] == e["rtol"] == 1e-2
        if e["recipe"] == "upstream":  # upstream is deterministic: every repeat is bit-identical
            assert e["max_absolute_error"] == 0
    assert any(e["max_absolute_error"] > 0 for e in errors if e["recipe"] == "optimized")
    for recipe in RECIPES:
        warm = [c["model_s"] for c in calls if c["recipe"] == recipe and c["iteration"] == 1]
        assert report[recipe + "_warm_mean_s"] == pytest.approx(sum(warm) / len(warm))
    assert report["saved_s"] == pytest.approx(report["upstream_warm_mean_s"] - report["optimized_warm_mean_s"])


def test_ab_benchmark_profiled_round(model, gpu, tmp_path):
    """``profile=True`` adds one optimized round under torch.profiler: its calls
    are marked profiled and left out of the warm means; the Chrome trace and
    the GPU self-time table are written next to timings.json."""
    report = ab_benchmark(model, step, candidates(gpu)[:1], repeats=1, fields=FIELDS, output=tmp_path,
                          profile=True)
    assert report["status"] == "complete"
    profiled = [c for c in report["model_calls"] if c["profiled"]]
    assert [(c["recipe"], c["iteration"]) for c in profiled] == [("optimized", 2)]
    warm = [c["model_s"] for c in report["model_calls"] if c["recipe"] == "optimized" and c["iteration"] == 1]
    assert report["optimized_warm_mean_s"] == pytest.approx(warm[0])
    assert json.loads((tmp_path / "trace.json").read_text())["traceEvents"]
    table = (tmp_path / "profile.txt").read_text().splitlines()
    assert table[0].startswith("Operator or kernel") and len(table) > 1


def test_ab_benchmark_flags_differences_and_failures(model, gpu, tmp_path):
    def shifted(m, batch):
        out = step(m, batch)
        if getattr(m, adapters.FLAG, False):
            out["plddt"] = out["plddt"] + 0.5
        return out

    with pytest.raises(RuntimeError, match="differ from upstream beyond the tolerance"):
        ab_benchmark(model, shifted, candidates(gpu)[:1], repeats=1, fields=FIELDS, output=tmp_path)
    report = json.loads((tmp_path / "timings.json").read_text())
    assert report["status"] == "numerical_difference"
    failing = {(e["recipe"], e["field"]) for e in report["errors"] if e["failing_values"]}
    assert failing == {("optimized", "plddt")}
    adapters.uninstall(model)

    def nonfinite(m, batch):
        out = step(m, batch)
        out["confidence_score"] = out["confidence_score"] / 0
        return out

    with pytest.raises(RuntimeError, match=r"non-finite output field\(s\) for first: confidence_score"):
        ab_benchmark(model, nonfinite, candidates(gpu)[:1], repeats=1, fields=FIELDS, output=tmp_path)
    report = json.loads((tmp_path / "timings.json").read_text())
    assert report["status"] == "failed" and "confidence_score" in report["error"]
