"""CPU tests of the Boltz integration layer (reference tests/test_workflow.py):
output validation, the CLI wrapper's argument forwarding and Trainer patch,
the Lightning callback's hooks and the A/B comparison rule.  Boltz and
pytorch_lightning are not installed here, so the tests put small stand-in
modules under those names into ``sys.modules``; without them ``run`` and
``main`` must refuse to start."""

import json
import sys
from types import ModuleType, SimpleNamespace
from unittest.mock import MagicMock

import pytest
import torch

from boltz_lumi_amd import SUPPORTED_BOLTZ_VERSION
from boltz_lumi_amd import __main__ as cli_main
from boltz_lumi_amd import benchmark
from boltz_lumi_amd.benchmark import CONFIDENCE_FIELDS, compare, validate_outputs


def write_prediction(root, candidate, samples, suffix=".cif", value=0.5):
    (root / candidate).mkdir(exist_ok=True)
    for rank in range(samples):
        stem = f"{candidate}_model_{rank}"
        (root / candidate / (stem + suffix)).write_text("structure")
        (root / candidate / f"confidence_{stem}.json").write_text(json.dumps(dict.fromkeys(CONFIDENCE_FIELDS, value)))


def test_every_candidate_and_sample_is_required(tmp_path):
    for candidate in ("first", "second"):
        write_prediction(tmp_path, candidate, 2)
    validate_outputs(tmp_path, ["first", "second"], 2)
    confidence = tmp_path / "second/confidence_second_model_1.json"
    confidence.unlink()
    with pytest.raises(RuntimeError, match=r"missing: confidence_second_model_1\.json"):
        validate_outputs(tmp_path, ["first", "second"], 2)
    confidence.write_text(json.dumps(dict.fromkeys(CONFIDENCE_FIELDS, float("nan"))))
    with pytest.raises(RuntimeError, match="lacks finite values for confidence_score"):
        validate_outputs(tmp_path, ["first", "second"], 2)
    (tmp_path / "first/first_model_0.cif").write_text("")
    with pytest.raises(RuntimeError, match=r"missing or empty: first_model_0\.cif"):
        validate_outputs(tmp_path, ["first"], 1)
    with pytest.raises(RuntimeError, match="no candidate was predicted"):
        validate_outputs(tmp_path, [], 1)


def test_pdb_and_affinity_outputs(tmp_path):
    write_prediction(tmp_path, "ligand", 1, suffix=".pdb")
    validate_outputs(tmp_path, ["ligand"], 1, output_format="pdb")
    with pytest.raises(RuntimeError, match=r"missing or empty: ligand_model_0\.cif"):
        validate_outputs(tmp_path, ["ligand"], 1)  # mmCIF expected, PDB written
    affinity = tmp_path / "ligand/affinity_ligand.json"
    affinity.write_text(json.dumps(dict(affinity_pred_value=-2.0, affinity_probability_binary=0.8)))
    validate_outputs(tmp_path, ["ligand"], 5, affinity=True)  # one summary, not one per sample
    for bad in ('{"affinity_pred_value": -2}', '{"affinity_pred_value": -2, "affinity_probability_binary": true}',
                '{"affinity_pred_value": "x", "affinity_probability_binary": 0.5}'):
        affinity.write_text(bad)
        with pytest.raises(RuntimeError, match="lacks finite values for affinity_"):
            validate_outputs(tmp_path, ["ligand"], 5, affinity=True)


@pytest.fixture()
def fake_boltz(monkeypatch):
    """Stand-in ``boltz.main`` and ``pytorch_lightning`` modules."""
    boltz, boltz_main, lightning = ModuleType("boltz"), ModuleType("boltz.main"), ModuleType("pytorch_lightning")
    boltz_main.cli = MagicMock(name="cli")
    boltz.main = boltz_main

    class Trainer:
        def predict(self, model, *args, **kwargs):
            return "predicted"

    lightning.Trainer = Trainer
    monkeypatch.setitem(sys.modules, "boltz", boltz)
    monkeypatch.setitem(sys.modules, "boltz.main", boltz_main)
    monkeypatch.setitem(sys.modules, "pytorch_lightning", lightning)
    monkeypatch.setattr(cli_main, "version", lambda name: SUPPORTED_BOLTZ_VERSION)
    return SimpleNamespace(cli=boltz_main.cli, Trainer=Trainer)


def test_native_options_are_forwarded(fake_boltz, tmp_path):
    arguments = ["predict", "input.yaml", "--out_dir", str(tmp_path), "--model", "boltz1", "--devices", "2",
                 "--output_format", "pdb", "--checkpoint", "custom.ckpt", "--cache", str(tmp_path), "--override"]
    cli_main.run(arguments)
    forwarded = fake_boltz.cli.call_args.args[0]
    extra = ["--no_kernels"] if torch.version.hip else []
    assert forwarded[:len(arguments)] == arguments
    assert forwarded[len(arguments):] == extra
    assert fake_boltz.cli.call_args.kwargs == {"standalone_mode": False}
    cli_main.run(arguments + ["--no_kernels"])  # not added twice
    assert fake_boltz.cli.call_args.args[0].count("--no_kernels") == 1
    cli_main.run(["--help"])  # only predict gets the flag
    assert fake_boltz.cli.call_args.args[0] == ["--help"]


def test_trainer_patch_and_callback_restored_after_failure(fake_boltz):
    trainer = SimpleNamespace(callbacks=[])
    Trainer = fake_boltz.Trainer

    def fail(self, model, *args, **kwargs):
        assert isinstance(self.callbacks[-1], cli_main.InferenceAdapter)
        raise RuntimeError("intentional failure")

    Trainer.predict = fail
    fake_boltz.cli.side_effect = lambda *a, **kw: Trainer.predict(trainer, None)
    with pytest.raises(RuntimeError, match="intentional failure"):
        cli_main.run(["predict", "input.yaml"])
    assert Trainer.predict is fail
    assert trainer.callbacks == []


def test_trainer_patch_passes_the_result_through(fake_boltz):
    trainer = SimpleNamespace(callbacks=["writer"])
    seen = []

    def predict(self, model, *args, **kwargs):
        seen.append((list(self.callbacks), model, args, kwargs))
        return "predicted"

    fake_boltz.Trainer.predict = predict
    fake_boltz.cli.side_effect = lambda *a, **kw: fake_boltz.Trainer.predict(trainer, "model", 1, datamodule="d")
    assert cli_main.run(["predict", "input.yaml"]) == "predicted"
    (callbacks, model, args, kwargs), = seen
    assert callbacks[0] == "writer" and isinstance(callbacks[1], cli_main.InferenceAdapter)
    assert (model, args, kwargs) == ("model", (1,), {"datamodule": "d"})
    assert trainer.callbacks == ["writer"]


def test_run_and_benchmark_refuse_without_boltz(monkeypatch):
    monkeypatch.delitem(sys.modules, "boltz", raising=False)
    with pytest.raises(RuntimeError, match=f"Boltz {SUPPORTED_BOLTZ_VERSION} is required"):
        cli_main.run(["predict", "input.yaml"])
    with pytest.raises(RuntimeError, match=f"Boltz {SUPPORTED_BOLTZ_VERSION} is required"):
        benchmark.main(["predict", "input.yaml"])
    monkeypatch.setattr(cli_main, "version", lambda name: "2.1.0")
    with pytest.raises(RuntimeError, match="supports Boltz 2.2.1, found 2.1.0"):
        cli_main.run(["predict", "input.yaml"])
    with pytest.raises(SystemExit):
        benchmark.main(["predict", "input.yaml", "--repeats", "0"])


def test_worker_installation_and_cpu_fallback(monkeypatch):
    adapter = cli_main.InferenceAdapter()
    model = SimpleNamespace(device=torch.device("cpu"), use_kernels=True)
    installed = []
    monkeypatch.setattr(cli_main, "install", installed.append)
    adapter.on_predict_start(None, model)
    assert installed == []
    model.device = torch.device("cuda", 1)
    adapter.on_predict_start(None, model)
    assert installed == [model]
    assert model.use_kernels is (not torch.version.hip)
    cli_main.InferenceAdapter(optimize=False).on_predict_start(None, model)
    assert installed == [model]


def test_affinity_and_swallowed_prediction_failures():
    adapter = cli_main.InferenceAdapter()
    adapter.on_predict_batch_end(None, None, dict(affinity_pred_value=torch.tensor(-2.0),
                                                  affinity_probability_binary=torch.tensor(0.8)), None, 0)
    adapter.on_predict_batch_end(None, None, dict(plddt=torch.tensor(float("nan"))), None, 0)  # not checked
    for output in ({"exception": True}, {"affinity_pred_value": torch.tensor(float("nan"))},
                   {"coords": torch.tensor([[0.0, float("inf"), 1.0]])}):
        with pytest.raises(RuntimeError):
            adapter.on_predict_batch_end(None, None, output, None, 0)


def test_compare_counts_values_outside_the_tolerance():
    expected = torch.tensor([1.0, -2.0, 100.0, 0.0])
    value = torch.tensor([1.0, -2.03, 100.5, 0.02])
    exact = compare(value, expected, 0.0, 0.0)
    assert exact["failing_values"] == 3
    assert exact["max_absolute_error"] == pytest.approx(0.5)
    assert exact["relative_l2_error"] == pytest.approx((0.03**2 + 0.5**2 + 0.02**2) ** 0.5 / expected.norm().item())
    # |d| <= atol + rtol |e|: 0.03 <= 0.01 + 0.02, 0.5 <= 0.01 + 1.0, 0.02 > 0.01 + 0
    assert compare(value, expected, 1e-2, 1e-2)["failing_values"] == 1
    assert compare(value, expected, 2e-2, 1e-2)["failing_values"] == 0
    assert compare(torch.tensor([float("nan")]), torch.tensor([1.0]), 1.0, 1.0)["failing_values"] == 1
    assert compare(torch.zeros(3), torch.zeros(3), 0.0, 0.0)["relative_l2_error"] is None


def test_benchmark_cli_shares_the_seed_and_restores_predict(fake_boltz, monkeypatch):
    """``benchmark.main`` hands Boltz's CLI its own arguments plus one seed
    for both recipes (42 unless given) and ``--no_kernels``; while the CLI
    runs, ``Trainer.predict`` is the A/B stand-in, afterwards the original."""
    monkeypatch.setattr(torch.cuda, "device_count", lambda: 1)
    original = fake_boltz.Trainer.predict
    seen = []
    fake_boltz.cli.side_effect = lambda argv, **kw: seen.append((argv, fake_boltz.Trainer.predict is original))
    benchmark.main(["predict", "input.yaml", "--out_dir", "out", "--repeats", "2"])
    benchmark.main(["predict", "input.yaml", "--seed=7", "--no_kernels", "--profile"])
    assert seen[0] == (["predict", "input.yaml", "--out_dir", "out", "--seed", "42", "--no_kernels"], False)
    assert seen[1] == (["predict", "input.yaml", "--seed=7", "--no_kernels"], False)
    assert fake_boltz.Trainer.predict is original
    monkeypatch.setattr(torch.cuda, "device_count", lambda: 2)
    with pytest.raises(RuntimeError, match="exactly one visible GPU"):
        benchmark.main(["predict", "input.yaml"])
