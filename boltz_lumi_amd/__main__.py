"""Run Boltz's ``predict`` CLI with the gfx950 forwards installed.

Reference: src/boltz_lumi/__main__.py:14-52.  ``python -m boltz_lumi_amd
predict input.yaml ...`` forwards every argument to Boltz's own CLI; on a ROCm
build it adds ``--no_kernels`` (Boltz's cuEquivariance kernels are CUDA-only),
and every ``Trainer.predict`` call runs with an :class:`InferenceAdapter` in the
trainer's callbacks, which installs the native forwards on the model once it
is on the GPU and turns swallowed prediction failures and non-finite outputs
into errors.  Boltz 2.2.1 and pytorch_lightning must be installed; without them
``run`` raises instead of running anything else.
"""

from __future__ import annotations

import sys
from contextlib import contextmanager
from importlib.metadata import PackageNotFoundError, version

import torch

from . import SUPPORTED_BOLTZ_VERSION
from .adapters import install

try:
    from pytorch_lightning import Callback as _Callback
except ImportError:  # Boltz cannot run without Lightning; the hooks below still can
    _Callback = object

# Prediction outputs that must be finite (reference __main__.py:26-28).
CHECKED_OUTPUTS = ("coords", "confidence_score", "affinity_pred_value", "affinity_probability_binary")


class InferenceAdapter(_Callback):
    """Lightning callback (reference __main__.py:14-30)."""

    def __init__(self, optimize: bool = True):
        self.optimize = optimize

    def on_predict_start(self, trainer, model):
        # Boltz's affinity loader does not forward --no_kernels, so the flag is
        # also cleared on the model itself.
        if torch.version.hip and hasattr(model, "use_kernels"):
            model.use_kernels = False
        if self.optimize and model.device.type == "cuda":
            install(model)

    def on_predict_batch_end(self, trainer, model, outputs, batch, batch_idx, dataloader_idx=0):
        if outputs.get("exception"):
            raise RuntimeError("Boltz prediction failed; inspect the preceding log")
        for key in CHECKED_OUTPUTS:
            if key in outputs and not torch.isfinite(outputs[key]).all():
                raise RuntimeError(f"Nonfinite prediction: {key}")


def require_boltz() -> str:
    """The installed Boltz version; RuntimeError unless it is the supported one."""
    try:
        found = version("boltz")
    except PackageNotFoundError:
        raise RuntimeError(f"Boltz {SUPPORTED_BOLTZ_VERSION} is required and is not installed") from None
    if found != SUPPORTED_BOLTZ_VERSION:
        raise RuntimeError(f"This adapter supports Boltz {SUPPORTED_BOLTZ_VERSION}, found {found}")
    return found


def native_arguments(arguments) -> list:
    """Boltz CLI arguments with ``--no_kernels`` added to ``predict`` on ROCm."""
    arguments = list(arguments)
    if torch.version.hip and arguments[:1] == ["predict"] and "--no_kernels" not in arguments:
        arguments.append("--no_kernels")
    return arguments


@contextmanager
def adapter_on_predict(optimize: bool = True):
    """Patch ``Trainer.predict`` so that each call runs with an
    :class:`InferenceAdapter` appended to the trainer's callbacks; the callback
    and the original method are restored also when the prediction raises."""
    from pytorch_lightning import Trainer

    original = Trainer.predict

    def predict(trainer, model, *args, **kwargs):
        adapter = InferenceAdapter(optimize)
        trainer.callbacks.append(adapter)
        try:
            return original(trainer, model, *args, **kwargs)
        finally:
            trainer.callbacks.remove(adapter)

    Trainer.predict = predict
    try:
        yield
    finally:
        Trainer.predict = original


def run(arguments=None, optimize: bool = True):
    """``boltz`` CLI entry with the adapter (reference __main__.py:33-52)."""
    require_boltz()
    from boltz.main import cli

    arguments = native_arguments(sys.argv[1:] if arguments is None else arguments)
    with adapter_on_predict(optimize):
        return cli(arguments, standalone_mode=False)


if __name__ == "__main__":
    run()
