"""``python -m boltz_lumi_amd predict input.yaml ...``: Boltz's CLI with the
gfx950 forwards.

Reference: src/boltz_lumi/__main__.py:14-52.  Every argument goes to Boltz's
own CLI unchanged, except that ``predict`` on a ROCm build also gets
``--no_kernels`` (Boltz's cuEquivariance kernels exist for CUDA only).  For
the duration of the CLI call, every ``Trainer.predict`` runs with an
:class:`InferenceAdapter` among the trainer's callbacks: it installs the
native forwards once the model sits on the GPU and turns a prediction
failure that Boltz logged and swallowed, or a non-finite output, into an
error.  Boltz 2.2.1 and pytorch_lightning must be installed; without them
``run`` raises before doing anything else.
"""

from __future__ import annotations

import sys
from contextlib import contextmanager
from functools import wraps
from importlib.metadata import PackageNotFoundError, version

import torch

from . import SUPPORTED_BOLTZ_VERSION
from .adapters import install

try:
    from pytorch_lightning import Callback as _Callback
except ImportError:  # Boltz cannot run without Lightning; the hooks below still can
    _Callback = object

# Outputs whose values must be finite after every prediction batch.
CHECKED_OUTPUTS = ("coords", "confidence_score", "affinity_pred_value", "affinity_probability_binary")


def _batch_problem(outputs) -> str | None:
    """Why a prediction batch's outputs are unusable, or None."""
    if outputs.get("exception"):
        return "Boltz caught an exception in this prediction batch (see its log above)"
    broken = [key for key in CHECKED_OUTPUTS if key in outputs and not bool(torch.isfinite(outputs[key]).all())]
    if broken:
        return f"prediction produced non-finite {', '.join(broken)}"
    return None


class InferenceAdapter(_Callback):
    """Lightning callback of the inference runs (reference __main__.py:14-30).

    ``optimize=False`` keeps the upstream forwards and only applies the ROCm
    setting and the output checks (the A/B harness's upstream recipe)."""

    def __init__(self, optimize: bool = True):
        self.optimize = optimize

    def on_predict_start(self, trainer, model):
        # Boltz's affinity data path does not pass --no_kernels on, so the
        # model's own flag is cleared as well.
        on_rocm = bool(torch.version.hip)
        if on_rocm and hasattr(model, "use_kernels"):
            model.use_kernels = False
        if self.optimize and model.device.type == "cuda":
            install(model)

    def on_predict_batch_end(self, trainer, model, outputs, batch, batch_idx, dataloader_idx=0):
        problem = _batch_problem(outputs)
        if problem is not None:
            raise RuntimeError(problem)


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
    out = list(arguments)
    wants_flag = bool(torch.version.hip) and out[:1] == ["predict"]
    return out + ["--no_kernels"] if wants_flag and "--no_kernels" not in out else out


@contextmanager
def adapter_on_predict(optimize: bool = True):
    """Within the context every ``Trainer.predict`` call carries a fresh
    :class:`InferenceAdapter` in its trainer's callbacks, removed again when
    the call returns or raises; the class method is restored on exit."""
    from pytorch_lightning import Trainer

    plain = Trainer.predict

    @wraps(plain)
    def predict_with_adapter(trainer, *args, **kwargs):
        adapter = InferenceAdapter(optimize)
        callbacks = trainer.callbacks
        callbacks.append(adapter)
        try:
            return plain(trainer, *args, **kwargs)
        finally:
            callbacks.remove(adapter)

    Trainer.predict = predict_with_adapter
    try:
        yield
    finally:
        Trainer.predict = plain


def run(arguments=None, optimize: bool = True):
    """The ``boltz`` CLI with the adapter (reference __main__.py:33-52)."""
    require_boltz()
    from boltz.main import cli

    argv = native_arguments(sys.argv[1:] if arguments is None else arguments)
    with adapter_on_predict(optimize):
        return cli(argv, standalone_mode=False)


if __name__ == "__main__":
    run()
