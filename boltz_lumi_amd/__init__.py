"""gfx950 (MI355X) kernels for Boltz-2's pair-representation hot path.

The package is a drop-in behind the module API that lauritsf/boltz-lumi
patches into Boltz: ``install(model)`` rebinds the forwards of
TriangleAttention (starting / ending node), TriangleMultiplication (outgoing /
incoming), the pair Transition and the diffusion AdaLN / conditioned
transition blocks to fused HIP kernels in ``libbmx.so`` (C ABI:
``include/bmx.h``).  ``layers`` holds Boltz-compatible modules that run the
same kernels directly.
"""

SUPPORTED_BOLTZ_VERSION = "2.2.1"
__version__ = f"{SUPPORTED_BOLTZ_VERSION}.0"


def install(model, **kwargs):
    """Patch a Boltz-2 model's hot-path modules (see ``adapters.install``)."""
    from .adapters import install as _install

    return _install(model, **kwargs)
