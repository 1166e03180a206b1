"""moa_amd -- MI355X (gfx950) decoder-layer hot path of Gemma-4-12B behind the reference's
operator interface (FO/src/ops.rs). The compute runs in libmoa_gfx950.so (hand-written HIP);
this package is the host-side mirror: ctypes bindings, torch front-ends and input synthesis.
"""
from . import formats, prng, synth  # noqa: F401 (numpy-only; importable without a GPU)
from ._lib import MoaError, load  # noqa: F401

__all__ = ["formats", "prng", "synth", "MoaError", "load", "ops"]


def __getattr__(name):
    if name == "ops":  # torch front-end, imported on first use
        import importlib
        return importlib.import_module(__name__ + ".ops")
    raise AttributeError(name)
