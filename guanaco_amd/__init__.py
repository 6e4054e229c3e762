"""guanaco_amd — MI355X (gfx950) decode hot path of the Guanaco runtime.

The product is libgq_hip.so (C ABI in include/gq_hip.h) and the host-side
KernelVTable binding in host/hip_backend.c.  This package holds the sources
(csrc/, host/), the synthetic-model geometry (spec.py) and the ctypes mirror
of the C ABI (hip.py, imported on demand because it loads the library).
"""
from . import spec, synth  # noqa: F401

__all__ = ["spec", "synth"]
