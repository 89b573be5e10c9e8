"""synapse_amd — MI355X (gfx950) `hip` backend for Synapse's quantized-linear path.

The compute lives in ``libsynapse_hip.so`` (hand-written HIP kernels + the C
ABI declared in ``include/synapse_hip.h``); :mod:`synapse_amd.hip` is the
ctypes view of it.  Build with ``python -m synapse_amd.build``.
"""
from . import hip  # noqa: F401

__all__ = ["hip"]
