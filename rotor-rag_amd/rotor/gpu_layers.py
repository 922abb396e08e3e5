"""GPU plug-in provider: ``get_gpu()`` returns the process-wide HIP backend.

Same contract as the reference (src/rotor/gpu_layers.py:11-25): a process-global
singleton created on first use, and a permanent latch when creation fails (``None``
is returned from then on, without retrying).  The failure text is kept in
``last_error()`` so callers that require the GPU can fail loudly with it.
"""
from __future__ import annotations

import os

_gpu_instance = None
_gpu_error = ""


def get_gpu():
    """Get or create the HIP backend (device ``$ROTOR_HIP_DEVICE``, default 0)."""
    global _gpu_instance, _gpu_error
    if _gpu_instance is None:
        try:
            from .gpu_ternary import HIPTernaryOps

            _gpu_instance = HIPTernaryOps(int(os.environ.get("ROTOR_HIP_DEVICE", "0")))
        except Exception as e:  # latch, as the reference does
            _gpu_error = f"{type(e).__name__}: {e}"
            _gpu_instance = False
    return _gpu_instance if _gpu_instance else None


def last_error() -> str:
    return _gpu_error


def _reset_for_tests():
    global _gpu_instance, _gpu_error
    _gpu_instance = None
    _gpu_error = ""
