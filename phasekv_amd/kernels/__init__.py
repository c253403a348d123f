"""Drop-in ``kernels`` namespace of PhaseKV Stage B, backed by HIP kernels for MI355X.

Mirrors ``src/phasekv/kernels/__init__.py`` of the reference (which re-exports
``packing`` and ``reference``) and adds ``attention_triton`` and
``launch_config`` under their reference names.
"""
from __future__ import annotations

from . import launch_config, packing, reference
from . import attention_triton

__all__ = ["packing", "reference", "attention_triton", "launch_config"]
