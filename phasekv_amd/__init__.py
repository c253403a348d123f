"""MI355X-native PhaseKV Stage-B decode path.

* ``phasekv_amd.kernels`` — drop-in for ``src/phasekv/kernels`` of the reference
  (``packing``, ``attention_triton``, ``launch_config``, ``reference``), backed by
  hand-written HIP kernels for gfx950 in ``libphasekv_hip.so``.
* ``phasekv_amd.tiers`` — the segment / layer-tiers data formats the path reads.
* ``phasekv_amd.workloads`` — seeded synthetic inputs of the benchmark configs.
"""
from __future__ import annotations

from . import kernels, tiers

__all__ = ["kernels", "tiers"]
