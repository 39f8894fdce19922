"""pulsarlm_amd: MI355X (gfx950) quantized-linear hot path for PulsarLM.

Replaces the reference's Marlin W4A16 / fp8 dequant-GEMMs
(pulsarlm-core/src/kernels/marlin.cu) with hand-written CDNA4 HIP kernels
behind a C ABI (include/pulsarlm_amd.h). Import is cheap; the HIP library is
loaded on first use and must have been built (``python -m pulsarlm_amd.build``).
"""

from . import _lib  # noqa: F401

__all__ = ["ops"]
