"""hi2_amd — the hi2 encode hot path on AMD Instinct MI355X (gfx950).

Drop-in for the reference's per-Linear encode numerics: the modules
``hi2_amd.hessian``, ``hi2_amd.encode``, ``hi2_amd.gptq_kernel``,
``hi2_amd.ladder_kernel``, ``hi2_amd.format``, ``hi2_amd.refine``,
``hi2_amd.refine_kernel``, ``hi2_amd.stats``, ``hi2_amd.cache``, ``hi2_amd.calibrate``,
``hi2_amd.checkpoint`` and ``hi2_amd.qad_kernel`` keep the names and call signatures of the reference's
modules of the same names (``hi2.hessian`` ... ``hi2.checkpoint``) for the encode path
and run every arithmetic step in the HIP kernels of ``libhi2x.so`` (C ABI:
``include/hi2x.h``).
"""

__version__ = "0.1.0"
