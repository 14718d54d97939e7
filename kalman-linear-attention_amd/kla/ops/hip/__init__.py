"""MI355X (gfx950) kernels of the KLA scan, reached through libkla_hip.so.

:func:`mobius_scan` and :func:`affine_scan` are the standalone, differentiable
scan ops; :mod:`kla.ops.hip_backend` builds the ``"hip"`` KLA backend on them.
"""

from kla.ops.hip.scans import affine_scan, mobius_scan

__all__ = ["affine_scan", "mobius_scan"]
