"""CPU oracle for the KLA scan hot path -- TEST INFRASTRUCTURE, NOT PRODUCT CODE.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this package, and only as the checker (or, for
``cpu_baseline``, as the timed CPU restatement of the reference). Nothing under
``kalman-linear-attention_amd/`` imports it: the ``hip`` backend fails loudly when
its native library is missing instead of falling back to anything here.

Contents (each function cites the reference file:line it restates):

* :mod:`oracle.scans`     numpy, any float dtype (float64 by default): the
  standalone Moebius and affine scans, forward and exact backward, in the
  per-step (lane-serial) form and in the reference's trace-normalised
  prefix-product form.
* :mod:`oracle.kla`       numpy float64: the full KLA scan as the sequential
  information-form filter (``kla_scan_reference``) and, independently, as a
  textbook covariance-form scalar Kalman filter.
* :mod:`oracle.torch_ref` torch (CPU, autograd): a restatement of the reference's
  pure-PyTorch path ``kla_scan_torch`` (doubling scan, linear and log Moebius
  combines) and of the standalone scans built from it -- the "reference CPU
  path" the GPU results are compared against and timed beside.

How each function is pinned (closed forms, finite differences, the covariance
filter, invariants of the trace-normalised combine, planted mistakes) is in
``tests/test_oracle_pins.py``. The reference ships no golden vectors for this
path; every pin is a mathematical one.
"""
