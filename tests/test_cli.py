"""``python -m kla``: the backend report and self-test (reference src/kla/__main__.py).

CPU cases here; the hip family's self-test on a GPU is
tests/test_gpu_backend.py::test_cli_self_test_passes_on_hip.
"""

import io
import os
import subprocess
import sys

import pytest
import torch

from kla import __main__ as cli


def run(*argv):
    out = io.StringIO()
    rc = cli.main(list(argv), out=out)
    return rc, out.getvalue()


def test_summary_names_the_auto_backend():
    rc, text = run()
    assert rc == 0
    assert "backend='auto' resolves to:" in text
    want = "hip" if torch.cuda.is_available() else "torch"
    assert text.splitlines()[1].endswith(want)


def test_check_backends_lists_every_family_once():
    rc, text = run("--check-backends")
    assert rc == 0
    rows = [line for line in text.splitlines() if line.startswith("  [") and " = " not in line]
    names = [row[6:].split()[0] for row in rows]
    assert names == ["torch", "hip", "triton", "cuda", "mps"]
    marks = {row[6:].split()[0]: row[3] for row in rows}
    # Exactly one [X]: what auto resolves to.
    assert sum(m == "X" for m in marks.values()) == 1
    assert marks["triton"] == marks["cuda"] == marks["mps"] == " "
    if not torch.cuda.is_available():
        assert marks["torch"] == "X" and marks["hip"] == " "
        assert "needs a ROCm GPU" in text


def test_torch_backend_self_test_passes():
    rc, text = run("--test-backends", "torch")
    assert rc == 0, text
    assert text.count(" ok ") == 2


def test_naming_an_unusable_backend_fails_but_a_survey_does_not():
    rc, text = run("--test-backends", "triton_fused")
    assert rc == 1
    assert "skipped" in text and "not part of this MI355X build" in text
    rc, text = run("--test-backends", "all")
    assert rc == 0
    assert "\nmps\n" in text and "(same reason)" in text


def test_bad_names_exit_with_the_choices():
    with pytest.raises(SystemExit, match="unknown backend"):
        run("--test-backends", "hipp")
    with pytest.raises(SystemExit, match="needs 'all'"):
        run("--test-backends")


def test_self_test_catches_a_wrong_backend(monkeypatch):
    """A backend whose forward is off fails the forward row; one whose gradient is off, the other."""
    from kla.ops import kla_ops

    real = kla_ops._BACKENDS["torch"]

    def biased(*args, **kwargs):
        y, y_var, st = real(*args, **kwargs)
        return y * 1.01, y_var, st

    def bad_grad(v, lambda_v, k, q, a, p, **kwargs):
        y, y_var, st = real(v, lambda_v, k, q, a, p, **kwargs)
        # Same values, but q's gradient through y is doubled.
        q2 = q + (q - q.detach())
        y2, _, _ = real(v, lambda_v, k, q2, a, p, **kwargs)
        return y2, y_var, st

    monkeypatch.setitem(kla_ops._BACKENDS, "torch", biased)
    rc, text = run("--test-backends", "torch")
    assert rc == 1 and "forward    FAILED" in text
    monkeypatch.setitem(kla_ops._BACKENDS, "torch", bad_grad)
    rc, text = run("--test-backends", "torch")
    assert rc == 1 and "forward    ok" in text and "gradients  FAILED" in text


def test_module_entry_point_runs():
    pkg = os.path.dirname(os.path.dirname(os.path.abspath(cli.__file__)))
    env = dict(os.environ, PYTHONPATH=os.pathsep.join([pkg, os.environ.get("PYTHONPATH", "")]))
    proc = subprocess.run([sys.executable, "-m", "kla", "--check-backends"], capture_output=True, text=True,
                          timeout=300, env=env)
    assert proc.returncode == 0, proc.stderr
    assert "[X]" in proc.stdout
