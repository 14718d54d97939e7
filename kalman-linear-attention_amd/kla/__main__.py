"""``python -m kla``: what this machine can run, and whether it runs correctly.

    python -m kla                          # version, device, what backend="auto" picks
    python -m kla --check-backends         # every backend family, and which are usable
    python -m kla --test-backends all      # run every family against the sequential reference
    python -m kla --test-backends hip      # ...or only the ones named (family or exact name)

Same flags and meaning as the reference CLI (src/kla/__main__.py:1-21, :285-354),
with argparse in place of tyro and a ``hip`` family row for this build:

* ``--check-backends`` is a cheap probe: device, ROCm torch, and whether
  ``libkla_hip.so`` loads with the ABI version the binding expects. No kernel
  runs. ``[X]`` marks what ``auto`` resolves to, ``[x]`` a usable family.
* ``--test-backends`` runs the forward and the backward of every implementation
  named and reports each against :func:`kla.ops.kla_scan_reference`. Naming a
  backend asserts it works (exit 1 if it fails or cannot run here); ``all`` is a
  survey and exits 0.
"""

from __future__ import annotations

import argparse
import sys

# One line per family (reference __main__.py:28-33 keeps the same kind of table).
_DESCRIPTIONS = {
    "torch": "the portable reference implementation",
    "hip": "MI355X (gfx950) HIP kernels: fused scan, composed scans, decode step",
    "triton": "Triton kernels - not part of this MI355X build",
    "cuda": "CUDA kernels - not part of this MI355X build",
    "mps": "Metal kernels - not part of this MI355X build",
}

# Accuracy budget of --test-backends, the reference CLI's (__main__.py:58-61):
# forward allclose at 5e-4, each input's gradient within 1e-2 of its own scale.
_FWD_TOL = 5e-4
_GRAD_TOL = 1e-2
_INPUT_NAMES = ("v", "lambda_v", "k", "q", "a", "p")


def _families(names) -> dict:
    """``<family>_<impl>`` names grouped by family, in registry order."""
    out: dict = {}
    for name in names:
        out.setdefault(name.split("_", 1)[0], []).append(name)
    return out


def _hip_requirements() -> list:
    """``(holds, what is missing)`` for the hip family; cheap, runs no kernel."""
    import torch

    rows = [
        (getattr(torch.version, "hip", None) is not None, "needs a ROCm build of torch"),
        (torch.cuda.is_available(), "needs a ROCm GPU (MI355X / gfx950)"),
    ]
    if all(ok for ok, _ in rows):
        try:
            from kla.ops.hip import _lib

            _lib.lib()
            rows.append((True, ""))
        except Exception as exc:  # noqa: BLE001 - reported, not raised
            rows.append((False, f"libkla_hip.so does not load - {_oneline(exc)}"))
    return rows


def _probe(family: str) -> tuple:
    """``(usable, description)`` of one family; nothing is launched."""
    described = _DESCRIPTIONS.get(family, "")
    if family == "torch":
        return True, described
    if family != "hip":
        return False, described
    for holds, missing in _hip_requirements():
        if not holds:
            return False, f"{described} - {missing}"
    return True, described


def _inputs(device: str, requires_grad: bool = False):
    """The probe batch: lambda_v, p > 0 and a in (0, 1), so a failure is the backend's.

    A ragged length (37 steps) and 12 channels make the HIP kernels run partial
    tiles and blocks.
    """
    import torch

    B, L, M, S = 2, 37, 12, 16
    gen = torch.Generator().manual_seed(0)

    def to(t):
        return t.to(device).requires_grad_(requires_grad)

    return (
        to(torch.randn(B, L, M, generator=gen)),
        to(torch.rand(B, L, M, generator=gen) + 0.5),
        to(torch.randn(B, L, S, generator=gen) * 0.3),
        to(torch.randn(B, L, S, generator=gen) * 0.3),
        to(torch.rand(M, S, generator=gen) * 0.5 + 0.4),
        to(torch.rand(M, S, generator=gen) * 0.05 + 0.01),
    )


def _oneline(exc: BaseException) -> str:
    lines = str(exc).strip().splitlines()
    return f"{type(exc).__name__}: {lines[0]}" if lines else type(exc).__name__


def _scaled_err(got, want) -> float:
    """Max deviation over the reference's own scale (+1), as the reference CLI's."""
    return ((got - want).abs().max() / (want.abs().max() + 1.0)).item()


def _check_forward(backend: str, device: str) -> tuple:
    import torch

    from kla.ops import kla_scan, kla_scan_reference

    args = _inputs(device)
    try:
        y, y_var, _ = kla_scan(*args, backend=backend)
    except NotImplementedError as exc:
        return "skipped", _oneline(exc)
    except Exception as exc:  # noqa: BLE001
        return "FAILED", _oneline(exc)
    if not (torch.isfinite(y).all() and torch.isfinite(y_var).all()):
        return "FAILED", "non-finite output"
    y_ref, var_ref, _ = kla_scan_reference(*args)
    ok = torch.allclose(y, y_ref, atol=_FWD_TOL, rtol=_FWD_TOL) and torch.allclose(
        y_var, var_ref, atol=_FWD_TOL, rtol=_FWD_TOL)
    detail = (f"max|dy| {(y - y_ref).abs().max().item():.1e}   "
              f"max|dvar| {(y_var - var_ref).abs().max().item():.1e}   (atol {_FWD_TOL:g})")
    return ("ok" if ok else "FAILED"), detail


def _check_gradients(backend: str, device: str) -> tuple:
    import torch

    from kla.ops import kla_scan, kla_scan_reference

    args = _inputs(device, requires_grad=True)
    refs = tuple(t.detach().clone().requires_grad_(True) for t in args)
    try:
        y, y_var, _ = kla_scan(*args, backend=backend)
        # y^2 keeps the read-out in the loss, y_var the precision path.
        (y.square().sum() + y_var.sum()).backward()
    except NotImplementedError as exc:
        return "skipped", _oneline(exc)
    except Exception as exc:  # noqa: BLE001
        return "FAILED", _oneline(exc)
    y_ref, var_ref, _ = kla_scan_reference(*refs)
    (y_ref.square().sum() + var_ref.sum()).backward()
    worst, worst_name = 0.0, ""
    for name, got, want in zip(_INPUT_NAMES, args, refs):
        if got.grad is None:
            return "FAILED", f"no gradient reached d{name}"
        if not torch.isfinite(got.grad).all():
            return "FAILED", f"non-finite d{name}"
        e = _scaled_err(got.grad, want.grad)
        if e >= worst:
            worst, worst_name = e, name
    return ("ok" if worst < _GRAD_TOL else "FAILED"), f"worst d{worst_name} {worst:.1e}   (budget {_GRAD_TOL:g})"


_CHECKS = (("forward", _check_forward), ("gradients", _check_gradients))


def _run_checks(backend: str, device: str, indent: str, out) -> bool:
    ok, last = True, None
    for label, check in _CHECKS:
        status, detail = check(backend, device)
        ok &= status == "ok"
        if (status, detail) == last:
            detail = "(same reason)"
        else:
            last = (status, detail)
        print(f"{indent}{label:<9}  {status:<7}  {detail}", file=out)
    return ok


def main(argv=None, out=None) -> int:
    """Report (and with ``--test-backends``, test) the scan backends on this machine."""
    out = out or sys.stdout
    parser = argparse.ArgumentParser(prog="python -m kla", description=__doc__.split("\n\n")[0])
    parser.add_argument("--check-backends", action="store_true",
                        help="show every backend family and whether it is usable here, without running it")
    parser.add_argument("--test-backends", nargs="*", default=None, metavar="NAME",
                        help="run the named backends (a family, an exact name, or 'all') against the reference")
    args = parser.parse_args(argv)

    import torch

    import kla
    from kla.ops.kla_ops import default_device

    families = _families(kla.backend_names())

    if args.check_backends:
        auto = kla.resolve_backend()
        width = max(len(f) for f in families)
        for family in families:
            usable, why = _probe(family)
            mark = "X" if family == auto else "x" if usable else " "
            print(f"  [{mark}] {family:<{width}}  {why}", file=out)
        print("\n  [X] = what backend='auto' resolves to here", file=out)
        return 0

    if args.test_backends is not None:
        # Exact names first, families last: a family name is also a registry
        # name, and naming it means the whole family.
        targets = {name: [name] for name in kla.backend_names()} | families
        if not args.test_backends:
            raise SystemExit(f"--test-backends needs 'all', or one of {', '.join(targets)}")
        survey = "all" in args.test_backends
        selected = list(families) if survey else list(args.test_backends)
        unknown = [n for n in selected if n not in targets]
        if unknown:
            raise SystemExit(f"unknown backend(s) {', '.join(unknown)}; expected 'all' or {', '.join(targets)}")
        device = default_device()
        failed = 0
        for name in selected:
            print(f"\n{name}", file=out)
            impls = targets[name]
            nested = len(impls) > 1
            ok = True
            for impl in impls:
                if nested:
                    print(f"  {impl}", file=out)
                ok &= _run_checks(impl, device, "    " if nested else "  ", out)
            failed += not ok
        return 1 if failed and not survey else 0

    device = default_device()
    shown = torch.cuda.get_device_name(0) if device == "cuda" else device
    hip = getattr(torch.version, "hip", None)
    print(f"kla {kla.__version__}   torch {torch.__version__}" + (f" (HIP {hip})" if hip else "")
          + f"   device: {shown}", file=out)
    print(f"backend='auto' resolves to: {kla.resolve_backend()}", file=out)
    print("\n  --check-backends to see them all, --test-backends to run them", file=out)
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
