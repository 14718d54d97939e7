"""Inclusive scans over tuples of tensors for the torch backend.

Same three implementations and names as the reference (src/kla/ops/scan.py:29-97):
``doubling`` (Hillis-Steele, O(L log L) elementwise work, autograd-friendly),
``associative`` (torch's higher-order associative_scan) and ``sequential`` (a
python loop). ``combine(left, right)`` composes an earlier prefix ``left`` with a
later element ``right``.
"""

from __future__ import annotations

import functools
from typing import Callable, Sequence

import torch

CombineFn = Callable[[tuple, tuple], tuple]


def doubling_scan(combine_fn: CombineFn, xs: Sequence[torch.Tensor], dim: int) -> tuple:
    """Inclusive scan: at round r every position i >= 2^r absorbs position i - 2^r."""
    cur = tuple(xs)
    length = cur[0].size(dim)
    step = 1
    while step < length:
        head = tuple(t.narrow(dim, 0, step) for t in cur)
        earlier = tuple(t.narrow(dim, 0, length - step) for t in cur)
        later = tuple(t.narrow(dim, step, length - step) for t in cur)
        merged = combine_fn(earlier, later)
        cur = tuple(torch.cat((h, m), dim=dim) for h, m in zip(head, merged))
        step <<= 1
    return cur


def sequential_scan(combine_fn: CombineFn, xs: Sequence[torch.Tensor], dim: int) -> tuple:
    """Inclusive scan by a python loop (correctness reference, decode-length inputs)."""
    length = xs[0].size(dim)
    acc = tuple(t.select(dim, 0) for t in xs)
    out = [acc]
    for i in range(1, length):
        acc = combine_fn(acc, tuple(t.select(dim, i) for t in xs))
        out.append(acc)
    return tuple(torch.stack([o[j] for o in out], dim=dim) for j in range(len(xs)))


@functools.cache
def _associative_scan_available() -> bool:
    try:
        from torch._higher_order_ops import associative_scan  # noqa: F401
    except ImportError:
        return False
    return True


def associative_scan(combine_fn: CombineFn, xs: Sequence[torch.Tensor], dim: int) -> tuple:
    """Inclusive scan through torch's higher-order ``associative_scan`` op."""
    from torch._higher_order_ops import associative_scan as _hop

    def combine(left, right):
        return combine_fn(tuple(left), tuple(right))

    return tuple(_hop(combine, tuple(x.contiguous() for x in xs), dim=dim, combine_mode="generic"))


def resolve_scan(scan_impl: str):
    """Scan function for a ``scan_impl`` name; "auto" prefers ``associative``."""
    if scan_impl == "auto":
        scan_impl = "associative" if _associative_scan_available() else "doubling"
    table = {
        "associative": associative_scan,
        "doubling": doubling_scan,
        "sequential": sequential_scan,
    }
    try:
        return table[scan_impl]
    except KeyError:
        raise ValueError(f"Unknown scan_impl: {scan_impl!r}") from None
