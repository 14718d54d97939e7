"""The two ways a kernel op is called: through the torch.library dispatcher, and
directly (kla.ops.hip._lib.call), which the wrappers take where the dispatcher
adds nothing -- no autograd to record, plain tensors, no torch.compile tracing.
Both run the same function, so their results are bit-identical; under
torch.compile the ops are traced through the dispatcher with their fake
(meta) functions, and the compiled function returns what eager returns.
"""

import pytest
import torch

from kla.ops.hip import _lib

pytestmark = pytest.mark.gpu


def _rand(*shape, seed=0, scale=1.0, dtype=torch.float32):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * scale).to(dtype)


def _same(a, b):
    if isinstance(a, torch.Tensor):
        assert torch.equal(a, b)
    else:
        assert len(a) == len(b)
        for x, y in zip(a, b):
            if x is None or y is None:
                assert x is None and y is None
            else:
                assert torch.equal(x, y)


def test_direct_call_equals_dispatched_call(cuda):
    """Each forward op, called through the dispatcher and through its undecorated
    function, on the same inputs: bit-identical outputs. Without autograd
    _lib.call takes the direct path; with an input that requires grad it takes
    the dispatcher."""
    from kla.ops.hip import conv, dynamics, fused, sensors, step, tail

    B, L, M, S, D = 2, 96, 24, 16, 48
    v, lv = _rand(B, L, M, seed=1).to(cuda), (_rand(B, L, M, seed=2).abs() + 0.5).to(cuda)
    k, q = (_rand(B, L, S, seed=3, scale=0.3).to(cuda), _rand(B, L, S, seed=4, scale=0.3).to(cuda))
    a, p = (torch.rand(M, S) * 0.5 + 0.45).to(cuda), (torch.rand(M, S) * 0.05 + 0.01).to(cuda)
    x, w, bias = _rand(B, L, D, seed=5).to(cuda), _rand(D, 4, seed=6, scale=0.3).to(cuda), _rand(D, seed=7).to(cuda)
    cases = [
        (fused._fused_fwd_op, (v, lv, k, q, a, p, None, None, False, False)),
        (fused._sensors_fwd_op, (v, lv, k, q, a, p, None, None, True, 1e-4, float("inf"), False, False, True)),
        (conv._conv_op, (x, None, w, bias, 1)),
        (tail._tail_op, (_rand(B, L, D, seed=8).to(cuda), x, _rand(B, L, D, seed=9).to(cuda),
                         torch.tensor(0.5, device=cuda), 1, False)),
        (sensors._qk_op, (k, q, True, True, 0.5)),
        (dynamics._disc_op, (_rand(M, S, seed=10).to(cuda), _rand(M, S, seed=11).to(cuda),
                             _rand(M, S, seed=12, scale=0.1).to(cuda), True, False, False, 0.0)),
        (step._step_op, (v[:, 0].contiguous(), lv[:, 0].contiguous(), k[:, 0].contiguous(), q[:, 0].contiguous(),
                         a, p, (torch.rand(B, M, S) + 0.5).to(cuda), _rand(B, M, S, seed=13).to(cuda), False)),
    ]
    with torch.no_grad():
        for op, args in cases:
            print(f"[dispatch] {op._qualname}", flush=True)
            _same(op(*args), _lib.call(op, *args))
            _same(op(*args), op.direct(*args))
    # With an input that requires grad, _lib.call goes through the dispatcher:
    # the output carries the op's autograd node.
    xx = x.clone().requires_grad_(True)
    y, _ = _lib.call(conv._conv_op, xx, None, w, bias, 1)
    assert y.grad_fn is not None
    # Parameters count as plain tensors: under no_grad a module's weights take the
    # direct path too (no autograd node, the same values).
    pw = torch.nn.Parameter(w.clone())
    calls = []
    direct = conv._conv_op.direct
    conv._conv_op.direct = lambda *a: calls.append(1) or direct(*a)
    try:
        with torch.no_grad():
            y2, _ = _lib.call(conv._conv_op, x, None, pw, bias, 1)
    finally:
        conv._conv_op.direct = direct
    assert calls == [1] and y2.grad_fn is None
    with torch.no_grad():
        _same(y2, conv._conv_op(x, None, w, bias, 1)[0])


def test_ops_trace_under_torch_compile(cuda):
    """A function of the causal conv, the fused scan and the output tail compiled
    with torch.compile (aot_eager: dynamo and AOT autograd with the ops' fake
    functions, no code generation) returns what the eager function returns, and
    so do its input gradients."""
    from kla.ops import kla_scan
    from kla.ops.hip.conv import causal_conv_hip
    from kla.ops.hip.tail import gate_skip_hip

    B, L, M, S = 2, 64, 32, 16
    w, bias = _rand(M, 4, seed=1, scale=0.3).to(cuda), _rand(M, seed=2).to(cuda)
    k, q = _rand(B, L, S, seed=3, scale=0.3).to(cuda), _rand(B, L, S, seed=4, scale=0.3).to(cuda)
    a, p = (torch.rand(M, S) * 0.5 + 0.45).to(cuda), (torch.rand(M, S) * 0.05 + 0.01).to(cuda)
    lv = (torch.rand(B, L, M) + 0.5).to(cuda)
    gate = _rand(B, L, M, seed=5).to(cuda)

    def f(x):
        h, _ = causal_conv_hip(x, None, w, bias, "silu")
        y, y_var, _ = kla_scan(h, lv, k, q, a, p, backend="hip_fused")
        return gate_skip_hip(y, x, gate, torch.tensor(0.5, device=cuda), "silu"), y_var

    x = _rand(B, L, M, seed=6).to(cuda)
    outs = []
    for fn in (f, torch.compile(f, backend="aot_eager", fullgraph=False)):
        xx = x.clone().requires_grad_(True)
        out, y_var = fn(xx)
        (out.square().sum() + y_var.sum()).backward()
        outs.append((out.detach(), y_var.detach(), xx.grad))
    for name, e, c in zip(("out", "y_var", "dx"), *outs):
        torch.testing.assert_close(c, e, rtol=1e-6, atol=1e-6, msg=name)


def test_stream_handle_is_torchs_current_stream(cuda):
    """_lib.stream (the handle every launch passes) is the value of
    torch.cuda.current_stream(device).cuda_stream: on the default stream, on a
    side stream, and under graph capture (the capture stream)."""
    assert _lib.stream(cuda) == torch.cuda.current_stream(cuda).cuda_stream
    side = torch.cuda.Stream(cuda)
    with torch.cuda.stream(side):
        assert _lib.stream(cuda) == side.cuda_stream
        assert _lib.stream(torch.device("cuda")) == side.cuda_stream
    assert _lib.stream(cuda) == torch.cuda.current_stream(cuda).cuda_stream
    x = torch.ones(4, device=cuda)
    g = torch.cuda.CUDAGraph()
    seen = []
    side.wait_stream(torch.cuda.current_stream(cuda))
    with torch.cuda.stream(side):
        with torch.cuda.graph(g):
            seen.append((_lib.stream(cuda), torch.cuda.current_stream(cuda).cuda_stream))
            y = x * 2
    torch.cuda.current_stream(cuda).wait_stream(side)
    g.replay()
    torch.cuda.synchronize()
    assert seen[0][0] == seen[0][1]
    assert torch.equal(y, torch.full_like(x, 2.0))
