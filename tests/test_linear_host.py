"""Host-side logic of the split projections (no GPU): how many token chunks a
weight gradient is split into, how a weight is cut into row blocks, and that
the projections fall back to torch's nn.Linear where the HIP path does not
apply (CPU tensors, no gradient, a bias)."""

import torch

from kla.ops.hip import linear as lin


def test_split_count_fills_the_cus(monkeypatch):
    monkeypatch.setattr(lin, "_cus", lambda index: 256)
    dev = torch.device("cuda", 0)
    T = 16384
    # C4's weight-gradient shapes: 64, 32, 128 and 8 output tiles of 256 x 256.
    assert lin.split_count(T, 4096, 1024, dev) == 4
    assert lin.split_count(T, 1024, 2048, dev) == 8
    assert lin.split_count(T, 4096, 2048, dev) == 2
    assert lin.split_count(T, 32, 2048, dev) == 32
    # Enough tiles already, too few tokens, or tokens that do not divide: one GEMM.
    assert lin.split_count(T, 8192, 8192, dev) == 1
    assert lin.split_count(1000, 64, 64, dev) == 1
    assert lin.split_count(1536, 64, 64, dev) == 2      # chunks of 768, not 384
    assert lin.split_count(4097, 64, 64, dev) == 1
    for tokens in (2048, 6144, 16384, 65536):
        p = lin.split_count(tokens, 300, 300, dev)
        assert tokens % p == 0 and (p == 1 or tokens // p >= lin._MIN_CHUNK) and p <= lin._MAX_PARTS


def test_row_blocks():
    assert lin.row_blocks(4128) == [(0, 4096), (4096, 4128)]
    assert lin.row_blocks(4096) == [(0, 4096)]
    assert lin.row_blocks(200) == [(0, 200)]
    assert lin.row_blocks(257) == [(0, 256), (256, 257)]


def test_projections_fall_back_to_torch_on_cpu():
    mod = torch.nn.Linear(8, 12, bias=False)
    x = torch.randn(2, 5, 8, requires_grad=True)
    assert torch.equal(lin.linear(mod, x), mod(x))
    assert lin.linear_split(mod, x, [6, 6]) is None
    assert lin.linear_split(mod, x, [4, 4]) is None          # sizes must cover the rows
    assert lin._bf16_operands(torch.nn.Linear(8, 12), x) is None   # a bias
    with torch.no_grad():
        assert lin._bf16_operands(mod, x) is None


def test_split_backward_with_an_empty_piece_and_no_input_gradient(monkeypatch):
    """The mamba preset (value_rank='conv') splits sensor_proj as [0, rank, S, S]:
    without an input gradient each piece's gradient forms its own rows of dw, and
    the empty piece has none (reference src/kla/layers/kla_layer.py:206)."""
    monkeypatch.setattr(lin, "_cus", lambda index: 256)
    x = torch.randn(2, 5, 6)
    w = torch.randn(16, 6, requires_grad=True)
    sizes = [0, 8, 4, 4]
    pieces = lin._SplitLinear.apply(x, w, sizes)
    assert [p.shape[-1] for p in pieces] == sizes
    gs = [torch.randn(2, 5, s) for s in sizes]
    torch.autograd.backward([pieces[1], pieces[2], pieces[3]], [gs[1], gs[2], gs[3]])
    want = torch.cat(gs, -1).reshape(-1, 16).t() @ x.reshape(-1, 6)
    torch.testing.assert_close(w.grad, want)
