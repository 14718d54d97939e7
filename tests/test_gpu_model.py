"""SequenceModel on the "hip" backend against the reference, and C5 at full size.

The golden model (vocab 64, d_model 32, 2 layers, d_state 4; seeded default
init) was run by the reference itself (tests/golden/make_layer_golden.py):
full-forward logits, a chunked stateful prefill with the per-layer state it
leaves, the step-by-step greedy decode logits and 16 generated token ids
(reference src/kla/models/sequence_model.py:150-173, :201-220). On the GPU the
hip model runs its own kernels for every part of that: the fused scan in the
prefill, the gather, norm, row-linear, conv/SSM step and argmax kernels in
decode, and the same decode captured as a HIP graph. Floating-point values are
compared at rtol 1e-5 with an absolute atol of 1e-6; token ids exactly.

C5 itself (vocab 50304, d_model 512, 6 layers, prefill 16 x 2048, 256 greedy
decode steps) is too large for the float64 oracle, so it is checked through
properties that do not depend on size: chunked prefill equals the full
forward, graph and eager decode choose the same tokens, every value is
finite, and the first decode step's logits agree with the torch backend run on
the same GPU from the same weights.
"""

import copy
import os

import numpy as np
import pytest
import torch

from kla import KLAConfig, KLALayer, ModelConfig, SequenceModel

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "layer_golden.npz")
RTOL, ATOL = 1e-5, 1e-6


def _close(name, got, want, rtol=RTOL, atol=ATOL):
    got = got.detach().double().cpu().numpy()
    want = np.asarray(want, dtype=np.float64).reshape(got.shape)
    assert np.isfinite(got).all(), f"{name}: non-finite values"
    worst = float((np.abs(got - want) / (atol + rtol * np.abs(want))).max())
    print(f"  {name:14s} worst |d|/(atol+rtol|ref|) = {worst:.3f}", flush=True)
    assert worst <= 1.0, f"{name}: outside rtol={rtol} atol={atol} (ratio {worst:.3f})"


@pytest.fixture(scope="module")
def golden():
    with np.load(GOLDEN, allow_pickle=False) as z:
        return {k: z[k] for k in z.files if k.startswith("model/")}


def _golden_model(cuda, golden):
    """The golden model with the reference's own parameters loaded (the seeded draw
    order itself is pinned on the CPU by tests/test_golden_layer.py; a different
    host CPU may round torch's initialisers differently in the last bit)."""
    model = SequenceModel(ModelConfig(vocab_size=64, d_model=32, n_layers=2), KLAConfig(d_state=4, backend="hip"))
    sd = {k[len("model/param/"):]: torch.from_numpy(v) for k, v in golden.items() if k.startswith("model/param/")}
    assert sorted(sd) == sorted(model.state_dict())
    model.load_state_dict(sd)
    return model.to(cuda).eval()


def test_golden_model_logits_on_hip(cuda, golden):
    """Full-forward logits of the seeded golden model on hip = the reference's."""
    model = _golden_model(cuda, golden)
    with torch.no_grad():
        logits = model(torch.from_numpy(golden["model/ids"]).to(cuda))
    _close("logits", logits, golden["model/logits"])


@pytest.mark.parametrize("cuda_graph", [False, True])
def test_golden_model_prefill_and_generate_on_hip(cuda, golden, cuda_graph):
    """Chunked stateful prefill, per-layer state, greedy decode logits and the 16
    generated ids of the golden model on hip (eager, and with the decode step
    replayed as a HIP graph) = the reference's."""
    model = _golden_model(cuda, golden)
    gids = torch.from_numpy(golden["model/gen_ids"]).to(cuda)
    with torch.no_grad():
        state = model.init_state(2)
        l1, state = model(gids[:, :5], state=state)
        l2, state = model(gids[:, 5:], state=state)
        _close("chunk logits", torch.cat([l1, l2], 1), golden["model/chunk_logits"])
        for i, st in enumerate(state):
            _close(f"lam[{i}]", st.ssm.lam, golden[f"model/prefill_lam/{i}"])
            _close(f"eta[{i}]", st.ssm.eta, golden[f"model/prefill_eta/{i}"])
        gen = model.generate(gids, 16, temperature=0.0, cuda_graph=cuda_graph)
    np.testing.assert_array_equal(gen.cpu().numpy(), golden["model/generate"])
    # The decode logits step by step, through the one-token kernels.
    want_gen = torch.from_numpy(golden["model/generate"]).to(cuda)
    with torch.no_grad():
        state = model.init_state(2)
        logits, state = model(gids, state=state)
        steps = [logits[:, -1]]
        if cuda_graph:
            from kla.models.decode_graph import DecodeGraph

            graph = DecodeGraph(model, state)
        for t in range(15):
            tok = want_gen[:, 8 + t: 9 + t]
            if cuda_graph:
                logits = graph.step(tok)
            else:
                logits, state = model(tok, state=state)
            steps.append(logits[:, -1].clone())   # a graph's output buffer is overwritten by the next replay
    _close("decode logits", torch.stack(steps, 1), golden["model/decode_logits"])


# ------------------------------------------------------------------ C5 at full size

C5_VOCAB, C5_D, C5_LAYERS = 50304, 512, 6
C5_BATCH, C5_PREFILL, C5_DECODE = 16, 2048, 256


def test_c5_full_size_prefill_and_decode(cuda):
    """C5 on hip: prefill 16 x 2048 in one pass and in two stateful chunks, then
    256 greedy decode steps eagerly and as a HIP graph."""
    torch.manual_seed(0)
    model = SequenceModel(ModelConfig(vocab_size=C5_VOCAB, d_model=C5_D, n_layers=C5_LAYERS),
                          KLAConfig(backend="hip")).to(cuda).eval()
    ids = torch.randint(0, C5_VOCAB, (C5_BATCH, C5_PREFILL), generator=torch.Generator().manual_seed(5)).to(cuda)
    half = C5_PREFILL // 2
    with torch.no_grad():
        print("[c5] full forward", flush=True)
        full = model(ids)
        assert torch.isfinite(full).all()
        print("[c5] chunked prefill", flush=True)
        state = model.init_state(C5_BATCH)
        l1, state = model(ids[:, :half], state=state)
        l2, state = model(ids[:, half:], state=state)
        scale = float(full.abs().max())
        for name, got, want in (("first half", l1, full[:, :half]), ("second half", l2, full[:, half:])):
            err = float((got - want).abs().max())
            print(f"  {name}: max |d| = {err:.3e} (scale {scale:.3e})", flush=True)
            assert err <= 1e-4 * scale, name
        del full, l1
        last = l2[:, -1].clone()
        del l2
        for st in state:
            assert torch.isfinite(st.ssm.lam).all() and torch.isfinite(st.ssm.eta).all()

        # The first decode step against the torch backend on the same weights and prefill.
        print("[c5] torch-backend prefill and first decode step", flush=True)
        ref = copy.deepcopy(model)
        for layer in ref.modules():
            if isinstance(layer, KLALayer):
                layer.config = KLAConfig(backend="torch")
            if hasattr(layer, "backend"):
                layer.backend = "torch"
        ref.norm_f.backend = "torch"
        st_r = ref.init_state(C5_BATCH)
        lr, st_r = ref(ids, state=st_r)
        scale = float(lr[:, -1].abs().max())
        err = float((last - lr[:, -1]).abs().max())
        print(f"  last prefill logits vs torch: max |d| = {err:.3e} (scale {scale:.3e})", flush=True)
        assert err <= 1e-4 * scale
        tok = last.argmax(-1, keepdim=True)
        st_h = [copy.deepcopy(s) for s in state]
        oh, st_h = model(tok, state=st_h)
        orf, st_r = ref(tok, state=st_r)
        del ref, st_r, lr
        scale = float(orf.abs().max())
        err = float((oh - orf).abs().max())
        print(f"  first decode logits vs torch: max |d| = {err:.3e} (scale {scale:.3e})", flush=True)
        assert err <= 1e-4 * scale

        print(f"[c5] {C5_DECODE} greedy decode steps, eager and graph", flush=True)
        eager = model.generate(ids, C5_DECODE, temperature=0.0)
        graph = model.generate(ids, C5_DECODE, temperature=0.0, cuda_graph=True)
        assert eager.shape == (C5_BATCH, C5_PREFILL + C5_DECODE)
        assert torch.equal(eager[:, :C5_PREFILL], ids)
        assert torch.equal(eager, graph)
        assert int(eager.min()) >= 0 and int(eager.max()) < C5_VOCAB


@pytest.mark.parametrize("mc_samples", [8])
def test_mc_readout_matches_torch_backend(cuda, mc_samples):
    """SequenceModel.logprobs with a Monte-Carlo read-out (reference
    src/kla/models/readout.py:34-89, sequence_model.py:175): the model's mixers
    emit their variance (KLAConfig(return_variance=True)), so on "hip" the fused
    scan's y_var feeds the sampled read-out. The deterministic and MC
    log-probabilities against the same weights on backend "torch" on the same
    GPU, with the same seeded generator (the same eps draws), at rtol 1e-5 /
    atol 1e-6; and both against float64 on the CPU for the deterministic part."""
    torch.manual_seed(3)
    cfg = ModelConfig(vocab_size=128, d_model=64, n_layers=2)
    hip = SequenceModel(cfg, KLAConfig(d_state=8, return_variance=True, backend="hip")).to(cuda).eval()
    ref = copy.deepcopy(hip)
    for layer in ref.modules():
        if isinstance(layer, KLALayer):
            layer.config = KLAConfig(d_state=8, return_variance=True, backend="torch")
        if hasattr(layer, "backend"):
            layer.backend = "torch"
    ref.norm_f.backend = "torch"
    ids = torch.randint(0, 128, (2, 48), generator=torch.Generator().manual_seed(4)).to(cuda)
    outs = []
    with torch.no_grad():
        for model in (hip, ref):
            gen = torch.Generator(device=cuda).manual_seed(5)
            det, mc = model.logprobs(ids, mc_samples=mc_samples, generator=gen)
            assert mc is not None and mc.shape == det.shape == (2, 48, 128)
            outs.append((det, mc))
        det64, _ = copy.deepcopy(ref).double().cpu().logprobs(ids.cpu(), mc_samples=0)
    (dh, mh), (dr, mr) = outs
    # The MC mixture differs from the deterministic read-out (the variance is used).
    assert float((mh - dh).abs().max()) > 1e-4
    _close("det vs torch", dh, dr.cpu().numpy())
    _close("mc vs torch", mh, mr.cpu().numpy())
    _close("det vs float64", dh, det64.numpy())
    _close("det torch vs f64", dr, det64.numpy())


def test_c5_prefill_logits_against_float64(cuda, monkeypatch):
    """C5's prefill on hip (fp32 GEMMs through torch, the fused scan and HIP glue)
    against the same model evaluated in float64 on the GPU: float64 GEMMs, and the
    reference layer's float32 scan inputs (kla_layer.py:224-231) evaluated by the
    scan in float64, on the same static dynamics (a_bar, p_bar) as the hip layers.
    The logits of the last position of every sequence, elementwise: the literal
    ratio under rtol 1e-5 / atol 1e-6 is printed; the bar is rtol 1e-5 with atol
    1e-5 max|logit| (six blocks of fp32 products over k = 512 to 1365 round at
    ~1e-6 of their terms)."""
    import kla.layers.kla_layer as kl
    from kla.ops import kla_scan as real_scan

    torch.manual_seed(0)
    model = SequenceModel(ModelConfig(vocab_size=C5_VOCAB, d_model=C5_D, n_layers=C5_LAYERS),
                          KLAConfig(backend="hip")).to(cuda).eval()
    ids = torch.randint(0, C5_VOCAB, (C5_BATCH, C5_PREFILL), generator=torch.Generator().manual_seed(5)).to(cuda)
    with torch.no_grad():
        print("[c5 f64] hip prefill", flush=True)
        got = model(ids)[:, -1].double()
        aq = [blk.mixer._compute_aq() for blk in model.blocks]
        ref = copy.deepcopy(model).double()
        for layer in ref.modules():
            if isinstance(layer, KLALayer):
                layer.config = KLAConfig(backend="torch")
            if hasattr(layer, "backend"):
                layer.backend = "torch"
        ref.norm_f.backend = "torch"
        calls = []

        def scan64(v, lv, k, q, a, p, **kw):
            a_h, p_h = aq[len(calls)]
            calls.append(1)
            return real_scan(v.double(), lv.double(), k.double(), q.double(), a_h.double(), p_h.double(), **kw)

        monkeypatch.setattr(kl, "kla_scan", scan64)
        print("[c5 f64] float64 prefill", flush=True)
        want = ref(ids)[:, -1]
        assert len(calls) == C5_LAYERS
    scale = float(want.abs().max())
    err = (got - want).abs()
    lit = float((err / (1e-6 + 1e-5 * want.abs())).max())
    bar = float((err / (1e-5 * scale + 1e-5 * want.abs())).max())
    print(f"  last-position logits vs float64: max |d| {float(err.max()):.3e} (scale {scale:.3e}); "
          f"literal rtol 1e-5 / atol 1e-6 ratio {lit:.3f}, rtol 1e-5 / atol 1e-5 max ratio {bar:.3f}", flush=True)
    assert bar <= 1.0


def _random_model(seed):
    """(ModelConfig, KLAConfig kwargs) drawn over the model's and the layer's options."""
    import random

    from test_gpu_backend import _random_layer

    r = random.Random(seed)
    _, kw = _random_layer(seed + 500)
    kw["return_variance"] = False   # the model reads out the mean only
    cfg = ModelConfig(vocab_size=r.choice([97, 256, 1000]), d_model=r.choice([24, 32, 48]),
                      n_layers=r.randint(1, 3), mlp=r.choice(["none", "swiglu", "gelu"]),
                      mlp_ratio=r.choice([2.0, 8.0 / 3.0, 4.0]), tie_embeddings=r.random() < 0.3,
                      logit_softcap=r.choice([None, 30.0]))
    return cfg, kw


@pytest.mark.parametrize("seed", range(8))
def test_random_models_match_float64(cuda, seed):
    """A SequenceModel with a randomly drawn model and layer configuration on hip
    against the same weights in float64 on the CPU (backend torch everywhere): the
    prefill logits of every position, the prefill state, and four decode steps
    (both models fed the float64 model's greedy tokens, so a near tie cannot make
    them diverge) at rtol 1e-5 / atol 1e-5 of each tensor's scale (fp32 products
    over the blocks round at ~1e-6 of their terms); the same steps replayed by a
    DecodeGraph from the prefill state give the eager hip logits bit for bit."""
    cfg, kw = _random_model(seed)
    print(f"[random model] seed={seed} {cfg} {kw}", flush=True)
    torch.manual_seed(seed)
    model = SequenceModel(cfg, KLAConfig(**kw, backend="hip")).to(cuda).eval()
    ref = copy.deepcopy(model).double().cpu()
    for m in ref.modules():
        if isinstance(m, KLALayer):
            m.config = KLAConfig(**kw, backend="torch")
        if hasattr(m, "backend"):
            m.backend = "torch"
    B, L = 2, 23
    ids = torch.randint(0, cfg.vocab_size, (B, L), generator=torch.Generator().manual_seed(seed + 7))

    def close(name, got, want):
        assert (got is None) == (want is None), name   # parts a configuration does not carry
        if want is None:
            return
        got = got.detach().double().cpu()
        assert got.shape == want.shape, name
        if not want.numel():   # e.g. the conv window of a width-1 conv
            return
        scale = max(float(want.abs().max()), 1e-30)
        ratio = float(((got - want).abs() / (1e-5 * scale + 1e-5 * want.abs())).max()) if want.numel() else 0.0
        print(f"  {name:14s} ratio {ratio:.3f}", flush=True)
        assert torch.isfinite(got).all() and ratio <= 1.0, f"{name}: ratio {ratio:.3f}"

    from kla.models.decode_graph import DecodeGraph

    with torch.no_grad():
        got, st = model(ids.to(cuda), state=model.init_state(B))
        want, st_ref = ref(ids, state=ref.init_state(B))
        close("prefill logits", got, want)
        for i, (a, b) in enumerate(zip(torch.utils._pytree.tree_leaves(st), torch.utils._pytree.tree_leaves(st_ref))):
            close(f"state[{i}]", a, b)
        graph = DecodeGraph(model, st)
        tok = want[:, -1:].argmax(-1)
        for step in range(4):
            got, st = model(tok.to(cuda), state=st)
            want, st_ref = ref(tok, state=st_ref)
            close(f"decode {step}", got, want)
            # The graph replays the same one-token step: the same bits.
            assert torch.equal(graph.step(tok.to(cuda)), got), f"graph decode {step}"
            tok = want[:, -1:].argmax(-1)
