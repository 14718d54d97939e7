"""The restated layer and model against golden vectors written by the reference.

tests/golden/layer_golden.npz comes from tests/golden/make_layer_golden.py,
which imports the reference package (in the build container) and records, for
seeded default-initialised KLALayer / SequenceModel instances, every parameter
and the outputs on fixed inputs: full forward, stateful prefill (final lam,
eta) and one O(1) decode step. This pins what mathematics leaves open -- the
parameter draw order of reference src/kla/layers/kla_layer.py:131-148 and
src/kla/models/sequence_model.py:126-137 -- and the caller code around the scan.
"""

import os

import numpy as np
import pytest
import torch

from kla import KLAConfig, KLALayer, ModelConfig, SequenceModel

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "layer_golden.npz")

CASES = {
    "default": (32, dict(d_state=4), (2, 12, 32)),
    "mamba_zoh": (24, dict(d_state=8, value_rank="conv", var_rank="dt", discretization="zoh",
                           lambda_skip_mode="vector", bias=True), (2, 10, 24)),
    "noconv_prior": (16, dict(d_state=4, use_conv=False, decode_from_prior=True, return_variance=True), (1, 9, 16)),
}


@pytest.fixture(scope="module")
def golden():
    with np.load(GOLDEN, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def _first(y):
    return y[0] if isinstance(y, tuple) else y


@pytest.mark.parametrize("tag", sorted(CASES))
def test_layer_matches_reference(golden, tag):
    d_model, cfg, shape = CASES[tag]
    torch.manual_seed(0)
    layer = KLALayer(d_model, KLAConfig(backend="torch", **cfg))
    sd = layer.state_dict()
    names = sorted(k[len(tag) + 7:] for k in golden if k.startswith(f"{tag}/param/"))
    assert names == sorted(sd), "parameter / buffer names differ from the reference"
    for name in names:
        np.testing.assert_array_equal(sd[name].numpy(), golden[f"{tag}/param/{name}"], err_msg=name)
    x = torch.from_numpy(golden[f"{tag}/x"])
    with torch.no_grad():
        np.testing.assert_allclose(_first(layer(x)).numpy(), golden[f"{tag}/y"], rtol=1e-5, atol=1e-6)
        state = layer.init_state(shape[0])
        _, state = layer(x[:, : shape[1] // 2], state=state)
        np.testing.assert_allclose(state.ssm.lam.numpy(), golden[f"{tag}/prefill_lam"], rtol=1e-5, atol=1e-6)
        np.testing.assert_allclose(state.ssm.eta.numpy(), golden[f"{tag}/prefill_eta"], rtol=1e-5, atol=1e-6)
        step, _ = layer(x[:, shape[1] // 2: shape[1] // 2 + 1], state=state)
        np.testing.assert_allclose(_first(step).numpy(), golden[f"{tag}/decode_y"], rtol=1e-5, atol=1e-6)


def test_sequence_model_matches_reference(golden):
    torch.manual_seed(0)
    model = SequenceModel(ModelConfig(vocab_size=64, d_model=32, n_layers=2), KLAConfig(d_state=4, backend="torch"))
    sd = model.state_dict()
    names = sorted(k[len("model/param/"):] for k in golden if k.startswith("model/param/"))
    assert names == sorted(sd)
    for name in names:
        np.testing.assert_array_equal(sd[name].numpy(), golden[f"model/param/{name}"], err_msg=name)
    with torch.no_grad():
        logits = _first(model(torch.from_numpy(golden["model/ids"])))
    np.testing.assert_allclose(logits.numpy(), golden["model/logits"], rtol=1e-5, atol=1e-6)


def test_sequence_model_stateful_prefill_and_generate_match_reference(golden):
    """Chunked stateful prefill (5 + 3 tokens), the per-layer state it leaves, the
    step-by-step greedy decode logits and the 16 generated token ids, all as the
    reference's SequenceModel.forward / generate wrote them (reference
    src/kla/models/sequence_model.py:150-173, :201-220). Token ids must match
    exactly; the golden script asserts a greedy margin above 1e-4."""
    torch.manual_seed(0)
    model = SequenceModel(ModelConfig(vocab_size=64, d_model=32, n_layers=2), KLAConfig(d_state=4, backend="torch"))
    gids = torch.from_numpy(golden["model/gen_ids"])
    with torch.no_grad():
        state = model.init_state(2)
        l1, state = model(gids[:, :5], state=state)
        l2, state = model(gids[:, 5:], state=state)
        np.testing.assert_allclose(torch.cat([l1, l2], 1).numpy(), golden["model/chunk_logits"], rtol=1e-5, atol=1e-6)
        for i, st in enumerate(state):
            np.testing.assert_allclose(st.ssm.lam.numpy(), golden[f"model/prefill_lam/{i}"], rtol=1e-5, atol=1e-6)
            np.testing.assert_allclose(st.ssm.eta.numpy(), golden[f"model/prefill_eta/{i}"], rtol=1e-5, atol=1e-6)
        gen = model.generate(gids, 16, temperature=0.0)
    np.testing.assert_array_equal(gen.numpy(), golden["model/generate"])
    with torch.no_grad():
        state = model.init_state(2)
        logits, state = model(gids, state=state)
        steps = [logits[:, -1]]
        for t in range(15):
            logits, state = model(gen[:, 8 + t: 9 + t], state=state)
            steps.append(logits[:, -1])
    np.testing.assert_allclose(torch.stack(steps, 1).numpy(), golden["model/decode_logits"], rtol=1e-5, atol=1e-6)
