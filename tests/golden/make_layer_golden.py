"""Write tests/golden/layer_golden.npz from the REFERENCE package (run in the
build container only; the reference does not travel to the GPU box).

What it pins: the one thing about the layer that mathematics does not fix --
the order in which a seeded, default-initialised KLALayer / SequenceModel draws
its parameters (reference src/kla/layers/kla_layer.py:131-148,
src/kla/layers/common.py:30-42 and :76-80, src/kla/models/sequence_model.py:126-137)
-- together with the outputs those parameters give on fixed inputs. The scan
itself is pinned by tests/test_oracle_pins.py and is not imported from here.

    PYTHONDONTWRITEBYTECODE=1 python tests/golden/make_layer_golden.py [REFERENCE_SRC]

The reference is imported in a child interpreter whose sys.path holds only the
reference's src/ (so this repository's own `kla` cannot shadow it); the child
writes plain float arrays (np.savez, no pickles).
"""

import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
OUT = os.path.join(HERE, "layer_golden.npz")

CHILD = r'''
import sys
import numpy as np
import torch
sys.path.insert(0, sys.argv[1])
import kla
from kla import KLAConfig, KLALayer, ModelConfig, SequenceModel

out = {}
torch.set_num_threads(1)

def layer_case(tag, d_model, cfg_kwargs, shape):
    torch.manual_seed(0)
    layer = KLALayer(d_model, KLAConfig(backend="torch", **cfg_kwargs))
    g = torch.Generator().manual_seed(1)
    x = torch.randn(*shape, generator=g)
    for name, p in layer.state_dict().items():
        out[f"{tag}/param/{name}"] = p.detach().numpy().copy()
    out[f"{tag}/x"] = x.numpy()
    with torch.no_grad():
        y = layer(x)
        y = y[0] if isinstance(y, tuple) else y
        out[f"{tag}/y"] = y.numpy()
        state = layer.init_state(shape[0])
        y1, state = layer(x[:, : shape[1] // 2], state=state)
        y1 = y1[0] if isinstance(y1, tuple) else y1
        out[f"{tag}/prefill_lam"] = state.ssm.lam.numpy()
        out[f"{tag}/prefill_eta"] = state.ssm.eta.numpy()
        step, state = layer(x[:, shape[1] // 2 : shape[1] // 2 + 1], state=state)
        step = step[0] if isinstance(step, tuple) else step
        out[f"{tag}/decode_y"] = step.numpy()

layer_case("default", 32, dict(d_state=4), (2, 12, 32))
layer_case("mamba_zoh", 24, dict(d_state=8, value_rank="conv", var_rank="dt", discretization="zoh",
                                   lambda_skip_mode="vector", bias=True), (2, 10, 24))
layer_case("noconv_prior", 16, dict(d_state=4, use_conv=False, decode_from_prior=True, return_variance=True),
           (1, 9, 16))

torch.manual_seed(0)
model = SequenceModel(ModelConfig(vocab_size=64, d_model=32, n_layers=2), KLAConfig(d_state=4, backend="torch"))
ids = torch.randint(0, 64, (2, 10), generator=torch.Generator().manual_seed(2))
for name, p in model.state_dict().items():
    out[f"model/param/{name}"] = p.detach().numpy().copy()
out["model/ids"] = ids.numpy()
with torch.no_grad():
    logits = model(ids)
    logits = logits[0] if isinstance(logits, tuple) else logits
    out["model/logits"] = logits.numpy()

# Stateful chunked prefill (forward with state, reference sequence_model.py:150-173)
# and a 16-token greedy generate (:201-220). The decode logits are recorded step
# by step with the same loop generate runs, and the greedy choices must have a
# clear margin so that float32 reassociation cannot flip them.
gids = torch.randint(0, 64, (2, 8), generator=torch.Generator().manual_seed(3))
out["model/gen_ids"] = gids.numpy()
with torch.no_grad():
    state = model.init_state(2)
    l1, state = model(gids[:, :5], state=state)
    l2, state = model(gids[:, 5:], state=state)
    out["model/chunk_logits"] = torch.cat([l1, l2], 1).numpy()
    for i, st in enumerate(state):
        out[f"model/prefill_lam/{i}"] = st.ssm.lam.numpy()
        out[f"model/prefill_eta/{i}"] = st.ssm.eta.numpy()
    gen = model.generate(gids, 16, temperature=0.0)
    out["model/generate"] = gen.numpy()
    state = model.init_state(2)
    logits, state = model(gids, state=state)
    steps = [logits[:, -1]]
    for t in range(15):
        logits, state = model(gen[:, 8 + t : 9 + t], state=state)
        steps.append(logits[:, -1])
    steps = torch.stack(steps, 1)
    out["model/decode_logits"] = steps.numpy()
    assert torch.equal(steps.argmax(-1), gen[:, 8:]), "step-by-step decode differs from generate"
    top2 = steps.topk(2, dim=-1).values
    margin = float((top2[..., 0] - top2[..., 1]).min())
    print(f"smallest greedy margin {margin:.3e}")
    assert margin > 1e-4, "greedy choice too close to a tie for an exact token check"

np.savez(sys.argv[2], **out)
print(f"wrote {len(out)} arrays to {sys.argv[2]}")
'''


def main(argv):
    ref_src = argv[1] if len(argv) > 1 else "/root/reference/src"
    env = dict(os.environ, PYTHONDONTWRITEBYTECODE="1")
    env.pop("PYTHONPATH", None)
    return subprocess.call([sys.executable, "-I", "-c", CHILD, ref_src, OUT], env=env, cwd="/tmp")


if __name__ == "__main__":
    raise SystemExit(main(sys.argv))
