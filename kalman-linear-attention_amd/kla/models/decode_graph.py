"""O(1) decode with the whole one-token model step replayed as a HIP graph.

Eager decode launches a few hundred small kernels per token (norms,
projections, the conv window, the filter step, the MLP, the LM head), so it is
bound by launch overhead, not by the GPU. :class:`DecodeGraph` captures one
call ``model(token, state=state)`` once -- with the state copied back into the
same buffers at the end of the captured region -- and then serves every token
with a single graph replay. The captured work is exactly the eager step
(``SequenceModel.forward`` with a one-token input and a state), so results
match eager decode; only the launch path changes.
"""

from __future__ import annotations

import torch


def _flat(state):
    """Every tensor of a (nested) state, in a fixed order."""
    out = []

    def walk(x):
        if isinstance(x, torch.Tensor):
            out.append(x)
        elif isinstance(x, (list, tuple)):
            for y in x:
                walk(y)
        elif x is not None:
            raise TypeError(f"unexpected state element {type(x).__name__}")

    walk(state)
    return out


def _clone(state):
    if isinstance(state, torch.Tensor):
        return state.clone()
    if isinstance(state, tuple) and hasattr(state, "_fields"):
        return type(state)(*(_clone(x) for x in state))
    if isinstance(state, (list, tuple)):
        return type(state)(_clone(x) for x in state)
    return state


class DecodeGraph:
    """One-token decode step of ``model`` as a replayable HIP graph.

    ``state`` is the recurrent state after prefill (``model(ids, state=...)``);
    it is copied into buffers the graph owns. ``step(token)`` ([B, 1] int64 on
    the model's device) advances that state by one token and returns the
    logits [B, 1, vocab] (a buffer the next ``step`` overwrites).
    """

    def __init__(self, model, state, warmup: int = 2):
        if not torch.cuda.is_available():
            raise RuntimeError("DecodeGraph needs a GPU")
        self.model = model
        self.state = _clone(state)
        batch = _flat(self.state)[0].shape[0]
        device = next(model.parameters()).device
        self.token = torch.zeros(batch, 1, dtype=torch.long, device=device)
        static = _flat(self.state)

        def run():
            logits, new_state = model(self.token, state=self.state)
            for dst, src in zip(static, _flat(new_state)):
                if src is not dst:
                    dst.copy_(src)
            return logits

        # Layers whose one-token step can write its new state over the old one
        # (the hip decode kernels) do so here: the graph owns the state buffers,
        # so no copy-back is captured for them.
        in_place = [m for m in model.modules() if hasattr(m, "_decode_in_place")]
        flags = [m._decode_in_place for m in in_place]
        for m in in_place:
            m._decode_in_place = True

        try:
            # Warm up on a side stream (allocator pools, library handles), then
            # restore the prefill state and capture.
            saved = [t.clone() for t in static]
            side = torch.cuda.Stream(device)
            side.wait_stream(torch.cuda.current_stream(device))
            with torch.no_grad(), torch.cuda.stream(side):
                for _ in range(warmup):
                    run()
            torch.cuda.current_stream(device).wait_stream(side)
            with torch.no_grad():
                for dst, src in zip(static, saved):
                    dst.copy_(src)
            self.graph = torch.cuda.CUDAGraph()
            with torch.no_grad(), torch.cuda.graph(self.graph):
                self.logits = run()
        finally:
            for m, f in zip(in_place, flags):
                m._decode_in_place = f
        # Capture does not execute the work; the state is still the prefill state.

    @torch.no_grad()
    def step(self, token: torch.Tensor) -> torch.Tensor:
        self.token.copy_(token)
        self.graph.replay()
        return self.logits
