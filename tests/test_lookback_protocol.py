"""CPU emulation of the decoupled look-back protocol of the single-pass scans
(kalman-linear-attention_amd/csrc/lookback_scan.hpp), under adversarial schedules.

The GPU kernel cannot be single-stepped, so its cross-workgroup protocol is
restated here step for step and run by an explicit scheduler that interleaves
the workgroups at every memory operation on the shared workspace:

* tickets: each workgroup draws one ticket from the header word
  (epoch << 32 | tickets drawn) and maps it chunk-major to (chunk, tile); the
  last ticket of a launch opens the next epoch, so the workspace is zero-filled
  only once and never between launches;
* records: every published float travels in one 64-bit word tagged with
  epoch + 1; a word is valid only if its tag matches the running launch;
* look-back: a chunk polls its predecessor's carry; while only the
  predecessor's aggregate is out it passes on to the chunk before, then
  re-applies the aggregates it skipped in chain order -- which computes the same
  float32 chain as the sequential carry, whatever the schedule;
* carry-only launches publish no aggregates: a chunk waits on its
  predecessor's carry alone (the chain then advances one chunk per hop), which
  computes the same chain;
* give-up: a wait that exceeds the spin limit yields NaN and counts a failure
  in the header (instead of hanging); a header left in a state no launch leaves
  (a workspace that was not zero-filled) makes every workgroup count a failure
  and touch nothing else.

The scan monoid is the affine map x -> g x + u in float32, as in the affine
scans (scan_ops.hpp AffineFwd): compose((g2, u2), (g1, u1)) = (g2 g1, g2 u1 + u2),
apply((g, u), x) = g x + u. Each workgroup holds W waves of S steps of a tile
of lanes, as lookback_scan_kernel does.
"""

import random

import numpy as np
import pytest

F = np.float32
K = 2             # aggregate words per record (affine: g, u)
HEADER = 32       # header words


def compose(later, earlier):
    g2, u2 = later
    g1, u1 = earlier
    return (F(g2 * g1), F(g2 * u1 + u2))


def apply(agg, x):
    g, u = agg
    return F(g * x + u)


def word(tag, value):
    return (int(tag) << 32) | int(np.array(value, dtype=F).view(np.uint32))


def word_ok(w, tag):
    return (w >> 32) == tag


def word_val(w):
    return np.array(w & 0xFFFFFFFF, dtype=np.uint32).view(F)[()]


class Launch:
    """One launch of the look-back scan over g, u [batch, steps, lanes] (float32)."""

    def __init__(self, ws, g, u, h0, W, S, tile, max_spin, carry_only=False):
        self.ws, self.g, self.u, self.h0 = ws, g, u, h0
        self.carry_only = carry_only
        self.batch, self.steps, self.lanes = g.shape
        self.W, self.S, self.tile, self.max_spin = W, S, tile, max_spin
        self.tiles_per_batch = -(-self.lanes // tile)
        self.n_tiles = self.batch * self.tiles_per_batch
        self.n_chunks = -(-self.steps // (W * S))
        self.plane = self.n_tiles * tile
        self.grid = self.n_tiles * self.n_chunks
        self.h = np.full_like(g, np.nan)
        self.ticket_of = {}   # workgroup -> ticket drawn (for the scheduler's starvation policy)

    def rec(self, plane_index, chunk, slot):
        return HEADER + (plane_index * self.n_chunks + chunk) * self.plane + slot

    def workgroup(self, idx):
        """Generator: one workgroup; yields before every access to the shared workspace."""
        ws = self.ws
        yield
        old = ws[0]
        ws[0] = old + 1                                   # atomic fetch_add on the header
        ticket, epoch = old & 0xFFFFFFFF, old >> 32
        self.ticket_of[idx] = ticket
        if ticket == self.grid - 1:
            nxt = epoch + 1
            if nxt == 0xFFFFFFFF:
                nxt = 0
            yield
            ws[0] = nxt << 32                             # open the next epoch
        tag = epoch + 1
        if ticket >= self.grid:
            yield
            ws[1] += 1                                    # header in no state a launch leaves
            return
        chunk, tile = divmod(ticket, self.n_tiles)
        b, n0 = divmod(tile, self.tiles_per_batch)
        n0 *= self.tile
        s0 = chunk * self.W * self.S
        lanes = [n for n in range(n0, min(n0 + self.tile, self.lanes))]
        for li, n in enumerate(lanes):
            slot = tile * self.tile + li
            # Wave aggregates, then the chunk aggregate (wave 0 composes them in order).
            waves = []
            for w in range(self.W):
                agg = (F(1), F(0))
                for t in range(s0 + w * self.S, min(s0 + (w + 1) * self.S, self.steps)):
                    agg = compose((self.g[b, t, n], self.u[b, t, n]), agg)
                waves.append(agg)
            tot = waves[0]
            for a in waves[1:]:
                tot = compose(a, tot)
            if chunk == 0:
                carry = F(self.h0[b, n])
            else:
                for k in range(0 if self.carry_only else K):
                    yield
                    ws[self.rec(k, chunk, slot)] = word(tag, tot[k])
                carry = yield from self.look_back(chunk, slot, tag)
            if chunk + 1 < self.n_chunks:
                yield
                ws[self.rec(K, chunk, slot)] = word(tag, apply(tot, carry))
            # Re-walk: each wave starts from the carry with the earlier waves' aggregates applied.
            for w in range(self.W):
                x = carry
                for a in waves[:w]:
                    x = apply(a, x)
                for t in range(s0 + w * self.S, min(s0 + (w + 1) * self.S, self.steps)):
                    x = apply((self.g[b, t, n], self.u[b, t, n]), x)
                    self.h[b, t, n] = x

    def look_back(self, chunk, slot, tag):
        ws = self.ws
        j = chunk - 1
        spins = 0
        while True:
            yield
            cw = ws[self.rec(K, j, slot)]
            if word_ok(cw, tag):
                x = word_val(cw)
                break
            ready = not self.carry_only and j > 0
            if ready:
                aw = []
                for k in range(K):
                    yield
                    aw.append(ws[self.rec(k, j, slot)])
                ready = all(word_ok(w, tag) for w in aw)
            if ready:
                j -= 1
                continue
            spins += 1
            if spins > self.max_spin:
                yield
                ws[1] += 1
                return F(np.nan)
        for i in range(j + 1, chunk):
            aw = []
            for k in range(K):
                yield
                aw.append(ws[self.rec(k, i, slot)])
            x = apply(tuple(word_val(w) for w in aw), x)
        return x


def run(launch, policy, rng, resident=None, starve=None):
    """Start the workgroups in a policy-chosen order, at most ``resident`` at a
    time, and interleave them one workspace access at a time. ``starve``:
    (ticket, steps) -- the workgroup that drew that ticket is not scheduled for
    the given number of scheduler steps after drawing it (while others can run)."""
    gens = [launch.workgroup(i) for i in range(launch.grid)]
    order = list(range(launch.grid))
    if policy == "reverse":
        order.reverse()
    elif policy in ("random", "starve"):
        rng.shuffle(order)
    pending = list(order)
    live = []
    clock = 0
    started = {}
    resident = resident or launch.grid
    while pending or live:
        while pending and len(live) < resident:
            idx = pending.pop(0)
            started[idx] = clock
            live.append(idx)
        choices = live
        if starve is not None:
            held = [i for i in live if launch.ticket_of.get(i) == starve[0]]
            if held and clock - started[held[0]] < starve[1]:
                choices = [i for i in live if i != held[0]] or live
        if policy == "round_robin":
            idx = choices[clock % len(choices)]
        elif policy == "lifo":
            idx = choices[-1]
        else:
            idx = rng.choice(choices)
        clock += 1
        try:
            next(gens[idx])
        except StopIteration:
            live.remove(idx)


def sequential(g, u, h0):
    h = np.empty_like(g)
    x = h0.astype(F).copy()
    for t in range(g.shape[1]):
        x = (g[:, t] * x + u[:, t]).astype(F)
        h[:, t] = x
    return h


def inputs(batch, steps, lanes, seed):
    r = np.random.default_rng(seed)
    g = (1.0 / (1.0 + np.exp(-r.standard_normal((batch, steps, lanes))))).astype(F)
    u = r.standard_normal((batch, steps, lanes)).astype(F)
    h0 = r.standard_normal((batch, lanes)).astype(F)
    return g, u, h0


def new_workspace(launch_like):
    return [0] * (HEADER + (K + 1) * launch_like.n_chunks * launch_like.plane)


GEOM = dict(W=3, S=4, tile=4, max_spin=10**9)


@pytest.mark.parametrize("policy", ["in_order", "reverse", "random", "round_robin", "lifo"])
@pytest.mark.parametrize("resident", [None, 3])
@pytest.mark.parametrize("modes", ["aggregates", "carry_only", "alternating"])
def test_every_schedule_gives_the_sequential_chain_bit_for_bit(policy, resident, modes):
    """Three launches on one workspace, never re-zeroed, with new inputs each time
    (a stale record of the previous launch read as valid would show; with
    alternating modes a carry-only launch finds the aggregates of the launch
    before it): every schedule gives the value of the in-order run, and that is
    the per-step chain up to the reassociation inside a chunk."""
    rng = random.Random(7)
    ws = None
    for rep in range(3):
        g, u, h0 = inputs(2, 61, 7, seed=10 + rep)
        co = modes == "carry_only" or (modes == "alternating" and rep % 2 == 1)
        la = Launch(ws, g, u, h0, **GEOM, carry_only=co)
        if ws is None:
            ws = la.ws = new_workspace(la)
        run(la, policy, rng, resident=resident)
        assert ws[1] == 0, "a wait gave up"
        assert ws[0] == (rep + 1) << 32, "the last ticket opens the next epoch"
        ref = Launch(None, g, u, h0, **GEOM)
        ref.ws = new_workspace(ref)
        run(ref, "in_order", random.Random(0), resident=1)
        assert np.array_equal(la.h, ref.h)
        np.testing.assert_allclose(la.h, sequential(g, u, h0), rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("carry_only", [False, True])
def test_results_do_not_depend_on_the_schedule(carry_only):
    g, u, h0 = inputs(1, 97, 5, seed=2)
    base = None
    for seed in range(12):
        la = Launch(None, g, u, h0, **GEOM, carry_only=carry_only)
        la.ws = new_workspace(la)
        run(la, "random", random.Random(seed), resident=1 + seed % 4)
        if base is None:
            base = la.h
        assert np.array_equal(la.h, base), f"schedule {seed} changed the result"


def test_epoch_wraps_without_a_zero_tag():
    g, u, h0 = inputs(1, 30, 3, seed=3)
    la = Launch(None, g, u, h0, **GEOM)
    ws = new_workspace(la)
    ws[0] = (0xFFFFFFFE) << 32                # the last epoch before the wrap
    outs = []
    for _ in range(3):
        la = Launch(ws, g, u, h0, **GEOM)
        run(la, "random", random.Random(1))
        outs.append(la.h)
        assert ws[1] == 0
    assert ws[0] >> 32 == 2                   # 0xFFFFFFFE -> 0 (not 0xFFFFFFFF) -> 1 -> 2
    assert all(np.array_equal(h, outs[0]) for h in outs)


@pytest.mark.parametrize("carry_only", [False, True])
def test_a_starved_predecessor_makes_the_wait_give_up_with_nan(carry_only):
    g, u, h0 = inputs(1, 48, 1, seed=4)
    geom = dict(GEOM, max_spin=20)
    la = Launch(None, g, u, h0, **geom, carry_only=carry_only)
    la.ws = new_workspace(la)
    # The workgroup holding ticket 0 (chunk 0, which publishes the first carry) stalls
    # after drawing it, for longer than its successors' spin limit.
    run(la, "in_order", random.Random(0), starve=(0, 10**4))
    assert la.ws[1] > 0, "no wait gave up"
    assert np.isnan(la.h[0, -1, 0]), "a given-up carry must poison the chunk (NaN), not be guessed"
    assert np.isfinite(la.h[0, :geom["W"] * geom["S"], 0]).all(), "chunk 0 needs no carry"


def test_a_workspace_that_was_not_zero_filled_is_detected():
    g, u, h0 = inputs(1, 24, 2, seed=5)
    la = Launch(None, g, u, h0, **GEOM)
    ws = new_workspace(la)
    ws[0] = (5 << 32) | 1000                  # tickets beyond any grid: garbage, not a launch's leftover
    la = Launch(ws, g, u, h0, **GEOM)
    run(la, "in_order", random.Random(0))
    assert ws[1] == la.grid, "every workgroup counts the failure"
    assert np.isnan(la.h).all(), "and writes nothing"
