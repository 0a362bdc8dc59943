"""CPU models of the cross-work-group protocols the kernels use, run over
every interleaving of a few work-groups (exhaustive for small counts,
randomised for larger ones).  They check the design, not the GPU code:

* split-K combine (decode3.hip, the split prefill kernel in prefill.hip):
  every work-group stores its partial (o, m, l), waits for the stores, then
  adds one to its head's arrival counter; the one that reads n-1 resets the
  counter and merges all partials in split order, its own from registers.
  Nobody waits on another work-group, so every interleaving terminates;
  exactly one work-group merges; the counter is 0 again after the launch, so
  the next launch starts clean; the merged bytes do not depend on the order
  of arrival.
* the whole-block prefill merge (prefill_block_kernel): two halves, a barrier,
  half 1's rows in LDS, half 0 merges in half order: the same merge, fixed
  order.

The merge arithmetic is the kernels' (exp2 of the difference to the running
max, fp32 throughout); a planted mistake (merging in arrival order) makes
the order-independence check fail, so the check has teeth.
"""
from __future__ import annotations

import itertools

import numpy as np
import pytest


def merge(parts, order):
    """The kernels' ordered merge of partials (m, l, o): running max M, scale
    factors exp2(M - Mn) and exp2(m - Mn), fp32."""
    f = np.float32
    M, L = f(-np.inf), f(0.0)
    acc = np.zeros_like(parts[0][2])
    for i in order:
        m, l, o = parts[i]
        Mn = max(M, m)
        fo = np.exp2(f(M - Mn)) if M != -np.inf else f(0.0)
        fs = np.exp2(f(m - Mn)) if m != -np.inf else f(0.0)
        acc = (acc * fo + o * fs).astype(np.float32)
        L = f(L * fo + l * fs)
        M = Mn
    return acc / L


def run_launch(parts, arrival, counter, merge_in_arrival_order=False):
    """One launch under a given arrival order.  Returns (who merged, result)
    and leaves the counter as the kernel would."""
    n = len(parts)
    stored = [False] * n
    mergers, result = [], None
    for s in arrival:
        stored[s] = True                      # stores acknowledged before the add
        old = counter[0]
        counter[0] += 1                       # the atomic add returns the old value
        if old == n - 1:
            counter[0] = 0                    # the merger resets it
            assert all(stored), "a partial was read before its stores were acknowledged"
            mergers.append(s)
            order = list(arrival) if merge_in_arrival_order else list(range(n))
            result = merge(parts, order)
    return mergers, result


def random_parts(rng, n, width=8, spread=2.0):
    parts = []
    for _ in range(n):
        m = np.float32(rng.normal(0, spread))
        parts.append((m, np.float32(rng.uniform(1, 50)), rng.standard_normal(width).astype(np.float32) * 30))
    return parts


@pytest.mark.parametrize("n", [1, 2, 3, 4, 5])
def test_split_combine_every_order(n):
    rng = np.random.default_rng(n)
    parts = random_parts(rng, n)
    counter = [0]
    ref = None
    for arrival in itertools.permutations(range(n)):
        mergers, res = run_launch(parts, arrival, counter)
        assert mergers == [arrival[-1]], "exactly one merger, the last to arrive"
        assert counter[0] == 0, "the counter is back to 0 for the next launch"
        ref = res if ref is None else ref
        assert res.tobytes() == ref.tobytes(), "merged bytes depend on the arrival order"


@pytest.mark.parametrize("n", [8, 32, 64])
def test_split_combine_random_orders(n):
    rng = np.random.default_rng(100 + n)
    parts = random_parts(rng, n)
    # one split with no key (m = -inf, l = 0, o = 0), as an empty split leaves it
    parts[n // 2] = (np.float32(-np.inf), np.float32(0.0), np.zeros(8, np.float32))
    counter = [0]
    ref = merge(parts, range(n))
    for _ in range(50):
        arrival = rng.permutation(n)
        mergers, res = run_launch(parts, arrival, counter)
        assert len(mergers) == 1 and counter[0] == 0
        assert res.tobytes() == ref.tobytes()
    # against fp64 softmax-weighted sum of the same partials
    m = np.array([p[0] for p in parts], np.float64)
    w = np.where(np.isfinite(m), np.exp2(m - m[np.isfinite(m)].max()), 0.0)
    num = sum(wi * p[2].astype(np.float64) for wi, p in zip(w, parts))
    den = sum(wi * float(p[1]) for wi, p in zip(w, parts))
    assert np.allclose(ref, num / den, rtol=1e-5, atol=1e-6)


def test_planted_arrival_order_merge_is_caught():
    """Merging in arrival order instead of split order changes the rounding:
    the order-independence check above would catch it."""
    rng = np.random.default_rng(7)
    parts = random_parts(rng, 6)
    counter = [0]
    outs = {run_launch(parts, p, counter, merge_in_arrival_order=True)[1].tobytes()
            for p in itertools.permutations(range(6))}
    assert len(outs) > 1


def test_consecutive_launches_start_clean():
    """Launches back to back on the same counter (stream order): each one's
    merger is its own last arrival and the counter is 0 between them."""
    rng = np.random.default_rng(3)
    counter = [0]
    for launch in range(20):
        n = int(rng.integers(1, 9))
        parts = random_parts(rng, n)
        mergers, res = run_launch(parts, rng.permutation(n), counter)
        assert len(mergers) == 1 and counter[0] == 0
        assert res.tobytes() == merge(parts, range(n)).tobytes()


def test_whole_block_two_halves():
    """prefill_block_kernel: half 0 merges its rows with half 1's in half
    order; a half with no key (the one-tile block) leaves half 0's rows
    exactly as they were."""
    rng = np.random.default_rng(9)
    h0, h1 = random_parts(rng, 2)
    assert merge([h0, h1], [0, 1]).tobytes() == merge([h0, h1], [0, 1]).tobytes()
    empty = (np.float32(-np.inf), np.float32(0.0), np.zeros(8, np.float32))
    alone = merge([h0, empty], [0, 1])
    assert alone.tobytes() == (h0[2] / h0[1]).astype(np.float32).tobytes()
