"""Pins of the oracle's received-buffer order and its expert-major grouping (oracle/moe_ref.py).

The reference builds the order in resihp/runtime/moe.py:193-212: every source
walks its destination devices in rank order and, per device, the experts in
ascending id, sending the pairs ``(token, slot)`` routed there in ascending
order; the all-to-all concatenates the sources.  It has no stored fixture for
this order, so the oracle is pinned by a hand-worked example and by the
invariants that determine the order completely: every received row is a pair
of its chunk's source routed to its chunk's expert, chunks come source-major
then expert-major, rows ascend within a chunk, and every such pair arrives.
"""

from __future__ import annotations

import numpy as np
import pytest

from oracle import moe_ref as M
from resihp_megatron_amd.placement import smooth_weighted_round_robin


def test_received_rows_hand_worked():
    # two sources, k = 2, E = 4; this device holds experts 1 and 3
    s0 = np.array([[1, 3], [0, 1], [3, 2]])     # pairs (t, j): (0,0)->1 (0,1)->3 (1,1)->1 (2,0)->3
    s1 = np.array([[3, 1], [2, 0]])             # (0,0)->3 (0,1)->1
    src, tok, slot, counts = M.received_rows([s0, s1], [3, 1])
    # source 0: expert 1: (0,0) (1,1); expert 3: (0,1) (2,0); source 1: expert 1: (0,1); expert 3: (0,0)
    assert src.tolist() == [0, 0, 0, 0, 1, 1]
    assert tok.tolist() == [0, 1, 0, 2, 0, 0]
    assert slot.tolist() == [0, 1, 1, 0, 1, 0]
    assert counts.tolist() == [[2, 2], [1, 1]]
    plan = M.recv_plan(counts)
    # expert-major: expert 1 from source 0 (rows 0, 1) then source 1 (row 4); expert 3: rows 2, 3, 5
    assert plan["sort_row"].tolist() == [0, 1, 4, 2, 3, 5]
    assert plan["offsets"].tolist() == [0, 3, 6]
    assert plan["unsort_row"].tolist() == [0, 1, 3, 4, 2, 5]


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_received_rows_invariants(seed):
    rng = np.random.default_rng(seed)
    E, k, n_src = 12, 3, 5
    topis = [np.stack([rng.choice(E, k, replace=False) for _ in range(rng.integers(0, 40))]).reshape(-1, k)
             if seed != 2 or s != 1 else np.zeros((0, k), np.int64) for s in range(n_src)]
    local = [2, 5, 6, 11]
    src, tok, slot, counts = M.received_rows(topis, local)
    q = 0
    for s in range(n_src):
        for i, e in enumerate(local):
            expect = [(t, j) for t in range(topis[s].shape[0]) for j in range(k) if topis[s][t, j] == e]
            got = list(zip(tok[q:q + counts[s, i]].tolist(), slot[q:q + counts[s, i]].tolist()))
            assert got == expect and all(src[q:q + counts[s, i]] == s)
            q += counts[s, i]
    assert q == src.size


def test_received_rows_replicated_expert_split():
    """A replicated expert's pairs split over its holders by smooth weighted round robin
    (resihp/plan/expert_placement.py:150-164; the reference's own known answer: weights 10 and 5
    give 20 and 10 of 30 pairs, tests/unit/test_expert_placement.py:52-54)."""
    topis = [np.full((15, 2), 4)]        # 30 pairs, all to expert 4
    picks = smooth_weighted_round_robin(["x", "y"], {"y": 0.5}, 30)
    assert picks.count("x") == 20 and picks.count("y") == 10
    for me in ("x", "y"):
        src, tok, slot, counts = M.received_rows(topis, [4], assign=lambda s, e, n: [p == me for p in picks[:n]])
        mine = [i for i, p in enumerate(picks) if p == me]
        assert counts.tolist() == [[len(mine)]]
        assert (tok * 2 + slot).tolist() == mine


@pytest.mark.parametrize("shape", [(1, 1), (3, 4), (8, 16), (5, 7)])
def test_recv_plan_by_chunk_walk(shape):
    """The expert-major grouping walks the chunks expert by expert, sources in order."""
    rng = np.random.default_rng(sum(shape))
    counts = rng.integers(0, 6, size=shape)
    counts[rng.random(shape) < 0.3] = 0
    plan = M.recv_plan(counts)
    starts = np.concatenate([[0], np.cumsum(counts.reshape(-1))])
    n_src, L = shape
    walk = [r for i in range(L) for s in range(n_src) for r in range(starts[s * L + i], starts[s * L + i + 1])]
    assert plan["sort_row"].tolist() == walk
    assert sorted(plan["unsort_row"].tolist()) == list(range(len(walk)))
    assert np.array_equal(plan["unsort_row"][plan["sort_row"]], np.arange(len(walk)))
    assert plan["offsets"].tolist() == [0] + np.cumsum(counts.sum(0)).tolist()
