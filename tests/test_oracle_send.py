"""Pins of the oracle's send order (oracle/moe_ref.py: smooth_weighted_round_robin, send_order) and the
host-side pick tables of the GPU send plan (placement.holder_period, placement.send_tables).

The reference builds the send order in resihp/runtime/moe.py:189-207 and splits a replicated
expert's pairs with smooth_weighted_round_robin (resihp/plan/expert_placement.py:150-164).  Its own
test of the round robin checks the split's counts only (tests/unit/test_expert_placement.py:52-54);
the sequence itself is pinned here by a hand-worked example and by the period property, and the
array form of the order by the literal restatement of the reference's loops, by its invariants and
by the received order (``received_rows``, pinned in test_oracle_recv.py) that the sources' sends
concatenate to.
"""

from __future__ import annotations

import numpy as np
import pytest

from oracle import moe_ref as M
from resihp_megatron_amd import placement as PL


def test_round_robin_reference_known_answer():
    # tests/unit/test_expert_placement.py:52-54 of the reference
    split = M.smooth_weighted_round_robin(["x", "y"], {"y": 0.5}, 30)
    assert split.count("x") == 20 and split.count("y") == 10
    assert M.smooth_weighted_round_robin(["z"], {}, 3) == ["z", "z", "z"]


def test_round_robin_hand_worked():
    # weights a 5, b 1, c 1 (total 7); running weights after adding, the pick, after paying:
    #   (5,1,1) a -> (-2,1,1); (3,2,2) a -> (-4,2,2); (1,3,3) tie b/c: the larger name c -> (1,3,-4)
    #   (6,4,-3) a -> (-1,4,-3); (4,5,-2) b -> (4,-2,-2); (9,-1,-1) a -> (2,-1,-1); (7,0,0) a -> (0,0,0)
    seq = M.smooth_weighted_round_robin(["a", "b", "c"], {"a": 0.5, "b": 0.1, "c": 0.1}, 14)
    assert seq[:7] == ["a", "a", "c", "a", "b", "a", "a"]
    assert seq[7:] == seq[:7]   # every running weight is back at zero after the total


@pytest.mark.parametrize("seed", range(6))
def test_round_robin_period_and_host_copy(seed):
    rng = np.random.default_rng(seed)
    holders = [f"n{i}g{j}" for i, j in rng.integers(0, 4, size=(int(rng.integers(2, 5)), 2))]
    holders = sorted(set(holders)) or ["n0g0", "n1g0"]
    speeds = {h: float(rng.choice([0.25, 0.5, 0.8, 1.0, 1.25, 1.5, 2.0])) for h in holders}
    W = sum(max(1, round(10 * speeds[h])) for h in holders)
    seq = M.smooth_weighted_round_robin(holders, speeds, 3 * W + 5)
    assert seq[W:2 * W] == seq[:W] and seq[2 * W:3 * W] == seq[:W]
    for h in holders:   # each holder is picked exactly its weight's number of times per period
        assert seq[:W].count(h) == max(1, round(10 * speeds[h]))
    # the product's copy (placement.py) and its period
    assert PL.smooth_weighted_round_robin(holders, speeds, 3 * W + 5) == seq
    assert PL.holder_period(holders, speeds) == seq[:W]


def _random_placement(rng, E, devices, replicas):
    slots = {d: [] for d in devices}
    for e, d in enumerate(rng.permutation(E) % len(devices)):
        slots[devices[d]].append(e)
    for e in replicas:
        others = [d for d in devices if e not in slots[d]]
        for d in rng.choice(others, size=min(len(others), int(rng.integers(1, 3))), replace=False):
            slots[d].append(e)
    return PL.ExpertPlacement(E, (tuple(devices),), {d: tuple(sorted(v)) for d, v in slots.items()})


@pytest.mark.parametrize("seed", range(5))
def test_send_order_array_form_equals_literal(seed):
    rng = np.random.default_rng(100 + seed)
    E, k, T = 7, 2, 40
    devices = ["n0g1", "n0g0", "n1g0", "n1g1"]
    pl = _random_placement(rng, E, devices, replicas=[0, 3, 5])
    speeds = {"n0g1": 1.0, "n0g0": 0.8, "n1g0": 1.5, "n1g1": 0.5}
    topi = np.stack([rng.choice(E, size=k, replace=False) for _ in range(T)])
    ep = devices   # world order
    holders_of = lambda e: pl.group_holders(0, e)  # noqa: E731
    order, counts = M.send_order(topi, E, ep, holders_of, speeds)
    order_l, counts_l = M.send_order_literal(topi, E, ep, holders_of, speeds)
    assert np.array_equal(order, order_l) and np.array_equal(counts, counts_l)
    # invariants: every pair exactly once, chunk (d, e) holds pairs of e in ascending order
    assert np.array_equal(np.sort(order), np.arange(T * k))
    assert np.array_equal(counts.sum(0), np.bincount(topi.reshape(-1), minlength=E))
    flat = topi.reshape(-1)
    starts = np.concatenate([[0], np.cumsum(counts.reshape(-1))])
    for c in range(len(ep) * E):
        chunk = order[starts[c]:starts[c + 1]]
        assert (flat[chunk] == c % E).all() and (np.diff(chunk) > 0).all()
        d = ep[c // E]
        assert chunk.size == 0 or d in holders_of(c % E)


def test_send_order_single_device_is_the_dispatch_order():
    rng = np.random.default_rng(7)
    topi = np.stack([rng.choice(9, size=3, replace=False) for _ in range(50)])
    order, counts = M.send_order(topi, 9, ["g"], lambda e: ["g"], {})
    ref = M.dispatch(topi, 9)
    assert np.array_equal(order, ref["perm"]) and np.array_equal(counts[0], ref["counts"][:9])


def test_sends_concatenate_to_the_received_order():
    # three sources of one EP group send to the four devices; what each device receives, sources in
    # rank order, is received_rows with each replicated expert's pairs split by the round robin
    rng = np.random.default_rng(11)
    E, k = 6, 2
    devices = ["a", "b", "c", "d"]
    pl = _random_placement(rng, E, devices, replicas=[1, 4])
    speeds = {"a": 1.0, "b": 0.7, "c": 1.3, "d": 1.0}
    topis = [np.stack([rng.choice(E, size=k, replace=False) for _ in range(T)]) for T in (13, 17, 9)]
    holders_of = lambda e: pl.group_holders(0, e)  # noqa: E731
    sends = [M.send_order(t, E, devices, holders_of, speeds) for t in topis]
    for di, d in enumerate(devices):
        local = sorted(pl.slots[d])

        def assign(s, e, n, d=d):
            return [h == d for h in M.smooth_weighted_round_robin(holders_of(e), speeds, n)]

        src, tok, slot, rcounts = M.received_rows(topis, local, assign)
        got = []
        for s, (order, counts) in enumerate(sends):
            lo = counts[:di].sum()
            got += [(s, p // k, p % k) for p in order[lo:lo + counts[di].sum()]]
        assert got == list(zip(src.tolist(), tok.tolist(), slot.tolist()))
        assert np.array_equal(rcounts, np.stack([c[di, local] for _, c in sends]))


def test_send_tables_layout():
    pl = PL.ExpertPlacement(3, (("p", "q", "r"),), {"p": (0, 1), "q": (1, 2), "r": (0, 1)})
    speeds = {"p": 1.0, "q": 0.5, "r": 1.0}
    off, dev, rank, cnt = PL.send_tables(pl, 0, ["r", "p", "q"], speeds)
    # expert 0: holders p, r (weights 10, 10); expert 1: p, q, r (10, 5, 10); expert 2: q alone
    p0 = PL.holder_period(["p", "r"], speeds)
    p1 = PL.holder_period(["p", "q", "r"], speeds)
    idx = {"r": 0, "p": 1, "q": 2}
    assert off == [0, len(p0), len(p0) + len(p1), len(p0) + len(p1) + 1]
    assert dev == [idx[h] for h in p0] + [idx[h] for h in p1] + [2]
    for e, per in enumerate([p0, p1, ["q"]]):
        seg = slice(off[e], off[e + 1])
        for r, (d, rk) in enumerate(zip(dev[seg], rank[seg])):
            assert rk == dev[seg][:r].count(d)
        for h, d in idx.items():
            assert cnt[e * 3 + d] == per.count(h)
    with pytest.raises(RuntimeError):
        PL.send_tables(PL.ExpertPlacement(2, (("p",), ("q",)), {"p": (0, 1), "q": (0,)}), 1, ["q"], {})
