"""The sending side of expert parallelism on the GPU (rhp_ep_send_plan, EPRuntime.send).

A source's send order (resihp/runtime/moe.py:189-207): each expert's pairs in (token, slot) order
are split over the expert's holders in the EP group by smooth_weighted_round_robin
(resihp/plan/expert_placement.py:150-164), then sent device-major, expert-major, (token, slot)
ascending, with counts[d, e] exchanged first.  The send plan must equal ``oracle.moe_ref.send_order``
bit for bit, and what every device receives from the sources must equal ``received_rows``.  The
full-size case is configuration 4's layer seen from all of its sources: 32768 tokens in 8 sources
of 4096, 128 experts, top-8 under a Zipf(1.1) selection prior, over 8 devices in a placement shaped
like the one planned after a failure (non-contiguous slot sets, the hot experts replicated on two or
three devices of unequal speeds).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from _helpers import DEV, say, zipf_prior
from oracle import moe_ref as M
from resihp_megatron_amd import kernels as K
from resihp_megatron_amd import moe
from resihp_megatron_amd import placement as PL

pytestmark = pytest.mark.gpu


def post_failure_placement(E: int, devices: list[str], hot: int, seed: int) -> PL.ExpertPlacement:
    """Every expert on one device of a shuffled round robin, then the ``hot`` most popular experts
    (the lowest ids under the Zipf prior) copied to one more device, expert 0 to two more."""
    rng = np.random.default_rng(seed)
    slots = {d: [] for d in devices}
    for i, e in enumerate(rng.permutation(E)):
        slots[devices[i % len(devices)]].append(int(e))
    for e in range(hot):
        others = [d for d in devices if e not in slots[d]]
        for d in rng.choice(others, size=2 if e == 0 else 1, replace=False):
            slots[str(d)].append(e)
    p = PL.ExpertPlacement(E, (tuple(devices),), {d: tuple(sorted(v)) for d, v in slots.items()})
    p.validate()
    return p


def zipf_topi(T: int, E: int, k: int, seed: int) -> np.ndarray:
    rng = np.random.default_rng(seed)
    keys = rng.standard_normal((T, E)) + zipf_prior(E).numpy()
    return np.argsort(-keys, axis=1, kind="stable")[:, :k].astype(np.int32)


def check_plan(plan: K.SendPlan, topi: np.ndarray, E: int, ep, holders_of, speeds) -> np.ndarray:
    order, counts = M.send_order(topi, E, ep, holders_of, speeds)
    P = order.size
    assert np.array_equal(plan.counts.cpu().numpy(), counts)
    offs = np.concatenate([[0], np.cumsum(counts.reshape(-1))])
    assert np.array_equal(plan.offsets.cpu().numpy(), offs)
    assert np.array_equal(plan.perm[:P].cpu().numpy(), order)
    row = plan.row.cpu().numpy()
    expect = np.full(topi.size, -1, np.int64)
    expect[order] = np.arange(P)
    assert np.array_equal(row, expect)
    return order


@pytest.mark.parametrize("n_src,T_src,E,k,n_dev", [(8, 4096, 128, 8, 8), (2, 300, 8, 2, 3)])
def test_send_plans_bit_exact_and_received_order(n_src, T_src, E, k, n_dev):
    devices = [f"n{i // 4}g{i % 4}" for i in range(n_dev)]
    placement = post_failure_placement(E, devices, hot=min(16, E // 2), seed=E + n_dev)
    speed_set = [1.0, 0.8, 1.25, 1.0, 0.5, 1.0, 1.5, 0.9]
    speeds = {d: speed_set[i % len(speed_set)] for i, d in enumerate(devices)}
    ep = devices   # the world order of the group's devices
    holders_of = lambda e: placement.group_holders(0, e)  # noqa: E731
    off, dev, rank, cnt = PL.send_tables(placement, 0, ep, speeds)
    tables = K.SendTables.from_lists(off, dev, rank, cnt, n_dev, DEV)
    topis = [zipf_topi(T_src, E, k, seed=1000 + s) for s in range(n_src)]
    sent = []
    for s, topi in enumerate(topis):
        say(f"send plan: source {s}, {T_src} tokens, E={E}, top-{k}, {n_dev} devices")
        plan = K.ep_send_plan(torch.from_numpy(topi).to(DEV), E, tables)
        torch.cuda.synchronize()
        order = check_plan(plan, topi, E, ep, holders_of, speeds)
        sent.append((order, plan.counts.cpu().numpy()))
    replicated = [e for e in range(E) if len(holders_of(e)) > 1]
    assert replicated and any(len(holders_of(e)) == 3 for e in replicated)
    for di, d in enumerate(devices):
        local = sorted(placement.slots[d])

        def assign(s, e, n, d=d):
            return [h == d for h in M.smooth_weighted_round_robin(holders_of(e), speeds, n)]

        src, tok, slot, rcounts = M.received_rows(topis, local, assign)
        got_src, got_pair = [], []
        for s, (order, counts) in enumerate(sent):
            lo = int(counts[:di].sum())
            chunk = order[lo:lo + int(counts[di].sum())]
            got_src.append(np.full(chunk.size, s))
            got_pair.append(chunk)
        got_src, got_pair = np.concatenate(got_src), np.concatenate(got_pair)
        assert np.array_equal(got_src, src)
        assert np.array_equal(got_pair // k, tok) and np.array_equal(got_pair % k, slot)
        assert np.array_equal(np.stack([c[di, local] for _, c in sent]), rcounts)


def test_send_plan_skips_unrouted_ids():
    E, k = 5, 3
    placement = PL.ExpertPlacement(E, (("a", "b"),), {"a": (0, 1, 2, 4), "b": (2, 3, 4)})
    speeds = {"a": 1.0, "b": 0.6}
    topi = zipf_topi(64, E, k, seed=3)
    topi[5, 1] = -1
    topi[9, 0] = E
    topi[9, 2] = 77
    tables = K.SendTables.from_lists(*PL.send_tables(placement, 0, ["a", "b"], speeds), 2, DEV)
    say("send plan with ids outside [0, E)")
    plan = K.ep_send_plan(torch.from_numpy(topi).to(DEV), E, tables)
    torch.cuda.synchronize()
    check_plan(plan, topi, E, ["a", "b"], lambda e: placement.group_holders(0, e), speeds)
    assert plan.row.cpu().numpy()[[5 * k + 1, 9 * k, 9 * k + 2]].tolist() == [-1, -1, -1]


def test_ep_runtime_send_rows_and_combine_of_returned_rows():
    cfg = moe.MoEConfig(hidden=32, ffn=16, num_experts=6, top_k=2, tokens=96, dtype=torch.float64, device=DEV)
    world = ["n0g0", "n0g1", "n1g0"]
    placement = PL.ExpertPlacement(6, (tuple(world),), {"n0g0": (0, 1, 2), "n0g1": (2, 3, 4, 0),
                                                         "n1g0": (5, 0, 1)})
    speeds = {"n0g0": 1.0, "n0g1": 0.7, "n1g0": 1.2}
    specs = moe.moe_specs(cfg)
    params = {key: torch.nn.Parameter(moe.init_param(cfg, s)) for key, s in specs.items() if s.trainable}
    rt = moe.EPRuntime(cfg, placement, "n0g1", world, None, None, params, speeds=speeds)
    x, _ = moe.batch(cfg, 0)
    say("EPRuntime.send, 3-device group with replicas")
    rows, counts, in_splits, plan, gates = rt.send(x)
    topi, _ = moe.route(cfg, x, params["router.weight"])
    t_np = topi.cpu().numpy()
    order, ref_counts = M.send_order(t_np, 6, world, lambda e: placement.group_holders(0, e), speeds)
    assert np.array_equal(counts.numpy(), ref_counts) and in_splits == ref_counts.sum(1).tolist()
    assert torch.equal(rows, x[torch.from_numpy(order // 2).to(DEV)])   # x.index_select(0, idx_i), moe.py:212
    assert torch.equal(rt.tokens_per_expert.cpu(), torch.bincount(topi.reshape(-1).cpu(), minlength=6).double())
    # the rows come back (here: any values in send order) and combine into token order (moe.py:225-226)
    back = torch.randn(rows.shape, dtype=torch.float64, generator=torch.Generator().manual_seed(2)).to(DEV)
    out = K.combine(back, x, gates, plan.dispatch.pair_row.new_tensor(t_np.astype(np.int32)), plan.row)
    idx_i = torch.from_numpy(order // 2).to(DEV)
    idx_j = torch.from_numpy(order % 2).to(DEV)
    ref = x + torch.zeros_like(x).index_add(0, idx_i, gates[idx_i, idx_j].unsqueeze(1) * back)
    assert torch.allclose(out, ref, rtol=0, atol=1e-12)
