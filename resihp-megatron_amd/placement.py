"""Expert placement types consumed by the MoE layer.

Mirrors the consumer-facing half of resihp/plan/expert_placement.py: the
``ExpertPlacement`` record (:21-51), ``expert_dp_groups`` (:142-147) and the
deterministic speed-proportional token split ``smooth_weighted_round_robin``
(:150-164), and the per-expert pick periods the GPU send plan applies it
with (``send_tables``).  The placement planner itself (``plan_expert_placement``) is
control-plane code and is not part of this package; any object with the same
fields works.
"""

from __future__ import annotations

from dataclasses import dataclass


@dataclass(frozen=True)
class ExpertPlacement:
    num_experts: int
    groups: tuple[tuple[str, ...], ...]
    slots: dict[str, tuple[int, ...]]

    def holders(self, expert: int) -> list[str]:
        return sorted(d for g in self.groups for d in g if expert in self.slots[d])

    def group_holders(self, group: int, expert: int) -> list[str]:
        return [d for d in self.groups[group] if expert in self.slots[d]]

    def group_of(self, device: str) -> int:
        return next(i for i, g in enumerate(self.groups) if device in g)

    def validate(self) -> None:
        for i, g in enumerate(self.groups):
            hosted = {e for d in g for e in self.slots[d]}
            if hosted != set(range(self.num_experts)):
                raise ValueError(f"EP group {i} misses experts {set(range(self.num_experts)) - hosted}")
            for d in g:
                if len(set(self.slots[d])) != len(self.slots[d]):
                    raise ValueError(f"{d} hosts duplicate copies")


def single_device(num_experts: int, device: str = "gpu0") -> ExpertPlacement:
    """Every expert on one device: the one-GPU layout."""
    return ExpertPlacement(num_experts, ((device,),), {device: tuple(range(num_experts))})


def expert_dp_groups(placement: ExpertPlacement) -> dict[tuple[str, ...], list[int]]:
    """Experts with identical holder sets share one gradient all-reduce group."""
    out: dict[tuple[str, ...], list[int]] = {}
    for e in range(placement.num_experts):
        out.setdefault(tuple(placement.holders(e)), []).append(e)
    return out


def smooth_weighted_round_robin(holders: list[str], speeds: dict[str, float], n: int) -> list[str]:
    """Deterministic speed-proportional assignment of ``n`` tokens to an expert's replicas.

    Weights are ``max(1, round(10 * speed))``; each step every holder gains its
    weight and the largest (ties to the larger name) is picked and pays the total.
    """
    if len(holders) == 1:
        return holders * n
    weights = {h: max(1, round(10 * speeds.get(h, 1.0))) for h in holders}
    total = sum(weights.values())
    current = {h: 0 for h in holders}
    out = []
    for _ in range(n):
        for h in holders:
            current[h] += weights[h]
        pick = max(holders, key=lambda h: (current[h], h))
        current[pick] -= total
        out.append(pick)
    return out


def holder_period(holders: list[str], speeds: dict[str, float]) -> list[str]:
    """One period of ``smooth_weighted_round_robin`` over ``holders``.

    Over W = sum of the weights picks every holder is picked exactly its weight's number of times
    and the running weights return to zero, so the picks repeat with period W; this is checked on
    two periods.  One holder: a period of one.
    """
    if len(holders) == 1:
        return list(holders)
    W = sum(max(1, round(10 * speeds.get(h, 1.0))) for h in holders)
    picks = smooth_weighted_round_robin(holders, speeds, 2 * W)
    if picks[:W] != picks[W:]:
        raise AssertionError(f"round robin over {holders} does not repeat after {W} picks")
    return picks[:W]


def send_tables(placement: ExpertPlacement, group: int, ep: list[str], speeds: dict[str, float] | None = None):
    """The pick periods of every expert for the EP group ``group``, whose devices ``ep`` are listed in
    send order (world order, resihp/runtime/moe.py:180, 199): ``(pick_off, pick_dev, pick_rank,
    period_cnt)`` as int lists.  Expert e's period is positions ``pick_off[e] .. pick_off[e + 1]``;
    position r sends to ``ep[pick_dev[r]]`` as that device's ``pick_rank[r]``-th pick of the period;
    ``period_cnt[e * len(ep) + d]`` counts device d's picks.  An expert with no holder in the group
    raises (the reference cannot dispatch it either)."""
    speeds = speeds or {}
    index = {d: i for i, d in enumerate(ep)}
    n = len(ep)
    off, dev, rank, cnt = [0], [], [], [0] * (placement.num_experts * n)
    for e in range(placement.num_experts):
        holders = placement.group_holders(group, e)
        if not holders:
            raise RuntimeError(f"expert {e} has no holder in EP group {group}")
        seen: dict[int, int] = {}
        for h in holder_period(holders, speeds):
            d = index[h]
            dev.append(d)
            rank.append(seen.get(d, 0))
            seen[d] = seen.get(d, 0) + 1
        for d, c in seen.items():
            cnt[e * n + d] = c
        off.append(len(dev))
    return off, dev, rank, cnt
