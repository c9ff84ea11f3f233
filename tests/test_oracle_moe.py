"""Pins of the float64 oracle (oracle/moe_ref.py) against the reference's own outputs and mathematics.

The fixtures in tests/golden/reference_moe.npz were written by
tests/golden/make_reference_vectors.py from resihp/runtime/moe.py itself.
"""

from __future__ import annotations

import itertools
import math
import pathlib

import numpy as np
import pytest
import torch

from oracle import moe_ref as M

GOLD = np.load(pathlib.Path(__file__).resolve().parent / "golden" / "reference_moe.npz")

CASES = {
    "default": M.OracleConfig(),
    "bias": M.OracleConfig(bias_update_rate=0.01),
    "wide": M.OracleConfig(hidden=16, ffn=32, num_experts=8, top_k=3, tokens=64, seed=77, bias_update_rate=0.05),
}


def test_derive_seed_matches_reference_values():
    for parts, val in zip(GOLD["derive_seed_parts"], GOLD["derive_seed_values"]):
        p = [int(v) for v in parts.decode().split(",")]
        assert M.derive_seed(*p) == int(val.decode())


def test_splitmix64_published_vector():
    # SplitMix64 seeded with 0: the first output is 0xE220A8397B1DCDAF (Steele, Lea, Flood 2014;
    # Vigna's reference splitmix64.c).  splitmix64(x) is the first output for state x.
    assert M.splitmix64(0) == 0xE220A8397B1DCDAF


@pytest.mark.parametrize("name", list(CASES))
def test_init_batch_route_match_reference(name):
    cfg = CASES[name]
    w = M.init_param(cfg, "router.weight", (cfg.num_experts, cfg.hidden), True)
    assert torch.equal(w, torch.from_numpy(GOLD[f"{name}/init/router.weight"]))
    x, y = M.batch(cfg, 0)
    assert torch.equal(x, torch.from_numpy(GOLD[f"{name}/x"]))
    assert torch.equal(y, torch.from_numpy(GOLD[f"{name}/y"]))
    bias = torch.zeros(cfg.num_experts, dtype=torch.float64) if M.has_bias(cfg) else None
    topi, gates = M.route(cfg, x, w, bias)
    assert torch.equal(topi, torch.from_numpy(GOLD[f"{name}/route/topi"]))
    torch.testing.assert_close(gates, torch.from_numpy(GOLD[f"{name}/route/gates"]), rtol=1e-14, atol=1e-15)


@pytest.mark.parametrize("name", list(CASES))
def test_forward_and_grads_match_reference(name):
    cfg = CASES[name]
    params = M.init_params(cfg)
    shapes = M.param_shapes(cfg)
    leaves = {k: torch.nn.Parameter(v.clone()) for k, v in params.items() if shapes[k][1]}
    bufs = {k: v.clone() for k, v in params.items() if not shapes[k][1]}
    x, y = M.batch(cfg, 0)
    xl = x.clone().requires_grad_(True)
    out = M.layer_forward(cfg, {**leaves, **bufs}, xl)
    (M.token_loss(out, y) / cfg.tokens).backward()
    torch.testing.assert_close(out.detach(), torch.from_numpy(GOLD[f"{name}/fwd/out"]), rtol=1e-12, atol=1e-13)
    torch.testing.assert_close(xl.grad, torch.from_numpy(GOLD[f"{name}/fwd/grad/x"]), rtol=1e-10, atol=1e-13)
    for k, p in leaves.items():
        torch.testing.assert_close(p.grad, torch.from_numpy(GOLD[f"{name}/fwd/grad/{k}"]), rtol=1e-10, atol=1e-13)
    for k, b in bufs.items():
        assert torch.equal(b, torch.from_numpy(GOLD[f"{name}/fwd/after/{k}"]))


@pytest.mark.parametrize("name", list(CASES))
def test_training_matches_reference(name):
    cfg = CASES[name]
    losses, final = M.reference_train(cfg, 8)
    np.testing.assert_allclose(losses, GOLD[f"{name}/train/losses"], rtol=1e-10)
    for k, v in final.items():
        torch.testing.assert_close(v, torch.from_numpy(GOLD[f"{name}/train/final/{k}"]), rtol=1e-10, atol=1e-12)


def test_selection_lowest_id_ties_and_nan():
    keys = torch.tensor([[1.0, 3.0, 3.0, 2.0, 3.0], [float("nan"), 0.0, 0.0, -1.0, float("nan")]])
    assert M.select(keys, 3).tolist() == [[1, 2, 4], [1, 2, 3]]


def test_selection_brute_force_small():
    # The chosen set maximises the key sum; with distinct keys it is unique, and
    # the order is descending.
    g = torch.Generator().manual_seed(3)
    for _ in range(50):
        E, k = 6, 3
        keys = torch.randn(1, E, generator=g, dtype=torch.float64)
        best = max(itertools.combinations(range(E), k), key=lambda c: sum(keys[0, i].item() for i in c))
        got = M.select(keys, k)[0].tolist()
        assert set(got) == set(best)
        assert all(keys[0, got[i]] > keys[0, got[i + 1]] for i in range(k - 1))


def test_dispatch_invariants_and_reference_order():
    rng = np.random.default_rng(0)
    T, k, E = 37, 3, 7
    topi = np.stack([rng.choice(E, k, replace=False) for _ in range(T)])
    d = M.dispatch(topi, E)
    assert d["counts"][:E].sum() == T * k and d["counts"][E] == 0
    assert sorted(d["perm"].tolist()) == list(range(T * k))
    # Reference order (moe.py:199-205 on one device): per expert, sorted (token, slot) pairs.
    ref = [t * k + j for e in range(E) for (t, j) in sorted((t, j) for t in range(T) for j in range(k)
                                                               if topi[t, j] == e)]
    assert d["perm"].tolist() == ref
    assert all(d["pair_row"][p] == r for r, p in enumerate(d["perm"]))


def test_dispatch_local_window_and_sources():
    rng = np.random.default_rng(1)
    T, k, E, e0, e1, n_src = 50, 2, 10, 3, 7, 4
    topi = np.stack([rng.choice(E, k, replace=False) for _ in range(T)])
    d = M.dispatch(topi, E, e0, e1, n_src)
    flat = topi.reshape(-1)
    local = np.flatnonzero((flat >= e0) & (flat < e1))
    assert d["perm"].size == local.size and d["offsets"][-1] == local.size
    assert (d["pair_row"][flat < e0] == -1).all() and (d["pair_row"][flat >= e1] == -1).all()
    # even_split(50, 4) = 13,13,12,12 tokens
    bounds = [0, 13, 26, 38, 50]
    for s in range(n_src):
        for i, e in enumerate(range(e0, e1)):
            assert d["src_counts"][s, i] == (topi[bounds[s]:bounds[s + 1]] == e).sum()


def test_swiglu_known_answer():
    # h = f = 1: x = 1, gate weight 2, up weight 3, fc2 = 1  ->  silu(2) * 3 = 6 / (1 + e^-2).
    x = torch.ones(1, 1, dtype=torch.float64)
    fc1 = torch.tensor([[2.0], [3.0]], dtype=torch.float64)
    fc2 = torch.ones(1, 1, dtype=torch.float64)
    y = M.expert_ffn(x, fc1, fc2, "swiglu")
    assert y.item() == pytest.approx(6.0 / (1.0 + math.exp(-2.0)), rel=1e-15)
    # Swapping the halves gives silu(3) * 2, a different number: the half order is observable.
    assert M.expert_ffn(x, fc1.flip(0), fc2, "swiglu").item() == pytest.approx(6.0 / (1.0 + math.exp(-3.0)))


def test_gelu_expert_matches_reference_shape_known_answer():
    # exact-erf GELU at 1: 0.5 * (1 + erf(1/sqrt 2)) = 0.8413447460685429
    x = torch.ones(1, 1, dtype=torch.float64)
    y = M.expert_ffn(x, torch.ones(1, 1, dtype=torch.float64), torch.ones(1, 1, dtype=torch.float64), "gelu")
    assert y.item() == pytest.approx(0.8413447460685429, rel=1e-15)


def test_sigmoid_gates_normalised_and_bias_selection_only():
    cfg = M.OracleConfig(hidden=8, num_experts=6, top_k=2, score="sigmoid")
    g = torch.Generator().manual_seed(5)
    x = torch.randn(20, 8, generator=g, dtype=torch.float64)
    w = torch.randn(6, 8, generator=g, dtype=torch.float64)
    bias = torch.zeros(6, dtype=torch.float64)
    bias[5] = 100.0
    topi, gates = M.route(cfg, x, w, bias)
    assert (topi[:, 0] == 5).all()
    torch.testing.assert_close(gates.sum(-1), torch.ones(20, dtype=torch.float64))
    s = torch.sigmoid(x @ w.t())
    torch.testing.assert_close(gates[:, 0] / gates[:, 1], s.gather(1, topi)[:, 0] / s.gather(1, topi)[:, 1])


def test_layer_gradcheck_tiny_swiglu_shared():
    cfg = M.OracleConfig(hidden=4, ffn=6, num_experts=3, top_k=2, tokens=5, act="swiglu", num_shared=1,
                         shared_ffn=4)
    params = {k: v.clone().requires_grad_(tr) for (k, v), tr in
              zip(M.init_params(cfg).items(), [t for _, (s, t) in M.param_shapes(cfg).items()])}
    x, _ = M.batch(cfg, 0)
    topi, _ = M.route(cfg, x, params["router.weight"])
    keys = [k for k, (_, tr) in M.param_shapes(cfg).items() if tr]

    def f(xx, *ws):
        return M.layer_forward(cfg, dict(zip(keys, ws)), xx, topi=topi)

    assert torch.autograd.gradcheck(f, (x.clone().requires_grad_(True), *[params[k] for k in keys]))


def test_amax_roll_newest_first_and_scale():
    h = torch.tensor([4.0, 3.0, 2.0, 1.0], dtype=torch.float64)
    assert M.amax_roll(h, torch.tensor(9.0)).tolist() == [9.0, 4.0, 3.0, 2.0]
    assert M.fp8_scale(h, "e4m3") == 448.0 / 4.0
    assert M.fp8_scale(torch.zeros(3), "e5m2") == 1.0


def test_quantize_saturates_and_rounds_to_nearest_even():
    x = torch.tensor([1000.0, -1000.0, 1.0625, 1.1875, 0.0], dtype=torch.float64)
    q = M.quantize(x, 1.0, "e4m3")
    # e4m3 spacing in [1, 2) is 1/8: 1.0625 ties to 1.0 (even), 1.1875 ties to 1.25.
    assert q.tolist() == [448.0, -448.0, 1.0, 1.25, 0.0]


def test_shared_expert_term_known_answer():
    """One token, top-1 (gate 1), GELU experts with h = f = 1: out = x + 2 gelu(1) (routed) + 3 gelu(1)
    (shared, gate 1, added after the routed sum).  gelu(1) = 0.8413447460685429."""
    cfg = M.OracleConfig(hidden=1, ffn=1, num_experts=2, top_k=1, tokens=1, act="gelu", num_shared=1, shared_ffn=1)
    one = lambda v: torch.tensor([[v]], dtype=torch.float64)  # noqa: E731
    params = {"router.weight": torch.tensor([[0.0], [1.0]], dtype=torch.float64),
              "experts.0.fc1.weight": one(7.0), "experts.0.fc2.weight": one(7.0),
              "experts.1.fc1.weight": one(1.0), "experts.1.fc2.weight": one(2.0),
              "shared_experts.0.fc1.weight": one(1.0), "shared_experts.0.fc2.weight": one(3.0)}
    out = M.layer_forward(cfg, params, one(1.0))
    assert out.item() == pytest.approx(1.0 + 5.0 * 0.8413447460685429, rel=1e-15)
    # the shared expert's weight follows its own key: scaling it moves only its term
    params["shared_experts.0.fc2.weight"] = one(30.0)
    assert M.layer_forward(cfg, params, one(1.0)).item() == pytest.approx(1.0 + 32.0 * 0.8413447460685429, rel=1e-15)


def test_sigmoid_gates_unnormalised_and_scaled_known_answer():
    """logits [0, ln 3] score sigmoid [1/2, 3/4]: top-1 unnormalised gate 3/4; times gate_scale 2.5 = 15/8;
    top-2 normalised [3/4, 1/2] / (5/4) = [3/5, 2/5], times 2.5 = [3/2, 1], slots in descending score."""
    x = torch.ones(1, 1, dtype=torch.float64)
    w = torch.tensor([[0.0], [math.log(3.0)]], dtype=torch.float64)
    c1 = M.OracleConfig(hidden=1, num_experts=2, top_k=1, score="sigmoid", normalize=False)
    topi, g = M.route(c1, x, w)
    assert topi.tolist() == [[1]] and g.item() == pytest.approx(0.75, rel=1e-15)
    c2 = M.OracleConfig(hidden=1, num_experts=2, top_k=1, score="sigmoid", normalize=False, gate_scale=2.5)
    assert M.route(c2, x, w)[1].item() == pytest.approx(1.875, rel=1e-15)
    c3 = M.OracleConfig(hidden=1, num_experts=2, top_k=2, score="sigmoid", normalize=True, gate_scale=2.5)
    topi, g = M.route(c3, x, w)
    assert topi.tolist() == [[1, 0]]
    assert g[0].tolist() == pytest.approx([1.5, 1.0], rel=1e-15)
