"""Pins of the C routing oracle (oracle/route_ref.c) -- the bit-exact contract the kernels follow.

Checks that a plausible mistake fails: a wrong reduction order (closed-form
cancellation cases), a wrong tie-break (planted ties), a wrong selection
(brute force over k-subsets), a wrong permutation (numpy stable argsort) and
a wrong exp (libm to < 2 ulp).
"""

from __future__ import annotations

import itertools
import math

import numpy as np
import pytest
import torch

from oracle import moe_ref as M
from oracle import route_c as R


def _ulp_diff32(a: float, b: float) -> int:
    ia = np.array([a], np.float32).view(np.int32)[0]
    ib = np.array([b], np.float32).view(np.int32)[0]
    return abs(int(ia) - int(ib))


def test_expf_within_two_ulp_of_libm():
    xs = np.concatenate([np.linspace(-86.9, 88.7, 20001), np.linspace(-1, 1, 2001), [0.0, -0.0, 1e-30, -1e-30]])
    for x in xs.astype(np.float32):
        got = R.expf(float(x))
        ref = np.float32(math.exp(float(x)))
        assert _ulp_diff32(got, float(ref)) <= 2, (x, got, ref)


def test_expf_special_values():
    assert R.expf(float("inf")) == float("inf")
    assert R.expf(float("-inf")) == 0.0
    assert math.isnan(R.expf(float("nan")))
    assert R.expf(89.0) == float("inf")
    assert R.expf(-87.5) == 0.0       # flushed below -87 by definition
    assert R.expf(0.0) == 1.0


def test_exp_double_within_two_ulp_of_libm():
    for x in np.linspace(-707.9, 709.7, 20001):
        got, ref = R.exp(float(x)), math.exp(float(x))
        assert abs(got - ref) <= 2 * math.ulp(ref), (x, got, ref)


def test_logit_order_segments_closed_form():
    # h = 512: two segments of 256.  x = 1 everywhere; w[0] = 2^24, w[1:256] = 1, w[256:512] = 1.
    # Segment 0: 2^24 + 1 + ... each +1 ties to even and is lost -> 2^24.  Segment 1: 256.
    # Total 2^24 + 256.  A single serial chain would give 2^24; an exact sum 2^24 + 511 -> 2^24 + 512.
    h = 512
    x = np.ones((1, h), np.float32)
    w = np.ones((1, h), np.float32)
    w[0, 0] = 2.0 ** 24
    got = R.router_logits(x, w, "f32")[0, 0]
    assert got == 2.0 ** 24 + 256
    # Ascending order inside a segment: move the big weight to the end of segment 1.
    w = np.ones((1, h), np.float32)
    w[0, 511] = 2.0 ** 24
    got = R.router_logits(x, w, "f32")[0, 0]
    # seg0 = 256; seg1 = 255 then + 2^24 -> 2^24 + 255 ties to 2^24 + 256; total 2^24 + 512.
    assert got == 2.0 ** 24 + 512


def test_logits_close_to_float64_and_bf16_input():
    rng = np.random.default_rng(2)
    for h, E in ((64, 8), (2048, 16), (4096, 8)):
        x = rng.standard_normal((9, h)).astype(np.float32)
        w = (rng.standard_normal((E, h)) * 0.02).astype(np.float32)
        ref = x.astype(np.float64) @ w.astype(np.float64).T
        got = R.router_logits(x, w, "f32")
        assert np.abs(got - ref).max() <= 1e-5 * np.abs(ref).max()
        xb = torch.from_numpy(x).to(torch.bfloat16)
        got_b = R.router_logits(xb.view(torch.int16).numpy().view(np.uint16), w, "bf16")
        ref_b = xb.to(torch.float64).numpy() @ w.astype(np.float64).T
        assert np.abs(got_b - ref_b).max() <= 1e-5 * np.abs(ref_b).max()
        got64 = R.router_logits(x.astype(np.float64), w.astype(np.float64), "f64")
        assert np.abs(got64 - ref).max() <= 1e-13 * np.abs(ref).max()


def test_topk_brute_force_and_descending():
    rng = np.random.default_rng(3)
    for _ in range(40):
        E, k = 7, 3
        logits = rng.standard_normal((1, E)).astype(np.float32)
        topi, _ = R.topk(logits, k)
        best = max(itertools.combinations(range(E), k), key=lambda c: sum(float(logits[0, i]) for i in c))
        assert set(topi[0].tolist()) == set(best)
        assert all(logits[0, topi[0, i]] > logits[0, topi[0, i + 1]] for i in range(k - 1))


def test_topk_matches_stable_sort_with_planted_ties():
    rng = np.random.default_rng(4)
    T, E, k = 500, 16, 4
    logits = np.round(rng.standard_normal((T, E)) * 2).astype(np.float32)   # many exact ties
    logits[0, :] = 1.0
    logits[1, 3] = np.nan
    topi, _ = R.topk(logits, k)
    ref = M.select(torch.from_numpy(logits), k).numpy()
    assert np.array_equal(topi, ref)
    assert topi[0].tolist() == [0, 1, 2, 3]


def test_topk_bias_selects_only_and_sigmoid_gates():
    rng = np.random.default_rng(5)
    T, E, k = 200, 12, 3
    logits = rng.standard_normal((T, E)).astype(np.float32)
    bias = (rng.standard_normal(E) * 0.5).astype(np.float32)
    topi, gates = R.topk(logits, k, bias=bias)
    ref = M.select(torch.from_numpy(logits) + torch.from_numpy(bias), k).numpy()
    assert np.array_equal(topi, ref)
    sel = np.take_along_axis(logits.astype(np.float64), topi, 1)
    soft = np.exp(sel - sel.max(1, keepdims=True))
    np.testing.assert_allclose(gates, soft / soft.sum(1, keepdims=True), rtol=2e-6)
    topi_s, gates_s = R.topk(logits, k, bias=bias, score="sigmoid", scale=2.5)
    sig = 1 / (1 + np.exp(-logits.astype(np.float64)))
    ref_s = M.select(torch.from_numpy(sig.astype(np.float32)) + torch.from_numpy(bias), k).numpy()
    assert np.array_equal(topi_s, ref_s)
    s_sel = np.take_along_axis(sig, topi_s, 1)
    np.testing.assert_allclose(gates_s, 2.5 * s_sel / s_sel.sum(1, keepdims=True), rtol=2e-6)
    _, raw = R.topk(logits, k, score="sigmoid", normalize=False)
    np.testing.assert_allclose(raw.sum(1) > 0, True)


def test_topk_double_matches_float64_oracle_route():
    cfg = M.OracleConfig(hidden=16, num_experts=8, top_k=2)
    g = torch.Generator().manual_seed(9)
    x = torch.randn(100, 16, generator=g, dtype=torch.float64)
    w = torch.randn(8, 16, generator=g, dtype=torch.float64)
    logits = R.router_logits(x.numpy(), w.numpy(), "f64")
    topi, gates = R.topk(logits, 2)
    ref_topi, ref_gates = M.route(cfg, x, w)
    assert np.array_equal(topi, ref_topi.numpy())
    np.testing.assert_allclose(gates, ref_gates.numpy(), rtol=1e-14)


@pytest.mark.parametrize("T,k,E,e0,e1,n_src", [(1, 1, 1, 0, 1, 1), (333, 2, 8, 0, 8, 1), (400, 8, 128, 16, 32, 8),
                                               (64, 6, 64, 0, 64, 3), (0, 2, 4, 0, 4, 1)])
def test_dispatch_matches_numpy_stable_argsort(T, k, E, e0, e1, n_src):
    rng = np.random.default_rng(T + E)
    topi = np.array([rng.choice(E, k, replace=False) for _ in range(T)], np.int32).reshape(T, k)
    got = R.dispatch(topi, E, e0, e1, n_src)
    ref = M.dispatch(topi, E, e0, e1, n_src)
    for key in ("counts", "offsets", "src_counts", "perm", "pair_row"):
        assert np.array_equal(got[key], ref[key]), key


def test_dispatch_invalid_ids_are_counted_and_dropped():
    topi = np.array([[0, 9], [-1, 1]], np.int32)
    got = R.dispatch(topi, 4)
    assert got["counts"].tolist() == [1, 1, 0, 0, 2]
    assert got["pair_row"].tolist() == [0, -1, -1, 1]
