"""Routing and dispatch on the GPU, bit for bit against the C oracle (oracle/route_ref.c).

Logits, top-k ids, gates, per-expert counts, offsets, per-source counts and the
permutation must be identical bit patterns, on the benchmark shapes (router on
full token counts for the Mixtral and DeepSeek-like layers) and on edge cases:
exact ties, NaN logits, empty experts, one token, invalid ids.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from _helpers import DEV, host_x, say, seeded, x_kind, zipf_prior
from oracle import route_c as R
from resihp_megatron_amd import kernels as K

pytestmark = pytest.mark.gpu

# (name, T, h, E, k, x dtype, score, bias, router std)
ROUTE_CASES = [
    ("tiny-f64", 512, 64, 8, 2, torch.float64, "softmax", None, 0.125),
    ("tiny-f32", 512, 64, 8, 2, torch.float32, "softmax", None, 0.125),
    ("mixtral", 8192, 4096, 8, 2, torch.bfloat16, "softmax", None, 0.02),
    ("dsv2lite-sigmoid-bias", 16384, 2048, 64, 6, torch.bfloat16, "sigmoid", "normal", 0.02),
    ("ep128-zipf", 8192, 2048, 128, 8, torch.bfloat16, "softmax", "zipf", 0.02),
    ("reference-default", 48, 8, 6, 2, torch.float64, "softmax", None, 0.35),
    ("odd-e", 333, 256, 5, 3, torch.bfloat16, "sigmoid", None, 0.05),
    # bfloat16 kernel edges: a hidden size below one 256-element segment (ragged last 64-element group),
    # expert counts that are not a multiple of the 8- or 16-expert groups, 32 segments (waves loop over
    # segments), the expert-parallel mode (at least as many expert groups as segments), and more experts
    # than its LDS holds (generic kernel)
    ("bf16-h200-e20", 130, 200, 20, 4, torch.bfloat16, "softmax", "normal", 0.05),
    ("bf16-h8192-e72", 100, 8192, 72, 6, torch.bfloat16, "sigmoid", "normal", 0.02),
    ("bf16-expert-mode-e200", 150, 1024, 200, 8, torch.bfloat16, "softmax", "zipf", 0.02),
    ("bf16-e300-generic", 70, 256, 300, 4, torch.bfloat16, "softmax", None, 0.05),
]


def _bias(kind, E, dtype):
    if kind is None:
        return None
    if kind == "zipf":
        return zipf_prior(E).to(dtype)
    return seeded((E,), 99, 0.1, dtype)


@pytest.mark.parametrize("case", ROUTE_CASES, ids=[c[0] for c in ROUTE_CASES])
def test_route_bit_exact(case):
    name, T, h, E, k, xdt, score, bias_kind, wstd = case
    rdt = torch.float64 if xdt == torch.float64 else torch.float32
    x = seeded((T, h), 1, 1.0, xdt)
    w = seeded((E, h), 2, wstd, rdt)
    bias = _bias(bias_kind, E, rdt)
    say(f"route {name}: T={T} h={h} E={E} k={k} {xdt} {score}")
    logits, topi, gates = K.route(x.to(DEV), w.to(DEV), None if bias is None else bias.to(DEV), k, score,
                                  True, 1.0)
    torch.cuda.synchronize()
    ref_logits = R.router_logits(host_x(x), w.numpy(), x_kind(xdt))
    ref_topi, ref_gates = R.topk(ref_logits, k, None if bias is None else bias.numpy(), score)
    got_l = logits.cpu().numpy()
    assert got_l.dtype == ref_logits.dtype
    assert np.array_equal(got_l.view(np.uint8), ref_logits.view(np.uint8)), "logit bits differ"
    assert np.array_equal(topi.cpu().numpy(), ref_topi), "selection differs"
    assert np.array_equal(gates.cpu().numpy().view(np.uint8), ref_gates.view(np.uint8)), "gate bits differ"


def test_route_ties_and_nan():
    T, h, E, k = 64, 64, 16, 4
    x = seeded((T, h), 3, 1.0, torch.float32)
    x[0] = 0.0                              # every logit of token 0 is +0: ids 0..3 win
    w = seeded((E, h), 4, 0.1, torch.float32)
    w[9] = w[2]                             # experts 2 and 9 always tie: 2 must win
    w[13] = w[5]
    x[1, 0] = float("nan")                  # NaN logits rank last
    say("route ties/nan")
    logits, topi, gates = K.route(x.to(DEV), w.to(DEV), None, k, "softmax", True, 1.0)
    torch.cuda.synchronize()
    ref_logits = R.router_logits(x.numpy(), w.numpy(), "f32")
    ref_topi, _ = R.topk(ref_logits, k)
    assert np.array_equal(topi.cpu().numpy(), ref_topi)
    assert topi[0].tolist() == [0, 1, 2, 3]
    t = topi.cpu().numpy()
    assert not ((t == 9) & ~(t == 2).any(1, keepdims=True)).any(), "expert 9 chosen without its tie twin 2"


DISPATCH_CASES = [
    # (name, T, k, E, e0, e1, n_src, skew)
    ("tiny", 512, 2, 8, 0, 8, 1, 0.0),
    ("mixtral", 8192, 2, 8, 0, 8, 1, 0.0),
    ("dsv2lite", 16384, 6, 64, 0, 64, 1, 0.0),
    ("ep128-hot-share", 32768, 8, 128, 0, 16, 8, 1.1),
    ("ep128-tail-share", 32768, 8, 128, 112, 128, 8, 1.1),
    ("one-token", 1, 2, 4, 0, 4, 1, 0.0),
    ("ragged-sources", 1001, 3, 10, 2, 9, 7, 0.5),
]

# Experts that never receive a token in the tail-share case (empty groups in the window).
EMPTY = (113, 120, 121, 127)


def _topi(T, k, E, skew, seed, never=()):
    g = torch.Generator().manual_seed(seed)
    keys = torch.randn(T, E, generator=g, dtype=torch.float64) + (zipf_prior(E, skew) if skew else 0.0)
    keys[:, list(never)] = -torch.inf
    return torch.sort(keys, dim=1, descending=True, stable=True).indices[:, :k].to(torch.int32)


@pytest.mark.parametrize("case", DISPATCH_CASES, ids=[c[0] for c in DISPATCH_CASES])
def test_dispatch_bit_exact(case):
    name, T, k, E, e0, e1, n_src, skew = case
    topi = _topi(T, k, E, skew, 7, EMPTY if e0 == 112 else ())
    say(f"dispatch {name}: T={T} k={k} E={E} window=[{e0},{e1}) n_src={n_src}")
    plan = K.dispatch(topi.to(DEV), E, e0, e1, n_src)
    torch.cuda.synchronize()
    ref = R.dispatch(topi.numpy(), E, e0, e1, n_src)
    P = int(ref["offsets"][-1])
    assert np.array_equal(plan.counts.cpu().numpy(), ref["counts"])
    assert np.array_equal(plan.offsets.cpu().numpy(), ref["offsets"])
    assert np.array_equal(plan.src_counts.cpu().numpy(), ref["src_counts"])
    assert np.array_equal(plan.perm[:P].cpu().numpy(), ref["perm"])
    assert np.array_equal(plan.pair_row.cpu().numpy(), ref["pair_row"])
    if e0 == 112:
        assert (ref["counts"][list(EMPTY)] == 0).all() and P > 0


def test_dispatch_invalid_ids_dropped():
    topi = torch.tensor([[0, 9], [-1, 1], [3, 2]], dtype=torch.int32)
    say("dispatch invalid ids")
    plan = K.dispatch(topi.to(DEV), 4)
    torch.cuda.synchronize()
    ref = R.dispatch(topi.numpy(), 4)
    assert plan.counts.cpu().tolist() == ref["counts"].tolist() == [1, 1, 1, 1, 2]
    assert np.array_equal(plan.pair_row.cpu().numpy(), ref["pair_row"])


def test_expert_bias_update_matches_reference_rule():
    counts = torch.tensor([5, 1, 3, 3, 0, 6], dtype=torch.int32)   # mean 3
    bias = torch.zeros(6, dtype=torch.float64)
    say("bias update")
    b = bias.to(DEV)
    K.update_expert_bias(b, counts.to(DEV), 0.01)
    torch.cuda.synchronize()
    ref = bias + 0.01 * torch.sign(counts.double().mean() - counts.double())
    assert torch.equal(b.cpu(), ref)
