"""The C Adam oracle against the reference's update on torch's CPU kernels (CPU only).

resihp/runtime/optim.py:32-46 is asserted by the reference to be bit for bit
torch.optim.Adam(foreach=False) (tests/unit/test_state_basics.py:108-120): the
two run the same torch CPU kernels.  Those kernels pin every operation of the
update but one: torch's CPU square root in this build is accurate to 1 ulp,
not correctly rounded (about 1 % of float32/float64 elements differ from the
IEEE square root, at every tensor size), and which approximation runs depends
on the host's vector unit.  The oracle (and the GPU kernel) use the correctly
rounded square root.  So the oracle must equal, bit for bit, the reference's
sequence of torch tensor operations with only ``sqrt`` replaced by the IEEE
square root -- over several steps, in float64, float32 and bfloat16, with and
without weight decay, on sizes that leave vector tails and with a parameter
that has no gradient -- and must agree with torch.optim.Adam itself wherever
torch's square root is exact.  A plain-arithmetic variant (no fused
multiply-adds) is checked to differ, so the test would catch a dropped fma.

One more torch detail: for bfloat16, ``g.add(p, alpha=wd)`` rounds ``wd`` to
bfloat16 and does one float multiply-add in its vector body, but its scalar
tail (the last elements of each thread's chunk) rounds ``wd * p`` to bfloat16
before the add, so torch's own bfloat16 weight-decay result depends on where
its chunks end.  The oracle follows the vector body; the bfloat16
weight-decay cases run torch on one thread with sizes that leave no tail.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import adam_c

DTYPES = [torch.float64, torch.float32, torch.bfloat16]
SHAPES = [(1000, 37), (5,), (3, 7), (64, 64), (15,)]


def _np(t: torch.Tensor) -> np.ndarray:
    t = t.detach().contiguous()
    return t.view(torch.int16).numpy().view(np.uint16).copy() if t.dtype == torch.bfloat16 else t.numpy().copy()


def _bits(a: np.ndarray) -> np.ndarray:
    return a.view({8: np.uint64, 4: np.uint32, 2: np.uint16}[a.dtype.itemsize])


def _ieee_sqrt(v: torch.Tensor) -> torch.Tensor:
    if v.dtype == torch.bfloat16:   # float square root of the bf16 values, rounded to bf16
        return torch.from_numpy(np.sqrt(v.float().numpy())).to(torch.bfloat16)
    return torch.from_numpy(np.sqrt(v.numpy()))


@torch.no_grad()
def _reference_step(p, grad, m, v, lr, betas, eps, wd, step):
    """optim.py:35-46 for one tensor, torch CPU kernels, with the IEEE square root."""
    b1, b2 = betas
    bc1 = 1 - b1 ** step
    bc2_sqrt = math.sqrt(1 - b2 ** step)
    g = grad if grad is not None else torch.zeros_like(p)
    if wd:
        g = g.add(p, alpha=wd)
    m.lerp_(g, 1 - b1)
    v.mul_(b2).addcmul_(g, g.conj(), value=1 - b2)
    denom = (_ieee_sqrt(v) / bc2_sqrt).add_(eps)
    p.addcdiv_(m, denom, value=-lr / bc1)


@pytest.mark.parametrize("dtype", DTYPES, ids=str)
@pytest.mark.parametrize("wd", [0.0, 0.1])
def test_oracle_matches_reference_ops_bitwise(dtype, wd):
    tailless = dtype == torch.bfloat16 and wd != 0.0
    shapes = [(1000, 64), (64,), (3, 64), (64, 64)] if tailless else SHAPES
    threads = torch.get_num_threads()
    if tailless:
        torch.set_num_threads(1)
    try:
        _check_reference_ops(dtype, wd, shapes)
    finally:
        torch.set_num_threads(threads)


def _check_reference_ops(dtype, wd, shapes):
    SHAPES = shapes   # noqa: N806
    g = torch.Generator().manual_seed(7)
    lr, betas, eps = 3e-3, (0.9, 0.999), 1e-8
    ref = [[(torch.randn(s, generator=g) * 0.5).to(dtype)] for s in SHAPES]
    for r in ref:
        r += [torch.zeros_like(r[0]), torch.zeros_like(r[0])]
    mine = [[_np(t) for t in r] for r in ref]
    for step in range(1, 7):
        for i, s in enumerate(SHAPES):
            grad = None if (i == 1 and step == 3) else (torch.randn(s, generator=g) * (0.1 * step)).to(dtype)
            _reference_step(*ref[i][:1], grad, *ref[i][1:], lr, betas, eps, wd, step)
            adam_c.adam_step(mine[i][0], None if grad is None else _np(grad), mine[i][1], mine[i][2], lr, betas, eps,
                             wd, step)
            for t, a in zip(ref[i], mine[i]):
                assert np.array_equal(_bits(_np(t)), _bits(a)), (dtype, wd, step, s)


@pytest.mark.parametrize("dtype", DTYPES, ids=str)
def test_oracle_matches_torch_adam_where_sqrt_is_exact(dtype):
    """torch.optim.Adam(foreach=False) itself: equal bits except where torch's sqrt is 1 ulp off."""
    threads = torch.get_num_threads()
    torch.set_num_threads(1)   # no thread-chunk tails (see the module docstring)
    try:
        _check_torch_adam(dtype)
    finally:
        torch.set_num_threads(threads)


def _check_torch_adam(dtype):
    g = torch.Generator().manual_seed(9)
    p = torch.nn.Parameter((torch.randn(4096, generator=g) * 0.5).to(dtype))
    opt = torch.optim.Adam([p], lr=1e-3, weight_decay=0.01, foreach=False)
    P, Mo, V = _np(p), np.zeros_like(_np(p)), np.zeros_like(_np(p))
    grad = (torch.randn(4096, generator=g) * 0.1).to(dtype)
    p.grad = grad.clone()
    v_before = opt.state.get(p, {}).get("exp_avg_sq")
    assert v_before is None
    opt.step()
    adam_c.adam_step(P, _np(grad), Mo, V, 1e-3, weight_decay=0.01, step=1)
    vt = opt.state[p]["exp_avg_sq"]
    assert np.array_equal(_bits(_np(vt)), _bits(V)) and np.array_equal(_bits(_np(opt.state[p]["exp_avg"])), _bits(Mo))
    exact = (vt.sqrt() == _ieee_sqrt(vt)).numpy()
    same = _bits(_np(p)) == _bits(P)
    assert same[exact].all()
    assert exact.mean() > 0.95


def test_skipped_gradient_is_a_zero_gradient():
    """optim.py:38 uses zeros_like(p) when p.grad is None: same as passing zeros."""
    rng = np.random.default_rng(3)
    p = rng.standard_normal(100)
    a = [p.copy(), np.full(100, 0.01), np.full(100, 0.02)]
    b = [p.copy(), np.full(100, 0.01), np.full(100, 0.02)]
    adam_c.adam_step(a[0], None, a[1], a[2], 1e-3, step=4, weight_decay=0.1)
    adam_c.adam_step(b[0], np.zeros(100), b[1], b[2], 1e-3, step=4, weight_decay=0.1)
    assert all(np.array_equal(x, y) for x, y in zip(a, b))


def test_dropped_fma_is_detected():
    """Rounding c*g*g before the add (no fma) in the second moment changes bits on random data."""
    rng = np.random.default_rng(5)
    n = 4096
    v = np.abs(rng.standard_normal(n))
    gr = rng.standard_normal(n)
    p1, m1, v1 = np.zeros(n), np.zeros(n), v.copy()
    adam_c.adam_step(p1, gr, m1, v1, 1e-3, step=1)
    plain = v * 0.999 + ((1 - 0.999) * gr) * gr
    assert not np.array_equal(v1, plain)
