"""Fused Adam step (rhp_adam_step) on the GPU against the C oracle, bit for bit.

The oracle (oracle/adam_ref.c) restates resihp/runtime/optim.py:32-46 element
by element and is pinned against torch's CPU kernels in
tests/test_oracle_adam.py.  Cases: float64, float32 and bfloat16; with and
without weight decay; six steps; tensors of 0, 1, 7, 8, 9 elements, one that
spans several blocks with a ragged end, a parameter without a gradient on
some steps, and 70 tensors in one call (two launches).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from _helpers import DEV, say
from oracle import adam_c
from resihp_megatron_amd import kernels as K
from resihp_megatron_amd import moe

pytestmark = pytest.mark.gpu

DTYPES = [torch.float64, torch.float32, torch.bfloat16]
SIZES = [0, 1, 7, 8, 9, 33, 100003, 4096 * 3 + 5]


def _np(t: torch.Tensor) -> np.ndarray:
    t = t.detach().cpu().contiguous()
    return t.view(torch.int16).numpy().view(np.uint16).copy() if t.dtype == torch.bfloat16 else t.numpy().copy()


def _bits(a: np.ndarray) -> np.ndarray:
    return a.view({8: np.uint64, 4: np.uint32, 2: np.uint16}[a.dtype.itemsize])


@pytest.mark.parametrize("dtype", DTYPES, ids=str)
@pytest.mark.parametrize("wd", [0.0, 0.1])
def test_fused_adam_matches_oracle_bitwise(dtype, wd):
    g = torch.Generator().manual_seed(21)
    lr, betas, eps = 2e-3, (0.9, 0.95), 1e-8
    params = [(torch.randn(n, generator=g) * 0.5).to(dtype) for n in SIZES]
    dev_p = [p.to(DEV) for p in params]
    dev_m = [torch.zeros_like(p) for p in dev_p]
    dev_v = [torch.zeros_like(p) for p in dev_p]
    host = [[_np(p), _np(torch.zeros_like(p)), _np(torch.zeros_like(p))] for p in params]
    say(f"adam {dtype} wd={wd}")
    for step in range(1, 7):
        grads = [None if (i == 3 and step % 2 == 0) else (torch.randn(n, generator=g) * 0.2 * step).to(dtype)
                 for i, n in enumerate(SIZES)]
        K.adam_step(dev_p, [None if gr is None else gr.to(DEV) for gr in grads], dev_m, dev_v, lr, betas, eps, wd,
                    step)
        for i, gr in enumerate(grads):
            adam_c.adam_step(host[i][0], None if gr is None else _np(gr), host[i][1], host[i][2], lr, betas, eps, wd,
                             step)
        torch.cuda.synchronize()
        for i in range(len(SIZES)):
            for t, a, what in zip((dev_p[i], dev_m[i], dev_v[i]), host[i], ("param", "exp_avg", "exp_avg_sq")):
                assert np.array_equal(_bits(_np(t)), _bits(a)), (dtype, wd, step, SIZES[i], what)


def test_fused_adam_many_tensors_one_call():
    """More tensors than one launch takes (64): the call splits them; every one is updated."""
    g = torch.Generator().manual_seed(5)
    ps = [(torch.randn(37 + i, generator=g)).to(torch.float32) for i in range(70)]
    gs = [torch.randn(p.shape, generator=g) for p in ps]
    dp, dm, dv = [p.to(DEV) for p in ps], [torch.zeros(p.shape, device=DEV) for p in ps], \
        [torch.zeros(p.shape, device=DEV) for p in ps]
    say("adam 70 tensors")
    K.adam_step(dp, [x.to(DEV) for x in gs], dm, dv, 1e-3, (0.9, 0.999), 1e-8, 0.0, 1)
    torch.cuda.synchronize()
    for i, p in enumerate(ps):
        hp, hm, hv = _np(p), np.zeros(p.numel(), np.float32), np.zeros(p.numel(), np.float32)
        adam_c.adam_step(hp, _np(gs[i]), hm, hv, 1e-3, step=1)
        assert np.array_equal(_bits(_np(dp[i])), _bits(hp)), i


def test_dropin_adam_uses_fused_step_and_keeps_state_names():
    """moe.Adam on the GPU: name-keyed state (optim.py:24-25, 48-55) and the oracle's bits for mixed dtypes."""
    g = torch.Generator().manual_seed(3)
    params = {"router.weight": torch.nn.Parameter(torch.randn(8, 64, generator=g).to(DEV)),
              "experts.0.fc1.weight": torch.nn.Parameter(torch.randn(256, 64, generator=g).to(torch.bfloat16).to(DEV))}
    host = {n: [_np(p), np.zeros_like(_np(p)), np.zeros_like(_np(p))] for n, p in params.items()}
    opt = moe.Adam(params, lr=1e-2, weight_decay=0.01)
    say("adam drop-in")
    for step in range(1, 4):
        for n, p in params.items():
            p.grad = torch.randn(p.shape, generator=g).to(p.dtype).to(DEV)
            adam_c.adam_step(host[n][0], _np(p.grad), host[n][1], host[n][2], 1e-2, weight_decay=0.01, step=step)
        opt.step()
    torch.cuda.synchronize()
    st = opt.state_tensors()
    assert sorted(st) == sorted(f"{k}/{n}" for n in params for k in ("param", "exp_avg", "exp_avg_sq"))
    for n in params:
        assert np.array_equal(_bits(_np(st[f"param/{n}"])), _bits(host[n][0])), n
        assert np.array_equal(_bits(_np(st[f"exp_avg_sq/{n}"])), _bits(host[n][2])), n
