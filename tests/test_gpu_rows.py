"""Row kernels (permute, combine, their backward, token backward, router weight gradient) on the GPU.

Permute, combine, the combine input-gradient and the token backward are
checked bit for bit against a numpy emulation that performs the same IEEE
operations in the same order (the kernels are built without contraction);
the two reductions (gate gradient, router weight gradient) against float64.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from _helpers import DEV, rel_err, say, seeded
from oracle import route_c as R
from resihp_megatron_amd import kernels as K

pytestmark = pytest.mark.gpu

DTYPES = [torch.bfloat16, torch.float32, torch.float64]
NP_ACC = {torch.bfloat16: np.float32, torch.float32: np.float32, torch.float64: np.float64}


def _plan_inputs(T, k, E, e0, e1, seed):
    g = torch.Generator().manual_seed(seed)
    keys = torch.randn(T, E, generator=g)
    topi = torch.sort(keys, dim=1, descending=True, stable=True).indices[:, :k].to(torch.int32)
    ref = R.dispatch(topi.numpy(), E, e0, e1, 1)
    return topi, ref


def _to_np(t: torch.Tensor, acc) -> np.ndarray:
    return t.detach().cpu().to(torch.float64 if acc is np.float64 else torch.float32).numpy()


def _store(a: np.ndarray, dtype: torch.dtype) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a)).to(dtype)


# (T, h, k, E, window, shared experts): the bfloat16 kernels are compiled for k <= 2 and k <= 8 with up to
# two shared experts (one or several 64-lane passes, ragged last pass) and fall back to a generic kernel
# beyond; every case holds slots of other devices (pair_row = -1).
BF16_SHAPES = [
    (97, 4096, 2, 8, (0, 6), 0),
    (64, 2056, 2, 8, (2, 8), 2),
    (50, 1024, 1, 4, (0, 3), 1),
    (70, 1032, 8, 16, (4, 16), 2),
    (33, 2048, 6, 64, (0, 40), 2),
    (45, 2048, 8, 128, (16, 32), 0),
    (21, 1000, 5, 12, (0, 12), 0),
    (40, 512, 12, 16, (0, 12), 1),
    (30, 768, 4, 8, (0, 8), 5),
]


@pytest.mark.parametrize("dtype", DTYPES, ids=str)
@pytest.mark.parametrize("window", [(0, 10), (3, 7)], ids=["all", "share"])
def test_permute_combine_token_bwd_bit_exact(dtype, window):
    _rows_bit_exact(dtype, 300, 256, 3, 10, window, 1)


@pytest.mark.parametrize("shape", BF16_SHAPES, ids=lambda s: f"T{s[0]}-h{s[1]}-k{s[2]}-E{s[3]}-S{s[5]}")
def test_rows_bf16_shapes_bit_exact(shape):
    _rows_bit_exact(torch.bfloat16, *shape)


def _rows_bit_exact(dtype, T, h, k, E, window, n_shared):
    e0, e1 = window
    acc = NP_ACC[dtype]
    gdt = torch.float64 if dtype == torch.float64 else torch.float32
    topi, plan = _plan_inputs(T, k, E, e0, e1, 11)
    P = int(plan["offsets"][-1])
    x = seeded((T, h), 1, 1.0, dtype)
    y = seeded((P, h), 2, 1.0, dtype)
    gates = seeded((T, k), 3, 0.5, gdt).abs()
    shared = [seeded((T, h), 40 + s, 1.0, dtype) for s in range(n_shared)]
    pair_row = torch.from_numpy(plan["pair_row"].astype(np.int32))
    say(f"rows {dtype} window={window} T={T} h={h} k={k} E={E} shared={n_shared} P={P}")

    xp = K.permute(x.to(DEV), pair_row.to(DEV), k, P)
    out = K.combine(y.to(DEV), x.to(DEV), gates.to(DEV), topi.to(DEV), pair_row.to(DEV), [s.to(DEV) for s in shared])
    torch.cuda.synchronize()

    # permute: an exact row copy
    ref_xp = torch.empty(P, h, dtype=dtype)
    for p in range(T * k):
        r = plan["pair_row"][p]
        if r >= 0:
            ref_xp[r] = x[p // k]
    assert torch.equal(xp.cpu(), ref_xp)

    # combine: acc = 0; acc += g * y in ascending expert id; out = x + acc + shared
    xn, yn, gn = _to_np(x, acc), _to_np(y, acc), gates.numpy().astype(acc)
    order = np.argsort(topi.numpy(), axis=1, kind="stable")
    accum = np.zeros((T, h), acc)
    rows = plan["pair_row"].reshape(T, k)
    for rk in range(k):
        j = order[:, rk]
        r = rows[np.arange(T), j]
        gj = gn[np.arange(T), j][:, None]
        contrib = gj * yn[np.clip(r, 0, None)]
        accum = np.where((r >= 0)[:, None], accum + contrib, accum)
    ref = xn + accum
    for sh in shared:
        ref = ref + _to_np(sh, acc)
    ref_out = _store(ref, dtype)
    assert torch.equal(out.cpu(), ref_out)

    # combine backward: dy = g * dout (exact); dgates = <dout, y> (reduction)
    dout = seeded((T, h), 5, 1.0, dtype)
    dy, dgates = K.combine_bwd(dout.to(DEV), y.to(DEV), gates.to(DEV), pair_row.to(DEV), P)
    torch.cuda.synchronize()
    dn = _to_np(dout, acc)
    ref_dy = np.zeros((P, h), acc)
    ref_dg = np.zeros((T, k))
    for j in range(k):
        r = rows[:, j]
        m = r >= 0
        ref_dy[r[m]] = gn[m, j][:, None] * dn[m]
        ref_dg[m, j] = (dout[m].double() * y[r[m]].double()).sum(1).numpy()
    assert torch.equal(dy.cpu(), _store(ref_dy, dtype))
    assert rel_err(dgates, torch.from_numpy(ref_dg)) <= (1e-12 if dtype == torch.float64 else 1e-5)

    # token backward: acc = dout; += dxp rows in slot order; += dl_j * w[topi_j]; += shared dx
    dxp = seeded((P, h), 6, 1.0, dtype)
    dl = seeded((T, k), 7, 0.3, gdt)
    w = seeded((E, h), 8, 0.05, gdt)
    sdx = [seeded((T, h), 90 + s, 1.0, dtype) for s in range(n_shared)]
    dx = K.token_bwd(dout.to(DEV), dxp.to(DEV), pair_row.to(DEV), dl.to(DEV), topi.to(DEV), w.to(DEV),
                     [s.to(DEV) for s in sdx])
    torch.cuda.synchronize()
    a = dn.copy()
    dxpn = _to_np(dxp, acc)
    for j in range(k):
        r = rows[:, j]
        a = np.where((r >= 0)[:, None], a + dxpn[np.clip(r, 0, None)], a)
    a_rows = a.copy()
    dln, wn = dl.numpy(), w.numpy()
    for j in range(k):
        a = a + (dln[:, j][:, None] * wn[topi.numpy()[:, j]]).astype(acc)
    for sh in sdx:
        a = a + _to_np(sh, acc)
        a_rows = a_rows + _to_np(sh, acc)
    assert torch.equal(dx.cpu(), _store(a, dtype))
    # without the router term (the layer adds it in fc1's input-gradient epilogue when every expert is local)
    dx0 = K.token_bwd(dout.to(DEV), dxp.to(DEV), pair_row.to(DEV), None, topi.to(DEV), w.to(DEV),
                      [s.to(DEV) for s in sdx])
    torch.cuda.synchronize()
    assert torch.equal(dx0.cpu(), _store(a_rows, dtype))


@pytest.mark.parametrize("dtype", DTYPES, ids=str)
def test_router_wgrad(dtype):
    T, h, k, E = 700, 512, 4, 12
    gdt = torch.float64 if dtype == torch.float64 else torch.float32
    topi, plan = _plan_inputs(T, k, E, 0, E, 21)
    x = seeded((T, h), 1, 1.0, dtype)
    dl = seeded((T, k), 2, 0.3, gdt)
    say(f"router wgrad {dtype}")
    dw = K.router_wgrad(dl.to(DEV), torch.from_numpy(plan["perm"]).to(DEV),
                        torch.from_numpy(plan["offsets"].astype(np.int32)).to(DEV), x.to(DEV), E, gdt)
    torch.cuda.synchronize()
    ref = torch.zeros(E, h, dtype=torch.float64)
    ref.index_add_(0, topi.reshape(-1).long(), dl.reshape(-1, 1).double() * x.double().repeat_interleave(k, 0))
    assert rel_err(dw, ref) <= (1e-12 if dtype == torch.float64 else 1e-5)
    # deterministic: a second run gives the same bits
    dw2 = K.router_wgrad(dl.to(DEV), torch.from_numpy(plan["perm"]).to(DEV),
                         torch.from_numpy(plan["offsets"].astype(np.int32)).to(DEV), x.to(DEV), E, gdt)
    assert torch.equal(dw, dw2)
