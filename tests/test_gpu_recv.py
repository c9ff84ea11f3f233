"""The receiving side of expert parallelism on the GPU (rhp_recv_plan, rhp_gather_rows, expert_chunks).

Configuration 4 starts here from what one GPU of a 128-expert top-8 layer
receives: 8 sources route their tokens (Zipf(1.1) selection prior), and the
GPU holding experts [e0, e0 + 16) receives each source's rows for them in the
reference's order (resihp/runtime/moe.py:193-212, restated by
``oracle.moe_ref.received_rows``).  Plans and row maps must be bit-exact with
the oracle; expert outputs and gradients are checked against float64.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from _helpers import DEV, TOL, host_x, rel_err, say, seeded, zipf_prior
from oracle import moe_ref as M
from oracle import route_c as R
from resihp_megatron_amd import kernels as K
from resihp_megatron_amd import moe
from resihp_megatron_amd.placement import ExpertPlacement

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("shape,hi", [((1, 1), 5), ((8, 16), 3000), ((3, 5), 0), ((64, 128), 40), ((128, 64), 7)])
def test_recv_plan_bit_exact(shape, hi):
    rng = np.random.default_rng(shape[0] * 1000 + shape[1])
    counts = rng.integers(0, hi + 1, size=shape)
    counts[rng.random(shape) < 0.25] = 0
    if shape == (8, 16):
        counts[3, :] = 0          # an empty source
        counts[:, 7] = 0          # an empty expert
    ref = M.recv_plan(counts)
    say(f"recv plan {shape}: {int(counts.sum())} rows")
    plan = K.recv_plan(torch.from_numpy(counts).to(torch.int32).to(DEV))
    torch.cuda.synchronize()
    assert plan.rows == int(counts.sum())
    assert np.array_equal(plan.offsets.cpu().numpy(), ref["offsets"])
    assert np.array_equal(plan.sort_row.cpu().numpy(), ref["sort_row"])
    assert np.array_equal(plan.unsort_row.cpu().numpy(), ref["unsort_row"])


@pytest.mark.parametrize("delta", [-37, 0, 53])
def test_recv_plan_with_a_wrong_row_count(delta):
    """A caller's row count that differs from the counts' sum never leaves a map entry unwritten: rows
    without a partner among the first `rows` map to -1 (read as zero rows, their stores dropped), the
    rest as with the true count, and offsets[L] holds the true sum."""
    rng = np.random.default_rng(77)
    counts = rng.integers(0, 40, size=(4, 6))
    total = int(counts.sum())
    rows = total + delta
    ref = M.recv_plan(counts)
    say(f"recv plan with rows = sum {delta:+d}")
    plan = K.recv_plan(torch.from_numpy(counts).to(torch.int32).to(DEV), rows=rows)
    torch.cuda.synchronize()
    sort_row = plan.sort_row.cpu().numpy()
    unsort_row = plan.unsort_row.cpu().numpy()
    assert sort_row.size == rows and unsort_row.size == rows
    exp_sort = np.full(rows, -1)
    exp_unsort = np.full(rows, -1)
    n = min(rows, total)
    for r in range(n):
        q = ref["sort_row"][r]
        exp_sort[r] = q if q < rows else -1
    for q in range(n):
        r = ref["unsort_row"][q]
        exp_unsort[q] = r if r < rows else -1
    assert np.array_equal(sort_row, exp_sort) and np.array_equal(unsort_row, exp_unsort)
    assert int(plan.offsets[-1].item()) == total


@pytest.mark.parametrize("dtype,h", [(torch.bfloat16, 2048), (torch.bfloat16, 8), (torch.float32, 100),
                                     (torch.float64, 6), (torch.bfloat16, 4096)])
def test_gather_rows_bit_exact(dtype, h):
    n_src, rows = 1000, 1500
    src = seeded((n_src, h), 3, 1.0, torch.float64).to(dtype)
    idx = torch.from_numpy(np.random.default_rng(h).integers(-3, n_src + 3, rows)).to(torch.int32)
    say(f"gather rows {dtype} h={h}")
    out = K.gather_rows(src.to(DEV), idx.to(DEV))
    torch.cuda.synchronize()
    ok = (idx >= 0) & (idx < n_src)
    ref = torch.zeros(rows, h, dtype=dtype)
    ref[ok] = src[idx[ok].long()]
    assert torch.equal(out.cpu(), ref)


def test_gather_rows_rejects_unaligned_rows():
    src = torch.zeros(4, 1001, dtype=torch.bfloat16, device=DEV)
    with pytest.raises(RuntimeError, match="multiple of 16 bytes"):
        K.gather_rows(src, torch.zeros(2, dtype=torch.int32, device=DEV))


def _map_case(counts, src_rows, seed, invalid):
    """Offsets of ragged groups and a row map: distinct received rows (a random subset of src_rows in
    random order), optionally with a few indices outside the buffer."""
    rng = np.random.default_rng(seed)
    P = int(sum(counts))
    idx = rng.permutation(src_rows)[:P].astype(np.int32)
    if invalid:
        bad = rng.choice(P, 5, replace=False)
        idx[bad[:3]] = -1
        idx[bad[3:]] = src_rows + np.array([0, 7])
    offsets = np.concatenate([[0], np.cumsum(counts)]).astype(np.int32)
    return torch.from_numpy(offsets).to(DEV), torch.from_numpy(idx).to(DEV), P


@pytest.mark.parametrize("dtype,h,f,invalid", [(torch.bfloat16, 256, 128, False), (torch.bfloat16, 2048, 768, True),
                                               (torch.bfloat16, 256, 4096, True), (torch.bfloat16, 96, 40, True),
                                               (torch.float32, 128, 64, True)],
                         ids=["bf16-mfma", "bf16-mfma-ep128-dims-bad-idx", "bf16-mfma-k-split", "bf16-generic",
                              "f32-generic"])
def test_row_map_products_equal_gather_then_product(dtype, h, f, invalid):
    """The four products on received rows (gathered inputs, scattered outputs) equal rhp_gather_rows
    followed by the plain product, bit for bit, on both kernels: ragged groups (one empty), distinct
    received rows in random order, indices outside the buffer (zero rows in, rows dropped out), and
    buffer rows that no index names (left untouched).  With f = 4096 fc1's input-gradient product
    reduces over 8192 and its last round is split along K (the scatter then runs in the epilogue of
    the piece that finishes last)."""
    counts = [300, 0, 517, 64, 1029] if dtype == torch.bfloat16 and h >= 256 else [33, 0, 70, 5]
    src_rows = int(sum(counts)) + 41
    offsets, idx, P = _map_case(counts, src_rows, h + f, invalid)
    G = len(counts)
    gen = torch.Generator(device=DEV).manual_seed(h * 7 + f)
    rnd = lambda *sh, std=1.0: (torch.randn(*sh, generator=gen, device=DEV) * std).to(dtype)  # noqa: E731
    w1 = [rnd(2 * f, h, std=0.05) for _ in range(G)]
    w2 = [rnd(h, f, std=0.05) for _ in range(G)]
    src, dy_src = rnd(src_rows, h), rnd(src_rows, h)
    kind = K.gemm_kernel(dtype, "swiglu", h, f)
    assert kind == ("mfma" if dtype == torch.bfloat16 and h % 64 == 0 and f % 64 == 0 else "generic")
    say(f"row-map products {dtype} h={h} f={f} ({kind}), P={P}, invalid={invalid}")
    empty = lambda n, c: torch.empty(n, c, dtype=dtype, device=DEV)  # noqa: E731
    # forward: fc1 on gathered rows
    xs = K.gather_rows(src, idx)
    hpre_r, a_r = empty(P, 2 * f), empty(P, f)
    K.expert_fc1_fwd([xs] * G, offsets, True, P, w1, f, "swiglu", [hpre_r] * G, [a_r] * G)
    hpre, a = empty(P, 2 * f), empty(P, f)
    K.expert_fc1_fwd_gather(src, idx, offsets, P, w1, f, "swiglu", hpre, a)
    # forward: fc2 scattered back
    y_r = empty(P, h)
    K.expert_fc2_fwd([a_r] * G, offsets, True, P, w2, [y_r] * G)
    sentinel = torch.full((src_rows, h), 7.0, dtype=dtype, device=DEV)
    y = sentinel.clone()
    K.expert_fc2_fwd_scatter(a_r, offsets, P, w2, y, idx)
    # backward: fc2 input gradient on gathered output gradients, fc1 input gradient scattered
    dys = K.gather_rows(dy_src, idx)
    dh_r = empty(P, 2 * f)
    K.expert_fc2_bwd([dys] * G, [a_r] * G, [hpre_r] * G, offsets, True, P, w2, "swiglu", [dh_r] * G, None)
    dh = empty(P, 2 * f)
    K.expert_fc2_dgrad_gather(dy_src, idx, offsets, P, w2, "swiglu", hpre_r, dh)
    dx_r = empty(P, h)
    K.expert_fc1_bwd([dh_r] * G, [xs] * G, offsets, True, P, w1, f, "swiglu", [dx_r] * G, None)
    dx = sentinel.clone()
    K.expert_fc1_dgrad_scatter(dh_r, offsets, P, w1, f, "swiglu", dx, idx)
    torch.cuda.synchronize()
    assert torch.equal(hpre, hpre_r) and torch.equal(a, a_r)
    assert torch.equal(dh, dh_r)
    ix = idx.long()
    ok = (ix >= 0) & (ix < src_rows)
    named = torch.zeros(src_rows, dtype=torch.bool, device=DEV)
    named[ix[ok]] = True
    for out, ref in ((y, y_r), (dx, dx_r)):
        assert torch.equal(out[ix[ok]], ref[ok])
        assert torch.equal(out[~named], sentinel[~named])
    if invalid:
        assert not bool(ok.all()) and bool((xs[~ok] == 0).all())


def test_row_map_products_reject_bad_maps():
    h, f = 256, 128
    w1 = [torch.zeros(2 * f, h, dtype=torch.bfloat16, device=DEV)]
    w2 = [torch.zeros(h, f, dtype=torch.bfloat16, device=DEV)]
    offsets = torch.tensor([0, 4], dtype=torch.int32, device=DEV)
    idx = torch.arange(4, dtype=torch.int32, device=DEV)
    act = torch.zeros(4, f, dtype=torch.bfloat16, device=DEV)
    with pytest.raises(K.KernelArgumentError, match="row map"):
        K.expert_fc2_fwd_scatter(act, offsets, 4, w2, torch.zeros(4, h, dtype=torch.bfloat16, device=DEV), idx[:3])
    with pytest.raises(K.KernelArgumentError, match="row map"):
        K.expert_fc2_fwd_scatter(act, offsets, 4, w2, torch.zeros(4, h, dtype=torch.bfloat16, device=DEV),
                                 idx.to(torch.int64))
    # a mapped buffer of 2 GiB does not fit the MFMA kernel's 31-bit views: an error, not a wrong result
    big = torch.empty((1 << 31) // (2 * h), h, dtype=torch.bfloat16, device=DEV)
    with pytest.raises(RuntimeError, match="below 2 GiB"):
        K.expert_fc1_fwd_gather(big, idx, offsets, 4, w1, f, "swiglu",
                                torch.zeros(4, 2 * f, dtype=torch.bfloat16, device=DEV), act.clone())
    del big


def _ep_share(T: int, window: tuple[int, int], n_src: int = 8, empty: tuple[int, ...] = ()):
    """Routing of T source tokens (n_src sources by even_split) over 128 experts, top-8, with the Zipf
    selection prior; the received buffer of the device holding the window, in the reference's order.
    Experts in ``empty`` get a selection bias of -64, far below any logit: no token picks them."""
    cfg = moe.MoEConfig(hidden=2048, ffn=768, num_experts=128, top_k=8, tokens=T, act="swiglu",
                        dtype=torch.bfloat16, init_std=0.02, device=DEV)
    specs = moe.moe_specs(cfg)
    e0, e1 = window
    router = moe.init_param(cfg, specs["router.weight"])
    bias = zipf_prior(128).float()
    bias[list(empty)] -= 64.0
    bias = bias.to(DEV)
    x = seeded((T, 2048), 23, 1.0, torch.bfloat16).to(DEV)
    _, topi, _ = K.route(x, router, bias, 8)
    plan = K.dispatch(topi, 128, e0, e1, n_src)
    torch.cuda.synchronize()
    topi_h = topi.cpu().numpy()
    if T <= 4096:   # full-size routing is checked bit for bit in test_gpu_route.py
        lg = R.router_logits(host_x(x), router.cpu().numpy(), "bf16")
        ref_topi, _ = R.topk(lg, 8, bias.cpu().numpy(), "softmax")
        assert np.array_equal(topi_h, ref_topi), "routing is bit-exact with the oracle"
    bounds = moe.even_split(T, n_src)
    src, tok, slot, counts = M.received_rows([topi_h[a:b] for a, b in bounds], list(range(e0, e1)))
    # the dispatch plan's per-source counts are the counts this device receives
    assert np.array_equal(plan.src_counts.cpu().numpy(), counts)
    starts = np.array([a for a, _ in bounds])
    gtok = torch.from_numpy(starts[src] + tok).to(DEV)
    recv = x[gtok].contiguous()
    w1 = {e: moe.init_param(cfg, specs[f"experts.{e}.fc1.weight"]) for e in range(e0, e1)}
    w2 = {e: moe.init_param(cfg, specs[f"experts.{e}.fc2.weight"]) for e in range(e0, e1)}
    return cfg, recv, counts, src, w1, w2


def _runtime(cfg, window, w1, w2):
    e0, e1 = window
    params = {}
    for e in range(e0, e1):
        params[f"experts.{e}.fc1.weight"] = torch.nn.Parameter(w1[e])
        params[f"experts.{e}.fc2.weight"] = torch.nn.Parameter(w2[e])
    placement = ExpertPlacement(cfg.num_experts, (("gpu0",),), {"gpu0": tuple(range(e0, e1))})
    return moe.EPRuntime(cfg, placement, "gpu0", ["gpu0"], None, None, params), params


def _swiglu64(x, w1, w2):
    f = w2.shape[1]
    h = x @ w1.t()
    return (F.silu(h[:, :f]) * h[:, f:]) @ w2.t()


@pytest.mark.parametrize("window", [(0, 16), (112, 128)], ids=["hot-share", "tail-share"])
def test_config4_from_received_buffer(window):
    """Config 4 at 2048 source tokens (8 sources of 256): outputs, input and weight gradients of the
    received rows against float64 autograd of the reference's per-chunk expert_ffn (moe.py:213-223)."""
    e0, e1 = window
    cfg, recv, counts, src, w1, w2 = _ep_share(2048, window)
    full = np.zeros((8, 128), np.int64)
    full[:, e0:e1] = counts
    rt, params = _runtime(cfg, window, w1, w2)
    recv = recv.requires_grad_(True)
    dy = seeded(tuple(recv.shape), 41, 1.0, torch.bfloat16).to(DEV)
    say(f"config 4 received buffer {window}: {recv.shape[0]} rows, counts per expert {counts.sum(0).tolist()}")
    y = rt.expert_outputs(recv, torch.from_numpy(full))
    y.backward(dy)
    plan = K.recv_plan(torch.from_numpy(counts).to(torch.int32).to(DEV))
    torch.cuda.synchronize()
    assert np.array_equal(plan.offsets.cpu().numpy(), M.recv_plan(counts)["offsets"])
    if e0 == 112:
        assert (counts.sum(0) == 0).any(), "the Zipf tail share holds empty experts"
    # float64: the reference's chunk loop, chunk (s, e) by chunk, on the same (bf16) inputs
    x64 = recv.detach().cpu().double().requires_grad_(True)
    p64 = {k: v.detach().cpu().double().requires_grad_(True) for k, v in params.items()}
    outs, q = [], 0
    for s in range(8):
        for i, e in enumerate(range(e0, e1)):
            c = int(counts[s, i])
            if c:
                outs.append(_swiglu64(x64[q:q + c], p64[f"experts.{e}.fc1.weight"], p64[f"experts.{e}.fc2.weight"]))
                q += c
    ref = torch.cat(outs)
    ref.backward(dy.cpu().double())
    bar = TOL[torch.bfloat16]
    errs = {"y": rel_err(y, ref), "drecv": rel_err(recv.grad, x64.grad)}
    for k, p in params.items():
        g64 = p64[k].grad if p64[k].grad is not None else torch.zeros_like(p64[k])
        errs[k] = rel_err(p.grad, g64)
    worst = max(errs, key=errs.get)
    say(f"  worst {worst}: {errs[worst]:.3e}")
    assert errs[worst] <= bar, errs


def test_expert_outputs_reject_unhosted_expert():
    cfg, recv, counts, src, w1, w2 = _ep_share(256, (0, 16))
    rt, _ = _runtime(cfg, (0, 16), w1, w2)
    full = np.zeros((8, 128), np.int64)
    full[:, :16] = counts
    full[2, 40] = 1
    with pytest.raises(RuntimeError, match="does not host"):
        rt.expert_outputs(recv, torch.from_numpy(full))


@pytest.mark.parametrize("window", [(0, 16), (112, 128)], ids=["hot-share", "tail-share"])
def test_config4_from_received_buffer_full_size(window):
    """Config 4 at its full size: 32768 source tokens (8 x 4096) and the received rows of the hot share
    (~226 K) or of the tail share, the least chosen experts, three of which no token picks (under the
    Zipf prior alone every tail expert still gets a few rows at this size).  Plan bit-exact; 256 sampled
    rows' outputs and input gradients, and 16 x 16 sampled elements of each expert's two weight
    gradients (each a sum over all of the expert's rows; zero for an empty expert), against float64."""
    e0, e1 = window
    empty = (115, 120, 127) if e0 == 112 else ()
    cfg, recv, counts, src, w1, w2 = _ep_share(32768, window, empty=empty)
    P = recv.shape[0]
    rt, params = _runtime(cfg, window, w1, w2)
    full = np.zeros((8, 128), np.int64)
    full[:, e0:e1] = counts
    if empty:
        assert (counts.sum(0)[[e - e0 for e in empty]] == 0).all() and (counts.sum(0) > 0).sum() >= 8
    recv = recv.requires_grad_(True)
    g = torch.Generator(device=DEV).manual_seed(17)
    dy = torch.randn(P, 2048, generator=g, device=DEV).to(torch.bfloat16)
    say(f"config 4 full size {window}: {P} received rows, counts per expert {counts.sum(0).tolist()}")
    y = rt.expert_outputs(recv, torch.from_numpy(full))
    y.backward(dy)
    torch.cuda.synchronize()
    ref_plan = M.recv_plan(counts)
    plan = K.recv_plan(torch.from_numpy(counts).to(torch.int32).to(DEV))
    assert np.array_equal(plan.sort_row.cpu().numpy(), ref_plan["sort_row"])
    # expert of every received row
    chunk_exp = np.repeat(np.tile(np.arange(16), 8), counts.reshape(-1))
    rng = np.random.default_rng(5)
    rows = torch.from_numpy(rng.choice(P, min(256, P), replace=False))
    c64 = lambda t: t.detach().cpu().double()  # noqa: E731
    xs, dys = c64(recv[rows.to(DEV)]), c64(dy[rows.to(DEV)])
    yr, dxr = torch.zeros(rows.numel(), 2048, dtype=torch.float64), torch.zeros(rows.numel(), 2048, dtype=torch.float64)
    for i, e in enumerate(range(e0, e1)):
        sel = torch.from_numpy(np.nonzero(chunk_exp[rows.numpy()] == i)[0])
        if sel.numel():
            xe = xs[sel].clone().requires_grad_(True)
            out = _swiglu64(xe, c64(w1[e]), c64(w2[e]))
            out.backward(dys[sel])
            yr[sel], dxr[sel] = out.detach(), xe.grad
    assert rel_err(c64(y[rows.to(DEV)]), yr) <= 2e-2
    assert rel_err(c64(recv.grad[rows.to(DEV)]), dxr) <= 2e-2
    f = 768
    cols = torch.from_numpy(rng.choice(f, 16, replace=False))
    outs = torch.from_numpy(rng.choice(2048, 16, replace=False))
    for i, e in enumerate(range(e0, e1)):
        q = torch.from_numpy(np.nonzero(chunk_exp == i)[0]).to(DEV)
        xe, dye = c64(recv[q]), c64(dy[q])
        W1, W2 = c64(w1[e]), c64(w2[e])
        gt, up = xe @ W1[cols].t(), xe @ W1[f + cols].t()
        act = F.silu(gt) * up
        dact = dye @ W2[:, cols]
        sg = torch.sigmoid(gt)
        dgate, dup = dact * up * sg * (1 + gt * (1 - sg)), dact * F.silu(gt)
        ref_dw2 = dye[:, outs].t() @ act
        ref_dw1g, ref_dw1u = dgate.t() @ xe[:, outs], dup.t() @ xe[:, outs]
        gw1, gw2 = c64(params[f"experts.{e}.fc1.weight"].grad), c64(params[f"experts.{e}.fc2.weight"].grad)
        assert rel_err(gw2[outs][:, cols], ref_dw2) <= 2e-2, ("dw2", e)
        assert rel_err(gw1[cols][:, outs], ref_dw1g) <= 2e-2, ("dw1 gate", e)
        assert rel_err(gw1[f + cols][:, outs], ref_dw1u) <= 2e-2, ("dw1 up", e)
