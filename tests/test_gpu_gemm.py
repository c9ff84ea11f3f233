"""Grouped expert GEMMs on the GPU against float64.

Each entry point is checked in isolation: the float64 reference consumes
exactly the (rounded) inputs the kernel consumed, so the bar is the output
rounding of the storage type.  Cases cover the bfloat16 MFMA path (ragged and
empty groups, partial tiles in every dimension, more groups than one launch
takes, per-group buffers as used by shared experts) and the generic path
(float32, float64, shapes the MFMA path does not take).
"""

from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F

from _helpers import DEV, rel_err, say, seeded
from resihp_megatron_amd import kernels as K

pytestmark = pytest.mark.gpu

# Isolated-kernel bars: output rounding of the storage type (bf16 8 bits).
BAR = {torch.bfloat16: 1e-2, torch.float32: 1e-5, torch.float64: 1e-12}

CASES = [
    # (name, dtype, h, f, counts)
    ("bf16-ragged", torch.bfloat16, 512, 384, [300, 0, 17, 700, 1, 256]),
    ("bf16-multi-tile", torch.bfloat16, 1024, 1024, [1024, 513]),
    ("bf16-70-groups", torch.bfloat16, 128, 128, [(7 * i) % 41 for i in range(70)]),
    # 9 (fc2) and 15 (fc1) weight-gradient tiles per expert: the per-XCD slices
    # of each expert's tiles hold 1 or 2 tiles; skewed counts with an empty expert.
    ("bf16-skewed-uneven-slices", torch.bfloat16, 768, 640, [2000, 900, 0, 257, 64, 3]),
    ("bf16-generic-shape", torch.bfloat16, 40, 24, [9, 3, 0]),
    ("f32", torch.float32, 64, 128, [33, 0, 100, 5]),
    ("f64", torch.float64, 64, 128, [33, 0, 100, 5]),
    ("f64-reference-default", torch.float64, 8, 12, [10, 20, 0, 18]),
]


def _act(act, hp, f):
    if act == "swiglu":
        return F.silu(hp[:, :f]) * hp[:, f:]
    return F.gelu(hp)


def _saved(act, hp, f):
    """What the forward saves for the activation's backward: SwiGLU [up silu'(gate) | silu(gate)], GELU the
    pre-activation."""
    if act == "swiglu":
        g, u = hp[:, :f], hp[:, f:]
        s = torch.sigmoid(g)
        return torch.cat([u * s * (1 + g * (1 - s)), g * s], 1)
    return hp


def _act_bwd(act, da, hp, f):
    if act == "swiglu":
        g, u = hp[:, :f], hp[:, f:]
        s = torch.sigmoid(g)
        return torch.cat([da * u * s * (1 + g * (1 - s)), da * g * s], 1)
    phi = torch.exp(-0.5 * hp * hp) / (2 * torch.pi) ** 0.5
    cdf = 0.5 * (1 + torch.erf(hp / 2 ** 0.5))
    return da * (cdf + hp * phi)


@pytest.mark.parametrize("act", ["swiglu", "gelu"])
@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_grouped_expert_gemms(case, act):
    name, dt, h, f, counts = case
    G = len(counts)
    F1 = 2 * f if act == "swiglu" else f
    offs = torch.tensor([0] + list(torch.tensor(counts).cumsum(0).tolist()), dtype=torch.int32)
    P = int(offs[-1])
    xp = seeded((P, h), 1, 1.0, dt)
    w1 = [seeded((F1, h), 10 + g, 0.05, dt) for g in range(G)]
    w2 = [seeded((h, f), 100 + g, 0.05, dt) for g in range(G)]
    d = lambda t: t.to(DEV)  # noqa: E731
    xp_d, offs_d = d(xp), d(offs)
    w1_d, w2_d = [d(w) for w in w1], [d(w) for w in w2]
    say(f"gemm {name} {act}: G={G} P={P} h={h} f={f}")

    hpre = torch.empty(P, F1, dtype=dt, device=DEV)
    a = torch.empty(P, f, dtype=dt, device=DEV)
    y = torch.empty(P, h, dtype=dt, device=DEV)
    K.expert_fc1_fwd([xp_d] * G, offs_d, True, P, w1_d, f, act, [hpre] * G, [a] * G)
    K.expert_fc2_fwd([a] * G, offs_d, True, P, w2_d, [y] * G)
    dy = seeded((P, h), 2, 1.0, dt)
    dhpre = torch.empty(P, F1, dtype=dt, device=DEV)
    dw2 = [torch.empty_like(w) for w in w2_d]
    K.expert_fc2_bwd([d(dy)] * G, [a] * G, [hpre] * G, offs_d, True, P, w2_d, act, [dhpre] * G, dw2)
    dxp = torch.empty(P, h, dtype=dt, device=DEV)
    dw1 = [torch.empty_like(w) for w in w1_d]
    K.expert_fc1_bwd([dhpre] * G, [xp_d] * G, offs_d, True, P, w1_d, f, act, [dxp] * G, dw1)
    torch.cuda.synchronize()

    bar = BAR[dt]
    c64 = lambda t: t.detach().cpu().double()  # noqa: E731
    hp_g, a_g, dh_g = c64(hpre), c64(a), c64(dhpre)
    for g in range(G):
        r0, r1 = int(offs[g]), int(offs[g + 1])
        xs = c64(xp[r0:r1])
        ref_h = xs @ c64(w1[g]).t()
        assert rel_err(hp_g[r0:r1], _saved(act, ref_h, f)) <= bar, ("hpre", g)
        assert rel_err(a_g[r0:r1], _act(act, ref_h, f)) <= bar, ("act", g)
        ref_y = a_g[r0:r1] @ c64(w2[g]).t()
        assert rel_err(c64(y)[r0:r1], ref_y) <= bar, ("y", g)
        dys = c64(dy[r0:r1])
        ref_dh = _act_bwd(act, dys @ c64(w2[g]), ref_h, f)
        assert rel_err(dh_g[r0:r1], ref_dh) <= bar, ("dhpre", g)
        assert rel_err(c64(dw2[g]), dys.t() @ a_g[r0:r1]) <= bar, ("dw2", g)
        assert rel_err(c64(dxp)[r0:r1], dh_g[r0:r1] @ c64(w1[g])) <= bar, ("dxp", g)
        assert rel_err(c64(dw1[g]), dh_g[r0:r1].t() @ xs) <= bar, ("dw1", g)


@pytest.mark.parametrize("T", [200, 513, 2048])
def test_per_group_buffers_shared_expert_mode(T):
    """rows_from_offsets = 0: each group reads and writes its own buffer from row 0 (shared experts).

    The grid must cover every group's row tiles: with two groups of T rows each that is 2 ceil(T / 256)
    row tiles, more than ceil(T / 256) + 2 once T exceeds 512 (2048: 16 against 10).  Every output and
    gradient of both groups is checked, forward and backward.
    """
    dt, h, f, S, act = torch.bfloat16, 256, 128, 2, "swiglu"
    offs = (torch.arange(S + 1, dtype=torch.int32) * T).to(DEV)
    xs = [seeded((T, h), 5 + s, 1.0, dt) for s in range(S)]
    w1 = [seeded((2 * f, h), 50 + s, 0.05, dt) for s in range(S)]
    w2 = [seeded((h, f), 60 + s, 0.05, dt) for s in range(S)]
    dys = [seeded((T, h), 70 + s, 1.0, dt) for s in range(S)]
    d = lambda ts: [t.to(DEV) for t in ts]  # noqa: E731
    xs_d, w1_d, w2_d, dys_d = d(xs), d(w1), d(w2), d(dys)
    say(f"gemm shared-expert buffers T={T}")
    hs = [torch.empty(T, 2 * f, dtype=dt, device=DEV) for _ in range(S)]
    as_ = [torch.empty(T, f, dtype=dt, device=DEV) for _ in range(S)]
    ys = [torch.empty(T, h, dtype=dt, device=DEV) for _ in range(S)]
    K.expert_fc1_fwd(xs_d, offs, False, T, w1_d, f, act, hs, as_)
    K.expert_fc2_fwd(as_, offs, False, T, w2_d, ys)
    dh = [torch.empty(T, 2 * f, dtype=dt, device=DEV) for _ in range(S)]
    dw2 = [torch.empty_like(w) for w in w2_d]
    K.expert_fc2_bwd(dys_d, as_, hs, offs, False, T, w2_d, act, dh, dw2)
    dx = [torch.empty(T, h, dtype=dt, device=DEV) for _ in range(S)]
    dw1 = [torch.empty_like(w) for w in w1_d]
    K.expert_fc1_bwd(dh, xs_d, offs, False, T, w1_d, f, act, dx, dw1)
    torch.cuda.synchronize()
    c64 = lambda t: t.detach().cpu().double()  # noqa: E731
    for s in range(S):
        x64, a64, h64, dh64, dy64 = c64(xs[s]), c64(as_[s]), c64(hs[s]), c64(dh[s]), c64(dys[s])
        ref_h = x64 @ c64(w1[s]).t()
        assert rel_err(h64, _saved(act, ref_h, f)) <= 1e-2, ("hpre", s)
        assert rel_err(a64, _act(act, ref_h, f)) <= 1e-2, ("act", s)
        assert rel_err(ys[s], a64 @ c64(w2[s]).t()) <= 1e-2, ("y", s)
        assert rel_err(dh64, _act_bwd(act, dy64 @ c64(w2[s]), ref_h, f)) <= 1e-2, ("dhpre", s)
        assert rel_err(dw2[s], dy64.t() @ a64) <= 1e-2, ("dw2", s)
        assert rel_err(dx[s], dh64 @ c64(w1[s])) <= 1e-2, ("dx", s)
        assert rel_err(dw1[s], dh64.t() @ x64) <= 1e-2, ("dw1", s)


def test_gemm_deterministic():
    dt, h, f = torch.bfloat16, 512, 256
    counts = [400, 333]
    offs = torch.tensor([0, 400, 733], dtype=torch.int32).to(DEV)
    xp = seeded((733, h), 1, 1.0, dt).to(DEV)
    w1 = [seeded((2 * f, h), 3 + g, 0.05, dt).to(DEV) for g in range(2)]
    say("gemm determinism")
    outs = []
    for _ in range(2):
        hp = torch.empty(733, 2 * f, dtype=dt, device=DEV)
        a = torch.empty(733, f, dtype=dt, device=DEV)
        K.expert_fc1_fwd([xp] * 2, offs, True, 733, w1, f, "swiglu", [hp] * 2, [a] * 2)
        outs.append((hp, a))
    torch.cuda.synchronize()
    assert torch.equal(outs[0][0], outs[1][0]) and torch.equal(outs[0][1], outs[1][1])
    assert sum(counts) == 733


# K split of the last round of tiles.  Each XCD runs its share of tiles in rounds of one tile per CU;
# where a tile's reduction is long (at least 128 K steps of 64), the tiles of an XCD's last, partial
# round are cut along K into pieces whose fp32 partial tiles the last piece to finish adds in piece
# order.  (name, h, f, counts, rows checked against float64): "deep" puts one fc2 forward and one fc1
# input-gradient tile on each of six XCDs, cut in eight pieces; "rounds" gives every XCD 33 tiles of
# each, one whole round of 32 and one tile (the last row tile) cut in eight.
SPLIT_CASES = [
    ("deep", 512, 8192, [300, 40], None),
    ("rounds", 2048, 8192, [8448], list(range(0, 64)) + list(range(8192, 8448))),
]


@pytest.mark.parametrize("case", SPLIT_CASES, ids=[c[0] for c in SPLIT_CASES])
def test_k_split_tiles(case):
    name, h, f, counts, rows = case
    dt, G, act = torch.bfloat16, len(counts), "swiglu"
    F1 = 2 * f
    offs = torch.tensor([0] + list(torch.tensor(counts).cumsum(0).tolist()), dtype=torch.int32)
    P = int(offs[-1])
    a = seeded((P, f), 1, 1.0, dt)
    dh = seeded((P, F1), 2, 1.0, dt)
    w1 = [seeded((F1, h), 10 + g, 0.02, dt) for g in range(G)]
    w2 = [seeded((h, f), 100 + g, 0.02, dt) for g in range(G)]
    d = lambda t: t.to(DEV)  # noqa: E731
    offs_d, a_d, dh_d = d(offs), d(a), d(dh)
    w1_d, w2_d = [d(w) for w in w1], [d(w) for w in w2]
    xp_d = d(seeded((P, h), 3, 1.0, dt))
    say(f"gemm k-split {name}: G={G} P={P} h={h} f={f}")

    def run(split):
        y = torch.empty(P, h, dtype=dt, device=DEV)
        K.expert_fc2_fwd([a_d] * G, offs_d, True, P, w2_d, [y] * G, split=split)
        dxp = torch.empty(P, h, dtype=dt, device=DEV)
        dw1 = [torch.empty_like(w) for w in w1_d]
        K.expert_fc1_bwd([dh_d] * G, [xp_d] * G, offs_d, True, P, w1_d, f, act, [dxp] * G, dw1, split=split)
        torch.cuda.synchronize()
        return y.cpu(), dxp.cpu()

    y_s, dx_s = run(True)
    y_s2, dx_s2 = run(True)
    y_n, dx_n = run(False)
    # the last piece sums in piece order: the same bits on every run
    assert torch.equal(y_s, y_s2) and torch.equal(dx_s, dx_s2)
    # split and unsplit differ only in fp32 summation order before the bf16 rounding
    assert rel_err(y_s, y_n.double()) <= 1e-2 and rel_err(dx_s, dx_n.double()) <= 1e-2
    c64 = lambda t: t.detach().cpu().double()  # noqa: E731
    for g in range(G):
        r0, r1 = int(offs[g]), int(offs[g + 1])
        sel = torch.tensor([r for r in (rows if rows is not None else range(r0, r1)) if r0 <= r < r1])
        ref_y = c64(a[sel]) @ c64(w2[g]).t()
        ref_dx = c64(dh[sel]) @ c64(w1[g])
        assert rel_err(c64(y_s[sel]), ref_y) <= 1e-2, ("y", g)
        assert rel_err(c64(dx_s[sel]), ref_dx) <= 1e-2, ("dxp", g)


def test_mixtral_shape_beyond_2gib_buffers():
    """Row buffers past 2 GiB on the MFMA kernel: the Mixtral hidden/ffn sizes with 40960 routed pairs
    (20480 tokens at top-2), pre-activations [40960, 28672] bf16 = 2.35 GB.  One hot expert holds 38000
    rows, so its weight-gradient reduction runs past 2 GiB of its own pre-activation gradient rows (37449
    rows of 57 KB).  Sampled rows of every output and sampled elements of both weight gradients are
    checked against float64 on the kernel's own inputs."""
    dt, h, f, act = torch.bfloat16, 4096, 14336, "swiglu"
    counts = [38000, 2960]
    G, F1 = len(counts), 2 * f
    assert K.gemm_kernel(dt, act, h, f) == "mfma"
    offs = torch.tensor([0] + list(torch.tensor(counts).cumsum(0).tolist()), dtype=torch.int32)
    P = int(offs[-1])
    gen = torch.Generator(device=DEV).manual_seed(11)
    rnd = lambda *s, std=1.0: (torch.randn(*s, generator=gen, device=DEV) * std).to(dt)  # noqa: E731
    xp, dy = rnd(P, h), rnd(P, h)
    w1 = [rnd(F1, h, std=0.02) for _ in range(G)]
    w2 = [rnd(h, f, std=0.02) for _ in range(G)]
    offs_d = offs.to(DEV)
    say(f"gemm beyond 2 GiB: P={P} counts={counts}")
    hpre = torch.empty(P, F1, dtype=dt, device=DEV)
    a = torch.empty(P, f, dtype=dt, device=DEV)
    y = torch.empty(P, h, dtype=dt, device=DEV)
    K.expert_fc1_fwd([xp] * G, offs_d, True, P, w1, f, act, [hpre] * G, [a] * G)
    K.expert_fc2_fwd([a] * G, offs_d, True, P, w2, [y] * G)
    dhpre = torch.empty(P, F1, dtype=dt, device=DEV)
    dw2 = [torch.empty_like(w) for w in w2]
    K.expert_fc2_bwd([dy] * G, [a] * G, [hpre] * G, offs_d, True, P, w2, act, [dhpre] * G, dw2)
    dxp = torch.empty(P, h, dtype=dt, device=DEV)
    dw1 = [torch.empty_like(w) for w in w1]
    K.expert_fc1_bwd([dhpre] * G, [xp] * G, offs_d, True, P, w1, f, act, [dxp] * G, dw1)
    torch.cuda.synchronize()
    assert hpre.numel() * 2 > 2 ** 31
    c64 = lambda t: t.detach().cpu().double()  # noqa: E731
    g8 = torch.Generator().manual_seed(3)
    for g in range(G):
        r0, r1 = int(offs[g]), int(offs[g + 1])
        # 16 rows of the group, always including its first and last
        rows = torch.cat([torch.tensor([r0, r1 - 1]), torch.randint(r0, r1, (14,), generator=g8)]).to(DEV)
        x64, dy64, h64, a64, dh64 = (c64(t[rows]) for t in (xp, dy, hpre, a, dhpre))
        ref_h = x64 @ c64(w1[g]).t()
        assert rel_err(h64, _saved(act, ref_h, f)) <= 1e-2, ("hpre", g)
        assert rel_err(a64, _act(act, ref_h, f)) <= 1e-2, ("act", g)
        assert rel_err(c64(y[rows]), a64 @ c64(w2[g]).t()) <= 1e-2, ("y", g)
        assert rel_err(dh64, _act_bwd(act, dy64 @ c64(w2[g]), ref_h, f)) <= 1e-2, ("dhpre", g)
        assert rel_err(c64(dxp[rows]), dh64 @ c64(w1[g])) <= 1e-2, ("dxp", g)
        # weight gradients: 16 x 64 sampled elements, each a sum over all of the group's rows
        o2 = torch.randint(0, h, (16,), generator=g8)
        i2 = torch.randint(0, f, (64,), generator=g8)
        ref2 = c64(dy[r0:r1][:, o2.to(DEV)]).t() @ c64(a[r0:r1][:, i2.to(DEV)])
        assert rel_err(c64(dw2[g])[o2][:, i2], ref2) <= 1e-2, ("dw2", g)
        o1 = torch.cat([torch.tensor([0, F1 - 1]), torch.randint(0, F1, (14,), generator=g8)])
        i1 = torch.randint(0, h, (64,), generator=g8)
        ref1 = c64(dhpre[r0:r1][:, o1.to(DEV)]).t() @ c64(xp[r0:r1][:, i1.to(DEV)])
        assert rel_err(c64(dw1[g])[o1][:, i1], ref1) <= 1e-2, ("dw1", g)


def test_kernel_choice_and_alignment():
    """bfloat16 shapes the MFMA kernel takes run on it (any row count); an unaligned bfloat16 operand
    is an error, not a silent switch to the generic kernel; other shapes and dtypes take the generic one."""
    assert K.gemm_kernel(torch.bfloat16, "swiglu", 4096, 14336) == "mfma"
    assert K.gemm_kernel(torch.bfloat16, "gelu", 40, 24) == "generic"
    assert K.gemm_kernel(torch.float32, "swiglu", 4096, 14336) == "generic"
    assert K.gemm_kernel(torch.float64, "gelu", 64, 128) == "generic"
    dt, h, f, P = torch.bfloat16, 256, 128, 300
    offs = torch.tensor([0, P], dtype=torch.int32, device=DEV)
    flat = torch.zeros(P * h + 1, dtype=dt, device=DEV)
    xp = flat[1:].view(P, h)      # 2 bytes past a 16-byte boundary
    w1 = [seeded((2 * f, h), 1, 0.05, dt).to(DEV)]
    hp = torch.empty(P, 2 * f, dtype=dt, device=DEV)
    a = torch.empty(P, f, dtype=dt, device=DEV)
    say("gemm unaligned operand")
    with pytest.raises(RuntimeError, match="16-byte aligned"):
        K.expert_fc1_fwd([xp], offs, True, P, w1, f, "swiglu", [hp], [a])


def test_k_split_workspace_per_stream():
    """Each stream gets its own K-split workspace, so split products on two streams at once do not
    share arrival counters: both give the bits of the same product run alone.  A reset leaves the
    counters zero and the next call correct."""
    dt, h, f, counts = torch.bfloat16, 512, 8192, [300, 40]
    G = len(counts)
    offs = torch.tensor([0, 300, 340], dtype=torch.int32, device=DEV)
    P = 340
    gen = torch.Generator(device=DEV).manual_seed(5)
    a = [(torch.randn(P, f, generator=gen, device=DEV)).to(dt) for _ in range(2)]
    w2 = [(torch.randn(h, f, generator=gen, device=DEV) * 0.02).to(dt) for _ in range(G)]
    say("gemm k-split workspace per stream")
    alone = []
    for i in range(2):
        y = torch.empty(P, h, dtype=dt, device=DEV)
        K.expert_fc2_fwd([a[i]] * G, offs, True, P, w2, [y] * G)
        alone.append(y)
    torch.cuda.synchronize()
    side = torch.cuda.Stream(device=DEV)
    main = torch.cuda.current_stream(DEV)
    assert K.split_workspace(torch.device(DEV), side).data_ptr() != K.split_workspace(torch.device(DEV), main).data_ptr()
    side.wait_stream(main)
    outs = [torch.empty(P, h, dtype=dt, device=DEV) for _ in range(2)]
    for _ in range(3):
        with torch.cuda.stream(side):
            K.expert_fc2_fwd([a[1]] * G, offs, True, P, w2, [outs[1]] * G)
        K.expert_fc2_fwd([a[0]] * G, offs, True, P, w2, [outs[0]] * G)
    main.wait_stream(side)
    torch.cuda.synchronize()
    assert torch.equal(outs[0], alone[0]) and torch.equal(outs[1], alone[1])
    ws = K.split_workspace(torch.device(DEV))
    K.reset_split_workspace(ws)
    y = torch.empty(P, h, dtype=dt, device=DEV)
    K.expert_fc2_fwd([a[0]] * G, offs, True, P, w2, [y] * G)
    torch.cuda.synchronize()
    assert torch.equal(y, alone[0])
    counters = ws[K.C.lib().rhp_expert_split_workspace_bytes() - 4 * 256:].view(torch.int32)
    assert int(counters.abs().sum()) == 0


def test_k_split_workspaces_stay_bounded_over_fresh_streams():
    """A stream per call (a serving loop) does not grow device memory: only the last few streams of a
    device keep a K-split workspace, and split products on fresh streams keep giving the same bits."""
    dt, h, f, counts = torch.bfloat16, 256, 8192, [200, 60]
    G = len(counts)
    offs = torch.tensor([0, 200, 260], dtype=torch.int32, device=DEV)
    P = 260
    gen = torch.Generator(device=DEV).manual_seed(6)
    a = (torch.randn(P, f, generator=gen, device=DEV)).to(dt)
    w2 = [(torch.randn(h, f, generator=gen, device=DEV) * 0.02).to(dt) for _ in range(G)]
    say("gemm k-split workspaces over 10 fresh streams")
    ref = torch.empty(P, h, dtype=dt, device=DEV)
    K.expert_fc2_fwd([a] * G, offs, True, P, w2, [ref] * G)
    torch.cuda.synchronize()
    dev_idx = torch.device(DEV).index or 0
    sizes = []
    for i in range(10):
        s = torch.cuda.Stream(device=DEV)
        s.wait_stream(torch.cuda.current_stream(DEV))
        y = torch.empty(P, h, dtype=dt, device=DEV)
        with torch.cuda.stream(s):
            K.expert_fc2_fwd([a] * G, offs, True, P, w2, [y] * G)
        s.synchronize()
        assert torch.equal(y, ref), i
        sizes.append(sum(1 for key in K._split_ws_cache if key[0] == dev_idx))
    assert max(sizes) <= K._SPLIT_WS_PER_DEVICE and sizes[-1] == K._SPLIT_WS_PER_DEVICE


@pytest.mark.parametrize("dtype,h,f,counts,e0", [(torch.bfloat16, 256, 128, [300, 0, 517], 2),
                                                 (torch.bfloat16, 512, 256, [40, 700, 129, 1], 0),
                                                 (torch.bfloat16, 1024, 8192, [200, 330], 1),
                                                 (torch.float32, 96, 40, [33, 0, 70], 1)],
                         ids=["bf16", "bf16-ragged", "bf16-k-split", "f32-generic"])
def test_fc1_dgrad_router_term(dtype, h, f, counts, e0):
    """fc1's input gradient with the router term in its epilogue: dxp[r] = dhpre[r] @ w1 + dl[perm[r]] *
    W_router[e0 + g] against float64 on the same inputs (the third case's reduction of 16384 is K-split)."""
    G, P = len(counts), sum(counts)
    E, k = e0 + G + 2, 2
    T = (P + k - 1) // k + 3
    offsets = torch.tensor([0] + torch.tensor(counts).cumsum(0).tolist(), dtype=torch.int32, device=DEV)
    g = torch.Generator().manual_seed(h + f)
    perm = torch.randperm(T * k, generator=g)[:P].to(torch.int32)
    dl = torch.randn(T, k, generator=g) * 0.5
    W = torch.randn(E, h, generator=g) * 0.1 * (2 * f) ** 0.5   # router term as large as the product's rows
    dh = seeded((P, 2 * f), 3, 1.0, dtype)
    w1 = [seeded((2 * f, h), 10 + i, 0.05, dtype) for i in range(G)]
    say(f"fc1 dgrad + router term {dtype} h={h} f={f} counts={counts} e0={e0}")
    dx = torch.empty(P, h, dtype=dtype, device=DEV)
    K.expert_fc1_dgrad_router([dh.to(DEV)] * G, offsets, P, [w.to(DEV) for w in w1], f, "swiglu", W.to(DEV), e0,
                              perm.to(DEV), dl.to(DEV), [dx] * G)
    torch.cuda.synchronize()
    ref = torch.empty(P, h, dtype=torch.float64)
    o = offsets.cpu().tolist()
    for i in range(G):
        r = slice(o[i], o[i + 1])
        ref[r] = dh[r].double() @ w1[i].double() + dl.double().view(-1)[perm[r].long()][:, None] * W[e0 + i].double()
    assert rel_err(dx, ref) <= (2e-2 if dtype == torch.bfloat16 else 1e-5)
    # the router term is really there: without it the rows differ by far more than the rounding
    bare = torch.cat([dh[o[i]:o[i + 1]].double() @ w1[i].double() for i in range(G)])
    assert rel_err(bare, ref) > 1e-2
