"""FP8 experts on the GPU: delayed-scaling casts bit for bit against the oracle, and every fp8
product against float64 on the dequantised operands.

The cast must reproduce oracle/moe_ref.py's recipe exactly (scale from the
amax history, saturating round-to-nearest-even to OCP e4m3 / e5m2), including
the per-expert transposed copies with zero padding, the running amax and the
history roll.  The products consume exactly the codes the cast wrote, so the
float64 reference (codes / scale) differs from the kernel only by fp32
accumulation and the bf16 rounding of the outputs.
"""

from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F

from _helpers import DEV, rel_err, say, seeded
from oracle import moe_ref as M
from resihp_megatron_amd import kernels as K

pytestmark = pytest.mark.gpu

BAR = 1e-2   # bf16 output rounding of products of exact fp8 codes
# Whole layer against the quantised emulation: an intermediate computed in fp32 on the GPU and in
# float64 here can land on the other side of a bf16 or fp8 rounding boundary before the next cast.
# The fc1 weight gradient passes two such roundings (bf16 dhpre, then its e5m2 code, 25 % apart at a
# binade edge), and with few rows per expert one flipped code shows in the max-relative error.
LAYER_BAR = 2e-2
DW1_BAR = 5e-2


def _offsets(counts):
    return torch.tensor([0] + torch.tensor(counts).cumsum(0).tolist(), dtype=torch.int32)


def _history(seed, L=16, scale=3.0):
    return (torch.rand(L, generator=torch.Generator().manual_seed(seed), dtype=torch.float32) * scale + 0.1)


def _cast(x, counts, hist, fmt, q=True, qt=True, margin=0):
    """GPU cast of bf16 rows x (host) split into experts of `counts`."""
    offs = _offsets(counts).to(DEV)
    poff = K.fp8_padded_offsets(offs)
    rows, cols = x.shape
    _, fdt, _ = K.FP8_FORMATS[fmt]
    amax = torch.zeros(1, dtype=torch.int32, device=DEV)
    sinv = torch.zeros(1, dtype=torch.float32, device=DEV)
    qd = torch.empty(rows, cols, dtype=fdt, device=DEV) if q else None
    qtd = torch.zeros(K.fp8_transposed_numel(cols, rows, len(counts)), dtype=fdt, device=DEV) if qt else None
    K.fp8_cast(x.to(DEV), offs, poff, rows, hist.to(DEV), fmt, amax, sinv, qd, qtd, margin)
    return offs, poff, qd, qtd, amax, sinv


def _codes(t):
    return t.detach().cpu().view(torch.uint8)


@pytest.mark.parametrize("fmt,margin", [("e4m3", 0), ("e5m2", 0), ("e4m3", 1)])
def test_cast_matches_oracle_bits(fmt, margin):
    counts = [300, 0, 17, 129]
    cols = 192
    x = seeded((sum(counts), cols), 11, 2.0, torch.bfloat16)
    x[5, 7] = 900.0                      # saturates in e4m3 at scale > 0.5
    hist = _history(3)
    say(f"fp8 cast {fmt} margin={margin}")
    offs, poff, q, qt, amax, sinv = _cast(x, counts, hist, fmt, margin=margin)
    torch.cuda.synchronize()
    scale = M.fp8_scale(hist.double(), fmt, margin)
    ref = M.quantize(x.double(), scale, fmt).to(K.FP8_FORMATS[fmt][1])
    assert torch.equal(_codes(q), ref.view(torch.uint8)), "row-major codes differ"
    # transposed copies: expert g at cols * poff[g], [cols, R_g], zero past its rows
    po = poff.cpu().tolist()
    assert po == [0, 384, 384, 512, 768]
    qt_h = _codes(qt)
    o = _offsets(counts).tolist()
    for g, n in enumerate(counts):
        Rg = po[g + 1] - po[g]
        blk = qt_h[cols * po[g]: cols * po[g + 1]].reshape(cols, Rg)
        assert torch.equal(blk[:, :n], ref.view(torch.uint8)[o[g]:o[g + 1]].t()), f"expert {g} transposed codes differ"
        assert not blk[:, n:].any(), f"expert {g} padding is not zero"
    assert torch.equal(amax.cpu().view(torch.float32), x.float().abs().max().reshape(1))
    assert sinv.item() == (torch.tensor(1.0) / torch.tensor(scale, dtype=torch.float32)).item()


def test_cast_scale_falls_back_to_one():
    x = seeded((64, 64), 12, 1.0, torch.bfloat16)
    for hist in (torch.zeros(4), torch.tensor([1.0, float("nan"), 2.0, 3.0]), torch.tensor([float("inf"), 1.0])):
        say(f"fp8 cast history {hist.tolist()}")
        _, _, q, _, _, sinv = _cast(x, [64], hist, "e4m3", qt=False)
        torch.cuda.synchronize()
        assert M.fp8_scale(hist.double(), "e4m3") == 1.0
        assert sinv.item() == 1.0
        assert torch.equal(_codes(q), M.quantize(x.double(), 1.0, "e4m3").to(torch.float8_e4m3fn).view(torch.uint8))


def test_amax_roll_newest_first():
    hist = torch.tensor([[4.0, 3.0, 2.0, 1.0], [1.0, 1.0, 1.0, 1.0], [0.5, 0.25, 0.0, 0.0]])
    amax = torch.tensor([9.0, 0.0, 7.5]).view(torch.int32)
    h, a = hist.to(DEV), amax.to(DEV)
    say("fp8 amax roll")
    K.fp8_amax_roll(h, a)
    torch.cuda.synchronize()
    for i in range(3):
        assert torch.equal(h[i].cpu(), M.amax_roll(hist[i], amax.view(torch.float32)[i]).float())
    assert not a.cpu().any()


def _deq(q, sinv):
    return q.detach().cpu().to(torch.float64) * float(sinv.item())


def _swiglu_saved(hp, f):
    """What the SwiGLU forward saves for the backward: [up silu'(gate) | silu(gate)]."""
    g, u = hp[:, :f], hp[:, f:]
    s = torch.sigmoid(g)
    return torch.cat([u * s * (1 + g * (1 - s)), g * s], 1)


def _swiglu_bwd(da, saved, f):
    """The SwiGLU backward from the saved factors."""
    return torch.cat([da * saved[:, :f], da * saved[:, f:]], 1)


GEMM_CASES = [
    # (name, h, f, counts)
    ("ragged", 256, 384, [200, 0, 300]),
    ("one-expert-multi-tile", 512, 256, [700]),
]


@pytest.mark.parametrize("case", GEMM_CASES, ids=[c[0] for c in GEMM_CASES])
def test_fp8_expert_products(case):
    name, h, f, counts = case
    G, P = len(counts), sum(counts)
    o = _offsets(counts).tolist()
    say(f"fp8 products {name}: h={h} f={f} counts={counts}")
    x = seeded((P, h), 21, 1.0, torch.bfloat16)
    w1 = [seeded((2 * f, h), 30 + g, 0.05, torch.bfloat16) for g in range(G)]
    w2 = [seeded((h, f), 40 + g, 0.05, torch.bfloat16) for g in range(G)]
    a = seeded((P, f), 22, 0.5, torch.bfloat16)
    dy = seeded((P, h), 23, 0.01, torch.bfloat16)
    dh = seeded((P, 2 * f), 24, 0.01, torch.bfloat16)
    hist = _history(5)

    offs, poff, xq, xqt, _, sx = _cast(x, counts, hist, "e4m3")
    _, _, aq, aqt, _, sa = _cast(a, counts, hist, "e4m3")
    _, _, dyq, dyqt, _, sdy = _cast(dy, counts, _history(6, scale=0.05), "e5m2")
    _, _, dhq, dhqt, _, sdh = _cast(dh, counts, _history(7, scale=0.05), "e5m2")
    w1q, w1qt, w2q, w2qt = [], [], [], []
    sw1 = torch.empty(G, dtype=torch.float32, device=DEV)
    sw2 = torch.empty(G, dtype=torch.float32, device=DEV)
    for g in range(G):
        hw = _history(50 + g, scale=0.2)
        _, _, q1, t1, _, s1 = _cast(w1[g], [2 * f], hw, "e4m3")
        _, _, q2, t2, _, s2 = _cast(w2[g], [h], hw, "e4m3")
        w1q.append(q1); w1qt.append(t1[: 2 * f * h].view(h, 2 * f)); sw1[g:g + 1].copy_(s1)
        w2q.append(q2); w2qt.append(t2[: h * f].view(f, h)); sw2[g:g + 1].copy_(s2)

    hpre = torch.empty(P, 2 * f, dtype=torch.bfloat16, device=DEV)
    act = torch.empty(P, f, dtype=torch.bfloat16, device=DEV)
    y = torch.empty(P, h, dtype=torch.bfloat16, device=DEV)
    dhpre = torch.empty(P, 2 * f, dtype=torch.bfloat16, device=DEV)
    dxp = torch.empty(P, h, dtype=torch.bfloat16, device=DEV)
    dw2 = [torch.empty(h, f, dtype=torch.bfloat16, device=DEV) for _ in range(G)]
    dw1 = [torch.empty(2 * f, h, dtype=torch.bfloat16, device=DEV) for _ in range(G)]
    hp_in = seeded((P, 2 * f), 25, 1.0, torch.bfloat16).to(DEV)

    K.fp8_gemm(False, "swiglu_fwd", offs, P, [xq] * G, "e4m3", w1q, "e4m3", f, h, 0, f, [hpre] * G, sx, sw1,
               c2s=[act] * G)
    K.fp8_gemm(False, "store", offs, P, [aq] * G, "e4m3", w2q, "e4m3", h, f, 0, f, [y] * G, sa, sw2)
    K.fp8_gemm(False, "swiglu_bwd", offs, P, [dyq] * G, "e5m2", w2qt, "e4m3", f, h, 0, f, [dhpre] * G, sdy, sw2,
               auxs=[hp_in] * G)
    K.fp8_gemm(False, "store", offs, P, [dhq] * G, "e5m2", w1qt, "e4m3", h, 2 * f, 0, f, [dxp] * G, sdh, sw1)
    K.fp8_gemm(True, "store", poff, P, [dyqt], "e5m2", [aqt], "e4m3", f, 0, h, f, dw2, sdy, sa)
    K.fp8_gemm(True, "store", poff, P, [dhqt], "e5m2", [xqt], "e4m3", h, 0, 2 * f, f, dw1, sdh, sx)
    # The same backward products on the row-major codes (modes 2 and 3: N-contiguous operands, transposed in
    # LDS): every lane multiplies the same k as in modes 0 and 1, so the results are the same bits.
    dhpre_kn, dxp_kn = torch.empty_like(dhpre), torch.empty_like(dxp)
    dw2_mn, dw1_mn = [torch.empty_like(w) for w in dw2], [torch.empty_like(w) for w in dw1]
    K.fp8_gemm(2, "swiglu_bwd", offs, P, [dyq] * G, "e5m2", w2q, "e4m3", f, h, 0, f, [dhpre_kn] * G, sdy, sw2,
               auxs=[hp_in] * G)
    K.fp8_gemm(2, "store", offs, P, [dhq] * G, "e5m2", w1q, "e4m3", h, 2 * f, 0, f, [dxp_kn] * G, sdh, sw1)
    K.fp8_gemm(3, "store", offs, P, [dyq], "e5m2", [aq], "e4m3", f, 0, h, f, dw2_mn, sdy, sa)
    K.fp8_gemm(3, "store", offs, P, [dhq], "e5m2", [xq], "e4m3", h, 0, 2 * f, f, dw1_mn, sdh, sx)
    torch.cuda.synchronize()
    _same_bits(dhpre_kn, dhpre, "fc2 dgrad on [K, N] weight codes")
    _same_bits(dxp_kn, dxp, "fc1 dgrad on [K, N] weight codes")
    for g in range(G):
        _same_bits(dw2_mn[g], dw2[g], f"fc2 wgrad on row-major codes, expert {g}")
        _same_bits(dw1_mn[g], dw1[g], f"fc1 wgrad on row-major codes, expert {g}")

    xd, ad, dyd, dhd = _deq(xq, sx), _deq(aq, sa), _deq(dyq, sdy), _deq(dhq, sdh)
    hp64 = hp_in.cpu().double()
    for g in range(G):
        r = slice(o[g], o[g + 1])
        w1d, w2d = _deq(w1q[g], sw1[g]), _deq(w2q[g], sw2[g])
        ref_h = xd[r] @ w1d.t()
        assert rel_err(hpre[r], _swiglu_saved(ref_h, f)) <= BAR, f"fc1 fwd expert {g}"
        assert rel_err(act[r], F.silu(ref_h[:, :f]) * ref_h[:, f:]) <= BAR, f"SwiGLU expert {g}"
        assert rel_err(y[r], ad[r] @ w2d.t()) <= BAR, f"fc2 fwd expert {g}"
        assert rel_err(dhpre[r], _swiglu_bwd(dyd[r] @ w2d, hp64[r], f)) <= BAR, f"fc2 dgrad expert {g}"
        assert rel_err(dxp[r], dhd[r] @ w1d) <= BAR, f"fc1 dgrad expert {g}"
        assert rel_err(dw2[g], dyd[r].t() @ ad[r]) <= BAR, f"fc2 wgrad expert {g}"
        assert rel_err(dw1[g], dhd[r].t() @ xd[r]) <= BAR, f"fc1 wgrad expert {g}"


def _fp8_weights(w1, w2):
    """Cast expert weights as the layer does: row-major fc1 codes, transposed fc2 codes, 1/scales [G]."""
    G = len(w1)
    w1q, w2qt = [], []
    sw1 = torch.empty(G, dtype=torch.float32, device=DEV)
    sw2 = torch.empty(G, dtype=torch.float32, device=DEV)
    for g in range(G):
        hw = _history(50 + g, scale=0.2)
        _, _, q1, _, _, s1 = _cast(w1[g], [w1[g].shape[0]], hw, "e4m3", qt=False)
        _, _, _, t2, _, s2 = _cast(w2[g], [w2[g].shape[0]], hw, "e4m3", q=False)
        w1q.append(q1); sw1[g:g + 1].copy_(s1)
        w2qt.append(t2[: w2[g].numel()].view(w2[g].shape[1], w2[g].shape[0])); sw2[g:g + 1].copy_(s2)
    return w1q, sw1, w2qt, sw2


def _cast_buffers(P, cols, G, fmt):
    """Code buffers for a cast, the transposed one pre-filled with a marker byte (padding must be written)."""
    fdt = K.FP8_FORMATS[fmt][1]
    amax = torch.zeros(1, dtype=torch.int32, device=DEV)
    sinv = torch.zeros(1, dtype=torch.float32, device=DEV)
    q = torch.empty(P, cols, dtype=fdt, device=DEV)
    qt = torch.full((K.fp8_transposed_numel(cols, P, G),), 0x55, dtype=torch.uint8, device=DEV).view(fdt)
    return amax, sinv, q, qt


def _same_bits(a, b, what):
    assert torch.equal(_codes(a), _codes(b)), f"{what} differ"


# Expert rows cover a full tile plus a tile whose second half is empty (300), a tile whose
# second half is partly filled (200) and one row into the second half (129); f = 384 leaves the
# backward products' last column tile half valid.
FUSED_COUNTS = [200, 0, 300, 129]


@pytest.mark.parametrize("act", ["swiglu", "gelu"])
@pytest.mark.parametrize("hist_scale,margin", [(3.0, 0), (0.02, 0), (3.0, 2)])
def test_fused_cast_matches_product_then_cast(act, hist_scale, margin):
    """rhp_fp8_gemm_cast = rhp_fp8_gemm + rhp_fp8_cast of its bf16 activation output, bit for bit."""
    _fused_case(act, hist_scale, margin, 256, 384, FUSED_COUNTS)


@pytest.mark.parametrize("act", ["swiglu", "gelu"])
def test_fused_cast_edge_rows(act):
    """Experts of 1, 255, 256, 257 and 513 rows and an empty one; h = 384, f = 640 (half-valid last tiles)."""
    _fused_case(act, 3.0, 0, 384, 640, [1, 255, 0, 256, 257, 513])


def test_fused_cast_many_tiles():
    """About 2300 tiles a product (7300 rows, h = 1024, f = 2048): every epilogue store of the fused
    products, factors and codes alike, bit for bit against the unfused pair.  A 16-byte store whose data
    registers were overwritten right after it (register soffset, no wait states) changed 64 of 483,072
    stored values in a 12-tile product; this one has 40 times the tiles."""
    _fused_case("swiglu", 3.0, 0, 1024, 2048, [2048, 1537, 0, 3000, 700])


def _fused_case(act, hist_scale, margin, h, f, counts):
    G, P = len(counts), sum(counts)
    F1 = 2 * f if act == "swiglu" else f
    say(f"fp8 fused cast {act} hist_scale={hist_scale} margin={margin}: h={h} f={f} counts={counts}")
    x = seeded((P, h), 61, 1.0, torch.bfloat16)
    dy = seeded((P, h), 62, 0.01, torch.bfloat16)
    hp_in = seeded((P, F1), 63, 1.0, torch.bfloat16).to(DEV)
    w1 = [seeded((F1, h), 70 + g, 0.05, torch.bfloat16) for g in range(G)]
    w2 = [seeded((h, f), 80 + g, 0.05, torch.bfloat16) for g in range(G)]
    offs, poff, xq, _, _, sx = _cast(x, counts, _history(64), "e4m3", qt=False)
    _, _, dyq, _, _, sdy = _cast(dy, counts, _history(65, scale=0.05), "e5m2", qt=False)
    w1q, sw1, w2qt, sw2 = _fp8_weights(w1, w2)
    # small histories saturate part of the outputs
    hist_a = _history(66, scale=hist_scale).to(DEV)
    hist_d = _history(67, scale=hist_scale * 0.01).to(DEV)

    # forward: pre-activation and activation codes
    hpre_u = torch.empty(P, F1, dtype=torch.bfloat16, device=DEV)
    act_u = torch.empty(P, f, dtype=torch.bfloat16, device=DEV)
    K.fp8_gemm(False, f"{act}_fwd", offs, P, [xq] * G, "e4m3", w1q, "e4m3", f, h, 0, f, [hpre_u] * G, sx, sw1,
               c2s=[act_u] * G)
    au = _cast_buffers(P, f, G, "e4m3")
    K.fp8_cast(act_u, offs, poff, P, hist_a, "e4m3", *au, margin)
    hpre_f = torch.empty(P, F1, dtype=torch.bfloat16, device=DEV)
    af = _cast_buffers(P, f, G, "e4m3")
    K.fp8_gemm_cast(f"{act}_fwd", offs, poff, P, [xq] * G, "e4m3", w1q, "e4m3", f, h, f, sx, sw1, hist_a, "e4m3",
                    *af, cs=[hpre_f] * G, margin=margin)

    # backward: pre-activation gradient codes
    dh_u = torch.empty(P, F1, dtype=torch.bfloat16, device=DEV)
    K.fp8_gemm(False, f"{act}_bwd", offs, P, [dyq] * G, "e5m2", w2qt, "e4m3", f, h, 0, f, [dh_u] * G, sdy, sw2,
               auxs=[hp_in] * G)
    du = _cast_buffers(P, F1, G, "e5m2")
    K.fp8_cast(dh_u, offs, poff, P, hist_d, "e5m2", *du, margin)
    df = _cast_buffers(P, F1, G, "e5m2")
    K.fp8_gemm_cast(f"{act}_bwd", offs, poff, P, [dyq] * G, "e5m2", w2qt, "e4m3", f, h, f, sdy, sw2, hist_d, "e5m2",
                    *df, auxs=[hp_in] * G, margin=margin)
    # the same on the row-major fc2 codes held [h, f] (x_kn): the same codes, amax and scale
    w2q = [wt.t().contiguous() for wt in w2qt]
    dk = _cast_buffers(P, F1, G, "e5m2")
    K.fp8_gemm_cast(f"{act}_bwd", offs, poff, P, [dyq] * G, "e5m2", w2q, "e4m3", f, h, f, sdy, sw2, hist_d, "e5m2",
                    *dk, auxs=[hp_in] * G, margin=margin, x_kn=True)
    torch.cuda.synchronize()
    _same_bits(dk[2], df[2], "pre-activation gradient codes from [K, N] weights")
    _same_bits(dk[3], df[3], "transposed pre-activation gradient codes from [K, N] weights")
    assert dk[0].item() == df[0].item() and dk[1].item() == df[1].item()

    _same_bits(hpre_f, hpre_u, "pre-activations")
    for name, (ua, us, uq, uqt), (fa, fs, fq, fqt) in (("activation", au, af), ("pre-activation gradient", du, df)):
        _same_bits(fq, uq, f"{name} codes")
        _same_bits(fqt, uqt, f"{name} transposed codes")
        assert fa.item() == ua.item() and fa.item() != 0, f"{name} amax"
        assert fs.item() == us.item(), f"{name} 1/scale"
    if hist_scale < 0.1:   # the saturating case really saturates
        lim = torch.tensor([0x7e, 0xfe], dtype=torch.uint8)
        assert torch.isin(_codes(af[2]), lim).any(), "no saturated activation code"


def _q(x64, sinv, fmt):
    """Oracle cast (oracle/moe_ref.py quantize) with the scale whose inverse the GPU used, dequantised."""
    scale = float((torch.tensor(1.0) / torch.tensor(float(sinv), dtype=torch.float32)).item())
    return M.quantize(x64, scale, fmt) / torch.tensor(scale, dtype=torch.float32).double()


def _bf16(t):
    return t.to(torch.bfloat16).double()


EMU_CASES = [
    # (name, T, h, f, E, weight std)
    ("small", 256, 256, 256, 4, 0.05),
    ("mixtral-shape-64-tokens", 64, 4096, 14336, 8, 0.02),
]


@pytest.mark.parametrize("case", EMU_CASES, ids=[c[0] for c in EMU_CASES])
def test_fp8_layer_matches_quantized_emulation(case):
    """The whole fp8 expert path (casts, products, SwiGLU, combine, weight gradients) against a float64
    emulation that quantises the same tensors with the same scales and rounds the same intermediates to
    bf16: what is left is fp32 accumulation and output rounding."""
    from resihp_megatron_amd.fp8 import ACT, DH, DY, X, Fp8State
    from resihp_megatron_amd.layer import LayerMeta, moe_layer

    name, T, h, f, E, std = case
    k = 2
    x = seeded((T, h), 61, 1.0, torch.bfloat16).to(DEV).requires_grad_(True)
    router = seeded((E, h), 62, 0.05, torch.float32).to(DEV).requires_grad_(True)
    fc1 = [seeded((2 * f, h), 63 + e, std, torch.bfloat16).to(DEV).requires_grad_(True) for e in range(E)]
    fc2 = [seeded((h, f), 73 + e, std, torch.bfloat16).to(DEV).requires_grad_(True) for e in range(E)]
    dout = seeded((T, h), 64, 1.0, torch.bfloat16).to(DEV)
    meta = LayerMeta(num_experts=E, top_k=k, ffn=f, act="swiglu")
    st = Fp8State(E, 4, device=DEV)
    st.seed_history({X: 4.0, ACT: 0.5, DY: 0.5, DH: 0.05, **{st.w1(e): 0.2 for e in range(E)},
                     **{st.w2(e): 0.2 for e in range(E)}}, seed=8)
    say(f"fp8 layer vs quantised emulation: {name}")
    out, _ = moe_layer(meta, x, router, None, fc1, fc2, fp8=st)
    out.backward(dout)
    _, topi, gates = K.route(x.detach(), router.detach(), None, k, "softmax", True, 1.0)
    torch.cuda.synchronize()
    s = st.scale_inv.cpu().tolist()
    topi, gates = topi.cpu().long(), gates.cpu().double()
    x64, d64 = x.detach().cpu().double(), dout.cpu().double()
    out_ref = x64.clone()
    for e in range(E):
        rows, slots = (topi == e).nonzero(as_tuple=True)      # ascending tokens, as the dispatch orders them
        w1 = fc1[e].detach().cpu().double()
        w2 = fc2[e].detach().cpu().double()
        w1q, w2q = _q(w1, s[st.w1(e)], "e4m3"), _q(w2, s[st.w2(e)], "e4m3")
        xq = _q(x64[rows], s[X], "e4m3")
        hp = xq @ w1q.t()
        a = _bf16(torch.nn.functional.silu(hp[:, :f]) * hp[:, f:])
        aq = _q(a, s[ACT], "e4m3")
        y = _bf16(aq @ w2q.t())
        g = gates[rows, slots].unsqueeze(1)
        out_ref.index_add_(0, rows, g * y)
        dy = _bf16(g * d64[rows])
        dyq = _q(dy, s[DY], "e4m3".replace("4m3", "5m2"))
        dact = dyq @ w2q
        dh = _bf16(_swiglu_bwd(dact, _bf16(_swiglu_saved(hp, f)), f))
        dhq = _q(dh, s[DH], "e5m2")
        say(f"  expert {e}: rows {rows.numel()} dW2 {rel_err(fc2[e].grad, dyq.t() @ aq):.2e} "
            f"dW1 {rel_err(fc1[e].grad, dhq.t() @ xq):.2e}")
        assert rel_err(fc2[e].grad, dyq.t() @ aq) <= LAYER_BAR, f"fc2 weight gradient of expert {e}"
        assert rel_err(fc1[e].grad, dhq.t() @ xq) <= DW1_BAR, f"fc1 weight gradient of expert {e}"
    assert rel_err(out, out_ref) <= LAYER_BAR


def test_cast_many_equals_one_cast_per_tensor():
    """rhp_fp8_cast_many (the expert weights in one launch) gives every tensor the codes, amax and 1/scale
    of its own rhp_fp8_cast: tensors of different shapes, rows not a multiple of 128, an empty one."""
    shapes = [(512, 256), (256, 384), (130, 64), (0, 128), (1000, 192)]
    xs = [seeded(s, 90 + i, 0.3, torch.bfloat16).to(DEV) for i, s in enumerate(shapes)]
    hists = [_history(95 + i, scale=0.5).to(DEV) for i in range(len(shapes))]
    say(f"fp8 cast_many over {shapes}")
    fdt = K.FP8_FORMATS["e4m3"][1]
    amax_m = [torch.zeros(1, dtype=torch.int32, device=DEV) for _ in shapes]
    sinv_m = [torch.zeros(1, dtype=torch.float32, device=DEV) for _ in shapes]
    q_m = [torch.empty(s, dtype=fdt, device=DEV) for s in shapes]
    K.fp8_cast_many(xs, hists, "e4m3", amax_m, sinv_m, q_m)
    for i, (x, hst) in enumerate(zip(xs, hists)):
        if x.shape[0] == 0:   # no codes; the 1/scale is still written, the amax stays 0
            x = torch.zeros(1, x.shape[1], dtype=torch.bfloat16, device=DEV)
        rows = x.shape[0]
        off = torch.tensor([0, rows], dtype=torch.int32, device=DEV)
        poff = torch.tensor([0, (rows + 127) // 128 * 128], dtype=torch.int32, device=DEV)
        a = torch.zeros(1, dtype=torch.int32, device=DEV)
        si = torch.zeros(1, dtype=torch.float32, device=DEV)
        q = torch.empty(x.shape, dtype=fdt, device=DEV)
        K.fp8_cast(x, off, poff, rows, hst, "e4m3", a, si, q, None)
        torch.cuda.synchronize()
        if shapes[i][0]:
            _same_bits(q_m[i], q, f"codes of tensor {i}")
        assert amax_m[i].item() == a.item() and sinv_m[i].item() == si.item(), f"amax / scale of tensor {i}"


# (T, h, k, E, window): k <= 2 and k <= 8 variants, one or several 64-lane passes, slots of other devices.
ROW_CODE_CASES = [(300, 4096, 2, 8, (0, 8)), (97, 2048, 6, 16, (4, 12)), (64, 1024, 8, 8, (0, 8)),
                  (33, 192, 1, 4, (1, 3)), (0, 256, 2, 8, (0, 8)), (5, 256, 1, 64, (63, 64))]


@pytest.mark.parametrize("fmt", ["e4m3", "e5m2"])
@pytest.mark.parametrize("case", ROW_CODE_CASES, ids=lambda c: f"T{c[0]}-h{c[1]}-k{c[2]}-E{c[3]}")
def test_row_kernels_emit_the_codes_of_the_cast(case, fmt):
    """rhp_permute_fp8 / rhp_combine_bwd_fp8 equal rhp_permute / rhp_combine_bwd followed by rhp_fp8_cast of
    the bf16 rows they would store: codes, amax and 1/scale bit for bit; dgates too."""
    from oracle import route_c as R

    T, h, k, E, (e0, e1) = case
    g = torch.Generator().manual_seed(7)
    topi = torch.sort(torch.randn(max(T, 1), E, generator=g), dim=1, descending=True).indices[:T, :k]
    plan = R.dispatch(topi.to(torch.int32).numpy(), E, e0, e1, 1)
    P = int(plan["offsets"][-1])
    pair_row = torch.from_numpy(plan["pair_row"].astype("int32")).to(DEV)
    off = torch.from_numpy(plan["offsets"].astype("int32")).to(DEV)
    x = seeded((T, h), 21, 1.0, torch.bfloat16).to(DEV)
    dout = seeded((T, h), 22, 1.0, torch.bfloat16).to(DEV)
    y = seeded((P, h), 23, 1.0, torch.bfloat16).to(DEV)
    gates = seeded((T, k), 24, 0.5, torch.float32).abs().to(DEV)
    hist = _history(25, scale=2.0).to(DEV)
    say(f"fp8 row codes {fmt} T={T} h={h} k={k} E={E} window={(e0, e1)} P={P}")
    fdt = K.FP8_FORMATS[fmt][1]
    poff = K.fp8_padded_offsets(off)
    state = lambda: (torch.zeros(1, dtype=torch.int32, device=DEV),  # noqa: E731
                     torch.zeros(1, dtype=torch.float32, device=DEV))

    a1, s1 = state()
    q1 = K.permute_fp8(x, pair_row, k, P, hist, fmt, a1, s1)
    a2, s2 = state()
    q2 = torch.empty(P, h, dtype=fdt, device=DEV)
    xp = K.permute(x, pair_row, k, P)
    if P:
        K.fp8_cast(xp, off, poff, P, hist, fmt, a2, s2, q2, None)
    torch.cuda.synchronize()
    _same_bits(q1, q2, "permute codes")
    assert a1.item() == a2.item(), "permute amax"
    if P:
        assert s1.item() == s2.item(), "permute 1/scale"

    a1, s1 = state()
    q1, dg1 = K.combine_bwd_fp8(dout, y, gates, pair_row, P, hist, fmt, a1, s1)
    a2, s2 = state()
    dy, dg2 = K.combine_bwd(dout, y, gates, pair_row, P)
    if P:
        K.fp8_cast(dy, off, poff, P, hist, fmt, a2, s2, q2, None)
    torch.cuda.synchronize()
    _same_bits(q1, q2, "combine backward codes")
    assert torch.equal(dg1, dg2), "dgates"
    assert a1.item() == a2.item(), "combine backward amax"
    if P:
        assert s1.item() == s2.item(), "combine backward 1/scale"
