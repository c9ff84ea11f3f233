"""The fused MoE layer (forward + backward) on the GPU against the float64 oracle, per benchmark configuration,
and the drop-in API against the reference's own recorded outputs.

Every layer case runs the GPU layer, takes its routing (bit-exact with the C
oracle, see test_gpu_route.py), and runs oracle/moe_ref.py in float64 on the
same cast inputs with that routing; the output, the input gradient and every
parameter gradient must be within the bar of the compute dtype (max abs error
over max abs reference value).  Token counts are reduced where the float64
oracle would take more than seconds; hidden, ffn, experts and top-k are the
configs' own.
"""

from __future__ import annotations

import pathlib

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from _helpers import DEV, TOL, frob_err, rel_err, say, seeded, zipf_prior
from oracle import moe_ref as M
from oracle import route_c as R
from resihp_megatron_amd import kernels as K
from resihp_megatron_amd import moe, placement
from resihp_megatron_amd.fp8 import ACT, DH, DY, X, Fp8State
from resihp_megatron_amd.layer import LayerMeta, moe_layer

pytestmark = pytest.mark.gpu

# fp8 experts (e4m3 forward, e5m2 gradients, per-tensor delayed scaling) against the unquantised float64
# layer.  The bar is max-relative 6e-2, except where exact quantisation alone already lands further away:
# the float64 emulation of the recipe (oracle.moe_ref.fp8_layer_emulation, with the scales the GPU used)
# measures that floor per tensor, and the GPU may then be 1.1 x the floor away (fp32 accumulation and the
# odd rounding flip on top of exact quantisation).  tests/test_oracle_fp8.py pins the emulation and the
# size of the floor: e4m3 keeps 3 mantissa bits, e5m2 2, and weight gradients land 8e-2 to 2e-1 away.
FP8_BAR = 6e-2
FP8_FLOOR_FACTOR = 1.1
GOLD = np.load(pathlib.Path(__file__).resolve().parent / "golden" / "reference_moe.npz")


def _calibrate(st, forward, dout, leaves, seed, iterations=2):
    """Delayed scaling from the reference's initial histories (all ones): each calibration iteration
    records every tensor's amax, which seeds the 16-step histories (values spread by +-25 %) of the next.
    The first iteration's scales come from the ones, so the activation and gradient amaxes it records
    are those of mis-scaled inputs; the second records the real ones, as training does after a step."""
    for _ in range(iterations):
        forward().backward(dout)
        st.finish_iteration()
        st.seed_history({i: float(a) for i, a in enumerate(st.history[:, 0].tolist())}, seed=seed)
        for t in leaves:
            t.grad = None


def _run(name, cfg: moe.MoEConfig, window=None, n_src=1, bias=None, check_route=False, fp8=False):
    E = cfg.num_experts
    e0, e1 = window or (0, E)
    specs = moe.moe_specs(cfg)
    keep = [k for k in specs if specs[k].trainable and (moe.expert_of(k) is None or e0 <= moe.expert_of(k) < e1)]
    params = {k: torch.nn.Parameter(moe.init_param(cfg, specs[k])) for k in keep}
    x, _ = moe.batch(cfg, 0)
    x = x.detach().requires_grad_(True)
    meta = LayerMeta(num_experts=E, top_k=cfg.top_k, ffn=cfg.ffn, act=cfg.act, score=cfg.score,
                     normalize=cfg.normalize, gate_scale=cfg.gate_scale, e0=e0, e1=e1, n_src=n_src,
                     num_shared=cfg.num_shared, shared_ffn=cfg.shared_ffn)
    fc1s = [params[f"experts.{e}.fc1.weight"] for e in range(e0, e1)]
    fc2s = [params[f"experts.{e}.fc2.weight"] for e in range(e0, e1)]
    s1 = [params[f"shared_experts.{s}.fc1.weight"] for s in range(cfg.num_shared)]
    s2 = [params[f"shared_experts.{s}.fc2.weight"] for s in range(cfg.num_shared)]
    bias_d = None if bias is None else bias.to(DEV, moe.router_dtype(cfg))
    say(f"layer {name}: T={cfg.tokens} h={cfg.hidden} f={cfg.ffn} E={E} k={cfg.top_k} window=[{e0},{e1})")
    dout = seeded((cfg.tokens, cfg.hidden), 77, 1.0, x.dtype).to(DEV)
    st = None
    if fp8:
        st = Fp8State(e1 - e0, 16, device=DEV)
        _calibrate(st, lambda: moe_layer(meta, x, params["router.weight"], bias_d, fc1s, fc2s, s1, s2, fp8=st)[0],
                   dout, (x, *params.values()), seed=5)
    out, counts = moe_layer(meta, x, params["router.weight"], bias_d, fc1s, fc2s, s1, s2, fp8=st)
    out.backward(dout)
    _, topi, _ = K.route(x.detach(), params["router.weight"].detach(), bias_d, cfg.top_k, cfg.score,
                         cfg.normalize, cfg.gate_scale)
    torch.cuda.synchronize()
    topi = topi.cpu()
    if check_route:
        xr = x.detach().cpu()
        kind = {torch.bfloat16: "bf16", torch.float32: "f32", torch.float64: "f64"}[x.dtype]
        xh = xr.view(torch.int16).numpy().view(np.uint16) if kind == "bf16" else xr.numpy()
        lg = R.router_logits(xh, params["router.weight"].detach().cpu().numpy(), kind)
        ref_topi, _ = R.topk(lg, cfg.top_k, None if bias is None else bias_d.cpu().numpy(), cfg.score)
        assert np.array_equal(topi.numpy(), ref_topi)
    plan = R.dispatch(topi.numpy(), E, e0, e1, n_src)
    assert np.array_equal(counts.cpu().numpy(), plan["counts"])

    ocfg = M.OracleConfig(hidden=cfg.hidden, ffn=cfg.ffn, num_experts=E, top_k=cfg.top_k, tokens=cfg.tokens,
                          act=cfg.act, score=cfg.score, normalize=cfg.normalize, gate_scale=cfg.gate_scale,
                          num_shared=cfg.num_shared, shared_ffn=cfg.shared_ffn)
    p64 = {k: v.detach().cpu().double().requires_grad_(True) for k, v in params.items()}
    x64 = x.detach().cpu().double().requires_grad_(True)
    ref = M.layer_forward(ocfg, p64, x64, topi=topi.long(), local=(e0, e1))
    ref.backward(dout.cpu().double())
    if fp8:
        _check_fp8_against_floor(cfg, st, params, x, out, dout, topi, ref, x64, p64, (e0, e1))
        return plan
    tol = TOL[cfg.dtype]
    errs = {"out": rel_err(out, ref), "dx": rel_err(x.grad, x64.grad)}
    for k in params:
        # An expert that received no token has no autograd gradient in the oracle; the GPU writes zeros.
        ref_g = p64[k].grad if p64[k].grad is not None else torch.zeros_like(p64[k])
        errs[k] = rel_err(params[k].grad, ref_g)
    worst = max(errs, key=errs.get)
    say(f"  worst {worst}: {errs[worst]:.3e} (bar {tol})")
    assert errs[worst] <= tol, errs
    return plan


def _fp8_scales(st, G):
    """The scales (fp8_max / max(history)) the GPU used: 1 / scale_inv, as float32."""
    inv = st.scale_inv.cpu()
    sc = lambda i: float(torch.tensor(1.0) / inv[i])  # noqa: E731
    return {"x": sc(X), "act": sc(ACT), "dy": sc(DY), "dh": sc(DH), "w1": [sc(st.w1(g)) for g in range(G)],
            "w2": [sc(st.w2(g)) for g in range(G)]}


def _check_fp8_against_floor(cfg, st, params, x, out, dout, topi, ref, x64, p64, window):
    """Every tensor of the fp8 layer against float64: within 6e-2, or 1.1 x the recipe's own floor."""
    e0, e1 = window
    assert (e0, e1) == (0, cfg.num_experts), "fp8 floor check: full window"
    E = cfg.num_experts
    fc1 = [params[f"experts.{e}.fc1.weight"].detach().cpu().double() for e in range(E)]
    fc2 = [params[f"experts.{e}.fc2.weight"].detach().cpu().double() for e in range(E)]
    emu = M.fp8_layer_emulation(x.detach().cpu().double(), params["router.weight"].detach().cpu().double(), fc1, fc2,
                                topi.long(), dout.cpu().double(), _fp8_scales(st, E), act=cfg.act)
    zero = lambda k: torch.zeros_like(p64[k])  # noqa: E731
    g64 = lambda k: p64[k].grad if p64[k].grad is not None else zero(k)  # noqa: E731
    rows = [("out", out, emu["out"], ref), ("dx", x.grad, emu["dx"], x64.grad),
            ("router", params["router.weight"].grad, emu["router"], g64("router.weight"))]
    for e in range(E):
        for n, em in (("fc1", emu["fc1"][e]), ("fc2", emu["fc2"][e])):
            k = f"experts.{e}.{n}.weight"
            rows.append((k, params[k].grad, em, g64(k)))
    bad = []
    for name, got, em, r in rows:
        # max-relative (the bar) and norm-wise ||a - b|| / ||b|| (how far the bulk of the tensor is), for
        # the GPU and for exact quantisation (the recipe's floor); both held to 6e-2 or 1.1 x the floor
        floor, err = rel_err(em, r), rel_err(got, r)
        nfloor, nerr = frob_err(em, r), frob_err(got, r)
        bar, nbar = max(FP8_BAR, FP8_FLOOR_FACTOR * floor), max(FP8_BAR, FP8_FLOOR_FACTOR * nfloor)
        say(f"  {name}: max-rel gpu {err:.3e} floor {floor:.3e} bar {bar:.3e} | norm-wise gpu {nerr:.3e} "
            f"floor {nfloor:.3e}")
        if err > bar or nerr > nbar:
            bad.append((name, err, floor, nerr, nfloor))
    assert not bad, bad


def test_config1_tiny_fp64():
    _run("c1-fp64", moe.MoEConfig(hidden=64, ffn=128, num_experts=8, top_k=2, tokens=512, act="swiglu",
                                  dtype=torch.float64, device=DEV), check_route=True)


def test_config1_tiny_fp32():
    _run("c1-fp32", moe.MoEConfig(hidden=64, ffn=128, num_experts=8, top_k=2, tokens=512, act="swiglu",
                                  dtype=torch.float32, device=DEV), check_route=True)


def test_config2_mixtral_shape():
    _run("c2-mixtral", moe.MoEConfig(hidden=4096, ffn=14336, num_experts=8, top_k=2, tokens=64, act="swiglu",
                                     dtype=torch.bfloat16, init_std=0.02, device=DEV), check_route=True)


def test_config3_fine_grained_shared_sigmoid_bias():
    bias = seeded((64,), 33, 0.1, torch.float32)
    _run("c3-dsv2lite", moe.MoEConfig(hidden=2048, ffn=1408, num_experts=64, top_k=6, tokens=512, act="swiglu",
                                      score="sigmoid", num_shared=2, shared_ffn=1408, dtype=torch.bfloat16,
                                      init_std=0.02, device=DEV), bias=bias, check_route=True)


@pytest.mark.parametrize("window", [(0, 16), (112, 128)], ids=["hot-share", "tail-share"])
def test_config4_ep_share_zipf(window):
    cfg = moe.MoEConfig(hidden=2048, ffn=768, num_experts=128, top_k=8, tokens=2048, act="swiglu",
                        dtype=torch.bfloat16, init_std=0.02, device=DEV)
    plan = _run(f"c4-ep-{window}", cfg, window=window, n_src=8, bias=zipf_prior(128).float(), check_route=True)
    assert plan["src_counts"].shape == (8, 16)
    if window[0] == 112:
        assert (plan["counts"][112:128] == 0).any(), "the Zipf tail share should hold empty experts"


def test_config5_fp8_mixtral_shape():
    """Config 5's layer shape at 512 tokens (about 128 rows, half a row tile, per expert)."""
    _run("c5-fp8-mixtral", moe.MoEConfig(hidden=4096, ffn=14336, num_experts=8, top_k=2, tokens=512, act="swiglu",
                                         dtype=torch.bfloat16, init_std=0.02, device=DEV), fp8=True)


def test_config5_fp8_gelu_ragged():
    _run("c5-fp8-gelu", moe.MoEConfig(hidden=256, ffn=384, num_experts=8, top_k=2, tokens=300, act="gelu",
                                      dtype=torch.bfloat16, init_std=0.05, device=DEV), fp8=True)


def _q64(v, scale, fmt):
    """The oracle cast of v with the given scale, dequantised (float64)."""
    return M.quantize(v, scale, fmt) / torch.tensor(scale, dtype=torch.float32).double()


def _sampled_expert_grads(xr, g, dout, w1, w2, cols, outs, scales=None, e=0):
    """Sampled elements of one SwiGLU expert's weight gradients, each a sum over all of the expert's rows:
    dW2[outs, cols], and dW1 rows cols (gate) and f + cols (up) at columns outs.  xr: the expert's input
    rows, g: their gates, dout: their tokens' output gradients (float64).  With ``scales`` the same
    elements under the fp8 recipe (every tensor cast with its scale, stored intermediates rounded to
    bf16), exactly as oracle.moe_ref.fp8_layer_emulation computes them."""
    f, n = w2.shape[1], len(cols)
    fp8 = scales is not None
    q = (lambda v, key, fmt: _q64(v, key, fmt)) if fp8 else (lambda v, key, fmt: v)  # noqa: E731
    bf = (lambda v: v.to(torch.bfloat16).double()) if fp8 else (lambda v: v)  # noqa: E731
    s = scales or {"x": 1, "act": 1, "dy": 1, "dh": 1, "w1": [1] * (e + 1), "w2": [1] * (e + 1)}
    xq = q(xr, s["x"], "e4m3")
    hp = xq @ q(torch.cat([w1[cols], w1[f + cols]]), s["w1"][e], "e4m3").t()
    gt, up = hp[:, :n], hp[:, n:]
    aq = q(bf(F.silu(gt) * up), s["act"], "e4m3")
    dyq = q(bf(g * dout), s["dy"], "e5m2")
    dact = dyq @ q(w2[:, cols], s["w2"][e], "e4m3")
    sg = torch.sigmoid(gt)   # the forward's saved factors [up silu'(gate) | silu(gate)], stored in bf16
    dg = q(bf(dact * bf(up * sg * (1 + gt * (1 - sg)))), s["dh"], "e5m2")
    du = q(bf(dact * bf(gt * sg)), s["dh"], "e5m2")
    return dyq[:, outs].t() @ aq, dg.t() @ xq[:, outs], du.t() @ xq[:, outs]


def _full_size_layer(name, T, h, f, E, k, score="softmax", S=0, bias=None, fp8=False, seed=9):
    """The GPU layer at a configuration's full size, then float64 on samples whose value depends only on
    the GPU's routing: out and dx of 256 sampled tokens (exact per token given the selection), and 16 x 16
    sampled elements of every expert's two weight gradients (each a sum over all of its rows).  bf16: within
    2e-2; fp8: within 6e-2 or 1.1 x the recipe's floor on the same samples."""
    g = torch.Generator(device=DEV).manual_seed(seed)
    rnd = lambda *sh, std=1.0, dt=torch.bfloat16: (torch.randn(*sh, generator=g, device=DEV) * std).to(dt)  # noqa: E731
    x = rnd(T, h).requires_grad_(True)
    router = rnd(E, h, std=0.02, dt=torch.float32).requires_grad_(True)
    fc1 = [rnd(2 * f, h, std=0.02).requires_grad_(True) for _ in range(E)]
    fc2 = [rnd(h, f, std=0.02).requires_grad_(True) for _ in range(E)]
    s1 = [rnd(2 * f, h, std=0.02).requires_grad_(True) for _ in range(S)]
    s2 = [rnd(h, f, std=0.02).requires_grad_(True) for _ in range(S)]
    dout = rnd(T, h)
    meta = LayerMeta(num_experts=E, top_k=k, ffn=f, act="swiglu", score=score, num_shared=S, shared_ffn=f if S else 0)
    st = None
    if fp8:
        st = Fp8State(E, 16, device=DEV)
        say(f"layer {name} full size: fp8 calibration iterations")
        _calibrate(st, lambda: moe_layer(meta, x, router, bias, fc1, fc2, fp8=st)[0], dout, (x, router, *fc1, *fc2),
                   seed=6)
    say(f"layer {name} full size: T={T} h={h} f={f} E={E} k={k} shared={S} fp8={fp8}")
    out, _ = moe_layer(meta, x, router, bias, fc1, fc2, s1, s2, fp8=st)
    out.backward(dout)
    _, topi, gates = K.route(x.detach(), router.detach(), bias, k, score)
    torch.cuda.synchronize()
    topi = topi.cpu().long()
    c64 = lambda t: t.detach().cpu().double()  # noqa: E731
    scales = _fp8_scales(st, E) if fp8 else None
    ocfg = M.OracleConfig(hidden=h, ffn=f, num_experts=E, top_k=k, tokens=256, act="swiglu", score=score,
                          num_shared=S, shared_ffn=f if S else 0)
    rng = np.random.default_rng(seed)
    tok = torch.from_numpy(np.sort(rng.choice(T, 256, replace=False)))
    W1, W2 = [c64(w) for w in fc1], [c64(w) for w in fc2]
    R64 = c64(router)
    p64 = {"router.weight": R64, **{f"experts.{e}.fc1.weight": W1[e] for e in range(E)},
           **{f"experts.{e}.fc2.weight": W2[e] for e in range(E)},
           **{f"shared_experts.{i}.fc1.weight": c64(w) for i, w in enumerate(s1)},
           **{f"shared_experts.{i}.fc2.weight": c64(w) for i, w in enumerate(s2)}}
    xs = c64(x[tok.to(DEV)]).requires_grad_(True)
    ds = c64(dout[tok.to(DEV)])
    ref = M.layer_forward(ocfg, p64, xs, topi=topi[tok])
    ref.backward(ds)
    got_out, got_dx = c64(out[tok.to(DEV)]), c64(x.grad[tok.to(DEV)])
    errs = [("out", rel_err(got_out, ref.detach()), None), ("dx", rel_err(got_dx, xs.grad), None)]
    if fp8:
        emu = M.fp8_layer_emulation(xs.detach(), R64, W1, W2, topi[tok], ds, scales)
        errs = [("out", errs[0][1], rel_err(emu["out"], ref.detach())), ("dx", errs[1][1], rel_err(emu["dx"], xs.grad))]
    # weight gradients: sampled elements per expert, over all of the expert's rows
    gates64 = M.gates_from_logits(ocfg, c64(x) @ R64.t(), topi)   # float64 gates of every token
    x64, d64 = c64(x), c64(dout)
    cols = torch.from_numpy(np.sort(rng.choice(f, 16, replace=False)))
    outs = torch.from_numpy(np.sort(rng.choice(h, 16, replace=False)))
    for e in range(E):
        rows, slots = (topi == e).nonzero(as_tuple=True)
        if rows.numel() == 0:
            continue
        xr, ge, de = x64[rows], gates64[rows, slots].unsqueeze(1), d64[rows]
        ref_w = _sampled_expert_grads(xr, ge, de, W1[e], W2[e], cols, outs)
        gw1, gw2 = c64(fc1[e].grad), c64(fc2[e].grad)
        got_w = (gw2[outs][:, cols], gw1[cols][:, outs], gw1[f + cols][:, outs])
        emu_w = _sampled_expert_grads(xr, ge, de, W1[e], W2[e], cols, outs, scales, e) if fp8 else (None,) * 3
        for nm, a, b, c in zip(("dW2", "dW1 gate", "dW1 up"), got_w, ref_w, emu_w):
            errs.append((f"expert {e} {nm}", rel_err(a, b), None if c is None else rel_err(c, b)))
    for i in range(S):   # shared experts: every token, gate 1
        ref_w = _sampled_expert_grads(x64, torch.ones(T, 1, dtype=torch.float64), d64, p64[f"shared_experts.{i}.fc1.weight"],
                                      p64[f"shared_experts.{i}.fc2.weight"], cols, outs)
        gw1, gw2 = c64(s1[i].grad), c64(s2[i].grad)
        for nm, a, b in zip(("dW2", "dW1 gate", "dW1 up"), (gw2[outs][:, cols], gw1[cols][:, outs],
                                                           gw1[f + cols][:, outs]), ref_w):
            errs.append((f"shared {i} {nm}", rel_err(a, b), None))
    bad = []
    for nm, err, floor in errs:
        bar = TOL[torch.bfloat16] if not fp8 else max(FP8_BAR, FP8_FLOOR_FACTOR * floor)
        if err > bar:
            bad.append((nm, err, floor))
    worst = max(errs, key=lambda r: r[1])
    say(f"  worst {worst[0]}: {worst[1]:.3e}" + (f" (floor {worst[2]:.3e})" if worst[2] is not None else ""))
    assert not bad, bad


def test_config2_mixtral_full_size():
    """Config 2 at its benchmarked size: 8192 tokens, Mixtral layer shape, bf16."""
    _full_size_layer("c2-mixtral", 8192, 4096, 14336, 8, 2)


def test_config3_fine_grained_full_size():
    """Config 3 at its benchmarked size: 16384 tokens, 64 routed + 2 shared experts, top-6 sigmoid + bias."""
    bias = seeded((64,), 33, 0.1, torch.float32).to(DEV)
    _full_size_layer("c3-dsv2lite", 16384, 2048, 1408, 64, 6, score="sigmoid", S=2, bias=bias)


def test_config5_fp8_full_size():
    """Config 5 at its full size: 16384 tokens, Mixtral shape, fp8 experts after two calibration iterations."""
    _full_size_layer("c5-fp8", 16384, 4096, 14336, 8, 2, fp8=True)


def test_reference_default_gelu_fp64():
    _run("reference-default", moe.MoEConfig(device=DEV), check_route=True)


# ----------------------------------------------------------------------------- drop-in API


@pytest.mark.parametrize("name,kw", [("default", {}), ("bias", {"bias_update_rate": 0.01}),
                                     ("wide", dict(hidden=16, ffn=32, num_experts=8, top_k=3, tokens=64, seed=77,
                                                   bias_update_rate=0.05))])
def test_reference_train_matches_reference_recording(name, kw):
    """reference_train on the GPU reproduces the reference's own 8-step float64 run (rel 1e-10,
    the bar the reference sets for its EP-vs-single-process test, tests/dist/test_moe_ep.py:108-112)."""
    cfg = moe.MoEConfig(device=DEV, **kw)
    say(f"reference_train {name}")
    losses, final = moe.reference_train(cfg, 8)
    np.testing.assert_allclose(losses, GOLD[f"{name}/train/losses"], rtol=1e-10)
    for k, v in final.items():
        torch.testing.assert_close(v.cpu(), torch.from_numpy(GOLD[f"{name}/train/final/{k}"]), rtol=1e-10,
                                   atol=1e-12)


def test_reference_forward_and_route_match_reference_recording():
    cfg = moe.MoEConfig(device=DEV, bias_update_rate=0.01)
    specs = moe.moe_specs(cfg)
    params = {k: moe.init_param(cfg, s) for k, s in specs.items()}
    x, y = moe.batch(cfg, 0)
    say("reference_forward bias")
    topi, gates = moe.route(cfg, x, params["router.weight"], params["router.expert_bias"])
    assert torch.equal(topi.cpu(), torch.from_numpy(GOLD["bias/route/topi"]))
    torch.testing.assert_close(gates.cpu(), torch.from_numpy(GOLD["bias/route/gates"]), rtol=1e-13, atol=1e-15)
    leaves = {k: torch.nn.Parameter(v) for k, v in params.items() if specs[k].trainable}
    xl = x.clone().requires_grad_(True)
    out = moe.reference_forward(cfg, {**leaves, "router.expert_bias": params["router.expert_bias"]}, xl)
    (moe.token_loss(out, y) / cfg.tokens).backward()
    torch.testing.assert_close(out.detach().cpu(), torch.from_numpy(GOLD["bias/fwd/out"]), rtol=1e-12, atol=1e-13)
    torch.testing.assert_close(xl.grad.cpu(), torch.from_numpy(GOLD["bias/fwd/grad/x"]), rtol=1e-10, atol=1e-13)
    for k, p in leaves.items():
        torch.testing.assert_close(p.grad.cpu(), torch.from_numpy(GOLD[f"bias/fwd/grad/{k}"]), rtol=1e-10,
                                   atol=1e-13)
    assert torch.equal(params["router.expert_bias"].cpu(), torch.from_numpy(GOLD["bias/fwd/after/router.expert_bias"]))


def test_expert_ffn_single_expert_autograd():
    g = torch.Generator().manual_seed(4)
    x = torch.randn(37, 8, generator=g, dtype=torch.float64)
    fc1 = torch.randn(12, 8, generator=g, dtype=torch.float64)
    fc2 = torch.randn(8, 12, generator=g, dtype=torch.float64)
    xd, f1, f2 = (t.to(DEV).requires_grad_(True) for t in (x, fc1, fc2))
    say("expert_ffn")
    y = moe.expert_ffn(xd, f1, f2)
    y.sum().backward()
    xr, f1r, f2r = (t.clone().requires_grad_(True) for t in (x, fc1, fc2))
    yr = M.expert_ffn(xr, f1r, f2r)
    yr.sum().backward()
    assert rel_err(y, yr) <= 1e-12
    for a, b in ((xd, xr), (f1, f1r), (f2, f2r)):
        assert rel_err(a.grad, b.grad) <= 1e-12


def test_ep_runtime_single_device_matches_reference_forward():
    cfg = moe.MoEConfig(device=DEV, bias_update_rate=0.01)
    specs = moe.moe_specs(cfg)
    params = {k: torch.nn.Parameter(moe.init_param(cfg, s)) for k, s in specs.items() if s.trainable}
    buffers = {k: moe.init_param(cfg, s) for k, s in specs.items() if not s.trainable}
    p = placement.single_device(cfg.num_experts, "gpu0")
    rt = moe.EPRuntime(cfg, p, "gpu0", ["gpu0"], None, None, params, buffers=buffers)
    x, y = moe.batch(cfg, 0)
    say("EPRuntime single device")
    out = rt.forward(x)
    (moe.token_loss(out, y) / cfg.tokens).backward()
    torch.testing.assert_close(out.detach().cpu(), torch.from_numpy(GOLD["bias/fwd/out"]), rtol=1e-12, atol=1e-13)
    assert rt.tokens_per_expert.sum().item() == cfg.tokens * cfg.top_k
    before = buffers["router.expert_bias"].clone()
    rt.finish_iteration()   # the bias moves only here, after the iteration (moe.py:236-240)
    assert torch.equal(buffers["router.expert_bias"].cpu(), torch.from_numpy(GOLD["bias/fwd/after/router.expert_bias"]))
    assert not torch.equal(before, buffers["router.expert_bias"])


def test_layer_error_leaves_bias_untouched():
    """A failing call raises RuntimeError (recoverable in the reference's trainer) and no bias moved."""
    cfg = moe.MoEConfig(device=DEV, bias_update_rate=0.01)
    specs = moe.moe_specs(cfg)
    params = {k: moe.init_param(cfg, s) for k, s in specs.items()}
    params["experts.3.fc1.weight"] = params["experts.3.fc1.weight"].float()   # wrong dtype for one expert
    before = params["router.expert_bias"].clone()
    x, _ = moe.batch(cfg, 0)
    say("layer error path")
    with pytest.raises(RuntimeError):
        moe.reference_forward(cfg, params, x)
    assert torch.equal(before, params["router.expert_bias"])
