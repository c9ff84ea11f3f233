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

from _helpers import DEV, TOL, rel_err, say, seeded, zipf_prior
from oracle import moe_ref as M
from oracle import route_c as R
from resihp_megatron_amd import kernels as K
from resihp_megatron_amd import moe, placement
from resihp_megatron_amd.layer import LayerMeta, moe_layer

pytestmark = pytest.mark.gpu

GOLD = np.load(pathlib.Path(__file__).resolve().parent / "golden" / "reference_moe.npz")


def _run(name, cfg: moe.MoEConfig, window=None, n_src=1, bias=None, check_route=False):
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
    out, counts = moe_layer(meta, x, params["router.weight"], bias_d, fc1s, fc2s, s1, s2)
    dout = seeded(out.shape, 77, 1.0, out.dtype).to(DEV)
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
