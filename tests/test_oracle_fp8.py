"""Pins of the oracle's fp8 layer emulation (oracle/moe_ref.py fp8_layer_emulation) and the floor of
the fp8 recipe against float64.

The emulation must be the float64 layer itself once every cast and rounding is switched off (a
dropped term, a transposed operand or a wrong gate derivative breaks equality at 1e-12); with only
the bf16 roundings of the stored intermediates it stays within bf16 precision; with the fp8 casts on
it measures the recipe's floor: e4m3 keeps 3 mantissa bits, e5m2 2, so exact quantisation of these
tensors alone moves the weight gradients further than the 6e-2 a bfloat16-style bar would allow.
"""

from __future__ import annotations

import pytest
import torch

from oracle import moe_ref as M


def _case(T, h, f, E, k, std, act, seed=0):
    g = torch.Generator().manual_seed(seed)
    F1 = 2 * f if act == "swiglu" else f
    x = torch.randn(T, h, generator=g).to(torch.bfloat16).double()
    router = (torch.randn(E, h, generator=g) * 0.05).float().double()
    fc1 = [(torch.randn(F1, h, generator=g) * std).to(torch.bfloat16).double() for _ in range(E)]
    fc2 = [(torch.randn(h, f, generator=g) * std).to(torch.bfloat16).double() for _ in range(E)]
    dout = torch.randn(T, h, generator=g).to(torch.bfloat16).double()
    cfg = M.OracleConfig(hidden=h, ffn=f, num_experts=E, top_k=k, tokens=T, act=act)
    topi, _ = M.route(cfg, x, router)
    return cfg, x, router, fc1, fc2, dout, topi


def _reference(cfg, x, router, fc1, fc2, dout, topi):
    params = {"router.weight": router.clone().requires_grad_(True)}
    for e in range(cfg.num_experts):
        params[f"experts.{e}.fc1.weight"] = fc1[e].clone().requires_grad_(True)
        params[f"experts.{e}.fc2.weight"] = fc2[e].clone().requires_grad_(True)
    xr = x.clone().requires_grad_(True)
    out = M.layer_forward(cfg, params, xr, topi=topi)
    out.backward(dout)
    grad = lambda k: params[k].grad if params[k].grad is not None else torch.zeros_like(params[k])  # noqa: E731
    return {"out": out.detach(), "dx": xr.grad, "router": grad("router.weight"),
            "fc1": [grad(f"experts.{e}.fc1.weight") for e in range(cfg.num_experts)],
            "fc2": [grad(f"experts.{e}.fc2.weight") for e in range(cfg.num_experts)]}


def _rel(a, b):
    return float((a - b).abs().max() / b.abs().max())


def _errors(emu, ref):
    out = {n: _rel(emu[n], ref[n]) for n in ("out", "dx", "router")}
    for n in ("fc1", "fc2"):
        out[n] = max(_rel(a, b) for a, b in zip(emu[n], ref[n]) if b.abs().max() > 0)
    return out


ONE = lambda E: {"x": 1.0, "act": 1.0, "dy": 1.0, "dh": 1.0, "w1": [1.0] * E, "w2": [1.0] * E}  # noqa: E731


@pytest.mark.parametrize("act", ["swiglu", "gelu"])
def test_emulation_without_casts_is_the_float64_layer(act):
    cfg, x, router, fc1, fc2, dout, topi = _case(40, 24, 16, 6, 2, 0.3, act)
    ref = _reference(cfg, x, router, fc1, fc2, dout, topi)
    emu = M.fp8_layer_emulation(x, router, fc1, fc2, topi, dout, ONE(6), quantize_on=False, round_bf16=False, act=act)
    errs = _errors(emu, ref)
    assert max(errs.values()) <= 1e-12, errs


def test_emulation_with_bf16_roundings_only():
    cfg, x, router, fc1, fc2, dout, topi = _case(64, 64, 32, 4, 2, 0.2, "swiglu")
    ref = _reference(cfg, x, router, fc1, fc2, dout, topi)
    emu = M.fp8_layer_emulation(x, router, fc1, fc2, topi, dout, ONE(4), quantize_on=False)
    errs = _errors(emu, ref)
    assert 0 < max(errs.values()) <= 2e-2, errs


def calibrated_scales(x, router, fc1, fc2, topi, dout, seed=5, spread=0.25, act="swiglu"):
    """Delayed scales as one calibration iteration seeds them: every tensor's amax, spread by +-25 %
    over a 16-entry history (the layer tests' Fp8State.seed_history), scale = fp8_max / max(history)."""
    E = len(fc1)
    am = {}
    M.fp8_layer_emulation(x, router, fc1, fc2, topi, dout, ONE(E), quantize_on=False, amax=am, act=act)
    g = torch.Generator().manual_seed(seed)

    def sc(a, fmt):
        u = torch.rand(16, generator=g, dtype=torch.float64) * 2 - 1
        return M.fp8_scale((a * (1 + spread * u)).float(), fmt)

    return {"x": sc(am["x"], "e4m3"), "act": sc(am["act"], "e4m3"), "dy": sc(am["dy"], "e5m2"),
            "dh": sc(am["dh"], "e5m2"), "w1": [sc(am[("w1", e)], "e4m3") for e in range(E)],
            "w2": [sc(am[("w2", e)], "e4m3") for e in range(E)]}


def test_fp8_recipe_floor():
    """The floor of exact e4m3 / e5m2 quantisation at 128 rows per expert (512 tokens, top-2, 8 experts):
    the weight gradients (max-relative) land 8e-2 to 2e-1 from float64, beyond a 6e-2 bar; the output's
    expert part (out - x) about 7e-2; the router gradient about 5e-2."""
    cfg, x, router, fc1, fc2, dout, topi = _case(512, 512, 1024, 8, 2, 0.02, "swiglu")
    ref = _reference(cfg, x, router, fc1, fc2, dout, topi)
    scales = calibrated_scales(x, router, fc1, fc2, topi, dout)
    emu = M.fp8_layer_emulation(x, router, fc1, fc2, topi, dout, scales)
    errs = _errors(emu, ref)
    expert_part = _rel(emu["out"] - x, ref["out"] - x)
    assert 0.08 <= errs["fc1"] <= 0.2 and 0.08 <= errs["fc2"] <= 0.2, errs
    assert 0.03 <= expert_part <= 0.12, expert_part
    assert 0.02 <= errs["router"] <= 0.1, errs
    # casts that round to nearest are unbiased: no tensor moves past 2e-1
    assert max(errs.values()) <= 0.2, errs
