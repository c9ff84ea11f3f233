"""Live re-placement on one device: state rebuilt by key mid-training, training continues unchanged.

Mirrors tests/dist/test_moe_ep.py:55-91 of the reference on a single GPU: train 4 iterations through
EPRuntime, snapshot the parameters, the Adam moments (``state_tensors``, resihp/runtime/optim.py:48-54)
and ``router.expert_bias`` by key (the state contract of resihp/runtime/moe.py:122-146), build fresh
Parameters, a new Adam with ``load_state_tensors`` (optim.py:56-62) and a new EPRuntime, then train 4
more.  Losses and final parameters must equal the reference's own 8-iteration recording at rtol 1e-10
(the bar of its EP test, test_moe_ep.py:108-112).  The fp8 variant also migrates the delayed-scaling
histories by key and must continue bit for bit like a run without the rebuild.
"""

from __future__ import annotations

import pathlib

import numpy as np
import pytest
import torch

from _helpers import DEV, say
from resihp_megatron_amd import moe, placement
from resihp_megatron_amd.fp8 import Fp8State
from resihp_megatron_amd.layer import LayerMeta, moe_layer

pytestmark = pytest.mark.gpu

GOLD = np.load(pathlib.Path(__file__).resolve().parent / "golden" / "reference_moe.npz")
KINDS = ("param", "exp_avg", "exp_avg_sq")
BEFORE, AFTER = 4, 4


def _train(cfg, rt, opt, it):
    """test_moe_ep.py:24-34 on one device: the whole batch is this device's token range."""
    opt.zero_grad()
    x, y = moe.batch(cfg, it)
    s, e = rt.token_range()
    loss = moe.token_loss(rt.forward(x[s:e]), y[s:e])
    (loss / cfg.tokens).backward()
    rt.sync_grads()
    rt.finish_iteration()
    opt.step()
    return loss.item()


def _migrate(state: dict[str, dict[str, torch.Tensor]]) -> dict[str, dict[str, torch.Tensor]]:
    """What the transfer engine delivers on the new holder: every tensor by key, in fresh device memory."""
    return {kind: {k: v.detach().clone() for k, v in ts.items()} for kind, ts in state.items()}


@pytest.mark.parametrize("name,bias_rate", [("default", 0.0), ("bias", 0.01)])
def test_rebuild_by_key_continues_training(name, bias_rate):
    cfg = moe.MoEConfig(bias_update_rate=bias_rate, device=DEV)
    specs = moe.moe_specs(cfg)
    ids = ["gpu0"]
    p1 = placement.single_device(cfg.num_experts, ids[0])
    mine = moe.local_keys(p1, ids[0], specs)
    params = {k: torch.nn.Parameter(moe.init_param(cfg, specs[k])) for k in mine if specs[k].trainable}
    buffers = {k: moe.init_param(cfg, specs[k]) for k in mine if not specs[k].trainable}
    opt = moe.Adam(params, lr=1e-2)
    rt = moe.EPRuntime(cfg, p1, ids[0], ids, None, None, params, buffers=buffers)
    say(f"re-placement {name}: {BEFORE} iterations")
    losses = [_train(cfg, rt, opt, it) for it in range(BEFORE)]

    old_state = {"param": {**{k: p.data for k, p in params.items()}, **buffers},
                 "exp_avg": {k: opt.state[k]["exp_avg"] for k in params},
                 "exp_avg_sq": {k: opt.state[k]["exp_avg_sq"] for k in params}}
    got = _migrate(old_state)
    p2 = placement.single_device(cfg.num_experts, ids[0])
    keys = moe.local_keys(p2, ids[0], specs)
    trainable = [k for k in keys if specs[k].trainable]
    old_ptrs = {p.data_ptr() for p in params.values()}
    params = {k: torch.nn.Parameter(got["param"][k].clone()) for k in trainable}
    buffers = {k: got["param"][k].clone() for k in keys if not specs[k].trainable}
    assert not old_ptrs & {p.data_ptr() for p in params.values()}, "the rebuilt parameters are new tensors"
    step = opt.step_count
    opt = moe.Adam(params, lr=1e-2)
    opt.load_state_tensors({f"{kind}/{k}": got[kind][k] for kind in KINDS for k in trainable}, step)
    rt = moe.EPRuntime(cfg, p2, ids[0], ids, None, None, params, buffers=buffers)
    say(f"re-placement {name}: {AFTER} iterations after the rebuild")
    losses += [_train(cfg, rt, opt, it) for it in range(BEFORE, BEFORE + AFTER)]

    np.testing.assert_allclose(np.array(losses) / cfg.tokens, GOLD[f"{name}/train/losses"], rtol=1e-10)
    final = {**{k: v.detach() for k, v in params.items()}, **buffers}
    for k, v in final.items():
        torch.testing.assert_close(v.cpu(), torch.from_numpy(GOLD[f"{name}/train/final/{k}"]), rtol=1e-10, atol=1e-12)
    if bias_rate:
        assert final["router.expert_bias"].abs().sum() > 0


def _fp8_setup(seed=3):
    E, h, f, T, k = 8, 256, 256, 256, 2
    g = torch.Generator(device=DEV).manual_seed(seed)
    rnd = lambda *s, std=1.0, dt=torch.bfloat16: (torch.randn(*s, generator=g, device=DEV) * std).to(dt)  # noqa: E731
    params = {"router.weight": rnd(E, h, std=0.05, dt=torch.float32)}
    for e in range(E):
        params[f"experts.{e}.fc1.weight"] = rnd(2 * f, h, std=0.05)
        params[f"experts.{e}.fc2.weight"] = rnd(h, f, std=0.05)
    batches = [(rnd(T, h), rnd(T, h)) for _ in range(BEFORE + AFTER)]
    meta = LayerMeta(num_experts=E, top_k=k, ffn=f, act="swiglu")
    return E, params, batches, meta


def _fp8_iteration(meta, E, params, opt, st, batch):
    x, y = batch
    opt.zero_grad()
    fc1 = [params[f"experts.{e}.fc1.weight"] for e in range(E)]
    fc2 = [params[f"experts.{e}.fc2.weight"] for e in range(E)]
    out, _ = moe_layer(meta, x, params["router.weight"], None, fc1, fc2, fp8=st)
    loss = moe.token_loss(out.float(), y.float()) / x.shape[0]
    loss.backward()
    st.finish_iteration()
    opt.step()
    return loss.item()


def test_rebuild_by_key_with_fp8_state():
    """fp8 experts: parameters, Adam moments and the delayed-scaling histories migrate by key; the
    rebuilt run's losses, parameters and histories equal those of a run without the rebuild, bit for bit."""
    E, init, batches, meta = _fp8_setup()
    experts = list(range(E))

    def fresh():
        params = {k: torch.nn.Parameter(v.clone()) for k, v in init.items()}
        st = Fp8State(E, 16, device=DEV)
        st.seed_history({i: 1.0 for i in range(4 + 2 * E)}, seed=1)
        return params, moe.Adam(params, lr=1e-3), st

    say("fp8 re-placement: continuous run")
    params, opt, st = fresh()
    ref_losses = [_fp8_iteration(meta, E, params, opt, st, b) for b in batches]
    ref_params = {k: v.detach().clone() for k, v in params.items()}
    ref_hist = st.history.clone()

    say("fp8 re-placement: rebuilt after 4 iterations")
    params, opt, st = fresh()
    losses = [_fp8_iteration(meta, E, params, opt, st, b) for b in batches[:BEFORE]]
    got = _migrate({"param": {k: p.data for k, p in params.items()},
                    "exp_avg": {k: opt.state[k]["exp_avg"] for k in params},
                    "exp_avg_sq": {k: opt.state[k]["exp_avg_sq"] for k in params},
                    "fp8": st.state_tensors(experts)})
    assert got["fp8"]["experts.3.fc1.amax_history"].shape == (16,)
    step = opt.step_count
    params = {k: torch.nn.Parameter(got["param"][k].clone()) for k in init}
    opt = moe.Adam(params, lr=1e-3)
    opt.load_state_tensors({f"{kind}/{k}": got[kind][k] for kind in KINDS for k in params}, step)
    st = Fp8State(E, 16, device=DEV)
    st.load_state_tensors(got["fp8"], experts)
    losses += [_fp8_iteration(meta, E, params, opt, st, b) for b in batches[BEFORE:]]

    assert losses == ref_losses
    for k in init:
        assert torch.equal(params[k].detach(), ref_params[k]), k
    assert torch.equal(st.history, ref_hist)


def test_fp8_state_by_key_follows_the_expert_not_the_slot():
    """A holder whose slots hold the experts in another order receives each expert's histories in the
    slot that now holds it; a state missing a key raises and changes nothing."""
    st = Fp8State(3, 4, device=DEV)
    st.history.copy_(torch.arange(st.history.numel(), dtype=torch.float32, device=DEV).view_as(st.history))
    src = st.state_tensors([5, 9, 2])
    dst = Fp8State(3, 4, device=DEV)
    dst.load_state_tensors(src, [2, 5, 9])
    for g_dst, e in enumerate([2, 5, 9]):
        g_src = [5, 9, 2].index(e)
        assert torch.equal(dst.history[dst.w1(g_dst)], st.history[st.w1(g_src)])
        assert torch.equal(dst.history[dst.w2(g_dst)], st.history[st.w2(g_src)])
    assert torch.equal(dst.history[:4], st.history[:4])
    before = dst.history.clone()
    partial = {k: v for k, v in src.items() if not k.startswith("experts.9.")}
    with pytest.raises(KeyError):
        dst.load_state_tensors(partial, [2, 5, 9])
    assert torch.equal(dst.history, before)
    # nothing is converted by value: a pending amax given as float32 (the reference's pending_amax)
    # arrives as its bits, any other dtype mismatch raises and changes nothing
    as_float = dict(src)
    as_float["experts.5.fc1.amax"] = torch.tensor([3.7], dtype=torch.float32, device=DEV)
    dst.load_state_tensors(as_float, [2, 5, 9])
    assert dst.amax[dst.w1(1)].view(torch.float32).item() == pytest.approx(3.7, rel=1e-7)
    bad = dict(src)
    bad["fp8.expert_input.amax_history"] = src["fp8.expert_input.amax_history"].double()
    before_amax = dst.amax.clone()
    with pytest.raises(TypeError):
        dst.load_state_tensors(bad, [2, 5, 9])
    assert torch.equal(dst.amax, before_amax)
