"""Host-side logic of the drop-in API, checked on the CPU against the oracle and the reference's
own known answers (tests/unit/test_expert_placement.py, resihp/runtime/moe.py defaults)."""

from __future__ import annotations

import pytest
import torch

from oracle import moe_ref as M
from resihp_megatron_amd import moe, placement, rng
from resihp_megatron_amd.layer import LayerMeta, moe_layer


def test_config_defaults_match_reference():
    cfg = moe.MoEConfig()
    # resihp/runtime/moe.py:29-37
    assert (cfg.hidden, cfg.ffn, cfg.num_experts, cfg.top_k, cfg.tokens, cfg.seed) == (8, 12, 6, 2, 48, 4321)
    assert cfg.dtype == torch.float64 and cfg.bias_update_rate == 0.0
    assert (cfg.act, cfg.score, cfg.num_shared) == ("gelu", "softmax", 0)


@pytest.mark.parametrize("kw", [dict(), dict(bias_update_rate=0.01),
                                dict(act="swiglu", num_shared=2, shared_ffn=16, ffn=24, expert_bias=True,
                                     bias_init_std=0.1, init_std=0.02, dtype=torch.bfloat16, score="sigmoid")])
def test_specs_and_init_match_oracle(kw):
    cfg = moe.MoEConfig(device="cpu", **kw)
    ocfg = M.OracleConfig(**{k: v for k, v in kw.items()})
    specs = moe.moe_specs(cfg)
    shapes = M.param_shapes(ocfg)
    assert list(specs) == list(shapes)
    for k, s in specs.items():
        assert (s.global_shape, s.trainable) == shapes[k]
        assert s.dim is None
        assert torch.equal(moe.init_param(cfg, s), M.init_param(ocfg, k, *shapes[k]))
    x, y = moe.batch(cfg, 3)
    ox, oy = M.batch(ocfg, 3)
    assert torch.equal(x, ox) and torch.equal(y, oy)


def test_seeds_match_oracle():
    for parts in [(0,), (1, 2, 3), (4321, 7, 5), (2 ** 64 - 1,)]:
        assert rng.derive_seed(*parts) == M.derive_seed(*parts)


def test_expert_of_and_keys():
    assert moe.expert_of("experts.12.fc1.weight") == 12
    assert moe.expert_of("router.weight") is None and moe.expert_of("shared_experts.0.fc1.weight") is None


def test_even_split_known_answers():
    assert moe.even_split(10, 3) == [(0, 4), (4, 7), (7, 10)]
    assert moe.even_split(0, 2) == [(0, 0), (0, 0)]
    with pytest.raises(ValueError):
        moe.even_split(4, 0)


def test_smooth_weighted_round_robin_reference_known_answer():
    # tests/unit/test_expert_placement.py:51-54 of the reference
    split = placement.smooth_weighted_round_robin(["x", "y"], {"y": 0.5}, 30)
    assert split.count("x") == 20 and split.count("y") == 10
    assert placement.smooth_weighted_round_robin(["x", "y"], {"y": 0.5}, 30) == split
    assert placement.smooth_weighted_round_robin(["z"], {}, 3) == ["z", "z", "z"]


def test_placement_holdings_and_groups():
    p = placement.ExpertPlacement(4, (("a", "b"), ("c", "d")),
                                  {"a": (0, 1), "b": (2, 3), "c": (0, 2), "d": (1, 3)})
    p.validate()
    assert p.holders(0) == ["a", "c"] and p.group_holders(1, 3) == ["d"] and p.group_of("c") == 1
    cfg = moe.MoEConfig(num_experts=4, device="cpu")
    specs = moe.moe_specs(cfg)
    hold = moe.moe_holdings(p, specs)
    assert hold["router.weight"] == [(d, (0, 1)) for d in "abcd"]
    assert hold["experts.0.fc1.weight"] == [("a", (0, 1)), ("c", (0, 1))]
    names = [g.name for g in moe.moe_group_specs(p, ["a", "b", "c", "d"])]
    assert names[:3] == ["dp", "ep/0", "ep/1"] and "edp/a,c" in names
    assert moe.local_keys(p, "b", specs) == ["router.weight", "experts.2.fc1.weight", "experts.2.fc2.weight",
                                             "experts.3.fc1.weight", "experts.3.fc2.weight"]
    with pytest.raises(ValueError):
        placement.ExpertPlacement(2, (("a",),), {"a": (0,)}).validate()


def test_kernels_refuse_cpu_tensors():
    x = torch.zeros(4, 8)
    w = torch.zeros(2, 8)
    meta = LayerMeta(num_experts=2, top_k=1, ffn=8)
    with pytest.raises(RuntimeError, match="HIP device"):
        moe_layer(meta, x, w, None, [torch.zeros(8, 8)] * 2, [torch.zeros(8, 8)] * 2)
    with pytest.raises(RuntimeError, match="HIP device"):
        moe.route(moe.MoEConfig(top_k=1, device="cpu"), x, w)


class _Comms:
    def __init__(self, grouped):
        self.grouped = grouped

    def group(self, name):
        return object() if name in self.grouped else None


def test_ep_runtime_refuses_cross_gpu_groups():
    p = placement.single_device(4, "gpu0")
    rt = moe.EPRuntime(moe.MoEConfig(num_experts=4, device="cpu"), p, "gpu0", ["gpu0"], _Comms({"ep/0"}), None, {})
    with pytest.raises(NotImplementedError):
        rt.forward(torch.zeros(2, 8))
    assert rt.token_range() == (0, 48)


def test_adam_refuses_host_parameters():
    """The fused optimizer step runs on the GPU only: no silent CPU fallback."""
    opt = moe.Adam({"w": torch.nn.Parameter(torch.zeros(4))})
    with pytest.raises(RuntimeError, match="HIP device"):
        opt.step()
    assert opt.state_tensors().keys() == {"param/w", "exp_avg/w", "exp_avg_sq/w"}
