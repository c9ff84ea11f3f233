"""Drop-in MoE block API on gfx950: the names and behaviour of resihp/runtime/moe.py.

Same functions, arguments and state keys as the reference module
(resihp/runtime/moe.py:28-269); the arithmetic runs in the HIP kernels of
``libresihp_moe.so`` on the GPU instead of torch CPU ops.  Differences, all
deliberate:

* ``MoEConfig`` gains fields for the extensions (SwiGLU experts, sigmoid
  scoring, shared experts, a seeded initial expert bias, Gaussian weight init
  with a fixed std, a separate router dtype, the device).  Defaults reproduce
  the reference configuration.
* Top-k ties go to the lowest expert id (the reference inherits torch.topk's
  unspecified order), and NaN router keys rank last.
* Cross-GPU expert parallelism is out of scope: ``EPRuntime`` runs when the EP
  group is a single device (``comms.group`` returns None, the reference's
  local-copy case, moe.py:150-151) and raises otherwise.  Both ends of the
  exchange are built for one GPU: ``EPRuntime.send`` (the send order, counts
  and rows of moe.py:189-212 for any placement, replicas included) and
  ``EPRuntime.expert_outputs`` (the received chunks, moe.py:213-224).

Errors surface as ``RuntimeError`` (as ``CommAborted`` / ``CommTimeout`` do in
the reference), which the resilient trainer treats as recoverable; no kernel
writes ``router.expert_bias`` until the forward has succeeded.
"""

from __future__ import annotations

import zlib
from dataclasses import dataclass

import torch

from . import kernels as K
from .layer import LayerMeta, expert_chunks, moe_layer
from .placement import ExpertPlacement, expert_dp_groups, send_tables
from .rng import generator
from .state import FULL, GroupSpec, Holdings, TensorSpec


@dataclass(frozen=True)
class MoEConfig:
    hidden: int = 8
    ffn: int = 12
    num_experts: int = 6
    top_k: int = 2
    tokens: int = 48
    seed: int = 4321
    dtype: torch.dtype = torch.float64
    bias_update_rate: float = 0.0
    """Aux-loss-free balancing: a non-trainable per-expert bias added to the router keys for
    expert *selection* only, moved by ``rate * sign(mean load - load)`` every iteration."""
    act: str = "gelu"               # "gelu" (reference) or "swiglu"
    score: str = "softmax"          # "softmax" (reference) or "sigmoid"
    normalize: bool = True          # sigmoid gates divided by their sum over the selected k
    gate_scale: float = 1.0
    num_shared: int = 0             # always-on shared experts, gate 1
    shared_ffn: int = 0             # 0 -> ffn
    expert_bias: bool = False       # keep a selection bias even when bias_update_rate == 0
    bias_init_std: float = 0.0      # seeded N(0, std) initial expert bias (0 -> zeros)
    init_std: float = 0.0           # weights N(0, std) (0 -> N(0, 1/fan_in) as the reference)
    router_dtype: torch.dtype | None = None   # None -> float64 for float64 models, else float32
    device: str = "cuda"


def router_dtype(cfg: MoEConfig) -> torch.dtype:
    if cfg.router_dtype is not None:
        return cfg.router_dtype
    return torch.float64 if cfg.dtype == torch.float64 else torch.float32


def _has_bias(cfg: MoEConfig) -> bool:
    return bool(cfg.bias_update_rate) or cfg.expert_bias


def _fc1_rows(cfg: MoEConfig, ffn: int) -> int:
    return 2 * ffn if cfg.act == "swiglu" else ffn


def moe_specs(cfg: MoEConfig) -> dict[str, TensorSpec]:
    """State contract (moe.py:42-50).  SwiGLU keeps ``experts.{e}.fc1.weight`` with 2*ffn rows
    (gate rows first); shared experts are ``shared_experts.{s}.*`` and replicated like the router."""
    h, f = cfg.hidden, cfg.ffn
    out = {"router.weight": TensorSpec("router.weight", (cfg.num_experts, h), None)}
    if _has_bias(cfg):
        out["router.expert_bias"] = TensorSpec("router.expert_bias", (cfg.num_experts,), None, trainable=False)
    for e in range(cfg.num_experts):
        out[f"experts.{e}.fc1.weight"] = TensorSpec(f"experts.{e}.fc1.weight", (_fc1_rows(cfg, f), h), None)
        out[f"experts.{e}.fc2.weight"] = TensorSpec(f"experts.{e}.fc2.weight", (h, f), None)
    fs = cfg.shared_ffn or f
    for s in range(cfg.num_shared):
        out[f"shared_experts.{s}.fc1.weight"] = TensorSpec(f"shared_experts.{s}.fc1.weight",
                                                           (_fc1_rows(cfg, fs), h), None)
        out[f"shared_experts.{s}.fc2.weight"] = TensorSpec(f"shared_experts.{s}.fc2.weight", (h, fs), None)
    return out


def expert_of(key: str) -> int | None:
    return int(key.split(".")[1]) if key.startswith("experts.") else None


def _param_dtype(cfg: MoEConfig, key: str) -> torch.dtype:
    return router_dtype(cfg) if key.startswith("router.") else cfg.dtype


def init_param(cfg: MoEConfig, spec: TensorSpec) -> torch.Tensor:
    """moe.py:57-61: randn(gen(seed, crc32(key))) / sqrt(fan_in), drawn on the CPU, then moved."""
    dt = _param_dtype(cfg, spec.key)
    gen_dt = torch.float64 if dt == torch.float64 else torch.float32
    if not spec.trainable:
        if not cfg.bias_init_std:
            return torch.zeros(spec.global_shape, dtype=dt, device=cfg.device)
        g = generator(cfg.seed, zlib.crc32(spec.key.encode()))
        return (torch.randn(spec.global_shape, generator=g, dtype=gen_dt) * cfg.bias_init_std).to(cfg.device, dt)
    g = generator(cfg.seed, zlib.crc32(spec.key.encode()))
    w = torch.randn(spec.global_shape, generator=g, dtype=gen_dt)
    w = w * cfg.init_std if cfg.init_std else w / spec.global_shape[-1] ** 0.5
    return w.to(cfg.device, dt)


def update_expert_bias(cfg: MoEConfig, bias: torch.Tensor, loads: torch.Tensor) -> None:
    """moe.py:64-66 on the device: bias += rate * sign(mean(loads) - loads)."""
    counts = loads if loads.dtype == torch.int32 else torch.round(loads).to(torch.int32)
    K.update_expert_bias(bias, counts.to(bias.device).contiguous(), cfg.bias_update_rate)


def batch(cfg: MoEConfig, iteration: int) -> tuple[torch.Tensor, torch.Tensor]:
    """moe.py:69-72: x ~ N(0,1) from gen(seed, it, 5); y = tanh(x @ teacher); drawn on the CPU."""
    gen_dt = torch.float64 if cfg.dtype == torch.float64 else torch.float32
    x = torch.randn(cfg.tokens, cfg.hidden, generator=generator(cfg.seed, iteration, 5), dtype=gen_dt)
    teacher = torch.randn(cfg.hidden, cfg.hidden, generator=generator(cfg.seed, 3), dtype=gen_dt)
    return x.to(cfg.device, cfg.dtype), torch.tanh(x @ teacher).to(cfg.device, cfg.dtype)


def route(cfg: MoEConfig, x: torch.Tensor, router: torch.Tensor,
          bias: torch.Tensor | None = None) -> tuple[torch.Tensor, torch.Tensor]:
    """moe.py:75-79: (top-k expert ids as int64 [T,k], gates [T,k] in the router dtype)."""
    _, topi, gates = K.route(x.detach().contiguous(), router.detach().contiguous(),
                             None if bias is None else bias.detach().contiguous(), cfg.top_k, cfg.score,
                             cfg.normalize, cfg.gate_scale)
    return topi.to(torch.int64), gates


def _layer_meta(cfg: MoEConfig, e0: int = 0, e1: int | None = None, n_src: int = 1) -> LayerMeta:
    return LayerMeta(num_experts=cfg.num_experts, top_k=cfg.top_k, ffn=cfg.ffn, act=cfg.act, score=cfg.score,
                     normalize=cfg.normalize, gate_scale=cfg.gate_scale, e0=e0, e1=e1, n_src=n_src,
                     num_shared=cfg.num_shared, shared_ffn=cfg.shared_ffn)


def expert_ffn(x: torch.Tensor, fc1: torch.Tensor, fc2: torch.Tensor, act: str = "gelu") -> torch.Tensor:
    """moe.py:82-83 for one expert, through the grouped-GEMM kernels (one group), with autograd."""
    return _ExpertFFN.apply(act, x.contiguous(), fc1, fc2)


class _ExpertFFN(torch.autograd.Function):
    @staticmethod
    def forward(ctx, act, x, fc1, fc2):
        M, h = x.shape
        f = fc2.shape[1]
        off = torch.tensor([0, M], dtype=torch.int32, device=x.device)
        hpre = x.new_empty(M, fc1.shape[0])
        a = x.new_empty(M, f)
        y = x.new_empty(M, h)
        if M:
            K.expert_fc1_fwd([x], off, False, M, [fc1], f, act, [hpre], [a])
            K.expert_fc2_fwd([a], off, False, M, [fc2], [y])
        ctx.act = act
        ctx.save_for_backward(x, fc1, fc2, off, hpre, a)
        return y

    @staticmethod
    def backward(ctx, dy):
        x, fc1, fc2, off, hpre, a = ctx.saved_tensors
        M = x.shape[0]
        dw1, dw2 = torch.empty_like(fc1), torch.empty_like(fc2)
        dx = torch.empty_like(x)
        if M:
            dh = torch.empty_like(hpre)
            K.expert_fc2_bwd([dy.contiguous()], [a], [hpre], off, False, M, [fc2], ctx.act, [dh], [dw2])
            K.expert_fc1_bwd([dh], [x], off, False, M, [fc1], fc2.shape[1], ctx.act, [dx], [dw1])
        else:
            dw1.zero_()
            dw2.zero_()
        return None, dx, dw1, dw2


def token_loss(out: torch.Tensor, y: torch.Tensor) -> torch.Tensor:
    """moe.py:86-87."""
    return ((out - y) ** 2).mean(dim=-1).sum()


def _weights(cfg: MoEConfig, params: dict[str, torch.Tensor], experts) -> tuple[list, list, list, list]:
    fc1s = [params[f"experts.{e}.fc1.weight"] for e in experts]
    fc2s = [params[f"experts.{e}.fc2.weight"] for e in experts]
    s1 = [params[f"shared_experts.{s}.fc1.weight"] for s in range(cfg.num_shared)]
    s2 = [params[f"shared_experts.{s}.fc2.weight"] for s in range(cfg.num_shared)]
    return fc1s, fc2s, s1, s2


def reference_forward(cfg: MoEConfig, params: dict[str, torch.Tensor], x: torch.Tensor) -> torch.Tensor:
    """moe.py:90-101: route, in-forward bias update from this batch's loads, experts, combine + residual."""
    bias = params.get("router.expert_bias")
    fc1s, fc2s, s1, s2 = _weights(cfg, params, range(cfg.num_experts))
    out, counts = moe_layer(_layer_meta(cfg), x, params["router.weight"], bias, fc1s, fc2s, s1, s2)
    if bias is not None and cfg.bias_update_rate:
        K.update_expert_bias(bias, counts[: cfg.num_experts].contiguous(), cfg.bias_update_rate)
    return out


class Adam:
    """Name-keyed Adam, the update of torch.optim.Adam(foreach=False) (resihp/runtime/optim.py:15-62)."""

    def __init__(self, params: dict[str, torch.nn.Parameter], lr: float = 1e-3, betas=(0.9, 0.999),
                 eps: float = 1e-8, weight_decay: float = 0.0):
        self.params = dict(params)
        self.lr, self.betas, self.eps, self.weight_decay = lr, betas, eps, weight_decay
        self.step_count = 0
        self.state = {n: {"exp_avg": torch.zeros_like(p), "exp_avg_sq": torch.zeros_like(p)}
                      for n, p in self.params.items()}

    def zero_grad(self) -> None:
        for p in self.params.values():
            p.grad = None

    @torch.no_grad()
    def step(self) -> None:
        """optim.py:32-46 as one fused pass per dtype (rhp_adam_step): the same operations per element,
        with IEEE square root and division."""
        self.step_count += 1
        groups: dict[torch.dtype, list[str]] = {}
        for n, p in self.params.items():
            if not p.is_cuda:
                raise RuntimeError(f"Adam: parameter {n} is not on a HIP device; the fused step runs on the GPU")
            groups.setdefault(p.dtype, []).append(n)
        for names in groups.values():
            K.adam_step([self.params[n].data for n in names], [self.params[n].grad for n in names],
                        [self.state[n]["exp_avg"] for n in names], [self.state[n]["exp_avg_sq"] for n in names],
                        self.lr, self.betas, self.eps, self.weight_decay, self.step_count)

    def state_tensors(self) -> dict[str, torch.Tensor]:
        out: dict[str, torch.Tensor] = {}
        for n, p in self.params.items():
            out[f"param/{n}"] = p.data
            out[f"exp_avg/{n}"] = self.state[n]["exp_avg"]
            out[f"exp_avg_sq/{n}"] = self.state[n]["exp_avg_sq"]
        return out

    def load_state_tensors(self, tensors: dict[str, torch.Tensor], step_count: int) -> None:
        with torch.no_grad():
            for n, p in self.params.items():
                p.data.copy_(tensors[f"param/{n}"])
                self.state[n]["exp_avg"].copy_(tensors[f"exp_avg/{n}"])
                self.state[n]["exp_avg_sq"].copy_(tensors[f"exp_avg_sq/{n}"])
        self.step_count = step_count


def reference_train(cfg: MoEConfig, iterations: int, lr: float = 1e-2):
    """moe.py:104-119 on the device: Adam on token_loss / tokens, bias updated in the forward."""
    specs = moe_specs(cfg)
    params = {k: torch.nn.Parameter(init_param(cfg, s)) for k, s in specs.items() if s.trainable}
    buffers = {k: init_param(cfg, s) for k, s in specs.items() if not s.trainable}
    opt = Adam(params, lr=lr)
    losses = []
    for it in range(iterations):
        opt.zero_grad()
        x, y = batch(cfg, it)
        loss = token_loss(reference_forward(cfg, {**params, **buffers}, x), y)
        (loss / cfg.tokens).backward()
        opt.step()
        losses.append(loss.item() / cfg.tokens)
    return losses, {**{k: v.detach().clone() for k, v in params.items()}, **{k: v.clone() for k, v in buffers.items()}}


def moe_holdings(placement: ExpertPlacement, specs: dict[str, TensorSpec]) -> Holdings:
    """moe.py:122-129: experts are held whole by their holders, everything else by every device."""
    devices = sorted(d for g in placement.groups for d in g)
    out: Holdings = {}
    for key in specs:
        e = expert_of(key)
        holders = devices if e is None else placement.holders(e)
        out[key] = [(d, FULL) for d in holders]
    return out


def edp_group_name(holders: tuple[str, ...]) -> str:
    return "edp/" + ",".join(holders)


def moe_group_specs(placement: ExpertPlacement, world: list[str]) -> list[GroupSpec]:
    """moe.py:136-146: dp over all devices, one ep group per EP group, one edp group per holder set."""
    rank = {d: i for i, d in enumerate(world)}
    specs = [GroupSpec("dp", tuple(range(len(world))), kind="dp")]
    for i, g in enumerate(placement.groups):
        specs.append(GroupSpec(f"ep/{i}", tuple(sorted(rank[d] for d in g)), kind="ep"))
    for holders in expert_dp_groups(placement):
        if len(holders) > 1:
            specs.append(GroupSpec(edp_group_name(holders), tuple(sorted(rank[d] for d in holders)), kind="edp"))
    return specs


def local_keys(placement: ExpertPlacement, me: str, specs: dict[str, TensorSpec]) -> list[str]:
    return [k for k in specs if expert_of(k) is None or expert_of(k) in placement.slots[me]]


def even_split(n: int, k: int) -> list[tuple[int, int]]:
    """resihp/utils/intervals.py:17-30: k contiguous parts, the first n % k one longer."""
    if k <= 0:
        raise ValueError(f"number of parts must be positive, got {k}")
    if n < 0:
        raise ValueError(f"length must be non-negative, got {n}")
    base, rem = divmod(n, k)
    out, start = [], 0
    for i in range(k):
        end = start + base + (1 if i < rem else 0)
        out.append((start, end))
        start = end
    return out


class EPRuntime:
    """One MoE block on one device: router (replicated) + the expert copies the placement gives it.

    moe.py:170-265 restricted to a single-device EP group: ``comms.group("ep/<i>")``
    must be None (the reference then exchanges nothing, moe.py:150-151), so every
    routed pair is processed locally by the fused GPU layer.  Data-parallel
    reductions of loads and gradients still go through ``comms``.
    """

    def __init__(self, cfg: MoEConfig, placement: ExpertPlacement, me: str, world: list[str], comms, mgr,
                 params: dict[str, torch.nn.Parameter], speeds: dict[str, float] | None = None, timeout: float = 60.0,
                 buffers: dict[str, torch.Tensor] | None = None):
        self.cfg, self.placement, self.me, self.world = cfg, placement, me, list(world)
        self.comms, self.mgr, self.timeout = comms, mgr, timeout
        self.speeds = speeds or {}
        self.gidx = placement.group_of(me)
        self.ep = sorted(placement.groups[self.gidx], key=self.world.index)
        self.params = params
        self.buffers = buffers or {}
        self.local_experts = placement.slots[me]
        self.wait = lambda w: mgr.guarded_wait(w, timeout=timeout, what="moe")
        self.tokens_per_expert: torch.Tensor | None = None

    def token_range(self) -> tuple[int, int]:
        return even_split(self.cfg.tokens, len(self.world))[self.world.index(self.me)]

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        cfg, E = self.cfg, self.cfg.num_experts
        if self.comms is not None and self.comms.group(f"ep/{self.gidx}") is not None:
            raise NotImplementedError("cross-GPU expert dispatch is not part of this build; "
                                      "the EP group must be a single device")
        missing = [e for e in range(E) if e not in self.local_experts]
        if missing:
            raise RuntimeError(f"{self.me} received tokens for expert {missing[0]} it does not host")
        fc1s, fc2s, s1, s2 = _weights(cfg, self.params, range(E))
        out, counts = moe_layer(_layer_meta(cfg), x, self.params["router.weight"],
                                self.buffers.get("router.expert_bias"), fc1s, fc2s, s1, s2)
        self.tokens_per_expert = counts[:E].to(torch.float64)
        return out

    def send_tables(self) -> K.SendTables:
        """The holder-pick periods of every expert for this device's EP group (built once)."""
        if getattr(self, "_send_tables", None) is None:
            off, dev, rank, cnt = send_tables(self.placement, self.gidx, self.ep, self.speeds)
            self._send_tables = K.SendTables.from_lists(off, dev, rank, cnt, len(self.ep),
                                                        self.params["router.weight"].device)
        return self._send_tables

    def send(self, x: torch.Tensor):
        """The sending side of the expert-parallel exchange (moe.py:189-212) for this device's tokens.

        Routes ``x``, splits each expert's pairs over its holders in the EP group
        (smooth_weighted_round_robin with ``speeds``, :193-198) and orders them device-major, then
        expert-major, then (token, slot) (:199-207).  Returns ``(rows, counts, in_splits, plan,
        gates)``: ``rows`` [P, h] = ``x.index_select(0, idx_i)`` in send order (:212), ``counts``
        the ``[|ep|, E]`` int64 matrix exchanged first (:199-209), ``in_splits`` its row sums
        (:210), the ``K.SendPlan`` (``plan.row`` is the pair -> row map the combine of the
        returned rows takes, :225-226) and the gates.  Sets ``tokens_per_expert`` like forward."""
        cfg, E = self.cfg, self.cfg.num_experts
        bias = self.buffers.get("router.expert_bias")
        _, topi, gates = K.route(x.detach().contiguous(), self.params["router.weight"].detach().contiguous(),
                                 None if bias is None else bias.detach().contiguous(), cfg.top_k, cfg.score,
                                 cfg.normalize, cfg.gate_scale)
        plan = K.ep_send_plan(topi, E, self.send_tables())
        self.tokens_per_expert = plan.dispatch.counts[:E].to(torch.float64)
        counts = plan.counts.to("cpu", torch.int64)
        P = int(counts.sum())
        rows = K.permute(x.detach().contiguous(), plan.row, cfg.top_k, P)
        return rows, counts, counts.sum(1).tolist(), plan, gates

    def expert_outputs(self, recv: torch.Tensor, recv_counts: torch.Tensor) -> torch.Tensor:
        """The receiving side of the expert-parallel exchange (moe.py:213-224) for this device's experts.

        ``recv`` holds the rows the dispatch all-to-all delivered, source-major, and ``recv_counts``
        ``[n_src, E]`` the exchanged counts (moe.py:209): chunk (s, e) holds ``recv_counts[s, e]``
        rows for expert e.  Returns the expert outputs in the received order, the order in which the
        reverse all-to-all sends them back (moe.py:224).  Rows for an expert this device does not
        host raise RuntimeError, as in the reference (moe.py:218-219).
        """
        cfg, E = self.cfg, self.cfg.num_experts
        counts = torch.as_tensor(recv_counts).detach().to("cpu", torch.int64)
        if counts.dim() != 2 or counts.shape[1] != E:
            raise ValueError(f"recv_counts must be [n_src, {E}]")
        local = sorted(self.local_experts)
        for e in range(E):
            if e not in local and bool((counts[:, e] != 0).any()):
                raise RuntimeError(f"{self.me} received tokens for expert {e} it does not host")
        local_counts = counts[:, local].to(torch.int32).to(recv.device).contiguous()
        fc1s = [self.params[f"experts.{e}.fc1.weight"] for e in local]
        fc2s = [self.params[f"experts.{e}.fc2.weight"] for e in local]
        return expert_chunks(recv, local_counts, fc1s, fc2s, cfg.act)

    def _single_device(self, name: str) -> None:
        """Collectives are not part of this build: a group with more than one device raises."""
        if self.comms is not None and self.comms.group(name) is not None:
            raise NotImplementedError(f"cross-GPU reductions over group {name!r} are not part of this build; "
                                      "every group must be a single device")

    def global_loads(self) -> list[float]:
        """Tokens routed to each expert in the last forward (moe.py:228-234).  On a single device the
        data-parallel group is the device itself, so the global loads are the local ones."""
        self._single_device("dp")
        return self.tokens_per_expert.detach().cpu().tolist()

    def finish_iteration(self) -> None:
        """Aux-loss-free bias update from the global loads (moe.py:236-240)."""
        bias = self.buffers.get("router.expert_bias")
        if bias is not None:
            loads = torch.tensor(self.global_loads(), dtype=torch.float64)
            update_expert_bias(self.cfg, bias, loads)

    def sync_grads(self) -> None:
        """moe.py:242-265 on a single device: the router's data-parallel group and every expert's
        holder group are this device alone, so there is nothing to reduce."""
        self._single_device("dp")
        for holders in expert_dp_groups(self.placement):
            if self.me in holders and len(holders) > 1:
                self._single_device(edp_group_name(holders))


__all__ = ["MoEConfig", "moe_specs", "expert_of", "init_param", "update_expert_bias", "batch", "route", "expert_ffn",
           "token_loss", "reference_forward", "reference_train", "moe_holdings", "edp_group_name", "moe_group_specs",
           "EPRuntime", "local_keys", "Adam", "even_split"]
