"""Float64 torch-CPU restatement of the reference MoE block -- TEST INFRASTRUCTURE ONLY.

Follows ``resihp/runtime/moe.py`` (reference) function by function; each
function cites the lines it restates.  The extensions the MI355X build adds
are marked as such: SwiGLU experts, sigmoid scoring, always-on shared experts,
a seeded (non-zero) initial expert bias, Gaussian weight init with a fixed std,
and FP8 delayed scaling.  None of them changes the reference defaults.

Every function takes a config object by duck typing (the attributes of
``OracleConfig``), so tests can pass either ``OracleConfig`` or the product's
``MoEConfig``.

What pins each function is checked in ``tests/test_oracle_moe.py``: the
reference's recorded float64 outputs, closed forms, brute force and gradcheck.
"""

from __future__ import annotations

import math
import zlib
from dataclasses import dataclass

import numpy as np
import torch
import torch.nn.functional as F

_MASK64 = (1 << 64) - 1


# --------------------------------------------------------------------------- seeds


def splitmix64(x: int) -> int:
    """SplitMix64 finaliser of ``x + golden gamma`` (resihp/state/rng_data.py:21-25)."""
    x = (x + 0x9E3779B97F4A7C15) & _MASK64
    x = ((x ^ (x >> 30)) * 0xBF58476D1CE4E5B9) & _MASK64
    x = ((x ^ (x >> 27)) * 0x94D049BB133111EB) & _MASK64
    return x ^ (x >> 31)


def derive_seed(*parts: int) -> int:
    """Fold the parts through splitmix64, keep 63 bits (resihp/state/rng_data.py:28-32)."""
    h = 0
    for p in parts:
        h = splitmix64(h ^ (int(p) & _MASK64))
    return h & ((1 << 63) - 1)


def generator(*parts: int) -> torch.Generator:
    """CPU generator seeded with ``derive_seed(*parts)`` (resihp/state/rng_data.py:35-38)."""
    g = torch.Generator(device="cpu")
    g.manual_seed(derive_seed(*parts))
    return g


# --------------------------------------------------------------------------- config


@dataclass(frozen=True)
class OracleConfig:
    """Fields of ``MoEConfig`` (resihp/runtime/moe.py:28-39) plus the build's extensions."""

    hidden: int = 8
    ffn: int = 12
    num_experts: int = 6
    top_k: int = 2
    tokens: int = 48
    seed: int = 4321
    dtype: torch.dtype = torch.float64
    bias_update_rate: float = 0.0
    act: str = "gelu"             # extension: "gelu" (reference) or "swiglu"
    score: str = "softmax"        # extension: "softmax" (reference) or "sigmoid"
    normalize: bool = True        # sigmoid gates divided by their sum over the selected k
    gate_scale: float = 1.0
    num_shared: int = 0           # extension: always-on shared experts (gate 1)
    shared_ffn: int = 0
    expert_bias: bool = False     # extension: keep a selection bias even when bias_update_rate == 0
    bias_init_std: float = 0.0    # extension: seeded N(0, std) initial expert bias
    init_std: float = 0.0         # extension: N(0, std) weights instead of N(0, 1/fan_in)
    router_dtype: torch.dtype | None = None   # dtype of router weight / logits; None = dtype


def router_dtype(cfg) -> torch.dtype:
    rd = getattr(cfg, "router_dtype", None)
    if rd is not None:
        return rd
    return torch.float64 if cfg.dtype == torch.float64 else torch.float32


def has_bias(cfg) -> bool:
    return bool(cfg.bias_update_rate) or bool(getattr(cfg, "expert_bias", False))


def fc1_rows(cfg, ffn: int | None = None) -> int:
    f = cfg.ffn if ffn is None else ffn
    return 2 * f if cfg.act == "swiglu" else f


def param_shapes(cfg) -> dict[str, tuple[tuple[int, ...], bool]]:
    """Key -> (shape, trainable); the key set of resihp/runtime/moe.py:42-50.

    SwiGLU experts keep the key ``experts.{e}.fc1.weight`` with ``2*ffn`` rows,
    gate rows first, then up rows.  Shared experts use ``shared_experts.{s}.*``
    keys, which ``expert_of`` (moe.py:53-54) maps to None, so they are replicated
    like the router.
    """
    h, f, E = cfg.hidden, cfg.ffn, cfg.num_experts
    out = {"router.weight": ((E, h), True)}
    if has_bias(cfg):
        out["router.expert_bias"] = ((E,), False)
    for e in range(E):
        out[f"experts.{e}.fc1.weight"] = ((fc1_rows(cfg), h), True)
        out[f"experts.{e}.fc2.weight"] = ((h, f), True)
    for s in range(getattr(cfg, "num_shared", 0)):
        fs = cfg.shared_ffn or f
        out[f"shared_experts.{s}.fc1.weight"] = ((fc1_rows(cfg, fs), h), True)
        out[f"shared_experts.{s}.fc2.weight"] = ((h, fs), True)
    return out


def param_dtype(cfg, key: str) -> torch.dtype:
    return router_dtype(cfg) if key.startswith("router.") else cfg.dtype


def init_param(cfg, key: str, shape: tuple[int, ...], trainable: bool) -> torch.Tensor:
    """resihp/runtime/moe.py:57-61: randn(gen(seed, crc32(key))) / sqrt(fan_in); buffers zero.

    Values are drawn on the CPU in float64 when the parameter dtype is float64,
    else in float32, and cast once.
    """
    dt = param_dtype(cfg, key)
    gen_dt = torch.float64 if dt == torch.float64 else torch.float32
    if not trainable:
        std = getattr(cfg, "bias_init_std", 0.0)
        if not std:
            return torch.zeros(shape, dtype=dt)
        g = generator(cfg.seed, zlib.crc32(key.encode()))
        return (torch.randn(shape, generator=g, dtype=gen_dt) * std).to(dt)
    g = generator(cfg.seed, zlib.crc32(key.encode()))
    w = torch.randn(shape, generator=g, dtype=gen_dt)
    std = getattr(cfg, "init_std", 0.0)
    w = w * std if std else w / shape[-1] ** 0.5
    return w.to(dt)


def init_params(cfg) -> dict[str, torch.Tensor]:
    return {k: init_param(cfg, k, s, tr) for k, (s, tr) in param_shapes(cfg).items()}


def batch(cfg, iteration: int) -> tuple[torch.Tensor, torch.Tensor]:
    """resihp/runtime/moe.py:69-72: x ~ N(0,1) from gen(seed, it, 5); y = tanh(x @ teacher)."""
    gen_dt = torch.float64 if cfg.dtype == torch.float64 else torch.float32
    x = torch.randn(cfg.tokens, cfg.hidden, generator=generator(cfg.seed, iteration, 5), dtype=gen_dt)
    teacher = torch.randn(cfg.hidden, cfg.hidden, generator=generator(cfg.seed, 3), dtype=gen_dt)
    return x.to(cfg.dtype), torch.tanh(x @ teacher).to(cfg.dtype)


# --------------------------------------------------------------------------- routing


def select(keys: torch.Tensor, k: int) -> torch.Tensor:
    """Top-k indices by descending key, ties to the lowest id, NaN ranked as -inf.

    Replaces torch.topk's unspecified tie order (resihp/runtime/moe.py:77) with a
    stable descending sort.
    """
    keys = torch.where(torch.isnan(keys), torch.full_like(keys, -math.inf), keys)
    return torch.sort(keys, dim=-1, descending=True, stable=True).indices[..., :k]


def gates_from_logits(cfg, logits: torch.Tensor, topi: torch.Tensor) -> torch.Tensor:
    """Gates of the selected experts (resihp/runtime/moe.py:79 for softmax)."""
    sel = logits.gather(-1, topi)
    if cfg.score == "softmax":
        g = torch.softmax(sel, dim=-1)
    else:
        s = torch.sigmoid(sel)
        g = s / s.sum(-1, keepdim=True) if cfg.normalize else s
    return g * cfg.gate_scale if cfg.gate_scale != 1.0 else g


def route(cfg, x: torch.Tensor, router: torch.Tensor, bias: torch.Tensor | None = None,
          topi: torch.Tensor | None = None) -> tuple[torch.Tensor, torch.Tensor]:
    """resihp/runtime/moe.py:75-79.  ``topi`` may be supplied to follow a given selection."""
    logits = x.to(router.dtype) @ router.t()
    if topi is None:
        key = logits if cfg.score == "softmax" else torch.sigmoid(logits)
        if bias is not None:
            key = key + bias
        topi = select(key.detach(), cfg.top_k)
    return topi, gates_from_logits(cfg, logits, topi)


def dispatch(topi: np.ndarray, E: int, e0: int = 0, e1: int | None = None, n_src: int = 1) -> dict[str, np.ndarray]:
    """Counts and the stable expert-major permutation (resihp/runtime/moe.py:94,97,192,199-205).

    On one device the reference order -- per expert, pairs ``(token, slot)`` in
    ascending order -- is a stable argsort of the flat expert ids.
    """
    e1 = E if e1 is None else e1
    flat = np.asarray(topi, np.int64).reshape(-1)
    T = np.asarray(topi).shape[0]
    valid = (flat >= 0) & (flat < E)
    counts = np.zeros(E + 1, np.int64)
    counts[:E] = np.bincount(flat[valid], minlength=E)
    counts[E] = int((~valid).sum())
    local = valid & (flat >= e0) & (flat < e1)
    order = np.argsort(np.where(local, flat, E + 1), kind="stable")[: int(local.sum())]
    pair_row = np.full(flat.shape, -1, np.int64)
    pair_row[order] = np.arange(order.size)
    offsets = np.concatenate([[0], np.cumsum(counts[e0:e1])])
    base, rem = divmod(T, n_src)
    bounds = [0]
    for s in range(n_src):
        bounds.append(bounds[-1] + base + (1 if s < rem else 0))
    src_of_tok = np.searchsorted(np.asarray(bounds[1:]), np.arange(T), side="right")
    src_counts = np.zeros((n_src, e1 - e0), np.int64)
    tok = np.arange(flat.size) // np.asarray(topi).shape[1]
    np.add.at(src_counts, (src_of_tok[tok[local]], flat[local] - e0), 1)
    return {"counts": counts, "offsets": offsets, "src_counts": src_counts, "perm": order, "pair_row": pair_row}


def received_rows(topis, local, assign=None):
    """The rows one device receives in expert-parallel dispatch, in order (resihp/runtime/moe.py:193-212).

    ``topis[s]`` holds source s's top-k expert ids ``[T_s, k]`` (sources in EP rank order); ``local``
    lists the receiving device's experts.  Source s sends this device, for each of its experts in
    ascending id, its pairs ``(token, slot)`` routed there in ascending order (:199-207); the
    all-to-all concatenates the sources in rank order (:209-212).  A replicated expert splits its
    pairs over its holders (:193-198): ``assign(s, e, n)`` then gives, for the n pairs of source s
    routed to e in that order, which ones come to this device (a boolean list); None keeps all.
    Returns the source, token and slot of every received row, and ``recv_counts [n_src, len(local)]``.
    """
    src, tok, slot = [], [], []
    local = sorted(local)
    counts = np.zeros((len(topis), len(local)), np.int64)
    for s, topi in enumerate(topis):
        topi = np.asarray(topi, np.int64)
        k = topi.shape[1]
        flat = topi.reshape(-1)
        for i, e in enumerate(local):
            pairs = np.nonzero(flat == e)[0]        # flat index t*k + j: ascending (token, slot)
            if assign is not None:
                pairs = pairs[np.asarray(assign(s, e, pairs.size), bool)]
            counts[s, i] = pairs.size
            src.append(np.full(pairs.size, s, np.int64))
            tok.append(pairs // k)
            slot.append(pairs % k)
    cat = lambda parts: np.concatenate(parts) if parts else np.zeros(0, np.int64)  # noqa: E731
    return cat(src), cat(tok), cat(slot), counts


def smooth_weighted_round_robin(holders, speeds, n):
    """resihp/plan/expert_placement.py:150-164: the n pairs of an expert over its holders.  Weights
    ``max(1, round(10 * speed))`` (speed 1.0 when absent); every step each holder gains its weight,
    the largest running weight (ties to the larger name) is picked and pays the total."""
    if len(holders) == 1:
        return list(holders) * n
    weights = {h: max(1, round(10 * speeds.get(h, 1.0))) for h in holders}
    total = sum(weights.values())
    current = {h: 0 for h in holders}
    out = []
    for _ in range(n):
        for h in holders:
            current[h] += weights[h]
        pick = max(holders, key=lambda h: (current[h], h))
        current[pick] -= total
        out.append(pick)
    return out


def send_order_literal(topi, E, ep, holders_of, speeds):
    """resihp/runtime/moe.py:189-207 as the reference writes it, for small inputs: a dict from
    (token, slot) to its destination, filled expert by expert in ``nonzero()`` order, then for
    every device of ``ep`` (send order) and every expert the sorted pairs sent there.
    ``holders_of(e)`` is ``placement.group_holders(gidx, e)``.  Returns the flat pair ids
    ``t*k + j`` in send order and ``counts [len(ep), E]``."""
    topi = torch.as_tensor(np.asarray(topi, np.int64))
    k = topi.shape[1]
    dest = {}
    for e in range(E):
        pairs = [tuple(p) for p in (topi == e).nonzero().tolist()]
        if pairs:
            picks = smooth_weighted_round_robin(holders_of(e), speeds, len(pairs))
            dest.update(zip(pairs, picks))
    order = []
    counts = np.zeros((len(ep), E), np.int64)
    for di, d in enumerate(ep):
        for e in range(E):
            rows = sorted(p for p, h in dest.items() if h == d and int(topi[p]) == e)
            order += rows
            counts[di, e] = len(rows)
    return np.asarray([i * k + j for i, j in order], np.int64), counts


def send_order(topi, E, ep, holders_of, speeds):
    """The same order as ``send_order_literal`` (resihp/runtime/moe.py:189-207) in array form, for
    large inputs: each expert's pairs in ascending flat id get their round-robin destination, then a
    stable sort by (destination, expert) keeps the pair order within every chunk.  Pairs with an id
    outside [0, E) are not sent."""
    flat = np.asarray(topi, np.int64).reshape(-1)
    index = {d: i for i, d in enumerate(ep)}
    dest = np.full(flat.size, -1, np.int64)
    for e in range(E):
        pairs = np.nonzero(flat == e)[0]
        if pairs.size:
            picks = smooth_weighted_round_robin(holders_of(e), speeds, pairs.size)
            dest[pairs] = [index[h] for h in picks]
    sent = np.nonzero(dest >= 0)[0]
    key = dest[sent] * E + flat[sent]
    order = sent[np.argsort(key, kind="stable")]
    counts = np.zeros((len(ep), E), np.int64)
    np.add.at(counts, (dest[sent], flat[sent]), 1)
    return order, counts


def recv_plan(recv_counts) -> dict[str, np.ndarray]:
    """Expert-major grouping of a received buffer (the chunk order of resihp/runtime/moe.py:213-222,
    regrouped by expert): group i holds the rows of local expert i, sources ascending, each chunk in
    its received order.  ``sort_row[r]`` is the received row at expert-major row r, ``unsort_row`` its
    inverse, ``offsets`` the group starts."""
    counts = np.asarray(recv_counts, np.int64)
    n_src, L = counts.shape
    chunk = np.repeat(np.arange(n_src * L), counts.reshape(-1))
    rows = chunk.size
    sort_row = np.lexsort((np.arange(rows), chunk // L, chunk % L))
    unsort_row = np.empty(rows, np.int64)
    unsort_row[sort_row] = np.arange(rows)
    offsets = np.concatenate([[0], np.cumsum(counts.sum(0))])
    return {"offsets": offsets, "sort_row": sort_row, "unsort_row": unsort_row}


# --------------------------------------------------------------------------- experts


def expert_ffn(x: torch.Tensor, fc1: torch.Tensor, fc2: torch.Tensor, act: str = "gelu") -> torch.Tensor:
    """resihp/runtime/moe.py:82-83 (exact-erf GELU); SwiGLU extension: fc2(silu(x Wg^T) * (x Wu^T))."""
    hpre = F.linear(x, fc1)
    if act == "gelu":
        return F.linear(F.gelu(hpre), fc2)
    f = fc1.shape[0] // 2
    return F.linear(F.silu(hpre[:, :f]) * hpre[:, f:], fc2)


def token_loss(out: torch.Tensor, y: torch.Tensor) -> torch.Tensor:
    """resihp/runtime/moe.py:86-87."""
    return ((out - y) ** 2).mean(dim=-1).sum()


def update_expert_bias(cfg, bias: torch.Tensor, loads: torch.Tensor) -> None:
    """resihp/runtime/moe.py:64-66: bias += rate * sign(mean(load) - load)."""
    with torch.no_grad():
        bias.add_(cfg.bias_update_rate * torch.sign(loads.mean() - loads))


def layer_forward(cfg, params: dict[str, torch.Tensor], x: torch.Tensor, topi: torch.Tensor | None = None,
                  update_bias: bool = True, local: tuple[int, int] | None = None) -> torch.Tensor:
    """resihp/runtime/moe.py:90-101 (+ shared experts).

    Combine order follows the reference: per expert in ascending id,
    ``combined.index_add(rows, g * y)``, then ``x + combined``.  Shared experts
    (extension) are added after the routed sum with gate 1.  ``local = (e0, e1)``
    keeps only the experts of that window (one device's expert-parallel share,
    moe.py:213-223); their weights are the only expert weights needed.
    """
    bias = params.get("router.expert_bias")
    topi, gates = route(cfg, x, params["router.weight"], bias, topi=topi)
    gates = gates.to(x.dtype)
    if bias is not None and update_bias and cfg.bias_update_rate:
        update_expert_bias(cfg, bias, torch.bincount(topi.reshape(-1), minlength=cfg.num_experts).to(bias.dtype))
    combined = torch.zeros_like(x)
    e_lo, e_hi = local if local is not None else (0, cfg.num_experts)
    for e in range(e_lo, e_hi):
        rows, slot = (topi == e).nonzero(as_tuple=True)
        if rows.numel():
            y = expert_ffn(x[rows], params[f"experts.{e}.fc1.weight"], params[f"experts.{e}.fc2.weight"], cfg.act)
            combined = combined.index_add(0, rows, gates[rows, slot].unsqueeze(1) * y)
    out = x + combined
    for s in range(getattr(cfg, "num_shared", 0)):
        out = out + expert_ffn(x, params[f"shared_experts.{s}.fc1.weight"], params[f"shared_experts.{s}.fc2.weight"],
                               cfg.act)
    return out


# --------------------------------------------------------------------------- training


class Adam:
    """Name-keyed Adam, the update of torch.optim.Adam(foreach=False) (resihp/runtime/optim.py:15-46)."""

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
        self.step_count += 1
        b1, b2 = self.betas
        bc1 = 1 - b1 ** self.step_count
        bc2_sqrt = math.sqrt(1 - b2 ** self.step_count)
        for n, p in self.params.items():
            g = p.grad if p.grad is not None else torch.zeros_like(p)
            if self.weight_decay:
                g = g.add(p, alpha=self.weight_decay)
            s = self.state[n]
            s["exp_avg"].lerp_(g, 1 - b1)
            s["exp_avg_sq"].mul_(b2).addcmul_(g, g.conj(), value=1 - b2)
            denom = (s["exp_avg_sq"].sqrt() / bc2_sqrt).add_(self.eps)
            p.addcdiv_(s["exp_avg"], denom, value=-self.lr / bc1)


def reference_train(cfg, iterations: int, lr: float = 1e-2):
    """resihp/runtime/moe.py:104-119: Adam on token_loss / tokens, bias updated in-forward."""
    shapes = param_shapes(cfg)
    params = {k: torch.nn.Parameter(init_param(cfg, k, s, tr)) for k, (s, tr) in shapes.items() if tr}
    buffers = {k: init_param(cfg, k, s, tr) for k, (s, tr) in shapes.items() if not tr}
    opt = Adam(params, lr=lr)
    losses = []
    for it in range(iterations):
        opt.zero_grad()
        x, y = batch(cfg, it)
        loss = token_loss(layer_forward(cfg, {**params, **buffers}, x), y)
        (loss / cfg.tokens).backward()
        opt.step()
        losses.append(loss.item() / cfg.tokens)
    return losses, {**{k: v.detach().clone() for k, v in params.items()}, **{k: v.clone() for k, v in buffers.items()}}


# --------------------------------------------------------------------------- FP8 delayed scaling

FP8_MAX = {"e4m3": 448.0, "e5m2": 57344.0}
FP8_DTYPE = {"e4m3": torch.float8_e4m3fn, "e5m2": torch.float8_e5m2}


def amax_roll(history: torch.Tensor, amax: torch.Tensor) -> torch.Tensor:
    """Newest-first history update (resihp/runtime/reference_model.py:215)."""
    return torch.cat([amax.reshape(1).to(history.dtype), history[:-1]])


def fp8_scale(history: torch.Tensor, fmt: str, margin: int = 0) -> float:
    """Delayed scaling: scale = fp8_max / max(history) / 2**margin (1 when the history is all zero)."""
    amax = float(history.max())
    if not amax > 0.0 or not math.isfinite(amax):
        return 1.0
    return FP8_MAX[fmt] / amax / (2.0 ** margin)


def quantize(x: torch.Tensor, scale: float, fmt: str) -> torch.Tensor:
    """Saturating round-to-nearest-even cast of ``x * scale`` to OCP fp8, returned as float64 codes' values."""
    m = FP8_MAX[fmt]
    y = (x.to(torch.float32) * torch.tensor(scale, dtype=torch.float32)).clamp(-m, m)
    return y.to(FP8_DTYPE[fmt]).to(torch.float64)


def fp8_layer_emulation(x, router, fc1s, fc2s, topi, dout, scales, quantize_on: bool = True,
                        round_bf16: bool = True, amax: dict | None = None, act: str = "swiglu") -> dict[str, torch.Tensor]:
    """Float64 emulation of the layer with fp8 SwiGLU or GELU experts (softmax top-k gates, no shared experts):
    forward and backward, every quantised tensor cast with its delayed scale, every bf16 intermediate
    the GPU stores rounded to bf16.  An extension of resihp/runtime/moe.py:90-101 (the reference has no
    fp8 math; its amax state is reference_model.py:204-216).

    ``scales``: the scale (fp8_max / max(history)) of "x", "act" (e4m3), "dy", "dh" (e5m2) and the lists
    "w1", "w2" (e4m3) per expert.  With ``quantize_on=False, round_bf16=False`` every cast and rounding is
    the identity and the result is the float64 layer itself (the structure check of the tests).
    ``amax``, if given, receives the largest magnitude of every tensor before its cast (what one
    iteration records into the histories).  Returns out, dx, router (weight gradient), fc1 and fc2
    (lists of weight gradients).
    """
    f64 = torch.float64

    def q(v, s, fmt, name=None):
        if amax is not None and name is not None and v.numel():
            amax[name] = max(amax.get(name, 0.0), float(v.abs().max()))
        if not quantize_on:
            return v
        return quantize(v, s, fmt) / torch.tensor(s, dtype=torch.float32).to(f64)

    def bf(v):
        return v.to(torch.bfloat16).to(f64) if round_bf16 else v

    x, router, dout = x.to(f64), router.to(f64), dout.to(f64)
    T, h = x.shape
    E, k = router.shape[0], topi.shape[1]
    logits = x @ router.t()
    sel = logits.gather(-1, topi)
    gates = torch.softmax(sel, dim=-1)
    out = x.clone()
    dx = dout.clone()
    dgates = torch.zeros(T, k, dtype=f64)
    dw1, dw2 = [], []
    ys = {}
    for e in range(E):
        rows, slots = (topi == e).nonzero(as_tuple=True)
        w1, w2 = fc1s[e].to(f64), fc2s[e].to(f64)
        f = w2.shape[1]
        w1q, w2q = q(w1, scales["w1"][e], "e4m3", ("w1", e)), q(w2, scales["w2"][e], "e4m3", ("w2", e))
        if rows.numel() == 0:
            dw1.append(torch.zeros_like(w1))
            dw2.append(torch.zeros_like(w2))
            continue
        xq = q(x[rows], scales["x"], "e4m3", "x")
        hp = xq @ w1q.t()
        a = bf(F.silu(hp[:, :f]) * hp[:, f:] if act == "swiglu" else F.gelu(hp))
        aq = q(a, scales["act"], "e4m3", "act")
        y = bf(aq @ w2q.t())
        g = gates[rows, slots].unsqueeze(1)
        out.index_add_(0, rows, g * y)
        dgates[rows, slots] = (dout[rows] * y).sum(1)
        dy = bf(g * dout[rows])
        dyq = q(dy, scales["dy"], "e5m2", "dy")
        hpb = bf(hp)
        dact = dyq @ w2q
        if act == "swiglu":
            # The forward stores the backward's factors [up silu'(gate) | silu(gate)] in bf16 (computed from
            # the unrounded products), and the backward multiplies them by dact.
            gg, uu = hp[:, :f], hp[:, f:]
            sg = torch.sigmoid(gg)
            dh = bf(torch.cat([dact * bf(uu * sg * (1 + gg * (1 - sg))), dact * bf(gg * sg)], 1))
        else:
            phi = torch.exp(-0.5 * hpb * hpb) / math.sqrt(2 * math.pi)
            dh = bf(dact * (0.5 * (1 + torch.erf(hpb / math.sqrt(2))) + hpb * phi))
        dhq = q(dh, scales["dh"], "e5m2", "dh")
        dw2.append(dyq.t() @ aq)
        dw1.append(dhq.t() @ xq)
        dx.index_add_(0, rows, bf(dhq @ w1q))
        ys[e] = y
    # softmax over the k selected logits: d sel = g * (dg - sum_j g dg)
    dsel = gates * (dgates - (gates * dgates).sum(1, keepdim=True))
    dlogits = torch.zeros(T, E, dtype=f64).scatter_add_(1, topi, dsel)
    dx += dlogits @ router
    return {"out": out, "dx": dx, "router": dlogits.t() @ x, "fc1": dw1, "fc2": dw2}
