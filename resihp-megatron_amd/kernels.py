"""Torch-facing wrappers of the gfx950 kernels.

Each function checks shapes, dtypes and devices (the C ABI sees raw pointers
only), allocates its outputs and workspace through PyTorch's caching
allocator, and enqueues the kernels on the current HIP stream of the tensors'
device.  Nothing here computes on the CPU; every entry point goes through
``libresihp_moe.so``.
"""

from __future__ import annotations

import collections
import ctypes

from dataclasses import dataclass

import torch

from . import _capi as C

_DT = {torch.float64: C.F64, torch.float32: C.F32, torch.bfloat16: C.BF16}

# Optional per-entry-point timer: an object with start(name, stream) / stop(name, stream)
# that records HIP events around every C call (None = no events).
_timer = None


def set_timer(timer) -> None:
    """Installs (or with None removes) the event timer used around each C call."""
    global _timer
    _timer = timer


def _call(name: str, dev: torch.device, *args) -> None:
    """Calls entry point ``name`` with ``args`` and the current stream of ``dev``."""
    stream = torch.cuda.current_stream(dev)
    with torch.cuda.device(dev):
        if _timer is not None:
            _timer.start(name, stream)
        C.call(name, *args, stream.cuda_stream)
        if _timer is not None:
            _timer.stop(name, stream)


def dtype_code(t: torch.Tensor) -> int:
    try:
        return _DT[t.dtype]
    except KeyError:
        raise KernelArgumentError(f"unsupported dtype {t.dtype}") from None


def _ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def _need_cuda(*ts: torch.Tensor | None) -> torch.device:
    dev = None
    for t in ts:
        if t is None:
            continue
        if not t.is_cuda:
            raise RuntimeError("MoE kernels need tensors on a HIP device (cuda:N); got a CPU tensor")
        if not t.is_contiguous():
            raise RuntimeError("MoE kernels need contiguous tensors")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise RuntimeError(f"tensors on different devices: {dev} and {t.device}")
    return dev


def need_device(*ts: torch.Tensor | None) -> torch.device:
    """The HIP device all of ``ts`` are on; raises RuntimeError for host tensors or mixed devices."""
    return _need_cuda(*ts)


class KernelArgumentError(RuntimeError):
    """Arguments the kernels cannot take.  A RuntimeError, like every failure of the layer, so the
    resilient trainer (resihp/train/resilient_loop.py:28) treats it as it treats the reference's."""


def _expect(cond: bool, msg: str) -> None:
    if not cond:
        raise KernelArgumentError(msg)


def _rows_of(t: torch.Tensor, name: str, cols: int, dtype: torch.dtype) -> int:
    _expect(t.dim() == 2 and t.shape[1] == cols, f"{name} must be [rows, {cols}], got {tuple(t.shape)}")
    _expect(t.dtype == dtype, f"{name} has dtype {t.dtype}, expected {dtype}")
    return t.shape[0]


def _index(t: torch.Tensor, name: str, shape: tuple[int, ...]) -> None:
    _expect(t.dtype == torch.int32 and tuple(t.shape) == shape, f"{name} must be int32 {shape}")


def score_code(score: str) -> int:
    return {"softmax": C.SCORE_SOFTMAX, "sigmoid": C.SCORE_SIGMOID}[score]


def act_code(act: str) -> int:
    return {"gelu": C.ACT_GELU, "swiglu": C.ACT_SWIGLU}[act]


# ----------------------------------------------------------------------------- routing


def route(x: torch.Tensor, router_w: torch.Tensor, bias: torch.Tensor | None, k: int, score: str = "softmax",
          normalize: bool = True, scale: float = 1.0) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Router logits [T,E], top-k expert ids [T,k] (int32) and gates [T,k] (router dtype)."""
    dev = _need_cuda(x, router_w, bias)
    T, h = x.shape
    E = router_w.shape[0]
    _rows_of(router_w, "router_w", h, router_w.dtype)
    _expect(bias is None or (bias.dtype == router_w.dtype and tuple(bias.shape) == (E,)),
            "bias must match the router dtype and have one entry per expert")
    logits = torch.empty(T, E, dtype=router_w.dtype, device=dev)
    topi = torch.empty(T, k, dtype=torch.int32, device=dev)
    gates = torch.empty(T, k, dtype=router_w.dtype, device=dev)
    _call("rhp_route", dev, _ptr(x), dtype_code(x), _ptr(router_w), dtype_code(router_w), _ptr(bias), T, h, E, k,
          score_code(score), int(normalize), float(scale), _ptr(logits), _ptr(topi), _ptr(gates))
    return logits, topi, gates


@dataclass
class DispatchPlan:
    """Dispatch plan of the local experts [e0, e1) (all int32 device tensors)."""

    counts: torch.Tensor       # [E + 1]; counts[E] = ids outside [0, E)
    offsets: torch.Tensor      # [L + 1]
    src_counts: torch.Tensor   # [n_src, L]
    perm: torch.Tensor         # [T * k]; rows [0, offsets[L]) valid
    pair_row: torch.Tensor     # [T * k]; -1 for pairs of other experts
    e0: int
    e1: int


def dispatch(topi: torch.Tensor, E: int, e0: int = 0, e1: int | None = None, n_src: int = 1) -> DispatchPlan:
    dev = _need_cuda(topi)
    _expect(topi.dtype == torch.int32 and topi.dim() == 2, "topi must be int32 [T, k]")
    e1 = E if e1 is None else e1
    T, k = topi.shape
    L = e1 - e0
    counts = torch.empty(E + 1, dtype=torch.int32, device=dev)
    offsets = torch.empty(L + 1, dtype=torch.int32, device=dev)
    src_counts = torch.empty(n_src, L, dtype=torch.int32, device=dev)
    perm = torch.empty(max(1, T * k), dtype=torch.int32, device=dev)
    pair_row = torch.empty(max(1, T * k), dtype=torch.int32, device=dev)
    ws_bytes = C.lib().rhp_dispatch_workspace_bytes(T, k, E, n_src)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
    _call("rhp_dispatch", dev, _ptr(topi), T, k, E, e0, e1, n_src, _ptr(counts), _ptr(offsets), _ptr(src_counts),
          _ptr(perm), _ptr(pair_row), _ptr(ws), ws_bytes)
    return DispatchPlan(counts, offsets, src_counts, perm[: T * k], pair_row[: T * k], e0, e1)


def update_expert_bias(bias: torch.Tensor, counts: torch.Tensor, rate: float) -> None:
    """bias += rate * sign(mean(counts) - counts), in place (counts: int32 [E])."""
    dev = _need_cuda(bias, counts)
    _expect(counts.dtype == torch.int32 and counts.numel() >= bias.numel(), "counts must be int32, one per expert")
    _call("rhp_update_expert_bias", dev, _ptr(bias), dtype_code(bias), _ptr(counts), bias.shape[0], float(rate))


def route_bwd(dgates: torch.Tensor, gates: torch.Tensor, logits: torch.Tensor, topi: torch.Tensor, score: str,
              normalize: bool, scale: float) -> torch.Tensor:
    """Gradient of the selected logits [T,k] from the gate gradient."""
    dev = _need_cuda(dgates, gates, logits, topi)
    T, k = topi.shape
    _index(topi, "topi", (T, k))
    _expect(logits.shape[0] == T, "logits must have one row per token")
    for name, t in (("dgates", dgates), ("gates", gates)):
        _expect(t.dtype == logits.dtype and tuple(t.shape) == (T, k), f"{name} must be {logits.dtype} [T, k]")
    dl = torch.empty(T, k, dtype=logits.dtype, device=dev)
    _call("rhp_route_bwd", dev, _ptr(dgates), _ptr(gates), _ptr(logits), _ptr(topi), dtype_code(logits), T,
          logits.shape[1], k, score_code(score), int(normalize), float(scale), _ptr(dl))
    return dl


# ----------------------------------------------------------------------------- rows


def permute(x: torch.Tensor, pair_row: torch.Tensor, k: int, rows: int) -> torch.Tensor:
    """Expert-contiguous copy of the token rows: out[pair_row[t*k+j]] = x[t]."""
    dev = _need_cuda(x, pair_row)
    T, h = x.shape
    _index(pair_row, "pair_row", (T * k,))
    xp = torch.empty(rows, h, dtype=x.dtype, device=dev)
    if rows == 0:
        return xp
    _call("rhp_permute", dev, _ptr(x), dtype_code(x), T, h, k, _ptr(pair_row), _ptr(xp))
    return xp


def combine(y: torch.Tensor, x: torch.Tensor, gates: torch.Tensor, topi: torch.Tensor, pair_row: torch.Tensor,
            shared: list[torch.Tensor] = ()) -> torch.Tensor:
    """out = x + sum of gate-weighted expert rows (ascending expert id) + shared expert rows."""
    dev = _need_cuda(y, x, gates, topi, pair_row, *shared)
    T, h = x.shape
    k = topi.shape[1]
    _index(topi, "topi", (T, k))
    _index(pair_row, "pair_row", (T * k,))
    _rows_of(y, "y", h, x.dtype)
    _expect(tuple(gates.shape) == (T, k), "gates must be [T, k]")
    for i, t in enumerate(shared):
        _expect(_rows_of(t, f"shared[{i}]", h, x.dtype) == T, "shared outputs need one row per token")
    out = torch.empty_like(x)
    arr = C.ptr_array([s.data_ptr() for s in shared])
    _call("rhp_combine", dev, _ptr(y), _ptr(x), _ptr(gates), dtype_code(gates), _ptr(topi), _ptr(pair_row), arr,
          len(shared), dtype_code(x), T, h, k, _ptr(out))
    return out


def combine_bwd(dout: torch.Tensor, y: torch.Tensor, gates: torch.Tensor, pair_row: torch.Tensor,
                rows: int) -> tuple[torch.Tensor, torch.Tensor]:
    """(dy [rows,h] = gate * dout row, dgates [T,k] = <dout, y row>)."""
    dev = _need_cuda(dout, y, gates, pair_row)
    T, h = dout.shape
    k = gates.shape[1]
    _index(pair_row, "pair_row", (T * k,))
    _expect(_rows_of(y, "y", h, dout.dtype) >= rows, "y has fewer rows than the plan")
    dy = torch.empty(rows, h, dtype=dout.dtype, device=dev)
    dgates = torch.empty_like(gates)
    _call("rhp_combine_bwd", dev, _ptr(dout), _ptr(y), _ptr(gates), dtype_code(gates), _ptr(pair_row),
          dtype_code(dout), T, h, k, _ptr(dy), _ptr(dgates))
    return dy, dgates


def token_bwd(dout: torch.Tensor, dxp: torch.Tensor | None, pair_row: torch.Tensor, dl: torch.Tensor | None,
              topi: torch.Tensor, router_w: torch.Tensor, shared_dx: list[torch.Tensor] = ()) -> torch.Tensor:
    """dx = dout + sum of the token's permuted-row gradients + router input gradient + shared gradients."""
    dev = _need_cuda(dout, dxp, pair_row, dl, topi, router_w, *shared_dx)
    T, h = dout.shape
    k = topi.shape[1]
    _index(topi, "topi", (T, k))
    _index(pair_row, "pair_row", (T * k,))
    _rows_of(router_w, "router_w", h, router_w.dtype)
    if dxp is not None:
        _rows_of(dxp, "dxp", h, dout.dtype)
    _expect(dl is None or (dl.dtype == router_w.dtype and tuple(dl.shape) == (T, k)), "dl must be router dtype [T,k]")
    for i, t in enumerate(shared_dx):
        _expect(_rows_of(t, f"shared_dx[{i}]", h, dout.dtype) == T, "shared gradients need one row per token")
    dx = torch.empty_like(dout)
    arr = C.ptr_array([s.data_ptr() for s in shared_dx])
    _call("rhp_token_bwd", dev, _ptr(dout), _ptr(dxp), _ptr(pair_row), _ptr(dl), _ptr(topi), _ptr(router_w),
          dtype_code(router_w), arr, len(shared_dx), dtype_code(dout), T, h, router_w.shape[0], k, _ptr(dx))
    return dx


def router_wgrad(dl: torch.Tensor, perm: torch.Tensor, offsets: torch.Tensor, x: torch.Tensor, E: int,
                 r_dtype: torch.dtype) -> torch.Tensor:
    """dW[e] = sum over pairs routed to e of dl * x[token]; perm/offsets from a plan over all E experts."""
    dev = _need_cuda(dl, perm, offsets, x)
    T, h = x.shape
    k = dl.shape[1]
    _expect(dl.dtype == r_dtype and tuple(dl.shape) == (T, k), "dl must be router dtype [T, k]")
    _index(offsets, "offsets", (E + 1,))
    _expect(perm.dtype == torch.int32 and perm.numel() == T * k, "perm must be int32 [T * k] over all experts")
    dw = torch.empty(E, h, dtype=r_dtype, device=dev)
    rc = _DT[r_dtype]
    ws_bytes = C.lib().rhp_router_wgrad_workspace_bytes(T, h, E, k, rc)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
    _call("rhp_router_wgrad", dev, _ptr(dl), _ptr(perm), _ptr(offsets), _ptr(x), dtype_code(x), rc, T, h, E, k,
          _ptr(dw), _ptr(ws), ws_bytes)
    return dw


# ----------------------------------------------------------------------------- sending side


@dataclass
class SendTables:
    """One period of every expert's holder picks for one EP group (int32 device tensors), as
    ``placement.send_tables`` lays them out."""

    pick_off: torch.Tensor     # [E + 1]
    pick_dev: torch.Tensor     # [pick_off[E]]: device (index in the group's send order) of each pick
    pick_rank: torch.Tensor    # [pick_off[E]]: picks of the same device earlier in the period
    period_cnt: torch.Tensor   # [E * n_dev]: picks of each device in expert e's period
    n_dev: int

    @classmethod
    def from_lists(cls, off, dev, rank, cnt, n_dev: int, device) -> "SendTables":
        mk = lambda v: torch.tensor(v if len(v) else [0], dtype=torch.int32, device=device)  # noqa: E731
        return cls(mk(off), mk(dev), mk(rank), mk(cnt), n_dev)


@dataclass
class SendPlan:
    """A source's send order for its EP group (all int32 device tensors)."""

    counts: torch.Tensor       # [n_dev, E]: pairs of expert e sent to device d (moe.py:199-207)
    offsets: torch.Tensor      # [n_dev * E + 1]: chunk starts in send order
    perm: torch.Tensor         # [T * k]: send row -> flat pair t*k + j (rows < offsets[-1] valid)
    row: torch.Tensor          # [T * k]: flat pair -> send row, -1 for ids outside [0, E)
    dispatch: DispatchPlan     # the expert-major plan it was built from (window [0, E))


def ep_send_plan(topi: torch.Tensor, E: int, tables: SendTables) -> SendPlan:
    """Send order of one source's routed pairs over its EP group (resihp/runtime/moe.py:193-211)."""
    dev = _need_cuda(topi, tables.pick_off)
    _expect(topi.dtype == torch.int32 and topi.dim() == 2, "topi must be int32 [T, k]")
    _expect(tables.pick_off.numel() == E + 1 and tables.period_cnt.numel() == E * tables.n_dev,
            f"send tables must cover {E} experts and {tables.n_dev} devices")
    T, k = topi.shape
    plan = dispatch(topi, E)
    n = tables.n_dev
    counts = torch.empty(n, E, dtype=torch.int32, device=dev)
    offsets = torch.empty(n * E + 1, dtype=torch.int32, device=dev)
    perm = torch.empty(max(1, T * k), dtype=torch.int32, device=dev)
    row = torch.empty(max(1, T * k), dtype=torch.int32, device=dev)
    _call("rhp_ep_send_plan", dev, _ptr(topi), T, k, E, n, _ptr(plan.counts), _ptr(plan.offsets),
          _ptr(plan.pair_row), _ptr(tables.pick_off), _ptr(tables.pick_dev), _ptr(tables.pick_rank),
          _ptr(tables.period_cnt), _ptr(counts), _ptr(offsets), _ptr(perm), _ptr(row))
    return SendPlan(counts, offsets, perm[: T * k], row[: T * k], plan)


# ----------------------------------------------------------------------------- received rows


@dataclass
class RecvPlan:
    """Expert-major grouping of a source-major received buffer (all int32 device tensors)."""

    offsets: torch.Tensor      # [L + 1] group offsets of the expert-major rows
    sort_row: torch.Tensor     # [rows]: expert-major row r holds received row sort_row[r]
    unsort_row: torch.Tensor   # [rows]: received row q is expert-major row unsort_row[q]
    rows: int


def recv_plan(recv_counts: torch.Tensor, rows: int | None = None) -> RecvPlan:
    """Plan of a received buffer from its per-(source, local expert) counts ``[n_src, L]``.

    ``rows`` is the counts' sum.  Without it the counts are read on the host (as the reference reads
    its split sizes, resihp/runtime/moe.py:210-211) and checked; a caller that already holds the sum
    passes it and saves the synchronisation.  With the true sum the two row maps are exact inverses.
    """
    dev = _need_cuda(recv_counts)
    _expect(recv_counts.dtype == torch.int32 and recv_counts.dim() == 2, "recv_counts must be int32 [n_src, L]")
    n_src, L = recv_counts.shape
    if rows is None:
        _expect(bool((recv_counts >= 0).all()), "recv_counts must be non-negative")
        rows = int(recv_counts.sum().item())
    offsets = torch.empty(L + 1, dtype=torch.int32, device=dev)
    sort_row = torch.empty(max(1, rows), dtype=torch.int32, device=dev)
    unsort_row = torch.empty(max(1, rows), dtype=torch.int32, device=dev)
    _call("rhp_recv_plan", dev, _ptr(recv_counts), n_src, L, rows, _ptr(offsets), _ptr(sort_row), _ptr(unsort_row))
    return RecvPlan(offsets, sort_row[:rows], unsort_row[:rows], rows)


def gather_rows(src: torch.Tensor, idx: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """out[r] = src[idx[r]] (whole rows; an index outside src's rows gives a zero row)."""
    dev = _need_cuda(src, idx, out)
    _expect(src.dim() == 2 and idx.dtype == torch.int32 and idx.dim() == 1, "src must be [rows, h], idx int32 [n]")
    rows, h = idx.numel(), src.shape[1]
    if out is None:
        out = torch.empty(rows, h, dtype=src.dtype, device=dev)
    _expect(out.dtype == src.dtype and tuple(out.shape) == (rows, h), f"out must be {src.dtype} [{rows}, {h}]")
    if rows:
        _call("rhp_gather_rows", dev, _ptr(src), dtype_code(src), src.shape[0], h, _ptr(idx), rows, _ptr(out))
    return out


# ----------------------------------------------------------------------------- expert GEMMs


def _arr(ts) -> object:
    return C.ptr_array([t.data_ptr() for t in ts])


def _check_groups(what: str, ts: list[torch.Tensor], G: int, dtype: torch.dtype, cols: int,
                  rows: int | None = None, exact_shape: tuple[int, int] | None = None) -> None:
    """Every group tensor must have the kernel's dtype and shape; the kernels cannot see either."""
    _expect(len(ts) == G, f"{what}: expected {G} tensors, got {len(ts)}")
    for i, t in enumerate(ts):
        _expect(t.dtype == dtype, f"{what}[{i}] has dtype {t.dtype}, expected {dtype}")
        _expect(t.dim() == 2, f"{what}[{i}] must be 2-D")
        _expect(exact_shape is None or tuple(t.shape) == exact_shape,
                f"{what}[{i}] has shape {tuple(t.shape)}, expected {exact_shape}")
        _expect(t.shape[1] == cols, f"{what}[{i}] has {t.shape[1]} columns, expected {cols}")
        _expect(rows is None or t.shape[0] >= rows, f"{what}[{i}] has {t.shape[0]} rows, fewer than {rows}")


def _check_offsets(offsets: torch.Tensor, G: int) -> None:
    _expect(offsets.dtype == torch.int32 and offsets.numel() == G + 1, f"offsets must be int32 with {G + 1} entries")


def _shared_rows(rows_from_offsets: bool, rows_cap: int) -> int:
    # Routed experts share one buffer indexed by the offsets, shared experts have a buffer each:
    # either way every buffer must hold rows_cap rows.
    return rows_cap


def gemm_kernel(dtype: torch.dtype, act: str, h: int, f: int) -> str:
    """Which kernel the expert GEMMs run for these operands: ``"mfma"`` or ``"generic"``."""
    code = C.lib().rhp_expert_gemm_kernel(dtype_code_of(dtype), act_code(act), h, f)
    return "mfma" if code == C.GEMM_KERNEL_MFMA else "generic"


def dtype_code_of(dtype: torch.dtype) -> int:
    try:
        return _DT[dtype]
    except KeyError:
        raise KernelArgumentError(f"unsupported dtype {dtype}") from None


# K-split workspaces, one per (device, stream): its arrival counters are shared by every launch that
# uses it, so launches on two streams must not share one.  At most _SPLIT_WS_PER_DEVICE streams per
# device keep one (the least recently used is dropped first), so callers that make a stream per
# request do not grow device memory without bound.  A workspace is allocated on its own stream, so
# the caching allocator hands a dropped one's memory only to later work on that stream.
_SPLIT_WS_PER_DEVICE = 4
_split_ws_cache: "collections.OrderedDict[tuple[int, int], torch.Tensor]" = collections.OrderedDict()


def split_workspace(dev: torch.device, stream: torch.cuda.Stream | None = None) -> torch.Tensor:
    """The K-split workspace of the expert GEMMs for ``stream`` (default: the current stream of ``dev``).

    Allocated and zeroed once per (device, stream), for the last few streams of a device.  Its arrival
    counters must be zero before a call; every call that completes leaves them zero, and a call that
    fails resets them.  Under HIP graph capture a workspace is never allocated: make one call outside
    the capture on the same stream first, or the call raises.
    """
    idx = torch.device(dev).index if torch.device(dev).index is not None else torch.cuda.current_device()
    stream = stream if stream is not None else torch.cuda.current_stream(idx)
    key = (idx, stream.cuda_stream)
    ws = _split_ws_cache.get(key)
    if ws is not None:
        _split_ws_cache.move_to_end(key)
        return ws
    if torch.cuda.is_current_stream_capturing():
        raise KernelArgumentError("the expert GEMMs' K-split workspace of this stream is not allocated: "
                                  "call them once on this stream before capturing a graph")
    with torch.cuda.stream(stream):
        ws = torch.zeros(C.lib().rhp_expert_split_workspace_bytes(), dtype=torch.uint8, device=f"cuda:{idx}")
    _split_ws_cache[key] = ws
    mine = [kk for kk in _split_ws_cache if kk[0] == idx]
    for kk in mine[:max(0, len(mine) - _SPLIT_WS_PER_DEVICE)]:
        del _split_ws_cache[kk]
    return ws


def reset_split_workspace(ws: torch.Tensor, stream: torch.cuda.Stream | None = None) -> None:
    """Zeroes a K-split workspace's arrival counters on ``stream`` (a fill kernel)."""
    stream = stream if stream is not None else torch.cuda.current_stream(ws.device)
    with torch.cuda.device(ws.device):
        C.call("rhp_expert_split_workspace_reset", _ptr(ws), ws.numel(), stream.cuda_stream)


def _split_call(name: str, dev: torch.device, split: bool, *args) -> None:
    """Calls a GEMM entry point with the K-split workspace of the current stream (or none)."""
    if not split:
        _call(name, dev, *args, None, 0)
        return
    ws = split_workspace(dev)
    try:
        _call(name, dev, *args, _ptr(ws), ws.numel())
    except RuntimeError:
        # A call that did not complete may have left arrival counters set.
        reset_split_workspace(ws)
        raise


def expert_fc1_fwd(xs: list[torch.Tensor], offsets: torch.Tensor, rows_from_offsets: bool, rows_cap: int,
                   w1: list[torch.Tensor], f: int, act: str, hpre: list[torch.Tensor],
                   act_out: list[torch.Tensor], split: bool = True) -> None:
    dev = _need_cuda(offsets, *xs, *w1, *hpre, *act_out)
    G, dt, h = len(w1), w1[0].dtype, w1[0].shape[1]
    F1 = 2 * f if act == "swiglu" else f
    rows = _shared_rows(rows_from_offsets, rows_cap)
    _check_offsets(offsets, G)
    _check_groups("w1", w1, G, dt, h, exact_shape=(F1, h))
    _check_groups("x", xs, G, dt, h, rows)
    _check_groups("hpre", hpre, G, dt, F1, rows)
    _check_groups("act", act_out, G, dt, f, rows)
    _split_call("rhp_expert_fc1_fwd", dev, split, G, _ptr(offsets), int(rows_from_offsets), rows_cap,
                dtype_code(w1[0]), act_code(act), h, f, _arr(xs), _arr(w1), _arr(hpre), _arr(act_out))


def expert_fc2_fwd(acts: list[torch.Tensor], offsets: torch.Tensor, rows_from_offsets: bool, rows_cap: int,
                   w2: list[torch.Tensor], ys: list[torch.Tensor], split: bool = True) -> None:
    dev = _need_cuda(offsets, *acts, *w2, *ys)
    G, dt, (h, f) = len(w2), w2[0].dtype, tuple(w2[0].shape)
    rows = _shared_rows(rows_from_offsets, rows_cap)
    _check_offsets(offsets, G)
    _check_groups("w2", w2, G, dt, f, exact_shape=(h, f))
    _check_groups("act", acts, G, dt, f, rows)
    _check_groups("y", ys, G, dt, h, rows)
    _split_call("rhp_expert_fc2_fwd", dev, split, G, _ptr(offsets), int(rows_from_offsets), rows_cap,
                dtype_code(w2[0]), h, f, _arr(acts), _arr(w2), _arr(ys))


def expert_fc2_bwd(dys: list[torch.Tensor], acts: list[torch.Tensor], hpres: list[torch.Tensor],
                   offsets: torch.Tensor, rows_from_offsets: bool, rows_cap: int, w2: list[torch.Tensor], act: str,
                   dhpre: list[torch.Tensor] | None, dw2: list[torch.Tensor] | None, split: bool = True) -> None:
    """Input-gradient product into ``dhpre`` and weight gradient into ``dw2``; either may be None (not
    both), so the two independent products can run on two streams.  ``w2`` gives the shapes either way."""
    _expect(dhpre is not None or dw2 is not None, "expert_fc2_bwd: nothing to compute")
    dev = _need_cuda(offsets, *dys, *acts, *hpres, *w2, *(dhpre or []), *(dw2 or []))
    G, dt, (h, f) = len(w2), w2[0].dtype, tuple(w2[0].shape)
    F1 = 2 * f if act == "swiglu" else f
    rows = _shared_rows(rows_from_offsets, rows_cap)
    _check_offsets(offsets, G)
    _check_groups("w2", w2, G, dt, f, exact_shape=(h, f))
    _check_groups("dy", dys, G, dt, h, rows)
    if dw2 is not None:
        _check_groups("dw2", dw2, G, dt, f, exact_shape=(h, f))
        _check_groups("act", acts, G, dt, f, rows)
    if dhpre is not None:
        _check_groups("hpre", hpres, G, dt, F1, rows)
        _check_groups("dhpre", dhpre, G, dt, F1, rows)
    _split_call("rhp_expert_fc2_bwd", dev, split, G, _ptr(offsets), int(rows_from_offsets), rows_cap,
                dtype_code(w2[0]), act_code(act), h, f, _arr(dys), _arr(acts) if dw2 is not None else None,
                _arr(hpres) if dhpre is not None else None, _arr(w2), _arr(dhpre) if dhpre is not None else None,
                _arr(dw2) if dw2 is not None else None)


def expert_fc1_bwd(dhpre: list[torch.Tensor], xs: list[torch.Tensor], offsets: torch.Tensor,
                   rows_from_offsets: bool, rows_cap: int, w1: list[torch.Tensor], f: int, act: str,
                   dxs: list[torch.Tensor] | None, dw1: list[torch.Tensor] | None, split: bool = True) -> None:
    """Input gradient into ``dxs`` and weight gradient into ``dw1``; either may be None (not both)."""
    _expect(bool(dxs) or dw1 is not None, "expert_fc1_bwd: nothing to compute")
    dev = _need_cuda(offsets, *dhpre, *xs, *w1, *(dxs or []), *(dw1 or []))
    G, dt, h = len(w1), w1[0].dtype, w1[0].shape[1]
    F1 = 2 * f if act == "swiglu" else f
    rows = _shared_rows(rows_from_offsets, rows_cap)
    _check_offsets(offsets, G)
    _check_groups("w1", w1, G, dt, h, exact_shape=(F1, h))
    _check_groups("dhpre", dhpre, G, dt, F1, rows)
    if dw1 is not None:
        _check_groups("dw1", dw1, G, dt, h, exact_shape=(F1, h))
        _check_groups("x", xs, G, dt, h, rows)
    if dxs:
        _check_groups("dx", dxs, G, dt, h, rows)
    _split_call("rhp_expert_fc1_bwd", dev, split, G, _ptr(offsets), int(rows_from_offsets), rows_cap,
                dtype_code(w1[0]), act_code(act), h, f, _arr(dhpre), _arr(xs) if dw1 is not None else None, _arr(w1),
                _arr(dxs) if dxs else None, _arr(dw1) if dw1 is not None else None)


def _check_map(what: str, idx: torch.Tensor, rows_cap: int) -> None:
    _expect(idx.dtype == torch.int32 and idx.dim() == 1 and idx.is_contiguous() and idx.numel() >= rows_cap,
            f"{what}: the row map must be a contiguous int32 vector of at least {rows_cap} entries")


def expert_fc1_fwd_gather(src: torch.Tensor, src_idx: torch.Tensor, offsets: torch.Tensor, rows_cap: int,
                          w1: list[torch.Tensor], f: int, act: str, hpre: torch.Tensor, act_out: torch.Tensor,
                          split: bool = True) -> None:
    """expert_fc1_fwd on rows gathered from ``src``: grouped row r is ``src[src_idx[r]]`` (no copy)."""
    dev = _need_cuda(offsets, src, src_idx, *w1, hpre, act_out)
    G, dt, h = len(w1), w1[0].dtype, w1[0].shape[1]
    F1 = 2 * f if act == "swiglu" else f
    _check_offsets(offsets, G)
    _check_map("src_idx", src_idx, rows_cap)
    _check_groups("w1", w1, G, dt, h, exact_shape=(F1, h))
    _check_groups("src", [src], 1, dt, h)
    _check_groups("hpre", [hpre], 1, dt, F1, rows_cap)
    _check_groups("act", [act_out], 1, dt, f, rows_cap)
    _split_call("rhp_expert_fc1_fwd_gather", dev, split, G, _ptr(offsets), rows_cap, dtype_code(w1[0]),
                act_code(act), h, f, _ptr(src), src.shape[0], _ptr(src_idx), _arr(w1), _ptr(hpre), _ptr(act_out))


def expert_fc2_fwd_scatter(act_in: torch.Tensor, offsets: torch.Tensor, rows_cap: int, w2: list[torch.Tensor],
                           y: torch.Tensor, y_idx: torch.Tensor, split: bool = True) -> None:
    """expert_fc2_fwd writing grouped row r to ``y[y_idx[r]]`` (no copy)."""
    dev = _need_cuda(offsets, act_in, y, y_idx, *w2)
    G, dt, (h, f) = len(w2), w2[0].dtype, tuple(w2[0].shape)
    _check_offsets(offsets, G)
    _check_map("y_idx", y_idx, rows_cap)
    _check_groups("w2", w2, G, dt, f, exact_shape=(h, f))
    _check_groups("act", [act_in], 1, dt, f, rows_cap)
    _check_groups("y", [y], 1, dt, h)
    _split_call("rhp_expert_fc2_fwd_scatter", dev, split, G, _ptr(offsets), rows_cap, dtype_code(w2[0]), h, f,
                _ptr(act_in), _arr(w2), _ptr(y), y.shape[0], _ptr(y_idx))


def expert_fc2_dgrad_gather(dy: torch.Tensor, dy_idx: torch.Tensor, offsets: torch.Tensor, rows_cap: int,
                            w2: list[torch.Tensor], act: str, hpre: torch.Tensor, dhpre: torch.Tensor,
                            split: bool = True) -> None:
    """The input-gradient product of expert_fc2_bwd on output-gradient rows ``dy[dy_idx[r]]`` (no copy)."""
    dev = _need_cuda(offsets, dy, dy_idx, hpre, dhpre, *w2)
    G, dt, (h, f) = len(w2), w2[0].dtype, tuple(w2[0].shape)
    F1 = 2 * f if act == "swiglu" else f
    _check_offsets(offsets, G)
    _check_map("dy_idx", dy_idx, rows_cap)
    _check_groups("w2", w2, G, dt, f, exact_shape=(h, f))
    _check_groups("dy", [dy], 1, dt, h)
    _check_groups("hpre", [hpre], 1, dt, F1, rows_cap)
    _check_groups("dhpre", [dhpre], 1, dt, F1, rows_cap)
    _split_call("rhp_expert_fc2_dgrad_gather", dev, split, G, _ptr(offsets), rows_cap, dtype_code(w2[0]),
                act_code(act), h, f, _ptr(dy), dy.shape[0], _ptr(dy_idx), _ptr(hpre), _arr(w2), _ptr(dhpre))


def expert_fc1_dgrad_scatter(dhpre: torch.Tensor, offsets: torch.Tensor, rows_cap: int, w1: list[torch.Tensor],
                             f: int, act: str, dx: torch.Tensor, dx_idx: torch.Tensor, split: bool = True) -> None:
    """The input-gradient product of expert_fc1_bwd writing grouped row r to ``dx[dx_idx[r]]`` (no copy)."""
    dev = _need_cuda(offsets, dhpre, dx, dx_idx, *w1)
    G, dt, h = len(w1), w1[0].dtype, w1[0].shape[1]
    F1 = 2 * f if act == "swiglu" else f
    _check_offsets(offsets, G)
    _check_map("dx_idx", dx_idx, rows_cap)
    _check_groups("w1", w1, G, dt, h, exact_shape=(F1, h))
    _check_groups("dhpre", [dhpre], 1, dt, F1, rows_cap)
    _check_groups("dx", [dx], 1, dt, h)
    _split_call("rhp_expert_fc1_dgrad_scatter", dev, split, G, _ptr(offsets), rows_cap, dtype_code(w1[0]),
                act_code(act), h, f, _ptr(dhpre), _arr(w1), _ptr(dx), dx.shape[0], _ptr(dx_idx))


def expert_fc1_dgrad_router(dhpre: list[torch.Tensor], offsets: torch.Tensor, rows_cap: int, w1: list[torch.Tensor],
                            f: int, act: str, router_w: torch.Tensor, e0: int, perm: torch.Tensor, dl: torch.Tensor,
                            dxs: list[torch.Tensor], split: bool = True) -> None:
    """fc1's input gradient with the router term added per row: ``dxs[r] = dhpre[r] @ w1 + dl[perm[r]] *
    router_w[e0 + g]`` (then token_bwd runs without ``dl``).  Every expert of the layer must be local."""
    dev = _need_cuda(offsets, router_w, perm, dl, *dhpre, *w1, *dxs)
    G, dt, h = len(w1), w1[0].dtype, w1[0].shape[1]
    F1 = 2 * f if act == "swiglu" else f
    _check_offsets(offsets, G)
    _check_groups("w1", w1, G, dt, h, exact_shape=(F1, h))
    _check_groups("dhpre", dhpre, G, dt, F1, rows_cap)
    _check_groups("dx", dxs, G, dt, h, rows_cap)
    _expect(router_w.dtype == torch.float32 and router_w.dim() == 2 and router_w.shape[1] == h
            and router_w.is_contiguous() and 0 <= e0 and e0 + G <= router_w.shape[0],
            "router_w must be a contiguous float32 [E, h] holding experts e0 .. e0 + G")
    _expect(dl.dtype == torch.float32 and dl.is_contiguous(), "dl must be contiguous float32 [T, k]")
    _check_map("perm", perm, rows_cap)
    _split_call("rhp_expert_fc1_dgrad_router", dev, split, G, _ptr(offsets), rows_cap, dtype_code(w1[0]),
                act_code(act), h, f, _arr(dhpre), _arr(w1), _ptr(router_w), e0, _ptr(perm), _ptr(dl), _arr(dxs))


# ----------------------------------------------------------------------------- optimizer


def adam_step(params: list[torch.Tensor], grads: list[torch.Tensor | None], exp_avg: list[torch.Tensor],
              exp_avg_sq: list[torch.Tensor], lr: float, betas: tuple[float, float], eps: float,
              weight_decay: float, step: int) -> None:
    """One fused Adam step (resihp/runtime/optim.py:32-46) over tensors of one dtype, in place.

    ``step`` is the step number after this update (from 1); a ``None`` gradient steps with zeros.
    """
    if not params:
        return
    dev = _need_cuda(*params, *[g for g in grads if g is not None], *exp_avg, *exp_avg_sq)
    dt = params[0].dtype
    _expect(len(grads) == len(params) == len(exp_avg) == len(exp_avg_sq), "one grad and two moments per parameter")
    for i, p in enumerate(params):
        for what, t in (("grad", grads[i]), ("exp_avg", exp_avg[i]), ("exp_avg_sq", exp_avg_sq[i]), ("param", p)):
            if t is None:
                continue
            _expect(t.dtype == dt, f"{what} {i} has dtype {t.dtype}, expected {dt}")
            _expect(t.shape == p.shape and t.is_contiguous(), f"{what} {i} must be contiguous with the param's shape")
    numel = (ctypes.c_int64 * len(params))(*[p.numel() for p in params])
    garr = C.ptr_array([0 if g is None else g.data_ptr() for g in grads])
    _call("rhp_adam_step", dev, len(params), _arr(params), garr, _arr(exp_avg), _arr(exp_avg_sq), numel,
          dtype_code(params[0]), float(lr), float(betas[0]), float(betas[1]), float(eps), float(weight_decay),
          int(step))


# ----------------------------------------------------------------------------- fp8 experts

FP8_FORMATS = {"e4m3": (C.E4M3, torch.float8_e4m3fn, 448.0), "e5m2": (C.E5M2, torch.float8_e5m2, 57344.0)}
FP8_ALIGN = 128   # rows of each expert in the transposed copies are padded to this (the fp8 K step)
EPI_CODES = {"store": 0, "swiglu_fwd": 1, "gelu_fwd": 2, "swiglu_bwd": 3, "gelu_bwd": 4}


def fp8_padded_offsets(offsets: torch.Tensor) -> torch.Tensor:
    """poff[g+1] = poff[g] + roundup(rows of expert g, 128): where each expert starts in a transposed copy."""
    dev = _need_cuda(offsets)
    _expect(offsets.dtype == torch.int32 and offsets.dim() == 1 and offsets.numel() >= 2, "offsets must be int32 [G+1]")
    G = offsets.numel() - 1
    poff = torch.empty(G + 1, dtype=torch.int32, device=dev)
    _call("rhp_fp8_padded_offsets", dev, _ptr(offsets), G, FP8_ALIGN, _ptr(poff))
    return poff


def fp8_transposed_numel(cols: int, rows_cap: int, G: int) -> int:
    """Elements of a buffer that holds every expert's transposed, row-padded copy."""
    return cols * (rows_cap + (FP8_ALIGN - 1) * G)


def fp8_cast(x: torch.Tensor, offsets: torch.Tensor, poff: torch.Tensor, rows_cap: int, history: torch.Tensor,
             fmt: str, amax_bits: torch.Tensor, scale_inv: torch.Tensor, q: torch.Tensor | None = None,
             qt: torch.Tensor | None = None, margin: int = 0) -> None:
    """Delayed-scaling cast of bf16 rows to fp8 (row-major ``q`` and/or per-expert transposed ``qt``).

    ``amax_bits`` (int32 holding float bits) is raised to max |x|; ``scale_inv`` (float32 [1]) receives 1/scale.
    """
    dev = _need_cuda(x, offsets, poff, history, amax_bits, scale_inv, q, qt)
    code, fdt, _ = FP8_FORMATS[fmt]
    G = offsets.numel() - 1
    _expect(x.dtype == torch.bfloat16 and x.dim() == 2, "x must be bf16 [rows, cols]")
    rows, cols = x.shape
    _expect(cols % 64 == 0, "cols must be a multiple of 64")
    _expect(rows_cap <= rows, "rows_cap exceeds the rows of x")
    _expect(poff.dtype == torch.int32 and poff.numel() == G + 1, "poff must be int32 [G+1]")
    _expect(history.dtype == torch.float32 and history.dim() == 1, "history must be float32 [L]")
    _expect(amax_bits.dtype == torch.int32 and amax_bits.numel() == 1, "amax_bits must be int32 [1]")
    _expect(scale_inv.dtype == torch.float32 and scale_inv.numel() == 1, "scale_inv must be float32 [1]")
    _expect(q is not None or qt is not None, "nothing to write")
    if q is not None:
        _expect(q.dtype == fdt and tuple(q.shape) == (rows, cols), f"q must be {fdt} [{rows}, {cols}]")
    if qt is not None:
        _expect(qt.dtype == fdt and qt.numel() >= fp8_transposed_numel(cols, rows_cap, G), "qt is too small")
    _call("rhp_fp8_cast", dev, _ptr(x), C.BF16, cols, cols, G, _ptr(offsets), _ptr(poff), rows_cap, _ptr(history),
          history.numel(), code, margin, _ptr(amax_bits), _ptr(scale_inv), _ptr(q), _ptr(qt))


def fp8_cast_many(xs: list[torch.Tensor], histories: list[torch.Tensor], fmt: str, amax_bits: list[torch.Tensor],
                  scale_invs: list[torch.Tensor], qs: list[torch.Tensor], margin: int = 0) -> None:
    """fp8_cast of whole tensors in one launch (row-major codes only), each with its own scale state."""
    n = len(xs)
    _expect(len(histories) == n and len(amax_bits) == n and len(scale_invs) == n and len(qs) == n,
            "one history, amax, scale and code buffer per tensor")
    if n == 0:
        return
    dev = _need_cuda(*xs, *histories, *amax_bits, *scale_invs, *qs)
    code, fdt, _ = FP8_FORMATS[fmt]
    L = histories[0].numel()
    for x, hst, a, si, q in zip(xs, histories, amax_bits, scale_invs, qs):
        _expect(x.dtype == torch.bfloat16 and x.dim() == 2 and x.is_contiguous() and x.shape[1] % 64 == 0,
                "tensors must be contiguous bf16 [rows, cols], cols a multiple of 64")
        _expect(q.dtype == fdt and tuple(q.shape) == tuple(x.shape) and q.is_contiguous(), f"codes must be {fdt} like x")
        _expect(hst.dtype == torch.float32 and hst.numel() == L, f"histories must be float32 [{L}]")
        _expect(a.dtype == torch.int32 and a.numel() == 1 and si.dtype == torch.float32 and si.numel() == 1,
                "amax int32 [1] and 1/scale float32 [1] per tensor")
    rows = (ctypes.c_int64 * n)(*[x.shape[0] for x in xs])
    cols = (ctypes.c_int64 * n)(*[x.shape[1] for x in xs])
    _call("rhp_fp8_cast_many", dev, n, _arr(xs), rows, cols, _arr(histories), L, code, margin, _arr(amax_bits),
          _arr(scale_invs), _arr(qs))


def _code_state(history, amax_bits, scale_inv):
    _expect(history.dtype == torch.float32 and history.dim() == 1, "history must be float32 [L]")
    _expect(amax_bits.dtype == torch.int32 and amax_bits.numel() == 1, "amax_bits must be int32 [1]")
    _expect(scale_inv.dtype == torch.float32 and scale_inv.numel() == 1, "scale_inv must be float32 [1]")


def permute_fp8(x: torch.Tensor, pair_row: torch.Tensor, k: int, rows: int, history: torch.Tensor, fmt: str,
                amax_bits: torch.Tensor, scale_inv: torch.Tensor, margin: int = 0) -> torch.Tensor:
    """fp8 codes of ``permute(x, pair_row, k, rows)``, cast with the delayed scale of ``history`` in one pass."""
    dev = _need_cuda(x, pair_row, history, amax_bits, scale_inv)
    code, fdt, _ = FP8_FORMATS[fmt]
    _expect(x.dtype == torch.bfloat16 and x.dim() == 2 and x.is_contiguous(), "x must be contiguous bf16 [T, h]")
    T, h = x.shape
    _index(pair_row, "pair_row", (T * k,))
    _code_state(history, amax_bits, scale_inv)
    q = torch.empty(max(rows, 1), h, dtype=fdt, device=dev)   # a valid address also without rows
    _call("rhp_permute_fp8", dev, _ptr(x), T, h, k, _ptr(pair_row), code, _ptr(history), history.numel(), margin,
          _ptr(amax_bits), _ptr(scale_inv), _ptr(q))
    return q[:rows]


def combine_bwd_fp8(dout: torch.Tensor, y: torch.Tensor, gates: torch.Tensor, pair_row: torch.Tensor, rows: int,
                    history: torch.Tensor, fmt: str, amax_bits: torch.Tensor, scale_inv: torch.Tensor,
                    margin: int = 0) -> tuple[torch.Tensor, torch.Tensor]:
    """``combine_bwd`` with dy leaving as fp8 codes (the cast of its bf16 rows): (dy codes, dgates)."""
    dev = _need_cuda(dout, y, gates, pair_row, history, amax_bits, scale_inv)
    code, fdt, _ = FP8_FORMATS[fmt]
    _expect(dout.dtype == torch.bfloat16 and gates.dtype == torch.float32, "bf16 rows and float32 gates")
    T, h = dout.shape
    k = gates.shape[1]
    _index(pair_row, "pair_row", (T * k,))
    _expect(_rows_of(y, "y", h, dout.dtype) >= rows, "y has fewer rows than the plan")
    _code_state(history, amax_bits, scale_inv)
    q = torch.empty(max(rows, 1), h, dtype=fdt, device=dev)
    dgates = torch.empty_like(gates)
    _call("rhp_combine_bwd_fp8", dev, _ptr(dout), _ptr(y), _ptr(gates), _ptr(pair_row), T, h, k, _ptr(dgates), code,
          _ptr(history), history.numel(), margin, _ptr(amax_bits), _ptr(scale_inv), _ptr(q))
    return q[:rows], dgates


def fp8_amax_roll(history: torch.Tensor, amax_bits: torch.Tensor) -> None:
    """End of iteration: every history gets its pending amax prepended (newest first); the amax resets."""
    dev = _need_cuda(history, amax_bits)
    _expect(history.dtype == torch.float32 and history.dim() == 2, "history must be float32 [n, L]")
    _expect(amax_bits.dtype == torch.int32 and amax_bits.numel() == history.shape[0], "amax_bits must be int32 [n]")
    _call("rhp_fp8_amax_roll", dev, _ptr(history), _ptr(amax_bits), history.shape[0], history.shape[1])


def fp8_gemm(mode: int | bool, epi: str, offsets: torch.Tensor, rows_cap: int, ys: list[torch.Tensor], y_fmt: str,
             xs: list[torch.Tensor], x_fmt: str, N: int, K: int, Mo: int, f: int, cs: list[torch.Tensor],
             y_scale_inv: torch.Tensor, x_scale_inv: torch.Tensor, c2s: list[torch.Tensor] | None = None,
             auxs: list[torch.Tensor] | None = None) -> None:
    """Grouped fp8 product with bf16 outputs (rhp_fp8_gemm).  ``mode``: 0 (or False) row-grouped on [N, K]
    operands, 1 (or True) K-grouped on transposed copies, 2 row-grouped with x held [K, N], 3 K-grouped on
    the row-major codes [rows, Mo] and [rows, N]."""
    mode = int(mode)
    _expect(mode in (0, 1, 2, 3), "mode must be 0 to 3")
    kgroups = mode in (1, 3)
    G = offsets.numel() - 1
    dev = _need_cuda(offsets, *ys, *xs, *cs, *(c2s or []), *(auxs or []), y_scale_inv, x_scale_inv)
    ycode, ydt, _ = FP8_FORMATS[y_fmt]
    xcode, xdt, _ = FP8_FORMATS[x_fmt]
    _expect(len(cs) == G, f"expected {G} outputs")
    for t in ys:
        _expect(t.dtype == ydt, f"y operands must be {ydt}")
    for t in xs:
        _expect(t.dtype == xdt, f"x operands must be {xdt}")
    for t in cs + (c2s or []) + (auxs or []):
        _expect(t.dtype == torch.bfloat16 and t.dim() == 2, "outputs and pre-activations must be bf16 matrices")
    _expect(x_scale_inv.dtype == torch.float32 and x_scale_inv.numel() in (1, G), "x_scale_inv must be float32 [1] or [G]")
    _expect(y_scale_inv.dtype == torch.float32 and y_scale_inv.numel() == 1, "y_scale_inv must be float32 [1]")
    if mode == 3:
        _expect(len(ys) == 1 and len(xs) == 1, "K-grouped products take one buffer per operand")
        _expect(ys[0].dim() == 2 and ys[0].shape[1] == Mo and ys[0].shape[0] >= rows_cap and ys[0].is_contiguous(),
                f"y must be [>= {rows_cap}, {Mo}]")
        _expect(xs[0].dim() == 2 and xs[0].shape[1] == N and xs[0].shape[0] >= rows_cap and xs[0].is_contiguous(),
                f"x must be [>= {rows_cap}, {N}]")
        for t in cs:
            _expect(tuple(t.shape) == (Mo, N), f"outputs must be [{Mo}, {N}]")
        ldy, ldx = Mo, N
    elif kgroups:
        _expect(len(ys) == 1 and len(xs) == 1, "K-grouped products take one transposed buffer per operand")
        _expect(ys[0].numel() >= fp8_transposed_numel(Mo, rows_cap, G), "y is too small")
        _expect(xs[0].numel() >= fp8_transposed_numel(N, rows_cap, G), "x is too small")
        for t in cs:
            _expect(tuple(t.shape) == (Mo, N), f"outputs must be [{Mo}, {N}]")
        ldy = ldx = 0
    elif mode == 2:
        _expect(len(ys) == G and len(xs) == G, f"expected {G} operands per side")
        for t in ys:
            _expect(t.dim() == 2 and t.shape[1] == K and t.shape[0] >= rows_cap, f"y must be [>= {rows_cap}, {K}]")
        for t in xs:
            _expect(tuple(t.shape) == (K, N) and t.is_contiguous(), f"x must be [{K}, {N}]")
        ldy, ldx = K, N
    else:
        _expect(len(ys) == G and len(xs) == G, f"expected {G} operands per side")
        for t in ys:
            _expect(t.dim() == 2 and t.shape[1] == K and t.shape[0] >= rows_cap, f"y must be [>= {rows_cap}, {K}]")
        xrows = 2 * f if epi == "swiglu_fwd" else N
        for t in xs:
            _expect(tuple(t.shape) == (xrows, K), f"x must be [{xrows}, {K}]")
        ldy = ldx = K
    c2p = _arr(c2s) if c2s else None
    auxp = _arr(auxs) if auxs else None
    _call("rhp_fp8_gemm", dev, mode, EPI_CODES[epi], G, _ptr(offsets), rows_cap, ycode, xcode, N, K, Mo, f,
          _arr(ys), ldy, _arr(xs), ldx, _arr(cs), cs[0].shape[1], c2p, c2s[0].shape[1] if c2s else 0, auxp,
          auxs[0].shape[1] if auxs else 0, _ptr(y_scale_inv), _ptr(x_scale_inv),
          0 if x_scale_inv.numel() == 1 else 1)


def fp8_gemm_cast(epi: str, offsets: torch.Tensor, poff: torch.Tensor, rows_cap: int, ys: list[torch.Tensor],
                  y_fmt: str, xs: list[torch.Tensor], x_fmt: str, N: int, K: int, f: int,
                  y_scale_inv: torch.Tensor, x_scale_inv: torch.Tensor, history: torch.Tensor, q_fmt: str,
                  amax_bits: torch.Tensor, scale_inv: torch.Tensor, q: torch.Tensor | None, qt: torch.Tensor | None,
                  cs: list[torch.Tensor] | None = None, auxs: list[torch.Tensor] | None = None,
                  margin: int = 0, x_kn: bool = False) -> None:
    """Row-grouped fp8 product whose epilogue casts its activation output to fp8 (rhp_fp8_gemm_cast).
    ``x_kn``: the weights are held [K, N] (row-major codes; backward epilogues only).

    Forward epilogues store the pre-activation in ``cs`` and cast the activation; backward epilogues read
    the pre-activation from ``auxs`` and cast the pre-activation gradient.  The codes equal those of
    ``fp8_gemm`` followed by ``fp8_cast`` of its bf16 output, bit for bit.
    """
    G = offsets.numel() - 1
    dev = _need_cuda(offsets, poff, *ys, *xs, *(cs or []), *(auxs or []), y_scale_inv, x_scale_inv, history,
                     amax_bits, scale_inv, q, qt)
    ycode, ydt, _ = FP8_FORMATS[y_fmt]
    xcode, xdt, _ = FP8_FORMATS[x_fmt]
    qcode, qdt, _ = FP8_FORMATS[q_fmt]
    fwd = epi in ("swiglu_fwd", "gelu_fwd")
    _expect(epi in ("swiglu_fwd", "gelu_fwd", "swiglu_bwd", "gelu_bwd"), f"no quantising form of epilogue {epi!r}")
    _expect(len(ys) == G and len(xs) == G, f"expected {G} operands per side")
    for t in ys:
        _expect(t.dtype == ydt and t.dim() == 2 and t.shape[1] == K and t.shape[0] >= rows_cap,
                f"y operands must be {ydt} [>= {rows_cap}, {K}]")
    xrows = 2 * f if epi == "swiglu_fwd" else N
    xshape = (K, N) if x_kn else (xrows, K)
    _expect(not (x_kn and fwd), "[K, N] weights only with the backward epilogues")
    for t in xs:
        _expect(t.dtype == xdt and tuple(t.shape) == xshape and t.is_contiguous(),
                f"x operands must be {xdt} {list(xshape)}")
    if fwd:
        _expect(cs is not None and len(cs) == G and auxs is None, "forward epilogues take G pre-activation outputs")
    else:
        _expect(cs is None and auxs is not None and len(auxs) == G, "backward epilogues take G pre-activation inputs")
    for t in (cs or []) + (auxs or []):
        _expect(t.dtype == torch.bfloat16 and t.dim() == 2, "pre-activations must be bf16 matrices")
    _expect(poff.dtype == torch.int32 and poff.numel() == G + 1, "poff must be int32 [G+1]")
    _expect(history.dtype == torch.float32 and history.dim() == 1, "history must be float32 [L]")
    _expect(amax_bits.dtype == torch.int32 and amax_bits.numel() == 1, "amax_bits must be int32 [1]")
    _expect(scale_inv.dtype == torch.float32 and scale_inv.numel() == 1, "scale_inv must be float32 [1]")
    _expect(x_scale_inv.dtype == torch.float32 and x_scale_inv.numel() in (1, G), "x_scale_inv must be float32 [1] or [G]")
    _expect(y_scale_inv.dtype == torch.float32 and y_scale_inv.numel() == 1, "y_scale_inv must be float32 [1]")
    cols = 2 * N if epi == "swiglu_bwd" else N
    _expect(q is not None or qt is not None, "nothing to write")
    if q is not None:
        _expect(q.dtype == qdt and q.dim() == 2 and q.shape[1] == cols and q.shape[0] >= rows_cap,
                f"q must be {qdt} [>= {rows_cap}, {cols}]")
    if qt is not None:
        _expect(qt.dtype == qdt and qt.numel() >= fp8_transposed_numel(cols, rows_cap, G), "qt is too small")
    _call("rhp_fp8_gemm_cast", dev, EPI_CODES[epi], G, _ptr(offsets), _ptr(poff), rows_cap, ycode, xcode, N, K, f,
          _arr(ys), K, _arr(xs), N if x_kn else K, int(x_kn), _arr(cs) if cs else None, cs[0].shape[1] if cs else 0,
          _arr(auxs) if auxs else None, auxs[0].shape[1] if auxs else 0, _ptr(y_scale_inv), _ptr(x_scale_inv),
          0 if x_scale_inv.numel() == 1 else 1, _ptr(history), history.numel(), qcode, margin, _ptr(amax_bits),
          _ptr(scale_inv), _ptr(q), _ptr(qt))
