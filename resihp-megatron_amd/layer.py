"""The fused MoE layer: route -> dispatch -> permute -> grouped expert GEMMs -> combine, and its backward.

One ``torch.autograd.Function`` drives the gfx950 kernels of
``libresihp_moe.so``.  Its semantics are those of ``reference_forward``
(resihp/runtime/moe.py:90-101) for the experts in the local window
[e0, e1): ``out = x + sum over local slots of gate * expert(x) + sum of shared
experts(x)``.  With the full window it is the whole layer; with a partial
window it is one GPU's expert-parallel share with its tokens already received.

Expert weights stay separate tensors (one per expert and matrix), so the
autograd graph, the optimizer and expert re-placement see per-expert
parameters exactly as in the reference; the kernels reach them through
per-group pointers.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from . import kernels as K
from .fp8 import ACT, DH, DY, X, Fp8State


@dataclass(frozen=True)
class LayerMeta:
    num_experts: int
    top_k: int
    ffn: int
    act: str = "gelu"
    score: str = "softmax"
    normalize: bool = True
    gate_scale: float = 1.0
    e0: int = 0
    e1: int | None = None
    n_src: int = 1
    num_shared: int = 0
    shared_ffn: int = 0

    @property
    def window(self) -> tuple[int, int]:
        return self.e0, self.num_experts if self.e1 is None else self.e1

    @property
    def full(self) -> bool:
        return self.window == (0, self.num_experts)


def _fc1_rows(act: str, f: int) -> int:
    return 2 * f if act == "swiglu" else f


# The backward's input-gradient and weight-gradient products are independent.  Run concurrently, the
# weight gradients go to a second stream of the device (default priority), so their tiles fill the CUs
# the input-gradient products leave idle: every CU reaches a tile's epilogue at the same time, so the
# epilogues' HBM traffic comes in bursts, and the last round of a launch leaves CUs empty.  That pays
# for short reductions (measured: dsv2lite +1.4 %, the EP-128 share +2.7 %); input-gradient products
# whose reduction is long enough for the K split of their last round (h or the fc1 rows >= 8192) fill
# that round themselves and lose L2 locality to a concurrent launch (Mixtral shape: -4 %), so they keep
# the GPU to themselves.  "auto" chooses by that rule; True / False force it.
CONCURRENT_BACKWARD: bool | str = "auto"
SPLIT_MIN_K = 8192   # the reduction length from which the input-gradient products split their last round


def _concurrent(h: int, F1: int) -> bool:
    if CONCURRENT_BACKWARD == "auto":
        return max(h, F1) < SPLIT_MIN_K
    return bool(CONCURRENT_BACKWARD)
# Add the router term of the input gradient in fc1's input-gradient epilogue (layers whose experts are
# all local) instead of reading k router rows per token in the token backward.
FOLD_ROUTER_TERM = True
_side_streams: dict[int, torch.cuda.Stream] = {}


def _side_stream(dev: torch.device) -> torch.cuda.Stream:
    idx = dev.index if dev.index is not None else torch.cuda.current_device()
    st = _side_streams.get(idx)
    if st is None:
        st = torch.cuda.Stream(device=idx)
        _side_streams[idx] = st
    return st


def expert_backward(dys, acts, hpres, offsets, rows_from_offsets: bool, rows_cap: int, fc1s, fc2s, f: int,
                    act: str, dhpre, xs, dxs, dw1, dw2, router=None) -> None:
    """The expert FFN backward (fc2 then fc1, input and weight gradients) of a group launch.

    The weight gradients go to the side stream when the products run concurrently (CONCURRENT_BACKWARD);
    the current stream waits for them before returning, so every output is ordered on it as usual.
    ``router`` = (router_w, e0, perm, dl) folds the router term into fc1's input gradient."""
    fc1s, fc2s = list(fc1s), list(fc2s)

    def fc1_dgrad():
        if router is None:
            K.expert_fc1_bwd(dhpre, xs, offsets, rows_from_offsets, rows_cap, fc1s, f, act, dxs, None)
        else:
            K.expert_fc1_dgrad_router(dhpre, offsets, rows_cap, fc1s, f, act, *router, dxs)

    if not _concurrent(fc1s[0].shape[1], fc1s[0].shape[0]):
        K.expert_fc2_bwd(dys, acts, hpres, offsets, rows_from_offsets, rows_cap, fc2s, act, dhpre, dw2)
        if dxs:
            fc1_dgrad()
        K.expert_fc1_bwd(dhpre, xs, offsets, rows_from_offsets, rows_cap, fc1s, f, act, None, dw1)
        return
    main = torch.cuda.current_stream(offsets.device)
    side = _side_stream(offsets.device)
    side.wait_stream(main)
    with torch.cuda.stream(side):
        K.expert_fc2_bwd(dys, acts, hpres, offsets, rows_from_offsets, rows_cap, fc2s, act, None, dw2)
    K.expert_fc2_bwd(dys, acts, hpres, offsets, rows_from_offsets, rows_cap, fc2s, act, dhpre, None)
    side.wait_stream(main)
    with torch.cuda.stream(side):
        K.expert_fc1_bwd(dhpre, xs, offsets, rows_from_offsets, rows_cap, fc1s, f, act, None, dw1)
    if dxs:
        fc1_dgrad()
    main.wait_stream(side)


def _fp8_weight_casts(st: Fp8State, fc1s, fc2s, main: torch.cuda.Stream):
    """Starts the casts of the expert weights on the side stream: fc1's while the routing, dispatch and
    permute run, fc2's while fc1's product runs.  Returns the code buffers and the events that mark them
    written (the buffers are allocated on the caller's stream, which waits for the events before use)."""
    w1q, w2q = st.weight_codes(fc1s), st.weight_codes(fc2s)
    side = _side_stream(main.device)
    side.wait_stream(main)
    with torch.cuda.stream(side):
        st.cast_weights("fc1", fc1s, w1q)
        ev1 = torch.cuda.Event()
        ev1.record(side)
        st.cast_weights("fc2", fc2s, w2q)
        ev2 = torch.cuda.Event()
        ev2.record(side)
    return w1q, w2q, ev1, ev2


def _fp8_forward(st: Fp8State, meta: LayerMeta, offsets, P, xq, fc1s, fc2s, hpre, y, wcast):
    """Expert FFN forward in fp8 on the permuted input's codes ``xq``; returns what the backward needs
    (the row-major codes).

    The fc1 product's epilogue casts the activation straight to fp8 (no bf16 activation rows).  Every
    operand is kept as row-major codes only: the backward products read them N-contiguous and transpose
    in LDS (fp8 product modes 2 and 3).
    """
    G, f = st.G, meta.ffn
    h = xq.shape[1]
    w1q, w2q, ev1, ev2 = wcast
    main = torch.cuda.current_stream(xq.device)
    sw1 = st.scale_inv[st.w1(0):st.w1(0) + G]
    sw2 = st.scale_inv[st.w2(0):st.w2(0) + G]
    # The product casts tile each expert's rows in blocks of 128 (the padded offsets); no transposed copy
    # is written.
    poff = K.fp8_padded_offsets(offsets)
    aq = None
    if P > 0:
        epi = "swiglu_fwd" if meta.act == "swiglu" else "gelu_fwd"
        main.wait_event(ev1)
        aq, _ = st.gemm_cast(ACT, epi, offsets, poff, P, [xq] * G, "e4m3", w1q, f, h, f, st.scale_inv[X:X + 1],
                             sw1, cs=[hpre] * G, transposed=False)
        main.wait_event(ev2)
        K.fp8_gemm(0, "store", offsets, P, [aq] * G, "e4m3", w2q, "e4m3", h, f, 0, f, [y] * G,
                   st.scale_inv[ACT:ACT + 1], sw2)
    main.wait_event(ev2)   # the weight casts are complete (and their amax raised) before the layer returns
    return dict(poff=poff, xq=xq, aq=aq, w1q=w1q, w2q=w2q, sw1=sw1, sw2=sw2)


def _fp8_backward(st: Fp8State, q8: dict, meta: LayerMeta, offsets, P, dyq, hpre, dxp, dw1, dw2):
    """Expert FFN backward in fp8 (e5m2 gradients, e4m3 weights and activations) from the codes ``dyq`` of
    the output rows' gradient.

    The fc2 input-gradient product's epilogue casts the pre-activation gradient straight to fp8.  The
    input-gradient products read the row-major weight codes as [K, N] (mode 2) and the weight gradients
    the row-major activation and gradient codes (mode 3).
    """
    G, f = st.G, meta.ffn
    h = dyq.shape[1]
    F1 = _fc1_rows(meta.act, f)
    if P == 0:
        for w in (*dw1, *dw2):
            w.zero_()
        return
    s = st.scale_inv
    poff = q8["poff"]
    epi = "swiglu_bwd" if meta.act == "swiglu" else "gelu_bwd"
    dhq, _ = st.gemm_cast(DH, epi, offsets, poff, P, [dyq] * G, "e5m2", q8["w2q"], f, h, f, s[DY:DY + 1],
                          q8["sw2"], auxs=[hpre] * G, transposed=False, x_kn=True)
    K.fp8_gemm(3, "store", offsets, P, [dyq], "e5m2", [q8["aq"]], "e4m3", f, 0, h, f, list(dw2), s[DY:DY + 1],
               s[ACT:ACT + 1])
    if dxp is not None:
        K.fp8_gemm(2, "store", offsets, P, [dhq] * G, "e5m2", q8["w1q"], "e4m3", h, F1, 0, f, [dxp] * G,
                   s[DH:DH + 1], q8["sw1"])
    K.fp8_gemm(3, "store", offsets, P, [dhq], "e5m2", [q8["xq"]], "e4m3", h, 0, F1, f, list(dw1), s[DH:DH + 1],
               s[X:X + 1])


class _MoELayerFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, meta: LayerMeta, fp8, x, router_w, bias, *weights):
        e0, e1 = meta.window
        G = e1 - e0
        S = meta.num_shared
        fc1s, fc2s = list(weights[:G]), list(weights[G:2 * G])
        sfc1s, sfc2s = list(weights[2 * G:2 * G + S]), list(weights[2 * G + S:2 * G + 2 * S])
        T, h = x.shape
        k, f = meta.top_k, meta.ffn
        fs = meta.shared_ffn or f
        shared_off = shared_h = shared_a = shared_y = None
        K.need_device(x, router_w, *weights)
        main = torch.cuda.current_stream(x.device)
        # Shared experts need only x: concurrently with the routing and the routed experts on a side
        # stream where the products run concurrently, else after them.
        shared_side = S > 0 and T > 0 and _concurrent(h, _fc1_rows(meta.act, fs))
        if S:
            shared_off = torch.arange(S + 1, dtype=torch.int32, device=x.device) * T
            shared_h = [x.new_empty(T, _fc1_rows(meta.act, fs)) for _ in range(S)]
            shared_a = [x.new_empty(T, fs) for _ in range(S)]
            shared_y = [x.new_empty(T, h) for _ in range(S)]
        if shared_side:
            side = _side_stream(x.device)
            side.wait_stream(main)
            with torch.cuda.stream(side):
                K.expert_fc1_fwd([x] * S, shared_off, False, T, sfc1s, fs, meta.act, shared_h, shared_a)
                K.expert_fc2_fwd(shared_a, shared_off, False, T, sfc2s, shared_y)
        # fp8 experts (never with shared experts): the weight casts start now, on the side stream.
        wcast = _fp8_weight_casts(fp8, fc1s, fc2s, main) if fp8 is not None else None
        logits, topi, gates = K.route(x, router_w, bias, k, meta.score, meta.normalize, meta.gate_scale)
        plan = K.dispatch(topi, meta.num_experts, e0, e1, meta.n_src)
        # The reference materialises counts on the host here too (moe.py:210-211);
        # with every expert local the row count is known without a sync.
        P = T * k if meta.full else int(plan.offsets[-1].item())
        F1 = _fc1_rows(meta.act, f)
        # fp8 experts read only the input rows' codes: the permute writes them instead of bf16 rows.
        xp = K.permute(x, plan.pair_row, k, P) if fp8 is None else x.new_empty(0, h)
        hpre = x.new_empty(P, F1)
        act = x.new_empty(0 if fp8 is not None else P, f)   # the fp8 path keeps only the activation's codes
        y = x.new_empty(P, h)
        q8 = None
        if fp8 is not None:
            xq = fp8.permute(X, x, plan.pair_row, k, P)
            q8 = _fp8_forward(fp8, meta, plan.offsets, P, xq, fc1s, fc2s, hpre, y, wcast)
            q8["xq"] = xq
        elif P > 0:
            K.expert_fc1_fwd([xp] * G, plan.offsets, True, P, fc1s, f, meta.act, [hpre] * G, [act] * G)
            K.expert_fc2_fwd([act] * G, plan.offsets, True, P, fc2s, [y] * G)
        if S and T > 0 and not shared_side:
            K.expert_fc1_fwd([x] * S, shared_off, False, T, sfc1s, fs, meta.act, shared_h, shared_a)
            K.expert_fc2_fwd(shared_a, shared_off, False, T, sfc2s, shared_y)
        if shared_side:
            main.wait_stream(_side_stream(x.device))
        out = K.combine(y, x, gates, topi, plan.pair_row, shared_y or [])
        ctx.meta = meta
        ctx.fp8 = (fp8, q8)
        ctx.dims = (T, h, P, G, S)
        ctx.save_for_backward(x, router_w, logits, topi, gates, plan.perm, plan.offsets, plan.pair_row, xp, hpre,
                              act, y, *fc1s, *fc2s, *sfc1s, *sfc2s)
        ctx.shared = (shared_off, shared_h, shared_a)
        ctx.mark_non_differentiable(plan.counts)
        return out, plan.counts

    @staticmethod
    def backward(ctx, dout, _dcounts):
        meta = ctx.meta
        T, h, P, G, S = ctx.dims
        (x, router_w, logits, topi, gates, perm, offsets, pair_row, xp, hpre, act, y, *ws) = ctx.saved_tensors
        fc1s, fc2s = ws[:G], ws[G:2 * G]
        sfc1s, sfc2s = ws[2 * G:2 * G + S], ws[2 * G + S:]
        shared_off, shared_h, shared_a = ctx.shared
        f = meta.ffn
        fs = meta.shared_ffn or f
        dout = dout.contiguous()
        need_x = ctx.needs_input_grad[2]
        main = torch.cuda.current_stream(x.device)
        sdw1 = [torch.empty_like(w) for w in sfc1s]
        sdw2 = [torch.empty_like(w) for w in sfc2s]
        shared_dx = []
        shared_side = S > 0 and T > 0 and _concurrent(h, _fc1_rows(meta.act, fs))
        if S and T > 0:
            dh = [x.new_empty(T, _fc1_rows(meta.act, fs)) for _ in range(S)]
            shared_dx = [x.new_empty(T, h) for _ in range(S)] if need_x else []
        if shared_side:
            # The shared experts' whole backward (it needs only dout) on the side stream, ahead of the
            # routed experts' weight gradients that expert_backward queues there.
            side = _side_stream(x.device)
            side.wait_stream(main)
            with torch.cuda.stream(side):
                K.expert_fc2_bwd([dout] * S, shared_a, shared_h, shared_off, False, T, list(sfc2s), meta.act, dh, sdw2)
                K.expert_fc1_bwd(dh, [x] * S, shared_off, False, T, list(sfc1s), fs, meta.act, shared_dx or None, sdw1)
        fp8, q8 = ctx.fp8
        if fp8 is None:
            dy, dgates = K.combine_bwd(dout, y, gates, pair_row, P)
        else:   # the fp8 products read only the codes of the rows' gradient
            dy, dgates = fp8.combine_bwd(DY, dout, y, gates, pair_row, P)
        dl = K.route_bwd(dgates, gates, logits, topi, meta.score, meta.normalize, meta.gate_scale)
        dwr = None
        if ctx.needs_input_grad[3]:
            # The router's weight gradient needs only dl and x: on the side stream, beside the expert
            # products, instead of an HBM-bound pass that ends the backward on its own.
            side = _side_stream(x.device)
            side.wait_stream(main)
            with torch.cuda.stream(side):
                if meta.full:
                    rperm, roff = perm, offsets
                else:
                    full_plan = K.dispatch(topi, meta.num_experts)
                    rperm, roff = full_plan.perm, full_plan.offsets
                dwr = K.router_wgrad(dl, rperm, roff, x, meta.num_experts, router_w.dtype)
        # With every expert local each routed slot has a row, so fc1's input-gradient product can add the
        # router term to its rows (the token backward then sums it with the rows).
        fold = (need_x and meta.full and ctx.fp8[0] is None and P > 0 and x.dtype != torch.float64
                and router_w.dtype == torch.float32 and FOLD_ROUTER_TERM)
        dw2 = [torch.empty_like(w) for w in fc2s]
        dw1 = [torch.empty_like(w) for w in fc1s]
        dxp = x.new_empty(P, h) if need_x else None
        if fp8 is not None:
            _fp8_backward(fp8, q8, meta, offsets, P, dy, hpre, dxp, dw1, dw2)
        elif P > 0:
            dhpre = x.new_empty(P, _fc1_rows(meta.act, f))
            expert_backward([dy] * G, [act] * G, [hpre] * G, offsets, True, P, fc1s, fc2s, f, meta.act, [dhpre] * G,
                            [xp] * G, [dxp] * G if need_x else None, dw1, dw2,
                            router=(router_w, meta.window[0], perm, dl) if fold else None)
        else:
            for w in (*dw1, *dw2):
                w.zero_()
        if S and T > 0 and not shared_side:
            expert_backward([dout] * S, shared_a, shared_h, shared_off, False, T, sfc1s, sfc2s, fs, meta.act, dh,
                            [x] * S, shared_dx or None, sdw1, sdw2)
        if shared_side:
            main.wait_stream(_side_stream(x.device))
        dx = K.token_bwd(dout, dxp, pair_row, None if fold else dl, topi, router_w, shared_dx) if need_x else None
        if dwr is not None:
            main.wait_stream(_side_stream(x.device))
            dwr.record_stream(main)   # made on the side stream, used on the caller's
        return (None, None, dx, dwr, None, *dw1, *dw2, *sdw1, *sdw2)


class _ExpertChunksFn(torch.autograd.Function):
    """The receiving side of expert parallelism: the expert FFN over a source-major received buffer.

    resihp/runtime/moe.py:213-224 runs ``expert_ffn`` on every (source, expert) chunk of the received
    rows in order and returns the outputs in that order.  Here every local expert is one group of the
    grouped GEMMs over the chunks' expert-major order (the recv plan), and the products read and write
    received rows through the plan's row map: fc1 gathers its input rows, fc2 scatters its outputs
    back into the received order, and in the backward fc2's input-gradient product gathers the output
    gradient rows and fc1's scatters the input gradient.  Only the weight gradients need expert-major
    copies (of the inputs and of the output gradients); those gathers run on the side stream, beside
    the products.
    """

    @staticmethod
    def forward(ctx, act, f, rows, recv_counts, recv, *weights):
        G = len(weights) // 2
        fc1s, fc2s = list(weights[:G]), list(weights[G:])
        plan = K.recv_plan(recv_counts, rows)
        P, h = plan.rows, recv.shape[1]
        if recv.shape[0] != P:
            raise K.KernelArgumentError(f"the received buffer has {recv.shape[0]} rows, the counts {P}")
        F1 = _fc1_rows(act, f)
        xs = recv.new_empty(P, h)
        hpre = recv.new_empty(P, F1)
        a = recv.new_empty(P, f)
        y = recv.new_empty(P, h)
        if P > 0:
            main = torch.cuda.current_stream(recv.device)
            side = _side_stream(recv.device)
            side.wait_stream(main)
            with torch.cuda.stream(side):
                K.gather_rows(recv, plan.sort_row, out=xs)   # expert-major inputs, for the fc1 weight gradient
            K.expert_fc1_fwd_gather(recv, plan.sort_row, plan.offsets, P, fc1s, f, act, hpre, a)
            K.expert_fc2_fwd_scatter(a, plan.offsets, P, fc2s, y, plan.sort_row)
            main.wait_stream(side)
        ctx.act, ctx.f, ctx.P = act, f, P
        ctx.save_for_backward(plan.offsets, plan.sort_row, xs, hpre, a, *fc1s, *fc2s)
        return y

    @staticmethod
    def backward(ctx, dy_recv):
        offsets, sort_row, xs, hpre, a, *ws = ctx.saved_tensors
        G = len(ws) // 2
        fc1s, fc2s = ws[:G], ws[G:]
        act, f, P = ctx.act, ctx.f, ctx.P
        dw1 = [torch.empty_like(w) for w in fc1s]
        dw2 = [torch.empty_like(w) for w in fc2s]
        drecv = None
        need_x = ctx.needs_input_grad[4]
        if P > 0:
            dy_recv = dy_recv.contiguous()
            h = xs.shape[1]
            dys = torch.empty_like(xs)          # expert-major output gradients, for the fc2 weight gradient
            dhpre = torch.empty_like(hpre)
            main = torch.cuda.current_stream(xs.device)
            if _concurrent(h, hpre.shape[1]):
                # Weight gradients (and the gather they need) on the side stream, input gradients here.
                side = _side_stream(xs.device)
                side.wait_stream(main)
                with torch.cuda.stream(side):
                    K.gather_rows(dy_recv, sort_row, out=dys)
                    K.expert_fc2_bwd([dys] * G, [a] * G, [hpre] * G, offsets, True, P, fc2s, act, None, dw2)
                K.expert_fc2_dgrad_gather(dy_recv, sort_row, offsets, P, fc2s, act, hpre, dhpre)
                side.wait_stream(main)
                with torch.cuda.stream(side):
                    K.expert_fc1_bwd([dhpre] * G, [xs] * G, offsets, True, P, fc1s, f, act, None, dw1)
                if need_x:
                    drecv = torch.empty_like(dy_recv)
                    K.expert_fc1_dgrad_scatter(dhpre, offsets, P, fc1s, f, act, drecv, sort_row)
                main.wait_stream(side)
            else:
                K.gather_rows(dy_recv, sort_row, out=dys)
                K.expert_fc2_dgrad_gather(dy_recv, sort_row, offsets, P, fc2s, act, hpre, dhpre)
                K.expert_fc2_bwd([dys] * G, [a] * G, [hpre] * G, offsets, True, P, fc2s, act, None, dw2)
                K.expert_fc1_bwd([dhpre] * G, [xs] * G, offsets, True, P, fc1s, f, act, None, dw1)
                if need_x:
                    drecv = torch.empty_like(dy_recv)
                    K.expert_fc1_dgrad_scatter(dhpre, offsets, P, fc1s, f, act, drecv, sort_row)
        else:
            for w in (*dw1, *dw2):
                w.zero_()
            drecv = torch.zeros_like(xs)
        return (None, None, None, None, drecv, *dw1, *dw2)


def expert_chunks(recv: torch.Tensor, recv_counts: torch.Tensor, fc1s: list[torch.Tensor],
                  fc2s: list[torch.Tensor], act: str = "swiglu", rows: int | None = None) -> torch.Tensor:
    """Expert outputs of a received buffer, in the received order (with autograd).

    ``recv`` holds the rows the all-to-all delivered, source-major: chunk (s, i) of
    ``recv_counts[s, i]`` rows for local expert i (``fc1s[i]``, ``fc2s[i]``), rows in the sender's
    (token, slot) order, as resihp/runtime/moe.py:199-212 builds and exchanges them.
    ``recv_counts`` is an int32 ``[n_src, L]`` device tensor; ``rows``, its sum, may be given to spare
    reading the counts on the host.
    """
    if len(fc1s) != len(fc2s) or recv_counts.dim() != 2 or recv_counts.shape[1] != len(fc1s):
        raise ValueError("need one fc1 and one fc2 weight per column of recv_counts")
    f = fc2s[0].shape[1]
    return _ExpertChunksFn.apply(act, f, rows, recv_counts.contiguous(), recv.contiguous(), *fc1s, *fc2s)


def moe_layer(meta: LayerMeta, x: torch.Tensor, router_w: torch.Tensor, bias: torch.Tensor | None,
              fc1s: list[torch.Tensor], fc2s: list[torch.Tensor], shared_fc1s: list[torch.Tensor] = (),
              shared_fc2s: list[torch.Tensor] = (), fp8: Fp8State | None = None) -> tuple[torch.Tensor, torch.Tensor]:
    """Layer output and the int32 per-expert counts (``counts[E]`` counts invalid ids).

    With ``fp8`` the routed experts run in fp8 (e4m3 weights and activations, e5m2 gradients) with the
    delayed scaling of that state; the caller ends each iteration with ``fp8.finish_iteration()``.
    """
    e0, e1 = meta.window
    if fp8 is not None:
        if fp8.G != e1 - e0:
            raise ValueError(f"the fp8 state holds {fp8.G} experts, the window {e1 - e0}")
        if meta.num_shared:
            raise ValueError("fp8 experts: shared experts are not supported")
        h, F1 = fc1s[0].shape[1], _fc1_rows(meta.act, meta.ffn)
        if x.dtype != torch.bfloat16 or h % K.FP8_ALIGN or meta.ffn % K.FP8_ALIGN:
            raise ValueError(f"fp8 experts need bf16 tokens and hidden/ffn sizes that are multiples of {K.FP8_ALIGN}")
    if len(fc1s) != e1 - e0 or len(fc2s) != e1 - e0:
        raise ValueError(f"need one fc1 and one fc2 weight per local expert ({e1 - e0})")
    if len(shared_fc1s) != meta.num_shared or len(shared_fc2s) != meta.num_shared:
        raise ValueError(f"need {meta.num_shared} shared expert weight pairs")
    return _MoELayerFn.apply(meta, fp8, x.contiguous(), router_w.contiguous(),
                             None if bias is None else bias.detach().contiguous(),
                             *fc1s, *fc2s, *shared_fc1s, *shared_fc2s)
