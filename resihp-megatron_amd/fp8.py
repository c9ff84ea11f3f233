"""Delayed-scaling state of one MoE layer whose experts run in fp8.

The reference keeps an FP8-style amax history per layer
(resihp/runtime/reference_model.py:44-46, 204-207): a buffer of L entries, a
pending amax raised during the iteration, and at the end of the iteration the
amax prepended newest-first (:212-216).  Here every quantised tensor of the
layer has such a history:

    0  expert-input rows (fc1 input)          e4m3
    1  SwiGLU / GELU output rows (fc2 input)  e4m3
    2  gradient of the expert outputs         e5m2
    3  gradient of the pre-activations        e5m2
    4 + g        fc1 weight of local expert g   e4m3
    4 + G + g    fc2 weight of local expert g   e4m3

All of it lives on the device; casts raise the pending amax with atomics and
``finish_iteration`` rolls every history in one kernel, so the layer never
synchronises with the host for scaling.
"""

from __future__ import annotations

import torch

from . import kernels as K

X, ACT, DY, DH = 0, 1, 2, 3
FORMATS = {X: "e4m3", ACT: "e4m3", DY: "e5m2", DH: "e5m2"}


class Fp8State:
    """Histories [n, L] (float32), pending amax [n] (float bits in int32) and 1/scale [n] (float32)."""

    def __init__(self, num_local_experts: int, history_len: int = 16, margin: int = 0,
                 device: torch.device | str = "cuda"):
        if num_local_experts < 1 or history_len < 1 or margin < 0:
            raise ValueError("need at least one expert, a positive history length and a margin >= 0")
        self.G = num_local_experts
        self.L = history_len
        self.margin = margin
        n = 4 + 2 * num_local_experts
        self.history = torch.ones(n, history_len, dtype=torch.float32, device=device)   # reference init: ones
        self.amax = torch.zeros(n, dtype=torch.int32, device=device)
        self.scale_inv = torch.ones(n, dtype=torch.float32, device=device)
        self._ranges: dict[tuple[int, str], tuple[torch.Tensor, torch.Tensor]] = {}

    def w1(self, g: int) -> int:
        return 4 + g

    def w2(self, g: int) -> int:
        return 4 + self.G + g

    def seed_history(self, priors: dict[int, float], seed: int = 0, spread: float = 0.25) -> None:
        """Prior amax values: history[i] = priors[i] * (1 + spread * u), u ~ U(-1, 1) from a seeded generator.

        ``priors`` maps a tensor index (X, ACT, DY, DH, w1(g), w2(g)) to its nominal amax; indices not
        given keep their history.
        """
        g = torch.Generator().manual_seed(seed)
        h = self.history.cpu()
        for i, a in priors.items():
            u = torch.rand(self.L, generator=g, dtype=torch.float64) * 2 - 1
            h[i] = (a * (1 + spread * u)).float()
        self.history.copy_(h)

    # Layer-wide tensors of the state, by key (the expert weights' rows go by expert id).
    LAYER_KEYS = (("fp8.expert_input", X), ("fp8.activation", ACT), ("fp8.grad_output", DY),
                  ("fp8.grad_preactivation", DH))

    def state_tensors(self, experts: list[int]) -> dict[str, torch.Tensor]:
        """The state by key, for live re-placement: histories and pending amaxes of the layer-wide tensors,
        and of every local expert's two weights under ``experts.{e}.fc1`` / ``experts.{e}.fc2`` (``experts``
        lists the expert id of each local slot).  The reference migrates its amax buffer with its layer
        and restores it on rollback (resihp/runtime/reference_model.py:44-46; transaction.py:41-43, 59-65);
        the values returned are views of this state."""
        if len(experts) != self.G:
            raise ValueError(f"need the expert id of each of the {self.G} local slots")
        rows = [(k, i) for k, i in self.LAYER_KEYS]
        for g, e in enumerate(experts):
            rows += [(f"experts.{e}.fc1", self.w1(g)), (f"experts.{e}.fc2", self.w2(g))]
        out = {}
        for key, i in rows:
            out[f"{key}.amax_history"] = self.history[i]
            out[f"{key}.amax"] = self.amax[i:i + 1]
        return out

    def load_state_tensors(self, tensors: dict[str, torch.Tensor], experts: list[int]) -> None:
        """Copies a keyed state (``state_tensors`` of any holder) into this one, whose local slots hold
        ``experts``; a missing key, a wrong shape or a wrong dtype raises and leaves this state unchanged.

        Nothing is converted by value: a pending amax (``.amax``, a float held as its bits in int32) also
        accepts a float32 tensor of the amax itself, as the reference keeps its pending amax
        (resihp/runtime/reference_model.py:207, 263), and takes its bits."""
        mine = self.state_tensors(experts)
        missing = [k for k in mine if k not in tensors]
        if missing:
            raise KeyError(f"fp8 state misses {missing[0]}")
        src = {}
        for k, dst in mine.items():
            t = tensors[k]
            if tuple(t.shape) != tuple(dst.shape):
                raise ValueError(f"{k} has shape {tuple(t.shape)}, expected {tuple(dst.shape)}")
            if k.endswith(".amax") and t.dtype == torch.float32:
                t = t.contiguous().view(torch.int32)
            if t.dtype != dst.dtype:
                raise TypeError(f"{k} has dtype {t.dtype}, expected {dst.dtype}")
            src[k] = t
        with torch.no_grad():
            for k, dst in mine.items():
                dst.copy_(src[k].to(dst.device))

    def finish_iteration(self) -> None:
        """Prepend every pending amax to its history and reset it (reference_model.py:212-216)."""
        K.fp8_amax_roll(self.history, self.amax)

    def single_range(self, rows: int, device: torch.device) -> tuple[torch.Tensor, torch.Tensor]:
        """Offsets [0, rows] and padded offsets of a one-group cast (a weight matrix), cached per size."""
        key = (rows, str(device))
        if key not in self._ranges:
            if rows % K.FP8_ALIGN:
                raise ValueError(f"fp8 weights need row counts that are multiples of {K.FP8_ALIGN}, got {rows}")
            t = torch.tensor([0, rows], dtype=torch.int32, device=device)
            self._ranges[key] = (t, t.clone())
        return self._ranges[key]

    def codes(self, i: int, rows: int, cols: int, rows_cap: int, G: int, device: torch.device,
              row_major: bool = True, transposed: bool = True) -> tuple[torch.Tensor | None, torch.Tensor | None]:
        """Uninitialised (row-major, per-expert transposed) code buffers for a cast of tensor i."""
        fdt = K.FP8_FORMATS[FORMATS.get(i, "e4m3")][1]
        q = torch.empty(rows, cols, dtype=fdt, device=device) if row_major else None
        qt = torch.empty(K.fp8_transposed_numel(cols, rows_cap, G), dtype=fdt, device=device) if transposed else None
        return q, qt

    def cast(self, i: int, x: torch.Tensor, offsets: torch.Tensor, poff: torch.Tensor, rows_cap: int,
             row_major: bool = True, transposed: bool = True) -> tuple[torch.Tensor | None, torch.Tensor | None]:
        """Casts rows of ``x`` with tensor i's scale; returns (row-major fp8, per-expert transposed fp8)."""
        rows, cols = x.shape
        if row_major and not transposed and rows == rows_cap and x.is_contiguous():
            # Row-major codes of the whole buffer: one scale for every expert's rows, so the grouping plays
            # no part and the whole-tensor cast (no transposition stage) does it.
            q = torch.empty(rows, cols, dtype=K.FP8_FORMATS[FORMATS.get(i, "e4m3")][1], device=x.device)
            K.fp8_cast_many([x], [self.history[i]], FORMATS.get(i, "e4m3"), [self.amax[i:i + 1]],
                            [self.scale_inv[i:i + 1]], [q], self.margin)
            return q, None
        q, qt = self.codes(i, rows, cols, rows_cap, offsets.numel() - 1, x.device, row_major, transposed)
        K.fp8_cast(x, offsets, poff, rows_cap, self.history[i], FORMATS.get(i, "e4m3"), self.amax[i:i + 1],
                   self.scale_inv[i:i + 1], q, qt, self.margin)
        return q, qt

    def permute(self, i: int, x: torch.Tensor, pair_row: torch.Tensor, k: int, rows: int) -> torch.Tensor:
        """Row-major codes of the permuted rows of ``x`` cast as tensor i, without the bf16 rows: the codes
        that ``cast`` gives for ``K.permute(x, pair_row, k, rows)`` when every row is filled."""
        return K.permute_fp8(x, pair_row, k, rows, self.history[i], FORMATS.get(i, "e4m3"), self.amax[i:i + 1],
                             self.scale_inv[i:i + 1], self.margin)

    def combine_bwd(self, i: int, dout: torch.Tensor, y: torch.Tensor, gates: torch.Tensor, pair_row: torch.Tensor,
                    rows: int) -> tuple[torch.Tensor, torch.Tensor]:
        """``K.combine_bwd`` with the row gradients cast as tensor i: (row-major codes, gate gradients)."""
        return K.combine_bwd_fp8(dout, y, gates, pair_row, rows, self.history[i], FORMATS.get(i, "e4m3"),
                                 self.amax[i:i + 1], self.scale_inv[i:i + 1], self.margin)

    def weight_codes(self, ws: list[torch.Tensor]) -> list[torch.Tensor]:
        """Uninitialised row-major e4m3 code buffers for expert weights (``cast_weights`` fills them)."""
        fdt = K.FP8_FORMATS["e4m3"][1]
        return [torch.empty(w.shape, dtype=fdt, device=w.device) for w in ws]

    def cast_weights(self, which: str, ws: list[torch.Tensor], qs: list[torch.Tensor]) -> None:
        """Row-major e4m3 codes of every local expert's fc1 (``which`` = "fc1") or fc2 weight into ``qs``, each
        with its own scale, in one launch."""
        rows = [self.w1(g) if which == "fc1" else self.w2(g) for g in range(self.G)]
        K.fp8_cast_many(list(ws), [self.history[i] for i in rows], "e4m3", [self.amax[i:i + 1] for i in rows],
                        [self.scale_inv[i:i + 1] for i in rows], qs, self.margin)

    def gemm_cast(self, i: int, epi: str, offsets: torch.Tensor, poff: torch.Tensor, rows_cap: int,
                  ys: list[torch.Tensor], y_fmt: str, xs: list[torch.Tensor], N: int, K_: int, f: int,
                  y_scale_inv: torch.Tensor, x_scale_inv: torch.Tensor, cs: list[torch.Tensor] | None = None,
                  auxs: list[torch.Tensor] | None = None, transposed: bool = True,
                  x_kn: bool = False) -> tuple[torch.Tensor, torch.Tensor | None]:
        """An fp8 product whose epilogue casts its activation output as tensor i (``K.fp8_gemm_cast``).

        Returns the (row-major, per-expert transposed or None) codes, equal to those of the product's bf16
        output cast with ``cast``.  ``x_kn``: the weights are the row-major codes held [K, N].
        """
        cols = 2 * N if epi == "swiglu_bwd" else N
        q, qt = self.codes(i, ys[0].shape[0], cols, rows_cap, offsets.numel() - 1, ys[0].device,
                           transposed=transposed)
        K.fp8_gemm_cast(epi, offsets, poff, rows_cap, ys, y_fmt, xs, "e4m3", N, K_, f, y_scale_inv, x_scale_inv,
                        self.history[i], FORMATS.get(i, "e4m3"), self.amax[i:i + 1], self.scale_inv[i:i + 1], q, qt,
                        cs=cs, auxs=auxs, margin=self.margin, x_kn=x_kn)
        return q, qt
