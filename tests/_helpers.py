"""Shared helpers of the GPU parity tests (imported by test files; not a test module)."""

from __future__ import annotations

import sys

import numpy as np
import torch

DEV = "cuda:0"

# Max relative error bars: max|a - b| / max|b| against the float64 oracle.
TOL = {torch.bfloat16: 2e-2, torch.float32: 1e-5, torch.float64: 1e-10}


def say(msg: str) -> None:
    """Names the case on stdout before a GPU step (flushed, so it survives a crash)."""
    print(msg, flush=True)
    sys.stdout.flush()


def rel_err(a: torch.Tensor, b: torch.Tensor) -> float:
    a = a.detach().to("cpu", torch.float64)
    b = b.detach().to("cpu", torch.float64)
    if b.numel() == 0:
        return 0.0
    denom = b.abs().max().item()
    if denom == 0.0:
        return a.abs().max().item() if a.numel() else 0.0
    return (a - b).abs().max().item() / denom


def frob_err(a: torch.Tensor, b: torch.Tensor) -> float:
    """||a - b|| / ||b|| (Frobenius), the usual accuracy measure of fp8 training."""
    a = a.detach().to("cpu", torch.float64)
    b = b.detach().to("cpu", torch.float64)
    nb = b.norm().item()
    return (a - b).norm().item() / nb if nb else a.norm().item()


def bf16_bits(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def x_kind(dtype: torch.dtype) -> str:
    return {torch.bfloat16: "bf16", torch.float32: "f32", torch.float64: "f64"}[dtype]


def host_x(x: torch.Tensor) -> np.ndarray:
    """Token rows in the form the C oracle takes (raw bits for bfloat16)."""
    return bf16_bits(x) if x.dtype == torch.bfloat16 else x.detach().cpu().numpy()


def zipf_prior(E: int, s: float = 1.1) -> torch.Tensor:
    """Selection prior of a Zipf(s) expert popularity: -s * ln(e + 1)."""
    return -s * torch.log(torch.arange(1, E + 1, dtype=torch.float64))


def seeded(shape, seed: int, std: float = 1.0, dtype=torch.float32) -> torch.Tensor:
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(shape, generator=g, dtype=torch.float32) * std).to(dtype)
