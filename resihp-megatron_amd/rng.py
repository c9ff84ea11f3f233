"""Counter-based seeds: every parameter and batch is a pure function of its identity.

Mirrors resihp/state/rng_data.py:21-38 (same algorithm and values): a part tuple
is folded through the SplitMix64 finaliser and seeds a CPU ``torch.Generator``.
Values are always drawn on the CPU and then moved, so every device and every
placement sees identical numbers.
"""

from __future__ import annotations

import torch

_MASK64 = (1 << 64) - 1


def splitmix64(x: int) -> int:
    x = (x + 0x9E3779B97F4A7C15) & _MASK64
    x = ((x ^ (x >> 30)) * 0xBF58476D1CE4E5B9) & _MASK64
    x = ((x ^ (x >> 27)) * 0x94D049BB133111EB) & _MASK64
    return x ^ (x >> 31)


def derive_seed(*parts: int) -> int:
    h = 0
    for p in parts:
        h = splitmix64(h ^ (int(p) & _MASK64))
    return h & ((1 << 63) - 1)


def generator(*parts: int) -> torch.Generator:
    g = torch.Generator(device="cpu")
    g.manual_seed(derive_seed(*parts))
    return g
