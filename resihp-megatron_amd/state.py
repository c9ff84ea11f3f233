"""State contract of the MoE layer: stable tensor keys, shapes and holders.

Mirrors the parts of resihp/state/layer_registry.py:17-38 that the MoE layer
uses: ``TensorSpec(key, global_shape, dim, trainable)`` and the ``FULL`` slice.
Expert tensors are replicated slices (``dim=None``) keyed
``experts.{e}.fc{1,2}.weight``, so expert re-placement moves whole tensors by
key and the kernels see the same per-expert tensors before and after.
"""

from __future__ import annotations

from dataclasses import dataclass

FULL = (0, 1)

Holdings = dict[str, list[tuple[str, tuple[int, int]]]]


@dataclass(frozen=True)
class TensorSpec:
    key: str
    global_shape: tuple[int, ...]
    dim: int | None
    trainable: bool = True
    """Non-trainable tensors (router expert bias, FP8 amax histories) carry no optimizer state."""

    @property
    def extent(self) -> int:
        return self.global_shape[self.dim] if self.dim is not None else 1

    def local_shape(self, interval: tuple[int, int]) -> tuple[int, ...]:
        if self.dim is None:
            return self.global_shape
        shape = list(self.global_shape)
        shape[self.dim] = interval[1] - interval[0]
        return tuple(shape)


@dataclass(frozen=True)
class GroupSpec:
    """Name, member ranks and kind of a communication group (resihp/comm/group_spec.py)."""

    name: str
    ranks: tuple[int, ...]
    kind: str = "dp"
