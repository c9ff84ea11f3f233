"""MI355X-native (gfx950) MoE expert-parallel layer hot path of ResiHP-Megatron.

A drop-in for resihp/runtime/moe.py: the same Python API (``moe`` module) on
top of hand-written HIP kernels reached through the C ABI of
``libresihp_moe.so`` (declared in ``include/resihp_moe.h``):

* ``moe``        -- MoEConfig, route, expert_ffn, reference_forward, reference_train, EPRuntime, ...
* ``layer``      -- the fused autograd layer (route, dispatch, permute, grouped GEMMs, combine)
* ``kernels``    -- torch-facing wrappers of each C entry point
* ``build``      -- hipcc recipe for the shared library
"""

from . import placement, rng, state  # noqa: F401

__all__ = ["build", "kernels", "layer", "moe", "placement", "rng", "state"]
