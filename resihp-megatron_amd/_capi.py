"""ctypes binding of the C ABI in ``include/resihp_moe.h`` (``libresihp_moe.so``).

Loading fails loudly: there is no CPU fallback.  Build the library first with
``python resihp-megatron_amd/build.py`` (``__graft_entry__.build()`` does it).
"""

from __future__ import annotations

import ctypes
import pathlib

LIB_PATH = pathlib.Path(__file__).resolve().parent / "libresihp_moe.so"

F64, F32, BF16, E4M3, E5M2 = 0, 1, 2, 3, 4
SCORE_SOFTMAX, SCORE_SIGMOID = 0, 1
ACT_GELU, ACT_SWIGLU = 0, 1
GEMM_KERNEL_GENERIC, GEMM_KERNEL_MFMA = 0, 1
MAX_GROUPS_PER_LAUNCH = 64

_p = ctypes.c_void_p
_i = ctypes.c_int
_i64 = ctypes.c_int64
_d = ctypes.c_double
_sz = ctypes.c_size_t
_pp = ctypes.POINTER(ctypes.c_void_p)
_pi64 = ctypes.POINTER(ctypes.c_int64)

# name -> (restype, argtypes); mirrors include/resihp_moe.h
SIGNATURES: dict[str, tuple[object, list]] = {
    "rhp_abi_version": (_i, []),
    "rhp_last_error": (ctypes.c_char_p, []),
    "rhp_route": (_i, [_p, _i, _p, _i, _p, _i64, _i, _i, _i, _i, _i, _d, _p, _p, _p, _p]),
    "rhp_dispatch_workspace_bytes": (_sz, [_i64, _i, _i, _i]),
    "rhp_dispatch": (_i, [_p, _i64, _i, _i, _i, _i, _i, _p, _p, _p, _p, _p, _p, _sz, _p]),
    "rhp_dispatch_noalloc": (_i, [_p, _i64, _i, _i, _i, _i, _i, _p, _p, _p, _p, _p, _p]),
    "rhp_update_expert_bias": (_i, [_p, _i, _p, _i, _d, _p]),
    "rhp_permute": (_i, [_p, _i, _i64, _i, _i, _p, _p, _p]),
    "rhp_combine": (_i, [_p, _p, _p, _i, _p, _p, _pp, _i, _i, _i64, _i, _i, _p, _p]),
    "rhp_combine_bwd": (_i, [_p, _p, _p, _i, _p, _i, _i64, _i, _i, _p, _p, _p]),
    "rhp_route_bwd": (_i, [_p, _p, _p, _p, _i, _i64, _i, _i, _i, _i, _d, _p, _p]),
    "rhp_token_bwd": (_i, [_p, _p, _p, _p, _p, _p, _i, _pp, _i, _i, _i64, _i, _i, _i, _p, _p]),
    "rhp_router_wgrad_workspace_bytes": (_sz, [_i64, _i, _i, _i, _i]),
    "rhp_router_wgrad": (_i, [_p, _p, _p, _p, _i, _i, _i64, _i, _i, _i, _p, _p, _sz, _p]),
    "rhp_ep_send_plan": (_i, [_p, _i64, _i, _i, _i, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p]),
    "rhp_recv_plan": (_i, [_p, _i, _i, _i64, _p, _p, _p, _p]),
    "rhp_gather_rows": (_i, [_p, _i, _i64, _i, _p, _i64, _p, _p]),
    "rhp_expert_split_workspace_bytes": (_sz, []),
    "rhp_expert_split_workspace_reset": (_i, [_p, _sz, _p]),
    "rhp_expert_gemm_kernel": (_i, [_i, _i, _i, _i]),
    "rhp_expert_fc1_fwd": (_i, [_i, _p, _i, _i64, _i, _i, _i, _i, _pp, _pp, _pp, _pp, _p, _sz, _p]),
    "rhp_expert_fc2_fwd": (_i, [_i, _p, _i, _i64, _i, _i, _i, _pp, _pp, _pp, _p, _sz, _p]),
    "rhp_expert_fc2_bwd": (_i, [_i, _p, _i, _i64, _i, _i, _i, _i, _pp, _pp, _pp, _pp, _pp, _pp, _p, _sz, _p]),
    "rhp_expert_fc1_bwd": (_i, [_i, _p, _i, _i64, _i, _i, _i, _i, _pp, _pp, _pp, _pp, _pp, _p, _sz, _p]),
    "rhp_expert_fc1_fwd_gather": (_i, [_i, _p, _i64, _i, _i, _i, _i, _p, _i64, _p, _pp, _p, _p, _p, _sz, _p]),
    "rhp_expert_fc2_fwd_scatter": (_i, [_i, _p, _i64, _i, _i, _i, _p, _pp, _p, _i64, _p, _p, _sz, _p]),
    "rhp_expert_fc2_dgrad_gather": (_i, [_i, _p, _i64, _i, _i, _i, _i, _p, _i64, _p, _p, _pp, _p, _p, _sz, _p]),
    "rhp_expert_fc1_dgrad_scatter": (_i, [_i, _p, _i64, _i, _i, _i, _i, _p, _pp, _p, _i64, _p, _p, _sz, _p]),
    "rhp_expert_fc1_dgrad_router": (_i, [_i, _p, _i64, _i, _i, _i, _i, _pp, _pp, _p, _i, _p, _p, _pp, _p, _sz, _p]),
    "rhp_adam_step": (_i, [_i, _pp, _pp, _pp, _pp, _p, _i, _d, _d, _d, _d, _d, _i64, _p]),
    "rhp_fp8_padded_offsets": (_i, [_p, _i, _i, _p, _p]),
    "rhp_fp8_cast": (_i, [_p, _i, _i64, _i, _i, _p, _p, _i64, _p, _i, _i, _i, _p, _p, _p, _p, _p]),
    "rhp_fp8_cast_many": (_i, [_i, _pp, _pi64, _pi64, _pp, _i, _i, _i, _pp, _pp, _pp, _p]),
    "rhp_fp8_amax_roll": (_i, [_p, _p, _i, _i, _p]),
    "rhp_permute_fp8": (_i, [_p, _i64, _i, _i, _p, _i, _p, _i, _i, _p, _p, _p, _p]),
    "rhp_combine_bwd_fp8": (_i, [_p, _p, _p, _p, _i64, _i, _i, _p, _i, _p, _i, _i, _p, _p, _p, _p]),
    "rhp_fp8_gemm": (_i, [_i, _i, _i, _p, _i64, _i, _i, _i, _i, _i, _i, _pp, _i64, _pp, _i64, _pp, _i64, _pp, _i64,
                          _pp, _i64, _p, _p, _i, _p]),
    "rhp_fp8_gemm_cast": (_i, [_i, _i, _p, _p, _i64, _i, _i, _i, _i, _i, _pp, _i64, _pp, _i64, _i, _pp, _i64, _pp,
                               _i64, _p, _p, _i, _p, _i, _i, _i, _p, _p, _p, _p, _p]),
}

_lib: ctypes.CDLL | None = None


def lib() -> ctypes.CDLL:
    """The loaded library; raises if it has not been built."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"{LIB_PATH.name} is not built; run `python resihp-megatron_amd/build.py` "
                               "(there is no CPU fallback for the MoE kernels)")
        L = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        if L.rhp_abi_version() != 1:
            raise RuntimeError("libresihp_moe.so ABI version mismatch; rebuild it")
        _lib = L
    return _lib


def call(name: str, *args) -> None:
    """Calls an entry point and turns a nonzero status into RuntimeError."""
    L = lib()
    rc = getattr(L, name)(*args)
    if rc != 0:
        msg = L.rhp_last_error().decode(errors="replace")
        raise RuntimeError(f"{name} failed: {msg}")


def ptr_array(ptrs) -> ctypes.Array:
    """Host array of device pointers (``const void* const*``)."""
    arr = (ctypes.c_void_p * max(1, len(ptrs)))()
    for i, p in enumerate(ptrs):
        arr[i] = p
    return arr
