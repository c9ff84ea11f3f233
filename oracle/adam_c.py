"""ctypes bridge to the C Adam oracle (``oracle/adam_ref.c``) -- test infrastructure only.

One Adam step (resihp/runtime/optim.py:32-46) on numpy arrays in place:
float64, float32, or bfloat16 held as uint16 bit patterns.  The shared
library is built by ``make -C oracle``; if it is missing it is built here on
first use.
"""

from __future__ import annotations

import ctypes
import pathlib
import subprocess

import numpy as np

_DIR = pathlib.Path(__file__).resolve().parent
_SO = _DIR / "_build" / "liboracle_adam.so"
_lib = None
_KINDS = {np.dtype(np.float64): "f64", np.dtype(np.float32): "f32", np.dtype(np.uint16): "bf16"}


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not _SO.exists():
            subprocess.run(["make", "-s", "-C", str(_DIR)], check=True)
        L = ctypes.CDLL(str(_SO))
        for kind, dt in (("f64", np.float64), ("f32", np.float32), ("bf16", np.uint16)):
            arr = np.ctypeslib.ndpointer(dtype=dt, flags="C_CONTIGUOUS")
            fn = getattr(L, f"oracle_adam_{kind}")
            fn.restype = None
            fn.argtypes = [arr, ctypes.c_void_p, arr, arr, ctypes.c_int64, ctypes.c_double, ctypes.c_double,
                           ctypes.c_double, ctypes.c_double, ctypes.c_double, ctypes.c_int64]
        _lib = L
    return _lib


def adam_step(p: np.ndarray, grad: np.ndarray | None, m: np.ndarray, v: np.ndarray, lr: float, betas=(0.9, 0.999),
              eps: float = 1e-8, weight_decay: float = 0.0, step: int = 1) -> None:
    """Updates p, m, v in place (all the same dtype; grad None = no gradient)."""
    kind = _KINDS[p.dtype]
    for a in (m, v) + ((grad,) if grad is not None else ()):
        assert a.dtype == p.dtype and a.shape == p.shape and a.flags.c_contiguous
    g = None if grad is None else grad.ctypes.data_as(ctypes.c_void_p)
    getattr(lib(), f"oracle_adam_{kind}")(p, g, m, v, p.size, lr, betas[0], betas[1], eps, weight_decay, step)
