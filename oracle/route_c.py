"""ctypes bridge to the C routing oracle (``oracle/route_ref.c``) -- test infrastructure only.

The shared library is built by ``make -C oracle`` (``__graft_entry__.build()``
runs it); if it is missing it is built here on first use.
"""

from __future__ import annotations

import ctypes
import pathlib
import subprocess

import numpy as np

_DIR = pathlib.Path(__file__).resolve().parent
_SO = _DIR / "_build" / "liboracle_route.so"
_lib = None

_i32p = np.ctypeslib.ndpointer(dtype=np.int32, flags="C_CONTIGUOUS")
_f32p = np.ctypeslib.ndpointer(dtype=np.float32, flags="C_CONTIGUOUS")
_f64p = np.ctypeslib.ndpointer(dtype=np.float64, flags="C_CONTIGUOUS")


def build() -> pathlib.Path:
    subprocess.run(["make", "-s", "-C", str(_DIR)], check=True)
    return _SO


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not _SO.exists():
            build()
        L = ctypes.CDLL(str(_SO))
        L.oracle_expf.restype = ctypes.c_float
        L.oracle_expf.argtypes = [ctypes.c_float]
        L.oracle_exp.restype = ctypes.c_double
        L.oracle_exp.argtypes = [ctypes.c_double]
        L.oracle_router_segment.argtypes = [ctypes.c_int]
        L.oracle_router_logits_f32.argtypes = [ctypes.c_void_p, ctypes.c_int, _f32p, ctypes.c_int64, ctypes.c_int,
                                               ctypes.c_int, _f32p]
        L.oracle_router_logits_f64.argtypes = [_f64p, _f64p, ctypes.c_int64, ctypes.c_int, ctypes.c_int, _f64p]
        for suf, fp, ft in (("f32", _f32p, ctypes.c_float), ("f64", _f64p, ctypes.c_double)):
            getattr(L, f"oracle_topk_{suf}").argtypes = [fp, ctypes.c_void_p, ctypes.c_int64, ctypes.c_int,
                                                         ctypes.c_int, ctypes.c_int, ctypes.c_int, ft, _i32p, fp]
        L.oracle_dispatch.argtypes = [_i32p, ctypes.c_int64, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                      ctypes.c_int, _i32p, _i32p, _i32p, _i32p, _i32p]
        _lib = L
    return _lib


def _check(rc: int, what: str) -> None:
    if rc != 0:
        raise ValueError(f"oracle {what} rejected its arguments (status {rc})")


def expf(x: float) -> float:
    return lib().oracle_expf(x)


def exp(x: float) -> float:
    return lib().oracle_exp(x)


def router_logits(x: np.ndarray, w: np.ndarray, x_kind: str) -> np.ndarray:
    """Fixed-order router logits.

    ``x_kind`` is ``"bf16"`` (``x`` holds raw uint16 bfloat16 bits), ``"f32"`` or
    ``"f64"``; ``w`` is float32 for the first two and float64 for the last.
    """
    T, h = x.shape
    E = w.shape[0]
    if x_kind == "f64":
        out = np.empty((T, E), np.float64)
        _check(lib().oracle_router_logits_f64(np.ascontiguousarray(x, np.float64),
                                              np.ascontiguousarray(w, np.float64), T, h, E, out), "logits")
        return out
    kind = {"f32": 1, "bf16": 2}[x_kind]
    xa = np.ascontiguousarray(x, np.uint16 if kind == 2 else np.float32)
    out = np.empty((T, E), np.float32)
    _check(lib().oracle_router_logits_f32(xa.ctypes.data, kind, np.ascontiguousarray(w, np.float32), T, h, E, out),
           "logits")
    return out


def topk(logits: np.ndarray, k: int, bias: np.ndarray | None = None, score: str = "softmax",
         normalize: bool = True, scale: float = 1.0) -> tuple[np.ndarray, np.ndarray]:
    """Lowest-id top-k with softmax or sigmoid gates, in the precision of ``logits``."""
    T, E = logits.shape
    f64 = logits.dtype == np.float64
    dt = np.float64 if f64 else np.float32
    lg = np.ascontiguousarray(logits, dt)
    b = None if bias is None else np.ascontiguousarray(bias, dt)
    topi = np.empty((T, k), np.int32)
    gates = np.empty((T, k), dt)
    fn = lib().oracle_topk_f64 if f64 else lib().oracle_topk_f32
    _check(fn(lg, None if b is None else b.ctypes.data, T, E, k, {"softmax": 0, "sigmoid": 1}[score],
              int(normalize), scale, topi, gates), "topk")
    return topi, gates


def dispatch(topi: np.ndarray, E: int, e0: int = 0, e1: int | None = None, n_src: int = 1) -> dict[str, np.ndarray]:
    """Counts, offsets, per-source counts and the stable expert-major permutation."""
    e1 = E if e1 is None else e1
    T, k = topi.shape
    L = e1 - e0
    out = {"counts": np.empty(E + 1, np.int32), "offsets": np.empty(L + 1, np.int32),
           "src_counts": np.empty((n_src, L), np.int32), "perm": np.empty(T * k, np.int32),
           "pair_row": np.empty(T * k, np.int32)}
    _check(lib().oracle_dispatch(np.ascontiguousarray(topi, np.int32), T, k, E, e0, e1, n_src, out["counts"],
                                 out["offsets"], out["src_counts"], out["perm"], out["pair_row"]), "dispatch")
    out["perm"] = out["perm"][: int(out["offsets"][-1])].copy()
    return out
