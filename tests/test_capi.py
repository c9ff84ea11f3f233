"""The C ABI library: it loads, exports exactly what include/resihp_moe.h declares, and rejects
bad arguments with a message before touching the GPU (no kernel is launched in these tests)."""

from __future__ import annotations

import ctypes
import pathlib
import re

import pytest

from resihp_megatron_amd import _capi as C

HEADER = pathlib.Path(__file__).resolve().parent.parent / "include" / "resihp_moe.h"


def declared_symbols() -> set[str]:
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return set(re.findall(r"\b(rhp_\w+)\s*\(", text))


def test_library_exports_every_declared_symbol():
    L = C.lib()
    names = declared_symbols()
    assert len(names) >= 17
    for n in names:
        assert hasattr(L, n), n
    assert names == set(C.SIGNATURES), "ctypes signatures and header differ"


def test_abi_version_and_enums_match_header():
    text = HEADER.read_text()
    assert C.lib().rhp_abi_version() == int(re.search(r"#define RHP_ABI_VERSION (\d+)", text).group(1))
    assert int(re.search(r"#define RHP_MAX_GROUPS_PER_LAUNCH (\d+)", text).group(1)) == C.MAX_GROUPS_PER_LAUNCH
    enum = dict(re.findall(r"(RHP_\w+) = (\d+)", text))
    assert int(enum["RHP_BF16"]) == C.BF16 and int(enum["RHP_F64"]) == C.F64 and int(enum["RHP_E5M2"]) == C.E5M2
    assert int(enum["RHP_SCORE_SIGMOID"]) == C.SCORE_SIGMOID and int(enum["RHP_ACT_SWIGLU"]) == C.ACT_SWIGLU


@pytest.mark.parametrize("args,msg", [
    # k > E
    (dict(T=4, h=64, E=4, k=5, xd=C.BF16, rd=C.F32), "1 <= k"),
    # h not a multiple of 8
    (dict(T=4, h=60, E=4, k=2, xd=C.BF16, rd=C.F32), "multiple of 8"),
    # float64 model with a float32 router
    (dict(T=4, h=64, E=4, k=2, xd=C.F64, rd=C.F32), "float64 router"),
])
def test_route_rejects_bad_arguments(args, msg):
    fake = ctypes.c_void_p(4096)   # never dereferenced: validation fails first
    with pytest.raises(RuntimeError, match=msg):
        C.call("rhp_route", fake, args["xd"], fake, args["rd"], None, args["T"], args["h"], args["E"], args["k"],
               0, 1, 1.0, fake, fake, fake, None)


def test_dispatch_and_gemm_reject_bad_arguments():
    fake = ctypes.c_void_p(4096)
    with pytest.raises(RuntimeError, match="e0 < e1"):
        C.call("rhp_dispatch", fake, 10, 2, 8, 5, 5, 1, fake, fake, fake, fake, fake, fake, 1 << 20, None)
    with pytest.raises(RuntimeError, match="workspace"):
        C.call("rhp_dispatch", fake, 10, 2, 8, 0, 8, 1, fake, fake, fake, fake, fake, fake, 0, None)
    ptrs = C.ptr_array([4096])
    with pytest.raises(RuntimeError, match="at least one group"):
        C.call("rhp_expert_fc1_fwd", 0, fake, 1, 0, C.BF16, C.ACT_SWIGLU, 64, 64, ptrs, ptrs, ptrs, ptrs, None, 0,
               None)
    with pytest.raises(RuntimeError, match="unsupported dtype"):
        C.call("rhp_expert_fc2_fwd", 1, fake, 1, 0, C.E4M3, 64, 64, ptrs, ptrs, ptrs, None, 0, None)
    with pytest.raises(RuntimeError, match="split workspace"):
        C.call("rhp_expert_fc2_fwd", 1, fake, 1, 0, C.BF16, 64, 64, ptrs, ptrs, ptrs, fake, 1024, None)
    with pytest.raises(RuntimeError, match="split workspace"):
        C.call("rhp_expert_fc1_bwd", 1, fake, 1, 0, C.BF16, C.ACT_SWIGLU, 64, 64, ptrs, ptrs, ptrs, ptrs, ptrs,
               ctypes.c_void_p(4097), C.lib().rhp_expert_split_workspace_bytes(), None)
    with pytest.raises(RuntimeError, match="at most 8 shared"):
        C.call("rhp_combine", fake, fake, fake, C.F32, fake, fake, ptrs, 9, C.BF16, 4, 64, 2, fake, None)


def _gemm_cast(epi=1, q_fmt=C.E4M3, c=True, history=True, q=True, qt=True, margin=0, x_kn=0):
    fake = ctypes.c_void_p(4096)   # 16-byte aligned, never dereferenced: validation fails first
    C.call("rhp_fp8_gemm_cast", epi, 2, fake, fake, 512, C.E4M3, C.E4M3, 256, 256, 256, fake, 256, fake, 256, x_kn,
           fake if c else None, 512, fake, 512, fake, fake, 1, fake if history else None, 16, q_fmt, margin, fake,
           fake, fake if q else None, fake if qt else None, None)


@pytest.mark.parametrize("kw,msg", [
    (dict(epi=0), "activation forward or backward"),
    (dict(q_fmt=C.BF16), "RHP_E4M3 or RHP_E5M2"),
    (dict(history=False), "null pointer"),
    (dict(q=False, qt=False), "nothing to write"),
    (dict(margin=64), "bad history or margin"),
    (dict(epi=1, c=False), "store the pre-activation in c"),
    (dict(epi=3, c=True), "store no bf16 output"),
    (dict(epi=1, x_kn=1), r"\[K, N\] weights only with the backward"),
    (dict(epi=3, c=False, x_kn=2), "x_kn must be 0 or 1"),
])
def test_fp8_gemm_cast_rejects_bad_arguments(kw, msg):
    with pytest.raises(RuntimeError, match=msg):
        _gemm_cast(**kw)


def test_workspace_queries_are_pure():
    L = C.lib()
    assert L.rhp_dispatch_workspace_bytes(8192, 2, 8, 1) > 0
    assert L.rhp_dispatch_workspace_bytes(-1, 2, 8, 1) == 0
    a = L.rhp_router_wgrad_workspace_bytes(8192, 4096, 8, 2, C.F32)
    # one float32 row of partial sums per 64-row piece of each expert's segment (at most T k / 64 + E pieces)
    assert a == ((8192 * 2 + 63) // 64 + 8) * 4096 * 4
    assert L.rhp_router_wgrad_workspace_bytes(8192, 4096, 8, 2, C.F64) == 2 * a
    # K-split workspace: 8 XCDs x 32 CUs of one fp32 256 x 256 tile each, then one int32 counter per slot
    assert L.rhp_expert_split_workspace_bytes() == 256 * 256 * 256 * 4 + 256 * 4


def _row_codes(entry, fmt=C.E4M3, q=True, hist_len=16, margin=0, k=2, T=4, h=64):
    fake = ctypes.c_void_p(4096)   # 16-byte aligned, never dereferenced: validation fails first
    qp = fake if q else None
    if entry == "rhp_permute_fp8":
        C.call(entry, fake, T, h, k, fake, fmt, fake, hist_len, margin, fake, fake, qp, None)
    else:
        C.call(entry, fake, fake, fake, fake, T, h, k, fake, fmt, fake, hist_len, margin, fake, fake, qp, None)


@pytest.mark.parametrize("entry", ["rhp_permute_fp8", "rhp_combine_bwd_fp8"])
@pytest.mark.parametrize("kw,msg", [
    (dict(fmt=C.BF16), "RHP_E4M3 or RHP_E5M2"),
    (dict(q=False), "null code output"),
    (dict(hist_len=0), "bad history length or margin"),
    (dict(margin=64), "bad history length or margin"),
    (dict(h=60), "h must be a multiple of 8"),
    (dict(k=17), "1 <= k <= 16"),
])
def test_fp8_row_entries_reject_bad_arguments(entry, kw, msg):
    with pytest.raises(RuntimeError, match=msg):
        _row_codes(entry, **kw)


def test_combine_bwd_fp8_rejects_top_k_above_8():
    with pytest.raises(RuntimeError, match="top-k above 8"):
        _row_codes("rhp_combine_bwd_fp8", k=9)
