"""rhp_dispatch_noalloc (the dispatch plan with the library's own fixed scratch array, no allocation)
against rhp_dispatch with a caller workspace, through the C ABI.

Two calls in a row on one GPU, the second smaller, each bit-exact with the workspace entry point; a
size past the 4 MiB scratch is rejected before any launch.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from _helpers import DEV, say
from resihp_megatron_amd import _capi as C
from resihp_megatron_amd import kernels as K

pytestmark = pytest.mark.gpu


def _outputs(T, k, E, e0, e1, n_src):
    z = lambda *s: torch.full(s, -7, dtype=torch.int32, device=DEV)  # noqa: E731
    return dict(counts=z(E + 1), offsets=z(e1 - e0 + 1), src_counts=z(n_src, e1 - e0), perm=z(max(1, T * k)),
                pair_row=z(max(1, T * k)))


def _noalloc(topi, E, e0, e1, n_src):
    T, k = topi.shape
    o = _outputs(T, k, E, e0, e1, n_src)
    with torch.cuda.device(DEV):
        C.call("rhp_dispatch_noalloc", topi.data_ptr(), T, k, E, e0, e1, n_src, o["counts"].data_ptr(),
               o["offsets"].data_ptr(), o["src_counts"].data_ptr(), o["perm"].data_ptr(), o["pair_row"].data_ptr(),
               torch.cuda.current_stream(DEV).cuda_stream)
    return o


def _topi(T, k, E, seed):
    rng = np.random.default_rng(seed)
    ids = np.stack([rng.choice(E, k, replace=False) for _ in range(T)]).astype(np.int32)
    ids[rng.random((T, k)) < 0.01] = -1          # a few invalid ids, counted in counts[E]
    return torch.from_numpy(ids).to(DEV)


@pytest.mark.parametrize("first,second", [((32768, 8, 128, (0, 16), 8), (3000, 8, 128, (112, 128), 3)),
                                          ((8192, 2, 8, (0, 8), 1), (700, 2, 8, (2, 5), 2))])
def test_noalloc_dispatch_matches_workspace_dispatch(first, second):
    for T, k, E, (e0, e1), n_src in (first, second):
        topi = _topi(T, k, E, T)
        say(f"dispatch noalloc T={T} k={k} E={E} window=[{e0},{e1}) n_src={n_src}")
        ref = K.dispatch(topi, E, e0, e1, n_src)
        got = _noalloc(topi, E, e0, e1, n_src)
        torch.cuda.synchronize()
        P = int(ref.offsets[-1])
        for name in ("counts", "offsets", "src_counts"):
            assert torch.equal(got[name].view(-1), getattr(ref, name).view(-1)), name
        assert torch.equal(got["perm"][:P], ref.perm[:P])
        assert torch.equal(got["pair_row"][:T * k], ref.pair_row)


def test_noalloc_dispatch_rejects_sizes_past_its_scratch():
    T, k, E = 300000, 8, 1024
    need = C.lib().rhp_dispatch_workspace_bytes(T, k, E, 1)
    assert need > 4 << 20
    topi = torch.zeros(T, k, dtype=torch.int32, device=DEV)
    say("dispatch noalloc past its scratch")
    with pytest.raises(RuntimeError, match="4 MiB"):
        _noalloc(topi, E, 0, E, 1)
