"""Write the reference's own float64 outputs as small fixtures for the oracle tests.

Run in the build container, where the reference checkout is mounted:

    python tests/golden/make_reference_vectors.py /root/reference

It imports ``resihp.runtime.moe`` (resihp/runtime/moe.py) and
``resihp.state.rng_data`` from that checkout and records, for the reference's
own ``MoEConfig`` defaults (with and without the aux-loss-free bias) and one
larger GELU shape:

* ``derive_seed`` on a few part tuples and ``init_param`` of ``router.weight``;
* ``route`` (top-k indices and gates) on ``batch(cfg, 0)``;
* ``reference_forward`` output, the expert bias after the in-forward update, and
  the gradients of ``token_loss / tokens`` with respect to ``x`` and every
  parameter;
* the per-iteration losses and final parameters of ``reference_train``.

These pin the float64 restatement in ``oracle/moe_ref.py``; nothing else in the
reference's tests does (it stores no golden tensors).  The output is
``tests/golden/reference_moe.npz`` (float64 / int64 arrays, no pickles).
"""

from __future__ import annotations

import pathlib
import sys

import numpy as np


def main(ref_root: str) -> None:
    sys.path.insert(0, ref_root)
    import torch

    from resihp.runtime.moe import (MoEConfig, batch, init_param, moe_specs, reference_forward, reference_train,
                                    route, token_loss)
    from resihp.state.rng_data import derive_seed

    torch.set_num_threads(1)
    out: dict[str, np.ndarray] = {}
    parts = [(0,), (1, 2, 3), (4321, 0, 5), (4321, 3), (2**63 + 5, 7)]
    out["derive_seed_parts"] = np.array([",".join(str(v) for v in p) for p in parts]).astype(np.bytes_)
    out["derive_seed_values"] = np.array([str(derive_seed(*p)) for p in parts]).astype(np.bytes_)

    cases = {
        "default": MoEConfig(),
        "bias": MoEConfig(bias_update_rate=0.01),
        "wide": MoEConfig(hidden=16, ffn=32, num_experts=8, top_k=3, tokens=64, seed=77, bias_update_rate=0.05),
    }
    for name, cfg in cases.items():
        specs = moe_specs(cfg)
        params = {k: init_param(cfg, s) for k, s in specs.items()}
        out[f"{name}/init/router.weight"] = params["router.weight"].numpy()
        x, y = batch(cfg, 0)
        out[f"{name}/x"] = x.numpy()
        out[f"{name}/y"] = y.numpy()
        topi, gates = route(cfg, x, params["router.weight"], params.get("router.expert_bias"))
        out[f"{name}/route/topi"] = topi.numpy()
        out[f"{name}/route/gates"] = gates.numpy()
        leaves = {k: torch.nn.Parameter(v.clone()) for k, v in params.items() if specs[k].trainable}
        bufs = {k: v.clone() for k, v in params.items() if not specs[k].trainable}
        xl = x.clone().requires_grad_(True)
        fwd = reference_forward(cfg, {**leaves, **bufs}, xl)
        (token_loss(fwd, y) / cfg.tokens).backward()
        out[f"{name}/fwd/out"] = fwd.detach().numpy()
        out[f"{name}/fwd/grad/x"] = xl.grad.numpy()
        for k, p in leaves.items():
            out[f"{name}/fwd/grad/{k}"] = p.grad.numpy()
        for k, b in bufs.items():
            out[f"{name}/fwd/after/{k}"] = b.numpy()
        losses, final = reference_train(cfg, 8)
        out[f"{name}/train/losses"] = np.array(losses, dtype=np.float64)
        for k, v in final.items():
            out[f"{name}/train/final/{k}"] = v.numpy()

    dest = pathlib.Path(__file__).resolve().parent / "reference_moe.npz"
    np.savez_compressed(dest, **out)
    print(f"wrote {dest} ({dest.stat().st_size} bytes, {len(out)} arrays)")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
