"""Shared pytest setup: the ``gpu`` marker, repo-root imports and the package loader.

The product package lives in the directory ``resihp-megatron_amd/`` (a name
that is not a Python identifier); it is imported under the module name
``resihp_megatron_amd``.
"""

from __future__ import annotations

import importlib.util
import pathlib
import sys

import pytest

ROOT = pathlib.Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def load_package():
    name = "resihp_megatron_amd"
    if name in sys.modules:
        return sys.modules[name]
    pkg_dir = ROOT / "resihp-megatron_amd"
    spec = importlib.util.spec_from_file_location(name, pkg_dir / "__init__.py",
                                                  submodule_search_locations=[str(pkg_dir)])
    mod = importlib.util.module_from_spec(spec)
    sys.modules[name] = mod
    spec.loader.exec_module(mod)
    return mod


load_package()


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")
    config.addinivalue_line("markers", "slow: long-running test")


def gpu_available() -> bool:
    import torch

    return torch.cuda.is_available()


@pytest.fixture
def rng():
    import numpy as np

    return np.random.default_rng(12345)
