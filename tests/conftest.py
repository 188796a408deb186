"""Shared test setup.

* registers the ``gpu`` marker (tests that need an MI355X);
* puts the repo root on sys.path (for ``oracle`` and ``__graft_entry__``) and
  imports the package directory ``dflash-mlx_amd`` as ``dflash_mlx_amd``;
* never leaks DFLASH_* environment flags between tests (the reference's
  tests/test_verify_linear_parity.py:13 sets one at import time; here every
  test that needs a flag sets it through ``monkeypatch``).
"""

from __future__ import annotations

import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

import __graft_entry__  # noqa: E402

__graft_entry__.load_package()

_FLAGS = ("DFLASH_VERIFY_LINEAR", "DFLASH_VERIFY_QMM", "DFLASH_VERIFY_VARIANT",
          "DFLASH_VERIFY_QMM_KPARTS", "DFLASH_VERIFY_MAX_N", "DFLASH_VERIFY_INCLUDE")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(autouse=True)
def _clean_flags(monkeypatch):
    for name in _FLAGS:
        monkeypatch.delenv(name, raising=False)
    yield


@pytest.fixture(scope="session")
def dev():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from dflash_mlx_amd import _lib

    _lib.load()
    return torch.device("cuda:0")


# ---- numpy <-> torch helpers (bf16 carried as uint16 bit patterns) ----

def to_dev(a: np.ndarray, dtype: str, dev):
    """Oracle storage array -> GPU tensor of the matching torch dtype."""
    import torch

    a = np.ascontiguousarray(a)
    if dtype == "bf16":
        return torch.from_numpy(a.astype(np.uint16).view(np.int16)).view(torch.bfloat16).to(dev)
    if dtype == "f16":
        return torch.from_numpy(a.astype(np.float16)).to(dev)
    if dtype == "f32":
        return torch.from_numpy(a.astype(np.float32)).to(dev)
    if dtype == "u32":
        return torch.from_numpy(a.astype(np.uint32).view(np.int32)).to(dev)
    if dtype == "i32":
        return torch.from_numpy(a.astype(np.int32)).to(dev)
    raise ValueError(dtype)


def from_dev(t, dtype: str) -> np.ndarray:
    """GPU tensor -> oracle storage array."""
    import torch

    t = t.detach().cpu()
    if dtype == "bf16":
        return t.view(torch.int16).numpy().view(np.uint16)
    if dtype == "f16":
        return t.numpy().astype(np.float16)
    if dtype == "f32":
        return t.to(torch.float32).numpy()
    raise ValueError(dtype)


def make_qmm_case(M, K, N, gs=64, dtype="bf16", seed=0, x_std=1.0, w_std=0.02, bits=4):
    """Seeded inputs: x ~ N(0, x_std) and W ~ N(0, w_std) quantised with the
    oracle's MLX-rule restatement.  Returns storage arrays."""
    import oracle

    rng = np.random.default_rng(seed)
    xf = (rng.standard_normal((M, K)) * x_std).astype(np.float32)
    wf = (rng.standard_normal((N, K)) * w_std).astype(np.float32)
    x = oracle.round_to_dtype(xf, dtype)
    w_q, s, b = oracle.quantize(wf, gs, bits, out_dtype=dtype)
    return x, w_q, s, b
