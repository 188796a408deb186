"""The persistent stream-K matmul (tuning path 3) against the oracle.

Same bar as the dense tests: the reference's metric max|d| / (max|ref| +
1e-3) <= 1e-2 plus 2 output ulps element-wise around the exact result;
bit-exact on closed-form integer cases."""

from __future__ import annotations

import numpy as np
import pytest

import oracle
from tests.conftest import from_dev, make_qmm_case, to_dev

pytestmark = pytest.mark.gpu

REL_TOL = 1e-2


def _tuning(path):
    from dflash_mlx_amd import _lib

    return _lib.QmmTuning(path, 0, 0, 0)


def _run(dev, x, w_q, s, b, gs, dtype="bf16", path=3):
    import torch

    from dflash_mlx_amd import verify_qmm as vq

    y = vq.quantized_matmul(to_dev(x, dtype, dev), to_dev(w_q, "u32", dev), to_dev(s, dtype, dev),
                            to_dev(b, dtype, dev), group_size=gs, bits=4,
                            tuning=_tuning(path) if path else None)
    torch.cuda.synchronize()
    return from_dev(y, dtype)


def _check(got, x, w_q, s, b, gs, dtype="bf16"):
    ref = oracle.quantized_matmul(x, w_q, s, b, group_size=gs, bits=4, dtype=dtype)
    g = oracle.to_f32(got, dtype).astype(np.float64)
    _, rel = oracle.parity_metrics(g, ref)
    assert np.all(np.isfinite(g))
    assert rel <= REL_TOL, rel
    ulp = 2.0 ** -8 if dtype == "bf16" else 2.0 ** -11
    assert np.all(np.abs(g - ref) <= 2 * ulp * np.abs(ref) + 1e-4 * np.abs(ref).max())


def _kernel(M, K, N, gs=64, path=3):
    import ctypes

    from dflash_mlx_amd import _lib

    t = _tuning(path)
    name = _lib.load().dfmi_qmm_kernel_name(M, K, N, gs, 4, ctypes.byref(t))
    return name.decode() if name else None


@pytest.mark.parametrize("M,K,N", [
    (16, 5120, 5120),    # 40 blocks of 128 rows, 5 per XCD: ranges of 3-4 steps
    (16, 5120, 1024),    # 8 blocks, one per XCD: 20 one-step parts per block
    (16, 5120, 17408),   # 136 blocks: ranges of 10-11 steps across block ends
    (16, 17408, 5120),   # 68 steps per block: several window segments per range
    (16, 4096, 12288),   # 96 blocks
    (16, 5120, 34816),   # 272 blocks, 34 per XCD (fused gate/up size)
    (16, 12288, 4096)])  # 32 blocks, 48 steps
def test_persist_layer_shapes(dev, M, K, N):
    assert _kernel(M, K, N) == "qmm_persist_kernel"
    x, w_q, s, b = make_qmm_case(M, K, N, 64, seed=K + N + 7)
    _check(_run(dev, x, w_q, s, b, 64), x, w_q, s, b, 64)


@pytest.mark.parametrize("M", [1, 4, 9, 16])
@pytest.mark.parametrize("gs", [32, 64, 128])
@pytest.mark.parametrize("dtype", ["bf16", "f16"])
def test_persist_m_gs_dtype(dev, M, gs, dtype):
    # 2048 x 3000: ragged N (the last block's rows past N are clamped loads,
    # never stored), 24 blocks x 8 steps: one-step parts, 8 per block
    K, N = 2048, 3000
    x, w_q, s, b = make_qmm_case(M, K, N, gs, dtype=dtype, seed=M * 10 + gs)
    _check(_run(dev, x, w_q, s, b, gs, dtype), x, w_q, s, b, gs, dtype)


@pytest.mark.parametrize("K,N", [(1024, 70000), (2048, 20000), (1024, 13)])
def test_persist_many_units_and_tiny(dev, K, N):
    # 547 and 157 blocks (several whole blocks per range, four-step blocks
    # at K = 1024), and a single ragged block on one XCD (four one-step parts)
    x, w_q, s, b = make_qmm_case(16, K, N, 64, seed=K + N)
    _check(_run(dev, x, w_q, s, b, 64), x, w_q, s, b, 64)


def test_persist_closed_form_exact(dev):
    # scale 1/8, bias -1, sparse +-1 activations: exact in fp32 and bf16, so
    # whole units, parts and the split exchange must all be bit-exact
    rng = np.random.default_rng(43)
    M, K, gs = 16, 2048, 64
    for N in (64 * 300, 640, 96):
        q = rng.integers(0, 16, size=(N, K))
        w_q = oracle.pack(q, 4)
        s = oracle.f32_to_bf16_bits(np.full((N, K // gs), 0.125, np.float32))
        b = oracle.f32_to_bf16_bits(np.full((N, K // gs), -1.0, np.float32))
        xf = np.zeros((M, K), np.float32)
        for m in range(M):
            idx = rng.choice(K, size=6, replace=False)
            xf[m, idx] = rng.choice([-1.0, 1.0], size=6)
        x = oracle.f32_to_bf16_bits(xf)
        want = oracle.quantized_matmul(x, w_q, s, b, group_size=gs, out_dtype="bf16")
        assert np.array_equal(_run(dev, x, w_q, s, b, gs), want), N


def test_persist_deterministic(dev):
    x, w_q, s, b = make_qmm_case(16, 5120, 17408, 64, seed=3)
    first = _run(dev, x, w_q, s, b, 64)
    x2, w2, s2, b2 = make_qmm_case(16, 5120, 1024, 64, seed=4)
    for _ in range(3):
        _run(dev, x2, w2, s2, b2, 64)
        assert np.array_equal(_run(dev, x, w_q, s, b, 64), first)


def test_persist_rejects_outside_shapes(dev):
    assert _kernel(24, 2048, 256) is None      # M > 16
    assert _kernel(16, 1088, 256) is None      # K not a multiple of 256


def test_persist_single_step(dev):
    # K = 256 (group 32, so K holds whole 8-group pieces): one step per
    # block, every range one position
    x, w_q, s, b = make_qmm_case(16, 256, 3000, 32, seed=9)
    _check(_run(dev, x, w_q, s, b, 32), x, w_q, s, b, 32)
