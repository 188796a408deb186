"""Routed-expert kernels vs the oracle (mx.gather_qmm / SwitchGLU / top-k
combine restated in oracle/moe.py and oracle/qmm.py).

gather_qmm parity is tolerance-based (the reference's arithmetic lives in
mlx, not vendored; parity against mlx itself is unpinned): the same metric
and 1e-2 bound as the dense qmm tests, on products that the oracle computes
in float64 from the same packed weights.  The combine is checked to within
one bf16 ulp (fp32 in-order accumulation vs float64).
"""

from __future__ import annotations

import numpy as np
import pytest

import oracle
from oracle import moe as omoe

from .conftest import from_dev, to_dev

pytestmark = pytest.mark.gpu

TOL = 1e-2


def _experts(E, N, K, gs, dtype, seed, w_std=0.02):
    rng = np.random.default_rng(seed)
    wq, ss, bb = [], [], []
    for _ in range(E):
        w = (rng.standard_normal((N, K)) * w_std).astype(np.float32)
        q, s, b = oracle.quantize(w, gs, 4, out_dtype=dtype)
        wq.append(q)
        ss.append(s)
        bb.append(b)
    return np.stack(wq), np.stack(ss), np.stack(bb)


def _x(R, K, dtype, seed):
    rng = np.random.default_rng(seed)
    return oracle.round_to_dtype(rng.standard_normal((R, K)).astype(np.float32), dtype)


def _check(got, want, dtype):
    _, rel = oracle.parity_metrics(oracle.to_f32(got, dtype), want)
    assert rel <= TOL, rel


@pytest.mark.parametrize("dtype", ["bf16", "f16"])
@pytest.mark.parametrize("gs", [32, 64, 128])
@pytest.mark.parametrize("sort", [False, True])
def test_gather_qmm_matches_oracle(dev, dtype, gs, sort):
    import torch

    from dflash_mlx_amd.moe import gather_qmm

    E, N, K, R, P = 12, 96, 512, 9, 40
    wq, s, b = _experts(E, N, K, gs, dtype, seed=gs)
    x = _x(R, K, dtype, seed=5)
    rng = np.random.default_rng(11)
    rhs = rng.integers(0, E, size=P)
    lhs = rng.integers(0, R, size=P)
    if sort:
        order = np.argsort(rhs, kind="stable")
        rhs, lhs = rhs[order], lhs[order]
    want = oracle.gather_qmm(x, wq, s, b, lhs, rhs, group_size=gs, dtype=dtype)
    got = gather_qmm(to_dev(x, dtype, dev), to_dev(wq, "u32", dev), to_dev(s, dtype, dev),
                     to_dev(b, dtype, dev), torch.tensor(rhs, device=dev),
                     lhs_indices=torch.tensor(lhs, device=dev), group_size=gs)
    _check(from_dev(got, dtype), want, dtype)


@pytest.mark.parametrize("K,N,gs", [
    (320, 40, 32),     # general loop, ragged K (tail chunk) and N
    (2048, 512, 64),   # persistent loop (the expert gate/up shape)
    (1536, 200, 64),   # persistent loop, 3 steps per unit, ragged N
    (2048, 512, 32),   # streaming loop (64 groups: past the persistent window)
    (512, 2048, 64),   # general loop (the expert down shape)
    (96, 16, 32)])
def test_gather_qmm_shapes(dev, K, N, gs):
    """Every gather main loop, ragged K and N, and the MoE expert shapes."""
    import torch

    from dflash_mlx_amd.moe import gather_qmm

    E, R, P = 6, 16, 24
    wq, s, b = _experts(E, N, K, gs, "bf16", seed=K + N)
    x = _x(R, K, "bf16", seed=3)
    rhs = np.sort(np.random.default_rng(K).integers(0, E, size=P))
    want = oracle.gather_qmm(x, wq, s, b, np.arange(P) % R, rhs, group_size=gs)
    got = gather_qmm(to_dev(x, "bf16", dev), to_dev(wq, "u32", dev), to_dev(s, "bf16", dev),
                     to_dev(b, "bf16", dev), torch.tensor(rhs, device=dev),
                     lhs_indices=torch.tensor(np.arange(P) % R, device=dev), group_size=gs)
    _check(from_dev(got, "bf16"), want, "bf16")


@pytest.mark.parametrize("K", [256, 1024])  # general and persistent main loops
def test_gather_qmm_long_runs(dev, K):
    """Runs of more than 16 pairs on one expert (several MFMA row blocks), and
    lhs_indices=None (row p for pair p)."""
    import torch

    from dflash_mlx_amd.moe import gather_qmm

    E, N = 4, 64
    rhs = np.array([1] * 37 + [3] * 5 + [0] * 17 + [2])
    P = rhs.shape[0]
    wq, s, b = _experts(E, N, K, 64, "bf16", seed=9)
    x = _x(P, K, "bf16", seed=4)
    want = oracle.gather_qmm(x, wq, s, b, np.arange(P), rhs, group_size=64)
    got = gather_qmm(to_dev(x, "bf16", dev), to_dev(wq, "u32", dev), to_dev(s, "bf16", dev),
                     to_dev(b, "bf16", dev), torch.tensor(rhs, device=dev), group_size=64)
    _check(from_dev(got, "bf16"), want, "bf16")


@pytest.mark.parametrize("K", [256, 1024])  # general and persistent main loops
def test_gather_qmm_invalid_ids_give_nan_rows(dev, K):
    import torch

    from dflash_mlx_amd.moe import gather_qmm

    E, N, R = 3, 32, 4
    wq, s, b = _experts(E, N, K, 64, "bf16", seed=1)
    x = _x(R, K, "bf16", seed=2)
    rhs = np.array([0, 7, 1, -1, 2, 2])
    lhs = np.array([0, 1, 9, 2, 3, -3])
    got = gather_qmm(to_dev(x, "bf16", dev), to_dev(wq, "u32", dev), to_dev(s, "bf16", dev),
                     to_dev(b, "bf16", dev), torch.tensor(rhs, device=dev),
                     lhs_indices=torch.tensor(lhs, device=dev), group_size=64)
    g = oracle.to_f32(from_dev(got, "bf16"), "bf16")
    bad = [1, 2, 3, 5]
    assert np.isnan(g[bad]).all()
    good = [0, 4]
    want = oracle.gather_qmm(x, wq, s, b, lhs[good], rhs[good], group_size=64)
    _check(from_dev(got, "bf16")[good], want, "bf16")


@pytest.mark.parametrize("T,k,E,D,I", [(4, 2, 8, 256, 128), (16, 8, 32, 2048, 512),
                                       (5, 3, 6, 1024, 192),
                                       (16, 8, 128, 1024, 256)])  # ~1 routed row per expert
def test_switch_glu_matches_oracle(dev, T, k, E, D, I):
    import torch

    from dflash_mlx_amd.moe import switch_glu

    gate = _experts(E, I, D, 64, "bf16", seed=21)
    up = _experts(E, I, D, 64, "bf16", seed=22)
    down = _experts(E, D, I, 64, "bf16", seed=23)
    x = _x(T, D, "bf16", seed=24)
    logits = np.random.default_rng(7).standard_normal((T, E)).astype(np.float32)
    inds, _ = omoe.route_topk(logits, k)
    h_want, y_want = omoe.switch_glu(x, inds, gate, up, down, group_size=64, dtype="bf16")

    def dv(tr):
        return (to_dev(tr[0], "u32", dev), to_dev(tr[1], "bf16", dev), to_dev(tr[2], "bf16", dev))

    h, y = switch_glu(to_dev(x, "bf16", dev), torch.tensor(inds, device=dev), dv(gate), dv(up),
                      dv(down), group_size=64)
    # h: same products, each rounded to bf16 before the op-by-op SwiGLU
    _check(from_dev(h, "bf16"), oracle.to_f32(h_want, "bf16"), "bf16")
    _check(from_dev(y, "bf16"), oracle.to_f32(y_want, "bf16"), "bf16")


@pytest.mark.parametrize("T,k,D", [(16, 8, 2048), (3, 2, 100), (1, 1, 7), (4, 10, 2048),
                                   (2, 3, 16)])
def test_moe_combine(dev, T, k, D):
    import torch

    from dflash_mlx_amd.moe import moe_combine

    rng = np.random.default_rng(T * k + D)
    y = oracle.round_to_dtype(rng.standard_normal((T * k, D)).astype(np.float32), "bf16")
    sc = rng.random((T, k)).astype(np.float32)
    sc /= sc.sum(axis=1, keepdims=True)
    want = omoe.moe_combine(y, sc, dtype="bf16", out_dtype="bf16")
    got = from_dev(moe_combine(to_dev(y, "bf16", dev), torch.tensor(sc, device=dev)), "bf16")
    diff = np.abs(got.astype(np.int32) - want.astype(np.int32))
    assert diff.max() <= 1
    assert (diff == 0).mean() > 0.99


@pytest.mark.parametrize("T,k,D", [(16, 8, 2048), (3, 2, 100), (4, 10, 520)])
def test_moe_combine_unsort(dev, T, k, D):
    """y handed over in a permuted (expert-sorted) order with y_rows = the
    inverse permutation gives the same bits as the combine over y in pair
    order; a row id out of range makes only its token's output NaN."""
    import torch

    from dflash_mlx_amd.moe import moe_combine

    rng = np.random.default_rng(100 + T * k + D)
    y = oracle.round_to_dtype(rng.standard_normal((T * k, D)).astype(np.float32), "bf16")
    sc = rng.random((T, k)).astype(np.float32)
    sc /= sc.sum(axis=1, keepdims=True)
    order = rng.permutation(T * k)
    inv = np.empty_like(order)
    inv[order] = np.arange(T * k)
    want = omoe.moe_combine(y, sc, dtype="bf16", out_dtype="bf16")
    scd = torch.tensor(sc, device=dev)
    plain = from_dev(moe_combine(to_dev(y, "bf16", dev), scd), "bf16")
    y_sorted = to_dev(y[order], "bf16", dev)
    rows = torch.tensor(inv, dtype=torch.int32, device=dev)
    got = from_dev(moe_combine(y_sorted, scd, y_rows=rows), "bf16")
    assert np.array_equal(got, plain)
    diff = np.abs(got.astype(np.int32) - want.astype(np.int32))
    assert diff.max() <= 1
    bad = rows.clone()
    bad[k * (T - 1)] = T * k  # first pair of the last token
    out = oracle.to_f32(from_dev(moe_combine(y_sorted, scd, y_rows=bad), "bf16"), "bf16")
    assert np.isnan(out[T - 1]).all()
    assert np.array_equal(from_dev(moe_combine(y_sorted, scd, y_rows=bad), "bf16")[: T - 1],
                          got[: T - 1])


def test_empty_calls(dev):
    """Zero tokens: no pairs, no activation rows; every MoE operator returns
    empty results without a launch."""
    import torch

    from dflash_mlx_amd.moe import gather_qmm, gather_swiglu, moe_combine

    E, N, K = 3, 32, 256
    wq, s, b = _experts(E, N, K, 64, "bf16", seed=1)
    tr = (to_dev(wq, "u32", dev), to_dev(s, "bf16", dev), to_dev(b, "bf16", dev))
    x = torch.empty((0, K), dtype=torch.bfloat16, device=dev)
    rhs = torch.empty((0,), dtype=torch.int32, device=dev)
    assert tuple(gather_qmm(x, *tr, rhs, group_size=64).shape) == (0, N)
    assert tuple(gather_swiglu(x, tr, tr, rhs, group_size=64).shape) == (0, N)
    y = torch.empty((0, N), dtype=torch.bfloat16, device=dev)
    sc = torch.empty((0, 2), dtype=torch.float32, device=dev)
    assert tuple(moe_combine(y, sc).shape) == (0, N)
    torch.cuda.synchronize()
