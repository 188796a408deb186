"""The pair-streaming gathers (dfmi_gather_qmm_affine_pairs /
dfmi_gather_qmm_swiglu_pairs, moe_stream_kernel) and their pair tables
(dfmi_moe_pairs).

The table layout is checked bit for bit against a numpy restatement; the
gathers against the oracle's products (same 1e-2 metric as every gather
test), against the plain gather entry points on the same inputs, and on the
edge cases the kernel's segment table has to get right: runs longer than 16
pairs, unsorted pairs, invalid ids (NaN rows), one pair, and the 256-pair
limit (257 pairs take the plain main loops)."""

from __future__ import annotations

import numpy as np
import pytest

import oracle
from oracle import moe as omoe

from .conftest import from_dev, to_dev
from .test_moe_gpu import _check, _experts, _x

pytestmark = pytest.mark.gpu


def _bits16(a, dtype):
    a = np.ascontiguousarray(a)
    return a.astype(np.float16).view(np.uint16) if dtype == "f16" else a.astype(np.uint16)


def _table(s, b, dtype, up=None):
    """numpy restatement of the dfmi_moe_pairs layout."""
    t = _bits16(s, dtype).astype(np.uint32) | (_bits16(b, dtype).astype(np.uint32) << 16)
    t = np.transpose(t, (0, 2, 1))  # [E][G][N]
    if up is None:
        return t
    tu = _bits16(up[0], dtype).astype(np.uint32) | (_bits16(up[1], dtype).astype(np.uint32) << 16)
    tu = np.transpose(tu, (0, 2, 1))
    E, G, N = t.shape
    out = np.empty((E, G, 2 * N), np.uint32)
    for n in range(N):
        out[:, :, 64 * (n // 32) + n % 32] = t[:, :, n]
        out[:, :, 64 * (n // 32) + 32 + n % 32] = tu[:, :, n]
    return out


def _dv(tr, dtype, dev):
    return (to_dev(tr[0], "u32", dev), to_dev(tr[1], dtype, dev), to_dev(tr[2], dtype, dev))


@pytest.mark.parametrize("dtype", ["bf16", "f16"])
@pytest.mark.parametrize("glu", [False, True])
def test_moe_pairs_layout(dev, dtype, glu):
    import torch

    from dflash_mlx_amd import _runtime

    E, N, K, gs = 3, 96, 640, 64  # 10 groups: a ragged 64-group tile
    _, s, b = _experts(E, N, K, gs, dtype, seed=31)
    _, su, bu = _experts(E, N, K, gs, dtype, seed=32)
    ts, tb = to_dev(s, dtype, dev), to_dev(b, dtype, dev)
    up = (to_dev(su, dtype, dev), to_dev(bu, dtype, dev)) if glu else None
    got = _runtime.build_moe_pairs(ts, tb, *(up or ()))
    torch.cuda.synchronize()
    want = _table(s, b, dtype, (su, bu) if glu else None)
    assert np.array_equal(got.cpu().numpy().view(np.uint32), want)


def _gather(dev, dtype, glu, x, gate, up, lhs, rhs, gs, use_pairs):
    import torch

    from dflash_mlx_amd.moe import gather_qmm, gather_swiglu

    xd = to_dev(x, dtype, dev)
    r = torch.tensor(rhs, device=dev)
    l_ = torch.tensor(lhs, device=dev) if lhs is not None else None
    if glu:
        out = gather_swiglu(xd, _dv(gate, dtype, dev), _dv(up, dtype, dev), r, lhs_indices=l_,
                            group_size=gs, use_pairs=use_pairs)
    else:
        out = gather_qmm(xd, *_dv(gate, dtype, dev), r, lhs_indices=l_, group_size=gs,
                         use_pairs=use_pairs)
    return from_dev(out, dtype)


def _want(x, gate, up, lhs, rhs, gs, dtype, glu):
    lhs = np.arange(len(rhs)) if lhs is None else lhs
    g = oracle.gather_qmm(x, *gate, lhs, rhs, group_size=gs, dtype=dtype)
    if not glu:
        return g
    u = oracle.gather_qmm(x, *up, lhs, rhs, group_size=gs, dtype=dtype)
    h = omoe._silu_mul(oracle.round_to_dtype(g, dtype), oracle.round_to_dtype(u, dtype), dtype)
    return oracle.to_f32(h, dtype)


@pytest.mark.parametrize("dtype", ["bf16", "f16"])
@pytest.mark.parametrize("gs", [64, 128])
@pytest.mark.parametrize("glu", [False, True])
@pytest.mark.parametrize("sort", [False, True])
def test_gather_pairs_matches_oracle(dev, dtype, gs, glu, sort):
    E, K, R, P = 10, 1024, 9, 40
    N = 192 if glu else 256
    gate = _experts(E, N, K, gs, dtype, seed=gs + 1)
    up = _experts(E, N, K, gs, dtype, seed=gs + 2) if glu else None
    x = _x(R, K, dtype, seed=5)
    rng = np.random.default_rng(11)
    rhs = rng.integers(0, E, size=P)
    lhs = rng.integers(0, R, size=P)
    if sort:
        order = np.argsort(rhs, kind="stable")
        rhs, lhs = rhs[order], lhs[order]
    got = _gather(dev, dtype, glu, x, gate, up, lhs, rhs, gs, True)
    want = _want(x, gate, up, lhs, rhs, gs, dtype, glu)
    _check(got, want, dtype)
    plain = _gather(dev, dtype, glu, x, gate, up, lhs, rhs, gs, False)
    _, rel = oracle.parity_metrics(oracle.to_f32(got, dtype), oracle.to_f32(plain, dtype))
    assert rel <= 1e-2
    again = _gather(dev, dtype, glu, x, gate, up, lhs, rhs, gs, True)
    assert np.array_equal(got, again)  # deterministic


@pytest.mark.parametrize("glu", [False, True])
def test_gather_pairs_long_runs_no_lhs(dev, glu):
    """Runs of 37 and 17 pairs (segments cut every 16 pairs), a run of one at
    the end, lhs_indices=None."""
    E, N, K = 4, 128, 512
    rhs = np.array([1] * 37 + [3] * 5 + [0] * 17 + [2])
    P = rhs.shape[0]
    gate = _experts(E, N, K, 64, "bf16", seed=9)
    up = _experts(E, N, K, 64, "bf16", seed=10) if glu else None
    x = _x(P, K, "bf16", seed=4)
    got = _gather(dev, "bf16", glu, x, gate, up, None, rhs, 64, True)
    _check(got, _want(x, gate, up, None, rhs, 64, "bf16", glu), "bf16")


@pytest.mark.parametrize("glu", [False, True])
def test_gather_pairs_invalid_ids_give_nan_rows(dev, glu):
    E, N, K, R = 3, 128, 256, 4
    gate = _experts(E, N, K, 64, "bf16", seed=1)
    up = _experts(E, N, K, 64, "bf16", seed=2) if glu else None
    x = _x(R, K, "bf16", seed=2)
    rhs = np.array([0, 7, 1, -1, 2, 2])
    lhs = np.array([0, 1, 9, 2, 3, -3])
    got = _gather(dev, "bf16", glu, x, gate, up, lhs, rhs, 64, True)
    g = oracle.to_f32(got, "bf16")
    assert np.isnan(g[[1, 2, 3, 5]]).all()
    good = [0, 4]
    _check(got[good], _want(x, gate, up, lhs[good], rhs[good], 64, "bf16", glu), "bf16")


@pytest.mark.parametrize("P", [1, 256, 257])
def test_gather_pairs_pair_counts(dev, P):
    """One pair (one unit per column block, two workgroups), the 256-pair
    limit of the kernel's LDS tables, and 257 pairs (the plain main loops)."""
    E, N, K, R = 64, 128, 512, 32
    gate = _experts(E, N, K, 64, "bf16", seed=P)
    up = _experts(E, N, K, 64, "bf16", seed=P + 1)
    x = _x(R, K, "bf16", seed=P + 2)
    rng = np.random.default_rng(P)
    rhs = np.sort(rng.integers(0, E, size=P))
    lhs = rng.integers(0, R, size=P)
    for glu in (False, True):
        got = _gather(dev, "bf16", glu, x, gate, up if glu else None, lhs, rhs, 64, True)
        _check(got, _want(x, gate, up, lhs, rhs, 64, "bf16", glu), "bf16")


def test_gather_pairs_explicit_table_and_cache(dev):
    """An explicit table gives the cached table's bits; the cache entry is
    rebuilt after an in-place update of the scales; a wrong table shape is
    rejected on the host."""
    import torch

    from dflash_mlx_amd import _runtime
    from dflash_mlx_amd.moe import gather_qmm

    E, N, K = 5, 128, 512
    wq, s, b = _experts(E, N, K, 64, "bf16", seed=3)
    x = _x(8, K, "bf16", seed=4)
    w_d, s_d, b_d = to_dev(wq, "u32", dev), to_dev(s, "bf16", dev), to_dev(b, "bf16", dev)
    rhs = torch.tensor([0, 0, 2, 4, 4, 4], device=dev)
    xd = to_dev(x, "bf16", dev)
    cached = gather_qmm(xd, w_d, s_d, b_d, rhs, group_size=64)
    table = _runtime.build_moe_pairs(s_d, b_d)
    explicit = gather_qmm(xd, w_d, s_d, b_d, rhs, group_size=64, pairs=table)
    assert torch.equal(cached, explicit)
    p0 = _runtime.PAIRS.get(s_d, b_d, experts=True)
    assert p0 is not None and _runtime.PAIRS.get(s_d, b_d, experts=True) is p0
    s_d.mul_(2)
    p1 = _runtime.PAIRS.get(s_d, b_d, experts=True)
    assert p1 is not p0
    with pytest.raises(ValueError):
        gather_qmm(xd, w_d, s_d, b_d, rhs, group_size=64, pairs=table[:, :, :64].contiguous())


@pytest.mark.parametrize("glu,E,K,N", [(True, 16, 2048, 256), (False, 16, 2048, 128),
                                       (False, 12, 1024, 256), (True, 256, 2048, 512),
                                       (False, 256, 512, 2048)])
def test_gather_pairs_tail_split(dev, glu, E, K, N):
    """Shapes whose last partial round of units is split along K (16 tokens
    top-8: every expert's run is one unit per column block): results match
    the oracle and the plain gathers, repeat bit for bit, and the workspace
    counters are back at zero."""
    import torch

    from dflash_mlx_amd import _lib, _runtime

    T, k = 16, 8
    gate = _experts(E, N, K, 64, "bf16", seed=E + K)
    up = _experts(E, N, K, 64, "bf16", seed=E + K + 1) if glu else None
    x = _x(T, K, "bf16", seed=N)
    rng = np.random.default_rng(E)
    inds = np.stack([rng.permutation(E)[:k] for _ in range(T)])
    flat = inds.reshape(-1)
    order = np.argsort(flat, kind="stable")
    rhs, lhs = flat[order], order // k
    got = _gather(dev, "bf16", glu, x, gate, up, lhs, rhs, 64, True)
    _check(got, _want(x, gate, up, lhs, rhs, 64, "bf16", glu), "bf16")
    plain = _gather(dev, "bf16", glu, x, gate, up, lhs, rhs, 64, False)
    _, rel = oracle.parity_metrics(oracle.to_f32(got, "bf16"), oracle.to_f32(plain, "bf16"))
    assert rel <= 1e-2
    for _ in range(3):
        assert np.array_equal(got, _gather(dev, "bf16", glu, x, gate, up, lhs, rhs, 64, True))
    torch.cuda.synchronize()
    ws = _runtime.WORKSPACES.get(torch.device(dev), int(_lib.load().dfmi_gather_workspace_bytes())
                                 + 256, "gather")
    off = (ws.data_ptr() + 255) // 256 * 256 - ws.data_ptr()  # the aligned workspace start
    assert int(ws[off:off + 4096].to(torch.int64).abs().sum()) == 0  # tail-split counters
