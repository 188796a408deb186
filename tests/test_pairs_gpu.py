"""GPU tests of the pair-streaming path: the (scale, bias) pair table
(``dfmi_sb_pairs``) and the streaming matmul reading it
(``dfmi_qmm_affine_pairs``, ``dfmi_qmm_affine_multi`` segments with a table).

The launch plan does not depend on the table, so with and without it the
result must be bit-identical on every plan (automatic, forced splits, whole
blocks + split pieces, ragged N, M < 16, both dtypes, both group sizes that
take it); the oracle checks (1e-2 metric) come from test_qmm_gpu.py, whose
calls use the table through the functional cache."""

from __future__ import annotations

import ctypes

import numpy as np
import pytest

import oracle
from tests.conftest import from_dev, make_qmm_case, to_dev

pytestmark = pytest.mark.gpu


def _lib():
    from dflash_mlx_amd import _lib as L

    return L


def _pairs(st, bt):
    from dflash_mlx_amd import _runtime

    return _runtime.build_sb_pairs(st, bt)


def _launch(dev, xt, wt, st, bt, pt, N, gs, tuning=None):
    """One dfmi_qmm_affine_pairs call with the given table (or none)."""
    import torch

    from dflash_mlx_amd import _runtime

    L = _lib()
    lib = L.load()
    M, K = int(xt.shape[0]), int(xt.shape[1])
    y = torch.full((M, N), float("nan"), dtype=xt.dtype, device=dev)
    tptr = ctypes.byref(tuning) if tuning is not None else None
    need = int(lib.dfmi_qmm_workspace_bytes_ex(M, K, N, gs, 4, tptr))
    ws, wsb = _runtime.workspace(dev, need) if need else (0, 0)
    rc = lib.dfmi_qmm_affine_pairs(xt.data_ptr(), _runtime.dtype_code(xt.dtype), wt.data_ptr(),
                                   st.data_ptr(), bt.data_ptr(),
                                   pt.data_ptr() if pt is not None else 0, y.data_ptr(), M, K, N,
                                   gs, 4, ws, wsb, tptr, _runtime.stream_ptr(dev))
    L.check(rc, "dfmi_qmm_affine_pairs")
    torch.cuda.synchronize()
    return y


def _case(dev, M, K, N, gs, dtype, seed):
    x, w_q, s, b = make_qmm_case(M, K, N, gs, dtype=dtype, seed=seed)
    return (x, w_q, s, b), (to_dev(x, dtype, dev), to_dev(w_q, "u32", dev),
                            to_dev(s, dtype, dev), to_dev(b, dtype, dev))


def _plan(M, K, Ns, gs, tuning=None):
    L = _lib()
    ns = (ctypes.c_int64 * len(Ns))(*Ns)
    info = L.QmmPlanInfo()
    tptr = ctypes.byref(tuning) if tuning is not None else None
    assert L.load().dfmi_qmm_plan(M, K, ns, len(Ns), gs, 4, tptr, ctypes.byref(info)) == 0
    return info


@pytest.mark.parametrize("N,G,dtype", [(1000, 70, "bf16"), (64, 1, "f16"), (65, 130, "bf16"),
                                       (5120, 80, "f16"), (7, 3, "bf16")])
def test_sb_pairs_layout(dev, N, G, dtype):
    import torch

    rng = np.random.default_rng(N + G)
    s = rng.standard_normal((N, G)).astype(np.float32)
    b = rng.standard_normal((N, G)).astype(np.float32)
    if dtype == "bf16":
        s16, b16 = oracle.f32_to_bf16_bits(s), oracle.f32_to_bf16_bits(b)
        st, bt = to_dev(s16, "bf16", dev), to_dev(b16, "bf16", dev)
        sbits, bbits = s16.astype(np.uint32), b16.astype(np.uint32)
    else:
        st, bt = to_dev(s, "f16", dev), to_dev(b, "f16", dev)
        sbits = s.astype(np.float16).view(np.uint16).astype(np.uint32)
        bbits = b.astype(np.float16).view(np.uint16).astype(np.uint32)
    pt = _pairs(st, bt)
    torch.cuda.synchronize()
    assert tuple(pt.shape) == (G, N)
    got = pt.cpu().numpy().view(np.uint32)
    want = (sbits | (bbits << 16)).T
    assert np.array_equal(got, want)


@pytest.mark.parametrize("M,K,N,gs", [
    (16, 4096, 4096, 64),        # 64 blocks: 4 splits, one workgroup per CU
    (16, 17408, 5120, 64),       # 68 steps: 6 splits, two per CU
    (16, 5120, 7168, 64),        # 27B q/k/v rows: 2 splits
    (16, 5120, 34816, 64),       # 544 blocks: 512 whole + 32 x 8 pieces
    (16, 5120, 512 * 64 + 6 * 64 - 51, 64),  # ragged N, 6 blocks x 20 one-step pieces
    (16, 2048, 40960, 64),       # 640 blocks: 512 whole + 128 x 2
    (16, 1024, 49152 + 70 * 64, 64),  # >= 768 blocks: 768 whole + 70 split over every slot
    (8, 12288, 4096, 64),
    (1, 2048, 1000, 128),
    (4, 5120, 5120, 128),
    (12, 4096, 12288, 64),
    # two activation blocks (M = 17..32)
    (32, 5120, 5120, 64),        # 80 blocks: 3 splits
    (32, 17408, 5120, 64),       # 68 steps: 6 splits, two per CU
    (24, 5120, 7168, 64),        # q/k/v rows: 2 splits
    (32, 5120, 34816, 64),       # 544 blocks: 512 whole + 32 x 8 pieces
    (17, 2048, 64 * 70 - 13, 128)])  # ragged N, gs 128
@pytest.mark.parametrize("dtype", ["bf16", "f16"])
def test_pairs_bit_identical_automatic_plans(dev, M, K, N, gs, dtype):
    host, (xt, wt, st, bt) = _case(dev, M, K, N, gs, dtype, seed=M * 7 + K + N)
    assert _plan(M, K, [N], gs).pair_streaming == 1
    y0 = _launch(dev, xt, wt, st, bt, None, N, gs)
    y1 = _launch(dev, xt, wt, st, bt, _pairs(st, bt), N, gs)
    a, b = from_dev(y0, dtype), from_dev(y1, dtype)
    assert np.array_equal(a, b)
    if N * K <= 64 << 20:  # and the oracle (the reference's metric) on the table's result
        ref = oracle.quantized_matmul(*host, group_size=gs, bits=4, dtype=dtype)
        _, rel = oracle.parity_metrics(oracle.to_f32(b, dtype).astype(np.float64), ref)
        assert rel <= 1e-2


@pytest.mark.parametrize("kp", [1, 2, 3, 5, 8])
def test_pairs_bit_identical_forced_splits(dev, kp):
    L = _lib()
    M, K, N, gs = 16, 5120, 3000, 64
    _, (xt, wt, st, bt) = _case(dev, M, K, N, gs, "bf16", seed=kp)
    t = L.QmmTuning(2, 0, 4, kp)
    info = _plan(M, K, [N], gs, t)
    assert (info.waves, info.k_splits, info.pair_streaming) == (4, kp, 1)
    y0 = _launch(dev, xt, wt, st, bt, None, N, gs, t)
    y1 = _launch(dev, xt, wt, st, bt, _pairs(st, bt), N, gs, t)
    assert np.array_equal(from_dev(y0, "bf16"), from_dev(y1, "bf16"))


@pytest.mark.parametrize("N,K,kp", [(5120, 5120, 3), (5120, 17408, 6), (7168, 5120, 2),
                                    (34816, 2048, 1), (1024, 4096, 8)])
def test_rows128_matches_rows64(dev, N, K, kp):
    """128-row blocks (two row groups of 4 wavefronts sharing the activation
    stage) give the same sums as 64-row blocks under the same K splits:
    bit-identical with the table, and without it (the 64-row equivalent the
    launcher runs)."""
    L = _lib()
    M, gs = 16, 64
    _, (xt, wt, st, bt) = _case(dev, M, K, N, gs, "bf16", seed=N + K + kp)
    pt = _pairs(st, bt)
    t128 = L.QmmTuning(0, 0, 0, kp, 128)
    t64 = L.QmmTuning(0, 0, 0, kp, 64)
    i128, i64 = _plan(M, K, [N], gs, t128), _plan(M, K, [N], gs, t64)
    assert (i128.rows_per_block, i128.waves, i128.k_splits) == (128, 8, kp)
    assert (i64.rows_per_block, i64.waves, i64.k_splits) == (64, 4, kp)
    ys = [from_dev(_launch(dev, xt, wt, st, bt, p, N, gs, t), "bf16")
          for (p, t) in ((pt, t128), (None, t128), (pt, t64), (None, t64))]
    for y in ys[1:]:
        assert np.array_equal(ys[0], y)


def test_pairs_closed_form_exact(dev):
    # dyadic scales / biases, +-1 activations: every product and sum is exact
    # in fp32, so the table path must reproduce the oracle bit for bit on a
    # whole + pieces plan
    rng = np.random.default_rng(51)
    M, K, N, gs = 16, 2048, 34816, 64  # 544 blocks: 512 whole + 32 x 8 pieces of one step
    q = rng.integers(0, 16, size=(N, K), dtype=np.uint8)
    w_q = oracle.pack(q, 4)
    s = oracle.f32_to_bf16_bits(rng.choice([0.125, 0.25, 0.5], size=(N, K // gs)).astype(np.float32))
    b = oracle.f32_to_bf16_bits(rng.choice([-1.0, -0.5, 0.0], size=(N, K // gs)).astype(np.float32))
    xf = np.zeros((M, K), np.float32)
    for m in range(M):
        xf[m, rng.choice(K, size=6, replace=False)] = rng.choice([-1.0, 1.0], size=6)
    x = oracle.f32_to_bf16_bits(xf)
    xt, wt, st, bt = (to_dev(x, "bf16", dev), to_dev(w_q, "u32", dev), to_dev(s, "bf16", dev),
                      to_dev(b, "bf16", dev))
    info = _plan(M, K, [N], gs)
    assert (info.whole_blocks, info.k_splits) == (512, 8)
    y = _launch(dev, xt, wt, st, bt, _pairs(st, bt), N, gs)
    want = oracle.quantized_matmul(x, w_q, s, b, group_size=gs, out_dtype="bf16")
    assert np.array_equal(from_dev(y, "bf16"), want)


@pytest.mark.parametrize("Ns", [(5120, 1024, 1024), (17408, 17408), (4096, 1024, 1024),
                                (12288, 12288), (300, 700, 64)])
def test_multi_pairs_bit_identical(dev, Ns):
    import torch

    from dflash_mlx_amd import _runtime

    L = _lib()
    lib = L.load()
    M, K, gs = 16, 5120 if Ns[0] in (5120, 17408, 300) else 4096, 64
    rng = np.random.default_rng(sum(Ns))
    xh = oracle.f32_to_bf16_bits(rng.standard_normal((M, K)).astype(np.float32))
    xt = to_dev(xh, "bf16", dev)
    mats = []
    for i, N in enumerate(Ns):
        _, (_, wt, st, bt) = _case(dev, 1, K, N, gs, "bf16", seed=1000 + i + N)
        mats.append((wt, st, bt, _pairs(st, bt)))
    n = len(Ns)
    ns = (ctypes.c_int64 * n)(*Ns)
    need = int(lib.dfmi_qmm_multi_workspace_bytes(M, K, ns, n, gs, 4))
    outs = []
    for use in (False, True):
        ys = [torch.full((M, N), float("nan"), dtype=torch.bfloat16, device=dev) for N in Ns]
        segs = (L.QmmSegment * n)()
        for i, ((wt, st, bt, pt), y) in enumerate(zip(mats, ys)):
            segs[i].w_q, segs[i].scales, segs[i].biases = wt.data_ptr(), st.data_ptr(), bt.data_ptr()
            segs[i].y, segs[i].N = y.data_ptr(), Ns[i]
            segs[i].sb_pairs = pt.data_ptr() if use else 0
        ws, wsb = _runtime.workspace(dev, need) if need else (0, 0)
        rc = lib.dfmi_qmm_affine_multi(xt.data_ptr(), 0, segs, n, M, K, gs, 4, ws, wsb,
                                       _runtime.stream_ptr(dev))
        L.check(rc, "dfmi_qmm_affine_multi")
        torch.cuda.synchronize()
        outs.append([from_dev(y, "bf16") for y in ys])
    for a, b in zip(*outs):
        assert np.array_equal(a, b)


def test_functional_cache_and_module_tables(dev):
    """verify_matmul builds the table once per (scales, biases) and rebuilds
    it after an in-place update; a module builds its own on first use."""
    import torch

    from dflash_mlx_amd import _runtime
    from dflash_mlx_amd import verify_qmm as vq

    host, (xt, wt, st, bt) = _case(dev, 16, 2048, 640, 64, "bf16", seed=3)
    y0 = vq.quantized_matmul(xt, wt, st, bt, group_size=64, bits=4)
    p0 = _runtime.PAIRS.get(st, bt)
    assert p0 is not None and _runtime.PAIRS.get(st, bt) is p0
    bt.mul_(0.5)  # in place: the cached table is stale
    p1 = _runtime.PAIRS.get(st, bt)
    assert p1 is not p0
    y1 = vq.quantized_matmul(xt, wt, st, bt, group_size=64, bits=4)
    x, w_q, s, b = host
    b_half = oracle.f32_to_bf16_bits(oracle.to_f32(b, "bf16") * 0.5)
    ref = oracle.quantized_matmul(x, w_q, s, b_half, group_size=64, bits=4, dtype="bf16")
    _, rel = oracle.parity_metrics(oracle.to_f32(from_dev(y1, "bf16"), "bf16").astype(np.float64),
                                   ref)
    assert rel <= 1e-2
    assert not torch.equal(y0, y1)


def _lmhead(dev, ht, wt, st, bt, pt, ids, M, K, V, gs, want_logits=True):
    """One dfmi_lmhead_greedy_accept_pairs call (with logits out unless
    want_logits is False)."""
    import torch

    from dflash_mlx_amd import _runtime

    L = _lib()
    lib = L.load()
    post = torch.full((M,), -1, dtype=torch.int32, device=dev)
    acc = torch.full((1,), -1, dtype=torch.int32, device=dev)
    bonus = torch.full((1,), -1, dtype=torch.int32, device=dev)
    logits = torch.full((M, V), float("nan"), dtype=ht.dtype, device=dev)
    ws, wsb = _runtime.workspace(dev, int(lib.dfmi_lmhead_workspace_bytes(M)), "greedy")
    rc = lib.dfmi_lmhead_greedy_accept_pairs(
        ht.data_ptr(), _runtime.dtype_code(ht.dtype), wt.data_ptr(), st.data_ptr(), bt.data_ptr(),
        pt.data_ptr() if pt is not None else 0, 0, 0.0, ids.data_ptr(), M, K, V, gs, 4,
        post.data_ptr(), acc.data_ptr(), bonus.data_ptr(),
        logits.data_ptr() if want_logits else 0, ws, wsb, _runtime.stream_ptr(dev))
    L.check(rc, "dfmi_lmhead_greedy_accept_pairs")
    torch.cuda.synchronize()
    return post.cpu().numpy(), int(acc.item()), int(bonus.item()), logits


@pytest.mark.parametrize("M,K,V,gs", [(16, 5120, 20000, 64), (15, 2048, 32000, 128),
                                      (16, 4096, 40000, 64), (1, 1024, 1000, 64),
                                      (16, 8192, 6000, 64), (16, 5120, 151936, 64),
                                      (7, 1024, 70037, 64), (16, 256, 3000, 128)])
def test_lmhead_pairs_identical(dev, M, K, V, gs):
    """The lm_head's pair-streaming sweep (128 vocabulary rows per
    workgroup; the full [16,5120]x[151936,5120] config, a ragged last block,
    one step per block at K = 256) gives the window loop's logits bit for
    bit, hence the same tokens, accept length and bonus, with or without the
    logits written out; a shape past one scale window (K = 8192 at gs 64:
    128 groups) takes the same general loop with or without the table."""
    import torch

    host, (ht, wt, st, bt) = _case(dev, M, K, V, gs, "bf16", seed=V + M)
    pt = _pairs(st, bt)
    r0 = _lmhead(dev, ht, wt, st, bt, None, torch.zeros(M, dtype=torch.int32, device=dev),
                 M, K, V, gs)
    # verify ids that accept part of the block: the window loop's own tokens
    ids = torch.tensor(np.concatenate([[0], r0[0][:M - 1]]).astype(np.int32), device=dev)
    if M > 4:
        ids[4] = (ids[4] + 1) % V  # break the chain after three accepted tokens
    r0 = _lmhead(dev, ht, wt, st, bt, None, ids, M, K, V, gs)
    r1 = _lmhead(dev, ht, wt, st, bt, pt, ids, M, K, V, gs)
    assert np.array_equal(r0[0], r1[0]) and r0[1:3] == r1[1:3]
    assert torch.equal(r0[3].view(torch.int16), r1[3].view(torch.int16))
    r2 = _lmhead(dev, ht, wt, st, bt, pt, ids, M, K, V, gs, want_logits=False)
    assert np.array_equal(r1[0], r2[0]) and r1[1:3] == r2[1:3]
    if M > 4:
        assert r1[1] == 3
    # and the oracle's greedy on the kernel's own logits
    lg = from_dev(r1[3], "bf16")
    want = oracle.greedy_tokens_with_mask(lg, None, dtype="bf16")
    assert np.array_equal(np.asarray(want).reshape(-1), r1[0].reshape(-1))
