"""Prepared launches (dfmi_qmm_prepare / dfmi_qmm_run) through the C ABI:
bit-identical to the one-shot entry points they stand for
(dfmi_qmm_affine_pairs, dfmi_qmm_affine_multi, dfmi_qmm_affine_multi_fused),
including a matrix that reads its column slice of a wider pair table
(sb_stride), shapes outside the streaming kernel, repeated runs over the same
workspace, and the 1e-2 oracle bar.  The reference computes a module's route
once and launches it from a closure per call
(dflash_mlx/verify_linear.py:118-309); the results must not depend on that
choice."""

from __future__ import annotations

import ctypes

import numpy as np
import pytest

import oracle
from tests.conftest import from_dev, make_qmm_case, to_dev

pytestmark = pytest.mark.gpu

REL_TOL = 1e-2


def _case(dev, M, K, Ns, gs, dtype, seed):
    cases = [make_qmm_case(M, K, N, gs, dtype=dtype, seed=seed + i) for i, N in enumerate(Ns)]
    x = to_dev(cases[0][0], dtype, dev)
    mats = [(to_dev(c[1], "u32", dev), to_dev(c[2], dtype, dev), to_dev(c[3], dtype, dev))
            for c in cases]
    return cases, x, mats


def _one_shot_multi(dev, x, mats, tables, fused, M, K, gs, bits=4):
    """dfmi_qmm_affine_multi(_fused) with a fresh zeroed workspace."""
    import torch

    from dflash_mlx_amd import _lib, _runtime

    lib = _lib.load()
    n = len(mats)
    Ns = [int(w.shape[0]) for (w, _, _) in mats]
    ns = (ctypes.c_int64 * n)(*Ns)
    need = int(lib.dfmi_qmm_multi_workspace_bytes(M, K, ns, n, gs, bits))
    ws = torch.zeros(need + 256, dtype=torch.uint8, device=dev)
    wsp = (ws.data_ptr() + 255) // 256 * 256 if need else 0
    ys = [torch.full((M, N), float("nan"), dtype=x.dtype, device=dev) for N in Ns]
    segs = (_lib.QmmSegment * n)()
    for i, ((w, s, b), y) in enumerate(zip(mats, ys)):
        segs[i].w_q, segs[i].scales, segs[i].biases = w.data_ptr(), s.data_ptr(), b.data_ptr()
        segs[i].y, segs[i].N = y.data_ptr(), Ns[i]
        segs[i].sb_pairs = tables[i].data_ptr() if tables[i] is not None else 0
    st = _runtime.stream_ptr(dev)
    if fused is not None:
        rc = lib.dfmi_qmm_affine_multi_fused(x.data_ptr(), _runtime.dtype_code(x.dtype), segs, n,
                                             fused.data_ptr(), M, K, gs, bits, wsp, need, st)
    else:
        rc = lib.dfmi_qmm_affine_multi(x.data_ptr(), _runtime.dtype_code(x.dtype), segs, n, M, K,
                                       gs, bits, wsp, need, st)
    _lib.check(rc, "multi")
    torch.cuda.synchronize()
    return ys


def _run_record(rec, x, Ns):
    import torch

    from dflash_mlx_amd.verify_qmm import current_stream

    ys = [torch.full((x.shape[0], N), float("nan"), dtype=x.dtype, device=x.device) for N in Ns]
    rec.run(x, ys, current_stream(x.get_device()))
    torch.cuda.synchronize()
    return ys


@pytest.mark.parametrize("M,K,Ns,gs", [
    (16, 5120, (5120,), 64),               # 64-row blocks, K split 3 ways
    (16, 5120, (17408,), 64),              # 128-row blocks, whole + split tail
    (4, 4096, (1024,), 64),
    (32, 2048, (1000,), 128),              # two activation blocks, ragged N
    (16, 5120, (5120, 1024, 1024), 64),    # q/k/v: the fused kernel
    (16, 5120, (17408, 17408), 64),        # gate/up: the fused kernel
    (8, 2048, (1000, 200, 136), 64)])
@pytest.mark.parametrize("dtype", ["bf16", "f16"])
def test_record_matches_one_shot(dev, M, K, Ns, gs, dtype):
    import torch

    from dflash_mlx_amd import _runtime
    from dflash_mlx_amd.verify_qmm import LaunchRecord, qmm_launch

    print(f"case: record M={M} K={K} Ns={Ns} gs={gs} {dtype}", flush=True)
    cases, x, mats = _case(dev, M, K, Ns, gs, dtype, seed=M + K + sum(Ns))
    tables = [_runtime.build_sb_pairs(s, b) for (_, s, b) in mats]
    if len(Ns) == 1:
        (w, s, b), t = mats[0], tables[0]
        want = [qmm_launch(x, w, s, b, Ns[0], gs, 4, pairs=t)]
        rec = LaunchRecord(M, K, x.dtype, dev, [(w, s, b, t)], gs, 4)
    else:
        fused = torch.cat(tables, dim=1).contiguous()
        want = _one_shot_multi(dev, x, mats, tables, fused, M, K, gs)
        rec = LaunchRecord(M, K, x.dtype, dev, mats, gs, 4, fused=fused)
    torch.cuda.synchronize()
    for _ in range(2):  # the workspace's counters are left at zero
        got = _run_record(rec, x, Ns)
        for g, w_ in zip(got, want):
            assert torch.equal(g, w_)
    for g, c in zip(got, cases):
        ref = oracle.quantized_matmul(cases[0][0], c[1], c[2], c[3], group_size=gs, dtype=dtype)
        _, rel = oracle.parity_metrics(oracle.to_f32(from_dev(g, dtype), dtype), ref)
        assert rel <= REL_TOL, rel


@pytest.mark.parametrize("M", [16, 4, 32])
def test_record_column_slice_of_wider_table(dev, M):
    """A matrix reading its column slice of a sibling group's combined table
    (sb_stride = the table's row length) gives its own table's bits, alone
    and as a subset of the siblings (segment-table kernel)."""
    import torch

    from dflash_mlx_amd import _runtime
    from dflash_mlx_amd.verify_qmm import LaunchRecord, qmm_launch

    K, gs, Ns = 5120, 64, (5120, 1024, 1024)
    cases, x, mats = _case(dev, M, K, Ns, gs, "bf16", seed=91 + M)
    tables = [_runtime.build_sb_pairs(s, b) for (_, s, b) in mats]
    fused = torch.cat(tables, dim=1).contiguous()
    stride = int(fused.shape[1])
    cols = [0, 5120, 6144]
    for i, (w, s, b) in enumerate(mats):
        sl = fused[:, cols[i]:cols[i] + Ns[i]]
        rec = LaunchRecord(M, K, x.dtype, dev, [(w, s, b, sl)], gs, 4, sb_stride=stride)
        want = qmm_launch(x, w, s, b, Ns[i], gs, 4, pairs=tables[i])
        got = _run_record(rec, x, [Ns[i]])[0]
        assert torch.equal(got, want)
    # q and v with their slices (a group whose k dropped out)
    sub = [0, 2]
    rec = LaunchRecord(M, K, x.dtype, dev,
                       [(*mats[i], fused[:, cols[i]:cols[i] + Ns[i]]) for i in sub], gs, 4,
                       sb_stride=stride)
    want = _one_shot_multi(dev, x, [mats[i] for i in sub], [tables[i] for i in sub], None, M, K,
                           gs)
    got = _run_record(rec, x, [Ns[i] for i in sub])
    for g, w_ in zip(got, want):
        assert torch.equal(g, w_)


@pytest.mark.parametrize("M,K,Ns", [(40, 2048, (512,)), (16, 1088, (640, 256)),
                                    (40, 2048, (512, 256))])
def test_record_outside_streaming_kernel(dev, M, K, Ns):
    """Shapes the streaming kernel does not take (M > 32, K % 256 != 0) run
    the one-shot entry point's own route: the same bits."""
    import torch

    from dflash_mlx_amd.verify_qmm import LaunchRecord

    cases, x, mats = _case(dev, M, K, Ns, 64, "bf16", seed=M + K)
    want = _one_shot_multi(dev, x, mats, [None] * len(Ns), None, M, K, 64)
    rec = LaunchRecord(M, K, x.dtype, dev, mats, 64, 4)
    got = _run_record(rec, x, Ns)
    for g, w_ in zip(got, want):
        assert torch.equal(g, w_)


def test_record_argument_checks(dev):
    """Prepare rejects bad strides and buffers; run rejects an unprepared
    record and a null output (nothing launched)."""
    import torch

    from dflash_mlx_amd import _lib

    lib = _lib.load()
    buf = ctypes.create_string_buffer(_lib.DFMI_QMM_RECORD_BYTES + 16)
    ptr = (ctypes.addressof(buf) + 15) // 16 * 16
    assert lib.dfmi_qmm_run(ptr, None, None, None, None, None, None) == _lib.DFMI_EINVAL
    assert b"not a prepared record" in lib.dfmi_last_error()
    w = torch.zeros((256, 1024 // 8), dtype=torch.int32, device=dev)
    s = torch.zeros((256, 16), dtype=torch.bfloat16, device=dev)
    t = torch.zeros((16, 256), dtype=torch.int32, device=dev)
    seg = (_lib.QmmSegment * 1)()
    seg[0].w_q, seg[0].scales, seg[0].biases = w.data_ptr(), s.data_ptr(), s.data_ptr()
    seg[0].N, seg[0].sb_pairs = 256, t.data_ptr()
    # stride below N, stride not a multiple of 4, record buffer too small
    for stride, size in ((128, _lib.DFMI_QMM_RECORD_BYTES), (258, _lib.DFMI_QMM_RECORD_BYTES),
                         (0, 64)):
        assert lib.dfmi_qmm_prepare(_lib.DFMI_BF16, seg, 1, None, stride, 16, 1024, 64, 4, None,
                                    0, ptr, size) == _lib.DFMI_EINVAL
    # a split plan without its workspace
    need = int(lib.dfmi_qmm_workspace_bytes(16, 1024, 256, 64, 4))
    assert need > 0
    assert lib.dfmi_qmm_prepare(_lib.DFMI_BF16, seg, 1, None, 0, 16, 1024, 64, 4, None, 0, ptr,
                                _lib.DFMI_QMM_RECORD_BYTES) == _lib.DFMI_ENOSPC
    ws = torch.zeros(need + 256, dtype=torch.uint8, device=dev)
    wsp = (ws.data_ptr() + 255) // 256 * 256
    assert lib.dfmi_qmm_prepare(_lib.DFMI_BF16, seg, 1, None, 0, 16, 1024, 64, 4, wsp, need, ptr,
                                _lib.DFMI_QMM_RECORD_BYTES) == _lib.DFMI_OK
    x = torch.zeros((16, 1024), dtype=torch.bfloat16, device=dev)
    assert lib.dfmi_qmm_run(ptr, x.data_ptr(), None, None, None, None, None) == _lib.DFMI_EINVAL
    assert b"null output" in lib.dfmi_last_error()
