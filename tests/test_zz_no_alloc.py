"""dfmi_qmm_affine_noalloc (split-K workspace in the library's static device
array) through the C ABI, against dfmi_qmm_affine with a caller workspace:
bit-identical (same plan, same kernels, fixed split summation order), on
consecutive calls whose second is smaller, and against the oracle."""

from __future__ import annotations

import ctypes

import numpy as np
import pytest

import oracle
from tests.conftest import from_dev, make_qmm_case, to_dev

pytestmark = pytest.mark.gpu


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr())


def _both(dev, M, K, N, gs, seed):
    import torch

    from dflash_mlx_amd import _lib, _runtime

    lib = _lib.load()
    x, w_q, s, b = make_qmm_case(M, K, N, gs, seed=seed)
    xd, wd = to_dev(x, "bf16", dev), to_dev(w_q, "u32", dev)
    sd, bd = to_dev(s, "bf16", dev), to_dev(b, "bf16", dev)
    need = lib.dfmi_qmm_workspace_bytes(M, K, N, gs, 4)
    assert 0 < need <= lib.dfmi_qmm_noalloc_scratch_bytes()  # the shape uses the scratch
    ws = torch.zeros(need // 4 + 4, dtype=torch.int32, device=dev)
    y_ref = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
    y_na = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device=dev)
    st = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
    rc = lib.dfmi_qmm_affine(_ptr(xd), _lib.DFMI_BF16, _ptr(wd), _ptr(sd), _ptr(bd), _ptr(y_ref),
                             M, K, N, gs, 4, _ptr(ws), need, st)
    assert rc == _lib.DFMI_OK, lib.dfmi_last_error()
    rc = lib.dfmi_qmm_affine_noalloc(_ptr(xd), _lib.DFMI_BF16, _ptr(wd), _ptr(sd), _ptr(bd),
                                     _ptr(y_na), M, K, N, gs, 4, st)
    assert rc == _lib.DFMI_OK, lib.dfmi_last_error()
    torch.cuda.synchronize(dev)
    del _runtime
    got, want = from_dev(y_na, "bf16"), from_dev(y_ref, "bf16")
    assert np.array_equal(got, want)
    ref = oracle.quantized_matmul(x, w_q, s, b, group_size=gs, bits=4, dtype="bf16")
    _, rel = oracle.parity_metrics(oracle.to_f32(got, "bf16").astype(np.float64), ref)
    assert rel <= 1e-2, rel


def test_noalloc_first_call_under_graph_capture(dev):
    """The process's first noalloc call on the device made under HIP graph
    capture (it looks the scratch address up and records the counter clear
    into the graph): every replay, with eager work and synchronisations in
    between, matches dfmi_qmm_affine with a workspace bit for bit, and so
    does an eager call after the replays.  (Collected before the other tests
    of this file, which then find the address cached.)"""
    import torch

    from dflash_mlx_amd import _lib

    lib = _lib.load()
    M, K, N, gs = 16, 4096, 4096, 64
    x, w_q, s, b = make_qmm_case(M, K, N, gs, seed=21)
    xd, wd = to_dev(x, "bf16", dev), to_dev(w_q, "u32", dev)
    sd, bd = to_dev(s, "bf16", dev), to_dev(b, "bf16", dev)
    need = lib.dfmi_qmm_workspace_bytes(M, K, N, gs, 4)
    assert 0 < need <= lib.dfmi_qmm_noalloc_scratch_bytes()
    ws = torch.zeros(need // 4 + 4, dtype=torch.int32, device=dev)
    y_ref = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
    st0 = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
    rc = lib.dfmi_qmm_affine(_ptr(xd), _lib.DFMI_BF16, _ptr(wd), _ptr(sd), _ptr(bd), _ptr(y_ref),
                             M, K, N, gs, 4, _ptr(ws), need, st0)
    assert rc == _lib.DFMI_OK, lib.dfmi_last_error()
    y_na = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device=dev)
    stream = torch.cuda.Stream()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        rc = lib.dfmi_qmm_affine_noalloc(_ptr(xd), _lib.DFMI_BF16, _ptr(wd), _ptr(sd), _ptr(bd),
                                         _ptr(y_na), M, K, N, gs, 4,
                                         ctypes.c_void_p(stream.cuda_stream))
    assert rc == _lib.DFMI_OK, lib.dfmi_last_error()
    want = from_dev(y_ref, "bf16")
    for _ in range(3):
        y_na.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        assert np.array_equal(from_dev(y_na, "bf16"), want)
        torch.randn((64, 64), device=dev).sum()  # eager work between replays
        torch.cuda.synchronize()
    y_na.fill_(float("nan"))
    rc = lib.dfmi_qmm_affine_noalloc(_ptr(xd), _lib.DFMI_BF16, _ptr(wd), _ptr(sd), _ptr(bd),
                                     _ptr(y_na), M, K, N, gs, 4, st0)
    assert rc == _lib.DFMI_OK, lib.dfmi_last_error()
    torch.cuda.synchronize()
    assert np.array_equal(from_dev(y_na, "bf16"), want)


def test_noalloc_matches_workspace_entry_on_consecutive_calls(dev):
    # 64 blocks split 4 ways, then a smaller call (16 blocks split 4 ways,
    # ragged N, M = 4) over the same scratch, then the first shape again
    _both(dev, 16, 4096, 4096, 64, seed=11)
    _both(dev, 4, 2048, 1000, 64, seed=12)
    _both(dev, 16, 4096, 4096, 64, seed=13)


def test_noalloc_rejects_plans_above_the_scratch(dev):
    from dflash_mlx_amd import _lib

    lib = _lib.load()
    # K = 262144 at group 32: 69 splits of 15 steps x 32 x 8192 fp32 partials
    need = lib.dfmi_qmm_workspace_bytes(32, 262144, 8192, 32, 4)
    assert need > lib.dfmi_qmm_noalloc_scratch_bytes()
    rc = lib.dfmi_qmm_affine_noalloc(None, _lib.DFMI_BF16, None, None, None, None, 32, 262144,
                                     8192, 32, 4, None)
    assert rc == _lib.DFMI_ENOSPC
    assert b"static scratch" in lib.dfmi_last_error()
