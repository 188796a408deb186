"""The shared-activation launch ``dfmi_qmm_affine_multi`` (q/k/v or gate/up
of a layer in one streaming grid) against the oracle and against separate
``dfmi_qmm_affine`` calls.

Same bar as the dense tests: the reference's metric max|d| / (max|ref| +
1e-3) <= 1e-2 plus 2 output ulps element-wise around the exact result;
bit-exact on closed-form integer cases; each matrix's result within fp32
summation order of its separate call."""

from __future__ import annotations

import ctypes

import numpy as np
import pytest

import oracle
from tests.conftest import from_dev, make_qmm_case, to_dev

pytestmark = pytest.mark.gpu

REL_TOL = 1e-2


def _run(dev, x, w_q, s, b, gs, dtype="bf16", bits=4):
    import torch

    from dflash_mlx_amd import verify_qmm as vq

    y = vq.quantized_matmul(to_dev(x, dtype, dev), to_dev(w_q, "u32", dev), to_dev(s, dtype, dev),
                            to_dev(b, dtype, dev), group_size=gs, bits=bits)
    torch.cuda.synchronize()
    return from_dev(y, dtype)


def _check(got, x, w_q, s, b, gs, dtype="bf16", bits=4):
    ref = oracle.quantized_matmul(x, w_q, s, b, group_size=gs, bits=bits, dtype=dtype)
    g = oracle.to_f32(got, dtype).astype(np.float64)
    _, rel = oracle.parity_metrics(g, ref)
    assert np.all(np.isfinite(g))
    assert rel <= REL_TOL, rel
    ulp = 2.0 ** -8 if dtype == "bf16" else 2.0 ** -11
    assert np.all(np.abs(g - ref) <= 2 * ulp * np.abs(ref) + 1e-4 * np.abs(ref).max())


def _kernel(M, K, Ns, bits=4):
    from dflash_mlx_amd import _lib

    ns = (ctypes.c_int64 * len(Ns))(*Ns)
    name = _lib.load().dfmi_qmm_multi_kernel_name(M, K, ns, len(Ns), 64, bits)
    return name.decode() if name else None


def _multi(dev, x, mats, gs, dtype="bf16", bits=4):
    import torch

    from dflash_mlx_amd.verify_qmm import quantized_matmul_multi

    ys = quantized_matmul_multi(to_dev(x, dtype, dev),
                                [(to_dev(w, "u32", dev), to_dev(s, dtype, dev),
                                  to_dev(b, dtype, dev)) for (w, s, b) in mats],
                                group_size=gs, bits=bits)
    torch.cuda.synchronize()
    return [from_dev(y, dtype) for y in ys]


@pytest.mark.parametrize("M,K,Ns,kernel", [
    (16, 5120, (5120, 1024, 1024), "qmm_stream_multi_kernel"),   # 27B q/k/v (K split)
    (16, 5120, (17408, 17408), "qmm_stream_multi_kernel"),       # 27B gate/up
    (16, 4096, (4096, 1024, 1024), "qmm_stream_multi_kernel"),   # 9B q/k/v
    (16, 4096, (12288, 12288), "qmm_stream_multi_kernel"),       # 9B gate/up
    (4, 2048, (100, 3000, 64, 7), "qmm_stream_multi_kernel"),    # ragged, four matrices
    (32, 2048, (300, 0, 700), "qmm_stream_multi_kernel"),        # two activation blocks; empty matrix
    (16, 1024, (65,), "qmm_stream_kernel"),
    (40, 2048, (512, 256), None),                                # M > 32: one call per matrix
    (16, 1088, (640, 256), None)])                               # K % 256 != 0: one call per matrix
@pytest.mark.parametrize("dtype", ["bf16", "f16"])
def test_multi_matches_oracle_and_separate_calls(dev, M, K, Ns, kernel, dtype):
    assert _kernel(M, K, Ns) == kernel
    mats = []
    x = None
    for i, N in enumerate(Ns):
        xx, w_q, s, b = make_qmm_case(M, K, max(N, 1), 64, dtype=dtype, seed=1000 * i + N + K)
        x = xx if x is None else x
        mats.append((w_q[:N], s[:N], b[:N]))
    got = _multi(dev, x, mats, 64, dtype)
    for (w_q, s, b), y in zip(mats, got):
        assert y.shape == (M, w_q.shape[0])
        if w_q.shape[0] == 0:
            continue
        _check(y, x, w_q, s, b, 64, dtype)
        single = _run(dev, x, w_q, s, b, 64, dtype)
        _, rel = oracle.parity_metrics(oracle.to_f32(y, dtype), oracle.to_f32(single, dtype))
        assert rel <= REL_TOL


@pytest.mark.parametrize("M,K,Ns", [(16, 4096, (4096, 1024, 1024)), (16, 2048, (3000, 100))])
def test_multi_8bit(dev, M, K, Ns):
    assert _kernel(M, K, Ns, bits=8) == "qmm_stream_multi_kernel"
    mats = []
    x = None
    for i, N in enumerate(Ns):
        xx, w_q, s, b = make_qmm_case(M, K, N, 64, bits=8, seed=77 + i)
        x = xx if x is None else x
        mats.append((w_q, s, b))
    for (w_q, s, b), y in zip(mats, _multi(dev, x, mats, 64, bits=8)):
        _check(y, x, w_q, s, b, 64, bits=8)


def test_multi_closed_form_exact(dev):
    rng = np.random.default_rng(44)
    M, K, gs = 16, 1024, 64
    mats = []
    for N in (5120, 1024, 192):
        q = rng.integers(0, 16, size=(N, K))
        mats.append((oracle.pack(q, 4),
                     oracle.f32_to_bf16_bits(np.full((N, K // gs), 0.125, np.float32)),
                     oracle.f32_to_bf16_bits(np.full((N, K // gs), -1.0, np.float32))))
    xf = np.zeros((M, K), np.float32)
    for m in range(M):
        xf[m, rng.choice(K, size=6, replace=False)] = rng.choice([-1.0, 1.0], size=6)
    x = oracle.f32_to_bf16_bits(xf)
    for (w_q, s, b), y in zip(mats, _multi(dev, x, mats, gs)):
        want = oracle.quantized_matmul(x, w_q, s, b, group_size=gs, out_dtype="bf16")
        assert np.array_equal(y, want)


@pytest.mark.parametrize("M,K,Ns,gs", [
    (16, 5120, (5120, 1024, 1024), 64),    # q/k/v rows: 64-row blocks, 2 splits
    (16, 5120, (17408, 17408), 64),        # gate/up: 128-row blocks, whole + pieces
    (16, 4096, (4096, 1024, 1024), 128),
    (32, 5120, (5120, 1024, 1024), 64),    # two activation blocks
    (8, 2048, (1000, 200, 136), 64),       # ragged N
    (4, 1024, (512, 512), 64)])
@pytest.mark.parametrize("dtype", ["bf16", "f16"])
def test_fused_pair_table_bit_identical(dev, M, K, Ns, gs, dtype):
    """dfmi_qmm_affine_multi_fused (the matrices' pair tables side by side)
    gives the same bits as dfmi_qmm_affine_multi with each matrix's own
    table, on the same plan; a second call over the same workspace too."""
    import torch

    from dflash_mlx_amd import _lib, _runtime

    lib = _lib.load()
    rng_seed = M + K + sum(Ns)
    cases = [make_qmm_case(M, K, N, gs, dtype=dtype, seed=rng_seed + i) for i, N in enumerate(Ns)]
    x = to_dev(cases[0][0], dtype, dev)
    mats = [(to_dev(c[1], "u32", dev), to_dev(c[2], dtype, dev), to_dev(c[3], dtype, dev))
            for c in cases]
    tables = [_runtime.build_sb_pairs(s, b) for (_, s, b) in mats]
    fused = torch.cat(tables, dim=1).contiguous()
    n = len(Ns)
    ns = (ctypes.c_int64 * n)(*Ns)
    need = int(lib.dfmi_qmm_multi_workspace_bytes(M, K, ns, n, gs, 4))
    ws = torch.zeros(need + 256, dtype=torch.uint8, device=dev)
    wsp = (ws.data_ptr() + 255) // 256 * 256 if need else 0

    def call(use_fused):
        ys = [torch.full((M, N), float("nan"), dtype=x.dtype, device=dev) for N in Ns]
        segs = (_lib.QmmSegment * n)()
        for i, ((w, s, b), y) in enumerate(zip(mats, ys)):
            segs[i].w_q, segs[i].scales, segs[i].biases = w.data_ptr(), s.data_ptr(), b.data_ptr()
            segs[i].y, segs[i].N = y.data_ptr(), Ns[i]
            segs[i].sb_pairs = 0 if use_fused else tables[i].data_ptr()
        st = _runtime.stream_ptr(dev)
        if use_fused:
            rc = lib.dfmi_qmm_affine_multi_fused(x.data_ptr(), _runtime.dtype_code(x.dtype), segs,
                                                 n, fused.data_ptr(), M, K, gs, 4, wsp, need, st)
        else:
            rc = lib.dfmi_qmm_affine_multi(x.data_ptr(), _runtime.dtype_code(x.dtype), segs, n,
                                           M, K, gs, 4, wsp, need, st)
        _lib.check(rc, "multi")
        torch.cuda.synchronize()
        return [from_dev(y, dtype) for y in ys]

    want = call(False)
    for _ in range(2):
        got = call(True)
        for g, w in zip(got, want):
            assert np.array_equal(g, w)
    for g, c in zip(got, cases):  # every matrix multiplies the shared x (cases[0][0])
        if g.size <= (1 << 22):
            _check(g, cases[0][0], c[1], c[2], c[3], gs, dtype)


def _gpu_quantized(dev, K, N, dtype, seed):
    """W ~ N(0, 0.02) [N, K] quantised on the GPU by the product quantiser
    (bit-identical to the oracle's rule: tests/test_quantize.py)."""
    import torch

    from dflash_mlx_amd.quantize import quantize

    tdt = torch.bfloat16 if dtype == "bf16" else torch.float16
    gen = torch.Generator(device=dev)
    gen.manual_seed(seed)
    w = torch.randn((N, K), generator=gen, device=dev) * 0.02
    return quantize(w, 64, 4, tdt)


@pytest.mark.parametrize("Ns", [(5120, 1024, 1024), (17408, 17408)])
@pytest.mark.parametrize("dtype", ["bf16", "f16"])
def test_fused_launch_27b_m8_m32(dev, Ns, dtype):
    """The launches the 27B-class M=8 and M=32 sweep lines time: q/k/v
    (5120 -> 5120/1024/1024) and gate/up (5120 -> 2x17408) through
    quantized_matmul_multi, i.e. the shared-activation kernel with the
    matrices' pair tables side by side, against the oracle."""
    import torch

    from dflash_mlx_amd import _lib, _runtime
    from dflash_mlx_amd.verify_qmm import quantized_matmul_multi

    K = 5120
    tdt = torch.bfloat16 if dtype == "bf16" else torch.float16
    mats = [_gpu_quantized(dev, K, N, dtype, seed=300 + i) for i, N in enumerate(Ns)]
    host = [(w.cpu().numpy().view(np.uint32), from_dev(s, dtype), from_dev(b, dtype))
            for (w, s, b) in mats]
    lib = _lib.load()
    for M in (8, 32):
        print(f"case: fused 27B launch Ns={Ns} M={M} {dtype}", flush=True)
        ns = (ctypes.c_int64 * len(Ns))(*Ns)
        info = _lib.QmmPlanInfo()
        assert lib.dfmi_qmm_plan(M, K, ns, len(Ns), 64, 4, None, ctypes.byref(info)) == 0
        assert info.streaming == 1 and info.pair_streaming == 1
        assert all(_runtime.pair_shape(M, K, N, 64, 4) for N in Ns)
        gen = torch.Generator(device=dev)
        gen.manual_seed(400 + M)
        x = torch.randn((M, K), generator=gen, device=dev).to(tdt)
        ys = quantized_matmul_multi(x, mats, group_size=64, bits=4)
        torch.cuda.synchronize()
        xs = from_dev(x, dtype)
        for (w_q, s, b), y in zip(host, ys):
            assert y.shape == (M, w_q.shape[0])
            _check(from_dev(y, dtype), xs, w_q, s, b, 64, dtype)
