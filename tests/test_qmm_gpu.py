"""GPU parity of the dense affine qmm (libdfmi ``dfmi_qmm_affine``) against the
CPU oracle, on seeded inputs.  Tolerance (written here, from the verify path's
contract): max|y - y_ref| / (max|y_ref| + 1e-3) <= 1e-2 (the reference's own
metric, tests/test_verify_qmm_parity.py:69-70, at half the reference's 2e-2),
plus an elementwise bound of 2 output ulps around the exact result."""

from __future__ import annotations

import json
import os

import numpy as np
import pytest

import oracle
from tests.conftest import from_dev, make_qmm_case, to_dev

pytestmark = pytest.mark.gpu

GOLD = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "reference_cases.json")))
REL_TOL = 1e-2


def _run(dev, x, w_q, s, b, gs, dtype="bf16", tuning=None, via="stock", monkeypatch=None,
         bits=4):
    import torch

    from dflash_mlx_amd import verify_qmm as vq

    xt, st, bt = to_dev(x, dtype, dev), to_dev(s, dtype, dev), to_dev(b, dtype, dev)
    wt = to_dev(w_q, "u32", dev)
    if via == "verify":
        y = vq.verify_matmul(xt, wt, st, bt, transpose=True, group_size=gs, bits=bits)
    else:
        y = vq.quantized_matmul(xt, wt, st, bt, transpose=True, group_size=gs, bits=bits,
                                tuning=tuning)
    torch.cuda.synchronize()
    return from_dev(y, dtype)


def _check(got, x, w_q, s, b, gs, dtype="bf16"):
    ref = oracle.quantized_matmul(x, w_q, s, b, group_size=gs, bits=4, dtype=dtype)
    g = oracle.to_f32(got, dtype).astype(np.float64)
    max_abs, max_rel = oracle.parity_metrics(g, ref)
    assert g.shape == ref.shape
    assert np.all(np.isfinite(g))
    assert max_rel <= REL_TOL, f"max_rel={max_rel:.3g} max_abs={max_abs:.3g}"
    ulp = 2.0 ** -8 if dtype == "bf16" else 2.0 ** -11
    bound = 2 * ulp * np.abs(ref) + 1e-4 * np.abs(ref).max()
    assert np.all(np.abs(g - ref) <= bound), "elementwise bound"
    return max_rel


def test_config1_single_call(dev):
    # [16,4096] x [4096,4096], x ~ N(0,1), W ~ N(0,0.02), int4 gs64
    x, w_q, s, b = make_qmm_case(16, 4096, 4096, 64, seed=1)
    _check(_run(dev, x, w_q, s, b, 64), x, w_q, s, b, 64)


@pytest.mark.parametrize("K,N", [(4096, 4096), (4096, 1024), (4096, 12288), (12288, 4096),
                                 (5120, 5120), (5120, 1024), (5120, 17408), (17408, 5120)])
def test_9b_27b_layer_shapes_m16(dev, K, N):
    x, w_q, s, b = make_qmm_case(16, K, N, 64, seed=K + N)
    _check(_run(dev, x, w_q, s, b, 64), x, w_q, s, b, 64)


@pytest.mark.parametrize("M", [4, 8, 32])
@pytest.mark.parametrize("K,N", [(4096, 12288), (4096, 1024), (17408, 5120), (5120, 17408),
                                 (5120, 5120), (5120, 1024)])
def test_layer_shapes_other_m(dev, M, K, N):
    """The adaptive M=4 block and the 27B sweep's M=8 / M=32 on every layer
    shape they run at (q/o 5120x5120 and k/v 5120x1024 take their own split
    plans, e.g. 3 splits at M=32 on 5120x5120)."""
    x, w_q, s, b = make_qmm_case(M, K, N, 64, seed=K + N + M)
    _check(_run(dev, x, w_q, s, b, 64), x, w_q, s, b, 64)


@pytest.mark.parametrize("M,K,N", [
    (16, 5120, 34816),                 # 544 blocks: 512 whole + 32 blocks x 8 pieces
    (32, 5120, 34816),                 # two activation blocks: 512 whole + 32 x 16 splits
    (16, 5120, 512 * 64 + 6 * 64 - 51),  # 518 blocks, ragged: 6 blocks x 20 one-step pieces
    (16, 2048, 40960)])                # 640 blocks: 512 whole + 128 x 2
def test_whole_rounds_then_split_tail(dev, M, K, N):
    """Grids just past 512 blocks: two whole blocks per CU, the leftover
    blocks split into one piece per CU (M <= 16); M = 17..32: whole rounds of
    512 workgroups, the leftover blocks split over every slot."""
    x, w_q, s, b = make_qmm_case(M, K, N, 64, seed=K + N + M + 1)
    _check(_run(dev, x, w_q, s, b, 64), x, w_q, s, b, 64)


def test_split_tail_closed_form_exact(dev):
    # the same dyadic construction as test_closed_form_exact on a 518-block
    # grid: unsplit blocks and one-step splits summed by the last arriver
    # must both be bit-exact
    rng = np.random.default_rng(47)
    M, K, N, gs = 16, 5120, 512 * 64 + 6 * 64 - 51, 64
    q = rng.integers(0, 16, size=(N, K))
    w_q = oracle.pack(q, 4)
    s = oracle.f32_to_bf16_bits(np.full((N, K // gs), 0.125, np.float32))
    b = oracle.f32_to_bf16_bits(np.full((N, K // gs), -1.0, np.float32))
    xf = np.zeros((M, K), np.float32)
    for m in range(M):
        xf[m, rng.choice(K, size=6, replace=False)] = rng.choice([-1.0, 1.0], size=6)
    x = oracle.f32_to_bf16_bits(xf)
    want = oracle.quantized_matmul(x, w_q, s, b, group_size=gs, out_dtype="bf16")
    assert np.array_equal(_run(dev, x, w_q, s, b, gs), want)


@pytest.mark.parametrize("M", [1, 4, 8, 12, 15, 17, 24, 32, 48, 80])
def test_m_sweep(dev, M):
    x, w_q, s, b = make_qmm_case(M, 2048, 768, 64, seed=100 + M)
    _check(_run(dev, x, w_q, s, b, 64), x, w_q, s, b, 64)


@pytest.mark.parametrize("gs", [32, 64, 128])
@pytest.mark.parametrize("dtype", ["bf16", "f16"])
def test_group_sizes_and_dtypes(dev, gs, dtype):
    x, w_q, s, b = make_qmm_case(16, 1536, 640, gs, dtype=dtype, seed=gs)
    _check(_run(dev, x, w_q, s, b, gs, dtype), x, w_q, s, b, gs, dtype)


@pytest.mark.parametrize("K,N", [(1088, 232), (448, 16), (128, 488), (96, 40), (2496, 72)])
def test_ragged_k_and_n(dev, K, N):
    # K not a multiple of 256 (partial last chunk), N not a multiple of 16.
    x, w_q, s, b = make_qmm_case(16, K, N, 32, seed=K * 7 + N)
    _check(_run(dev, x, w_q, s, b, 32), x, w_q, s, b, 32)


@pytest.mark.parametrize("name,M,K,N", GOLD["random_shapes"])
def test_reference_random_shapes(dev, name, M, K, N, monkeypatch):
    # tests/test_verify_qmm_parity.py:32-42 shape list, through verify_matmul
    monkeypatch.setenv("DFLASH_VERIFY_QMM", "1")
    x, w_q, s, b = make_qmm_case(M, K, N, 64, seed=int(name[3:]))
    _check(_run(dev, x, w_q, s, b, 64, via="verify"), x, w_q, s, b, 64)


@pytest.mark.parametrize("name,M,K,N", GOLD["real_mlp_shapes"])
@pytest.mark.parametrize("dtype", ["bf16", "f16"])
def test_reference_real_mlp_shapes(dev, name, M, K, N, dtype, monkeypatch):
    # tests/test_verify_qmm_parity.py:16-27, inputs N(0,1)/sqrt(K) as there (29-52)
    monkeypatch.setenv("DFLASH_VERIFY_QMM", "1")
    sc = 1.0 / np.sqrt(K)
    x, w_q, s, b = make_qmm_case(M, K, N, 64, dtype=dtype, seed=N + M, x_std=sc, w_std=sc)
    _check(_run(dev, x, w_q, s, b, 64, dtype, via="verify"), x, w_q, s, b, 64, dtype)


def test_closed_form_exact(dev):
    # scale 1/8, bias -1, sparse +-1 activations: every partial sum is a small
    # dyadic number, exact in fp32 and in bf16, so the output must be bit-exact.
    # Pins the nibble order, the activation permutation and the MFMA lane layout.
    rng = np.random.default_rng(42)
    M, K, N, gs = 16, 1024, 128, 64
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
    for tuning in (None, (1, 1, 1, 0), (1, 2, 4, 0), (1, 4, 8, 0), (1, 1, 3, 0), (2, 1, 0, 1),
                   (2, 2, 0, 1), (2, 1, 0, 3), (2, 2, 0, 2), (2, 0, 8, 2), (2, 0, 4, 4)):
        got = _run(dev, x, w_q, s, b, gs, tuning=_tuning(tuning))
        assert np.array_equal(got, want), f"tuning {tuning}"


def _tuning(t):
    """(path, tiles_per_wave, waves_per_block, k_splits); path 1 general, 2 streaming."""
    if t is None:
        return None
    from dflash_mlx_amd import _lib

    return _lib.QmmTuning(*t)


@pytest.mark.parametrize("tuning", [(1, 1, 1, 0), (1, 2, 1, 0), (1, 1, 2, 0), (1, 2, 3, 0),
                                    (1, 1, 8, 0), (1, 4, 8, 0), (1, 4, 5, 0),
                                    (2, 1, 0, 1), (2, 2, 0, 1), (2, 1, 0, 2), (2, 1, 0, 5),
                                    (2, 2, 0, 4), (2, 1, 0, 16)])
def test_launch_shapes_agree(dev, tuning):
    x, w_q, s, b = make_qmm_case(16, 4096, 2048, 64, seed=77)
    got = _run(dev, x, w_q, s, b, 64, tuning=_tuning(tuning))
    _check(got, x, w_q, s, b, 64)


@pytest.mark.parametrize("M", [1, 8, 16, 24, 32])
@pytest.mark.parametrize("gs", [32, 64, 128])
def test_streaming_kernel_shapes(dev, M, gs):
    # forced onto the streaming kernel, with and without a K split
    K, N = 2048, 640
    x, w_q, s, b = make_qmm_case(M, K, N, gs, seed=M * 3 + gs)
    for t in ((2, 0, 0, 1), (2, 0, 0, 3), (2, 2, 0, 2)):
        _check(_run(dev, x, w_q, s, b, gs, tuning=_tuning(t)), x, w_q, s, b, gs)


def test_deterministic_and_workspace_reuse(dev):
    # The K-split reduction sums the wavefronts' partials in a fixed order, so
    # repeated calls are bit-identical, whatever ran in between.
    x, w_q, s, b = make_qmm_case(16, 4096, 4096, 64, seed=5)
    x2, w2, s2, b2 = make_qmm_case(16, 5120, 1024, 64, seed=6)
    first = _run(dev, x, w_q, s, b, 64)
    for _ in range(3):
        _run(dev, x2, w2, s2, b2, 64)
        assert np.array_equal(_run(dev, x, w_q, s, b, 64), first)


def test_unsupported_raises(dev):
    import torch

    from dflash_mlx_amd import _lib
    from dflash_mlx_amd import verify_qmm as vq

    x = torch.zeros((16, 100), dtype=torch.bfloat16, device=dev)  # K % 32 != 0
    w = torch.zeros((8, 100 // 8), dtype=torch.int32, device=dev)
    s = torch.zeros((8, 2), dtype=torch.bfloat16, device=dev)
    with pytest.raises(_lib.DfmiUnsupported):
        vq.quantized_matmul(x, w, s, s, group_size=50, bits=4)
    # (float32 activations are computed: tests/test_general_gpu.py; 3-bit
    # weights are not)
    xf = torch.zeros((16, 64), dtype=torch.float32, device=dev)
    with pytest.raises(_lib.DfmiUnsupported):
        vq.quantized_matmul(xf, w[:, :6], s[:, :1], s[:, :1], group_size=64, bits=3)


@pytest.mark.parametrize("M,K,N,gs", [
    (16, 4096, 1024, 64),   # streaming, 8 wavefronts, K split 4 ways
    (4, 512, 96, 32),       # streaming, 4 wavefronts in two LDS stages, one step, ragged N
    (16, 1024, 2048, 128),  # streaming, 4 wavefronts in two LDS stages
    (24, 2048, 200, 64),    # streaming, 4 wavefronts, two 16-row activation blocks
    (16, 512, 16448, 64),   # streaming, 4 wavefronts (257 blocks), unsplit
    (16, 4096, 12288, 64),  # streaming, 4 wavefronts in two stages, K split 2 ways (the 9B gate/up plan)
    (16, 2048, 12288, 64),  # the same plan at 4 steps per split
    (33, 256, 40, 64),      # register-load kernel (M > 32)
    (1, 96, 16, 32)])       # register-load kernel (K not whole 256-k steps)
@pytest.mark.parametrize("dtype", ["bf16", "f16"])
def test_8bit_matches_oracle(dev, M, K, N, gs, dtype):
    """bits=8 (the reference's mma2big_8bit layout, verify_qmm.py:593-598)."""
    x, w_q, s, b = make_qmm_case(M, K, N, gs, dtype=dtype, seed=M + K + N, bits=8)
    got = _run(dev, x, w_q, s, b, gs, dtype=dtype, bits=8)
    want = oracle.quantized_matmul(x, w_q, s, b, group_size=gs, bits=8, dtype=dtype)
    _, rel = oracle.parity_metrics(oracle.to_f32(got, dtype), want)
    assert rel <= 1e-2, rel


@pytest.mark.parametrize("K", [256, 1024])  # register-load kernel, streaming kernel
@pytest.mark.parametrize("dtype", ["bf16", "f16"])
def test_8bit_closed_form_exact(dev, K, dtype):
    """Integer activations, unit scales, small integer biases: the fp32 result is
    exact, so the 8-bit path must be bit-exact after rounding (every code
    0..255 occurs, so the exact bf16 conversion and the f16 magic are both
    pinned)."""
    rng = np.random.default_rng(8)
    M, N, gs = 16, 64, 64
    q = rng.integers(0, 256, size=(N, K))
    q[0, :256] = np.arange(256)
    w_q = oracle.pack(q, 8)
    s = oracle.round_to_dtype(np.ones((N, K // gs), np.float32), dtype)
    b = oracle.round_to_dtype(rng.integers(-2, 3, size=(N, K // gs)).astype(np.float32), dtype)
    x = oracle.round_to_dtype(rng.integers(-1, 2, size=(M, K)).astype(np.float32), dtype)
    exact = oracle.quantized_matmul(x, w_q, s, b, group_size=gs, bits=8, dtype=dtype)
    assert np.abs(exact).max() < 6e4  # inside the f16 range: the test is well posed
    want = oracle.quantized_matmul(x, w_q, s, b, group_size=gs, bits=8, dtype=dtype,
                                   out_dtype=dtype)
    got = _run(dev, x, w_q, s, b, gs, dtype=dtype, bits=8)
    assert np.array_equal(got, want)


def test_captured_graph_survives_workspace_growth(dev):
    """A graph captured with a split-K call keeps its workspace address: a
    later, larger call on the same stream grows the stream's workspace, the
    old buffer must stay allocated (the replay still writes partials and
    counters there), and memory handed out afterwards stays untouched."""
    import torch

    from dflash_mlx_amd import verify_qmm as vq

    M, K, N, gs = 16, 4096, 1024, 64  # K split over 8 workgroups: uses the workspace
    x, w_q, s, b = make_qmm_case(M, K, N, gs, seed=21)
    xt, wt, st_, bt = to_dev(x, "bf16", dev), to_dev(w_q, "u32", dev), to_dev(s, "bf16", dev), \
        to_dev(b, "bf16", dev)
    stream = torch.cuda.Stream()
    with torch.cuda.stream(stream):
        vq.quantized_matmul(xt, wt, st_, bt, group_size=gs)  # creates this stream's workspace
    stream.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        yg = vq.quantized_matmul(xt, wt, st_, bt, group_size=gs)
    # a larger split-K call on the same stream grows the workspace
    K2, N2 = 12288, 4096  # 8 splits: 2 MiB of partials against 512 KiB
    with torch.cuda.stream(stream):  # (values irrelevant: only the workspace size matters)
        vq.quantized_matmul(torch.zeros((M, K2), dtype=torch.bfloat16, device=dev),
                            torch.zeros((N2, K2 // 8), dtype=torch.int32, device=dev),
                            torch.zeros((N2, K2 // gs), dtype=torch.bfloat16, device=dev),
                            torch.zeros((N2, K2 // gs), dtype=torch.bfloat16, device=dev),
                            group_size=gs)
    stream.synchronize()
    fills = [torch.full((1 << 18,), 7, dtype=torch.int32, device=dev) for _ in range(16)]
    torch.cuda.synchronize()
    want = oracle.quantized_matmul(x, w_q, s, b, group_size=gs, dtype="bf16")
    for _ in range(3):
        graph.replay()
        torch.cuda.synchronize()
        _check(from_dev(yg, "bf16"), x, w_q, s, b, gs)
        _, rel = oracle.parity_metrics(oracle.to_f32(from_dev(yg, "bf16"), "bf16"), want)
        assert rel <= REL_TOL
    assert all(bool((f == 7).all()) for f in fills)


def test_empty_rows(dev):
    """x with no rows gives an empty [.., N] result through both Python entry
    points, without a launch."""
    import torch

    from dflash_mlx_amd.verify_qmm import quantized_matmul, verify_matmul

    K, N = 512, 96
    w = (np.random.default_rng(3).standard_normal((N, K)) * 0.02).astype(np.float32)
    q, s, b = oracle.quantize(w, 64, 4, out_dtype="bf16")
    args = (to_dev(q, "u32", dev), to_dev(s, "bf16", dev), to_dev(b, "bf16", dev))
    for fn in (quantized_matmul, verify_matmul):
        for shape in ((0, K), (2, 0, K)):
            x = torch.empty(shape, dtype=torch.bfloat16, device=dev)
            y = fn(x, *args, group_size=64, bits=4)
            assert tuple(y.shape) == shape[:-1] + (N,)
    torch.cuda.synchronize()
