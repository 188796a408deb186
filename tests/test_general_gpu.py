"""GPU parity of the rest of the stock quantized matmul (``dfmi_qmm_general``
through ``verify_qmm.quantized_matmul``): activations or scales in float32
(or of two different 16-bit dtypes) and ``transpose=False``, the inputs the
reference hands to ``mx.quantized_matmul`` (dflash_mlx/verify_qmm.py:915-919).

Tolerances (written here): float32 results ``max|y - y_ref| / (max|y_ref| +
1e-3) <= 2e-5`` against the float64 oracle (fp32 accumulation over K <=
4096); 16-bit results the verify path's metric ``<= 1e-2`` plus an
elementwise bound of 2 output ulps around the exact result; integer-valued
cases bit-exact."""

from __future__ import annotations

import numpy as np
import pytest

import oracle
from tests.conftest import from_dev, to_dev

pytestmark = pytest.mark.gpu

F32_TOL = 2e-5
REL_TOL = 1e-2


def _case(M, K, N, gs, bits, x_dtype, s_dtype, transpose, seed):
    """Seeded storage arrays: x [M, K] in x_dtype; W [N, K] (transpose) or
    [K, N] quantised along its last axis with the scales in s_dtype."""
    rng = np.random.default_rng(seed)
    x = oracle.round_to_dtype(rng.standard_normal((M, K)).astype(np.float32), x_dtype)
    shape = (N, K) if transpose else (K, N)
    w_q, s, b = oracle.quantize((rng.standard_normal(shape) * 0.02).astype(np.float32), gs, bits,
                                out_dtype=s_dtype)
    return x, w_q, s, b


def _run(dev, x, w_q, s, b, gs, bits, x_dtype, s_dtype, transpose):
    import torch

    from dflash_mlx_amd import verify_qmm as vq

    y = vq.quantized_matmul(to_dev(x, x_dtype, dev), to_dev(w_q, "u32", dev),
                            to_dev(s, s_dtype, dev), to_dev(b, s_dtype, dev),
                            transpose=transpose, group_size=gs, bits=bits)
    torch.cuda.synchronize()
    return y


def _ref(x, w_q, s, b, gs, bits, x_dtype, s_dtype, transpose):
    # both operands as float32 values (exact), the product in float64
    x32 = oracle.to_f32(x, x_dtype)
    s32, b32 = oracle.to_f32(s, s_dtype), oracle.to_f32(b, s_dtype)
    return oracle.quantized_matmul(x32, w_q, s32, b32, transpose=transpose, group_size=gs,
                                   bits=bits, dtype="f32")


def _check(y, ref, out_dtype):
    import torch

    want = {"f32": torch.float32, "bf16": torch.bfloat16, "f16": torch.float16}[out_dtype]
    assert y.dtype == want, (y.dtype, want)
    g = oracle.to_f32(from_dev(y, out_dtype), out_dtype).astype(np.float64)
    assert g.shape == ref.shape and np.all(np.isfinite(g))
    _, max_rel = oracle.parity_metrics(g, ref)
    if out_dtype == "f32":
        assert max_rel <= F32_TOL, f"max_rel={max_rel:.3g}"
    else:
        assert max_rel <= REL_TOL, f"max_rel={max_rel:.3g}"
        ulp = 2.0 ** -8 if out_dtype == "bf16" else 2.0 ** -11
        assert np.all(np.abs(g - ref) <= 2 * ulp * np.abs(ref) + 1e-4 * np.abs(ref).max())


def _out_dtype(x_dtype, s_dtype):
    return x_dtype if x_dtype == s_dtype else "f32"


TRANSPOSED_DTYPES = [("f32", "f32"), ("f32", "bf16"), ("f32", "f16"), ("bf16", "f32"),
                     ("bf16", "f16"), ("f16", "bf16")]
TRANSPOSED_SHAPES = [(1, 64, 16, 32, 4), (5, 320, 100, 64, 4), (16, 4096, 4096, 64, 4),
                     (33, 512, 70, 128, 8), (16, 1024, 512, 32, 8), (100, 256, 48, 64, 4)]


@pytest.mark.parametrize("x_dtype,s_dtype", TRANSPOSED_DTYPES)
@pytest.mark.parametrize("M,K,N,gs,bits", TRANSPOSED_SHAPES)
def test_transposed_other_dtypes(dev, x_dtype, s_dtype, M, K, N, gs, bits):
    args = (gs, bits, x_dtype, s_dtype, True)
    x, w_q, s, b = _case(M, K, N, gs, bits, x_dtype, s_dtype, True, seed=M * 7 + K + N)
    _check(_run(dev, x, w_q, s, b, *args), _ref(x, w_q, s, b, *args),
           _out_dtype(x_dtype, s_dtype))


UNTRANSPOSED_DTYPES = [("bf16", "bf16"), ("f16", "f16"), ("f32", "f32"), ("f32", "bf16"),
                       ("bf16", "f32")]
UNTRANSPOSED_SHAPES = [(1, 1, 32, 32, 4), (3, 7, 64, 32, 4), (16, 4096, 4096, 64, 4),
                       (5, 100, 256, 128, 8), (16, 513, 96, 32, 8), (40, 64, 128, 64, 4),
                       (9, 2000, 4160, 64, 4)]


@pytest.mark.parametrize("x_dtype,s_dtype", UNTRANSPOSED_DTYPES)
@pytest.mark.parametrize("M,K,N,gs,bits", UNTRANSPOSED_SHAPES)
def test_untransposed(dev, x_dtype, s_dtype, M, K, N, gs, bits):
    args = (gs, bits, x_dtype, s_dtype, False)
    x, w_q, s, b = _case(M, K, N, gs, bits, x_dtype, s_dtype, False, seed=M * 5 + K + N)
    _check(_run(dev, x, w_q, s, b, *args), _ref(x, w_q, s, b, *args),
           _out_dtype(x_dtype, s_dtype))


@pytest.mark.parametrize("transpose", [True, False])
@pytest.mark.parametrize("bits", [4, 8])
def test_integer_case_exact(dev, transpose, bits):
    # integer activations, scale 2^-2, integer biases: every product and sum
    # is exact in float32, so the result is the float64 one bit for bit
    rng = np.random.default_rng(17 + bits)
    M, K, N, gs = 7, 256, 128, 64
    x = rng.integers(-4, 5, size=(M, K)).astype(np.float32)
    shape = (N, K) if transpose else (K, N)
    q = rng.integers(0, 1 << bits, size=shape).astype(np.uint8)
    w_q = oracle.pack(q, bits)
    gshape = (shape[0], shape[1] // gs)
    s = np.full(gshape, 0.25, np.float32)
    b = rng.integers(-3, 4, size=gshape).astype(np.float32)
    y = _run(dev, x, w_q, s, b, gs, bits, "f32", "f32", transpose)
    ref = _ref(x, w_q, s, b, gs, bits, "f32", "f32", transpose)
    assert np.array_equal(from_dev(y, "f32").astype(np.float64), ref)


@pytest.mark.parametrize("transpose", [True, False])
def test_deterministic(dev, transpose):
    import torch

    x, w_q, s, b = _case(16, 1024, 512, 64, 4, "f32", "f32", transpose, seed=3)
    y0 = _run(dev, x, w_q, s, b, 64, 4, "f32", "f32", transpose)
    y1 = _run(dev, x, w_q, s, b, 64, 4, "f32", "f32", transpose)
    assert torch.equal(y0, y1)


def test_same_16bit_dtype_transposed_is_the_verify_kernel(dev):
    # dfmi_qmm_general with x and scales of one 16-bit dtype and transpose is
    # dfmi_qmm_affine_ex: the same bits
    import torch

    from dflash_mlx_amd import _lib, _runtime
    from dflash_mlx_amd import verify_qmm as vq

    x, w_q, s, b = _case(16, 4096, 1024, 64, 4, "bf16", "bf16", True, seed=9)
    xt, wt = to_dev(x, "bf16", dev), to_dev(w_q, "u32", dev)
    st, bt = to_dev(s, "bf16", dev), to_dev(b, "bf16", dev)
    want = vq.quantized_matmul(xt, wt, st, bt, transpose=True, group_size=64, bits=4)
    lib = _lib.load()
    y = torch.empty_like(want)
    need = int(lib.dfmi_qmm_workspace_bytes(16, 4096, 1024, 64, 4))
    ws, wsb = _runtime.workspace(dev, need) if need else (0, 0)
    rc = lib.dfmi_qmm_general(xt.data_ptr(), _lib.DFMI_BF16, wt.data_ptr(), st.data_ptr(),
                              bt.data_ptr(), _lib.DFMI_BF16, y.data_ptr(), 16, 4096, 1024, 64, 4, 1,
                              ws, wsb, _runtime.stream_ptr(dev))
    assert rc == 0
    torch.cuda.synchronize()
    assert torch.equal(y, want)


def test_drop_in_routes_take_float32(dev, monkeypatch):
    # verify_matmul and a VerifyQuantizedLinear hand float32 activations to
    # the stock path (the reference: mx.quantized_matmul), which now computes
    import torch

    from dflash_mlx_amd import verify_qmm as vq
    from dflash_mlx_amd.verify_linear import QuantizedLinear, install_verify_linears

    monkeypatch.setenv("DFLASH_VERIFY_QMM", "1")
    x, w_q, s, b = _case(16, 512, 256, 64, 4, "f32", "f32", True, seed=21)
    xt, wt = to_dev(x, "f32", dev), to_dev(w_q, "u32", dev)
    st, bt = to_dev(s, "f32", dev), to_dev(b, "f32", dev)
    direct = vq.quantized_matmul(xt, wt, st, bt, transpose=True, group_size=64, bits=4)
    assert torch.equal(vq.verify_matmul(xt, wt, st, bt, transpose=True, group_size=64, bits=4),
                       direct)
    root = torch.nn.Module()
    root.proj = QuantizedLinear(wt, st, bt, group_size=64, bits=4)
    install_verify_linears(root, enable_qmm=True)
    assert torch.equal(root.proj(xt.reshape(1, 16, 512)).reshape(16, 256), direct)
    torch.cuda.synchronize()
    _check(direct, _ref(x, w_q, s, b, 64, 4, "f32", "f32", True), "f32")


def test_general_argument_errors(dev):
    import torch

    from dflash_mlx_amd import _lib
    from dflash_mlx_amd import verify_qmm as vq

    x, w_q, s, b = _case(4, 256, 64, 64, 4, "f32", "f32", False, seed=2)
    xt, wt = to_dev(x, "f32", dev), to_dev(w_q, "u32", dev)
    st, bt = to_dev(s, "f32", dev), to_dev(b, "f32", dev)
    with pytest.raises(_lib.DfmiUnsupported):
        vq.quantized_matmul(xt, wt, st, bt, transpose=False, group_size=64, bits=4, mode="mxfp4")
    with pytest.raises(_lib.DfmiUnsupported):
        vq.quantized_matmul(xt, wt, st, bt, transpose=False, group_size=48, bits=4)
    with pytest.raises(ValueError):
        vq.quantized_matmul(xt[:, :128], wt, st, bt, transpose=False, group_size=64, bits=4)
    with pytest.raises(ValueError):  # scales of the other orientation
        vq.quantized_matmul(xt, wt, st.t().contiguous(), bt, transpose=False, group_size=64,
                            bits=4)
    y = vq.quantized_matmul(xt[:0], wt, st, bt, transpose=False, group_size=64, bits=4)
    assert tuple(y.shape) == (0, 64) and y.dtype == torch.float32
