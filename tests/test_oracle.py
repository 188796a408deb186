"""Pins the CPU oracle (no GPU).  Each check is chosen so that a plausible
mistake -- a wrong nibble order, a dropped bias term, a transposed operand,
a wrong tie-break -- fails it, without retyping the oracle's own formula."""

from __future__ import annotations

import json
import os

import numpy as np
import pytest

import oracle
from oracle import cpu as oracle_cpu

GOLD = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "reference_cases.json")))


# ---------------------------------------------------------------- layout

def test_unpack_hand_built_words():
    # dflash_mlx/verify_qmm.py:108-115: nibble i of word j is k = 8j + i.
    assert oracle.unpack(np.array([[0x76543210, 0xFEDCBA98]], np.uint32), 4).tolist() == \
        [list(range(16))]
    assert oracle.unpack(np.array([[0x03020100]], np.uint32), 8).tolist() == [[0, 1, 2, 3]]
    assert oracle.unpack(np.array([[0xE4]], np.uint32), 2).tolist()[0][:4] == [0, 1, 2, 3]


@pytest.mark.parametrize("bits", [2, 4, 8])
def test_pack_unpack_roundtrip(bits):
    rng = np.random.default_rng(bits)
    q = rng.integers(0, 1 << bits, size=(5, 128))
    assert np.array_equal(oracle.unpack(oracle.pack(q, bits), bits), q)


def test_pack_rejects_out_of_range():
    with pytest.raises(ValueError):
        oracle.pack(np.array([[16] * 8]), 4)


# ---------------------------------------------------------------- numerics

def test_bf16_rounding_known_values():
    vals = np.array([1.0, 1.0 + 2**-8, 1.0 + 3 * 2**-8, -2.5, np.inf, 0.0], np.float32)
    bits = oracle.f32_to_bf16_bits(vals)
    # ties go to even: 1+2^-8 -> 1.0, 1+3*2^-8 -> 1+2^-6 (0x3F82)
    assert bits.tolist() == [0x3F80, 0x3F80, 0x3F82, 0xC020, 0x7F80, 0x0000]
    assert np.isnan(oracle.bf16_bits_to_f32(oracle.f32_to_bf16_bits(np.float32(np.nan))))
    assert oracle.bf16_bits_to_f32(np.uint16(0x3F82)) == np.float32(1.0 + 2**-6)


# ---------------------------------------------------------------- quantize

def test_quantize_exact_on_affine_grid():
    # Groups that already are q*s + b with codes 0 and 15 present come back exactly.
    rng = np.random.default_rng(3)
    s, b = 2.0 ** -5, -0.25
    q = rng.integers(0, 16, size=(4, 128))
    q[:, ::64] = 0
    q[:, 1::64] = 15
    w = (q * s + b).astype(np.float32)
    w_q, sc, bi = oracle.quantize(w, 64, 4, out_dtype="f32")
    assert np.array_equal(oracle.unpack(w_q, 4), q)
    assert np.all(sc == np.float32(s)) and np.all(bi == np.float32(b))


@pytest.mark.parametrize("gs", [32, 64, 128])
@pytest.mark.parametrize("out_dtype", ["bf16", "f16", "f32"])
def test_quantize_reconstruction_bound(gs, out_dtype):
    rng = np.random.default_rng(gs)
    w = (rng.standard_normal((16, 512)) * 0.02).astype(np.float32)
    w_q, s, b = oracle.quantize(w, gs, 4, out_dtype=out_dtype)
    q = oracle.unpack(w_q, 4)
    assert q.min() >= 0 and q.max() <= 15
    deq = oracle.dequantize(w_q, s, b, gs, 4, out_dtype)
    sf = np.repeat(np.abs(oracle.to_f32(s, out_dtype)), gs, axis=-1)
    # Interior codes: half a step, plus the storage rounding of scale/bias.
    slack = {"bf16": 2**-8 * 16, "f16": 2**-11 * 16, "f32": 1e-5}[out_dtype]
    err = np.abs(deq - w)
    interior = (q > 0) & (q < 15)
    assert np.all(err[interior] <= sf[interior] * (0.5 + slack) + 1e-7)
    # The rule snaps the scale so that the edge value is an integer number of
    # steps from 0 (q0 = round(edge / scale)); that shrinks the step by at most
    # 0.5/7.5 and can clip the far end by up to one step -- never more.
    assert np.all(err <= sf * (1.0 + slack) + 1e-7)
    assert np.mean(err[~interior] > 0.5 * sf[~interior] * (1 + slack)) < 0.5


# ---------------------------------------------------------------- qmm

def test_qmm_closed_form_integer_case():
    # scale 1, bias 0, small-integer activations: y is an exact integer matmul.
    rng = np.random.default_rng(5)
    q = rng.integers(0, 16, size=(8, 64))
    x = rng.integers(-3, 4, size=(3, 64)).astype(np.float32)
    w_q = oracle.pack(q, 4)
    ones = oracle.f32_to_bf16_bits(np.ones((8, 1), np.float32))
    zeros = oracle.f32_to_bf16_bits(np.zeros((8, 1), np.float32))
    y = oracle.quantized_matmul(oracle.f32_to_bf16_bits(x), w_q, ones, zeros, group_size=64)
    assert np.array_equal(y, x.astype(np.int64) @ q.T)


def test_qmm_brute_force_elementwise():
    # Element-by-element restatement of the reference kernel's inner loop
    # (verify_qmm.py:243-249: nib = (packed >> 4*ki) & 0xF; w = nib*s + b).
    rng = np.random.default_rng(6)
    M, K, N, gs = 2, 128, 3, 32
    x, w_q, s, b = _case(M, K, N, gs, rng)
    xf = oracle.bf16_bits_to_f32(x).astype(np.float64)
    sf = oracle.bf16_bits_to_f32(s).astype(np.float64)
    bf = oracle.bf16_bits_to_f32(b).astype(np.float64)
    want = np.zeros((M, N))
    for m in range(M):
        for n in range(N):
            acc = 0.0
            for k in range(K):
                nib = (int(w_q[n, k // 8]) >> (4 * (k % 8))) & 0xF
                acc += xf[m, k] * (nib * sf[n, k // gs] + bf[n, k // gs])
            want[m, n] = acc
    got = oracle.quantized_matmul(x, w_q, s, b, group_size=gs)
    np.testing.assert_allclose(got, want, rtol=1e-12, atol=1e-12)


def test_qmm_bias_shift_identity():
    # Adding c to every bias adds c * sum_k x[m, k] to every output.
    rng = np.random.default_rng(7)
    x, w_q, s, b = _case(4, 256, 5, 64, rng, dtype="f32")
    b = (np.round(b * 4096) / 4096).astype(np.float32)  # so that b + c is exact
    c = 0.125
    y0 = oracle.quantized_matmul(x, w_q, s, b, group_size=64, dtype="f32")
    y1 = oracle.quantized_matmul(x, w_q, s, b + np.float32(c), group_size=64, dtype="f32")
    want = np.broadcast_to(c * x.astype(np.float64).sum(-1, keepdims=True), y0.shape)
    np.testing.assert_allclose(y1 - y0, want, rtol=1e-9, atol=1e-9)


def test_qmm_orientation():
    # y[m, n] uses row n of W (transpose=True): a one-hot activation picks a column.
    rng = np.random.default_rng(8)
    x, w_q, s, b = _case(1, 64, 4, 64, rng, dtype="f32")
    x = np.zeros_like(x)
    x[0, 10] = 1.0
    y = oracle.quantized_matmul(x, w_q, s, b, group_size=64, dtype="f32")
    w = oracle.dequantize(w_q, s, b, 64, 4, "f32")
    np.testing.assert_allclose(y[0], w[:, 10])


def test_cpu_restatement_matches_numpy_oracle():
    rng = np.random.default_rng(9)
    x, w_q, s, b = _case(16, 512, 96, 64, rng)
    want = oracle.quantized_matmul(x, w_q, s, b, group_size=64)
    got = oracle.bf16_bits_to_f32(oracle_cpu.qmm_bf16(x, w_q, s, b, 64, 4, threads=2))
    _, rel = oracle.parity_metrics(got, want)
    assert rel <= 1e-2
    # fp32 accumulation + one bf16 rounding: within a couple of bf16 ulps
    np.testing.assert_allclose(got, want, rtol=2**-7, atol=2**-7 * np.abs(want).max())


def test_gather_reduces_to_qmm():
    rng = np.random.default_rng(10)
    E, N, K = 3, 8, 128
    ws = [oracle.quantize((rng.standard_normal((N, K)) * 0.02).astype(np.float32), 64, 4)
          for _ in range(E)]
    w_q = np.stack([w[0] for w in ws])
    s = np.stack([w[1] for w in ws])
    b = np.stack([w[2] for w in ws])
    x = oracle.f32_to_bf16_bits(rng.standard_normal((4, 1, K)).astype(np.float32))
    lhs = np.array([0, 1, 2, 3, 0])
    rhs = np.array([2, 0, 1, 2, 1])
    y = oracle.gather_qmm(x, w_q, s, b, lhs, rhs, group_size=64)
    for p in range(5):
        want = oracle.quantized_matmul(x[lhs[p]], w_q[rhs[p]], s[rhs[p]], b[rhs[p]], group_size=64)
        np.testing.assert_array_equal(y[p], want)


# ---------------------------------------------------------------- greedy / accept

@pytest.mark.parametrize("drafted,posterior,expected", GOLD["acceptance_cases"])
def test_acceptance_known_answers(drafted, posterior, expected):
    # tests/test_engine_acceptance.py:11-24
    assert oracle.match_acceptance_length(drafted, posterior) == expected


def test_acceptance_brute_force():
    rng = np.random.default_rng(11)
    for _ in range(200):
        n = int(rng.integers(0, 16))
        d = rng.integers(0, 3, size=n)
        p = rng.integers(0, 3, size=n)
        want = 0
        while want < n and d[want] == p[want]:
            want += 1
        assert oracle.match_acceptance_length(d, p) == want


def test_greedy_ties_mask_and_nan():
    v = oracle.f32_to_bf16_bits(np.array([[1.0, 3.0, 3.0, 2.0],
                                          [np.nan, 0.5, 0.5, -1.0],
                                          [np.nan] * 4], np.float32))
    assert oracle.greedy_tokens_with_mask(v).tolist() == [1, 1, 0]
    mask = oracle.build_suppress_token_mask(4, [1, 9, -2])
    assert mask.tolist() == [False, True, False, False]
    assert oracle.greedy_tokens_with_mask(v, mask).tolist() == [2, 2, 1]  # -1e9 beats NaN
    assert oracle.build_suppress_token_mask(4, [7]) is None
    # masked ids become dtype(-1e9): an all-masked row picks index 0
    allm = np.ones(4, bool)
    assert oracle.greedy_tokens_with_mask(v[:1], allm).tolist() == [0]


def test_verify_cycle_accept_semantics():
    # spec_epoch.py:2011-2021, 2070-2072, 2129
    post = np.array([5, 6, 7, 8])
    assert oracle.verify_cycle_accept([1, 5, 6, 7], post) == (3, 8)
    assert oracle.verify_cycle_accept([1, 5, 9, 7], post) == (1, 6)
    assert oracle.verify_cycle_accept([1, 4, 6, 7], post) == (0, 5)


def test_softcap_identity_and_bound():
    v = oracle.f32_to_bf16_bits(np.array([-100.0, -1.0, 0.0, 2.0, 100.0], np.float32))
    assert np.array_equal(oracle.logit_softcap(v, None), v)
    out = oracle.bf16_bits_to_f32(oracle.logit_softcap(v, 30.0))
    assert np.all(np.abs(out) <= 30.0) and out[2] == 0.0
    assert abs(out[3] - 2.0) < 0.02  # tanh(x) ~ x for small x


def test_reference_shape_generator():
    # tests/test_verify_qmm_parity.py:32-42 regenerated with numpy
    from tests.golden.make_golden import random_shapes

    assert random_shapes() == GOLD["random_shapes"]


# ---------------------------------------------------------------- helpers

def _case(M, K, N, gs, rng, dtype="bf16"):
    x = oracle.round_to_dtype(rng.standard_normal((M, K)).astype(np.float32), dtype)
    w_q, s, b = oracle.quantize((rng.standard_normal((N, K)) * 0.02).astype(np.float32), gs, 4,
                                out_dtype=dtype)
    return x, w_q, s, b
