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


def test_quantize_code_order_known_answer():
    """MLX's affine_quantize computes the codes against the float32 scale and
    bias and casts them to the stored dtype afterwards.  A group whose codes
    differ between that order and codes taken against the stored bf16 scale,
    worked by hand:
      w_max = 1.0, w_min = 0.0: |w_min| > |w_max| is false, so
      scale = -(1 - 0) / 15 = -0.0666667 (float32), edge = w_max = 1.0,
      q0 = round(1.0 / -0.0666667) = -15 != 0, so scale = 1.0 / -15 and
      bias = 1.0;
      w = 0.498667: (w - 1) / scale = 15 * 0.501333 = 7.51999 -> code 8;
      (against bf16(scale) = -0.06689453125 it would be 7.4943 -> 7);
      w = 0: 15 -> code 15; w = 1: code 0.
      Stored scale bf16(-0.0666667) = -0.06689453125 (bits 0xBD89; the
      neighbours are -0.06640625 and -0.0673828125), bias 1.0 (0x3F80)."""
    w = np.zeros((1, 64), np.float32)
    w[0, 0] = 1.0
    w[0, 1] = np.float32(0.498667)
    w_q, s, b = oracle.quantize(w, 64, 4, out_dtype="bf16")
    codes = oracle.unpack(w_q, 4)[0]
    assert codes[0] == 0 and codes[1] == 8 and np.all(codes[2:] == 15)
    assert s.tolist() == [[0xBD89]] and b.tolist() == [[0x3F80]]


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


@pytest.mark.parametrize("bits", [4, 8])
def test_qmm_untransposed_brute_force_and_orientation(bits):
    # transpose=False: w_q [K, N*bits/32] quantised along N (groups of gs
    # columns of one row k), y = x . dequant(w); element by element, the code
    # of (k, n) taken straight from its word, the scale of (k, n // gs)
    rng = np.random.default_rng(61 + bits)
    M, K, N, gs = 2, 5, 64, 32
    x = oracle.round_to_dtype(rng.standard_normal((M, K)).astype(np.float32), "f32")
    w_q, s, b = oracle.quantize((rng.standard_normal((K, N)) * 0.02).astype(np.float32), gs, bits,
                                out_dtype="f32")
    vpw, mask = 32 // bits, (1 << bits) - 1
    want = np.zeros((M, N))
    for m in range(M):
        for n in range(N):
            acc = 0.0
            for k in range(K):
                q = (int(w_q[k, n // vpw]) >> (bits * (n % vpw))) & mask
                acc += float(x[m, k]) * (q * float(s[k, n // gs]) + float(b[k, n // gs]))
            want[m, n] = acc
    got = oracle.quantized_matmul(x, w_q, s, b, transpose=False, group_size=gs, bits=bits,
                                  dtype="f32")
    np.testing.assert_allclose(got, want, rtol=1e-12, atol=1e-12)
    # a one-hot activation picks row k of the dequantised [K, N] matrix
    e = np.zeros((1, K), np.float32)
    e[0, 3] = 1.0
    row = oracle.quantized_matmul(e, w_q, s, b, transpose=False, group_size=gs, bits=bits,
                                  dtype="f32")[0]
    np.testing.assert_allclose(row, oracle.dequantize(w_q, s, b, gs, bits, "f32")[3])


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


def test_softcap_rounds_every_step_known_answer():
    """engine/target_gemma4.py:33-40 in bf16, one op and one rounding at a
    time, worked by hand for l = 6.34375, cap = 30 (both exact in bf16):
      l / cap = 0.2114583 -> bf16 (step 2^-10 in [1/8, 1/4)) 217 * 2^-10 =
        0.2119140625;
      tanh(0.2119140625) = 0.2087978 -> 213.81 steps -> 214 * 2^-10 =
        0.208984375;
      0.208984375 * 30 = 6.26953125 -> bf16 (step 2^-5 in [4, 8)) 200.625
        steps -> 201 * 2^-5 = 6.28125 (bits 0x40C9).
    Without the first rounding: tanh(0.2114583) = 0.2083619 -> 213 steps ->
    * 30 = 6.2402 -> 6.25; without the second: 0.2087978 * 30 = 6.26394 ->
    6.25; so an oracle that drops either returns 0x40C8 instead."""
    v = oracle.f32_to_bf16_bits(np.array([6.34375, -6.34375], np.float32))
    out = oracle.logit_softcap(v, 30.0, dtype="bf16")
    assert out.tolist() == [0x40C9, 0xC0C9]


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


# --- GDN rollback pair (oracle/gdn.py) -------------------------------------

def _gdn_case(rng, B, T, Hk, Hv, Dk, Dv, vector_g=False):
    q = rng.standard_normal((B, T, Hk, Dk)).astype(np.float32) / np.sqrt(Dk)
    k = rng.standard_normal((B, T, Hk, Dk)).astype(np.float32) / np.sqrt(Dk)
    v = rng.standard_normal((B, T, Hv, Dv)).astype(np.float32)
    gshape = (B, T, Hv, Dk) if vector_g else (B, T, Hv)
    g = rng.uniform(0.8, 1.0, size=gshape).astype(np.float32)
    beta = rng.uniform(0.1, 0.9, size=(B, T, Hv)).astype(np.float32)
    state = rng.standard_normal((B, Hv, Dv, Dk)).astype(np.float32) * 0.1
    return q, k, v, g, beta, state


@pytest.mark.parametrize("vector_g", [False, True])
def test_gdn_tape_matches_brute_force_loops(vector_g):
    rng = np.random.default_rng(1 + vector_g)
    q, k, v, g, beta, state = _gdn_case(rng, 2, 4, 1, 2, 8, 3, vector_g)
    mask = np.array([[True, True, False, True], [True, False, True, True]])
    for m in (None, mask):
        y, s_out, tape = oracle.gated_delta_with_tape(q, k, v, g, beta, state, m,
                                                      in_dtype="f32", state_dtype="f32")
        y2, s2, t2 = oracle.gated_delta_with_tape_loops(q, k, v, g, beta, state, m)
        assert np.allclose(y, y2, rtol=1e-6, atol=1e-7)
        assert np.allclose(s_out, s2, rtol=1e-6, atol=1e-7)
        assert np.allclose(tape, t2, rtol=1e-6, atol=1e-7)


def test_gdn_closed_forms():
    rng = np.random.default_rng(7)
    q, k, v, g, beta, state = _gdn_case(rng, 1, 3, 2, 4, 8, 5)
    # beta = 0: no innovation, the state only decays
    y, s_out, tape = oracle.gated_delta_with_tape(q, k, v, g, np.zeros_like(beta), state,
                                                  in_dtype="f32", state_dtype="f32")
    assert not tape.any()
    decay = np.prod(g[0].astype(np.float64), axis=0)            # [Hv]
    assert np.allclose(s_out[0], state[0] * decay[:, None, None], rtol=1e-6)
    hk = np.arange(4) // 2
    S1 = state[0].astype(np.float64) * g[0, 0][:, None, None]
    assert np.allclose(y[0, 0], np.einsum("hvk,hk->hv", S1, q[0, 0, hk]), rtol=1e-5, atol=1e-7)
    # one step from a zero state: S = beta v k^T, y = beta v (k . q)
    z = np.zeros_like(state)
    y, s_out, tape = oracle.gated_delta_with_tape(q[:, :1], k[:, :1], v[:, :1], g[:, :1],
                                                  beta[:, :1], z, in_dtype="f32", state_dtype="f32")
    bv = beta[0, 0][:, None] * v[0, 0]                           # [Hv, Dv]
    assert np.allclose(tape[0, 0], bv, rtol=1e-6)
    assert np.allclose(s_out[0], bv[:, :, None] * k[0, 0, hk][:, None, :], rtol=1e-6, atol=1e-8)
    kq = np.einsum("hk,hk->h", k[0, 0, hk].astype(np.float64), q[0, 0, hk])
    assert np.allclose(y[0, 0], bv * kq[:, None], rtol=1e-5, atol=1e-8)
    # every step masked: nothing moves
    y, s_out, tape = oracle.gated_delta_with_tape(q, k, v, g, beta, state,
                                                  np.zeros((1, 3), bool), in_dtype="f32",
                                                  state_dtype="f32")
    assert np.array_equal(s_out, state) and not y.any() and not tape.any()


@pytest.mark.parametrize("vector_g", [False, True])
def test_gdn_replay_reproduces_the_accepted_state(vector_g):
    # the rollback invariant (recurrent_rollback_cache.py:142-165): replaying
    # the first a+1 steps of the tape from the snapshot gives the state the
    # recurrence reached after those steps
    rng = np.random.default_rng(11 + vector_g)
    q, k, v, g, beta, state = _gdn_case(rng, 1, 6, 2, 4, 16, 8, vector_g)
    _, s_full, tape = oracle.gated_delta_with_tape(q, k, v, g, beta, state,
                                                   in_dtype="f32", state_dtype="f32")
    for acc in (1, 3, 6):
        _, s_acc, _ = oracle.gated_delta_with_tape(q[:, :acc], k[:, :acc], v[:, :acc], g[:, :acc],
                                                   beta[:, :acc], state, in_dtype="f32",
                                                   state_dtype="f32")
        rep = oracle.tape_replay(tape[:, :acc], k[:, :acc], g[:, :acc], state, k_dtype="f32",
                                 state_dtype="f32")
        assert np.allclose(rep, s_acc, rtol=2e-6, atol=1e-7)
    assert np.allclose(rep, s_full, rtol=2e-6, atol=1e-7)


def test_gdn_reference_test_inputs():
    # the arange-based inputs of the reference's kernel tests
    # (tests/test_gated_delta_tree_kernel.py:22-54): B=1, T=4, Hk=1, Hv=2,
    # Dk=32, Dv=4, beta 0.25, g 0.91, zero state; replaying the tape over all
    # steps gives the recurrence's final state, and bf16 state rounding per
    # replay step stays within one bf16 step of it
    q = np.arange(4 * 32, dtype=np.float32).reshape(1, 4, 1, 32) / 100.0
    k = (np.arange(4 * 32, dtype=np.float32) + 3).reshape(1, 4, 1, 32) / 110.0
    v = (np.arange(4 * 2 * 4, dtype=np.float32) + 5).reshape(1, 4, 2, 4) / 20.0
    beta = np.full((1, 4, 2), 0.25, np.float32)
    state = np.zeros((1, 2, 4, 32), np.float32)
    for g in (np.full((1, 4, 2), 0.91, np.float32), np.full((1, 4, 2, 32), 0.91, np.float32)):
        y, s_out, tape = oracle.gated_delta_with_tape(q, k, v, g, beta, state, in_dtype="f32",
                                                      state_dtype="f32")
        assert np.all(np.isfinite(y)) and np.abs(s_out).max() > 0
        rep = oracle.tape_replay(tape, k, g, state, k_dtype="f32", state_dtype="f32")
        assert np.allclose(rep, s_out, rtol=2e-6, atol=1e-7)
        rep16 = oracle.to_f32(oracle.tape_replay(tape, k, g, state, k_dtype="f32",
                                                 state_dtype="bf16"), "bf16")
        assert np.all(np.abs(rep16 - s_out) <= 2 * 2.0 ** -8 * np.abs(s_out) + 1e-6)


# ---------------------------------------------------------------- MoE routing / SwiGLU / combine
#
# Each check below is independent of the oracle's own formulas: brute force
# with sorted(), math.exp and a bit-level bf16 rounding written here.

def _bf16_round(v: float) -> float:
    """float -> nearest bf16 value (via float32, round half to even on bits)."""
    import struct

    u = struct.unpack("<I", struct.pack("<f", v))[0]
    u = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
    return struct.unpack("<f", struct.pack("<I", u))[0]


def test_route_topk_brute_force_ties_and_renormalisation():
    import math

    rng = np.random.default_rng(31)
    for trial in range(50):
        E = int(rng.integers(2, 9))
        k = int(rng.integers(1, E + 1))
        lg = rng.integers(-3, 4, size=(3, E)).astype(np.float64) * 0.5  # many exact ties
        ids, sc = oracle.route_topk(lg, k, renormalize=True)
        ids_raw, sc_raw = oracle.route_topk(lg, k, renormalize=False)
        assert np.array_equal(ids, ids_raw)
        for t in range(3):
            den = sum(math.exp(v) for v in lg[t])
            p = [math.exp(v) / den for v in lg[t]]
            # descending probability, lowest expert id first among equals
            want = sorted(range(E), key=lambda e: (-p[e], e))[:k]
            assert ids[t].tolist() == want
            np.testing.assert_allclose(sc_raw[t], [p[e] for e in want], rtol=1e-6)
            assert abs(float(sc[t].astype(np.float64).sum()) - 1.0) < 1e-6
            np.testing.assert_allclose(sc[t], np.array([p[e] for e in want]) / sum(p[e] for e in want),
                                       rtol=1e-6)


def _expert_triple(E, N, K, rng, zero_expert=None):
    ws = []
    for e in range(E):
        w = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
        if e == zero_expert:
            w[:] = 0.0
        ws.append(oracle.quantize(w, 64, 4, out_dtype="bf16"))
    return tuple(np.stack([w[i] for w in ws]) for i in range(3))


def _deq_loop(trip, e, n, k):
    """Dequantised weight by hand: nibble k%8 of word k//8, affine per group."""
    wq, s, b = trip
    q = (int(wq[e, n, k // 8]) >> (4 * (k % 8))) & 0xF
    sc = float(oracle.bf16_bits_to_f32(s[e, n, k // 64]))
    bi = float(oracle.bf16_bits_to_f32(b[e, n, k // 64]))
    return q * sc + bi


def test_switch_glu_zero_gate_gives_zero_h():
    # an expert whose gate weights dequantise to 0 (scale = 1e-7 floor, codes
    # and bias 0 for an all-zero group) has silu(0) = 0, so h = 0 whatever up is
    rng = np.random.default_rng(32)
    T, k, E, D, I = 2, 2, 3, 128, 64
    gate = _expert_triple(E, I, D, rng, zero_expert=1)
    up = _expert_triple(E, I, D, rng)
    down = _expert_triple(E, D, I, rng)
    assert not oracle.dequantize(gate[0][1], gate[1][1], gate[2][1], 64, 4, "f32").any()
    x = oracle.f32_to_bf16_bits(rng.standard_normal((T, D)).astype(np.float32))
    inds = np.array([[1, 0], [2, 1]])
    h, y = oracle.switch_glu(x, inds, gate, up, down, group_size=64, dtype="bf16")
    hf = oracle.bf16_bits_to_f32(h)
    assert not hf[0].any() and not hf[3].any()       # pairs on expert 1
    assert hf[1].any() and hf[2].any()
    # the down projection of a zero activation row is exactly zero
    yf = oracle.bf16_bits_to_f32(y)
    assert not yf[0].any() and not yf[3].any()
    assert yf[1].any() and yf[2].any()


def test_switch_glu_element_loop():
    """2 tokens x 64 -> 64 (k = 2 of 3 experts) against an element-by-element
    loop with math.exp and bf16 rounding after gate, up, sigmoid, gate * sig
    and * up (MLX rounds every op to the activation dtype)."""
    import math

    rng = np.random.default_rng(33)
    T, k, E, D, I = 2, 2, 3, 64, 64
    gate, up, down = (_expert_triple(E, I, D, rng), _expert_triple(E, I, D, rng),
                      _expert_triple(E, D, I, rng))
    x = oracle.f32_to_bf16_bits(rng.standard_normal((T, D)).astype(np.float32))
    xf = oracle.bf16_bits_to_f32(x).astype(np.float64)
    inds = np.array([[2, 0], [1, 2]])
    h, y = oracle.switch_glu(x, inds, gate, up, down, group_size=64, dtype="bf16")
    for t in range(T):
        for j in range(k):
            e = int(inds[t, j])
            hrow = []
            for n in range(I):
                g = _bf16_round(sum(xf[t, kk] * _deq_loop(gate, e, n, kk) for kk in range(D)))
                u = _bf16_round(sum(xf[t, kk] * _deq_loop(up, e, n, kk) for kk in range(D)))
                sig = _bf16_round(1.0 / (1.0 + math.exp(-g)))
                hv = _bf16_round(_bf16_round(g * sig) * u)
                hrow.append(hv)
            got_h = oracle.bf16_bits_to_f32(h[t * k + j]).astype(np.float64)
            # bit-exact: both sides round every op's float64 value to bf16
            # (a dropped rounding point changes some of the 512 values)
            assert got_h.tolist() == hrow
            for n in range(0, D, 7):
                want = _bf16_round(sum(hrow[i] * _deq_loop(down, e, n, i) for i in range(I)))
                assert float(oracle.bf16_bits_to_f32(y[t * k + j, n])) == want


def test_moe_combine_one_hot_and_slot_permutation():
    rng = np.random.default_rng(34)
    T, k, D = 4, 3, 40
    y = oracle.f32_to_bf16_bits(rng.standard_normal((T * k, D)).astype(np.float32))
    # one-hot scores pick the selected pair's row exactly
    sel = rng.integers(0, k, size=T)
    sc = np.zeros((T, k), np.float32)
    sc[np.arange(T), sel] = 1.0
    out = oracle.moe_combine(y, sc, dtype="bf16", out_dtype="bf16")
    for t in range(T):
        assert np.array_equal(out[t], y[t * k + sel[t]])
    # permuting the k slots of each token (rows and scores together) leaves
    # the sum unchanged
    sc = rng.random((T, k)).astype(np.float32)
    base = oracle.moe_combine(y, sc, dtype="bf16")
    perm = np.stack([rng.permutation(k) for _ in range(T)])
    y_p = y.reshape(T, k, D)[np.arange(T)[:, None], perm].reshape(T * k, D)
    sc_p = sc[np.arange(T)[:, None], perm]
    np.testing.assert_allclose(oracle.moe_combine(y_p, sc_p, dtype="bf16"), base, rtol=1e-12)
    # and equals a plain loop
    yf = oracle.bf16_bits_to_f32(y).astype(np.float64)
    for t in range(T):
        want = sum(float(sc[t, j]) * yf[t * k + j] for j in range(k))
        np.testing.assert_allclose(base[t], want, rtol=1e-12)
