"""GDN rollback pair on the GPU (dfmi_gated_delta_tape, dfmi_tape_replay)
against the oracle (oracle/gdn.py, restating dflash_mlx/kernels.py:11-219 and
691-866) on the same seeded inputs.

Tolerances (written here): the recurrence carries its state in fp32 on both
sides with different summation orders, so the fp32 outputs (state, tape) must
agree to 1e-4 of their largest magnitude; outputs rounded to bf16 / f16 (y,
replayed states) to the parity metric 1e-2 and 4 units in the last place
elementwise.  The rollback invariant is checked on the GPU itself: replaying
the kernel's own tape over the first a+1 steps gives the state the kernel
reaches after those steps.
"""

from __future__ import annotations

import numpy as np
import pytest

import oracle

from .conftest import from_dev, to_dev

pytestmark = pytest.mark.gpu


def _case(seed, B, T, Hk, Hv, Dk, Dv, vector_g=False):
    rng = np.random.default_rng(seed)
    q = rng.standard_normal((B, T, Hk, Dk)).astype(np.float32) / np.sqrt(Dk)
    k = rng.standard_normal((B, T, Hk, Dk)).astype(np.float32) / np.sqrt(Dk)
    v = rng.standard_normal((B, T, Hv, Dv)).astype(np.float32)
    g = rng.uniform(0.85, 1.0, size=(B, T, Hv, Dk) if vector_g else (B, T, Hv)).astype(np.float32)
    beta = rng.uniform(0.1, 0.9, size=(B, T, Hv)).astype(np.float32)
    state = (rng.standard_normal((B, Hv, Dv, Dk)) * 0.1).astype(np.float32)
    return q, k, v, g, beta, state


def _st(a, dtype):
    return oracle.round_to_dtype(a, dtype)


def _close_f32(got, want, tol=1e-4):
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    assert got.shape == want.shape
    assert np.all(np.isfinite(got))
    assert np.abs(got - want).max() <= tol * (np.abs(want).max() + 1e-6)


def _close_lowp(got_bits, want_bits, dtype, ulps=4):
    g = oracle.to_f32(got_bits, dtype).astype(np.float64)
    w = oracle.to_f32(want_bits, dtype).astype(np.float64)
    _, rel = oracle.parity_metrics(g, w)
    assert rel <= 1e-2, rel
    ulp = 2.0 ** -8 if dtype == "bf16" else 2.0 ** -11
    assert np.all(np.abs(g - w) <= ulps * ulp * np.abs(w) + 1e-3 * np.abs(w).max() + 1e-6)


def _dev_tensors(dev, dtypes, q, k, v, g, beta, state):
    xd, gd, bd, sd = dtypes
    return (to_dev(_st(q, xd), xd, dev), to_dev(_st(k, xd), xd, dev), to_dev(_st(v, xd), xd, dev),
            to_dev(_st(g, gd), gd, dev), to_dev(_st(beta, bd), bd, dev),
            to_dev(_st(state, sd), sd, dev))


SHAPES = [  # B, T, Hk, Hv, Dk, Dv
    (1, 16, 16, 32, 128, 128),   # a GDN target's verify block (Qwen3-Next-like heads)
    (1, 4, 1, 2, 32, 4),         # the reference tests' shape
    (2, 7, 2, 4, 64, 20),        # Dv not a multiple of the 8 rows per workgroup
    (1, 40, 2, 2, 128, 16),      # several staged chunks of steps
    (1, 9, 1, 2, 512, 8),        # widest key dimension (4 steps per chunk)
    (1, 5, 2, 6, 256, 12),
]


@pytest.mark.parametrize("B,T,Hk,Hv,Dk,Dv", SHAPES)
@pytest.mark.parametrize("vector_g", [False, True])
def test_gated_delta_tape_matches_oracle(dev, B, T, Hk, Hv, Dk, Dv, vector_g):
    from dflash_mlx_amd.gdn import gated_delta_kernel_with_tape

    q, k, v, g, beta, state = _case(B * 131 + T + Dk + vector_g, B, T, Hk, Hv, Dk, Dv, vector_g)
    dtypes = ("bf16", "f32", "bf16", "f32")  # the target's q/k/v, g, beta, state
    y, s_out, tape = gated_delta_kernel_with_tape(*_dev_tensors(dev, dtypes, q, k, v, g, beta, state))
    wy, ws, wt = oracle.gated_delta_with_tape(_st(q, "bf16"), _st(k, "bf16"), _st(v, "bf16"),
                                              g, _st(beta, "bf16"), state, in_dtype="bf16",
                                              state_dtype="f32", g_dtype="f32",
                                              beta_dtype="bf16")
    _close_lowp(from_dev(y, "bf16"), wy, "bf16")
    _close_f32(from_dev(s_out, "f32"), ws)
    _close_f32(from_dev(tape, "f32"), wt)


@pytest.mark.parametrize("dtypes", [("f32", "f32", "f32", "f32"), ("bf16", "bf16", "bf16", "bf16"),
                                    ("f16", "f32", "f16", "f32")])
def test_gated_delta_tape_dtypes_and_mask(dev, dtypes):
    import torch

    from dflash_mlx_amd.gdn import gated_delta_kernel_with_tape

    B, T, Hk, Hv, Dk, Dv = 2, 6, 2, 4, 64, 24
    q, k, v, g, beta, state = _case(77, B, T, Hk, Hv, Dk, Dv)
    mask = np.array([[1, 1, 0, 1, 0, 1], [0, 1, 1, 1, 1, 0]], bool)
    xd, gd, bd, sd = dtypes
    y, s_out, tape = gated_delta_kernel_with_tape(*_dev_tensors(dev, dtypes, q, k, v, g, beta, state),
                                                  mask=torch.tensor(mask, device=dev))
    wy, ws, wt = oracle.gated_delta_with_tape(_st(q, xd), _st(k, xd), _st(v, xd), _st(g, gd),
                                              _st(beta, bd), _st(state, sd), mask, in_dtype=xd,
                                              state_dtype=sd, g_dtype=gd, beta_dtype=bd)
    if xd == "f32":
        _close_f32(from_dev(y, "f32"), wy)
    else:
        _close_lowp(from_dev(y, xd), wy, xd)
    if sd == "f32":
        _close_f32(from_dev(s_out, "f32"), ws)
    else:
        _close_lowp(from_dev(s_out, sd), ws, sd)
    got_tape = from_dev(tape, "f32")
    _close_f32(got_tape, wt)
    assert not got_tape[~mask].any()                       # masked steps record no innovation
    assert not oracle.to_f32(from_dev(y, xd), xd)[~mask].any()


@pytest.mark.parametrize("state_dtype", ["f32", "bf16"])
@pytest.mark.parametrize("vector_g", [False, True])
def test_tape_replay_matches_oracle_and_rolls_back(dev, state_dtype, vector_g):
    import torch

    from dflash_mlx_amd.gdn import gated_delta_kernel_with_tape, tape_replay_kernel

    B, T, Hk, Hv, Dk, Dv = 1, 16, 4, 8, 128, 64
    q, k, v, g, beta, state = _case(5 + vector_g, B, T, Hk, Hv, Dk, Dv, vector_g)
    dtypes = ("bf16", "f32", "bf16", state_dtype)
    qd, kd, vd, gd, bd, sd = _dev_tensors(dev, dtypes, q, k, v, g, beta, state)
    _, _, tape = gated_delta_kernel_with_tape(qd, kd, vd, gd, bd, sd)
    got_tape = from_dev(tape, "f32")
    for acc in (0, 5, 15):  # accepted drafts; the replay covers acc + 1 steps
        n = acc + 1
        rep = tape_replay_kernel(tape[:, :n], kd[:, :n], gd[:, :n], sd)
        want = oracle.tape_replay(got_tape[:, :n], _st(k, "bf16")[:, :n], g[:, :n],
                                  _st(state, state_dtype), k_dtype="bf16",
                                  state_dtype=state_dtype, g_dtype="f32")
        if state_dtype == "f32":
            _close_f32(from_dev(rep, "f32"), want)
            # rollback invariant on the GPU: the recurrence run for n steps
            _, s_n, _ = gated_delta_kernel_with_tape(qd[:, :n], kd[:, :n], vd[:, :n], gd[:, :n],
                                                     bd[:, :n], sd)
            _close_f32(from_dev(rep, "f32"), from_dev(s_n, "f32"))
        else:
            _close_lowp(from_dev(rep, "bf16"), want, "bf16")
    # a fully masked replay returns the snapshot unchanged
    rep0 = tape_replay_kernel(tape, kd, gd, sd, mask=torch.zeros((B, T), dtype=torch.bool, device=dev))
    assert torch.equal(rep0, sd)


def test_gdn_state_may_alias(dev):
    # the C ABI allows state_out == state_in (each workgroup reads its rows
    # before writing them): replay in place equals replay out of place
    import torch

    from dflash_mlx_amd import _lib, _runtime
    from dflash_mlx_amd.gdn import gated_delta_kernel_with_tape, tape_replay_kernel

    B, T, Hk, Hv, Dk, Dv = 1, 8, 2, 4, 128, 32
    q, k, v, g, beta, state = _case(9, B, T, Hk, Hv, Dk, Dv)
    qd, kd, vd, gd, bd, sd = _dev_tensors(dev, ("bf16", "f32", "bf16", "f32"), q, k, v, g, beta, state)
    _, _, tape = gated_delta_kernel_with_tape(qd, kd, vd, gd, bd, sd)
    want = tape_replay_kernel(tape, kd, gd, sd)
    inplace = sd.clone()
    lib = _lib.load()
    _lib.check(lib.dfmi_tape_replay(tape.data_ptr(), kd.data_ptr(), gd.data_ptr(), inplace.data_ptr(),
                                    None, inplace.data_ptr(), B, T, Hk, Hv, Dk, Dv, _lib.DFMI_BF16,
                                    _lib.DFMI_F32, _lib.DFMI_F32, 0, _runtime.stream_ptr(dev)),
               "dfmi_tape_replay")
    torch.cuda.synchronize()
    assert torch.equal(inplace, want)
