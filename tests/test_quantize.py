"""The product's load-time quantiser (dflash-mlx_amd/quantize.py, used by
``QuantizedLinear.from_linear`` and to build the benchmark weights) against
the oracle's restatement of MLX's affine rule, on the CPU: the packed words,
scales and biases must be bit-identical on seeded inputs, and the
reconstruction bounds hold independently of either implementation."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from dflash_mlx_amd.quantize import dequantize, quantize


def _bits16(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("gs", [32, 64, 128])
@pytest.mark.parametrize("std", [0.02, 1.0])
def test_quantize_matches_oracle_bitwise(bits, gs, std):
    rng = np.random.default_rng(bits * 1000 + gs + int(std * 10))
    w = (rng.standard_normal((96, 512)) * std).astype(np.float32)
    # exercise the edge cases of the rule: all-equal groups, all-zero groups,
    # groups whose minimum dominates and whose maximum dominates
    w[0, :gs] = 0.0
    w[1, :gs] = 0.37
    w[2, :gs] = -np.abs(w[2, :gs])
    w[3, :gs] = np.abs(w[3, :gs])
    q_p, s_p, b_p = quantize(torch.from_numpy(w), gs, bits, torch.bfloat16)
    q_o, s_o, b_o = oracle.quantize(w, gs, bits, out_dtype="bf16")
    assert np.array_equal(q_p.numpy().view(np.uint32), q_o)
    assert np.array_equal(_bits16(s_p), s_o)
    assert np.array_equal(_bits16(b_p), b_o)


@pytest.mark.parametrize("bits", [4, 8])
def test_quantize_reconstruction_bounds(bits):
    """Each weight is within half a quantisation step of its reconstruction,
    plus what the bf16 storage of scale and bias moves it (the codes are
    taken against the float32 values, MLX's order: code q moves by at most
    q * 2^-9 steps, the bias by 2^-9 |bias|), and at most one step at the
    clipped ends; codes stay in range, and dequantize is the affine map of
    the codes."""
    rng = np.random.default_rng(bits)
    w = torch.from_numpy((rng.standard_normal((64, 256)) * 0.05).astype(np.float32))
    q, s, b = quantize(w, 64, bits, torch.bfloat16)
    codes = oracle.unpack(q.numpy().view(np.uint32), bits)
    assert codes.min() >= 0 and codes.max() < (1 << bits)
    rec = dequantize(q, s, b, 64, bits)
    step = s.float().abs().repeat_interleave(64, dim=-1)
    err = (rec - w).abs()
    # bf16 storage of scale / bias: at most 2^-9 relative each (2^-8 taken)
    cf = torch.from_numpy(codes.astype(np.float32))
    storage = 2.0 ** -8 * (cf * step + b.float().abs().repeat_interleave(64, dim=-1))
    slack = 2.0 ** -8 * (1 << bits)
    interior = torch.from_numpy((codes > 0) & (codes < (1 << bits) - 1))
    assert bool((err[interior] <= 0.5 * step[interior] + storage[interior] + 1e-7).all())
    # the snapped scale can clip the far end of the range by one step
    assert bool((err <= step * (1.0 + slack) + storage + 1e-7).all())
    by_hand = torch.from_numpy(codes.astype(np.float32)) * s.float().repeat_interleave(64, -1) \
        + b.float().repeat_interleave(64, -1)
    assert torch.equal(rec, by_hand)
