"""CPU oracle for the dflash-mlx target-verify hot path (TEST INFRASTRUCTURE ONLY).

This package restates, in plain numpy, the arithmetic that the reference
(shaneholloman/dflash-mlx 0.1.7) and the MLX operators it calls perform on the
verify path.  It is the reference the HIP kernels are tested against: only ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may import
it, and never as the thing measured or shipped.  The product package must not
import it.

Functions and what pins each one (see ``tests/test_oracle.py``):

* ``pack`` / ``unpack``          -- packed-weight layout, restated from the
  reference kernels' unpack ``(w_q[n, k/8] >> 4*(k%8)) & 0xF``
  (dflash_mlx/verify_qmm.py:97-115, 243-249; 8-bit: 593-598).  Pinned by
  hand-built words (0x76543210 -> 0..7) and pack/unpack round trips.
* ``quantize``                   -- MLX affine quantize (mlx >= 0.31, the
  ``mx.quantize`` the reference tests call at tests/test_verify_qmm_parity.py:29-30).
  MLX is not vendored and not importable here: restated from its published
  algorithm.  Pinned by invariants (codes in range, per-group reconstruction
  error <= scale/2, exact on grids that are already affine) -- bit parity with
  mx.quantize itself is *parity unpinned* (it never affects matmul parity: both
  sides consume the same packed tensors).
* ``dequantize`` / ``quantized_matmul`` -- ``y = x . dequant(W)^T`` (the
  operator contract of verify_matmul, dflash_mlx/verify_qmm.py:905-1022, and of
  mx.quantized_matmul).  Exact float64 accumulate, optional RNE cast to the
  output dtype.  Pinned by closed-form integer cases (scale=1, bias=0), by a
  brute-force triple loop on tiny shapes, and by linearity.
* ``gather_qmm``                 -- mx.gather_qmm(transpose=True) restated as
  one quantized_matmul per (lhs, rhs) index pair (mlx-lm SwitchGLU call site).
  Pinned by reduction to quantized_matmul on single-expert routings.
* ``build_suppress_token_mask`` / ``greedy_tokens_with_mask`` --
  dflash_mlx/engine/sampling.py:29-55 (argmax over the masked logits, masked
  ids set to the logits dtype's -1e9, first index wins ties).
* ``match_acceptance_length``    -- dflash_mlx/engine/acceptance.py:9-16.
  Pinned by the reference's five known answers
  (tests/test_engine_acceptance.py:11-24) and brute force.
* ``verify_cycle_accept``        -- ids/accept/bonus semantics of one verify
  cycle, dflash_mlx/engine/spec_epoch.py:2011-2021, 2067-2072, 2129.
* ``logit_softcap``              -- dflash_mlx/engine/target_gemma4.py:33-40,
  op-by-op rounding to the logits dtype (parity unpinned against MLX's tanh).
* ``gated_delta_with_tape`` / ``tape_replay`` -- the GDN rollback pair,
  dflash_mlx/kernels.py:11-219 and 691-866 (gdn.py).  Pinned by a brute-force
  loop form, closed forms (beta = 0; one step from a zero state), masked
  steps, and the rollback invariant: replaying the full tape reproduces the
  recurrence's final state.

bf16 tensors are carried as ``uint16`` bit patterns; fp16 as ``numpy.float16``.
"""

from .numerics import (  # noqa: F401
    bf16_bits_to_f32,
    f32_to_bf16_bits,
    round_to_dtype,
    to_f32,
)
from .qmm import (  # noqa: F401
    dequantize,
    gather_qmm,
    pack,
    quantize,
    quantized_matmul,
    unpack,
    parity_metrics,
)
from .greedy import (  # noqa: F401
    build_suppress_token_mask,
    greedy_tokens_with_mask,
    logit_softcap,
    match_acceptance_length,
    verify_cycle_accept,
)
from .moe import (  # noqa: F401
    route_topk,
    switch_glu,
    moe_combine,
)
from .gdn import (  # noqa: F401
    gated_delta_with_tape,
    gated_delta_with_tape_loops,
    tape_replay,
)
