"""dflash-mlx target-verify hot path, MI355X-native (gfx950 HIP kernels).

Operator API (same names and meaning as the reference's):

* ``verify_qmm.verify_matmul`` / ``verify_qmm.is_enabled``
  (dflash_mlx/verify_qmm.py) and ``verify_qmm.quantized_matmul`` (the stock
  quantized matmul the verify path falls back to);
* ``verify_linear.QuantizedLinear``, ``VerifyQuantizedLinear``,
  ``is_verify_eligible``, ``install_verify_linears``,
  ``prewarm_verify_kernels`` (dflash_mlx/verify_linear.py);
* ``sampling.greedy_tokens_with_mask``, ``sampling.build_suppress_token_mask``
  (dflash_mlx/engine/sampling.py) and ``acceptance.match_acceptance_length``
  (dflash_mlx/engine/acceptance.py);
* ``lm_head.lm_head_greedy_accept`` -- lm_head + greedy + accept fused;
* ``moe.gather_qmm`` / ``moe.switch_glu`` -- the routed-expert matmuls.

The directory name contains a hyphen, so the package is imported as
``dflash_mlx_amd`` through ``__graft_entry__.load_package()``.
"""

__version__ = "0.1.0"
