"""Writes tests/golden/reference_cases.json -- data the reference's own tests
and dispatch rules hold for the verify path.  Nothing here imports or runs
reference code: the values are the literal cases of the reference tests and
the outcomes its (restated) dispatch predicates give, with the file:line
they come from.  Run: ``python tests/golden/make_golden.py``.
"""

from __future__ import annotations

import json
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))


def random_shapes(n=30, seed=0xDF1A, group_size=64):
    """tests/test_verify_qmm_parity.py:32-42 (shape list only; its value seeds
    use per-process randomized hash() and are not reproducible)."""
    rng = np.random.default_rng(seed)
    levels = [1, 4, 8, 12, 15, 16]
    out = []
    for i in range(n):
        m = levels[i % len(levels)]
        k = int(rng.integers(2, 40)) * group_size
        nn = int(rng.integers(1, 64)) * 8
        out.append([f"rnd{i:02d}", m, k, nn])
    return out


def main():
    cases = {
        "source": "shaneholloman/dflash-mlx 0.1.7 tests and dispatch rules (read as text)",
        # tests/test_engine_acceptance.py:12-18: (drafted, posterior, expected)
        "acceptance_cases": [
            [[], [], 0],
            [[1, 2, 3, 4], [1, 2, 3, 4], 4],
            [[5, 5, 5], [1, 5, 5], 0],
            [[1, 2, 9, 4, 5], [1, 2, 3, 4, 5], 2],
            [[7, 7, 7, 0], [7, 7, 7, 1], 3],
        ],
        # tests/test_verify_qmm_parity.py:16-27
        "real_mlp_shapes": [
            ["gate_proj", 16, 5120, 17408], ["up_proj", 16, 5120, 17408],
            ["down_proj", 16, 17408, 5120],
            ["gate_proj_m4", 4, 5120, 17408], ["up_proj_m4", 4, 5120, 17408],
            ["down_proj_m4", 4, 17408, 5120],
        ],
        "random_shapes": random_shapes(),
        # tests/test_verify_qmm_parity.py:77-81, 96-100 (bf16 abs, fp16 abs, rel)
        "reference_tolerances": {"bf16_abs": 8e-3, "f16_abs": 4e-3, "rel": 2e-2},
        # Default-env M=16 / M=4 kernel per 9B / 27B layer shape: dflash_mlx/verify_qmm.py:21-51,
        # verify_linear.py:141-211 -> [K, N, m16_variant, m4_kparts]
        "dispatch_table": [
            [4096, 4096, "combo_ktmpl", 2], [4096, 1024, "combo_ktmpl", 4],
            [4096, 12288, "super_tree_fp16_ktmpl", 2], [12288, 4096, "combo_ktmpl", 2],
            [5120, 5120, "combo_ktmpl", 2], [5120, 1024, "combo_ktmpl", 4],
            [5120, 17408, "super_tree_fp16_ktmpl", 2], [17408, 5120, "combo_ktmpl", 2],
        ],
        # tests/test_verify_linear_parity.py:31-39, 140-159 and verify_linear.py:54-87:
        # [K, N, bits, group_size, eligible]
        "eligibility": [
            [512, 1024, 4, 64, True], [512, 150000, 4, 64, False], [512, 16, 4, 64, True],
            [64, 12, 4, 64, True], [512, 1000, 8, 64, False], [512, 1024, 8, 64, True],
            [512, 1024, 4, 16, False], [512, 1024, 3, 64, False], [48, 1024, 4, 16, False],
        ],
        # engine/target_qwen_gdn.py:811-828 and tests/test_target_ops.py:341-366:
        # [num_layers, hidden, heads, kv_heads, num_experts, supports_verify_linear]
        "verify_linear_policy": [
            [40, 2048, 16, 2, 128, False], [40, 5120, 40, 8, 128, True],
            [32, 4096, 32, 8, 0, False], [64, 5120, 40, 8, 0, True], [40, 4096, 32, 8, 0, True],
        ],
    }
    path = os.path.join(HERE, "reference_cases.json")
    with open(path, "w") as f:
        f.write("{\n")
        items = list(cases.items())
        for i, (key, val) in enumerate(items):
            sep = "," if i + 1 < len(items) else ""
            f.write(f" {json.dumps(key)}: {json.dumps(val)}{sep}\n")
        f.write("}\n")
    print(f"wrote {path}")


if __name__ == "__main__":
    main()
