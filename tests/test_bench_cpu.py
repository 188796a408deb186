"""bench.py's accounting, on the CPU: the algorithmic bytes of each workload
against the closed-form figures of the byte formula N·K·bits/8 + 4·N·K/gs +
2·M·K + 2·M·N (packed weights, bf16 scales and biases, activations in, rows
out), and the committed counter summaries it reads."""

from __future__ import annotations

import json
import os

import bench

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_single_call_bytes():
    # [16,4096] x [4096,4096] int4 gs64: 8 MiB of nibbles + 1 MiB of scales/biases
    # + 128 KiB of x + 128 KiB of y
    assert bench.alg_bytes(16, 4096, 4096) == 8 * 2**20 + 2**20 + 2 * 2**17 == 9_699_328


def test_sweep_bytes():
    per_layer = sum(bench.alg_bytes(16, K, N) for (_, K, N) in bench.SHAPES_9B)
    assert 32 * per_layer == 3_550_478_336
    # 27B at M = 8 / 16 / 32
    for M, want in ((8, 11_993_612_288), (16, 12_096_372_736), (32, 12_301_893_632)):
        assert 64 * sum(bench.alg_bytes(M, K, N) for (_, K, N) in bench.SHAPES_27B) == want


def test_eight_bit_bytes():
    # 8-bit weights: one byte per weight, scales/biases unchanged
    assert bench.alg_bytes(16, 4096, 4096, bits=8) == 16 * 2**20 + 2**20 + 2 * 2**17


def test_lmhead_bytes():
    M, K, V = 16, 5120, 151936
    nbytes = V * K // 2 + 4 * V * K // 64 + 2 * M * K + 12 * M
    assert nbytes == 388_956_160 + 48_619_520 + 163_840 + 192
    assert abs(nbytes / 1e6 - 437.74) < 0.01


def test_mfma_report():
    r = bench.mfma_report("no-such-workload", "k", 2 * 16 * 4096 * 4096, 5.0)
    assert r["busy_pct_counter"] is None
    assert abs(r["achieved_tflops"] - 2 * 16 * 4096 * 4096 / 5e-6 / 1e12) < 0.01
    assert abs(r["frac"] - r["achieved_tflops"] / bench.MFMA_PEAK_TFLOPS) < 1e-5


def test_committed_counter_summaries_are_read():
    with open(os.path.join(ROOT, "profiles", "traffic.json")) as f:
        traffic = json.load(f)
    for workload, kernels in traffic.items():
        for kernel, e in kernels.items():
            assert bench.measured_traffic(workload, kernel) == e["bytes_per_launch"]
            # measured = scaled FETCH + scaled WRITE, never below the algorithmic bytes
            assert e["bytes_per_launch"] == e["fetch_bytes_per_launch"] + e["write_bytes_per_launch"]
            assert e["bytes_per_launch"] >= e["algorithmic_bytes_per_launch"]
    with open(os.path.join(ROOT, "profiles", "mfma.json")) as f:
        mfma = json.load(f)
    for workload, kernels in mfma.items():
        for kernel, e in kernels.items():
            r = bench.mfma_report(workload, kernel, 1e9, 10.0)
            assert r["busy_pct_counter"] == e["util_pct"]
            assert 0 < e["util_pct"] < 100
