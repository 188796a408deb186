"""Host-side routing, eligibility, install and load-time policy (CPU only).

Known answers restated from the reference's tests and dispatch rules
(tests/golden/reference_cases.json, written by tests/golden/make_golden.py
from tests/test_verify_linear_parity.py:31-159, tests/test_target_ops.py:341-385,
tests/test_runtime_verify_config.py:90-241 and dflash_mlx/verify_qmm.py:21-51).
"""

from __future__ import annotations

import json
import os

import pytest
import torch
from torch import nn

from dflash_mlx_amd import policy, verify_linear, verify_qmm

GOLD = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "reference_cases.json")))


def _ql(K, N, bits=4, gs=64, bias=False):
    w = torch.zeros((N, K * bits // 32), dtype=torch.int32)
    s = torch.ones((N, K // gs), dtype=torch.bfloat16)
    b = torch.zeros((N, K // gs), dtype=torch.bfloat16)
    return verify_linear.QuantizedLinear(w, s, b, torch.zeros(N, dtype=torch.bfloat16) if bias else None,
                                         group_size=gs, bits=bits)


@pytest.mark.parametrize("K,N,variant,m4_kparts", GOLD["dispatch_table"])
def test_m16_variant_and_m4_kparts_known_answers(K, N, variant, m4_kparts):
    assert verify_qmm._m16_ktmpl_variant(K, N, 4) == variant
    assert verify_qmm._resolve_m16_ktmpl_variant(K, N, 4, "auto") == variant
    assert verify_qmm._m4_ksplit_np_kparts(N) == m4_kparts


def test_variant_rules_outside_the_table():
    # the k-templated kernels need K % 256 == 0 and N % 16 == 0 and bits 4
    assert verify_qmm._m16_ktmpl_variant(4096 + 32, 4096, 4) is None
    assert verify_qmm._m16_ktmpl_variant(4096, 4104, 4) is None
    assert verify_qmm._m16_ktmpl_variant(4096, 4096, 8) is None
    # explicit variant overrides auto; unknown names fall through to mma2big*
    assert verify_qmm._resolve_m16_ktmpl_variant(4096, 12288, 4, "combo_ktmpl") == "combo_ktmpl"
    assert verify_qmm._resolve_m16_ktmpl_variant(4096, 12288, 4, "mma2big") is None
    # _auto_variant (verify_qmm.py:21-24)
    assert verify_qmm._auto_variant(8192, 20000) == ("mma2big_pipe", 8)
    assert verify_qmm._auto_variant(4096, 8192) == ("mma2big_pipe", 8)
    assert verify_qmm._auto_variant(4096, 8193) == ("mma2big", 1)


def test_verify_route_fallbacks():
    # M=4 needs bits 4, N % 4 == 0, K % 32 == 0
    assert verify_qmm.verify_route(4, 4096, 1024, 4)[0] == "m4_ksplit_np"
    assert verify_qmm.verify_route(4, 4096, 1026, 4)[0] == "stock"
    assert verify_qmm.verify_route(4, 4096, 1024, 8)[0] == "stock"
    # M=16, K % 256 != 0: auto -> mma2big_pipe(8) needs K % 256 == 0 -> stock ...
    assert verify_qmm.verify_route(16, 4128, 4096, 4)[0] == "stock"
    # ... while an N > 8192 shape with K < 8192 takes plain mma2big
    assert verify_qmm.verify_route(16, 4128, 8224, 4)[0] == "mma2big"
    # N % 32 != 0 outside the k-templated shapes -> stock
    assert verify_qmm.verify_route(16, 4128, 4112, 4)[0] == "stock"


def test_verify_route_launch_shape(monkeypatch):
    """The mma2big routes admit calls by the reference's rules but launch the
    library's automatic plan (the reference's K_PARTS defaults are Metal
    launch choices): 8-bit gate/up at M=16 must not be forced to one split.
    DFLASH_VERIFY_QMM_KPARTS, when the user sets it, becomes the split count."""
    assert verify_qmm.verify_route(16, 4096, 12288, 8) == ("mma2big", None)
    assert verify_qmm.verify_route(16, 4096, 4096, 8) == ("mma2big_pipe", None)
    assert verify_qmm.verify_route(16, 4128, 8224, 4) == ("mma2big", None)
    monkeypatch.setenv("DFLASH_VERIFY_QMM_KPARTS", "4")
    name, t = verify_qmm.verify_route(16, 4096, 12288, 8)
    assert name == "mma2big" and (t.k_splits, t.waves_per_block) == (4, 4)
    monkeypatch.setenv("DFLASH_VERIFY_QMM_KPARTS", "0")
    assert verify_qmm.verify_route(16, 4096, 12288, 8) == ("mma2big", None)


def test_module_dispatch_launch_shape(monkeypatch):
    """VerifyQuantizedLinear's precomputed M=16 route uses the same launch
    shape as verify_matmul (automatic unless DFLASH_VERIFY_QMM_KPARTS is set)."""
    def forced(mod):  # launch-shape overrides captured by the module's call
        return [c.cell_contents.k_splits for c in (mod._call_fn.__closure__ or ())
                if hasattr(c.cell_contents, "k_splits")]

    monkeypatch.setenv("DFLASH_VERIFY_QMM", "1")
    assert forced(verify_linear.VerifyQuantizedLinear.from_quantized(_ql(4096, 12288, bits=8))) == []
    monkeypatch.setenv("DFLASH_VERIFY_QMM_KPARTS", "4")
    assert forced(verify_linear.VerifyQuantizedLinear.from_quantized(_ql(4096, 12288, bits=8))) == [4]


@pytest.mark.parametrize("K,N,bits,gs,eligible", GOLD["eligibility"])
def test_eligibility_known_answers(K, N, bits, gs, eligible):
    if K * bits % 32:
        pytest.skip("not representable as packed words")
    assert verify_linear.is_verify_eligible(_ql(K, N, bits, gs)) is eligible


def test_eligibility_flags(monkeypatch):
    ql = _ql(512, 1024)
    assert verify_linear.is_verify_eligible(ql, path="model.layers.0.mlp.gate_proj")
    monkeypatch.setenv("DFLASH_VERIFY_MAX_N", "1024")
    assert not verify_linear.is_verify_eligible(ql)
    monkeypatch.delenv("DFLASH_VERIFY_MAX_N")
    monkeypatch.setenv("DFLASH_VERIFY_INCLUDE", "attn")
    assert not verify_linear.is_verify_eligible(ql, path="model.layers.0.mlp.gate_proj")
    assert verify_linear.is_verify_eligible(ql, path="model.layers.0.self_attn.q_proj")
    monkeypatch.setenv("DFLASH_VERIFY_INCLUDE", "mlp_down,attn_o")
    assert verify_linear.is_verify_eligible(ql, path="model.layers.3.mlp.down_proj")
    assert not verify_linear.is_verify_eligible(ql, path="model.layers.3.mlp.up_proj")
    assert not verify_linear.is_verify_eligible(nn.Linear(512, 1024))


def _toy_model():
    m = nn.Module()
    m.layers = nn.ModuleList()
    for _ in range(2):
        layer = nn.Module()
        layer.mlp = nn.Module()
        layer.mlp.gate_proj = _ql(512, 1024)
        layer.mlp.up_proj = _ql(512, 1024)
        layer.mlp.down_proj = _ql(1024, 512, bias=True)
        layer.mlp.odd = _ql(512, 150000 // 4 * 4 + 4)  # too wide: stays stock
        layer.norm = nn.LayerNorm(8)
        m.layers.append(layer)
    m.lm_head = nn.Linear(8, 8)
    return m


def test_install_counts_and_idempotence():
    m = _toy_model()
    assert verify_linear.install_verify_linears(m) == 6
    assert isinstance(m.layers[1].mlp.down_proj, verify_linear.VerifyQuantizedLinear)
    assert not isinstance(m.layers[0].mlp.odd, verify_linear.VerifyQuantizedLinear)
    assert verify_linear.install_verify_linears(m) == 0
    m2 = _toy_model()
    only_gate = verify_linear.install_verify_linears(m2, predicate=lambda p, q: p.endswith("gate_proj"))
    assert only_gate == 2


@pytest.mark.parametrize("layers,hidden,heads,kv,experts,expected", GOLD["verify_linear_policy"])
def test_target_policy_known_answers(layers, hidden, heads, kv, experts, expected):
    assert policy.supports_verify_linear(num_layers=layers, num_experts=experts,
                                         hidden_size=hidden, num_heads=heads,
                                         num_kv_heads=kv) is expected


def test_verify_config_and_loader_gate(monkeypatch):
    assert policy.VerifyConfig.from_mode(None).mode == "dflash"
    assert policy.VerifyConfig.from_mode(" Adaptive ").mode == "adaptive"
    with pytest.raises(ValueError):
        policy.VerifyConfig.from_mode("fast")
    off = policy.VerifyConfig.from_mode("off")
    assert not policy.verify_enabled_for(off)
    assert policy.verify_enabled_for(policy.VerifyConfig())
    assert policy.verify_enabled_for(None)
    monkeypatch.setenv("DFLASH_VERIFY_LINEAR", "0")
    assert not policy.verify_enabled_for(None)
    assert policy.verify_enabled_for(policy.VerifyConfig())  # config wins over env
    assert not policy.verify_qmm_enabled_for(None)
    monkeypatch.setenv("DFLASH_VERIFY_QMM", "1")
    assert policy.verify_qmm_enabled_for(None)
    assert not policy.verify_qmm_enabled_for(policy.VerifyConfig(enable_qmm=False))
    m = _toy_model()
    assert policy.install_for_target(m, supports_verify_linear_=True, verify_config=off) == 0
    assert policy.install_for_target(m, supports_verify_linear_=False) == 0
    assert policy.install_for_target(m, supports_verify_linear_=True,
                                     verify_config=policy.VerifyConfig()) == 6
