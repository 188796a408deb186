"""The drop-in module on the GPU: the reference's bit-identity invariants for
``VerifyQuantizedLinear`` (tests/test_verify_linear_parity.py:41-138) and the
disabled-path identity of ``verify_matmul``
(tests/test_verify_qmm_parity.py:102-106), restated with this framework's
modules; plus the bias add (dflash_mlx/verify_linear.py:250,261) and 8-bit
modules on the 9B layer shapes against the oracle.

Bit-identity is the reference's own bar for these (``allclose(atol=0,
rtol=0)``); tolerance checks use the oracle and the 1e-2 metric."""

from __future__ import annotations

import numpy as np
import pytest

import oracle
from tests.conftest import from_dev

pytestmark = pytest.mark.gpu

REL_TOL = 1e-2


def _mk_ql(dev, K, N, *, bits=4, gs=64, bias=False, seed=0, std=0.1):
    import torch

    from dflash_mlx_amd.verify_linear import QuantizedLinear

    g = torch.Generator(device="cpu").manual_seed(seed)
    lin = torch.nn.Linear(K, N, bias=bias)
    with torch.no_grad():
        lin.weight.copy_((torch.randn((N, K), generator=g) * std).to(torch.bfloat16))
        if bias:
            lin.bias.copy_(torch.randn((N,), generator=g))
    ql = QuantizedLinear.from_linear(lin.to(dev), group_size=gs, bits=bits, dtype=torch.bfloat16)
    return ql


def _x(dev, M, K, seed=1, scale=0.5):
    import torch

    g = torch.Generator(device="cpu").manual_seed(seed)
    return (torch.randn((M, K), generator=g) * scale).to(torch.bfloat16).to(dev)


def _direct(ql, x):
    from dflash_mlx_amd.verify_qmm import verify_matmul

    return verify_matmul(x, ql.weight, ql.scales, ql.biases, transpose=True,
                         group_size=ql.group_size, bits=ql.bits)


def _oracle_check(ql, x, y):
    import torch

    xs = from_dev(x, "bf16")
    w = ql.weight.cpu().numpy().view(np.uint32)
    s = from_dev(ql.scales, "bf16")
    b = from_dev(ql.biases, "bf16")
    want = oracle.quantized_matmul(xs, w, s, b, group_size=ql.group_size, bits=ql.bits)
    if ql.has_bias():
        want = want + oracle.to_f32(from_dev(ql.bias, "bf16"), "bf16")
    got = oracle.to_f32(from_dev(y, "bf16"), "bf16")
    _, rel = oracle.parity_metrics(got, want)
    assert rel <= REL_TOL, rel
    torch.cuda.synchronize()


@pytest.mark.parametrize("M", [1, 8, 32])
def test_parity_non_verify_is_stock(dev, monkeypatch, M):
    # test_verify_linear_parity.py:41-49: M outside {4, 16} routes through
    # the stock matmul, bit-identical to the unswapped module
    import torch

    from dflash_mlx_amd.verify_linear import VerifyQuantizedLinear

    monkeypatch.setenv("DFLASH_VERIFY_QMM", "1")
    ql = _mk_ql(dev, 512, 1024)
    verify = VerifyQuantizedLinear.from_quantized(ql)
    x = _x(dev, M, 512)
    assert torch.equal(verify(x), ql(x))


@pytest.mark.parametrize("M,K,N", [(16, 512, 1024), (16, 512, 16), (4, 512, 1024), (4, 64, 12),
                                   (16, 4096, 12288), (4, 5120, 1024)])
def test_wrapper_matches_direct_bitwise(dev, monkeypatch, M, K, N):
    # test_verify_linear_parity.py:51-72 (M=16, N=1024 and N=16) and 116-138
    # (M=4, N=1024 and N=12), plus two layer shapes
    import torch

    from dflash_mlx_amd.verify_linear import VerifyQuantizedLinear, is_verify_eligible

    monkeypatch.setenv("DFLASH_VERIFY_QMM", "1")
    ql = _mk_ql(dev, K, N, seed=K + N)
    assert is_verify_eligible(ql)
    verify = VerifyQuantizedLinear.from_quantized(ql)
    x = _x(dev, M, K, seed=M)
    y_verify = verify(x)
    assert torch.equal(y_verify, _direct(ql, x))
    _oracle_check(ql, x, y_verify)


@pytest.mark.parametrize("variant", ["combo_ktmpl", "super_tree_fp16_ktmpl"])
def test_wrapper_honors_forced_variant(dev, monkeypatch, variant):
    # test_verify_linear_parity.py:74-114: a forced variant, wrapper == direct
    # bitwise and both within the reference's bounds of the stock result
    import torch

    from dflash_mlx_amd.verify_linear import VerifyQuantizedLinear

    monkeypatch.setenv("DFLASH_VERIFY_QMM", "1")
    monkeypatch.setenv("DFLASH_VERIFY_VARIANT", variant)
    ql = _mk_ql(dev, 512, 1024, seed=3)
    verify = VerifyQuantizedLinear.from_quantized(ql)
    x = _x(dev, 16, 512, seed=4)
    y_direct, y_verify = _direct(ql, x), verify(x)
    assert torch.equal(y_direct, y_verify)
    y_stock = ql(x).float()
    ref_max = float(y_stock.abs().max())
    for y in (y_direct.float(), y_verify.float()):
        d = float((y - y_stock).abs().max())
        assert d <= 6e-2 and d / (ref_max + 1e-3) <= 5e-2


@pytest.mark.parametrize("K,N", [(5120, 8), (512, 1024)])
def test_disabled_path_is_exactly_stock(dev, K, N):
    # test_verify_qmm_parity.py:102-106: DFLASH_VERIFY_QMM unset -> the stock result
    import torch

    from dflash_mlx_amd.verify_qmm import is_enabled, quantized_matmul

    assert not is_enabled()
    ql = _mk_ql(dev, K, N, seed=5)
    x = _x(dev, 16, K, seed=6)
    y_stock = quantized_matmul(x, ql.weight, ql.scales, ql.biases, group_size=64, bits=4)
    assert torch.equal(_direct(ql, x), y_stock)


@pytest.mark.parametrize("M", [16, 4, 8])
def test_bias_add(dev, monkeypatch, M):
    # verify_linear.py:250,261: y = verify_matmul(x) + bias on every route
    import torch

    from dflash_mlx_amd.verify_linear import VerifyQuantizedLinear

    monkeypatch.setenv("DFLASH_VERIFY_QMM", "1")
    ql = _mk_ql(dev, 1024, 512, bias=True, seed=7)
    assert ql.has_bias()
    verify = VerifyQuantizedLinear.from_quantized(ql)
    x = _x(dev, M, 1024, seed=8)
    y = verify(x)
    assert torch.equal(y, _direct(ql, x) + ql.bias)
    assert torch.equal(y, ql(x))
    _oracle_check(ql, x, y)


@pytest.mark.parametrize("K,N", [(4096, 4096), (4096, 1024), (4096, 12288), (12288, 4096)])
def test_8bit_module_on_layer_shapes(dev, monkeypatch, K, N):
    """8-bit modules at M=16 with the verify kernels on (mma2big routes): the
    automatic plan, wrapper == direct bitwise, and within 1e-2 of the oracle."""
    import torch

    from dflash_mlx_amd.verify_linear import VerifyQuantizedLinear
    from dflash_mlx_amd.verify_qmm import verify_route

    monkeypatch.setenv("DFLASH_VERIFY_QMM", "1")
    assert verify_route(16, K, N, 8)[1] is None
    ql = _mk_ql(dev, K, N, bits=8, seed=K + N, std=0.02)
    verify = VerifyQuantizedLinear.from_quantized(ql)
    x = _x(dev, 16, K, seed=9, scale=1.0)
    y = verify(x)
    assert torch.equal(y, _direct(ql, x))
    _oracle_check(ql, x, y)


def _layer(dev, K, Nq, Nkv, Ni, seed, bias=False):
    import torch

    class Attn(torch.nn.Module):
        def __init__(self):
            super().__init__()
            self.q_proj = _mk_ql(dev, K, Nq, seed=seed, std=0.02, bias=bias)
            self.k_proj = _mk_ql(dev, K, Nkv, seed=seed + 1, std=0.02, bias=bias)
            self.v_proj = _mk_ql(dev, K, Nkv, seed=seed + 2, std=0.02, bias=bias)

    class MLP(torch.nn.Module):
        def __init__(self):
            super().__init__()
            self.gate_proj = _mk_ql(dev, K, Ni, seed=seed + 3, std=0.02)
            self.up_proj = _mk_ql(dev, K, Ni, seed=seed + 4, std=0.02)

    class Layer(torch.nn.Module):
        def __init__(self):
            super().__init__()
            self.self_attn = Attn()
            self.mlp = MLP()

    return Layer()


@pytest.mark.parametrize("M", [16, 4])
@pytest.mark.parametrize("bias", [False, True])
def test_fused_siblings(dev, monkeypatch, M, bias):
    """install_verify_linears (fuse_siblings, the default): q/k/v and gate/up each run
    as one shared-activation launch in the model's own call order; every
    member's output equals quantized_matmul_multi's for it (+ bias) bit for
    bit, whatever order the members are called in, and is within 1e-2 of the
    unfused module."""
    import torch

    from dflash_mlx_amd.verify_linear import install_verify_linears
    from dflash_mlx_amd.verify_qmm import quantized_matmul_multi

    monkeypatch.setenv("DFLASH_VERIFY_QMM", "1")
    K = 2048
    fused = _layer(dev, K, 2048, 512, 4096, seed=11, bias=bias)
    plain = _layer(dev, K, 2048, 512, 4096, seed=11, bias=bias)
    assert install_verify_linears(fused) == 5  # grouped by default
    assert install_verify_linears(plain, fuse_siblings=False) == 5
    x = _x(dev, M, K, seed=12, scale=1.0)
    for parent, names in ((fused.self_attn, ("q_proj", "k_proj", "v_proj")),
                          (fused.mlp, ("gate_proj", "up_proj"))):
        mods = [getattr(parent, n) for n in names]
        direct = quantized_matmul_multi(x, [(m.weight, m.scales, m.biases) for m in mods],
                                        group_size=64, bits=4)
        want = [d + m.bias if m.has_bias() else d for d, m in zip(direct, mods)]
        for order in (range(len(mods)), reversed(range(len(mods)))):
            got = {i: mods[i](x) for i in order}
            for i in range(len(mods)):
                assert torch.equal(got[i], want[i])
        ref_parent = plain.self_attn if parent is fused.self_attn else plain.mlp
        for n, w in zip(names, want):
            ref = getattr(ref_parent, n)(x).float()
            rel = float((w.float() - ref).abs().max() / (ref.abs().max() + 1e-3))
            assert rel <= REL_TOL
    # a member called with another input recomputes its group for that input
    x2 = _x(dev, M, K, seed=13, scale=1.0)
    q1 = fused.self_attn.q_proj(x)
    k2 = fused.self_attn.k_proj(x2)
    direct2 = quantized_matmul_multi(
        x2, [(m.weight, m.scales, m.biases) for m in
             (fused.self_attn.q_proj, fused.self_attn.k_proj, fused.self_attn.v_proj)],
        group_size=64, bits=4)
    kb = fused.self_attn.k_proj.bias
    assert torch.equal(k2, direct2[1] + kb if kb is not None else direct2[1])
    assert q1.shape == (M, 2048)


def test_fused_siblings_graph_replay(dev, monkeypatch):
    """The grouped calls captured in a HIP graph replay to the eager result
    (replays interleaved with eager work and synchronisations)."""
    import torch

    from dflash_mlx_amd.verify_linear import install_verify_linears, prewarm_verify_kernels

    monkeypatch.setenv("DFLASH_VERIFY_QMM", "1")
    K = 2048
    model = _layer(dev, K, 2048, 512, 4096, seed=21)
    install_verify_linears(model, fuse_siblings=True)
    prewarm_verify_kernels(model)
    x = _x(dev, 16, K, seed=22, scale=1.0)

    def fwd():
        a = model.self_attn
        return (a.q_proj(x), a.k_proj(x), a.v_proj(x), model.mlp.gate_proj(x),
                model.mlp.up_proj(x))

    eager = [t.clone() for t in fwd()]
    stream = torch.cuda.Stream()
    with torch.cuda.stream(stream):
        fwd()
    stream.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        outs = fwd()
    for _ in range(3):
        graph.replay()
        torch.cuda.synchronize()
        for o, e in zip(outs, eager):
            assert torch.equal(o, e)
        fwd()  # eager work between replays
        torch.cuda.synchronize()


def test_capture_without_prewarm_uses_the_pair_table(dev, monkeypatch):
    """A module captured into a graph without prewarm_verify_kernels already
    has its pair table (built with the route at install): the capture warns
    nothing and replays bit-identical to the eager launch.  A module whose
    table is missing at capture (constructed under capture: forced here by
    dropping it) warns once, and its table-free launch replays bit-identical
    to the eager launch with the table (the same plan with or without it)."""
    import warnings

    import torch

    from dflash_mlx_amd import _runtime
    from dflash_mlx_amd import verify_linear as vl

    monkeypatch.setenv("DFLASH_VERIFY_QMM", "1")
    monkeypatch.setattr(vl, "_CAPTURE_WARNED", False)
    K = N = 4096
    ql = _mk_ql(dev, K, N, seed=41, std=0.02)
    verify = vl.VerifyQuantizedLinear.from_quantized(ql)
    state = verify._verify_state
    assert state.pairs is not None  # built at install
    x = _x(dev, 16, K, seed=42, scale=1.0)
    stream = torch.cuda.Stream()
    with torch.cuda.stream(stream):
        _runtime.WORKSPACES.reserve(x.device, 16 << 20)
    stream.synchronize()

    def capture():
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            out = verify(x)
        return graph, out

    with warnings.catch_warnings():
        warnings.simplefilter("error", RuntimeWarning)
        g1, out1 = capture()
    eager = verify(x)
    torch.cuda.synchronize()
    state.pairs = None  # as if the module had been built under capture
    state.recs.clear()
    with pytest.warns(RuntimeWarning, match="before its pair table"):
        g2, out2 = capture()
    assert state.pairs is None
    assert torch.equal(verify(x), eager)  # rebuilds the table
    torch.cuda.synchronize()
    assert state.pairs is not None
    for _ in range(3):
        for g, out in ((g1, out1), (g2, out2)):
            g.replay()
            torch.cuda.synchronize()
            assert torch.equal(out, eager)
            verify(x)
            torch.cuda.synchronize()
    assert torch.equal(eager, _direct(ql, x))
    _oracle_check(ql, x, eager)


def _multi_of(mods, x, active=None):
    from dflash_mlx_amd.verify_qmm import quantized_matmul_multi

    idx = list(range(len(mods))) if active is None else list(active)
    ys = quantized_matmul_multi(x, [(mods[i].weight, mods[i].scales, mods[i].biases)
                                    for i in idx], group_size=64, bits=4)
    return dict(zip(idx, ys))


def test_siblings_hold_their_input(dev, monkeypatch):
    """A group keeps the input of a launch whose outputs are not all taken,
    so a freed input's storage cannot pass to a new tensor that the group
    would take for it (the new tensor gets its own product); an in-place
    update of the input (a version bump) launches again."""
    import torch

    from dflash_mlx_amd.verify_linear import install_verify_linears, prewarm_verify_kernels

    monkeypatch.setenv("DFLASH_VERIFY_QMM", "1")
    K = 2048
    model = _layer(dev, K, 2048, 512, 4096, seed=31)
    install_verify_linears(model)
    prewarm_verify_kernels(model)
    a = model.self_attn
    mods = [a.q_proj, a.k_proj, a.v_proj]
    x1 = _x(dev, 16, K, seed=32, scale=1.0)
    a.q_proj(x1)
    p1 = x1.data_ptr()
    del x1  # k and v have not taken theirs: the group still holds x1
    x2 = torch.empty((16, K), dtype=torch.bfloat16, device=dev)
    assert x2.data_ptr() != p1
    x2.copy_(_x(dev, 16, K, seed=33, scale=1.0))
    got = {1: a.k_proj(x2), 2: a.v_proj(x2), 0: a.q_proj(x2)}
    want = _multi_of(mods, x2)
    for i in range(3):
        assert torch.equal(got[i], want[i])
    x3 = _x(dev, 16, K, seed=34, scale=1.0)
    a.q_proj(x3)
    x3.mul_(2.0)
    k3 = a.k_proj(x3)
    assert torch.equal(k3, _multi_of(mods, x3)[1])


def test_siblings_after_prewarm_in_any_order(dev, monkeypatch):
    """After prewarm (which warms the group and leaves nothing pending),
    up_proj called before gate_proj on a fresh (1, 16, K) input returns the
    shared launch's products, within 1e-2 of the ungrouped modules."""
    import torch

    from dflash_mlx_amd.verify_linear import install_verify_linears, prewarm_verify_kernels

    monkeypatch.setenv("DFLASH_VERIFY_QMM", "1")
    K = 2048
    grouped = _layer(dev, K, 2048, 512, 4096, seed=41)
    plain = _layer(dev, K, 2048, 512, 4096, seed=41)
    install_verify_linears(grouped)
    install_verify_linears(plain, fuse_siblings=False)
    prewarm_verify_kernels(grouped)
    x = _x(dev, 16, K, seed=42, scale=1.0).reshape(1, 16, K)
    up = grouped.mlp.up_proj(x)
    gate = grouped.mlp.gate_proj(x)
    want = _multi_of([grouped.mlp.gate_proj, grouped.mlp.up_proj], x)
    assert torch.equal(gate, want[0]) and torch.equal(up, want[1])
    for got, ref in ((gate, plain.mlp.gate_proj(x)), (up, plain.mlp.up_proj(x))):
        rel = float((got.float() - ref.float()).abs().max() / (ref.float().abs().max() + 1e-3))
        assert rel <= REL_TOL


@pytest.mark.parametrize("called", [(0,), (0, 1)])
def test_siblings_drop_members_never_called(dev, monkeypatch, called):
    """A layer that calls only q_proj (a shared-KV attention layer) or q and k
    (keys used as values): the uncalled members leave the shared launch after
    two launches whose outputs they did not take; every output is the shared
    launch's product over the members active at that call (or, with one
    member left, the member's own verify_matmul), bit for bit."""
    import torch

    from dflash_mlx_amd.verify_linear import install_verify_linears, prewarm_verify_kernels
    from dflash_mlx_amd.verify_qmm import verify_matmul

    monkeypatch.setenv("DFLASH_VERIFY_QMM", "1")
    K = 2048
    model = _layer(dev, K, 2048, 512, 4096, seed=51)
    install_verify_linears(model)
    prewarm_verify_kernels(model)
    a = model.self_attn
    mods = [a.q_proj, a.k_proj, a.v_proj]
    grp = a.q_proj._verify_state.group
    assert grp.active == (0, 1, 2)
    for cycle in range(4):
        x = _x(dev, 16, K, seed=60 + cycle, scale=1.0)
        got = {i: mods[i](x) for i in called}
        act = grp.active
        if len(act) >= 2:
            want = _multi_of(mods, x, act)
        else:
            want = {i: verify_matmul(x, mods[i].weight, mods[i].scales, mods[i].biases,
                                     group_size=64, bits=4) for i in called}
        for i in called:
            assert torch.equal(got[i], want[i]), (cycle, i, act)
    assert grp.active == (called if len(called) >= 2 else ())
    # a dropped member still answers when called, with its own launch
    x = _x(dev, 16, K, seed=70, scale=1.0)
    v = a.v_proj(x)
    assert torch.equal(v, verify_matmul(x, a.v_proj.weight, a.v_proj.scales, a.v_proj.biases,
                                        group_size=64, bits=4))


def test_siblings_share_one_pair_table(dev, monkeypatch):
    """Grouped members keep one combined (scale, bias) pair table: each
    member's table is a column slice of it (no per-member copy), and a
    member's own launch over its slice equals its launch over a table of its
    own."""
    import torch

    from dflash_mlx_amd import _runtime
    from dflash_mlx_amd.verify_linear import install_verify_linears
    from dflash_mlx_amd.verify_qmm import qmm_launch

    monkeypatch.setenv("DFLASH_VERIFY_QMM", "1")
    K = 2048
    model = _layer(dev, K, 2048, 512, 4096, seed=81)
    install_verify_linears(model)
    for parent, names in ((model.self_attn, ("q_proj", "k_proj", "v_proj")),
                          (model.mlp, ("gate_proj", "up_proj"))):
        states = [getattr(parent, n)._verify_state for n in names]
        fused = states[0].group.fused
        assert fused is not None and fused.shape[1] == sum(q.N for q in states)
        for q in states:
            assert q.pairs.untyped_storage().data_ptr() == fused.untyped_storage().data_ptr()
            assert q.stride == fused.shape[1]
            x = _x(dev, 4, K, seed=q.N, scale=1.0)
            own = qmm_launch(x, q.w, q.s, q.b, q.N, 64, 4,
                             pairs=_runtime.build_sb_pairs(q.s, q.b))
            st = torch.cuda.current_stream(dev).cuda_stream
            assert torch.equal(q.launch(x, 4, st), own)
