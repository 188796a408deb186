"""Parity at the benchmarked workloads' real sizes (the shapes the bench
times), each run once:

* the fused lm_head + greedy + accept on ``[16,5120] x [151936,5120]`` int4
  gs64 (the reference's path: dflash_mlx/engine/target_qwen_gdn.py:774-778 ->
  engine/sampling.py:48-55 -> engine/acceptance.py:9-16 with the cycle
  semantics of engine/spec_epoch.py:2067-2072,2129), with and without the
  logits written;
* one MoE layer of 16 tokens routed top-8 over 256 experts, hidden 2048,
  expert width 512 (mlx-lm SwitchGLU reached from
  engine/target_qwen_gdn.py:865,874): gather SwiGLU -> gather down ->
  unsorting combine.

Weights are quantised on the GPU by the product quantiser (bit-identical to
the oracle's rule, tests/test_quantize.py); both sides then consume the same
packed tensors.  The dense product is checked against the oracle's C
restatement (fp32 accumulation, oracle/cpu_qmm.c, itself pinned against the
float64 numpy oracle), the rest against the numpy oracle.  Tolerances: the
1e-2 metric for values, bit-exact for token ids, accept length and bonus."""

from __future__ import annotations

import numpy as np
import pytest

import oracle
from oracle import cpu as ocpu
from oracle import moe as omoe
from tests.conftest import from_dev

pytestmark = pytest.mark.gpu

REL_TOL = 1e-2


def _quantize_rows(torch, N, K, gen, dev, block=16384):
    from dflash_mlx_amd.quantize import quantize

    w_q = torch.empty((N, K // 8), dtype=torch.int32, device=dev)
    s = torch.empty((N, K // 64), dtype=torch.bfloat16, device=dev)
    b = torch.empty_like(s)
    for r0 in range(0, N, block):  # fp32 W of the whole head would be 3 GB
        r1 = min(N, r0 + block)
        w = torch.randn((r1 - r0, K), generator=gen, device=dev) * 0.02
        w_q[r0:r1], s[r0:r1], b[r0:r1] = quantize(w, 64, 4, torch.bfloat16)
        del w
    return w_q, s, b


def test_lmhead_greedy_accept_full_vocab(dev):
    import torch

    from dflash_mlx_amd.lm_head import lm_head_greedy_accept

    M, K, V = 16, 5120, 151936
    print(f"case: fused lm_head M={M} K={K} V={V} seed 5", flush=True)
    gen = torch.Generator(device=dev)
    gen.manual_seed(5)
    w_q, s, b = _quantize_rows(torch, V, K, gen, dev)
    h = torch.randn((M, K), generator=gen, device=dev).to(torch.bfloat16)
    torch.cuda.synchronize()
    hx = from_dev(h, "bf16")
    hw = w_q.cpu().numpy().view(np.uint32)
    hs, hb = from_dev(s, "bf16"), from_dev(b, "bf16")
    exact = oracle.bf16_bits_to_f32(ocpu.qmm_bf16(hx, hw, hs, hb, 64, 4))
    argmax_exact = oracle.greedy_tokens_with_mask(oracle.f32_to_bf16_bits(exact), dtype="bf16")
    # verify ids: a staged token, then each draft equals the previous row's
    # argmax with probability 0.88, else a uniform token
    rng = np.random.default_rng(5)
    ids = np.empty(M, dtype=np.int64)
    ids[0] = rng.integers(V)
    for i in range(1, M):
        ids[i] = argmax_exact[i - 1] if rng.random() < 0.88 else rng.integers(V)
    ids_t = torch.tensor(ids, dtype=torch.int32, device=dev)

    res = lm_head_greedy_accept(h, w_q, s, b, verify_ids=ids_t, group_size=64, bits=4,
                                return_logits=True)
    got = from_dev(res.logits, "bf16")
    _, rel = oracle.parity_metrics(oracle.bf16_bits_to_f32(got), exact)
    assert rel <= REL_TOL, rel
    post = oracle.greedy_tokens_with_mask(got, dtype="bf16")
    assert np.array_equal(res.posterior.cpu().numpy(), post)
    a, bonus = oracle.verify_cycle_accept(ids, post)
    assert int(res.accept_len.item()) == a and int(res.bonus.item()) == bonus
    # the fused path without the logits write: same tokens, accept and bonus
    res2 = lm_head_greedy_accept(h, w_q, s, b, verify_ids=ids_t, group_size=64, bits=4)
    assert np.array_equal(res2.posterior.cpu().numpy(), post)
    assert int(res2.accept_len.item()) == a and int(res2.bonus.item()) == bonus
    # the kernel's tokens agree with the exact logits' argmax on most rows
    assert (post == argmax_exact).mean() >= 0.75
    print(f"accept={a} bonus={bonus} rel={rel:.2e}", flush=True)


def test_moe_layer_top8_of_256(dev):
    import torch

    from dflash_mlx_amd.moe import gather_qmm, gather_swiglu, moe_combine
    from dflash_mlx_amd.quantize import quantize

    T, k, E, D, I = 16, 8, 256, 2048, 512
    print(f"case: MoE layer T={T} top-{k} of E={E} D={D} I={I} seed 7", flush=True)
    gen = torch.Generator(device=dev)
    gen.manual_seed(7)

    def experts(N, K):
        w = torch.randn((E * N, K), generator=gen, device=dev) * 0.02
        wq, sc, bi = quantize(w, 64, 4, torch.bfloat16)
        del w
        return wq.reshape(E, N, K // 8), sc.reshape(E, N, K // 64), bi.reshape(E, N, K // 64)

    gate, up, down = experts(I, D), experts(I, D), experts(D, I)
    x = torch.randn((T, D), generator=gen, device=dev).to(torch.bfloat16)
    logits = np.random.default_rng(7).standard_normal((T, E)).astype(np.float32)
    inds, scores = omoe.route_topk(logits, k)
    assert len(np.unique(inds)) > 64  # a realistic spread of distinct experts
    flat = inds.reshape(-1)
    order = np.argsort(flat, kind="stable")
    inv = np.empty_like(order)
    inv[order] = np.arange(order.size)
    rhs = torch.tensor(flat[order], dtype=torch.int32, device=dev)
    lhs = torch.tensor(order // k, dtype=torch.int32, device=dev)
    h_sorted = gather_swiglu(x, gate, up, rhs, lhs_indices=lhs, group_size=64)
    y_sorted = gather_qmm(h_sorted, *down, rhs, group_size=64)
    out = moe_combine(y_sorted, torch.tensor(scores, device=dev),
                      y_rows=torch.tensor(inv, dtype=torch.int32, device=dev))
    torch.cuda.synchronize()

    def host(tr):
        return (tr[0].cpu().numpy().view(np.uint32), from_dev(tr[1], "bf16"),
                from_dev(tr[2], "bf16"))

    hx = from_dev(x, "bf16")
    h_want, y_want = omoe.switch_glu(hx, inds, host(gate), host(up), host(down),
                                     group_size=64, dtype="bf16")
    h_got = from_dev(h_sorted, "bf16")[inv]
    y_got = from_dev(y_sorted, "bf16")[inv]
    for got, want in ((h_got, h_want), (y_got, y_want)):
        _, rel = oracle.parity_metrics(oracle.bf16_bits_to_f32(got), oracle.bf16_bits_to_f32(want))
        assert rel <= REL_TOL, rel
    out_got = oracle.bf16_bits_to_f32(from_dev(out, "bf16"))
    _, rel = oracle.parity_metrics(out_got, omoe.moe_combine(y_want, scores, dtype="bf16"))
    assert rel <= REL_TOL, rel
    # the combine itself on the kernel's own y: within one bf16 rounding step
    own = omoe.moe_combine(y_got, scores, dtype="bf16", out_dtype="bf16")
    diff = np.abs(from_dev(out, "bf16").astype(np.int32) - own.astype(np.int32))
    assert diff.max() <= 1
