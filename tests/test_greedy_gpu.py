"""GPU greedy / accept / fused lm_head vs the oracle.  Token ids, accept
lengths and bonus tokens must be bit-exact given identical logits; the fused
kernel's logits (returned on request) must be within rel 1e-2 of the exact
lm_head product, and its tokens must equal the oracle's argmax of those very
logits."""

from __future__ import annotations

import json
import os

import numpy as np
import pytest

import oracle
from tests.conftest import from_dev, make_qmm_case, to_dev

pytestmark = pytest.mark.gpu

GOLD = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "reference_cases.json")))


def _logits(M, V, dtype, seed, ties=True, nans=False):
    rng = np.random.default_rng(seed)
    v = rng.standard_normal((M, V)).astype(np.float32) * 3
    if ties and V > 8:
        v = np.round(v * 4) / 4  # coarse grid: many exact ties
        top = rng.integers(0, V, size=(M, 2))
        v[np.arange(M), top[:, 0]] = 50.0
        v[np.arange(M), top[:, 1]] = 50.0
    if nans:
        v[0, :: max(1, V // 7)] = np.nan
    if dtype == "f32":
        return v
    return oracle.round_to_dtype(v, dtype)


@pytest.mark.parametrize("dtype", ["bf16", "f16", "f32"])
@pytest.mark.parametrize("M,V", [(1, 1), (16, 17), (16, 4096), (15, 4097), (32, 151936), (40, 1000)])
def test_greedy_tokens_exact(dev, dtype, M, V):
    import torch

    from dflash_mlx_amd import sampling

    lg = _logits(M, V, dtype, seed=M * 1000 + V, nans=(M > 1))
    t = torch.from_numpy(lg).to(dev) if dtype == "f32" else to_dev(lg, dtype, dev)
    got = sampling.greedy_tokens_with_mask(t).cpu().numpy()
    want = oracle.greedy_tokens_with_mask(lg, None, dtype=dtype)
    assert np.array_equal(got, want)


def test_greedy_mask(dev):
    import torch

    from dflash_mlx_amd import sampling

    M, V = 16, 5000
    lg = _logits(M, V, "bf16", seed=3)
    want_unmasked = oracle.greedy_tokens_with_mask(lg, dtype="bf16")
    ids = list(want_unmasked[:5]) + [V + 3, -1]
    mask = sampling.build_suppress_token_mask(V, ids, device=dev)
    omask = oracle.build_suppress_token_mask(V, ids)
    assert np.array_equal(mask.cpu().numpy(), omask)
    got = sampling.greedy_tokens_with_mask(to_dev(lg, "bf16", dev), mask).cpu().numpy()
    assert np.array_equal(got, oracle.greedy_tokens_with_mask(lg, omask, dtype="bf16"))
    assert sampling.build_suppress_token_mask(V, [V, -3]) is None
    # every id suppressed: all rows equal bf16(-1e9) -> index 0
    allm = torch.ones(V, dtype=torch.bool, device=dev)
    assert np.all(sampling.greedy_tokens_with_mask(to_dev(lg, "bf16", dev), allm).cpu().numpy() == 0)


@pytest.mark.parametrize("drafted,posterior,expected", GOLD["acceptance_cases"])
def test_match_acceptance_known_answers(dev, drafted, posterior, expected):
    import torch

    from dflash_mlx_amd.acceptance import match_acceptance_length

    d = torch.tensor(drafted, dtype=torch.int32, device=dev)
    p = torch.tensor(posterior, dtype=torch.int32, device=dev)
    assert int(match_acceptance_length(d, p).item()) == expected


def test_greedy_accept_cycle_semantics(dev):
    import torch

    from dflash_mlx_amd.lm_head import greedy_accept

    rng = np.random.default_rng(9)
    M, V = 16, 3000
    for trial in range(12):
        lg = _logits(M, V, "bf16", seed=100 + trial)
        post = oracle.greedy_tokens_with_mask(lg, dtype="bf16")
        ids = np.concatenate([[rng.integers(V)], post[:-1]])
        cut = int(rng.integers(1, M + 1))
        if cut < M:
            ids[cut] = (ids[cut] + 1) % V
        res = greedy_accept(to_dev(lg, "bf16", dev),
                            verify_ids=torch.tensor(ids, dtype=torch.int32, device=dev))
        a, bonus = oracle.verify_cycle_accept(ids, post)
        assert np.array_equal(res.posterior.cpu().numpy(), post)
        assert int(res.accept_len.item()) == a == cut - 1
        assert int(res.bonus.item()) == bonus


def _lm_case(M, K, V, gs, seed, dtype="bf16"):
    return make_qmm_case(M, K, V, gs, dtype=dtype, seed=seed)


@pytest.mark.parametrize("M,K,V,gs,dtype", [(16, 512, 1000, 64, "bf16"), (16, 2048, 32000, 64, "bf16"),
                                            (4, 1024, 5003, 32, "f16"), (32, 768, 2048, 128, "bf16"),
                                            (1, 256, 129, 64, "bf16"), (16, 1088, 4099, 64, "bf16"),
                                            (32, 1024, 3001, 64, "bf16"), (24, 2048, 777, 128, "f16"),
                                            (16, 5120, 20000, 64, "bf16"), (16, 2048, 777, 64, "bf16"),
                                            (12, 4096, 9000, 128, "f16")])
def test_lmhead_fused_matches_oracle(dev, M, K, V, gs, dtype):
    import torch

    from dflash_mlx_amd.lm_head import lm_head_greedy_accept

    x, w_q, s, b = _lm_case(M, K, V, gs, seed=M + K + V, dtype=dtype)
    exact = oracle.quantized_matmul(x, w_q, s, b, group_size=gs, dtype=dtype)
    post_exact = oracle.greedy_tokens_with_mask(oracle.round_to_dtype(exact, dtype), dtype=dtype)
    rng = np.random.default_rng(V)
    ids = np.concatenate([[rng.integers(V)], post_exact[:-1]]).astype(np.int64)
    flip = rng.random(M) > 0.88
    ids[1:][flip[1:]] = rng.integers(0, V, size=int(flip[1:].sum()))
    res = lm_head_greedy_accept(to_dev(x, dtype, dev), to_dev(w_q, "u32", dev),
                                to_dev(s, dtype, dev), to_dev(b, dtype, dev),
                                verify_ids=torch.tensor(ids, dtype=torch.int32, device=dev),
                                group_size=gs, bits=4, return_logits=True)
    got_logits = from_dev(res.logits, dtype)
    _, rel = oracle.parity_metrics(oracle.to_f32(got_logits, dtype), exact)
    assert rel <= 1e-2
    post_on_got = oracle.greedy_tokens_with_mask(got_logits, dtype=dtype)
    assert np.array_equal(res.posterior.cpu().numpy(), post_on_got)
    a, bonus = oracle.verify_cycle_accept(ids, post_on_got)
    assert int(res.accept_len.item()) == a and int(res.bonus.item()) == bonus
    # Without logits output the tokens are the same (the logits write is optional).
    res2 = lm_head_greedy_accept(to_dev(x, dtype, dev), to_dev(w_q, "u32", dev),
                                 to_dev(s, dtype, dev), to_dev(b, dtype, dev),
                                 verify_ids=torch.tensor(ids, dtype=torch.int32, device=dev),
                                 group_size=gs, bits=4)
    assert np.array_equal(res2.posterior.cpu().numpy(), post_on_got)
    assert int(res2.accept_len.item()) == a and int(res2.bonus.item()) == bonus


@pytest.mark.parametrize("K", [256, 512, 2048])  # general and streaming main loops, 4 K steps
def test_lmhead_exact_ties_pick_lowest_index(dev, K):
    from dflash_mlx_amd.lm_head import lm_head_greedy_accept

    M, V, gs = 16, 700, 64
    x, w_q, s, b = _lm_case(M, K, V, gs, seed=11)
    # positive activations; rows 333 and 91 get identical weights and a large
    # bias, so both hold the row maximum exactly (an exact tie)
    x = x & np.uint16(0x7FFF)
    b = b.copy()
    big = oracle.f32_to_bf16_bits(np.float32(4.0))
    w_q[333] = w_q[91]
    s[333] = s[91]
    b[91] = big
    b[333] = big
    res = lm_head_greedy_accept(to_dev(x, "bf16", dev), to_dev(w_q, "u32", dev),
                                to_dev(s, "bf16", dev), to_dev(b, "bf16", dev),
                                group_size=gs, bits=4, return_logits=True)
    lg = from_dev(res.logits, "bf16")
    assert np.array_equal(lg[:, 91], lg[:, 333])
    post = res.posterior.cpu().numpy()
    want = oracle.greedy_tokens_with_mask(lg, dtype="bf16")
    assert np.array_equal(post, want)
    assert np.all(post == 91)


def test_lmhead_mask_and_softcap(dev):
    import torch

    from dflash_mlx_amd import sampling
    from dflash_mlx_amd.lm_head import lm_head_greedy_accept

    M, K, V, gs = 16, 512, 3000, 64
    x, w_q, s, b = make_qmm_case(M, K, V, gs, seed=21, w_std=0.2)  # logits spread over +-30
    args = (to_dev(x, "bf16", dev), to_dev(w_q, "u32", dev), to_dev(s, "bf16", dev),
            to_dev(b, "bf16", dev))
    raw = lm_head_greedy_accept(*args, group_size=gs, bits=4, return_logits=True)
    raw_l = from_dev(raw.logits, "bf16")
    ids = list(raw.posterior.cpu().numpy()[:6])
    mask = sampling.build_suppress_token_mask(V, ids, device=dev)
    capped = lm_head_greedy_accept(*args, group_size=gs, bits=4, softcap=30.0,
                                   suppress_token_mask=mask, return_logits=True)
    cap_l = from_dev(capped.logits, "bf16")
    want = oracle.logit_softcap(raw_l, 30.0)
    diff = np.abs(oracle.bf16_bits_to_f32(cap_l) - oracle.bf16_bits_to_f32(want))
    ulp = np.abs(oracle.bf16_bits_to_f32(want)) * 2.0 ** -7 + 1e-30
    assert np.all(diff <= ulp)  # tanh may differ from numpy's by one rounding step
    omask = oracle.build_suppress_token_mask(V, ids)
    assert np.array_equal(capped.posterior.cpu().numpy(),
                          oracle.greedy_tokens_with_mask(cap_l, omask, dtype="bf16"))
    assert torch.equal(capped.posterior, sampling.greedy_tokens_with_mask(capped.logits, mask))


@pytest.mark.parametrize("K", [1024, 2048])  # streaming main loop, 2 and 4 K steps
def test_lmhead_repeatable_and_workspace_clean(dev, K):
    from dflash_mlx_amd import sampling
    from dflash_mlx_amd.lm_head import lm_head_greedy_accept

    M, V, gs = 16, 10007, 64
    x, w_q, s, b = _lm_case(M, K, V, gs, seed=5)
    args = (to_dev(x, "bf16", dev), to_dev(w_q, "u32", dev), to_dev(s, "bf16", dev),
            to_dev(b, "bf16", dev))
    first = lm_head_greedy_accept(*args, group_size=gs, bits=4).posterior.cpu().numpy()
    for i in range(3):
        lg = _logits(16, 999, "bf16", seed=i)
        assert np.array_equal(sampling.greedy_tokens_with_mask(to_dev(lg, "bf16", dev)).cpu().numpy(),
                              oracle.greedy_tokens_with_mask(lg, dtype="bf16"))
        again = lm_head_greedy_accept(*args, group_size=gs, bits=4).posterior.cpu().numpy()
        assert np.array_equal(again, first)


@pytest.mark.parametrize("block_len,K,V,gs", [(16, 2048, 32000, 64), (16, 1024, 5003, 32),
                                              (8, 5120, 20000, 64)])
def test_draft_tokens_from_hidden(dev, block_len, K, V, gs):
    """Draft side (dflash_mlx/draft_backend.py:142-149): the target lm_head
    over draft_hidden[:, 1:, :] (block_len - 1 rows, e.g. 15) and the masked
    greedy argmax, fused, no accept.  Tokens equal the greedy argmax of the
    kernel's own logits (which are within the parity metric of the oracle),
    with and without a suppress mask."""
    import torch

    from dflash_mlx_amd.lm_head import draft_tokens_from_hidden, lm_head_greedy_accept
    from dflash_mlx_amd.sampling import build_suppress_token_mask

    M = block_len - 1
    x, w_q, s, b = _lm_case(block_len, K, V, gs, seed=block_len + K + V)
    hd = to_dev(x, "bf16", dev).reshape(1, block_len, K)
    wd, sd, bd = to_dev(w_q, "u32", dev), to_dev(s, "bf16", dev), to_dev(b, "bf16", dev)
    full = lm_head_greedy_accept(hd[0, 1:], wd, sd, bd, group_size=gs, return_logits=True)
    got_logits = from_dev(full.logits, "bf16")
    exact = oracle.quantized_matmul(x[1:], w_q, s, b, group_size=gs, dtype="bf16")
    _, rel = oracle.parity_metrics(oracle.to_f32(got_logits, "bf16"), exact)
    assert rel <= 1e-2
    toks = draft_tokens_from_hidden(hd, wd, sd, bd, group_size=gs)
    assert toks.shape == (M,)
    assert np.array_equal(toks.cpu().numpy(), oracle.greedy_tokens_with_mask(got_logits, dtype="bf16"))
    # suppress the current winners of the first rows: the next best take over
    banned = sorted(set(int(t) for t in toks.cpu().numpy()[:3]))
    mask = build_suppress_token_mask(V, banned, device=dev)
    toks_m = draft_tokens_from_hidden(hd, wd, sd, bd, suppress_token_mask=mask, group_size=gs)
    mask_np = np.zeros(V, bool)
    mask_np[banned] = True
    want = oracle.greedy_tokens_with_mask(got_logits, mask_np, dtype="bf16")
    assert np.array_equal(toks_m.cpu().numpy(), want)
    assert not np.isin(toks_m.cpu().numpy(), banned).any()
