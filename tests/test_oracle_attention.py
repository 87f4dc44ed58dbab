"""Pins the numpy oracle (oracle/attention.py) against checks that do not retype it:
torch's SDPA on contiguous K/V (the reference's own oracle test, tests/test_reference.py:
13-58), a token-by-token float64 brute force that reads the paged cache through the block
table, closed forms, and invariances. CPU only."""
import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle.attention import (build_paged_cache, merge_ref, normalize_splits,
                              paged_decode_attention_ref, split_decode_ref)

SHAPES = [(32, 8, 128), (4, 4, 64), (8, 1, 64)]  # Llama-3-8B GQA, MHA, MQA (test_reference.py:9)


def make_inputs(B, lens, Hq, Hkv, D, dtype, seed=0):
    rng = np.random.default_rng(seed)
    S = max(lens)
    q = rng.standard_normal((B, Hq, D)).astype(dtype)
    k = rng.standard_normal((B, S, Hkv, D)).astype(dtype)
    v = rng.standard_normal((B, S, Hkv, D)).astype(dtype)
    return q, k, v, np.array(lens, np.int32), rng


def sdpa(q, k, v, lens, dtype):
    """Non-paged SDPA per sequence over the first len tokens, K/V expanded to Hq heads
    with repeat_interleave (test_reference.py:13-24)."""
    B, Hq, D = q.shape
    group = Hq // k.shape[2]
    outs = []
    for b in range(B):
        n = int(lens[b])
        kb = torch.from_numpy(k[b, :n]).to(dtype).repeat_interleave(group, dim=1).permute(1, 0, 2)
        vb = torch.from_numpy(v[b, :n]).to(dtype).repeat_interleave(group, dim=1).permute(1, 0, 2)
        qb = torch.from_numpy(q[b]).to(dtype)[:, None, :]
        outs.append(F.scaled_dot_product_attention(qb, kb, vb)[:, 0])
    return torch.stack(outs).float().numpy()


@pytest.mark.parametrize("dtype,atol", [(np.float32, 1e-5), (np.float16, 2e-3)])
@pytest.mark.parametrize("block_size", [16, 32])
@pytest.mark.parametrize("lens", [[1], [37], [100, 33, 1, 64]])
@pytest.mark.parametrize("Hq,Hkv,D", SHAPES)
def test_matches_sdpa(Hq, Hkv, D, lens, block_size, dtype, atol):
    q, k, v, sl, rng = make_inputs(len(lens), lens, Hq, Hkv, D, dtype)
    kc, vc, bt = build_paged_cache(k, v, sl, block_size, rng)
    out = paged_decode_attention_ref(q, kc, vc, bt, sl)
    tdt = torch.float32 if dtype == np.float32 else torch.float16
    try:
        ref = sdpa(q, k, v, sl, tdt)
    except RuntimeError:
        pytest.skip("CPU SDPA lacks fp16 support in this torch build")
    assert out.dtype == dtype
    assert np.abs(out.astype(np.float32) - ref).max() < atol


def brute_force(q, kc, vc, bt, sl, scale):
    """float64, one token at a time through block_table[b][t // bs], slot t % bs."""
    B, Hq, D = q.shape
    _, bs, Hkv, _ = kc.shape
    group = Hq // Hkv
    out = np.zeros((B, Hq, D))
    for b in range(B):
        n = int(sl[b])
        for h in range(Hq):
            kh = h // group
            sc = []
            for t in range(n):
                blk, slot = int(bt[b, t // bs]), t % bs
                sc.append(sum(float(q[b, h, d]) * float(kc[blk, slot, kh, d]) for d in range(D)) * scale)
            mx = max(sc)
            w = [math.exp(x - mx) for x in sc]
            z = sum(w)
            for t in range(n):
                blk, slot = int(bt[b, t // bs]), t % bs
                for d in range(D):
                    out[b, h, d] += w[t] / z * float(vc[blk, slot, kh, d])
    return out


@pytest.mark.parametrize("Hq,Hkv,D,lens,bs", [(8, 2, 8, [5, 19], 16), (6, 3, 4, [33], 16),
                                               (4, 1, 8, [1, 40, 16], 32)])
def test_float64_brute_force(Hq, Hkv, D, lens, bs):
    q, k, v, sl, rng = make_inputs(len(lens), lens, Hq, Hkv, D, np.float64, seed=3)
    kc, vc, bt = build_paged_cache(k, v, sl, bs, rng)
    got = paged_decode_attention_ref(q, kc, vc, bt, sl, scale=0.37, acc_dtype=np.float64)
    want = brute_force(q, kc, vc, bt, sl, 0.37)
    np.testing.assert_allclose(got, want, rtol=0, atol=1e-12)


def test_len1_returns_that_tokens_v_for_every_group_member():
    """softmax over one token is 1: out[b, h] = v[b, 0, h // group] exactly."""
    Hq, Hkv, D = 32, 8, 128
    q, k, v, sl, rng = make_inputs(3, [1, 1, 1], Hq, Hkv, D, np.float16)
    kc, vc, bt = build_paged_cache(k, v, sl, 16, rng)
    out = paged_decode_attention_ref(q, kc, vc, bt, sl)
    for h in range(Hq):
        np.testing.assert_array_equal(out[:, h], v[:, 0, h // (Hq // Hkv)])


def test_zero_query_is_mean_of_values():
    q, k, v, sl, rng = make_inputs(2, [50, 7], 8, 2, 16, np.float32)
    q[:] = 0
    kc, vc, bt = build_paged_cache(k, v, sl, 16, rng)
    out = paged_decode_attention_ref(q, kc, vc, bt, sl)
    for b, n in enumerate([50, 7]):
        mean = v[b, :n].mean(axis=0)  # [Hkv, D]
        np.testing.assert_allclose(out[b], np.repeat(mean, 4, axis=0), atol=1e-6)


def test_dominant_key_selects_its_value():
    q, k, v, sl, rng = make_inputs(1, [64], 4, 1, 32, np.float32)
    k[0, 41, 0] = q[0, 2] * 50.0  # head 2's score at token 41 dwarfs the rest
    kc, vc, bt = build_paged_cache(k, v, sl, 16, rng)
    out = paged_decode_attention_ref(q, kc, vc, bt, sl)
    np.testing.assert_allclose(out[0, 2], v[0, 41, 0], atol=1e-5)


def test_garbage_in_unused_slots_is_ignored():
    """test_reference.py:61-69: different permutations and garbage, same result."""
    q, k, v, sl, _ = make_inputs(2, [37, 5], 8, 2, 32, np.float32)
    a = build_paged_cache(k, v, sl, 16, np.random.default_rng(1))
    b = build_paged_cache(k, v, sl, 16, np.random.default_rng(2))
    assert not np.array_equal(a[2], b[2])
    out_a = paged_decode_attention_ref(q, *a, sl)
    out_b = paged_decode_attention_ref(q, *b, sl)
    np.testing.assert_allclose(out_a, out_b, atol=1e-6)


def test_cache_builder_round_trip_and_garbage():
    q, k, v, sl, rng = make_inputs(3, [20, 1, 33], 4, 2, 8, np.float32)
    kc, vc, bt = build_paged_cache(k, v, sl, 16, rng)
    assert bt.dtype == np.int32 and sorted(bt.ravel().tolist()) == list(range(bt.size))
    for b, n in enumerate([20, 1, 33]):
        for t in range(n):
            np.testing.assert_array_equal(kc[bt[b, t // 16], t % 16], k[b, t])
            np.testing.assert_array_equal(vc[bt[b, t // 16], t % 16], v[b, t])
        # the tail slots of the last page hold large garbage, not the (zero-free) data
        last = bt[b, (n - 1) // 16]
        if n % 16:
            assert np.abs(kc[last, n % 16:]).max() > 10


@pytest.mark.parametrize("num_splits", [1, 2, 3, 7, 16])
def test_split_then_merge_equals_single_pass(num_splits):
    lens = [100, 33, 1, 64]
    q, k, v, sl, rng = make_inputs(4, lens, 32, 8, 128, np.float32)
    kc, vc, bt = build_paged_cache(k, v, sl, 16, rng)
    S, pps = normalize_splits(num_splits, bt.shape[1])
    o_part, lse = split_decode_ref(q, kc, vc, bt, sl, 1 / math.sqrt(128), S, pps)
    got = merge_ref(o_part, lse, out_dtype=np.float32)
    want = paged_decode_attention_ref(q, kc, vc, bt, sl)
    np.testing.assert_allclose(got, want, atol=2e-6)


def test_empty_splits_and_lse_closed_form():
    lens = [5, 40]
    q, k, v, sl, rng = make_inputs(2, lens, 4, 1, 16, np.float64)
    kc, vc, bt = build_paged_cache(k, v, sl, 16, rng)
    S, pps = normalize_splits(3, bt.shape[1])  # 3 pages -> 3 splits of 1 page
    assert (S, pps) == (3, 1)
    o_part, lse = split_decode_ref(q, kc, vc, bt, sl, 0.25, S, pps, acc_dtype=np.float64)
    # sequence 0 has one page: splits 1 and 2 are empty -> o = 0, lse = -inf
    assert np.all(np.isneginf(lse[0, :, 1:])) and np.all(o_part[0, :, 1:] == 0)
    # lse of sequence 1, split 1 (tokens 16..31) = log sum exp(q . k * scale)
    for h in range(4):
        s = np.array([q[1, h] @ k[1, t, 0] * 0.25 for t in range(16, 32)])
        assert lse[1, h, 1] == pytest.approx(np.log(np.exp(s).sum()), rel=1e-6)


@pytest.mark.parametrize("n,pages,expect", [(7, 3, (3, 1)), (32, 2048, (32, 64)), (5, 8, (4, 2)),
                                            (1, 10, (1, 10)), (100, 3, (3, 1)), (0, 4, (1, 4)),
                                            (3, 8, (3, 3))])
def test_normalize_splits(n, pages, expect):
    """triton_fp16.py:211-217; (5, 8) shows the 'drop always-empty tails' step."""
    assert normalize_splits(n, pages) == expect
