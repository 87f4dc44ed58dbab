"""Quantized caches whose every tensor is larger than 4 GiB, read at blocks above the 4 GiB
mark of each. Needs a GPU (about 41 GB of device memory for INT8, 23 GB for INT4).

The reference's layout puts no bound on num_blocks (src/bpt/reference.py:3-9), and a
288 GB MI355X holds quantized pools of tens of GB. A pool of 1.1 M blocks of 8 kv heads
makes the code tensors 18 GB (INT8) or 9 GB (INT4) and the K (scale, zero) tensor 4.5 GB.
A small cache is quantized by the library, its blocks are copied to the top of the big
pool, and the big pool is decoded through a block table naming those blocks: the result
must equal, bit for bit, the decode of the small cache (same codes and pairs, only their
addresses differ), and match the oracle over the dequantized small cache within the
north-star tolerance.
"""
import numpy as np
import pytest
import torch

from kvq_decode_amd import paged_decode_attention
from kvq_decode_amd.quant import allocate_quantized_cache, quantize_paged_cache
from oracle import kivi
from oracle.attention import build_paged_cache, paged_decode_attention_ref

pytestmark = pytest.mark.gpu

ATOL, RTOL = 2e-3, 1e-2
NB_BIG, HQ, HKV, D, BS = 1_100_000, 32, 8, 128, 16


@pytest.mark.parametrize("fmt", ["int8", "int4"])
def test_pool_above_4gib(fmt, cuda):
    rng = np.random.default_rng(5)
    lens = [300, 1000]
    B, S = len(lens), max(lens)
    q = rng.standard_normal((B, HQ, D)).astype(np.float16)
    k = rng.standard_normal((B, S, HKV, D)).astype(np.float16)
    v = rng.standard_normal((B, S, HKV, D)).astype(np.float16)
    sl = np.array(lens, np.int32)
    kc, vc, bt = build_paged_cache(k, v, sl, BS, rng)
    g = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(cuda)  # noqa: E731
    q_g, bt_g, sl_g = g(q), g(bt), g(sl)
    small = quantize_paged_cache(g(kc), g(vc), bt_g, sl_g, fmt)
    nb_small = kc.shape[0]

    big = allocate_quantized_cache(NB_BIG, BS, HKV, D, fmt, cuda)
    k_store = big.k_codes.permute(0, 2, 1, 3)  # head-major storage [nb, Hkv, bs, Dc]
    assert k_store.is_contiguous() and k_store.numel() > 1 << 32
    assert big.k_sz.numel() * 2 > 1 << 32
    top = torch.arange(NB_BIG - nb_small, NB_BIG, device=cuda)  # the pool's last blocks
    k_store[top] = small.k_codes.permute(0, 2, 1, 3)
    big.v_codes.permute(0, 2, 1, 3)[top] = small.v_codes.permute(0, 2, 1, 3)
    big.k_sz[top] = small.k_sz
    big.v_sz[top] = small.v_sz
    bt_big = (bt_g + (NB_BIG - nb_small)).to(torch.int32)
    torch.cuda.synchronize()

    for splits in (None, 1, 4):
        want = paged_decode_attention(q_g, small.k_codes, small.v_codes, bt_g, sl_g,
                                      num_splits=splits, **small.decode_kwargs())
        got = paged_decode_attention(q_g, big.k_codes, big.v_codes, bt_big, sl_g,
                                     num_splits=splits, **big.decode_kwargs())
        torch.cuda.synchronize()
        print(f"\n[{fmt} pool of {NB_BIG} blocks, num_splits={splits}]", flush=True)
        assert torch.equal(got, want), f"num_splits={splits}: big pool differs"

    host = {n: getattr(small, n).cpu().numpy() for n in
            ("k_codes", "v_codes", "k_scale", "k_zero", "v_scale", "v_zero")}
    kd, vd = kivi.dequantize_paged_cache(host, bt, sl, fmt)
    ref = paged_decode_attention_ref(q.astype(np.float32), kd, vd, bt, sl, out_dtype=np.float32)
    diff = np.abs(got.float().cpu().numpy() - ref)
    assert diff.max() < ATOL and np.all(diff <= ATOL + RTOL * np.abs(ref)), diff.max()
    del big, k_store
    torch.cuda.empty_cache()
