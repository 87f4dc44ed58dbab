"""The quantized write path's bounds and argument checks. Needs a GPU.

  * quantize-on-append for a sequence whose length has no slot in its table (below 1 or
    past the table's last slot), or whose new token's K group starts in a page outside the
    pool, writes nothing: every byte of both code tensors and both (scale, zero) tensors
    is unchanged, and so is the sequence's fp16 residual (the fp16 counterpart is
    test_write_gpu.py's test_append_kv_out_of_range_writes_nothing). A valid sequence of
    the same call is written as usual.
  * the bulk quantizer writes nothing into blocks no valid table entry names, when the
    table also holds entries outside the pool (-1, num_blocks).
  * quantize_append / quantize_paged_cache reject mismatched batch, kv heads, shapes and
    devices with KvqArgumentError before any launch.
"""
import numpy as np
import pytest
import torch

from kvq_decode_amd import KvqArgumentError
from kvq_decode_amd.quant import (allocate_quantized_cache, init_k_residual, quantize_append,
                                  quantize_paged_cache)

pytestmark = pytest.mark.gpu

FORMATS = ["int8", "fp8_e4m3", "int4"]
BS, HKV, D = 16, 2, 128


def storage(qc):
    """Every byte the cache owns: head-major codes and the interleaved pair tensors."""
    return [qc.k_codes.permute(0, 2, 1, 3).cpu().numpy().copy(),
            qc.v_codes.permute(0, 2, 1, 3).cpu().numpy().copy(),
            qc.k_sz.cpu().numpy().view(np.uint16).copy(),
            qc.v_sz.cpu().numpy().view(np.uint16).copy()]


def filled_cache(nb, fmt, seed):
    """A cache whose every byte holds a known random pattern."""
    qc = allocate_quantized_cache(nb, BS, HKV, D, fmt, "cuda")
    g = torch.Generator(device="cuda").manual_seed(seed)
    for t in (qc.k_codes.permute(0, 2, 1, 3), qc.v_codes.permute(0, 2, 1, 3)):
        t.copy_(torch.randint(0, 256, t.shape, generator=g, device="cuda", dtype=torch.uint8))
    for t in (qc.k_sz, qc.v_sz):
        t.copy_(torch.randn(t.shape, generator=g, device="cuda").half())
    return qc


@pytest.mark.parametrize("fmt", FORMATS)
def test_quantize_append_out_of_range_writes_nothing(fmt):
    nb, mb = 64, 12  # 12 pages per sequence: 192 slots
    qc = filled_cache(nb, fmt, 1)
    # sequences 0-3 own blocks 12b .. 12b + 11; the valid sequence 3 appends normally
    bt = torch.arange(4 * mb, dtype=torch.int32, device="cuda").view(4, mb).contiguous()
    bt[2, 8] = nb  # sequence 2's new token (position 128) opens a group in a page past the pool
    lens = torch.tensor([mb * BS + 1, 0, 129, 50], dtype=torch.int32, device="cuda")
    k_src = torch.randn(nb, BS, HKV, D, device="cuda").half()
    v_src = torch.randn(nb, BS, HKV, D, device="cuda").half()
    resid = init_k_residual(k_src, bt.clamp(0, nb - 1), torch.tensor([5, 5, 5, 49],
                            dtype=torch.int32, device="cuda"))
    resid0 = resid.clone()
    k_new = torch.randn(4, HKV, D, device="cuda").half()
    v_new = torch.randn(4, HKV, D, device="cuda").half()
    before = storage(qc)
    quantize_append(qc, k_new, v_new, bt, lens, resid)
    torch.cuda.synchronize()
    after = storage(qc)
    seq3 = list(range(36, 48))  # the blocks of the valid sequence
    for name, b_, a_ in zip(("k_codes", "v_codes", "k_sz", "v_sz"), before, after):
        keep = np.ones(b_.shape[0], bool)
        keep[seq3] = False
        assert np.array_equal(b_[keep], a_[keep]), f"{fmt} {name}: a skipped sequence wrote"
    # the valid sequence: its new V row (slot 49 = block 39, slot 1) was written
    assert not np.array_equal(before[1][39, :, 1], after[1][39, :, 1])
    # residuals: sequences 0-2 untouched, sequence 3 got its new K row (row 49 of group 0)
    r0, r1 = resid0.cpu().numpy(), resid.cpu().numpy()
    assert np.array_equal(r0[:3].view(np.uint16), r1[:3].view(np.uint16))
    assert np.array_equal(r1[3, :, 49], k_new[3].cpu().numpy())


@pytest.mark.parametrize("fmt", FORMATS)
def test_bulk_quantizer_skips_pages_outside_the_pool(fmt):
    nb = 40
    qc = filled_cache(nb, fmt, 2)
    # blocks 0-19 are used; 20-39 (the last one included) are named by no valid entry
    bt = torch.arange(20, dtype=torch.int32, device="cuda").view(2, 10).contiguous()
    bt[0, 3] = -1
    bt[1, 9] = nb
    bt[1, 0] = nb + 5  # sequence 1's first K group has no page for its pairs
    lens = torch.tensor([160, 160], dtype=torch.int32, device="cuda")
    k_src = torch.randn(nb, BS, HKV, D, device="cuda").half()
    v_src = torch.randn(nb, BS, HKV, D, device="cuda").half()
    before = storage(qc)
    quantize_paged_cache(k_src, v_src, bt, lens, fmt, out=qc)
    torch.cuda.synchronize()
    after = storage(qc)
    for name, b_, a_ in zip(("k_codes", "v_codes", "k_sz", "v_sz"), before, after):
        assert np.array_equal(b_[20:], a_[20:]), f"{fmt} {name}: wrote outside the table"
    # sequence 1's first K group (pages 0-7) has no pair page: its valid pages 1-7 keep
    # their K bytes. Its page 1 (block 11) shares its V (scale, zero) group with page 0,
    # also outside the pool, and keeps its V bytes; the V rows of pages 2-7 are written
    assert np.array_equal(before[0][11:18], after[0][11:18])
    assert np.array_equal(before[1][11], after[1][11])
    assert not np.array_equal(before[1][12:18], after[1][12:18])
    # sequence 0's page 3 is outside the pool; its other pages were written
    assert not np.array_equal(before[0][0:3], after[0][0:3])


def test_quantizer_argument_mismatches_raise(cuda):
    qc = allocate_quantized_cache(32, BS, HKV, D, "int4", cuda)
    bt = torch.zeros(4, 8, dtype=torch.int32, device=cuda)
    sl = torch.ones(4, dtype=torch.int32, device=cuda)
    k_new = torch.zeros(4, HKV, D, dtype=torch.float16, device=cuda)
    resid = torch.zeros(4, HKV, 128, D, dtype=torch.float16, device=cuda)
    cases = [
        # block_table rows != batch of new tokens
        lambda: quantize_append(qc, k_new[:3], k_new[:3], bt, sl, resid[:3]),
        # seq_lens length != block_table rows
        lambda: quantize_append(qc, k_new, k_new, bt, sl[:3], resid),
        # cache kv heads != k_new's
        lambda: quantize_append(qc, torch.zeros(4, 1, D, dtype=torch.float16, device=cuda),
                                torch.zeros(4, 1, D, dtype=torch.float16, device=cuda), bt, sl,
                                torch.zeros(4, 1, 128, D, dtype=torch.float16, device=cuda)),
        # block table / seq_lens / new rows on the host
        lambda: quantize_append(qc, k_new, k_new, bt.cpu(), sl, resid),
        lambda: quantize_append(qc, k_new, k_new, bt, sl.cpu(), resid),
        lambda: quantize_append(qc, k_new.cpu(), k_new, bt, sl, resid),
        lambda: quantize_append(qc, k_new, k_new, bt, sl, resid.cpu()),
        # a 1-D block table
        lambda: quantize_append(qc, k_new, k_new, bt[0], sl, resid),
    ]
    src = torch.zeros(16, BS, HKV, D, dtype=torch.float16, device=cuda)
    cases += [
        # an out= cache with more blocks than the source caches
        lambda: quantize_paged_cache(src, src, bt, sl, "int4", out=qc),
        # source caches on the host
        lambda: quantize_paged_cache(src.cpu(), src.cpu(), bt, sl, "int4",
                                     out=allocate_quantized_cache(16, BS, HKV, D, "int4", cuda)),
    ]
    for i, case in enumerate(cases):
        with pytest.raises(KvqArgumentError):
            case()
        torch.cuda.synchronize()
