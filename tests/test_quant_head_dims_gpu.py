"""Quantized decode at head_dim 64 and 256 (the Llama shape's 128 is covered by
test_quant_gpu.py and test_units_gpu.py). Needs a GPU.

Every case decodes INT8 / FP8-e4m3 / INT4 caches written by the library's bulk quantizer and
compares with float32 attention over the cache dequantized by the numpy spec, at the north
star's bar for quantized KV (|out - ref| <= 2e-3 + 1e-2 |ref|). Head dim 64 runs the same
kernel variants as 128 (chunk pairs for 1-8 q heads per kv head); 256 runs the single-chunk
kernel with at most 2 chunks in flight.
"""
import numpy as np
import pytest
import torch

from oracle import kivi
from oracle.attention import paged_decode_attention_ref

import test_quant_gpu as tq

pytestmark = pytest.mark.gpu

FORMATS = tq.FORMATS
HEAD_DIMS = [64, 256]


def case(fmt, D, lens, Hq=32, Hkv=8, bs=16, seed=1, k_group=128):
    """(gpu args, decode kwargs, float32 reference over the dequantized cache)."""
    from kvq_decode_amd.quant import quantize_paged_cache
    q, kc, vc, bt, sl = tq.make(lens, bs, Hq=Hq, Hkv=Hkv, D=D, seed=seed)
    qc = quantize_paged_cache(tq.gpu(kc), tq.gpu(vc), tq.gpu(bt), tq.gpu(sl), fmt,
                              k_group=k_group)
    host = {n: getattr(qc, n).cpu().numpy() for n in
            ("k_codes", "v_codes", "k_scale", "k_zero", "v_scale", "v_zero")}
    kd, vd = kivi.dequantize_paged_cache(host, bt, sl, fmt, group=k_group)
    ref = paged_decode_attention_ref(q.astype(np.float32), kd, vd, bt, sl, out_dtype=np.float32)
    args = (tq.gpu(q), qc.k_codes, qc.v_codes, tq.gpu(bt), tq.gpu(sl))
    return args, qc.decode_kwargs(), ref


@pytest.mark.parametrize("bs", [16, 32])
@pytest.mark.parametrize("fmt", FORMATS)
@pytest.mark.parametrize("D", HEAD_DIMS)
def test_decode_other_head_dims(D, fmt, bs):
    """Single pass, 3 splits, 7 work units and the default plan over ragged lengths (a
    length-1 sequence, partial last chunks, odd chunk counts)."""
    from kvq_decode_amd import paged_decode_attention
    args, kw, ref = case(fmt, D, [1, 37, 300, 2049, 129], bs=bs)
    for extra in ({"num_splits": 1}, {"num_splits": 3}, {"units": 7}, {}):
        out = paged_decode_attention(*args, **extra, **kw)
        tq.check_close(out, ref, f"{fmt} D={D} bs={bs} {extra}")


@pytest.mark.parametrize("fmt", FORMATS)
@pytest.mark.parametrize("D", HEAD_DIMS)
def test_head_groups_other_head_dims(D, fmt):
    """1, 2 and 4 q heads per kv head (chunk pairs at D = 64), 5 and 8 (chunk pairs with hi /
    lo columns at D = 64, one chain at 256), 16 (two chains) and 20 (two head blocks of 10),
    split and work-unit paths."""
    from kvq_decode_amd import paged_decode_attention
    for Hq, Hkv in ((8, 8), (4, 2), (8, 2), (10, 2), (16, 2), (32, 2), (40, 2)):
        args, kw, ref = case(fmt, D, [700, 3], Hq=Hq, Hkv=Hkv, seed=2)
        for extra in ({"num_splits": 2}, {"units": 3}):
            out = paged_decode_attention(*args, **extra, **kw)
            tq.check_close(out, ref, f"{fmt} D={D} Hq={Hq} Hkv={Hkv} {extra}")


@pytest.mark.parametrize("fmt", FORMATS)
@pytest.mark.parametrize("D", HEAD_DIMS)
def test_rings_and_workgroup_shapes_other_head_dims(D, fmt):
    """Every (waves per workgroup, loads in flight) variant the head dim takes (256: rings
    of 1 or 2 chunks; INT8 / FP8 up to 4 waves, whose staging tiles fill the 64 KB LDS
    budget at 8) is within tolerance, and the ring depth never changes a result bit."""
    from kvq_decode_amd import paged_decode_attention
    from kvq_decode_amd._lib import KvqError
    args, kw, ref = case(fmt, D, [1, 129, 300, 2049, 700], seed=5)
    rings = (1, 2, 4) if D < 256 else (1, 2)
    waves_all = (1, 2, 4) if D == 256 and fmt != "int4" else (1, 2, 4, 8)
    if D == 256:
        with pytest.raises(KvqError, match="unsupported"):  # ring depth 4 at head_dim 256
            paged_decode_attention(*args, num_splits=1, pipeline=4, **kw)
        if fmt != "int4":
            with pytest.raises(KvqError, match="unsupported"):
                paged_decode_attention(*args, num_splits=1, waves_per_group=8, **kw)
    for splits in (1, 3):
        by_waves = {}
        for waves in waves_all:
            for ring in rings:
                out = paged_decode_attention(*args, num_splits=splits, waves_per_group=waves,
                                             pipeline=ring, **kw)
                tq.check_close(out, ref, f"{fmt} D={D} splits={splits} waves={waves} "
                                         f"ring={ring}")
                by_waves.setdefault(waves, []).append(out)
        for waves, outs in by_waves.items():
            assert all(torch.equal(outs[0], o) for o in outs[1:]), (fmt, D, splits, waves)


@pytest.mark.parametrize("k_group", [16, 256])
@pytest.mark.parametrize("fmt", FORMATS)
@pytest.mark.parametrize("D", HEAD_DIMS)
def test_k_groups_other_head_dims(D, fmt, k_group):
    """K scale groups of 1 chunk (the single-chunk kernel at every head count) and 16
    chunks, on the split and work-unit paths."""
    from kvq_decode_amd import paged_decode_attention
    args, kw, ref = case(fmt, D, [5, 300, 1000], seed=6, k_group=k_group)
    for extra in ({"num_splits": 2}, {"units": 5}):
        out = paged_decode_attention(*args, **extra, **kw)
        tq.check_close(out, ref, f"{fmt} D={D} k_group={k_group} {extra}")


@pytest.mark.parametrize("fmt", FORMATS)
@pytest.mark.parametrize("D", HEAD_DIMS)
def test_nan_garbage_other_head_dims(D, fmt):
    """Codes and V (scale, zero) pairs past each sequence's end poisoned with NaN-producing
    bytes: the masked slots never reach the output."""
    from kvq_decode_amd import paged_decode_attention
    from kvq_decode_amd.quant import quantize_paged_cache
    lens, bs = [37, 300, 129], 16
    q, kc, vc, bt, sl = tq.make(lens, bs, D=D, seed=7)
    qc = quantize_paged_cache(tq.gpu(kc), tq.gpu(vc), tq.gpu(bt), tq.gpu(sl), fmt)
    host = {n: getattr(qc, n).cpu().numpy() for n in
            ("k_codes", "v_codes", "k_scale", "k_zero", "v_scale", "v_zero")}
    kd, vd = kivi.dequantize_paged_cache(host, bt, sl, fmt)
    ref = paged_decode_attention_ref(q.astype(np.float32), kd, vd, bt, sl, out_dtype=np.float32)
    nan16 = torch.tensor(float("nan"), dtype=torch.float16)
    vg = max(bs, 32)  # tokens per V (scale, zero) group
    for b, n in enumerate(lens):
        if n % bs:
            blk = int(bt[b, (n - 1) // bs])
            qc.k_codes[blk, n % bs:] = 0xFF
            qc.v_codes[blk, n % bs:] = 0xFF
        if n % vg:  # the pairs past the end of the sequence's last V group
            vlead = int(bt[b, ((n - 1) // vg) * vg // bs])
            qc.v_sz[vlead, :, n % vg:] = nan16
    args = (tq.gpu(q), qc.k_codes, qc.v_codes, tq.gpu(bt), tq.gpu(sl))
    for extra in ({"num_splits": 1}, {"num_splits": 3}, {"units": 4}):
        out = paged_decode_attention(*args, **extra, **qc.decode_kwargs())
        tq.check_close(out, ref, f"{fmt} D={D} poisoned {extra}")


@pytest.mark.parametrize("fmt, D, Hq, Hkv, lens", [
    ("int4", 256, 32, 4, [4096]),        # split plan: 8-wave workgroups would need 82944 B
    ("int8", 256, 32, 2, [4096]),        # split plan: 4 waves, 78336 B
    ("int8", 256, 32, 2, [4096, 3000]),  # work units: 4 waves, 78336 B
    ("fp8_e4m3", 256, 32, 2, [4096, 3000]),
    ("int4", 128, 128, 8, [4096]),       # 16 q heads per kv head: 8 waves, 74752 B
])
def test_default_plan_fits_lds(fmt, D, Hq, Hkv, lens):
    """The default plan (num_splits=None) at shapes whose first-choice workgroups would
    pass the 64 KB LDS budget: the plans halve the waves (more splits or units) instead of
    handing the decode a workgroup it must reject, and the result matches the oracle."""
    from kvq_decode_amd import paged_decode_attention
    from kvq_decode_amd.ops import head_blocks, plan_decode, plan_units
    args, kw, ref = case(fmt, D, lens, Hq=Hq, Hkv=Hkv, seed=11)
    grid_heads = Hkv * head_blocks(Hq, Hkv)
    pages = args[3].shape[1]
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    units, uw = plan_units(len(lens), grid_heads, 16, pages, cus, fmt, D, Hq)
    splits, sw = plan_decode(len(lens), grid_heads, 16, pages, cus, fmt, D, Hq)
    print(f"{fmt} D={D} {Hq}q/{Hkv}kv lens={lens}: units {units}x{uw}, splits {splits}x{sw}",
          flush=True)
    out = paged_decode_attention(*args, **kw)
    tq.check_close(out, ref, f"{fmt} D={D} Hq={Hq} Hkv={Hkv} default plan")
