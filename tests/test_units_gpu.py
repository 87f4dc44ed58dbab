"""Work-unit decode (kvq_decode_units) vs the numpy oracle. Needs a GPU.

The work-unit path computes the same attention as the split-KV path over a different
partition (per kv head, the concatenated chunks of the batch cut into equal ranges), so it
is held to the same bar: |out - ref| <= 2e-3 + 1e-2 * |ref| elementwise and max-abs < 2e-3
against the oracle's float32 output (reference tests/test_triton_fp16.py:42).
"""
import numpy as np
import pytest
import torch

from oracle.attention import paged_decode_attention_ref
from test_decode_gpu import check_close, make, to_gpu

pytestmark = pytest.mark.gpu


# units 1 = one wave per kv head runs the whole batch; 3 and 7 cut sequences at odd
# chunk boundaries; 1000 exceeds the chunk count (NU = N, one chunk per unit)
@pytest.mark.parametrize("units", [1, 3, 7, 64, 1000])
@pytest.mark.parametrize("Hq,Hkv,D", [(32, 8, 128), (4, 4, 64), (8, 1, 64)])
@pytest.mark.parametrize("block_size", [16, 32])
@pytest.mark.parametrize("lens", [[1], [37], [100, 33, 1, 64], [4096, 1000, 17, 2049]])
def test_units_match_reference(Hq, Hkv, D, block_size, lens, units):
    from kvq_decode_amd import paged_decode_attention
    q, kc, vc, bt, sl = make(Hq, Hkv, D, block_size, lens)
    ref = paged_decode_attention_ref(q, kc, vc, bt, sl, out_dtype=np.float32)
    out = paged_decode_attention(*to_gpu(q, kc, vc, bt, sl), units=units)
    torch.cuda.synchronize()
    check_close(out, ref, f"units={units} Hq={Hq} Hkv={Hkv} D={D} bs={block_size} lens={lens}")


@pytest.mark.parametrize("D", [16, 32, 256])
@pytest.mark.parametrize("pipeline", [1, 2, 4])
def test_units_head_dims_and_ring_depths(D, pipeline):
    from kvq_decode_amd import paged_decode_attention
    if D == 256 and pipeline == 4:
        pytest.skip("ring depth 4 is not built for head_dim 256")
    q, kc, vc, bt, sl = make(8, 2, D, 16, [700, 3, 129, 2000, 16], seed=3)
    ref = paged_decode_attention_ref(q, kc, vc, bt, sl, out_dtype=np.float32)
    out = paged_decode_attention(*to_gpu(q, kc, vc, bt, sl), units=13, pipeline=pipeline)
    torch.cuda.synchronize()
    check_close(out, ref, f"units=13 D={D} pipeline={pipeline}")


@pytest.mark.parametrize("B", [65, 256, 257, 1000, 1024])
def test_units_full_batch_ragged(B):
    """Up to 1024 sequences (the work-unit limit; past 64 every lane of the prefix scan
    takes several sequences, past 256 every merge thread several) of lengths 1 .. 600,
    fewer units than sequences and more, against the oracle."""
    from kvq_decode_amd import paged_decode_attention
    rng = np.random.default_rng(7 + B)
    lens = [int(x) for x in rng.integers(1, 600, B)]
    q, kc, vc, bt, sl = make(8, 2, 64, 16, lens, seed=7)
    ref = paged_decode_attention_ref(q, kc, vc, bt, sl, out_dtype=np.float32)
    args = to_gpu(q, kc, vc, bt, sl)
    for units in (40, 300, 5000):
        out = paged_decode_attention(*args, units=units)
        torch.cuda.synchronize()
        check_close(out, ref, f"B={B} units={units}")


def test_units_empty_sequences_give_zero_rows():
    """seq_lens 0 (which the split path's callers must not pass) yields a zero row here;
    the other sequences are unaffected."""
    from kvq_decode_amd import paged_decode_attention
    q, kc, vc, bt, sl = make(8, 2, 64, 16, [300, 40, 500, 17], seed=5)
    ref = paged_decode_attention_ref(q, kc, vc, bt, sl, out_dtype=np.float32)
    sl0 = sl.copy()
    sl0[1] = 0
    sl0[3] = 0
    out = paged_decode_attention(*to_gpu(q, kc, vc, bt, sl0), units=9)
    torch.cuda.synchronize()
    assert torch.count_nonzero(out[1]) == 0 and torch.count_nonzero(out[3]) == 0
    check_close(out[[0, 2]], ref[[0, 2]], "units with empty sequences")


def test_units_deterministic_and_agree_with_splits():
    from kvq_decode_amd import paged_decode_attention
    args = to_gpu(*make(32, 8, 128, 16, [4096, 1000, 17, 2049]))
    a = paged_decode_attention(*args, units=50)
    b = paged_decode_attention(*args, units=50)
    assert torch.equal(a, b)
    s = paged_decode_attention(*args, num_splits=8)
    assert (a.float() - s.float()).abs().max().item() < 2e-3


def test_units_workspace_and_limits():
    from kvq_decode_amd import paged_decode_attention
    q, kc, vc, bt, sl = to_gpu(*make(8, 2, 64, 16, [100, 200], seed=1))
    units = 6
    ws = (torch.empty((8, units + 2, 64), dtype=torch.float32, device="cuda"),
          torch.empty((8, units + 2), dtype=torch.float32, device="cuda"))
    a = paged_decode_attention(q, kc, vc, bt, sl, units=units, workspace=ws)
    b = paged_decode_attention(q, kc, vc, bt, sl, units=units)
    assert torch.equal(a, b)
    from kvq_decode_amd._lib import KvqError
    from kvq_decode_amd.ops import KvqArgumentError
    with pytest.raises(KvqArgumentError):
        paged_decode_attention(q, kc, vc, bt, sl, units=units,
                               workspace=(ws[0][:, :units].contiguous(), ws[1]))
    # more sequences than one workgroup's prefix table holds
    q2, kc2, vc2, bt2, sl2 = to_gpu(*make(2, 1, 32, 16, [5] * 1025, seed=2))
    with pytest.raises(KvqError):
        paged_decode_attention(q2, kc2, vc2, bt2, sl2, units=8)


def test_units_partition_past_32_bit_products():
    """65537 units over 65537 chunks (two sequences of about 512k tokens): the unit bounds
    u N / NU and the merge's unit lookups pass 2^32 for the upper units, where the kernels
    leave their 32-bit arithmetic for 64-bit. Held to the split plan's result (the split
    and unit paths are each checked against the oracle above)."""
    from kvq_decode_amd import paged_decode_attention
    g = torch.Generator(device="cuda").manual_seed(11)
    lens = [524288, 524304]  # 32768 + 32769 chunks
    Hq, Hkv, D, BS = 4, 1, 64, 16
    pages = [(n + BS - 1) // BS for n in lens]
    pool = sum(pages)
    q = torch.randn(2, Hq, D, generator=g, device="cuda").half()
    kc = torch.randn(pool, BS, Hkv, D, generator=g, device="cuda").half()
    vc = torch.randn(pool, BS, Hkv, D, generator=g, device="cuda").half()
    perm = torch.randperm(pool, generator=g, device="cuda").int()
    bt = torch.zeros(2, max(pages), dtype=torch.int32, device="cuda")
    bt[0, :pages[0]] = perm[:pages[0]]
    bt[1, :pages[1]] = perm[pages[0]:]
    sl = torch.tensor(lens, dtype=torch.int32, device="cuda")
    n_chunks = sum((n + 15) // 16 for n in lens)
    assert (n_chunks - 1) * n_chunks >= 1 << 32
    print(f"\n[units={n_chunks} over {n_chunks} chunks]", flush=True)
    big = paged_decode_attention(q, kc, vc, bt, sl, units=n_chunks)
    small = paged_decode_attention(q, kc, vc, bt, sl, units=1000)
    split = paged_decode_attention(q, kc, vc, bt, sl, num_splits=64)
    torch.cuda.synchronize()
    ref = split.float().cpu().numpy()
    for name, out in (("units=65537", big), ("units=1000", small)):
        o = out.float().cpu().numpy()
        diff = np.abs(o - ref)
        print(f"[{name} vs 64 splits] max_abs={diff.max():.3e}", flush=True)
        assert np.isfinite(o).all()
        assert diff.max() < 2e-3 and np.all(diff <= 2e-3 + 1e-2 * np.abs(ref))


QFORMATS = ["int8", "fp8_e4m3", "int4"]


def _quant_case(fmt, lens, Hq=32, Hkv=8, bs=16, seed=1, k_group=128):
    """(gpu args, decode kwargs, float32 reference over the dequantized cache)."""
    from oracle import kivi
    from kvq_decode_amd.quant import quantize_paged_cache
    import test_quant_gpu as tq
    q, kc, vc, bt, sl = tq.make(lens, bs, Hq=Hq, Hkv=Hkv, seed=seed)
    qc = quantize_paged_cache(tq.gpu(kc), tq.gpu(vc), tq.gpu(bt), tq.gpu(sl), fmt,
                              k_group=k_group)
    host = {n: getattr(qc, n).cpu().numpy() for n in
            ("k_codes", "v_codes", "k_scale", "k_zero", "v_scale", "v_zero")}
    kd, vd = kivi.dequantize_paged_cache(host, bt, sl, fmt, group=k_group)
    ref = paged_decode_attention_ref(q.astype(np.float32), kd, vd, bt, sl, out_dtype=np.float32)
    args = (tq.gpu(q), qc.k_codes, qc.v_codes, tq.gpu(bt), tq.gpu(sl))
    return args, qc.decode_kwargs(), ref


# units 3 and 7 cut sequences at odd chunks (the chunk-pair kernel's single-chunk edges
# and K groups split between units); 1000 gives one chunk per unit
@pytest.mark.parametrize("units", [1, 3, 7, 64, 1000])
@pytest.mark.parametrize("fmt", QFORMATS)
def test_units_quantized(fmt, units):
    from kvq_decode_amd import paged_decode_attention
    args, kw, ref = _quant_case(fmt, [1, 37, 300, 2049, 129])
    out = paged_decode_attention(*args, units=units, **kw)
    torch.cuda.synchronize()
    check_close(out, ref, f"{fmt} units={units}")


@pytest.mark.parametrize("fmt", QFORMATS)
def test_units_quantized_groups_rings_and_k_groups(fmt):
    """Head groups of every quantized kernel variant (pairs: 1-4 heads; one chain: 5-8;
    two chains: 9-16), ring depths 1, 2, 4 and K groups of 1 and 16 chunks."""
    from kvq_decode_amd import paged_decode_attention
    for Hq, Hkv in ((8, 8), (6, 2), (10, 2), (32, 2)):
        args, kw, ref = _quant_case(fmt, [700, 3, 129], Hq=Hq, Hkv=Hkv, seed=2)
        for ring in (1, 2, 4):
            out = paged_decode_attention(*args, units=11, pipeline=ring, **kw)
            torch.cuda.synchronize()
            check_close(out, ref, f"{fmt} Hq={Hq} Hkv={Hkv} ring={ring} units=11")
    for k_group in (16, 256):
        args, kw, ref = _quant_case(fmt, [5, 300, 1000], seed=6, k_group=k_group)
        out = paged_decode_attention(*args, units=9, **kw)
        torch.cuda.synchronize()
        check_close(out, ref, f"{fmt} k_group={k_group} units=9")


def test_units_c5_shape_int4():
    """The C5 shape (INT4, 64 sequences of U[1024, 32768] tokens) at a tenth of the
    lengths, with the unit count the work plan would use, against the oracle on every
    sequence."""
    from kvq_decode_amd import paged_decode_attention
    lens = (np.random.default_rng(0).integers(1024, 32769, 64) // 10).tolist()
    args, kw, ref = _quant_case("int4", lens, seed=3)
    out = paged_decode_attention(*args, units=256, **kw)
    torch.cuda.synchronize()
    check_close(out, ref, "int4 C5/10 units=256")


@pytest.mark.parametrize("waves", [2, 4])
@pytest.mark.parametrize("fmt", ["fp16"] + QFORMATS)
def test_units_multi_wave_workgroups(fmt, waves):
    """W waves per unit share each segment (contiguous shares, combined through LDS)."""
    from kvq_decode_amd import paged_decode_attention
    lens = [1, 37, 300, 2049, 129, 5000]
    if fmt == "fp16":
        q, kc, vc, bt, sl = make(32, 8, 128, 16, lens, seed=8)
        ref = paged_decode_attention_ref(q, kc, vc, bt, sl, out_dtype=np.float32)
        args, kw = to_gpu(q, kc, vc, bt, sl), {}
    else:
        args, kw, ref = _quant_case(fmt, lens, seed=8)
    for units in (1, 5, 40):
        out = paged_decode_attention(*args, units=units, waves_per_group=waves, **kw)
        torch.cuda.synchronize()
        check_close(out, ref, f"{fmt} units={units} W={waves}")


@pytest.mark.parametrize("bs", [32, 64])
@pytest.mark.parametrize("fmt", ["fp16"] + QFORMATS)
def test_units_larger_pages(fmt, bs):
    """Pages of 2 and 4 chunks: units that start and end inside a page, K groups of 128
    tokens spanning 4 and 2 pages."""
    from kvq_decode_amd import paged_decode_attention
    lens = [5, 1000, 64, 2500, 129, 33]
    if fmt == "fp16":
        q, kc, vc, bt, sl = make(32, 8, 128, bs, lens, seed=13)
        ref = paged_decode_attention_ref(q, kc, vc, bt, sl, out_dtype=np.float32)
        args, kw = to_gpu(q, kc, vc, bt, sl), {}
    else:
        args, kw, ref = _quant_case(fmt, lens, bs=bs, seed=13)
    for units in (7, 32, 128):
        out = paged_decode_attention(*args, units=units, **kw)
        torch.cuda.synchronize()
        check_close(out, ref, f"{fmt} bs={bs} units={units}")


@pytest.mark.parametrize("lens", [[3000, 17, 900, 64], [5000], [300] * 64])
def test_plan_workspace_shapes_fit_the_default_plan(lens):
    """A workspace preallocated from plan_workspace_shapes serves the default plan (work
    units, splits or a single pass) and gives the same output as the op's own."""
    from kvq_decode_amd import _sm_count, paged_decode_attention, plan_workspace_shapes
    q, kc, vc, bt, sl = make(32, 8, 128, 16, lens, seed=17)
    args = to_gpu(q, kc, vc, bt, sl)
    shapes = plan_workspace_shapes(len(lens), 32, 8, 128, 16, bt.shape[1], _sm_count(0))
    ws = None if shapes is None else tuple(
        torch.empty(s, dtype=torch.float32, device="cuda") for s in shapes)
    a = paged_decode_attention(*args, workspace=ws)
    b = paged_decode_attention(*args)
    torch.cuda.synchronize()
    assert torch.equal(a, b)


@pytest.mark.parametrize("D", [16, 32, 64])
@pytest.mark.parametrize("lens", [[3000, 17, 900, 64], [5000]])
def test_head_dim_plans_default_path(D, lens):
    """Below head_dim 128 the default plan runs more waves (fp16: work units in 4-wave
    workgroups; one sequence: splits in 4-wave workgroups): against the oracle, and a
    workspace preallocated from plan_workspace_shapes(head_dim=D) serves it bit for bit."""
    from kvq_decode_amd import _sm_count, paged_decode_attention, plan_workspace_shapes
    from kvq_decode_amd.ops import plan_decode, plan_units
    q, kc, vc, bt, sl = make(32, 8, D, 16, lens, seed=19)
    cus = _sm_count(0)
    B, pages = len(lens), bt.shape[1]
    units, waves = plan_units(B, 8, 16, pages, cus, "fp16", D)
    if units:
        assert waves == 4, (units, waves)
    else:
        assert plan_decode(B, 8, 16, pages, cus, "fp16", D)[1] == 4
    ref = paged_decode_attention_ref(q, kc, vc, bt, sl, out_dtype=np.float32)
    args = to_gpu(q, kc, vc, bt, sl)
    out = paged_decode_attention(*args)
    shapes = plan_workspace_shapes(B, 32, 8, D, 16, pages, cus)
    ws = None if shapes is None else tuple(
        torch.empty(sh, dtype=torch.float32, device="cuda") for sh in shapes)
    out_ws = paged_decode_attention(*args, workspace=ws)
    torch.cuda.synchronize()
    check_close(out, ref, f"default plan D={D} lens={lens}")
    assert torch.equal(out, out_ws)


@pytest.mark.parametrize("fmt", ["fp16"] + QFORMATS)
@pytest.mark.parametrize("Hq,Hkv", [(16, 2), (32, 2), (8, 1), (4, 2)])
def test_units_head_groups(fmt, Hq, Hkv):
    """Work units for every q-head group the kernels specialise: 2 (chunk pairs), 8 (one
    MFMA chain with hi / lo columns, MQA here too) and 16 (two chains), ragged lengths."""
    from kvq_decode_amd import paged_decode_attention
    lens = [900, 5, 2100, 300]
    if fmt == "fp16":
        q, kc, vc, bt, sl = make(Hq, Hkv, 128, 16, lens, seed=19)
        ref = paged_decode_attention_ref(q, kc, vc, bt, sl, out_dtype=np.float32)
        args, kw = to_gpu(q, kc, vc, bt, sl), {}
    else:
        args, kw, ref = _quant_case(fmt, lens, Hq=Hq, Hkv=Hkv, seed=19)
    for units in (9, 64):
        out = paged_decode_attention(*args, units=units, **kw)
        torch.cuda.synchronize()
        check_close(out, ref, f"{fmt} Hq={Hq} Hkv={Hkv} units={units}")
