"""KIVI-quantized KV on the GPU vs the numpy spec (oracle/kivi.py). Needs a GPU.

  * bulk quantizer: codes and scales bit-exact with the spec (valid slots only);
  * decode over INT8 / FP8-e4m3 / INT4 caches: within |out - ref| <= 2e-3 + 1e-2 |ref| of
    float32 attention over the dequantized cache (the north star's bar for quantized KV);
  * quantize-on-append: appending tokens one at a time leaves exactly the cache the bulk
    quantizer produces for all tokens.
K ~ N(0,1) with 4 random outlier channels per kv head scaled x10.
"""
import numpy as np
import pytest
import torch

from oracle import kivi
from oracle.attention import build_paged_cache, paged_decode_attention_ref

pytestmark = pytest.mark.gpu

ATOL, RTOL = 2e-3, 1e-2
FORMATS = ["int8", "fp8_e4m3", "int4"]


def make(lens, bs, Hq=32, Hkv=8, D=128, seed=0, outliers=True):
    rng = np.random.default_rng(seed)
    B, S = len(lens), max(lens)
    q = rng.standard_normal((B, Hq, D)).astype(np.float16)
    k = rng.standard_normal((B, S, Hkv, D)).astype(np.float32)
    if outliers:
        for h in range(Hkv):
            k[:, :, h, rng.choice(D, 4, replace=False)] *= 10
    k = k.astype(np.float16)
    v = rng.standard_normal((B, S, Hkv, D)).astype(np.float16)
    sl = np.array(lens, np.int32)
    kc, vc, bt = build_paged_cache(k, v, sl, bs, rng)
    return q, kc, vc, bt, sl


def gpu(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def valid_slots(bt, sl, bs):
    """(phys, slot) of every valid token."""
    out = []
    for b, n in enumerate(sl):
        for t in range(int(n)):
            out.append((int(bt[b, t // bs]), t % bs))
    return np.array(out)


def v_pair_slots(bt, sl, bs):
    """(block, index) of every valid token's V (scale, zero) pair: index t % VG of its V
    group's first page, VG = max(block_size, 32) (include/kvq.h)."""
    vg = max(bs, 32)
    out = []
    for b, n in enumerate(sl):
        for t in range(int(n)):
            out.append((int(bt[b, (t // vg) * vg // bs]), t % vg))
    return np.array(out)


def lead_blocks(bt, sl, bs, group=128):
    return sorted({int(bt[b, (g * group) // bs]) for b, n in enumerate(sl)
                   for g in range(-(-int(n) // group))})


def check_close(out, ref, tag):
    out = out.float().cpu().numpy()
    diff = np.abs(out - ref)
    print(f"\n[{tag}] max_abs={diff.max():.3e} "
          f"max_rel(clamp 1e-3)={(diff / np.maximum(np.abs(ref), 1e-3)).max():.3e}", flush=True)
    assert np.isfinite(out).all()
    assert diff.max() < ATOL
    assert np.all(diff <= ATOL + RTOL * np.abs(ref))


@pytest.mark.parametrize("fmt", FORMATS)
@pytest.mark.parametrize("bs", [16, 32])
def test_bulk_quantizer_bit_exact(fmt, bs):
    from kvq_decode_amd.quant import quantize_paged_cache
    q, kc, vc, bt, sl = make([1, 37, 128, 129, 300, 1000], bs)
    want = kivi.quantize_paged_cache(kc, vc, bt, sl, fmt)
    got = quantize_paged_cache(gpu(kc), gpu(vc), gpu(bt), gpu(sl), fmt)
    torch.cuda.synchronize()
    slots = valid_slots(bt, sl, bs)
    vsl = v_pair_slots(bt, sl, bs)
    for name in ("k_codes", "v_codes"):
        g = getattr(got, name).cpu().numpy()[slots[:, 0], slots[:, 1]]
        w = want[name][slots[:, 0], slots[:, 1]]
        assert np.array_equal(g, w), f"{name}: {np.sum(g != w)} of {g.size} bytes differ"
    lead = lead_blocks(bt, sl, bs)
    for name in ("k_scale", "k_zero"):
        g = getattr(got, name).cpu().numpy()[lead].view(np.uint16)
        assert np.array_equal(g, want[name][lead].view(np.uint16)), name
    for name in ("v_scale", "v_zero"):
        g = getattr(got, name).cpu().numpy()[vsl[:, 0], :, vsl[:, 1]].view(np.uint16)
        w = want[name][vsl[:, 0], :, vsl[:, 1]].view(np.uint16)
        assert np.array_equal(g, w), name


@pytest.mark.parametrize("D", [64, 256])
@pytest.mark.parametrize("fmt", FORMATS)
def test_bulk_quantizer_other_head_dims(fmt, D):
    """The quantizers take the decode's head dims 64, 128 and 256 (lanes of 8 channels: 8
    to 32 lanes per row), bit-exact with the spec, including K groups longer than the rows
    a lane keeps in registers (k_group 256)."""
    from kvq_decode_amd.quant import quantize_paged_cache
    q, kc, vc, bt, sl = make([1, 37, 300, 700], 16, Hq=4, Hkv=2, D=D, seed=9)
    for k_group in (128, 256):
        want = kivi.quantize_paged_cache(kc, vc, bt, sl, fmt, group=k_group)
        got = quantize_paged_cache(gpu(kc), gpu(vc), gpu(bt), gpu(sl), fmt, k_group=k_group)
        torch.cuda.synchronize()
        slots = valid_slots(bt, sl, 16)
        vsl = v_pair_slots(bt, sl, 16)
        for name in ("k_codes", "v_codes"):
            g = getattr(got, name).cpu().numpy()[slots[:, 0], slots[:, 1]]
            w = want[name][slots[:, 0], slots[:, 1]]
            assert np.array_equal(g, w), f"{name} D={D} k_group={k_group}"
        lead = lead_blocks(bt, sl, 16, k_group)
        for name in ("k_scale", "k_zero"):
            g = getattr(got, name).cpu().numpy()[lead].view(np.uint16)
            assert np.array_equal(g, want[name][lead].view(np.uint16)), name
        for name in ("v_scale", "v_zero"):
            g = getattr(got, name).cpu().numpy()[vsl[:, 0], :, vsl[:, 1]].view(np.uint16)
            w = want[name][vsl[:, 0], :, vsl[:, 1]].view(np.uint16)
            assert np.array_equal(g, w), name


@pytest.mark.parametrize("D", [64, 256])
@pytest.mark.parametrize("fmt", FORMATS)
def test_append_equals_bulk_other_head_dims(fmt, D):
    """Quantize-on-append at head_dim 64 and 256 (8 to 32 lanes per row): a few appended
    tokens, crossing a 128-token K group, leave the bulk quantization of all tokens."""
    from kvq_decode_amd.quant import init_k_residual, quantize_append, quantize_paged_cache
    bs, Hkv = 16, 2
    n0, n1 = [126, 40, 1], [130, 42, 3]
    q, kc, vc, bt, sl1 = make(n1, bs, Hq=4, Hkv=Hkv, D=D, seed=21)
    kc_g, vc_g, bt_g = gpu(kc), gpu(vc), gpu(bt)
    sl0 = torch.tensor(n0, dtype=torch.int32, device="cuda")
    qc = quantize_paged_cache(kc_g, vc_g, bt_g, sl0, fmt)
    resid = init_k_residual(kc_g, bt_g, sl0)
    cur = list(n0)
    while cur != n1:
        cur = [min(c + 1, e) for c, e in zip(cur, n1)]
        k_new = torch.stack([kc_g[bt_g[b, (t - 1) // bs], (t - 1) % bs] for b, t in enumerate(cur)])
        v_new = torch.stack([vc_g[bt_g[b, (t - 1) // bs], (t - 1) % bs] for b, t in enumerate(cur)])
        quantize_append(qc, k_new.contiguous(), v_new.contiguous(), bt_g,
                        torch.tensor(cur, dtype=torch.int32, device="cuda"), resid)
    want = quantize_paged_cache(kc_g, vc_g, bt_g, gpu(sl1), fmt)
    torch.cuda.synchronize()
    slots = valid_slots(bt, sl1, bs)
    vsl = v_pair_slots(bt, sl1, bs)
    for name in ("k_codes", "v_codes"):
        g = getattr(qc, name).cpu().numpy()[slots[:, 0], slots[:, 1]]
        w = getattr(want, name).cpu().numpy()[slots[:, 0], slots[:, 1]]
        assert np.array_equal(g, w), f"{name} D={D}"
    lead = lead_blocks(bt, sl1, bs)
    for name in ("k_scale", "k_zero"):
        assert np.array_equal(getattr(qc, name).cpu().numpy()[lead],
                              getattr(want, name).cpu().numpy()[lead]), name
    for name in ("v_scale", "v_zero"):
        g = getattr(qc, name).cpu().numpy()[vsl[:, 0], :, vsl[:, 1]]
        w = getattr(want, name).cpu().numpy()[vsl[:, 0], :, vsl[:, 1]]
        assert np.array_equal(g, w), name


@pytest.mark.parametrize("k_group", [16, 64, 256])
@pytest.mark.parametrize("fmt", FORMATS)
def test_append_equals_bulk_other_k_groups(fmt, k_group):
    """Quantize-on-append with K groups of 16-256 tokens (256: more rows than a lane keeps
    in registers), appended one token at a time across group boundaries: the cache equals
    the bulk quantization of all tokens with the same group size, bit for bit."""
    from kvq_decode_amd.quant import init_k_residual, quantize_append, quantize_paged_cache
    bs, Hkv = 16, 2
    n0, n1 = [250, 15, 60, 1], [258, 17, 66, 6]
    q, kc, vc, bt, sl1 = make(n1, bs, Hq=4, Hkv=Hkv, seed=23)
    kc_g, vc_g, bt_g = gpu(kc), gpu(vc), gpu(bt)
    sl0 = torch.tensor(n0, dtype=torch.int32, device="cuda")
    qc = quantize_paged_cache(kc_g, vc_g, bt_g, sl0, fmt, k_group=k_group)
    resid = init_k_residual(kc_g, bt_g, sl0, k_group)
    cur = list(n0)
    while cur != n1:
        cur = [min(c + 1, e) for c, e in zip(cur, n1)]
        k_new = torch.stack([kc_g[bt_g[b, (t - 1) // bs], (t - 1) % bs] for b, t in enumerate(cur)])
        v_new = torch.stack([vc_g[bt_g[b, (t - 1) // bs], (t - 1) % bs] for b, t in enumerate(cur)])
        quantize_append(qc, k_new.contiguous(), v_new.contiguous(), bt_g,
                        torch.tensor(cur, dtype=torch.int32, device="cuda"), resid)
    want = quantize_paged_cache(kc_g, vc_g, bt_g, gpu(sl1), fmt, k_group=k_group)
    torch.cuda.synchronize()
    slots = valid_slots(bt, sl1, bs)
    vsl = v_pair_slots(bt, sl1, bs)
    for name in ("k_codes", "v_codes"):
        g = getattr(qc, name).cpu().numpy()[slots[:, 0], slots[:, 1]]
        w = getattr(want, name).cpu().numpy()[slots[:, 0], slots[:, 1]]
        assert np.array_equal(g, w), f"{name} k_group={k_group}"
    lead = lead_blocks(bt, sl1, bs, k_group)
    for name in ("k_scale", "k_zero"):
        assert np.array_equal(getattr(qc, name).cpu().numpy()[lead],
                              getattr(want, name).cpu().numpy()[lead]), name
    for name in ("v_scale", "v_zero"):
        assert np.array_equal(getattr(qc, name).cpu().numpy()[vsl[:, 0], :, vsl[:, 1]],
                              getattr(want, name).cpu().numpy()[vsl[:, 0], :, vsl[:, 1]]), name


def _tie_rows(rng, n, width, fmt):
    """n rows of `width` fp16 values whose first two entries are the row's min and max,
    chosen so that scale and zero come out exact (INT: z = -1.5, s = 2^-6; FP8: z = 0,
    s = 2^-6), and whose other entries sit on rounding boundaries of the quantized
    value: half-integer codes (INT) or midpoints between e4m3 values (FP8), half of them
    moved by one fp16 ulp."""
    s0 = 2.0 ** -6
    if fmt == "fp8_e4m3":
        lo, hi = -448 * s0, 448 * s0
        e = rng.integers(-6, 8, (n, width))
        k = rng.integers(0, 8, (n, width))
        mid = (8 + k + 0.5) * 2.0 ** (e - 3)
        sub = rng.random((n, width)) < 0.2  # subnormal midpoints (k + 1/2) 2^-9
        mid = np.where(sub, (k + 0.5) / 512.0, mid)
        x = np.where(rng.random((n, width)) < 0.5, -mid, mid) * s0
    else:
        R = 15 if fmt == "int4" else 255
        lo, hi = -1.5, -1.5 + R * s0
        x = lo + (rng.integers(0, R, (n, width)) + 0.5) * s0
    x = x.astype(np.float16)
    nudge = rng.integers(-1, 2, (n, width)).astype(np.int16)
    x = (x.view(np.int16) + np.where(rng.random((n, width)) < 0.5, nudge, 0)).view(np.float16)
    x[:, 0], x[:, 1] = lo, hi
    return x


@pytest.mark.parametrize("fmt", FORMATS)
def test_quantizer_rounding_ties(fmt):
    """Values on and one ulp off the codes' rounding boundaries (ties to even), per K
    channel group and per V row: bit-exact with the spec."""
    from kvq_decode_amd.quant import quantize_paged_cache
    rng = np.random.default_rng(12)
    lens, bs, Hkv, D = [300, 129, 45], 16, 2, 128
    B, S = len(lens), max(lens)
    # K: per channel, every 128-token group holds its min and max in its first two tokens
    k = np.empty((B, S, Hkv, D), np.float16)
    for b in range(B):
        for h in range(Hkv):
            for g0 in range(0, S, 128):
                n = min(128, S - g0)
                k[b, g0:g0 + n, h, :] = _tie_rows(rng, D, n, fmt).T
    v = _tie_rows(rng, B * S * Hkv, D, fmt).reshape(B, S, Hkv, D)
    sl = np.array(lens, np.int32)
    kc, vc, bt = build_paged_cache(k, v, sl, bs, rng)
    want = kivi.quantize_paged_cache(kc, vc, bt, sl, fmt)
    got = quantize_paged_cache(gpu(kc), gpu(vc), gpu(bt), gpu(sl), fmt)
    torch.cuda.synchronize()
    slots = valid_slots(bt, sl, bs)
    vsl = v_pair_slots(bt, sl, bs)
    for name in ("k_codes", "v_codes"):
        g = getattr(got, name).cpu().numpy()[slots[:, 0], slots[:, 1]]
        w = want[name][slots[:, 0], slots[:, 1]]
        assert np.array_equal(g, w), f"{name}: {np.sum(g != w)} of {g.size} bytes differ"
    lead = lead_blocks(bt, sl, bs)
    for name in ("k_scale", "k_zero"):
        g = getattr(got, name).cpu().numpy()[lead].view(np.uint16)
        assert np.array_equal(g, want[name][lead].view(np.uint16)), name
    for name in ("v_scale", "v_zero"):
        g = getattr(got, name).cpu().numpy()[vsl[:, 0], :, vsl[:, 1]].view(np.uint16)
        w = want[name][vsl[:, 0], :, vsl[:, 1]].view(np.uint16)
        assert np.array_equal(g, w), name


@pytest.mark.parametrize("num_splits", [1, 3, None])
@pytest.mark.parametrize("fmt", FORMATS)
@pytest.mark.parametrize("bs", [16, 32])
def test_decode_matches_fp32_attention_over_dequantized_cache(fmt, bs, num_splits):
    from kvq_decode_amd import paged_decode_attention
    from kvq_decode_amd.quant import quantize_paged_cache
    lens = [1, 37, 300, 2049, 129]
    q, kc, vc, bt, sl = make(lens, bs, seed=1)
    qc = quantize_paged_cache(gpu(kc), gpu(vc), gpu(bt), gpu(sl), fmt)
    host = {n: getattr(qc, n).cpu().numpy() for n in
            ("k_codes", "v_codes", "k_scale", "k_zero", "v_scale", "v_zero")}
    kd, vd = kivi.dequantize_paged_cache(host, bt, sl, fmt)
    ref = paged_decode_attention_ref(q.astype(np.float32), kd, vd, bt, sl, out_dtype=np.float32)
    out = paged_decode_attention(gpu(q), qc.k_codes, qc.v_codes, gpu(bt), gpu(sl),
                                 num_splits=num_splits, **qc.decode_kwargs())
    check_close(out, ref, f"{fmt} bs={bs} splits={num_splits}")


@pytest.mark.parametrize("fmt", FORMATS)
def test_decode_group8_and_mqa_heads(fmt):
    """Other GQA groups over a quantized cache: 1, 2 and 3 q heads per kv head (the
    chunk-pair kernel with padded head columns), 5, 7 (Qwen2.5-7B's 28 / 4) and 8 (chunk
    pairs with hi / lo columns), MQA, and 16 (two chains)."""
    from kvq_decode_amd import paged_decode_attention
    from kvq_decode_amd.quant import quantize_paged_cache
    for Hq, Hkv in ((8, 8), (4, 2), (6, 2), (10, 2), (28, 4), (16, 2), (8, 1), (32, 2)):
        q, kc, vc, bt, sl = make([700, 3], 16, Hq=Hq, Hkv=Hkv, seed=2)
        qc = quantize_paged_cache(gpu(kc), gpu(vc), gpu(bt), gpu(sl), fmt)
        host = {n: getattr(qc, n).cpu().numpy() for n in
                ("k_codes", "v_codes", "k_scale", "k_zero", "v_scale", "v_zero")}
        kd, vd = kivi.dequantize_paged_cache(host, bt, sl, fmt)
        ref = paged_decode_attention_ref(q.astype(np.float32), kd, vd, bt, sl,
                                         out_dtype=np.float32)
        out = paged_decode_attention(gpu(q), qc.k_codes, qc.v_codes, gpu(bt), gpu(sl),
                                     num_splits=2, **qc.decode_kwargs())
        check_close(out, ref, f"{fmt} Hq={Hq} Hkv={Hkv}")


@pytest.mark.parametrize("G", [5, 6, 7, 8])
@pytest.mark.parametrize("fmt", FORMATS)
def test_chunk_pairs_five_to_eight_heads(fmt, G):
    """5 to 8 q heads per kv head run chunk pairs with every column holding both chunks
    (the hi and lo lanes of a head each weight one chunk): a one-token sequence, partial
    last chunks and odd chunk counts (single-chunk steps at both ends of a wave), single
    pass, splits, work units and the default plan; every ring depth and workgroup shape
    within tolerance, and the ring depth never changes a result bit; K groups of 16
    chunks."""
    from kvq_decode_amd import paged_decode_attention
    from kvq_decode_amd.quant import quantize_paged_cache
    Hkv = 2
    q, kc, vc, bt, sl = make([1, 17, 33, 300, 2049], 16, Hq=G * Hkv, Hkv=Hkv, seed=30 + G)
    qc = quantize_paged_cache(gpu(kc), gpu(vc), gpu(bt), gpu(sl), fmt)
    host = {n: getattr(qc, n).cpu().numpy() for n in
            ("k_codes", "v_codes", "k_scale", "k_zero", "v_scale", "v_zero")}
    kd, vd = kivi.dequantize_paged_cache(host, bt, sl, fmt)
    ref = paged_decode_attention_ref(q.astype(np.float32), kd, vd, bt, sl, out_dtype=np.float32)
    args = (gpu(q), qc.k_codes, qc.v_codes, gpu(bt), gpu(sl))
    for extra in ({"num_splits": 1}, {"num_splits": 3}, {"units": 5}, {"units": 7}, {}):
        out = paged_decode_attention(*args, **extra, **qc.decode_kwargs())
        check_close(out, ref, f"{fmt} G={G} {extra}")
    for splits in (1, 5):
        for waves in (1, 2, 4, 8):
            outs = [paged_decode_attention(*args, num_splits=splits, waves_per_group=waves,
                                           pipeline=ring, **qc.decode_kwargs())
                    for ring in (1, 2, 4)]
            check_close(outs[0], ref, f"{fmt} G={G} splits={splits} waves={waves}")
            assert all(torch.equal(outs[0], o) for o in outs[1:]), (fmt, G, splits, waves)
    # K groups of 16 chunks: a group's q'' serves several pair steps
    qc = quantize_paged_cache(gpu(kc), gpu(vc), gpu(bt), gpu(sl), fmt, k_group=256)
    host = {n: getattr(qc, n).cpu().numpy() for n in
            ("k_codes", "v_codes", "k_scale", "k_zero", "v_scale", "v_zero")}
    kd, vd = kivi.dequantize_paged_cache(host, bt, sl, fmt, group=256)
    ref = paged_decode_attention_ref(q.astype(np.float32), kd, vd, bt, sl, out_dtype=np.float32)
    args = (gpu(q), qc.k_codes, qc.v_codes, gpu(bt), gpu(sl))
    for extra in ({"num_splits": 3}, {"units": 7}):
        out = paged_decode_attention(*args, **extra, **qc.decode_kwargs())
        check_close(out, ref, f"{fmt} G={G} k_group=256 {extra}")


@pytest.mark.parametrize("fmt", FORMATS)
def test_code_layout_does_not_change_results(fmt):
    """The quantizer allocates head-major code storage; decode reads codes through their
    strides, so the same codes stored token-major (the fp16 cache's layout) and written
    by the quantizer into a token-major cache give bit-identical outputs."""
    from kvq_decode_amd import paged_decode_attention
    from kvq_decode_amd.quant import allocate_quantized_cache, quantize_paged_cache
    q, kc, vc, bt, sl = make([1, 37, 300, 2049], 16, seed=4)
    qc = quantize_paged_cache(gpu(kc), gpu(vc), gpu(bt), gpu(sl), fmt)
    assert not qc.k_codes.is_contiguous()
    tm = qc._replace(k_codes=qc.k_codes.contiguous(), v_codes=qc.v_codes.contiguous())
    assert tm.k_codes.stride(1) > tm.k_codes.stride(2)
    for splits in (1, None):
        a = paged_decode_attention(gpu(q), qc.k_codes, qc.v_codes, gpu(bt), gpu(sl),
                                   num_splits=splits, **qc.decode_kwargs())
        b = paged_decode_attention(gpu(q), tm.k_codes, tm.v_codes, gpu(bt), gpu(sl),
                                   num_splits=splits, **tm.decode_kwargs())
        assert torch.equal(a, b)
    # the quantizer writes through the destination's strides too
    nb, bs, hkv, _ = kc.shape
    dst = allocate_quantized_cache(nb, bs, hkv, 128, fmt, "cuda", qc.k_group)._replace(
        k_codes=torch.zeros_like(tm.k_codes), v_codes=torch.zeros_like(tm.v_codes))
    quantize_paged_cache(gpu(kc), gpu(vc), gpu(bt), gpu(sl), fmt, out=dst)
    slots = valid_slots(bt, sl, 16)
    vsl = v_pair_slots(bt, sl, 16)
    for name in ("k_codes", "v_codes"):
        g = getattr(dst, name).cpu().numpy()[slots[:, 0], slots[:, 1]]
        w = getattr(qc, name).cpu().numpy()[slots[:, 0], slots[:, 1]]
        assert np.array_equal(g, w), name
    for name in ("v_scale", "v_zero"):
        g = getattr(dst, name).cpu().numpy()[vsl[:, 0], :, vsl[:, 1]].view(np.uint16)
        w = getattr(qc, name).cpu().numpy()[vsl[:, 0], :, vsl[:, 1]].view(np.uint16)
        assert np.array_equal(g, w), name


@pytest.mark.parametrize("fmt", FORMATS)
def test_ring_depths_and_workgroup_shapes(fmt):
    """Every (waves per workgroup, loads in flight) variant is within tolerance, and the
    ring depth never changes a result bit (same arithmetic in the same order)."""
    from kvq_decode_amd import paged_decode_attention
    from kvq_decode_amd.quant import quantize_paged_cache
    q, kc, vc, bt, sl = make([1, 129, 300, 2049, 700], 16, seed=5)
    qc = quantize_paged_cache(gpu(kc), gpu(vc), gpu(bt), gpu(sl), fmt)
    host = {n: getattr(qc, n).cpu().numpy() for n in
            ("k_codes", "v_codes", "k_scale", "k_zero", "v_scale", "v_zero")}
    kd, vd = kivi.dequantize_paged_cache(host, bt, sl, fmt)
    ref = paged_decode_attention_ref(q.astype(np.float32), kd, vd, bt, sl, out_dtype=np.float32)
    for splits in (1, 3):
        by_ring = {}
        for waves in (1, 2, 4, 8):
            for ring in (1, 2, 4):
                out = paged_decode_attention(gpu(q), qc.k_codes, qc.v_codes, gpu(bt), gpu(sl),
                                             num_splits=splits, waves_per_group=waves,
                                             pipeline=ring, **qc.decode_kwargs())
                check_close(out, ref, f"{fmt} splits={splits} waves={waves} ring={ring}")
                by_ring.setdefault(waves, []).append(out)
        for waves, outs in by_ring.items():
            assert all(torch.equal(outs[0], o) for o in outs[1:]), (fmt, splits, waves)


@pytest.mark.parametrize("k_group", [16, 32, 64, 256])
@pytest.mark.parametrize("fmt", FORMATS)
def test_other_k_group_sizes(fmt, k_group):
    """K scale groups of 1, 2, 4 and 16 chunks (the default 128 tokens is 8): quantizer
    bit-exact and decode within tolerance, for every ring depth."""
    from kvq_decode_amd import paged_decode_attention
    from kvq_decode_amd.quant import quantize_paged_cache
    q, kc, vc, bt, sl = make([5, 300, 1000], 16, seed=6)
    qc = quantize_paged_cache(gpu(kc), gpu(vc), gpu(bt), gpu(sl), fmt, k_group=k_group)
    want = kivi.quantize_paged_cache(kc, vc, bt, sl, fmt, group=k_group)
    slots = valid_slots(bt, sl, 16)
    vsl = v_pair_slots(bt, sl, 16)
    for name in ("k_codes", "v_codes"):
        g = getattr(qc, name).cpu().numpy()[slots[:, 0], slots[:, 1]]
        assert np.array_equal(g, want[name][slots[:, 0], slots[:, 1]]), name
    lead = lead_blocks(bt, sl, 16, k_group)
    for name in ("k_scale", "k_zero"):
        g = getattr(qc, name).cpu().numpy()[lead].view(np.uint16)
        assert np.array_equal(g, want[name][lead].view(np.uint16)), name
    for name in ("v_scale", "v_zero"):
        g = getattr(qc, name).cpu().numpy()[vsl[:, 0], :, vsl[:, 1]].view(np.uint16)
        assert np.array_equal(g, want[name][vsl[:, 0], :, vsl[:, 1]].view(np.uint16)), name
    host = {n: getattr(qc, n).cpu().numpy() for n in
            ("k_codes", "v_codes", "k_scale", "k_zero", "v_scale", "v_zero")}
    kd, vd = kivi.dequantize_paged_cache(host, bt, sl, fmt, group=k_group)
    ref = paged_decode_attention_ref(q.astype(np.float32), kd, vd, bt, sl, out_dtype=np.float32)
    for ring in (1, 2, 4):
        out = paged_decode_attention(gpu(q), qc.k_codes, qc.v_codes, gpu(bt), gpu(sl),
                                     num_splits=2, pipeline=ring, **qc.decode_kwargs())
        check_close(out, ref, f"{fmt} k_group={k_group} ring={ring}")


@pytest.mark.parametrize("fmt", FORMATS)
def test_append_equals_bulk(fmt):
    """Bulk-quantize a prefix, then append tokens one by one across group boundaries; the
    cache must equal the bulk quantization of all tokens, bit for bit, and decode on it
    must match."""
    from kvq_decode_amd.quant import init_k_residual, quantize_append, quantize_paged_cache
    bs = 16
    n0 = [100, 1, 127, 250]
    n1 = [140, 40, 131, 260]
    q, kc, vc, bt, sl1 = make(n1, bs, Hkv=2, seed=3)
    Hkv = kc.shape[2]
    kc_g, vc_g, bt_g = gpu(kc), gpu(vc), gpu(bt)
    sl0 = torch.tensor(n0, dtype=torch.int32, device="cuda")
    qc = quantize_paged_cache(kc_g, vc_g, bt_g, sl0, fmt)
    resid = init_k_residual(kc_g, bt_g, sl0)
    cur = list(n0)
    while any(c < e for c, e in zip(cur, n1)):
        nxt = [min(c + 1, e) for c, e in zip(cur, n1)]
        grow = [b for b in range(4) if nxt[b] > cur[b]]
        # sequences that already reached their length re-append their last token (idempotent)
        k_new = torch.empty((4, Hkv, 128), dtype=torch.float16, device="cuda")
        v_new = torch.empty_like(k_new)
        for b in range(4):
            t = nxt[b] - 1
            k_new[b] = kc_g[bt_g[b, t // bs], t % bs]
            v_new[b] = vc_g[bt_g[b, t // bs], t % bs]
        sl = torch.tensor(nxt, dtype=torch.int32, device="cuda")
        quantize_append(qc, k_new, v_new, bt_g, sl, resid)
        cur = nxt
        assert grow
    torch.cuda.synchronize()
    want = quantize_paged_cache(kc_g, vc_g, bt_g, gpu(sl1), fmt)
    torch.cuda.synchronize()
    slots = valid_slots(bt, sl1, bs)
    vsl = v_pair_slots(bt, sl1, bs)
    for name in ("k_codes", "v_codes"):
        g = getattr(qc, name).cpu().numpy()[slots[:, 0], slots[:, 1]]
        w = getattr(want, name).cpu().numpy()[slots[:, 0], slots[:, 1]]
        assert np.array_equal(g, w), name
    lead = lead_blocks(bt, sl1, bs)
    for name in ("k_scale", "k_zero"):
        assert np.array_equal(getattr(qc, name).cpu().numpy()[lead],
                              getattr(want, name).cpu().numpy()[lead]), name
    for name in ("v_scale", "v_zero"):
        g = getattr(qc, name).cpu().numpy()[vsl[:, 0], :, vsl[:, 1]]
        w = getattr(want, name).cpu().numpy()[vsl[:, 0], :, vsl[:, 1]]
        assert np.array_equal(g, w), name


@pytest.mark.parametrize("fmt", ["int8", "fp8_e4m3"])
def test_c4_full_size(fmt):
    """B=16, seq_len 32768, bs 16, 32768-block pool, outlier K. The
    quantizer is checked bit-exact and the decode against the oracle on two sequences
    (the oracle takes seconds per sequence at this size)."""
    _full_size_case(fmt, [32768] * 16, check_seqs=(0, 15))


def test_c5_int4_full_size():
    """INT4, B=64, seq_lens ~ U[1024, 32768] (seed 0), shared pool."""
    lens = np.random.default_rng(0).integers(1024, 32769, 64).tolist()
    _full_size_case("int4", lens, check_seqs=(0, 31, 63))


def _full_size_case(fmt, lens, check_seqs):
    from kvq_decode_amd import paged_decode_attention
    from kvq_decode_amd.quant import quantize_paged_cache
    g = torch.Generator(device="cuda").manual_seed(0)
    B, Hq, Hkv, D, bs = len(lens), 32, 8, 128, 16
    pages = [-(-n // bs) for n in lens]
    pool = sum(pages)
    mb = max(pages)
    q = torch.randn(B, Hq, D, generator=g, device="cuda").half()
    k = torch.randn(pool, bs, Hkv, D, generator=g, device="cuda")
    for h in range(Hkv):
        ch = torch.randperm(D, generator=g, device="cuda")[:4]
        k[:, :, h, ch] *= 10
    k = k.half()
    v = torch.randn(pool, bs, Hkv, D, generator=g, device="cuda").half()
    perm = torch.randperm(pool, generator=g, device="cuda").int()
    bt = torch.zeros(B, mb, dtype=torch.int32, device="cuda")
    o = 0
    for b, n in enumerate(pages):
        bt[b, :n] = perm[o:o + n]
        o += n
    sl = torch.tensor(lens, dtype=torch.int32, device="cuda")
    qc = quantize_paged_cache(k, v, bt, sl, fmt)
    out = paged_decode_attention(q, qc.k_codes, qc.v_codes, bt, sl, **qc.decode_kwargs())
    torch.cuda.synchronize()
    btn, sln = bt.cpu().numpy(), sl.cpu().numpy()
    for b in check_seqs:
        blocks = btn[b, :pages[b]].astype(np.int64)
        sub_bt = np.arange(pages[b], dtype=np.int32)[None]
        sub_sl = sln[b:b + 1]
        kc, vc = k[blocks].cpu().numpy(), v[blocks].cpu().numpy()
        want = kivi.quantize_paged_cache(kc, vc, sub_bt, sub_sl, fmt)
        host = {n: getattr(qc, n)[blocks].cpu().numpy() for n in
                ("k_codes", "v_codes", "k_scale", "k_zero", "v_scale", "v_zero")}
        n = int(sub_sl[0])
        flat = lambda a: a.reshape(-1, *a.shape[2:])[:n]  # noqa: E731
        assert np.array_equal(flat(host["k_codes"]), flat(want["k_codes"]))
        assert np.array_equal(flat(host["v_codes"]), flat(want["v_codes"]))
        kd, vd = kivi.dequantize_paged_cache(host, sub_bt, sub_sl, fmt)
        ref = paged_decode_attention_ref(q[b:b + 1].cpu().numpy().astype(np.float32), kd, vd,
                                         sub_bt, sub_sl, out_dtype=np.float32)
        check_close(out[b:b + 1], ref, f"{fmt} full-size seq {b} len {n}")


def _dequant_int4_torch(qc, bt, b, L, h, bs, group=128):
    """float32 K, V [L, D] of kv head h of sequence b from an INT4 cache (x = c s + z;
    low nibble = even channel; K pairs in the K group's first block, V pairs at index
    t % VG of the V group's first block, VG = max(bs, 32))."""
    pages = bt[b, :-(-L // bs)].long()

    def codes(c):
        c = c[pages, :, h].reshape(-1, c.shape[-1])[:L]
        return torch.stack([c & 15, c >> 4], dim=-1).reshape(L, -1).float()
    t = torch.arange(L, device=bt.device)
    lead = bt[b, (t // group) * group // bs].long()
    ksz = qc.k_sz[lead, h].float()                       # [L, D, 2]
    k = codes(qc.k_codes) * ksz[..., 0] + ksz[..., 1]
    vg = max(bs, 32)
    vlead = bt[b, (t // vg) * vg // bs].long()
    vsz = qc.v_sz[vlead, h, t % vg].float()              # [L, 2]
    v = codes(qc.v_codes) * vsz[:, :1] + vsz[:, 1:]
    return k, v


def test_int4_maximum_context():
    """INT4 past a million tokens: two sequences of 70000 pages (1,120,000 tokens and 37
    fewer; more than the 65535 16-token chunks a 16-bit grid axis would allow the
    quantizers) on disjoint blocks of a 140016-block pool, needle keys at the last token and
    mid-sequence: the default plan (work units), 64 splits and the single pass against
    float32 attention over the dequantized cache."""
    from kvq_decode_amd import paged_decode_attention
    from kvq_decode_amd.quant import quantize_paged_cache
    g = torch.Generator(device="cuda").manual_seed(6)
    Hq, Hkv, D, bs, pool, pages = 32, 8, 128, 16, 140016, 70000
    lens = [pages * bs, pages * bs - 37]
    print(f"\n[int4 max context] lens={lens}", flush=True)
    k = torch.randn(pool, bs, Hkv, D, generator=g, device="cuda").half()
    v = torch.randn(pool, bs, Hkv, D, generator=g, device="cuda").half()
    q = torch.randn(2, Hq, D, generator=g, device="cuda").half()
    # disjoint tables: a block shared by both sequences would hold the K pairs of only one
    # of the two groups it leads
    bt = torch.randperm(pool, generator=g, device="cuda")[:2 * pages].view(2, pages).int()
    scale = 1.0 / np.sqrt(D)
    needles = {}
    for b, L in enumerate(lens):
        for h in range(Hkv):
            t = L - 1 if h % 2 == 0 else L // 2 + 11 * h
            qv = q[b, 4 * h].float()
            k[bt[b, t // bs].long(), t % bs, h] = (qv * (30.0 / scale / float(qv @ qv))).half()
            needles[(b, h)] = t
    sl = torch.tensor(lens, dtype=torch.int32, device="cuda")
    qc = quantize_paged_cache(k, v, bt, sl, "int4")
    del k, v
    ref = torch.empty(2, Hq, D, dtype=torch.float32, device="cuda")
    vneedle = {}
    for b, L in enumerate(lens):
        for h in range(Hkv):
            kd, vd = _dequant_int4_torch(qc, bt, b, L, h, bs)
            p = torch.softmax((q[b, 4 * h:4 * h + 4].float() @ kd.T) * scale, dim=1)
            ref[b, 4 * h:4 * h + 4] = p @ vd
            vneedle[(b, h)] = vd[needles[(b, h)]].clone()
            del kd, vd, p
    for kw in ({}, {"num_splits": 64}, {"num_splits": 1}):
        out = paged_decode_attention(q, qc.k_codes, qc.v_codes, bt, sl, **kw,
                                     **qc.decode_kwargs()).float()
        torch.cuda.synchronize()
        diff = (out - ref).abs()
        print(f"[int4 max context {kw}] max_abs={diff.max().item():.3e}", flush=True)
        assert torch.isfinite(out).all()
        assert diff.max().item() < ATOL
        assert bool((diff <= ATOL + RTOL * ref.abs()).all())
        for (b, h), want in vneedle.items():
            assert (out[b, 4 * h] - want).abs().max().item() < 2e-2, (kw, b, h)


@pytest.mark.parametrize("kw", [{"num_splits": 3}, {"units": 7}, {}],
                         ids=["splits3", "units7", "default"])
@pytest.mark.parametrize("fmt", FORMATS)
def test_nan_garbage_in_unused_quantized_slots(fmt, kw):
    """Slots past each sequence's end in its last page hold 0xFF codes and NaN (scale,
    zero) pairs: the decode never lets them into the result (masked scores, zero weights)."""
    from kvq_decode_amd import paged_decode_attention
    from kvq_decode_amd.quant import quantize_paged_cache
    lens = [37, 1, 250, 129]
    q, kc, vc, bt, sl = make(lens, 16, seed=23)
    qc = quantize_paged_cache(gpu(kc), gpu(vc), gpu(bt), gpu(sl), fmt)
    host = {n: getattr(qc, n).cpu().numpy() for n in
            ("k_codes", "v_codes", "k_scale", "k_zero", "v_scale", "v_zero")}
    kd, vd = kivi.dequantize_paged_cache(host, bt, sl, fmt)
    ref = paged_decode_attention_ref(q.astype(np.float32), kd, vd, bt, sl, out_dtype=np.float32)
    nan16 = torch.tensor(float("nan"), dtype=torch.float16)
    vg = 32  # tokens per V (scale, zero) group at block_size 16
    for b, n in enumerate(lens):
        if n % 16:
            blk = int(bt[b, (n - 1) // 16])
            qc.k_codes[blk, n % 16:] = 0xFF
            qc.v_codes[blk, n % 16:] = 0xFF
        if n % vg:  # the pairs past the end of the sequence's last V group
            vlead = int(bt[b, ((n - 1) // vg) * vg // 16])
            qc.v_sz[vlead, :, n % vg:] = nan16
    out = paged_decode_attention(gpu(q), qc.k_codes, qc.v_codes, gpu(bt), gpu(sl), **kw,
                                 **qc.decode_kwargs())
    torch.cuda.synchronize()
    check_close(out, ref, f"{fmt} nan-garbage {kw}")


@pytest.mark.parametrize("fmt", FORMATS)
def test_append_skips_empty_sequences(fmt):
    """One append launch over a batch holding an empty sequence (seq_len 0): the other
    sequences' new tokens land bit-exact with the bulk quantization, and no byte of the
    cache outside their new slots and K groups changes."""
    from kvq_decode_amd.quant import init_k_residual, quantize_append, quantize_paged_cache
    bs, n0, n1 = 16, [20, 0, 127], [21, 0, 128]
    q, kc, vc, bt, sl1 = make(n1, bs, Hkv=2, seed=29)
    kc_g, vc_g, bt_g = gpu(kc), gpu(vc), gpu(bt)
    sl0 = torch.tensor(n0, dtype=torch.int32, device="cuda")
    qc = quantize_paged_cache(kc_g, vc_g, bt_g, sl0, fmt)
    resid = init_k_residual(kc_g, bt_g, sl0)
    names = ("k_codes", "v_codes", "k_scale", "k_zero", "v_scale", "v_zero")
    before = {n: getattr(qc, n).clone() for n in names}
    k_new = torch.zeros((3, kc.shape[2], kc.shape[3]), dtype=torch.float16, device="cuda")
    v_new = torch.zeros_like(k_new)
    for b in (0, 2):
        t = n1[b] - 1
        k_new[b] = kc_g[bt_g[b, t // bs], t % bs]
        v_new[b] = vc_g[bt_g[b, t // bs], t % bs]
    quantize_append(qc, k_new, v_new, bt_g, gpu(sl1), resid)
    want = quantize_paged_cache(kc_g, vc_g, bt_g, gpu(sl1), fmt)
    torch.cuda.synchronize()
    slots = valid_slots(bt, sl1, bs)
    vsl = v_pair_slots(bt, sl1, bs)
    for name in ("k_codes", "v_codes"):
        g = getattr(qc, name).cpu().numpy()
        assert np.array_equal(g[slots[:, 0], slots[:, 1]],
                              getattr(want, name).cpu().numpy()[slots[:, 0], slots[:, 1]]), name
        # everything except the valid slots is as before the append
        mask = np.ones(g.shape[:2], bool)
        mask[slots[:, 0], slots[:, 1]] = False
        assert np.array_equal(g[mask], before[name].cpu().numpy()[mask]), name
    lead = lead_blocks(bt, sl1, bs)
    bits = lambda t: t.view(torch.int16).cpu().numpy()  # unwritten memory may hold NaNs
    for name in ("k_scale", "k_zero"):
        g = bits(getattr(qc, name))
        assert np.array_equal(g[lead], bits(getattr(want, name))[lead]), name
        mask = np.ones(g.shape[0], bool)
        mask[lead] = False
        assert np.array_equal(g[mask], bits(before[name])[mask]), name
    for name in ("v_scale", "v_zero"):
        g = bits(getattr(qc, name))
        assert np.array_equal(g[vsl[:, 0], :, vsl[:, 1]],
                              bits(getattr(want, name))[vsl[:, 0], :, vsl[:, 1]]), name
        mask = np.ones((g.shape[0], g.shape[2]), bool)  # [block, index]
        mask[vsl[:, 0], vsl[:, 1]] = False
        assert np.array_equal(g.transpose(0, 2, 1)[mask], bits(before[name]).transpose(0, 2, 1)[mask]), name
