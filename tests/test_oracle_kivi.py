"""Pins the KIVI quantizer spec (oracle/kivi.py). The reference has no quantizer code
(README.md:16), so there is no reference parity to check; these tests pin the spec with
hand-computed vectors, invariants and, for FP8, torch.float8_e4m3fn. CPU only."""
import numpy as np
import pytest
import torch

from oracle import kivi
from oracle.attention import build_paged_cache


def test_int4_hand_vector():
    # channel [0, 1, 2, 3]: s = fp16(3/15) = fp16(0.2) = 1638 * 2^-13, z = 0
    x = np.array([0, 1, 2, 3], np.float16)
    s, z = kivi.int_params(x.min(), x.max(), 4)
    assert float(s) == 1638 * 2.0 ** -13 == 0.199951171875 and float(z) == 0.0
    # 1/s = 5.0012, 2/s = 10.0024, 3/s = 15.0037 -> clamped to 15
    assert kivi.int_codes(x, s, z, 4).tolist() == [0, 5, 10, 15]


def test_int8_hand_vector():
    # s = fp16(3/255): 3/255 = 1.50588 * 2^-7, mantissa 1542/1024 -> 1542 * 2^-17
    x = np.array([0, 1, 2, 3], np.float16)
    s, z = kivi.int_params(x.min(), x.max(), 8)
    assert float(s) == 1542 * 2.0 ** -17
    assert kivi.int_codes(x, s, z, 8).tolist() == [0, 85, 170, 255]


def test_round_half_to_even():
    # range 15 -> s = 1 exactly for int4; 2.5 -> 2, 3.5 -> 4, 4.5 -> 4 (ties to even)
    x = np.array([0, 2.5, 3.5, 4.5, 15], np.float16)
    s, z = kivi.int_params(x.min(), x.max(), 4)
    assert float(s) == 1.0
    assert kivi.int_codes(x, s, z, 4).tolist() == [0, 2, 4, 4, 15]


def test_negative_offset_and_constant_channel():
    x = np.array([-3, -1, 0, 12], np.float16)         # s = 1, z = -3
    s, z = kivi.int_params(x.min(), x.max(), 4)
    assert (float(s), float(z)) == (1.0, -3.0)
    assert kivi.int_codes(x, s, z, 4).tolist() == [0, 2, 3, 15]
    c = np.full(5, 0.7, np.float16)                    # max == min -> s = 0 -> all codes 0
    s, z = kivi.int_params(c.min(), c.max(), 8)
    assert float(s) == 0.0 and kivi.int_codes(c, s, z, 8).tolist() == [0] * 5
    assert np.all(kivi.dequant(np.zeros(5, np.uint8), s, z, "int8") == np.float32(c[0]))


def test_fp8_hand_vector():
    # [-1, 1]: z = 0, s = fp16(2/896); +-1 -> +-448 = 0x7E / 0xFE
    x = np.array([-1, 0, 1], np.float16)
    s, z = kivi.fp8_params(x.min(), x.max())
    assert float(z) == 0.0 and float(s) == float(np.float16(np.float32(2) / np.float32(896)))
    codes = kivi.fp8_codes(x, s, z)
    assert codes.tolist() == [0xFE, 0x00, 0x7E]


def test_e4m3fn_matches_torch_on_every_code_and_midpoints():
    """Our bit conversion vs torch.float8_e4m3fn: all 254 finite codes decode alike, and
    every value and every midpoint between neighbours (ties) encodes alike."""
    codes = np.array([c for c in range(256) if (c & 0x7F) != 0x7F], np.uint8)
    ours = kivi.e4m3fn_bits_to_f32(codes)
    theirs = torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy()
    np.testing.assert_array_equal(ours, theirs)
    pos = np.unique(ours[ours >= 0])
    mids = (pos[:-1].astype(np.float64) + pos[1:]) / 2
    probe = np.concatenate([pos, mids, -pos, -mids, pos * 0.999, pos * 1.001]).astype(np.float32)
    probe = np.clip(probe, -448, 448)
    want = torch.from_numpy(probe).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    np.testing.assert_array_equal(kivi.f32_to_e4m3fn_bits(probe), want)


def test_e4m3fn_random_values_match_torch():
    rng = np.random.default_rng(0)
    t = np.concatenate([rng.uniform(-448, 448, 20000),
                        rng.standard_normal(20000) * 0.02,
                        rng.standard_normal(20000) * 2e-3]).astype(np.float32)
    want = torch.from_numpy(t).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    np.testing.assert_array_equal(kivi.f32_to_e4m3fn_bits(t), want)


def test_pack_unpack_and_nibble_order():
    assert kivi.pack_int4(np.array([1, 2, 15, 0], np.uint8)).tolist() == [0x21, 0x0F]
    c = np.random.default_rng(1).integers(0, 16, (7, 3, 128)).astype(np.uint8)
    np.testing.assert_array_equal(kivi.unpack_int4(kivi.pack_int4(c)), c)


@pytest.mark.parametrize("fmt", kivi.FORMATS)
def test_invariants_on_random_data(fmt):
    """Codes in range, extremes map to the range ends (int), and |x - dequant| <= s/2 plus
    the fp16 rounding of s and z (int) or the e4m3 half-ulp (fp8)."""
    rng = np.random.default_rng(2)
    x = (rng.standard_normal((64, 128)) * rng.uniform(0.01, 20, (1, 128))).astype(np.float16)
    s, z = kivi.params(x.min(axis=0), x.max(axis=0), fmt)
    c = kivi.codes(x, s[None], z[None], fmt)
    deq = kivi.dequant(c, s[None], z[None], fmt)
    err = np.abs(deq - x.astype(np.float32))
    s32 = s.astype(np.float32)[None]
    if fmt == "fp8_e4m3":
        # relative precision 2^-4 of |(x - z)/s| (<= 448) plus the subnormal step 2^-10
        t = np.abs((x.astype(np.float32) - z.astype(np.float32)[None]) / s32)
        assert np.all(err <= (t * 2.0 ** -4 + 2.0 ** -10) * s32 * 1.01 + 1e-6)
    else:
        R = 255 if fmt == "int8" else 15
        assert c.max() <= R
        assert np.all(c[x.argmin(axis=0), np.arange(128)] == 0)
        assert np.all(c[x.argmax(axis=0), np.arange(128)] == R)
        # half a step plus what fp16-rounding s moves the top of the range by
        assert np.all(err <= s32 / 2 + R * s32 * 2.0 ** -11 + 1e-3 * s32)


@pytest.mark.parametrize("fmt", kivi.FORMATS)
@pytest.mark.parametrize("bs", [16, 32, 64])
def test_paged_quantization_round_trip(fmt, bs):
    """quantize_paged_cache stores what the per-sequence quantizers compute, and
    dequantize_paged_cache reads it back through the block table (group-leading block).
    The V pairs sit where include/kvq.h puts them: token t at index t % VG of the block
    holding its V group's first token, VG = max(block_size, 32)."""
    rng = np.random.default_rng(3)
    lens = [5, 128, 129, 300]
    k = rng.standard_normal((4, 300, 2, 128)).astype(np.float16)
    v = rng.standard_normal((4, 300, 2, 128)).astype(np.float16)
    sl = np.array(lens, np.int32)
    kc, vc, bt = build_paged_cache(k, v, sl, bs, rng)
    qc = kivi.quantize_paged_cache(kc, vc, bt, sl, fmt)
    kd, vd = kivi.dequantize_paged_cache(qc, bt, sl, fmt)
    for b, n in enumerate(lens):
        kq, ks, kz = kivi.quantize_k_seq(k[b, :n], fmt)
        vq, vs, vz = kivi.quantize_v_seq(v[b, :n], fmt)
        want_k = kivi.dequant(kq, np.repeat(ks, 128, axis=0)[:n], np.repeat(kz, 128, axis=0)[:n], fmt)
        want_v = kivi.dequant(vq, vs[..., None], vz[..., None], fmt)
        vg = max(bs, 32)
        for t in range(n):
            np.testing.assert_array_equal(kd[bt[b, t // bs], t % bs], want_k[t])
            np.testing.assert_array_equal(vd[bt[b, t // bs], t % bs], want_v[t])
            lead = bt[b, (t // vg) * vg // bs]
            assert np.array_equal(qc["v_scale"][lead, :, t % vg].view(np.uint16), vs[t].view(np.uint16))
            assert np.array_equal(qc["v_zero"][lead, :, t % vg].view(np.uint16), vz[t].view(np.uint16))


def test_shared_lead_block_collides():
    """The hazard include/kvq.h states for quantized caches: a V group's (scale, zero)
    pairs (32 tokens with 16-token pages) and a K group's are stored in the group's lead
    block, also for the tokens of its other blocks. Two sequences that share page 0 but
    not page 1 (a prefix fork) therefore overwrite each other's pairs, and the first one
    no longer dequantizes to what it was quantized from; copying the shared page (so each
    sequence owns its lead block) removes the collision."""
    rng = np.random.default_rng(5)
    bs, hkv, d = 16, 2, 64
    k = rng.standard_normal((4, bs, hkv, d)).astype(np.float16)
    v = rng.standard_normal((4, bs, hkv, d)).astype(np.float16)
    k[3], v[3] = k[0], v[0]  # page 3: a copy of the shared page 0
    lens = np.array([32, 32], np.int32)
    alone = kivi.quantize_paged_cache(k, v, np.array([[0, 1]], np.int32), lens[:1], "int8")
    want_k, want_v = kivi.dequantize_paged_cache(alone, np.array([[0, 1]], np.int32),
                                                 lens[:1], "int8")
    for table, collide in (([[0, 1], [0, 2]], True), ([[0, 1], [3, 2]], False)):
        bt = np.array(table, np.int32)
        qc = kivi.quantize_paged_cache(k, v, bt, lens, "int8")
        got_k, got_v = kivi.dequantize_paged_cache(qc, bt, lens, "int8")
        same = (np.array_equal(got_k[[0, 1]], want_k[[0, 1]]) and
                np.array_equal(got_v[[0, 1]], want_v[[0, 1]]))
        assert same != collide, table
