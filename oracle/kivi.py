"""KIVI-style KV quantizer specification in numpy. TEST INFRASTRUCTURE.

The reference plans quantized KV (README.md:7, :16 "not started") and fixes only its byte
model (src/bpt/roofline.py:6-9, :22-31): asymmetric fp16 scale + zero, keys per channel
over groups of `group_size` tokens, values per token. There is no reference code, so this
module IS the spec the HIP kernels must match bit for bit. With no reference output to
compare against, it is pinned by the mathematics of the spec: hand-computed vectors and
invariants in tests/test_oracle_kivi.py and, for FP8, the library routine
torch.float8_e4m3fn.

Spec (all arithmetic IEEE float32, round-to-nearest-even, in this exact order):
  integer formats, b in {8, 4}, R = 2**b - 1, over a set X of fp16 values:
      s = fp16((max X - min X) / R)          z = fp16(min X)  (exact: min X is fp16)
      code(x) = 0                              if s == 0
              = clamp(rint((x - z) / s), 0, R) otherwise        (rint: half to even)
      dequant(c) = c * s + z
  fp8_e4m3 (OCP e4m3fn: bias 7, max 448, no infinities), E = 448:
      z = fp16((max X + min X) * 0.5)        s = fp16((max X - min X) / (2 * E))
      code(x) = 0x00                           if s == 0
              = e4m3fn_rne(clamp((x - z) / s, -E, E)) otherwise
      dequant(c) = f32(c) * s + z
  K: X = one channel of one kv head over the tokens of one group [g*G, (g+1)*G) that
     exist (a sequence's last group may be partial).
  V: X = the D channels of one kv head of one token.
  INT4 packing: byte j of a row holds code 2j in bits 0-3 and code 2j+1 in bits 4-7.
Paged storage (this build's format, layout of the codes follows the fp16 cache):
  codes     [num_blocks, block_size, Hkv, D]      uint8 (int8 / fp8 bit patterns)
            [num_blocks, block_size, Hkv, D // 2] uint8 (int4, packed)
  k_scale, k_zero  [num_blocks, Hkv, D] fp16: the scales of group g of sequence b are
            stored in physical block block_table[b, g * G // block_size] (the block that
            holds the group's first token); other blocks' entries are unused.
  v_scale, v_zero  [num_blocks, Hkv, VG] fp16, VG = max(block_size, 32) (v_group): the
            pairs of tokens [j*VG, (j+1)*VG) of sequence b are stored in physical block
            block_table[b, j*VG // block_size] (the block that holds the V group's first
            token), token t at index t % VG; other blocks' entries are unused.
"""

import numpy as np

F32 = np.float32
F16 = np.float16

FORMATS = ("int8", "fp8_e4m3", "int4")
FP8_MAX = 448.0
DEFAULT_GROUP = 128          # reference src/bpt/roofline.py:50 (group_size default)


def v_group(block_size):
    """Tokens per V (scale, zero) group: max(block_size, 32)."""
    return max(block_size, 32)


def _bits(fmt):
    return {"int8": 8, "int4": 4}[fmt]


# ------------------------------------------------------------------ scalar spec pieces

def int_params(mn, mx, bits):
    """(scale, zero) in fp16 from fp16 min/max arrays."""
    r = F32(2 ** bits - 1)
    s = ((np.asarray(mx, F16).astype(F32) - np.asarray(mn, F16).astype(F32)) / r).astype(F16)
    z = np.asarray(mn, F16).copy()
    return s, z


def int_codes(x, s, z, bits):
    """Codes for fp16 values x with broadcastable fp16 s, z."""
    r = F32(2 ** bits - 1)
    s32 = np.asarray(s, F16).astype(F32)
    with np.errstate(divide="ignore", invalid="ignore"):
        t = (np.asarray(x, F16).astype(F32) - np.asarray(z, F16).astype(F32)) / s32
        c = np.clip(np.rint(t), F32(0), r)
    c = np.where(s32 == 0, F32(0), c)
    return c.astype(np.uint8)


def fp8_params(mn, mx):
    mn32 = np.asarray(mn, F16).astype(F32)
    mx32 = np.asarray(mx, F16).astype(F32)
    z = ((mx32 + mn32) * F32(0.5)).astype(F16)
    s = ((mx32 - mn32) / F32(2.0 * FP8_MAX)).astype(F16)
    return s, z


def f32_to_e4m3fn_bits(t):
    """float32 -> OCP e4m3fn bit pattern, round to nearest even. Inputs must already be
    clamped to [-448, 448] (the quantizer does so); values outside raise."""
    t = np.asarray(t, F32)
    a = np.abs(t).astype(np.float64)
    if np.any(a > FP8_MAX) or np.any(np.isnan(a)):
        raise ValueError("e4m3fn conversion needs |t| <= 448 and no NaN")
    sign = np.signbit(t).astype(np.uint8) << 7
    bits = np.zeros(t.shape, np.int64)
    sub = a < 2.0 ** -6
    # subnormals (and zero): value = m * 2^-9, m in [0, 8]; m == 8 carries into exponent 1
    bits = np.where(sub, np.rint(a * 2.0 ** 9).astype(np.int64), bits)
    # normals: value = (1 + m/8) * 2^e, biased exponent e + 7
    with np.errstate(divide="ignore"):
        _, e2 = np.frexp(np.where(sub, 1.0, a))
    e = e2.astype(np.int64) - 1
    m = np.rint((np.where(sub, 1.0, a) / np.ldexp(1.0, e) - 1.0) * 8.0).astype(np.int64)
    carry = m == 8
    e = np.where(carry, e + 1, e)
    m = np.where(carry, 0, m)
    nbits = ((e + 7) << 3) | m
    bits = np.where(sub, bits, nbits)
    return (bits.astype(np.uint8) | sign).astype(np.uint8)


def e4m3fn_bits_to_f32(b):
    b = np.asarray(b, np.uint8).astype(np.int64)
    s = np.where(b & 0x80, -1.0, 1.0)
    e = (b >> 3) & 0xF
    m = b & 7
    val = np.where(e == 0, m * 2.0 ** -9, (1.0 + m / 8.0) * np.ldexp(1.0, e - 7))
    val = np.where((b & 0x7F) == 0x7F, np.nan, val)
    return (s * val).astype(F32)


def fp8_codes(x, s, z):
    s32 = np.asarray(s, F16).astype(F32)
    with np.errstate(divide="ignore", invalid="ignore"):
        t = (np.asarray(x, F16).astype(F32) - np.asarray(z, F16).astype(F32)) / s32
        t = np.clip(t, F32(-FP8_MAX), F32(FP8_MAX))
    t = np.where(s32 == 0, F32(0), t)
    return f32_to_e4m3fn_bits(t)


def codes_to_f32(codes, fmt):
    """Unpacked codes (uint8) -> float32 code values."""
    if fmt == "fp8_e4m3":
        return e4m3fn_bits_to_f32(codes)
    return np.asarray(codes, np.uint8).astype(F32)


def dequant(codes, s, z, fmt):
    """c * s + z in float32 (two roundings: multiply, then add)."""
    c = codes_to_f32(codes, fmt)
    return c * np.asarray(s, F16).astype(F32) + np.asarray(z, F16).astype(F32)


def pack_int4(codes):
    c = np.asarray(codes, np.uint8)
    assert c.shape[-1] % 2 == 0
    return (c[..., 0::2] & 0xF) | ((c[..., 1::2] & 0xF) << 4)


def unpack_int4(packed):
    p = np.asarray(packed, np.uint8)
    out = np.empty(p.shape[:-1] + (p.shape[-1] * 2,), np.uint8)
    out[..., 0::2] = p & 0xF
    out[..., 1::2] = p >> 4
    return out


def params(mn, mx, fmt):
    return fp8_params(mn, mx) if fmt == "fp8_e4m3" else int_params(mn, mx, _bits(fmt))


def codes(x, s, z, fmt):
    return fp8_codes(x, s, z) if fmt == "fp8_e4m3" else int_codes(x, s, z, _bits(fmt))


# ------------------------------------------------------------------ one sequence

def quantize_k_seq(k, fmt, group=DEFAULT_GROUP):
    """k [n, Hkv, D] fp16 -> (codes [n, Hkv, D] uint8 unpacked, scale [ng, Hkv, D],
    zero [ng, Hkv, D]) with per-channel parameters over each group of `group` tokens."""
    n, hkv, d = k.shape
    ng = -(-n // group)
    codes_ = np.empty((n, hkv, d), np.uint8)
    sc = np.empty((ng, hkv, d), F16)
    ze = np.empty((ng, hkv, d), F16)
    for g in range(ng):
        x = k[g * group:(g + 1) * group]
        s, z = params(x.min(axis=0), x.max(axis=0), fmt)
        sc[g], ze[g] = s, z
        codes_[g * group:(g + 1) * group] = codes(x, s[None], z[None], fmt)
    return codes_, sc, ze


def quantize_v_seq(v, fmt):
    """v [n, Hkv, D] fp16 -> (codes [n, Hkv, D], scale [n, Hkv], zero [n, Hkv])."""
    s, z = params(v.min(axis=-1), v.max(axis=-1), fmt)
    return codes(v, s[..., None], z[..., None], fmt), s, z


# ------------------------------------------------------------------ paged caches

def quantize_paged_cache(k_cache, v_cache, block_table, seq_lens, fmt, group=DEFAULT_GROUP,
                         rng=None):
    """Quantize the valid tokens of fp16 paged caches into this build's paged format.

    Returns dict(k_codes, v_codes, k_scale, k_zero, v_scale, v_zero). Slots and scale
    entries no sequence owns keep random bytes (from `rng`) so masking bugs show up."""
    nb, bs, hkv, d = k_cache.shape
    assert group % bs == 0, "a K scale group must span whole pages"
    rng = rng if rng is not None else np.random.default_rng(1234)
    dc = d // 2 if fmt == "int4" else d
    kc = rng.integers(0, 256, (nb, bs, hkv, dc), dtype=np.uint8)
    vc = rng.integers(0, 256, (nb, bs, hkv, dc), dtype=np.uint8)
    garbage = lambda shape: (rng.standard_normal(shape) * 100).astype(F16)  # noqa: E731
    vg = v_group(bs)
    ks, kz = garbage((nb, hkv, d)), garbage((nb, hkv, d))
    vs, vz = garbage((nb, hkv, vg)), garbage((nb, hkv, vg))
    for b in range(len(seq_lens)):
        n = int(seq_lens[b])
        npg = -(-n // bs)
        blocks = np.asarray(block_table[b, :npg], np.int64)
        k = k_cache[blocks].reshape(-1, hkv, d)[:n]
        v = v_cache[blocks].reshape(-1, hkv, d)[:n]
        kq, ksc, kze = quantize_k_seq(k, fmt, group)
        vq, vsc, vze = quantize_v_seq(v, fmt)
        if fmt == "int4":
            kq, vq = pack_int4(kq), pack_int4(vq)
        for i in range(npg):
            lo, hi = i * bs, min((i + 1) * bs, n)
            phys = blocks[i]
            kc[phys, :hi - lo] = kq[lo:hi]
            vc[phys, :hi - lo] = vq[lo:hi]
        for j in range(-(-n // vg)):
            lo, hi = j * vg, min((j + 1) * vg, n)
            lead = blocks[lo // bs]
            vs[lead, :, :hi - lo] = vsc[lo:hi].T
            vz[lead, :, :hi - lo] = vze[lo:hi].T
        for g in range(ksc.shape[0]):
            phys = blocks[g * group // bs]
            ks[phys], kz[phys] = ksc[g], kze[g]
    return dict(k_codes=kc, v_codes=vc, k_scale=ks, k_zero=kz, v_scale=vs, v_zero=vz)


def dequantize_paged_cache(qc, block_table, seq_lens, fmt, group=DEFAULT_GROUP):
    """Float32 paged caches holding c * s + z for every valid token slot (0 elsewhere)."""
    kc, vc = qc["k_codes"], qc["v_codes"]
    nb, bs, hkv, dc = kc.shape
    d = dc * 2 if fmt == "int4" else dc
    vg = v_group(bs)
    kd = np.zeros((nb, bs, hkv, d), F32)
    vd = np.zeros((nb, bs, hkv, d), F32)
    for b in range(len(seq_lens)):
        n = int(seq_lens[b])
        for i in range(-(-n // bs)):
            phys = int(block_table[b, i])
            cnt = min(bs, n - i * bs)
            gphys = int(block_table[b, (i * bs // group) * group // bs])
            kcode, vcode = kc[phys, :cnt], vc[phys, :cnt]
            if fmt == "int4":
                kcode, vcode = unpack_int4(kcode), unpack_int4(vcode)
            kd[phys, :cnt] = dequant(kcode, qc["k_scale"][gphys][None], qc["k_zero"][gphys][None], fmt)
            t0 = i * bs  # the page's first token; its V group starts at a multiple of vg
            vlead = int(block_table[b, (t0 // vg) * vg // bs])
            off = t0 % vg
            vs = qc["v_scale"][vlead, :, off:off + cnt].T[..., None]
            vz = qc["v_zero"][vlead, :, off:off + cnt].T[..., None]
            vd[phys, :cnt] = dequant(vcode, vs, vz, fmt)
    return kd, vd
