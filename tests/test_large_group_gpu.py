"""More than 16 q heads per kv head (MQA and wide GQA groups). Needs a GPU.

The reference's kernel takes any group (triton_fp16.py:196 asserts only Hq % Hkv == 0).
The kernels here serve at most 16 q heads per kv head in one MFMA column block, so the
library cuts a group G > 16 into k blocks of G / k heads (kvq_head_blocks: 32 -> 2 x 16,
24 -> 2 x 12, 20 -> 2 x 10, 71 -> 71 x 1) that each read the same cache head. Every path
(single pass, splits, the default plan) must match the oracle within the north-star
tolerance: fp16 against the paged fp32 reference, quantized formats against fp32
attention over the dequantized cache.
"""
import numpy as np
import pytest
import torch

from oracle import kivi
from oracle.attention import build_paged_cache, paged_decode_attention_ref

pytestmark = pytest.mark.gpu

ATOL, RTOL = 2e-3, 1e-2
LENS = [1, 37, 300, 1000]


def make(Hq, Hkv, D, lens, seed, bs=16):
    rng = np.random.default_rng(seed)
    B, S = len(lens), max(lens)
    q = rng.standard_normal((B, Hq, D)).astype(np.float16)
    k = rng.standard_normal((B, S, Hkv, D)).astype(np.float16)
    v = rng.standard_normal((B, S, Hkv, D)).astype(np.float16)
    sl = np.array(lens, np.int32)
    kc, vc, bt = build_paged_cache(k, v, sl, bs, rng)
    return q, kc, vc, bt, sl


def gpu(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def check_close(out, ref, tag):
    out = out.float().cpu().numpy()
    diff = np.abs(out - ref)
    print(f"\n[{tag}] max_abs={diff.max():.3e}", flush=True)
    assert np.isfinite(out).all()
    assert diff.max() < ATOL
    assert np.all(diff <= ATOL + RTOL * np.abs(ref))


@pytest.mark.parametrize("Hq,Hkv,D", [(32, 1, 128), (48, 2, 64), (40, 2, 128), (71, 1, 64),
                                      (64, 2, 256)])
def test_fp16_large_groups(Hq, Hkv, D):
    from kvq_decode_amd import head_blocks, paged_decode_attention
    assert head_blocks(Hq, Hkv) > 1
    q, kc, vc, bt, sl = make(Hq, Hkv, D, LENS, seed=Hq + D)
    ref = paged_decode_attention_ref(q, kc, vc, bt, sl, out_dtype=np.float32)
    args = [gpu(a) for a in (q, kc, vc, bt, sl)]
    for splits in (1, 3, None):
        out = paged_decode_attention(*args, num_splits=splits)
        torch.cuda.synchronize()
        check_close(out, ref, f"fp16 Hq={Hq} Hkv={Hkv} D={D} splits={splits}")
    out = paged_decode_attention(*args, units=5)
    torch.cuda.synchronize()
    check_close(out, ref, f"fp16 Hq={Hq} Hkv={Hkv} D={D} units=5")


@pytest.mark.parametrize("fmt", ["int8", "fp8_e4m3", "int4"])
@pytest.mark.parametrize("Hq,Hkv", [(32, 1), (48, 2), (40, 4)])
def test_quantized_large_groups(fmt, Hq, Hkv):
    """Blocks of 16 (two QK chains), 12 and 10 heads (one chain with hi / lo columns)."""
    from kvq_decode_amd import paged_decode_attention
    from kvq_decode_amd.quant import quantize_paged_cache
    q, kc, vc, bt, sl = make(Hq, Hkv, 128, LENS, seed=Hq + Hkv)
    qc = quantize_paged_cache(gpu(kc), gpu(vc), gpu(bt), gpu(sl), fmt)
    host = {n: getattr(qc, n).cpu().numpy() for n in
            ("k_codes", "v_codes", "k_scale", "k_zero", "v_scale", "v_zero")}
    kd, vd = kivi.dequantize_paged_cache(host, bt, sl, fmt)
    ref = paged_decode_attention_ref(q.astype(np.float32), kd, vd, bt, sl, out_dtype=np.float32)
    for splits in (1, 2, None):
        out = paged_decode_attention(gpu(q), qc.k_codes, qc.v_codes, gpu(bt), gpu(sl),
                                     num_splits=splits, **qc.decode_kwargs())
        torch.cuda.synchronize()
        check_close(out, ref, f"{fmt} Hq={Hq} Hkv={Hkv} splits={splits}")
