"""Numpy restatement of the reference's paged GQA decode attention. TEST INFRASTRUCTURE.

Layout (vLLM style, reference src/bpt/reference.py:3-9):
    q            [B, Hq, D]
    k_cache      [num_blocks, block_size, Hkv, D]
    v_cache      [num_blocks, block_size, Hkv, D]
    block_table  [B, max_blocks] int32   logical block -> physical block
    seq_lens     [B] int32               valid tokens per sequence
    returns      [B, Hq, D] in q's dtype

Math is float32 (float64 on request), q head h reads kv head h // (Hq // Hkv).
"""

import math

import numpy as np


def _cdiv(a, b):
    return -(-a // b)


def _next_pow2(x):
    x = int(x)
    return 1 if x <= 1 else 1 << (x - 1).bit_length()


def _gather_seq(cache, blocks, n):
    """[n_blocks, bs, Hkv, D] pages of one sequence -> contiguous [n, Hkv, D]
    (reference.py:39-42: index by the block table, flatten, drop the partial-page tail)."""
    _, bs, hkv, d = cache.shape
    return cache[blocks].reshape(-1, hkv, d)[:n]


def _attend(qb, k, v, scale, acc_dtype):
    """One sequence: qb [Hq, D], k/v [n, Hkv, D] -> [Hq, D] in acc_dtype.

    Follows reference.py:43-48: scores = q . k * scale, softmax over tokens, probs @ v,
    with q head h mapped to kv head h // group. The einsum over repeat_interleave'd
    K/V is computed per kv head with matmuls (same sums, no 4x copies)."""
    hq, d = qb.shape
    n, hkv, _ = k.shape
    group = hq // hkv
    q3 = qb.astype(acc_dtype).reshape(hkv, group, d)          # [Hkv, group, D]
    kt = k.astype(acc_dtype).transpose(1, 2, 0)               # [Hkv, D, n]
    vt = v.astype(acc_dtype).transpose(1, 0, 2)               # [Hkv, n, D]
    scores = np.matmul(q3, kt) * acc_dtype(scale)             # [Hkv, group, n]
    scores = scores - scores.max(axis=-1, keepdims=True)
    p = np.exp(scores)
    p = p / p.sum(axis=-1, keepdims=True)
    return np.matmul(p, vt).reshape(hq, d)                    # [Hq, D]


def paged_decode_attention_ref(q, k_cache, v_cache, block_table, seq_lens, scale=None,
                               acc_dtype=np.float32, out_dtype=None):
    """Reference oracle, reference.py:20-49.

    Loops over the batch (reference.py:36), gathers the sequence's pages
    (reference.py:38-42), computes softmax attention in `acc_dtype` and casts the
    result back to q's dtype (reference.py:48), or to `out_dtype` when given (the
    parity tests keep the float32 result to measure the kernel's own rounding)."""
    B, Hq, D = q.shape
    _, bs, Hkv, _ = k_cache.shape
    assert Hq % Hkv == 0, "q heads must be a multiple of kv heads"
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    out_dtype = q.dtype if out_dtype is None else out_dtype
    out = np.empty(q.shape, dtype=out_dtype)
    for b in range(B):
        n = int(seq_lens[b])
        nb = _cdiv(n, bs)
        blocks = np.asarray(block_table[b, :nb], dtype=np.int64)
        k = _gather_seq(k_cache, blocks, n)
        v = _gather_seq(v_cache, blocks, n)
        out[b] = _attend(q[b], k, v, scale, acc_dtype).astype(out_dtype)
    return out


def build_paged_cache(k, v, seq_lens, block_size, rng):
    """Scatter contiguous k/v [B, S, Hkv, D] into a paged cache, reference.py:52-82.

    Physical blocks are a random permutation of B * max_blocks blocks (reference.py:66-69)
    and every slot not covered by a sequence holds 100 * N(0, 1) garbage
    (reference.py:71-74), so block-table and masking bugs cannot pass by accident.
    `rng` is a numpy Generator; the random stream differs from torch's, the semantics
    do not. Returns (k_cache, v_cache, block_table int32)."""
    B, S, Hkv, D = k.shape
    max_blocks = _cdiv(S, block_size)
    num_blocks = B * max_blocks
    perm = rng.permutation(num_blocks)
    block_table = perm.reshape(B, max_blocks).astype(np.int32)

    def fill(x):
        cache = (100.0 * rng.standard_normal((num_blocks, block_size, Hkv, D))).astype(x.dtype)
        for b in range(B):
            n = int(seq_lens[b])
            for i in range(_cdiv(n, block_size)):
                lo, hi = i * block_size, min((i + 1) * block_size, n)
                cache[block_table[b, i], : hi - lo] = x[b, lo:hi]
        return cache

    return fill(k), fill(v), block_table


# ---------------------------------------------------------------- split-KV semantics

TARGET_PROGRAMS_PER_SM = 8     # reference src/bpt/triton_fp16.py:166
MIN_TOKENS_PER_SPLIT = 512     # reference src/bpt/triton_fp16.py:167


def choose_num_splits(batch, kv_heads, block_size, max_pages, sm_count,
                      target_programs_per_sm=TARGET_PROGRAMS_PER_SM,
                      min_tokens_per_split=MIN_TOKENS_PER_SPLIT):
    """Split heuristic, reference triton_fp16.py:175-180:
    S = max(1, min(next_pow2(cdiv(target * SMs, B * Hkv)), max_pages // max(1, 512 // bs)))."""
    want = _cdiv(target_programs_per_sm * sm_count, batch * kv_heads)
    cap = max(1, max_pages // max(1, min_tokens_per_split // block_size))
    return max(1, min(_next_pow2(want), cap))


def normalize_splits(num_splits, max_pages):
    """Clamp and re-derive the split count, reference triton_fp16.py:211-217.
    Returns (splits, pages_per_split); splits == 1 means the single-pass kernel."""
    splits = max(1, min(int(num_splits), int(max_pages)))
    pps = int(max_pages)
    if splits > 1:
        pps = _cdiv(max_pages, splits)
        splits = _cdiv(max_pages, pps)  # drop splits that are empty for every sequence
    return splits, pps


def split_decode_ref(q, k_cache, v_cache, block_table, seq_lens, scale, num_splits,
                     pages_per_split, acc_dtype=np.float32):
    """Stage 1 of split-KV, reference triton_fp16.py:83-144.

    Split s of sequence b covers pages [s * pps, min((s + 1) * pps, cdiv(len, bs)))
    (triton_fp16.py:114-116). Each split stores the NORMALIZED partial output
    o = acc / l and lse = m + log(l) (triton_fp16.py:138-143); an empty split stores
    o = 0, lse = -inf (triton_fp16.py:138-141). Returns o_part [B, Hq, S, D] and
    lse [B, Hq, S], both float32 (triton_fp16.py:219-220)."""
    B, Hq, D = q.shape
    _, bs, Hkv, _ = k_cache.shape
    group = Hq // Hkv
    o_part = np.zeros((B, Hq, num_splits, D), dtype=np.float32)
    lse = np.full((B, Hq, num_splits), -np.inf, dtype=np.float32)
    for b in range(B):
        n = int(seq_lens[b])
        n_pages = _cdiv(n, bs)
        for s in range(num_splits):
            lo_p = s * pages_per_split
            hi_p = min(lo_p + pages_per_split, n_pages)
            if lo_p >= hi_p:
                continue
            blocks = np.asarray(block_table[b, lo_p:hi_p], dtype=np.int64)
            t_lo, t_hi = lo_p * bs, min(hi_p * bs, n)
            k = _gather_seq(k_cache, blocks, t_hi - t_lo).astype(acc_dtype)
            v = _gather_seq(v_cache, blocks, t_hi - t_lo).astype(acc_dtype)
            q3 = q[b].astype(acc_dtype).reshape(Hkv, group, D)
            sc = np.matmul(q3, k.transpose(1, 2, 0)) * acc_dtype(scale)   # [Hkv, g, n]
            m = sc.max(axis=-1, keepdims=True)
            p = np.exp(sc - m)
            l_ = p.sum(axis=-1, keepdims=True)
            o = np.matmul(p, v.transpose(1, 0, 2)) / l_
            o_part[b, :, s] = o.reshape(Hq, D)
            lse[b, :, s] = (m + np.log(l_)).reshape(Hq)
    return o_part, lse


def merge_ref(o_part, lse, out_dtype=np.float16):
    """Stage 2, reference triton_fp16.py:147-163:
    out = sum_s w_s o_s / sum_s w_s with w_s = exp(lse_s - max_s lse_s); empty splits
    carry lse = -inf and so weigh zero."""
    mx = lse.max(axis=-1, keepdims=True)
    w = np.exp(lse - mx)                                   # [B, Hq, S]
    out = (w[..., None] * o_part).sum(axis=2) / w.sum(axis=-1)[..., None]
    return out.astype(out_dtype)
