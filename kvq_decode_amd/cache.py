"""fp16 KV write path: new token rows into a paged cache, on the GPU, through libkvq.so.

The reference builds its paged caches once, on the host (src/bpt/reference.py:52-82:
token i of sequence b goes to block block_table[b, i // block_size], slot
i % block_size) and has no decode-time write. A decode loop needs one; these are the
two shapes callers use:

  append_kv          one new token per sequence, at position seq_lens[b] - 1 (seq_lens
                     already counts it) - the fp16 counterpart of quant.quantize_append;
  reshape_and_cache  vLLM's form: rows [T, Hkv, D] and a flat slot per row
                     (block * block_size + offset; negative = padding, not written).

Both are a single kernel launch with no host synchronisation, so they can be captured in
a HIP graph with the decode that follows.
"""
import ctypes

import torch

from kvq_decode_amd import _lib
from kvq_decode_amd._lib import DecodeArgs, KV_FORMATS
from kvq_decode_amd.ops import _require


def _cache_args(k_cache: torch.Tensor, v_cache: torch.Tensor) -> DecodeArgs:
    _require(k_cache.dtype == v_cache.dtype == torch.float16, "caches must be float16")
    _require(k_cache.dim() == 4 and tuple(v_cache.shape) == tuple(k_cache.shape),
             "caches must be [num_blocks, block_size, Hkv, D] of the same shape")
    _require(k_cache.stride(3) == v_cache.stride(3) == 1, "cache head_dim must be contiguous")
    _require(k_cache.device.type == "cuda" and v_cache.device == k_cache.device,
             "kvq runs on the GPU only (no CPU fallback)")
    nb, bs, hkv, d = k_cache.shape
    a = DecodeArgs()
    a.k_cache = k_cache.data_ptr()
    a.k_stride_blk, a.k_stride_tok, a.k_stride_head = k_cache.stride()[:3]
    a.v_cache = v_cache.data_ptr()
    a.v_stride_blk, a.v_stride_tok, a.v_stride_head = v_cache.stride()[:3]
    a.kv_heads, a.head_dim, a.block_size, a.num_blocks = hkv, d, bs, nb
    a.kv_format = KV_FORMATS["fp16"]
    return a


def append_kv(k_cache: torch.Tensor, v_cache: torch.Tensor, k_new: torch.Tensor,
              v_new: torch.Tensor, block_table: torch.Tensor, seq_lens: torch.Tensor) -> None:
    """Write one new token per sequence into fp16 paged caches (in place).

    k_new / v_new: fp16 [B, Hkv, D] contiguous. The token of sequence b goes to position
    seq_lens[b] - 1 (seq_lens must already count it) through block_table [B, max_blocks]
    int32. A position past the table or a block outside the pool writes nothing."""
    a = _cache_args(k_cache, v_cache)
    B = block_table.shape[0]
    shape = (B, a.kv_heads, a.head_dim)
    for name, t in (("k_new", k_new), ("v_new", v_new)):
        _require(t.dtype == torch.float16 and tuple(t.shape) == shape and t.is_contiguous()
                 and t.device == k_cache.device,
                 f"{name} must be contiguous float16 {shape} on the caches' device")
    _require(block_table.dtype == seq_lens.dtype == torch.int32,
             "block_table and seq_lens must be int32")
    _require(block_table.dim() == 2 and block_table.stride(1) == 1 and
             seq_lens.shape == (B,) and seq_lens.is_contiguous(),
             "block_table must be [B, max_blocks] with contiguous rows, seq_lens [B]")
    _require(block_table.device == seq_lens.device == k_cache.device,
             "all tensors must be on the same device")
    a.block_table, a.bt_stride_b = block_table.data_ptr(), block_table.stride(0)
    a.seq_lens = seq_lens.data_ptr()
    a.batch, a.max_blocks = B, block_table.shape[1]
    stream = torch.cuda.current_stream(k_cache.device).cuda_stream
    _lib.check("kvq_append_kv", _lib.lib().kvq_append_kv(
        ctypes.byref(a), k_new.data_ptr(), v_new.data_ptr(), stream))


def reshape_and_cache(key: torch.Tensor, value: torch.Tensor, k_cache: torch.Tensor,
                      v_cache: torch.Tensor, slot_mapping: torch.Tensor) -> None:
    """vLLM-style scatter of T token rows into fp16 paged caches (in place).

    key / value: fp16 [T, Hkv, D] with a contiguous last dim; slot_mapping: int64 [T],
    flat slot block * block_size + offset, negative for padding rows (not written)."""
    a = _cache_args(k_cache, v_cache)
    T = key.shape[0]
    shape = (T, a.kv_heads, a.head_dim)
    for name, t in (("key", key), ("value", value)):
        _require(t.dtype == torch.float16 and tuple(t.shape) == shape and t.stride(2) == 1
                 and t.device == k_cache.device,
                 f"{name} must be float16 {shape} with a contiguous last dim")
    _require(key.stride() == value.stride(), "key and value must have the same strides")
    _require(slot_mapping.dtype == torch.int64 and slot_mapping.shape == (T,)
             and slot_mapping.is_contiguous() and slot_mapping.device == k_cache.device,
             "slot_mapping must be contiguous int64 [T] on the caches' device")
    stream = torch.cuda.current_stream(k_cache.device).cuda_stream
    _lib.check("kvq_reshape_and_cache", _lib.lib().kvq_reshape_and_cache(
        ctypes.byref(a), key.data_ptr(), value.data_ptr(), key.stride(0), key.stride(1),
        slot_mapping.data_ptr(), T, stream))


__all__ = ["append_kv", "reshape_and_cache"]
