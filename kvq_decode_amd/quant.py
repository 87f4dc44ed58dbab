"""KIVI-quantized paged KV cache: bulk quantization (prefill) and quantize-on-append
(decode), through libkvq.so.

The reference plans quantized KV (README.md:7, :16) but has no code for it; its byte
model (src/bpt/roofline.py:6-9) fixes the scheme: asymmetric fp16 scale + zero, keys per
channel over groups of `k_group` tokens, values per token. Storage (include/kvq.h):
    k_codes, v_codes  uint8 [num_blocks, block_size, Hkv, D]   (int8 / fp8_e4m3 bits)
                      uint8 [num_blocks, block_size, Hkv, D/2] (int4, low nibble = even channel)
                      stored head-major (strides of [num_blocks, Hkv, block_size, Dc]), so
                      the codes of one (block, kv head) are one contiguous run; any strides
                      with 16-byte aligned rows are accepted
    k_scale, k_zero   fp16 [num_blocks, Hkv, D]  - group g of sequence b lives in block
                      block_table[b, g * k_group // block_size]
    v_scale, v_zero   fp16 [num_blocks, Hkv, VG], VG = max(block_size, 32) - the pairs of
                      tokens [j * VG, (j + 1) * VG) of sequence b live in block
                      block_table[b, j * VG // block_size], token t at index t % VG
                      both pairs are strided views of interleaved storage, one fp16
                      [..., 2] tensor of (scale, zero) per channel (K) / token (V): a
                      decode reads both of a token with one access
"""
import ctypes
from typing import NamedTuple, Optional

import torch

from kvq_decode_amd import _lib
from kvq_decode_amd._lib import KV_FORMATS, DecodeArgs
from kvq_decode_amd.ops import (DEFAULT_K_GROUP, KvqArgumentError, _require, check_scale_pairs,
                                v_group_tokens)

QUANT_FORMATS = ("int8", "fp8_e4m3", "int4")
# head dims of the quantized decode kernels, and so of the quantizers (include/kvq.h)
QUANT_HEAD_DIMS = (64, 128, 256)


# The on-device format these caches follow (include/kvq.h KVQ_CACHE_FORMAT_VERSION); a
# cache kept across processes should be stored with it and read back only by a library
# reporting the same value (cache_format_version()).
CACHE_FORMAT_VERSION = 2


def cache_format_version() -> int:
    """The quantized cache format version of the loaded libkvq.so."""
    return int(_lib.lib().kvq_cache_format_version())


class QuantizedKVCache(NamedTuple):
    k_codes: torch.Tensor
    v_codes: torch.Tensor
    k_scale: torch.Tensor
    k_zero: torch.Tensor
    v_scale: torch.Tensor
    v_zero: torch.Tensor
    kv_format: str
    k_group: int

    def decode_kwargs(self):
        """Keyword arguments for paged_decode_attention."""
        return dict(kv_format=self.kv_format, k_scale=self.k_scale, k_zero=self.k_zero,
                    v_scale=self.v_scale, v_zero=self.v_zero, k_group=self.k_group)

    @property
    def k_sz(self) -> torch.Tensor:
        """The interleaved K (scale, zero) storage [num_blocks, Hkv, D, 2]."""
        return _pairs(self.k_scale, self.k_zero, "k")

    @property
    def v_sz(self) -> torch.Tensor:
        """The interleaved V (scale, zero) storage [num_blocks, Hkv, VG, 2]."""
        return _pairs(self.v_scale, self.v_zero, "v")


def _pairs(scale: torch.Tensor, zero: torch.Tensor, name: str) -> torch.Tensor:
    check_scale_pairs(scale, zero, tuple(scale.shape), name)
    return scale.as_strided(tuple(scale.shape) + (2,), tuple(scale.stride()) + (1,))


def allocate_quantized_cache(num_blocks: int, block_size: int, kv_heads: int, head_dim: int,
                             kv_format: str, device, k_group: int = DEFAULT_K_GROUP
                             ) -> QuantizedKVCache:
    """Uninitialized code and scale tensors for a quantized paged cache.

    The code tensors are [num_blocks, block_size, Hkv, Dc] views of head-major storage: a
    decode workgroup reads one kv head, and an int4 token row of one head is 64 bytes, half
    an HBM cache line - token-major storage would fetch every line twice, once for each
    of the two heads sharing it, from workgroups on different XCDs."""
    _require(kv_format in QUANT_FORMATS, f"kv_format must be one of {QUANT_FORMATS}")
    _require(head_dim in QUANT_HEAD_DIMS,
             f"quantized caches take head_dim {QUANT_HEAD_DIMS} (the decode's), not {head_dim}")
    dc = head_dim // 2 if kv_format == "int4" else head_dim
    shape = (num_blocks, kv_heads, block_size, dc)
    kc = torch.empty(shape, dtype=torch.uint8, device=device).permute(0, 2, 1, 3)
    vc = torch.empty(shape, dtype=torch.uint8, device=device).permute(0, 2, 1, 3)
    ksz = torch.empty((num_blocks, kv_heads, head_dim, 2), dtype=torch.float16, device=device)
    vsz = torch.empty((num_blocks, kv_heads, v_group_tokens(block_size), 2), dtype=torch.float16,
                      device=device)
    return QuantizedKVCache(kc, vc, ksz[..., 0], ksz[..., 1], vsz[..., 0], vsz[..., 1],
                            kv_format, k_group)


def _qargs(cache: QuantizedKVCache, block_table, seq_lens, head_dim):
    """kvq_decode_args describing the quantized cache as the destination."""
    nb, bs, hkv, _ = cache.k_codes.shape
    a = DecodeArgs()
    a.k_cache = cache.k_codes.data_ptr()
    a.k_stride_blk, a.k_stride_tok, a.k_stride_head = cache.k_codes.stride()[:3]
    a.v_cache = cache.v_codes.data_ptr()
    a.v_stride_blk, a.v_stride_tok, a.v_stride_head = cache.v_codes.stride()[:3]
    a.block_table, a.bt_stride_b = block_table.data_ptr(), block_table.stride(0)
    a.seq_lens = seq_lens.data_ptr()
    a.batch, a.kv_heads, a.head_dim = block_table.shape[0], hkv, head_dim
    a.q_heads = hkv
    a.block_size, a.max_blocks, a.num_blocks = bs, block_table.shape[1], nb
    a.kv_format = KV_FORMATS[cache.kv_format]
    a.k_group = cache.k_group
    a.k_scale, a.k_zero = cache.k_scale.data_ptr(), cache.k_zero.data_ptr()
    a.v_scale, a.v_zero = cache.v_scale.data_ptr(), cache.v_zero.data_ptr()
    return a


def _check_cache(cache: QuantizedKVCache, block_table, seq_lens, head_dim):
    """Every check the quantizer entry points share; all of them run on tensor metadata
    before any launch, so a mismatch raises instead of reading or writing out of bounds."""
    _require(cache.kv_format in QUANT_FORMATS, f"kv_format must be one of {QUANT_FORMATS}")
    _require(head_dim in QUANT_HEAD_DIMS,
             f"quantized caches take head_dim {QUANT_HEAD_DIMS} (the decode's), not {head_dim}")
    _require(block_table.dtype == seq_lens.dtype == torch.int32,
             "block_table and seq_lens must be int32")
    _require(block_table.dim() == 2 and seq_lens.dim() == 1
             and block_table.shape[0] == seq_lens.shape[0],
             "block_table must be [B, max_blocks] and seq_lens [B]")
    _require(block_table.stride(1) == 1 and seq_lens.is_contiguous(),
             "block_table rows and seq_lens must be contiguous")
    nb, bs, hkv, dc = cache.k_codes.shape
    _require(tuple(cache.v_codes.shape) == (nb, bs, hkv, dc),
             "k_codes and v_codes shapes differ")
    _require(cache.k_codes.dtype == cache.v_codes.dtype == torch.uint8,
             "code caches must be uint8")
    _require(dc == (head_dim // 2 if cache.kv_format == "int4" else head_dim),
             "code cache width does not match head_dim")
    check_scale_pairs(cache.k_scale, cache.k_zero, (nb, hkv, head_dim), "k")
    check_scale_pairs(cache.v_scale, cache.v_zero, (nb, hkv, v_group_tokens(bs)), "v")
    _require(cache.k_group % bs == 0, "k_group must be a multiple of block_size")
    dev = cache.k_codes.device
    _require(dev.type == "cuda", "kvq runs on the GPU only (no CPU fallback)")
    _check_devices(dev, v_codes=cache.v_codes, k_scale=cache.k_scale, v_scale=cache.v_scale,
                   block_table=block_table, seq_lens=seq_lens)


def _check_devices(dev, **tensors):
    for name, t in tensors.items():
        _require(t.device == dev, f"{name} must be on the cache's device {dev} (got {t.device})")


def quantize_paged_cache(k_cache: torch.Tensor, v_cache: torch.Tensor,
                         block_table: torch.Tensor, seq_lens: torch.Tensor, kv_format: str,
                         k_group: int = DEFAULT_K_GROUP,
                         out: Optional[QuantizedKVCache] = None) -> QuantizedKVCache:
    """Quantize the valid tokens of fp16 paged caches (bulk / prefill).

    Codes are written for the seq_lens[b] tokens of every sequence; K scales per channel
    for every group of k_group tokens (a sequence's last group may be partial), V scales
    per token. Slots past each sequence are left untouched."""
    _require(k_cache.dtype == v_cache.dtype == torch.float16, "source caches must be fp16")
    _require(k_cache.shape == v_cache.shape and k_cache.stride() == v_cache.stride(),
             "k_cache and v_cache must have the same shape and strides")
    _require(k_cache.stride(3) == 1, "innermost dimension must be contiguous")
    nb, bs, hkv, d = k_cache.shape
    if out is None:
        out = allocate_quantized_cache(nb, bs, hkv, d, kv_format, k_cache.device, k_group)
    _require(out.kv_format == kv_format and out.k_group == k_group,
             "out cache format / group differ")
    _require(tuple(out.k_codes.shape[:3]) == (nb, bs, hkv),
             f"out cache [num_blocks, block_size, kv_heads] = {tuple(out.k_codes.shape[:3])} "
             f"differs from the source caches' {(nb, bs, hkv)}")
    _check_cache(out, block_table, seq_lens, d)
    _check_devices(out.k_codes.device, k_cache=k_cache, v_cache=v_cache)
    args = _qargs(out, block_table, seq_lens, d)
    stream = torch.cuda.current_stream(k_cache.device).cuda_stream
    _lib.check("kvq_quantize_cache",
               _lib.lib().kvq_quantize_cache(ctypes.byref(args), k_cache.data_ptr(),
                                             v_cache.data_ptr(), k_cache.stride(0),
                                             k_cache.stride(1), k_cache.stride(2), stream))
    return out


def init_k_residual(k_cache: torch.Tensor, block_table: torch.Tensor, seq_lens: torch.Tensor,
                    k_group: int = DEFAULT_K_GROUP) -> torch.Tensor:
    """fp16 residual [B, Hkv, k_group + 2, D] holding, for each sequence, the K rows of its
    open (last, incomplete) group in rows 0 .. k_group - 1 and their per-channel min and max
    in rows k_group and k_group + 1 - what quantize_append needs after a bulk prefill. Rows
    of a complete last group are zero (the next token opens a new group, which ignores
    them)."""
    B = block_table.shape[0]
    nb, bs, hkv, d = k_cache.shape
    resid = torch.zeros((B, hkv, k_group + 2, d), dtype=torch.float16, device=k_cache.device)
    lens = seq_lens.tolist()
    for b, n in enumerate(lens):
        t0 = (n // k_group) * k_group
        if t0 >= n:
            continue
        t = torch.arange(t0, n, device=k_cache.device)
        phys = block_table[b, t // bs].long()
        rows = k_cache[phys, t % bs].permute(1, 0, 2)  # [Hkv, n - t0, D]
        resid[b, :, : n - t0] = rows
        resid[b, :, k_group] = rows.amin(dim=1)
        resid[b, :, k_group + 1] = rows.amax(dim=1)
    return resid


def quantize_append(cache: QuantizedKVCache, k_new: torch.Tensor, v_new: torch.Tensor,
                    block_table: torch.Tensor, seq_lens: torch.Tensor,
                    k_resid: torch.Tensor) -> None:
    """Quantize one new token per sequence into the cache (decode-time write path).

    seq_lens must already count the new token: the token is at position seq_lens[b] - 1.
    k_new / v_new: fp16 [B, Hkv, D]. V is quantized per token into its slot. K joins the
    fp16 residual k_resid [B, Hkv, k_group + 2, D] of its group (init_k_residual: the rows,
    then their running per-channel min and max), and the group's channels whose range moved
    are re-encoded from it, so the cache always equals quantize_paged_cache of all tokens.
    Appends are sequential per sequence (each one's position follows the last)."""
    _require(k_new.dim() == 3, "k_new must be [B, kv_heads, head_dim]")
    B, hkv, d = k_new.shape
    _check_cache(cache, block_table, seq_lens, d)
    _require(block_table.shape[0] == B,
             f"block_table has {block_table.shape[0]} rows for a batch of {B} new tokens")
    _require(cache.k_codes.shape[2] == hkv,
             f"the cache has {cache.k_codes.shape[2]} kv heads, k_new {hkv}")
    for name, t, shape in (("k_new", k_new, (B, hkv, d)), ("v_new", v_new, (B, hkv, d)),
                           ("k_resid", k_resid, (B, hkv, cache.k_group + 2, d))):
        _require(t.dtype == torch.float16 and tuple(t.shape) == shape and t.is_contiguous(),
                 f"{name} must be contiguous fp16 of shape {shape}")
    _check_devices(cache.k_codes.device, k_new=k_new, v_new=v_new, k_resid=k_resid)
    args = _qargs(cache, block_table, seq_lens, d)
    stream = torch.cuda.current_stream(k_new.device).cuda_stream
    _lib.check("kvq_quantize_append",
               _lib.lib().kvq_quantize_append(ctypes.byref(args), k_new.data_ptr(),
                                              v_new.data_ptr(), k_resid.data_ptr(), stream))


__all__ = ["QuantizedKVCache", "allocate_quantized_cache", "quantize_paged_cache",
           "init_k_residual", "quantize_append", "QUANT_FORMATS", "KvqArgumentError"]
