"""torch.library registration of the decode path: `torch.ops.kvq.*`.

The reference's op allocates per call and syncs on `seq_lens.min()`
(src/bpt/triton_fp16.py:201, 206, 219-220), which keeps it out of graph capture and of
traced model code. These custom ops wrap the same library calls with schemas, fake
(shape-only) kernels for tracing, and no host synchronisation: a decode step built from
them - append the new token, decode - can be captured in a HIP graph
(`torch.cuda.CUDAGraph`) and replayed.

Quantized caches pass their (scale, zero) storage as the interleaved pair tensors
k_sz [num_blocks, Hkv, D, 2] and v_sz [num_blocks, Hkv, max(block_size, 32), 2]
(QuantizedKVCache.k_sz / .v_sz), one tensor each, so that every mutated buffer is a
schema argument of its own.

  kvq::paged_decode(q, k_cache, v_cache, block_table, seq_lens, scale, num_splits,
                    kv_format, k_sz, v_sz, k_group) -> Tensor
  kvq::paged_decode_out(..., out!)            writes out, returns nothing
  kvq::append_kv(k_cache!, v_cache!, k_new, v_new, block_table, seq_lens)
  kvq::reshape_and_cache(key, value, k_cache!, v_cache!, slot_mapping)
  kvq::quantize_append(k_codes!, v_codes!, k_sz!, v_sz!, k_new, v_new, block_table,
                       seq_lens, k_resid!, kv_format, k_group)

All kernels are registered for CUDA (ROCm) devices only; other devices raise.
"""
from typing import Optional

import torch
from torch import Tensor

from kvq_decode_amd import cache as _cache
from kvq_decode_amd import quant as _quant
from kvq_decode_amd.ops import DEFAULT_K_GROUP, _require, paged_decode_attention


def _fmt_kwargs(kv_format: str, k_sz: Optional[Tensor], v_sz: Optional[Tensor],
                k_group: int) -> dict:
    if kv_format == "fp16":
        return {}
    _require(k_sz is not None and v_sz is not None,
             f"kv_format={kv_format!r} needs the k_sz / v_sz pair tensors")
    for name, t in (("k_sz", k_sz), ("v_sz", v_sz)):
        _require(t.dim() == 4 and t.shape[-1] == 2 and t.is_contiguous(),
                 f"{name} must be a contiguous [num_blocks, Hkv, n, 2] pair tensor")
    return dict(kv_format=kv_format, k_scale=k_sz[..., 0], k_zero=k_sz[..., 1],
                v_scale=v_sz[..., 0], v_zero=v_sz[..., 1], k_group=k_group)


@torch.library.custom_op("kvq::paged_decode", mutates_args=(), device_types="cuda")
def paged_decode(q: Tensor, k_cache: Tensor, v_cache: Tensor, block_table: Tensor,
                 seq_lens: Tensor, scale: Optional[float] = None,
                 num_splits: Optional[int] = None, kv_format: str = "fp16",
                 k_sz: Optional[Tensor] = None, v_sz: Optional[Tensor] = None,
                 k_group: int = DEFAULT_K_GROUP) -> Tensor:
    """paged_decode_attention as a custom op (new output tensor)."""
    return paged_decode_attention(q, k_cache, v_cache, block_table, seq_lens, scale,
                                  num_splits, **_fmt_kwargs(kv_format, k_sz, v_sz, k_group))


@paged_decode.register_fake
def _(q, k_cache, v_cache, block_table, seq_lens, scale=None, num_splits=None,
      kv_format="fp16", k_sz=None, v_sz=None, k_group=DEFAULT_K_GROUP):
    return q.new_empty(q.shape, dtype=torch.float16)


@torch.library.custom_op("kvq::paged_decode_out", mutates_args=("out",), device_types="cuda")
def paged_decode_out(q: Tensor, k_cache: Tensor, v_cache: Tensor, block_table: Tensor,
                     seq_lens: Tensor, out: Tensor, scale: Optional[float] = None,
                     num_splits: Optional[int] = None, kv_format: str = "fp16",
                     k_sz: Optional[Tensor] = None, v_sz: Optional[Tensor] = None,
                     k_group: int = DEFAULT_K_GROUP) -> None:
    """paged_decode_attention into a caller-owned `out` [B, Hq, D] fp16."""
    paged_decode_attention(q, k_cache, v_cache, block_table, seq_lens, scale, num_splits,
                           out=out, **_fmt_kwargs(kv_format, k_sz, v_sz, k_group))


@paged_decode_out.register_fake
def _(q, k_cache, v_cache, block_table, seq_lens, out, scale=None, num_splits=None,
      kv_format="fp16", k_sz=None, v_sz=None, k_group=DEFAULT_K_GROUP):
    return None


@torch.library.custom_op("kvq::append_kv", mutates_args=("k_cache", "v_cache"),
                         device_types="cuda")
def append_kv(k_cache: Tensor, v_cache: Tensor, k_new: Tensor, v_new: Tensor,
              block_table: Tensor, seq_lens: Tensor) -> None:
    """cache.append_kv: one new fp16 token per sequence at position seq_lens[b] - 1."""
    _cache.append_kv(k_cache, v_cache, k_new, v_new, block_table, seq_lens)


@append_kv.register_fake
def _(k_cache, v_cache, k_new, v_new, block_table, seq_lens):
    return None


@torch.library.custom_op("kvq::reshape_and_cache", mutates_args=("k_cache", "v_cache"),
                         device_types="cuda")
def reshape_and_cache(key: Tensor, value: Tensor, k_cache: Tensor, v_cache: Tensor,
                      slot_mapping: Tensor) -> None:
    """cache.reshape_and_cache: vLLM-style scatter of token rows by flat slot."""
    _cache.reshape_and_cache(key, value, k_cache, v_cache, slot_mapping)


@reshape_and_cache.register_fake
def _(key, value, k_cache, v_cache, slot_mapping):
    return None


@torch.library.custom_op("kvq::quantize_append",
                         mutates_args=("k_codes", "v_codes", "k_sz", "v_sz", "k_resid"),
                         device_types="cuda")
def quantize_append(k_codes: Tensor, v_codes: Tensor, k_sz: Tensor, v_sz: Tensor,
                    k_new: Tensor, v_new: Tensor, block_table: Tensor, seq_lens: Tensor,
                    k_resid: Tensor, kv_format: str, k_group: int = DEFAULT_K_GROUP) -> None:
    """quant.quantize_append on a cache given as codes + pair tensors."""
    kw = _fmt_kwargs(kv_format, k_sz, v_sz, k_group)
    qc = _quant.QuantizedKVCache(k_codes, v_codes, kw["k_scale"], kw["k_zero"],
                                 kw["v_scale"], kw["v_zero"], kv_format, k_group)
    _quant.quantize_append(qc, k_new, v_new, block_table, seq_lens, k_resid)


@quantize_append.register_fake
def _(k_codes, v_codes, k_sz, v_sz, k_new, v_new, block_table, seq_lens, k_resid, kv_format,
      k_group=DEFAULT_K_GROUP):
    return None


__all__ = ["paged_decode", "paged_decode_out", "append_kv", "reshape_and_cache",
           "quantize_append"]
