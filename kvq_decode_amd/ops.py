"""Host-side op: paged-KV GQA decode attention on MI355X through libkvq.so.

Drop-in for the reference's `paged_decode_attention_triton` (pawaryd/kvq-decode
src/bpt/triton_fp16.py:183-247): same positional/keyword signature, same vLLM-style
layout, same split-KV semantics and the same heuristic helpers (`choose_num_splits`,
`_sm_count`, `TARGET_PROGRAMS_PER_SM`, `MIN_TOKENS_PER_SPLIT`), which the reference's
bench imports (bench/bench_triton_fp16.py:11-12).

Differences, all on purpose:
  * No per-call device->host sync: the reference's `assert int(seq_lens.min()) >= 1`
    (triton_fp16.py:201) blocks graph capture; here seq_len >= 1 is a documented
    precondition, checked only when `check_seq_lens=True`.
  * The split-KV workspace can be passed in (`workspace=`) instead of being allocated per
    call (triton_fp16.py:219-220).
  * Keyword-only extensions for KIVI-quantized caches (`kv_format=`, scales) that the
    reference planned but never built.
"""
import ctypes
import functools
import math
from typing import Optional, Tuple

import torch

from kvq_decode_amd import _lib
from kvq_decode_amd._lib import DecodeArgs, KV_FORMATS

# triton_fp16.py:166-167 - the reference's heuristic constants, kept as its defaults.
TARGET_PROGRAMS_PER_SM = 8
MIN_TOKENS_PER_SPLIT = 512

DEFAULT_K_GROUP = 128  # tokens per K scale group (reference roofline.py:50 group_size)


def v_group_tokens(block_size: int) -> int:
    """Tokens per V (scale, zero) group of a quantized cache, max(block_size, 32): the
    pairs of a group live in its first page, so the 32 pairs of one kv head that a 128-byte
    line holds belong to 32 consecutive tokens of one sequence (include/kvq.h)."""
    return max(block_size, 32)


class KvqArgumentError(AssertionError, ValueError):
    """A precondition the reference asserts (triton_fp16.py:195-201) does not hold.
    Subclasses AssertionError so callers written against the reference still catch it."""


def _require(cond, msg):
    if not cond:
        raise KvqArgumentError(msg)


@functools.lru_cache(maxsize=None)
def _sm_count(device_index: int) -> int:
    """Compute units of the device (reference triton_fp16.py:170-172; 256 on MI355X)."""
    return torch.cuda.get_device_properties(device_index).multi_processor_count


def choose_num_splits(batch: int, kv_heads: int, block_size: int, max_pages: int,
                      sm_count: int) -> int:
    """Enough workgroups to fill the GPU, without splits shorter than a few pages.
    Same formula and constants as the reference (triton_fp16.py:175-180); computed by
    the library (kvq_choose_num_splits)."""
    s = _lib.lib().kvq_choose_num_splits(batch, kv_heads, block_size, max_pages, sm_count,
                                        TARGET_PROGRAMS_PER_SM, MIN_TOKENS_PER_SPLIT)
    return _lib.check("kvq_choose_num_splits", s)


@functools.lru_cache(maxsize=4096)  # a pure function of its arguments; saves a C call per op
def head_blocks(q_heads: int, kv_heads: int) -> int:
    """q-head blocks per kv head (kvq_head_blocks): a group of more than 16 q heads per kv
    head runs as k blocks of q_heads / (kv_heads * k) heads, each reading the caches; the
    plans below take kv_heads * k kv heads."""
    k = _lib.lib().kvq_head_blocks(q_heads, kv_heads)
    _require(k >= 1, "q heads must be a multiple of kv heads")
    return k


def plan_decode(batch: int, kv_heads: int, block_size: int, max_pages: int,
                cu_count: int, kv_format: str = "fp16", head_dim: int = 128,
                q_heads: Optional[int] = None) -> Tuple[int, int]:
    """(num_splits, waves_per_group) for the MI355X kernels when num_splits is None: the
    split-KV decomposition the reference's heuristic aims at (triton_fp16.py:175-180:
    enough programs to fill the GPU, no tiny splits), counted in waves because one
    workgroup here holds several waves that combine through LDS. Computed by the library
    (kvq_plan_decode): about 2 waves per CU for fp16, 4 for INT8 / FP8 and 8 for INT4, at most
    512 (fp16) / 256 or, for batches whose (sequence, kv head) pairs outnumber the CUs, 64
    (quantized) 16-token chunks per wave; up to 2 waves per workgroup for fp16, and for
    quantized caches one wave per 8 waves of the (sequence, kv head) pair, up to 4 (INT4:
    8). fp16 head dims below 128 get 128 / head_dim times the waves (16 and 32, whose rows
    share lines between kv heads: 64 / head_dim), in workgroups of up to 4 waves. Waves are halved (splits doubled) until a workgroup's LDS, which grows with
    the q heads per kv head, fits 64 KB. `kv_heads` counts the kernels' kv heads (see
    `head_blocks`); `q_heads` (default: kv_heads, one q head per kv head) all q heads."""
    _require(kv_format in KV_FORMATS, f"kv_format must be one of {tuple(KV_FORMATS)}")
    s, w = ctypes.c_int32(), ctypes.c_int32()
    _lib.check("kvq_plan_decode",
               _lib.lib().kvq_plan_decode(batch, q_heads or kv_heads, kv_heads, block_size,
                                          max_pages, KV_FORMATS[kv_format], head_dim, cu_count,
                                          ctypes.byref(s), ctypes.byref(w)))
    return s.value, w.value


def auto_splits(batch: int, kv_heads: int, block_size: int, max_pages: int,
                cu_count: int, kv_format: str = "fp16", head_dim: int = 128,
                q_heads: Optional[int] = None) -> int:
    return plan_decode(batch, kv_heads, block_size, max_pages, cu_count, kv_format,
                       head_dim, q_heads)[0]


@functools.lru_cache(maxsize=4096)
def normalize_splits(num_splits: int, max_pages: int) -> Tuple[int, int]:
    """(splits, pages_per_split) after the reference's clamp/re-derivation
    (triton_fp16.py:211-217)."""
    s, pps = ctypes.c_int32(), ctypes.c_int32()
    _lib.check("kvq_normalize_splits",
               _lib.lib().kvq_normalize_splits(int(num_splits), int(max_pages),
                                               ctypes.byref(s), ctypes.byref(pps)))
    return s.value, pps.value


@functools.lru_cache(maxsize=4096)
def plan_units(batch: int, kv_heads: int, block_size: int, max_pages: int,
               cu_count: int, kv_format: str = "fp16", head_dim: int = 128,
               q_heads: Optional[int] = None) -> Tuple[int, int]:
    """(units, waves_per_group) of the work-unit partition when the library prefers it
    for num_splits=None, else (0, 0) (kvq_plan_units): batches of 2 to 1024 sequences
    whose split plan (`plan_decode`) has 2 or more splits, or whose longest context is at
    least 4096 tokens, get 2 waves per CU in 2-wave
    unit workgroups (fp16), 4 in 4-wave workgroups (INT8, FP8) or 8 in 2-wave workgroups
    (INT4), which keeps ragged batches balanced. Head dims below 128 get 128 / head_dim
    times the waves per CU (16 and 32: 64 / head_dim), and fp16 / INT4 unit workgroups of up
    to 4 waves. As in
    `plan_decode`, waves are halved (units doubled) until a workgroup's LDS fits 64 KB, and
    `q_heads` defaults to kv_heads."""
    _require(kv_format in KV_FORMATS, f"kv_format must be one of {tuple(KV_FORMATS)}")
    u, w = ctypes.c_int32(), ctypes.c_int32()
    _lib.check("kvq_plan_units",
               _lib.lib().kvq_plan_units(batch, q_heads or kv_heads, kv_heads, block_size,
                                         max_pages, KV_FORMATS[kv_format], head_dim, cu_count,
                                         ctypes.byref(u), ctypes.byref(w)))
    return u.value, w.value


def workspace_shapes(batch: int, q_heads: int, head_dim: int, splits: int):
    """Shapes of the split-KV workspace (o_part, lse) for `splits` splits."""
    return (batch, q_heads, splits, head_dim), (batch, q_heads, splits)


def units_workspace_shapes(batch: int, q_heads: int, head_dim: int, units: int):
    """Shapes of the work-unit workspace (o_part, lse) for `units` units per kv head."""
    return (q_heads, units + batch, head_dim), (q_heads, units + batch)


def plan_workspace_shapes(batch: int, q_heads: int, kv_heads: int, head_dim: int,
                          block_size: int, max_pages: int, cu_count: int,
                          kv_format: str = "fp16"):
    """Shapes of the workspace (o_part, lse) the op needs with num_splits=None for these
    sizes (work units or splits, as `plan_units` / `plan_decode` choose), or None when
    the plan runs a single pass and needs none. For callers that preallocate, e.g. before
    a graph capture."""
    grid_heads = kv_heads * head_blocks(q_heads, kv_heads)
    units, _ = plan_units(batch, grid_heads, block_size, max_pages, cu_count, kv_format,
                          head_dim, q_heads)
    if units:
        return units_workspace_shapes(batch, q_heads, head_dim, units)
    splits, _ = plan_decode(batch, grid_heads, block_size, max_pages, cu_count, kv_format,
                            head_dim, q_heads)
    splits = normalize_splits(splits, max_pages)[0]
    return None if splits == 1 else workspace_shapes(batch, q_heads, head_dim, splits)


def check_scale_pairs(scale: torch.Tensor, zero: torch.Tensor, shape, name: str) -> None:
    """The scale / zero tensors of a quantized cache are views of one interleaved fp16
    [..., 2] tensor of (scale, zero) pairs (include/kvq.h): element strides
    (2 * prod(shape[1:]), ..., 2) and the zero one element after the scale."""
    shape = tuple(shape)
    want = []
    acc = 2
    for n in reversed(shape):
        want.append(acc)
        acc *= n
    want = tuple(reversed(want))
    for t in (scale, zero):
        _require(t is not None, f"{name}_scale / {name}_zero are required for a quantized cache")
        _require(t.dtype == torch.float16 and tuple(t.shape) == shape and t.stride() == want,
                 f"{name}_scale / {name}_zero must be fp16 {shape} views of an interleaved "
                 f"(scale, zero) tensor {shape + (2,)} (strides {want})")
    _require(zero.data_ptr() == scale.data_ptr() + 2,
             f"{name}_zero must be the element after {name}_scale (interleaved pairs)")


def _ptr(t: Optional[torch.Tensor]) -> int:
    return 0 if t is None else t.data_ptr()


def _is_pow2(x: int) -> bool:
    return x > 0 and (x & (x - 1)) == 0


def build_args(q, k_cache, v_cache, block_table, seq_lens, out, scale, kv_format="fp16",
               k_scale=None, k_zero=None, v_scale=None, v_zero=None,
               k_group=DEFAULT_K_GROUP, waves_per_group=0, pipeline=0) -> DecodeArgs:
    """Fill a kvq_decode_args from tensors (no validation beyond what ctypes needs)."""
    B, Hq, D = q.shape
    nb, bs, Hkv, _ = k_cache.shape
    a = DecodeArgs()
    a.q, a.q_stride_b, a.q_stride_h = q.data_ptr(), q.stride(0), q.stride(1)
    a.k_cache = k_cache.data_ptr()
    a.k_stride_blk, a.k_stride_tok, a.k_stride_head = k_cache.stride()[:3]
    a.v_cache = v_cache.data_ptr()
    a.v_stride_blk, a.v_stride_tok, a.v_stride_head = v_cache.stride()[:3]
    a.block_table, a.bt_stride_b = block_table.data_ptr(), block_table.stride(0)
    a.seq_lens = seq_lens.data_ptr()
    if out is not None:
        a.out, a.o_stride_b, a.o_stride_h = out.data_ptr(), out.stride(0), out.stride(1)
    a.batch, a.q_heads, a.kv_heads, a.head_dim = B, Hq, Hkv, D
    a.block_size, a.max_blocks, a.num_blocks = bs, block_table.shape[1], nb
    a.scale = float(scale)
    a.kv_format = KV_FORMATS[kv_format]
    a.k_group = int(k_group)
    a.k_scale, a.k_zero = _ptr(k_scale), _ptr(k_zero)
    a.v_scale, a.v_zero = _ptr(v_scale), _ptr(v_zero)
    a.waves_per_group = int(waves_per_group)
    a.pipeline = int(pipeline)
    return a


def _stream(device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def paged_decode_attention(
    q: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    block_table: torch.Tensor,
    seq_lens: torch.Tensor,
    scale: Optional[float] = None,
    num_splits: Optional[int] = None,
    *,
    kv_format: str = "fp16",
    k_scale: Optional[torch.Tensor] = None,
    k_zero: Optional[torch.Tensor] = None,
    v_scale: Optional[torch.Tensor] = None,
    v_zero: Optional[torch.Tensor] = None,
    k_group: int = DEFAULT_K_GROUP,
    out: Optional[torch.Tensor] = None,
    workspace: Optional[Tuple[torch.Tensor, torch.Tensor]] = None,
    check_seq_lens: bool = False,
    waves_per_group: int = 0,
    pipeline: int = 0,
    units: int = 0,
) -> torch.Tensor:
    """GQA decode attention over a paged KV cache (reference triton_fp16.py:183-247).

    q [B, Hq, D] fp16; k_cache/v_cache [num_blocks, block_size, Hkv, D] fp16 (or uint8
    codes for a quantized `kv_format`); block_table [B, max_blocks] int32; seq_lens [B]
    int32 (every entry >= 1). num_splits: None = heuristic, 1 = single pass, n = split
    each sequence n ways. Returns [B, Hq, D] fp16 (written into `out` when given).
    `workspace` = (o_part, lse) float32 buffers of at least the shapes
    `workspace_shapes(B, Hq, D, S)` for the normalized split count S (work units:
    `units_workspace_shapes(B, Hq, D, units)`; with num_splits=None,
    `plan_workspace_shapes` gives whichever the plan needs). With num_splits=None the partition comes
    from `plan_units` (work units: batches of 2 to 1024 with 4096-token contexts or that the
    split plan would split) or else `plan_decode` (`choose_num_splits` keeps the reference's formula for callers
    that want it). `units` > 0 (B <= 1024) asks for the work-unit partition: per kv head,
    all sequences' 16-token chunks in batch order cut into `units` equal ranges
    (`kvq_decode_units`)."""
    _require(kv_format in KV_FORMATS, f"unknown kv_format {kv_format!r}")
    _require(units >= 0, "units must be >= 0")
    _require(units == 0 or num_splits is None, "give num_splits or units, not both")
    B, Hq, D = q.shape
    _, block_size, Hkv, Dc = k_cache.shape
    quant = kv_format != "fp16"
    _require(q.dtype == torch.float16, "q must be float16")
    if quant:
        _require(k_cache.dtype == v_cache.dtype == torch.uint8,
                 "quantized caches hold uint8 codes")
        _require(Dc == (D // 2 if kv_format == "int4" else D),
                 "code cache last dim must be head_dim (head_dim/2 for int4)")
        check_scale_pairs(k_scale, k_zero, (k_cache.shape[0], Hkv, D), "k")
        check_scale_pairs(v_scale, v_zero, (k_cache.shape[0], Hkv, v_group_tokens(block_size)),
                          "v")
    else:
        _require(k_cache.dtype == v_cache.dtype == torch.float16,
                 "q, k_cache and v_cache must all be float16")
        _require(Dc == D, "cache head_dim must match q")
    _require(tuple(v_cache.shape) == tuple(k_cache.shape), "k_cache and v_cache shapes differ")
    _require(Hq % Hkv == 0, "q heads must be a multiple of kv heads")
    _require(_is_pow2(D) and D >= 16, "head_dim must be a power of two >= 16")
    _require(_is_pow2(block_size) and block_size >= 16, "block_size must be a power of two >= 16")
    _require(q.stride(2) == k_cache.stride(3) == v_cache.stride(3) == 1,
             "innermost dimension of q and the caches must be contiguous")
    _require(block_table.dtype == seq_lens.dtype == torch.int32,
             "block_table and seq_lens must be int32")
    _require(block_table.dim() == 2 and block_table.shape[0] == B and block_table.stride(1) == 1,
             "block_table must be [B, max_blocks] with contiguous rows")
    _require(seq_lens.shape == (B,) and seq_lens.is_contiguous(), "seq_lens must be [B] contiguous")
    dev = q.device
    _require(dev.type == "cuda", "kvq runs on the GPU only (no CPU fallback)")
    for t in (k_cache, v_cache, block_table, seq_lens):
        _require(t.device == dev, "all tensors must be on the same device")
    if check_seq_lens:  # the reference's per-call sync (triton_fp16.py:201), opt-in here
        _require(int(seq_lens.min()) >= 1, "empty sequences are not supported")
    if scale is None:
        scale = 1.0 / math.sqrt(D)

    if q.stride(0) % 8 or q.stride(1) % 8 or q.data_ptr() % 16:
        q = q.contiguous()  # 16-byte aligned rows for the kernel's vector loads
    if out is None:
        out = torch.empty((B, Hq, D), dtype=torch.float16, device=dev)
    else:
        _require(out.shape == (B, Hq, D) and out.dtype == torch.float16 and out.stride(2) == 1,
                 "out must be float16 [B, Hq, D] with a contiguous last dim")

    max_pages = block_table.shape[1]
    grid_heads = Hkv * head_blocks(Hq, Hkv)  # the plans count the kernels' kv heads
    if num_splits is None and units == 0:
        units, planned_waves = plan_units(B, grid_heads, block_size, max_pages,
                                          _sm_count(dev.index or 0), kv_format, D, Hq)
        if units > 0 and waves_per_group == 0:
            waves_per_group = planned_waves
    if units > 0:
        args = build_args(q, k_cache, v_cache, block_table, seq_lens, out, scale, kv_format,
                          k_scale, k_zero, v_scale, v_zero, k_group, waves_per_group, pipeline)
        if workspace is None:
            o_shape, l_shape = units_workspace_shapes(B, Hq, D, units)
            o_part = torch.empty(o_shape, dtype=torch.float32, device=dev)
            lse = torch.empty(l_shape, dtype=torch.float32, device=dev)
        else:
            o_part, lse = workspace
            _require(o_part.dtype == lse.dtype == torch.float32 and o_part.is_contiguous()
                     and lse.is_contiguous() and o_part.device == dev and lse.device == dev,
                     "workspace must be contiguous float32 on the op's device")
            _require(o_part.numel() >= Hq * (units + B) * D and lse.numel() >= Hq * (units + B),
                     f"workspace too small for {units} units")
        _lib.check("kvq_decode_units",
                   _lib.lib().kvq_decode_units(ctypes.byref(args), units, o_part.data_ptr(),
                                               lse.data_ptr(), _stream(dev)))
        return out
    if num_splits is None:
        splits, planned_waves = plan_decode(B, grid_heads, block_size, max_pages,
                                            _sm_count(dev.index or 0), kv_format, D, Hq)
        if waves_per_group == 0:
            waves_per_group = planned_waves
    else:
        splits = num_splits
    splits, pps = normalize_splits(splits, max_pages)
    args = build_args(q, k_cache, v_cache, block_table, seq_lens, out, scale, kv_format,
                      k_scale, k_zero, v_scale, v_zero, k_group, waves_per_group, pipeline)
    L = _lib.lib()
    stream = _stream(dev)
    if splits == 1:
        _lib.check("kvq_decode_single", L.kvq_decode_single(ctypes.byref(args), stream))
        return out
    if workspace is None:
        o_shape, l_shape = workspace_shapes(B, Hq, D, splits)
        o_part = torch.empty(o_shape, dtype=torch.float32, device=dev)
        lse = torch.empty(l_shape, dtype=torch.float32, device=dev)
    else:
        o_part, lse = workspace
        _require(o_part.dtype == lse.dtype == torch.float32 and o_part.is_contiguous()
                 and lse.is_contiguous() and o_part.device == dev and lse.device == dev,
                 "workspace must be contiguous float32 on the op's device")
        _require(o_part.numel() >= B * Hq * splits * D and lse.numel() >= B * Hq * splits,
                 f"workspace too small for {splits} splits")
    _lib.check("kvq_decode_split",
               L.kvq_decode_split(ctypes.byref(args), splits, pps, o_part.data_ptr(),
                                  lse.data_ptr(), stream))
    _lib.check("kvq_decode_merge",
               L.kvq_decode_merge(o_part.data_ptr(), lse.data_ptr(), out.data_ptr(),
                                  out.stride(0), out.stride(1), B, Hq, D, splits, stream))
    return out


def paged_decode_split(q, k_cache, v_cache, block_table, seq_lens, scale, num_splits,
                       pages_per_split, **fmt):
    """Stage 1 only (reference _split_kernel, triton_fp16.py:83-144): returns
    (o_part [B, Hq, S, D] float32, lse [B, Hq, S] float32). Used by the parity tests."""
    B, Hq, D = q.shape
    o_part = torch.empty((B, Hq, num_splits, D), dtype=torch.float32, device=q.device)
    lse = torch.empty((B, Hq, num_splits), dtype=torch.float32, device=q.device)
    args = build_args(q, k_cache, v_cache, block_table, seq_lens, None, scale, **fmt)
    _lib.check("kvq_decode_split",
               _lib.lib().kvq_decode_split(ctypes.byref(args), num_splits, pages_per_split,
                                           o_part.data_ptr(), lse.data_ptr(), _stream(q.device)))
    return o_part, lse
