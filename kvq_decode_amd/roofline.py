"""KV bytes read per decode step and the bandwidth-bound minimum time.

Restates the reference's byte model (pawaryd/kvq-decode src/bpt/roofline.py:1-67) with two
changes: MI355X is in the GPU table, and FP8 carries fp16 scale + zero like INT8 (this
build's FP8 format is KIVI-style with scales; the reference modelled FP8 as a plain cast,
roofline.py:9, 25). Only KV-cache reads are counted - q, the output, the block table and
the split-KV partials are excluded (roofline.py:1-4).
"""
from dataclasses import dataclass
from typing import Dict

# Peak HBM bandwidth, GB/s (1e9 B/s). The first four are the reference's (roofline.py:15-20).
GPUS: Dict[str, float] = {
    "T4": 320.0,
    "A100-80GB": 2039.0,
    "H100-SXM": 3350.0,
    "B200": 8000.0,
    "MI355X": 8000.0,
}

# (bytes per element, has scale/zero) - roofline.py:23-28, FP8 with scales here.
KV_DTYPES: Dict[str, tuple] = {
    "fp16": (2.0, False),
    "fp8_e4m3": (1.0, True),
    "int8": (1.0, True),
    "int4": (0.5, True),
}

SCALE_BYTES = 2   # fp16 (roofline.py:30)
ZP_PER_SCALE = 2  # scale + zero (roofline.py:31)


@dataclass(frozen=True)
class ModelShape:
    layers: int
    q_heads: int
    kv_heads: int
    head_dim: int


# roofline.py:42-47
MODELS: Dict[str, ModelShape] = {
    "llama3-8b": ModelShape(32, 32, 8, 128),
    "llama3-70b": ModelShape(80, 64, 8, 128),
    "llama2-7b": ModelShape(32, 32, 32, 128),
    "qwen2.5-7b": ModelShape(28, 28, 4, 128),
}


def bytes_per_token_head(head_dim: int, kv_dtype: str, group_size: int = 128) -> float:
    """KV bytes read per context token per kv head per layer: K + V payload plus, for
    quantized formats, K per-channel scale+zero amortized over `group_size` tokens and V
    per-token scale+zero (roofline.py:50-58)."""
    elem, quant = KV_DTYPES[kv_dtype]
    per_head = 2 * head_dim * elem
    if quant:
        per_head += head_dim * SCALE_BYTES * ZP_PER_SCALE / group_size
        per_head += SCALE_BYTES * ZP_PER_SCALE
    return per_head


def kv_bytes_per_token(shape: ModelShape, kv_dtype: str, group_size: int = 128) -> float:
    """KV bytes read per context token per decode step, summed over all layers."""
    return shape.layers * shape.kv_heads * bytes_per_token_head(shape.head_dim, kv_dtype,
                                                                group_size)


def bytes_per_step(shape: ModelShape, ctx: int, batch: int, kv_dtype: str,
                   group_size: int = 128) -> float:
    return kv_bytes_per_token(shape, kv_dtype, group_size) * ctx * batch


def min_time_ms(nbytes: float, gpu: str) -> float:
    return nbytes / (GPUS[gpu] * 1e9) * 1e3
