"""Algorithmic KV-read bytes of a decode step: the byte count every bandwidth figure of
this package (TB/s, % of the HBM peak, roofline.frac) divides by.

What is counted, and why it matches the reference's model (pawaryd/kvq-decode
src/bpt/roofline.py:1-9, 50-58) term for term, so that bandwidth figures compare across
the two projects:
  * only the KV cache: the query, the output, the block table and the split-KV partials
    are left out;
  * per context token and kv head: the K and V codes, 2 * head_dim * (bytes per code);
  * for formats with (scale, zero) pairs (fp16 each, 4 bytes a pair): one pair per
    channel per K group of `group_size` tokens for K, one pair per token for V.

Format keys are this library's kv_format names ('fp16', 'int8', 'fp8_e4m3', 'int4') plus
the reference's 'fp8', which its model prices as a bare one-byte cast without pairs. The
library's 'fp8_e4m3' cache carries pairs like INT8 and is priced that way.
"""
from typing import Dict, Iterable, NamedTuple, Tuple

HBM_PEAK_GBPS = 8000.0  # MI355X HBM3E, GB/s (1e9 bytes/s)

PAIR_BYTES = 4  # one fp16 scale and one fp16 zero

# kv format -> (bytes per code, carries (scale, zero) pairs)
KV_DTYPES: Dict[str, Tuple[float, bool]] = {
    "fp16": (2.0, False),
    "fp8": (1.0, False),      # the reference's plain-cast FP8 (no pairs)
    "fp8_e4m3": (1.0, True),  # this library's FP8 cache (KVQ_KV_FP8_E4M3)
    "int8": (1.0, True),
    "int4": (0.5, True),
}


class ModelShape(NamedTuple):
    layers: int
    q_heads: int
    kv_heads: int
    head_dim: int


# The attention shapes of the reference's model table (roofline.py:42-47), used for the
# whole-model decode step.
MODELS: Dict[str, ModelShape] = {
    "llama3-8b": ModelShape(32, 32, 8, 128),
    "llama3-70b": ModelShape(80, 64, 8, 128),
    "llama2-7b": ModelShape(32, 32, 32, 128),
    "qwen2.5-7b": ModelShape(28, 28, 4, 128),
}


def bytes_per_token_head(head_dim: int, kv_dtype: str, group_size: int = 128) -> float:
    """Bytes a decode reads for one context token of one kv head in one layer: K and V
    codes, plus, for paired formats, the token's V pair and its 1/group_size share of the
    K group's head_dim pairs. At head_dim 128 and groups of 128: fp16 512, int8 and
    fp8_e4m3 264, int4 136 (the reference's 'fp8': 256)."""
    code_bytes, paired = KV_DTYPES[kv_dtype]
    total = 2 * head_dim * code_bytes
    if paired:
        total += PAIR_BYTES * head_dim / group_size + PAIR_BYTES
    return total


def kv_bytes_per_token(model: ModelShape, kv_dtype: str, group_size: int = 128) -> float:
    """Bytes one decode step reads per context token across all of a model's layers
    (Llama-3-8B fp16: 128 KiB)."""
    return model.layers * model.kv_heads * bytes_per_token_head(model.head_dim, kv_dtype,
                                                                group_size)


def step_bytes(seq_lens: Iterable[int], kv_heads: int, head_dim: int, kv_dtype: str,
               group_size: int = 128) -> int:
    """Algorithmic bytes of one single-layer decode over a batch with these lengths."""
    th = sum(int(n) for n in seq_lens) * kv_heads
    return int(round(th * bytes_per_token_head(head_dim, kv_dtype, group_size)))


def min_time_us(nbytes: float, peak_gbps: float = HBM_PEAK_GBPS) -> float:
    """Time to move `nbytes` at the HBM peak: the roofline floor of a step, µs."""
    return nbytes / (peak_gbps * 1e9) * 1e6
