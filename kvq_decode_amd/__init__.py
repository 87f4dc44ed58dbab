"""kvq_decode_amd - MI355X (gfx950) paged-KV GQA decode attention.

A from-scratch HIP implementation of the decode hot path of pawaryd/kvq-decode (`bpt`):
the split-KV decode kernel, the partial-softmax merge and KIVI-quantized KV, behind the
reference's call signature (src/bpt/triton_fp16.py:183-191) and a C ABI (include/kvq.h).
"""
from kvq_decode_amd.ops import (  # noqa: F401
    MIN_TOKENS_PER_SPLIT,
    TARGET_PROGRAMS_PER_SM,
    KvqArgumentError,
    _sm_count,
    choose_num_splits,
    head_blocks,
    normalize_splits,
    paged_decode_attention,
    plan_decode,
    plan_units,
    plan_workspace_shapes,
    units_workspace_shapes,
    workspace_shapes,
)
from kvq_decode_amd._lib import KvqError, version  # noqa: F401
from kvq_decode_amd import library  # noqa: F401  (registers torch.ops.kvq.*)

__all__ = [
    "paged_decode_attention",
    "choose_num_splits",
    "head_blocks",
    "normalize_splits",
    "workspace_shapes",
    "units_workspace_shapes",
    "plan_workspace_shapes",
    "plan_decode",
    "plan_units",
    "TARGET_PROGRAMS_PER_SM",
    "MIN_TOKENS_PER_SPLIT",
    "KvqArgumentError",
    "KvqError",
    "version",
]
