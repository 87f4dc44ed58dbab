"""The C ABI (include/kvq.h) on the CPU: the library loads, exports exactly the functions
the header declares, computes the split heuristic/normalization, and rejects bad
arguments with the documented status before any HIP call. No GPU is touched: every
rejected call below breaks exactly one precondition, so no launch is ever reached."""
import ctypes
import json
import os
import re
import subprocess

import pytest

from kvq_decode_amd import _lib
from kvq_decode_amd._lib import DecodeArgs

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(REPO, "include", "kvq.h")
GOLDEN = os.path.join(REPO, "tests", "golden", "reference_known_answers.json")


def declared_functions():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:int|const char\*)\s+(kvq_\w+)\s*\(", text, re.M)))


def test_library_exports_every_declared_symbol():
    names = declared_functions()
    assert names == sorted(_lib.EXPORTED_SYMBOLS)
    L = _lib.lib()
    for n in names:
        assert hasattr(L, n), n
    out = subprocess.run(["nm", "-D", "--defined-only", _lib.LIB_PATH], capture_output=True,
                         text=True).stdout
    exported = sorted(set(re.findall(r"\bT (kvq_\w+)$", out, re.M)))
    assert exported == names
    # and no other C-linkage function (C++ helpers are mangled, runtime symbols start with _)
    c_functions = sorted(set(re.findall(r"\bT ([A-Za-z]\w*)$", out, re.M)))
    assert c_functions == names, sorted(set(c_functions) - set(names))


def test_struct_layout_matches_header():
    """ctypes mirror of kvq_decode_args: same field names in the same order."""
    text = open(HEADER).read()
    body = text[text.index("typedef struct kvq_decode_args {"):text.index("} kvq_decode_args;")]
    body = re.sub(r"/\*.*?\*/", "", body, flags=re.S)
    fields = []
    for line in body.splitlines()[1:]:
        line = line.strip().rstrip(";")
        if not line:
            continue
        line = re.sub(r"^(const\s+)?(void|int64_t|int32_t|float|int32_t)\s*\*?\s*", "", line)
        fields += [f.strip().lstrip("*") for f in line.split(",")]
    assert fields == [f[0] for f in DecodeArgs._fields_]


def test_struct_abi_matches_c_compiler(tmp_path):
    """Offsets, sizes and total size of kvq_decode_args as gcc lays it out from the header
    (tests/cpu_checks/abi_layout.c) equal the ctypes mirror's: a type change in the header
    (int32 -> int64, a field inserted) would misalign every call, even with the names and
    their order unchanged."""
    exe = tmp_path / "abi_layout"
    subprocess.run(["gcc", "-std=c99", "-Wall", "-Werror", f"-I{os.path.join(REPO, 'include')}",
                    os.path.join(REPO, "tests", "cpu_checks", "abi_layout.c"), "-o", str(exe)],
                   check=True)
    lines = subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.split("\n")
    c_fields = [ln.split() for ln in lines if ln and not ln.startswith("sizeof")]
    c_size = int([ln for ln in lines if ln.startswith("sizeof")][0].split()[1])
    py = [(name, getattr(DecodeArgs, name).offset, getattr(DecodeArgs, name).size)
          for name, _ in DecodeArgs._fields_]
    assert [(n, int(o), int(s)) for n, o, s in c_fields] == py
    assert c_size == ctypes.sizeof(DecodeArgs)


def test_version_and_status_strings():
    assert _lib.version().startswith("kvq ")
    L = _lib.lib()
    assert L.kvq_status_string(0) == b"ok"
    assert L.kvq_status_string(-3) == b"unsupported configuration"


def test_cache_format_version():
    """The header's format version, the library's and the Python package's agree."""
    from kvq_decode_amd.quant import CACHE_FORMAT_VERSION, cache_format_version
    header = open(os.path.join(os.path.dirname(__file__), "..", "include", "kvq.h")).read()
    m = re.search(r"#define KVQ_CACHE_FORMAT_VERSION (\d+)", header)
    assert m and int(m.group(1)) == cache_format_version() == CACHE_FORMAT_VERSION


@pytest.mark.parametrize("q_heads,kv_heads,blocks", [
    (32, 8, 1), (128, 8, 1), (16, 1, 1),   # up to 16 q heads per kv head: one block
    (32, 1, 2), (48, 2, 2), (40, 2, 2),     # 32, 24, 20 -> blocks of 16, 12, 10
    (48, 1, 3), (34, 1, 17), (71, 1, 71),   # 48 -> 16; 34 = 2 x 17 -> 2; 71 prime -> 1
    (64, 1, 4), (256, 2, 8),
])
def test_head_blocks(q_heads, kv_heads, blocks):
    """A group G > 16 runs as k blocks of G / k q heads, k the smallest divisor of G with
    G / k <= 16 (checked here against a brute-force search)."""
    G = q_heads // kv_heads
    want = min(k for k in range(1, G + 1) if G % k == 0 and G // k <= 16)
    assert want == blocks
    assert _lib.lib().kvq_head_blocks(q_heads, kv_heads) == blocks
    from kvq_decode_amd import head_blocks
    assert head_blocks(q_heads, kv_heads) == blocks


def test_head_blocks_rejects_and_grid_limit():
    L = _lib.lib()
    for qh, kvh in ((30, 8), (0, 1), (8, 0), (4, 8)):
        assert L.kvq_head_blocks(qh, kvh) == _lib.KVQ_ERR_SHAPE
    a = good_args()
    a.q_heads, a.kv_heads = 71 * 1000, 1000  # 71 blocks per kv head: 71000 grid kv heads
    assert L.kvq_decode_single(ctypes.byref(a), None) == _lib.KVQ_ERR_UNSUPPORTED


def test_choose_num_splits_known_answers():
    """The reference's own recorded auto split counts (results/*.json, A100 108 SMs and
    T4 40 SMs, block_size 32) from its heuristic (triton_fp16.py:175-180)."""
    L = _lib.lib()
    rows = json.load(open(GOLDEN))["auto_splits"]
    assert len(rows) == 16
    for r in rows:
        got = L.kvq_choose_num_splits(r["batch"], 8, r["block_size"], r["ctx"] // r["block_size"],
                                      r["sms"], 8, 512)
        assert got == r["auto_splits"], r


def test_plan_decode():
    """The MI355X planner's choices for the benchmark shapes (256 CUs, 8 kv heads, block
    16), its caps, and its argument errors."""
    from kvq_decode_amd.ops import plan_decode
    cases = [  # batch, max_pages, format -> (splits, waves)
        (8, 2048, "fp16", (4, 2)),      # 2 waves/CU: 8 per (sequence, kv head)
        (16, 2048, "fp16", (2, 2)),
        (1, 8192, "fp16", (32, 2)),     # 64 per pair
        (64, 2048, "fp16", (2, 2)),     # raised to 4 per pair: <= 512 chunks per wave
        (16, 2048, "int4", (8, 2)),     # INT4: 8 waves per CU, 16 per pair
        (16, 2048, "int8", (8, 1)),     # INT8 / FP8: 4 waves per CU, single-wave workgroups
        (64, 2048, "int8", (8, 4)),     # 512 pairs > 256 CUs: 64-chunk partitions, 4 waves
        (1, 4096, "int4", (32, 8)),     # 256 per pair: 8 waves per workgroup (INT4 cap)
        (1, 4096, "int8", (32, 4)),     # 128 per pair: 4 waves per workgroup (INT8 cap)
        (8, 2048, "int4", (8, 4)),      # 32 per pair
        (8, 2048, "fp8_e4m3", (8, 2)),  # 16 per pair
        (64, 64, "fp16", (1, 1)),       # 1 per pair from 2 waves/CU
        (2, 3, "fp16", (1, 1)),         # at least 4 chunks per wave
    ]
    for batch, pages, fmt, want in cases:
        assert plan_decode(batch, 8, 16, pages, 256, fmt) == want, (batch, pages, fmt)
    assert plan_decode(1, 8, 32, 4096, 256, "fp16") == (32, 2)  # 2 chunks per page
    L = _lib.lib()
    s, w = ctypes.c_int32(), ctypes.c_int32()
    assert L.kvq_plan_decode(0, 32, 8, 16, 64, 0, 128, 256, ctypes.byref(s), ctypes.byref(w)) == \
        _lib.KVQ_ERR_SHAPE
    assert L.kvq_plan_decode(1, 32, 8, 16, 64, 7, 128, 256, ctypes.byref(s), ctypes.byref(w)) == \
        _lib.KVQ_ERR_FORMAT
    assert L.kvq_plan_decode(1, 32, 8, 24, 64, 0, 128, 256, ctypes.byref(s), ctypes.byref(w)) == \
        _lib.KVQ_ERR_SHAPE
    assert L.kvq_plan_decode(1, 32, 8, 16, 64, 0, 128, 256, None, ctypes.byref(w)) == \
        _lib.KVQ_ERR_NULL_POINTER
    for hd in (0, 24, -64):  # head_dim: a power of two >= 16
        assert L.kvq_plan_decode(1, 32, 8, 16, 64, 0, hd, 256, ctypes.byref(s),
                                 ctypes.byref(w)) == _lib.KVQ_ERR_SHAPE, hd


def test_plan_head_dims():
    """Head dims below 128 get 128 / head_dim times the waves per CU (16 and 32, whose rows
    share lines between kv heads: 64 / head_dim) in the work-unit plan (fp16 and INT4 unit
    workgroups of up to 4 waves) and, for fp16 only, in the split plan (workgroups of up to
    4); 256 keeps the 128 plan."""
    from kvq_decode_amd.ops import plan_decode, plan_units
    decode_cases = [  # batch, max_pages, format, head_dim -> (splits, waves)
        (8, 2048, "fp16", 64, (4, 4)),    # 4 waves per CU: 16 per pair
        (8, 2048, "fp16", 32, (4, 4)),    # 4 waves per CU: 16 per pair
        (8, 2048, "fp16", 16, (8, 4)),    # 8 waves per CU: 32 per pair
        (8, 2048, "fp16", 256, (4, 2)),   # as at 128
        (16, 2048, "int8", 64, (8, 1)),   # quantized split plans: as at 128
        (16, 2048, "int4", 64, (8, 2)),
        (16, 2048, "int4", 256, (8, 2)),
    ]
    for batch, pages, fmt, hd, want in decode_cases:
        assert plan_decode(batch, 8, 16, pages, 256, fmt, hd) == want, (batch, fmt, hd)
    units_cases = [  # batch, max_pages, format, head_dim -> (units, waves)
        (8, 2048, "fp16", 64, (32, 4)),    # 4 waves per CU in 4-wave workgroups
        (8, 2048, "fp16", 32, (32, 4)),    # 4 waves per CU
        (8, 2048, "fp16", 16, (64, 4)),    # 8 waves per CU
        (8, 2048, "fp16", 256, (32, 2)),   # as at 128
        (64, 2048, "int4", 64, (128, 4)),  # 16 waves per CU
        (16, 2048, "int8", 64, (64, 4)),   # 8 waves per CU
        (16, 2048, "fp8_e4m3", 256, (32, 4)),
    ]
    for batch, pages, fmt, hd, want in units_cases:
        assert plan_units(batch, 8, 16, pages, 256, fmt, hd) == want, (batch, fmt, hd)
    # the default argument is head_dim 128
    assert plan_units(8, 8, 16, 2048, 256, "fp16") == plan_units(8, 8, 16, 2048, 256, "fp16", 128)


def test_plan_units():
    """The work-unit plan is chosen for batches of 2 to 1024 whose split plan splits or
    whose longest context is at least 4096 tokens:
    2 waves per CU in 2-wave unit workgroups (fp16), 4 in 4-wave workgroups (INT8, FP8),
    8 in 2-wave workgroups (INT4); else (0, 0)."""
    from kvq_decode_amd.ops import plan_units
    cases = [  # batch, max_pages, format -> (units, waves)
        (8, 2048, "fp16", (32, 2)),     # C2: 32 units x 8 kv heads x 2 waves = 2 per CU
        (16, 2048, "fp16", (32, 2)),
        (64, 2048, "int4", (128, 2)),   # C5: 8 waves per CU
        (16, 2048, "int8", (32, 4)),    # C4: 4 waves per CU
        (16, 2048, "fp8_e4m3", (32, 4)),
        (1, 8192, "fp16", (0, 0)),      # one sequence: the split plan
        (64, 64, "fp16", (0, 0)),       # a single pass over 1024-token contexts
        (64, 256, "fp16", (32, 2)),     # a single pass in the split plan, 4096 tokens
        (64, 255, "fp16", (0, 0)),
        (1024, 256, "fp16", (32, 2)),   # the largest batch one workgroup's prefix table holds
        (1025, 2048, "fp16", (0, 0)),   # beyond it
    ]
    for batch, pages, fmt, want in cases:
        assert plan_units(batch, 8, 16, pages, 256, fmt) == want, (batch, pages, fmt)
    assert plan_units(8, 32, 16, 2048, 256, "fp16") == (8, 2)   # MHA: 32 kv heads
    assert plan_units(8, 1, 16, 2048, 256, "fp16") == (256, 2)  # MQA
    L = _lib.lib()
    u, w = ctypes.c_int32(), ctypes.c_int32()
    assert L.kvq_plan_units(0, 32, 8, 16, 64, 0, 128, 256, ctypes.byref(u), ctypes.byref(w)) == \
        _lib.KVQ_ERR_SHAPE
    assert L.kvq_plan_units(2, 32, 8, 16, 64, 7, 128, 256, ctypes.byref(u), ctypes.byref(w)) == \
        _lib.KVQ_ERR_FORMAT
    assert L.kvq_plan_units(2, 32, 8, 16, 64, 0, 128, 256, None, ctypes.byref(w)) == \
        _lib.KVQ_ERR_NULL_POINTER


def test_plan_lds_budget():
    """The plans keep a workgroup's LDS within 64 KB: where the waves they would pick give
    a cross-wave combine larger than that (large q-head groups at head dim 256 or 16 q
    heads per kv head), they halve the waves and double the splits or units, so the waves
    per CU stay. LDS bytes (quantized) = 4 * (max(W*G*D + 32*W, W*D*(4 INT4 | 9 INT8)) +
    D*W) + 32*D."""
    from kvq_decode_amd.ops import plan_decode, plan_units
    # INT4, head_dim 256, 32 q / 4 kv heads, batch 1 x 32k: 512 waves per pair; 8-wave
    # workgroups would need 82944 B, 4-wave ones 45568 B
    assert plan_decode(1, 4, 16, 2048, 256, "int4", 256, q_heads=32) == (128, 4)
    assert plan_decode(1, 4, 16, 2048, 256, "int4", 256) == (64, 8)  # 1 q head per kv head
    # INT8, head_dim 256, 32 q / 2 kv heads: 4-wave workgroups need 78336 B, 2-wave 43264 B
    assert plan_units(16, 2, 16, 2048, 256, "int8", 256, q_heads=32) == (256, 2)
    assert plan_decode(1, 2, 16, 2048, 256, "int8", 256, q_heads=32) == (256, 2)
    # INT4, head_dim 128, 16 q heads per kv head, batch 1: 8 waves need 74752 B, 4 39424 B
    assert plan_decode(1, 8, 16, 2048, 256, "int4", 128, q_heads=128) == (64, 4)
    # the common shapes are unchanged (4 q heads per kv head)
    assert plan_decode(1, 8, 16, 4096, 256, "int4", 128, q_heads=32) == (32, 8)
    assert plan_units(8, 8, 16, 2048, 256, "fp16", 128, q_heads=32) == (32, 2)
    L = _lib.lib()
    s, w = ctypes.c_int32(), ctypes.c_int32()
    for hq, hkv in ((7, 8), (12, 8), (136, 8)):  # q_heads / kv_heads must be 1..16
        assert L.kvq_plan_decode(1, hq, hkv, 16, 64, 0, 128, 256, ctypes.byref(s),
                                 ctypes.byref(w)) == _lib.KVQ_ERR_SHAPE, (hq, hkv)
        assert L.kvq_plan_units(2, hq, hkv, 16, 64, 0, 128, 256, ctypes.byref(s),
                                ctypes.byref(w)) == _lib.KVQ_ERR_SHAPE, (hq, hkv)


def test_plan_workspace_shapes():
    """The workspace shapes the default plan needs: work units, splits, or none."""
    from kvq_decode_amd.ops import plan_workspace_shapes
    # C2: 32 units per kv head -> [Hq, units + B, D]
    assert plan_workspace_shapes(8, 32, 8, 128, 16, 2048, 256) == ((32, 40, 128), (32, 40))
    # one sequence: the split plan, 32 splits of 64k tokens
    assert plan_workspace_shapes(1, 32, 8, 128, 16, 4096, 256) == ((1, 32, 32, 128), (1, 32, 32))
    # a single pass over short contexts needs none
    assert plan_workspace_shapes(64, 32, 8, 128, 16, 64, 256) is None
    # head_dim 32: 4 waves per CU in 4-wave unit workgroups, 32 units per kv head
    assert plan_workspace_shapes(8, 32, 8, 32, 16, 2048, 256) == ((32, 40, 32), (32, 40))


def test_normalize_splits():
    L = _lib.lib()
    s, pps = ctypes.c_int32(), ctypes.c_int32()
    for n, pages, want in [(7, 3, (3, 1)), (32, 2048, (32, 64)), (5, 8, (4, 2)), (0, 4, (1, 4))]:
        assert L.kvq_normalize_splits(n, pages, ctypes.byref(s), ctypes.byref(pps)) == 0
        assert (s.value, pps.value) == want
    assert L.kvq_normalize_splits(4, 0, ctypes.byref(s), ctypes.byref(pps)) == _lib.KVQ_ERR_SHAPE


def good_args():
    """A fully valid argument block with fake (never dereferenced) 256-aligned pointers."""
    a = DecodeArgs()
    base = 1 << 40
    a.q, a.q_stride_b, a.q_stride_h = base, 32 * 128, 128
    a.k_cache, a.k_stride_blk, a.k_stride_tok, a.k_stride_head = base + (1 << 30), 16 * 8 * 128, 8 * 128, 128
    a.v_cache, a.v_stride_blk, a.v_stride_tok, a.v_stride_head = base + (2 << 30), 16 * 8 * 128, 8 * 128, 128
    a.block_table, a.bt_stride_b = base + (3 << 30), 64
    a.seq_lens = base + (4 << 30)
    a.out, a.o_stride_b, a.o_stride_h = base + (5 << 30), 32 * 128, 128
    a.batch, a.q_heads, a.kv_heads, a.head_dim = 2, 32, 8, 128
    a.block_size, a.max_blocks, a.num_blocks = 16, 64, 128
    a.scale = 0.088
    a.kv_format = 0
    a.k_group = 128
    return a


BAD_CASES = [
    ("q", 0, _lib.KVQ_ERR_NULL_POINTER),
    ("block_table", 0, _lib.KVQ_ERR_NULL_POINTER),
    ("out", 0, _lib.KVQ_ERR_NULL_POINTER),
    ("batch", 0, _lib.KVQ_ERR_SHAPE),
    ("q_heads", 30, _lib.KVQ_ERR_SHAPE),           # not a multiple of kv_heads
    ("head_dim", 96, _lib.KVQ_ERR_SHAPE),          # not a power of two (reference asserts too)
    ("head_dim", 512, _lib.KVQ_ERR_UNSUPPORTED),   # valid for the reference, not built here
    ("block_size", 8, _lib.KVQ_ERR_SHAPE),
    ("kv_format", 9, _lib.KVQ_ERR_FORMAT),
    ("kv_format", 1, _lib.KVQ_ERR_FORMAT),          # quantized without scale tensors
    ("q", (1 << 40) + 8, _lib.KVQ_ERR_ALIGNMENT),
    ("k_stride_tok", 8 * 128 + 4, _lib.KVQ_ERR_ALIGNMENT),
    ("k_stride_tok", 1 << 27, _lib.KVQ_ERR_UNSUPPORTED),   # 32-bit lane offsets
    ("waves_per_group", 3, _lib.KVQ_ERR_UNSUPPORTED),
    ("pipeline", 5, _lib.KVQ_ERR_UNSUPPORTED),
    ("k_stride_blk", 1 << 31, _lib.KVQ_ERR_UNSUPPORTED),   # 2^32-byte block stride
    ("v_stride_blk", -16 * 8 * 128, _lib.KVQ_ERR_UNSUPPORTED),
]


@pytest.mark.parametrize("field,value,status", BAD_CASES)
def test_single_pass_rejects(field, value, status):
    a = good_args()
    setattr(a, field, value)
    assert _lib.lib().kvq_decode_single(ctypes.byref(a), None) == status


def set_scale_pairs(a, base=1 << 43):
    """Fake (never dereferenced) interleaved (scale, zero) pair pointers."""
    a.k_scale, a.k_zero = base, base + 2
    a.v_scale, a.v_zero = base + (1 << 30), base + (1 << 30) + 2


def test_scale_pairs_must_interleave():
    """Quantized caches: each zero must be the fp16 right after its scale (interleaved
    pairs); separate scale and zero tensors are a format error."""
    L = _lib.lib()
    a = good_args()
    a.kv_format = 3
    set_scale_pairs(a)
    a.waves_per_group = 16  # unsupported for quantized: proves the pair check passed
    assert L.kvq_decode_single(ctypes.byref(a), None) == _lib.KVQ_ERR_UNSUPPORTED
    for field, value in (("k_zero", (1 << 43) + 16), ("v_zero", (1 << 43) + (1 << 30))):
        b = good_args()
        b.kv_format = 3
        set_scale_pairs(b)
        setattr(b, field, value)
        assert L.kvq_decode_single(ctypes.byref(b), None) == _lib.KVQ_ERR_FORMAT, field
        assert L.kvq_quantize_cache(ctypes.byref(b), 1 << 40, 1 << 40, 0, 0, 0, None) == \
            _lib.KVQ_ERR_FORMAT, field


def test_op_requires_interleaved_scale_pairs():
    """The Python op accepts scale / zero tensors only as views of one interleaved
    (scale, zero) tensor; separate tensors are rejected before any device work."""
    import torch
    from kvq_decode_amd import KvqArgumentError, paged_decode_attention
    nb, bs, hkv, d, B = 4, 16, 2, 128, 1
    q = torch.zeros(B, 4, d, dtype=torch.float16)
    kc = torch.zeros(nb, bs, hkv, d // 2, dtype=torch.uint8)
    bt = torch.zeros(B, nb, dtype=torch.int32)
    sl = torch.ones(B, dtype=torch.int32)
    ksz = torch.zeros(nb, hkv, d, 2, dtype=torch.float16)
    vsz = torch.zeros(nb, hkv, 32, 2, dtype=torch.float16)  # V groups of max(bs, 32) tokens
    good = dict(kv_format="int4", k_scale=ksz[..., 0], k_zero=ksz[..., 1],
                v_scale=vsz[..., 0], v_zero=vsz[..., 1])
    with pytest.raises(KvqArgumentError, match="GPU only"):  # the pair check passed
        paged_decode_attention(q, kc, kc, bt, sl, **good)
    per_page = torch.zeros(nb, hkv, bs, 2, dtype=torch.float16)  # the version-1 V layout
    with pytest.raises(KvqArgumentError, match="interleaved"):
        paged_decode_attention(q, kc, kc, bt, sl,
                               **dict(good, v_scale=per_page[..., 0], v_zero=per_page[..., 1]))
    bad = dict(good, k_scale=torch.zeros(nb, hkv, d, dtype=torch.float16),
               k_zero=torch.zeros(nb, hkv, d, dtype=torch.float16))
    with pytest.raises(KvqArgumentError, match="interleaved"):
        paged_decode_attention(q, kc, kc, bt, sl, **bad)
    swapped = dict(good, v_scale=vsz[..., 1], v_zero=vsz[..., 0])
    with pytest.raises(KvqArgumentError, match="interleaved"):
        paged_decode_attention(q, kc, kc, bt, sl, **swapped)


def test_quantized_tuning_limits():
    """Quantized kernels: up to 8 waves per workgroup and 1, 2 or 4 chunks in flight."""
    L = _lib.lib()
    for field, value in (("waves_per_group", 16), ("pipeline", 3), ("pipeline", 8)):
        a = good_args()
        a.kv_format = 3
        set_scale_pairs(a)
        setattr(a, field, value)
        assert L.kvq_decode_single(ctypes.byref(a), None) == _lib.KVQ_ERR_UNSUPPORTED, field


def test_quantized_head_dims():
    """Quantized caches: head_dim 64, 128 or 256 (fp16 takes 16-256); head_dim 256 takes
    rings of 1 or 2 chunks. A call whose arguments pass the checks reaches the split-count
    check (KVQ_ERR_SPLITS for num_splits 0)."""
    L = _lib.lib()
    op, lse = 1 << 41, 1 << 42
    for fmt in (1, 2, 3):
        for D, want in ((32, _lib.KVQ_ERR_UNSUPPORTED), (64, _lib.KVQ_ERR_SPLITS),
                        (128, _lib.KVQ_ERR_SPLITS), (256, _lib.KVQ_ERR_SPLITS)):
            a = good_args()
            a.kv_format = fmt
            set_scale_pairs(a)
            a.head_dim, a.q_stride_b, a.q_stride_h = D, 32 * D, D
            a.o_stride_b, a.o_stride_h = 32 * D, D
            assert L.kvq_decode_split(ctypes.byref(a), 0, 4, op, lse, None) == want, (fmt, D)
        a.pipeline = 4  # head_dim 256
        assert L.kvq_decode_split(ctypes.byref(a), 4, 16, op, lse, None) == \
            _lib.KVQ_ERR_UNSUPPORTED, fmt


def test_fp16_ring_depth_limits():
    """fp16: ring depth 1, 2 or 4 up to head_dim 128; head_dim 256 takes 1 or 2."""
    L = _lib.lib()
    a = good_args()
    a.head_dim, a.q_stride_b, a.q_stride_h = 256, 32 * 256, 256
    a.pipeline = 4
    assert L.kvq_decode_single(ctypes.byref(a), None) == _lib.KVQ_ERR_UNSUPPORTED


def test_split_rejects_bad_split_geometry():
    L = _lib.lib()
    a = good_args()
    op, lse = 1 << 41, 1 << 42
    assert L.kvq_decode_split(ctypes.byref(a), 0, 4, op, lse, None) == _lib.KVQ_ERR_SPLITS
    assert L.kvq_decode_split(ctypes.byref(a), 4, 8, op, lse, None) == _lib.KVQ_ERR_SPLITS  # 32 < 64 pages
    assert L.kvq_decode_split(ctypes.byref(a), 4, 16, 0, lse, None) == _lib.KVQ_ERR_NULL_POINTER
    assert L.kvq_decode_split(None, 4, 16, op, lse, None) == _lib.KVQ_ERR_NULL_POINTER


def test_units_reject():
    L = _lib.lib()
    a = good_args()
    op, lse = 1 << 41, 1 << 42
    for fn in (L.kvq_decode_units, L.kvq_decode_units_split, L.kvq_decode_units_merge):
        assert fn(ctypes.byref(a), 0, op, lse, None) == _lib.KVQ_ERR_SPLITS
        assert fn(ctypes.byref(a), 8, 0, lse, None) == _lib.KVQ_ERR_NULL_POINTER
        assert fn(None, 8, op, lse, None) == _lib.KVQ_ERR_NULL_POINTER
    a.batch = 1025  # one workgroup reads every seq_len of the batch
    assert L.kvq_decode_units(ctypes.byref(a), 8, op, lse, None) == _lib.KVQ_ERR_UNSUPPORTED
    # a kv head's chunks over the batch must stay below 2^31: 1024 x 2^21 chunks do not
    a.batch, a.max_blocks, a.num_blocks = 1024, 2**21, 2**22
    assert L.kvq_decode_units(ctypes.byref(a), 8, op, lse, None) == _lib.KVQ_ERR_UNSUPPORTED
    from kvq_decode_amd.ops import plan_units
    assert plan_units(1024, 8, 16, 2**21, 256, "fp16") == (0, 0)  # the split plan instead
    assert plan_units(1024, 8, 16, 2**21 - 1, 256, "fp16") == (32, 2)
    a.max_blocks, a.num_blocks = 64, 128
    a.batch = 2
    a.waves_per_group = 8  # unit workgroups: 1, 2 or 4 waves
    assert L.kvq_decode_units(ctypes.byref(a), 8, op, lse, None) == _lib.KVQ_ERR_UNSUPPORTED
    a.waves_per_group = 0
    a.kv_format = 3  # quantized without scale tensors
    assert L.kvq_decode_units(ctypes.byref(a), 8, op, lse, None) == _lib.KVQ_ERR_FORMAT


def test_merge_and_quantize_reject():
    L = _lib.lib()
    assert L.kvq_decode_merge(0, 1 << 41, 1 << 42, 128, 128, 1, 32, 128, 4, None) == \
        _lib.KVQ_ERR_NULL_POINTER
    assert L.kvq_decode_merge(1 << 40, 1 << 41, 1 << 42, 128, 128, 1, 32, 100, 4, None) == \
        _lib.KVQ_ERR_SHAPE
    a = good_args()  # kv_format fp16 is not a quantization target
    assert L.kvq_quantize_cache(ctypes.byref(a), 1 << 40, 1 << 40, 0, 0, 0, None) == \
        _lib.KVQ_ERR_FORMAT
    a.kv_format = 3
    set_scale_pairs(a)
    a.k_group = 100  # not a multiple of block_size
    assert L.kvq_quantize_cache(ctypes.byref(a), 1 << 40, 1 << 40, 0, 0, 0, None) == \
        _lib.KVQ_ERR_UNSUPPORTED
    a.k_group = 128
    assert L.kvq_quantize_append(ctypes.byref(a), 0, 1 << 40, 1 << 41, None) == \
        _lib.KVQ_ERR_NULL_POINTER


def test_quantizers_take_the_decode_head_dims():
    """The quantizers write exactly the head dims the quantized decode reads (64, 128,
    256): head_dim 32 (and 512) is KVQ_ERR_UNSUPPORTED for both the bulk quantizer and the
    append, as for the decode, so no cache can be built that no decode reads. Accepted
    head dims reach the next check (a null source pointer)."""
    L = _lib.lib()
    op, lse = 1 << 41, 1 << 42
    for fmt in (1, 2, 3):
        for D in (32, 512):
            a = good_args()
            a.kv_format = fmt
            set_scale_pairs(a)
            a.head_dim, a.q_stride_b, a.q_stride_h = D, 32 * D, D
            a.o_stride_b, a.o_stride_h = 32 * D, D
            assert L.kvq_quantize_cache(ctypes.byref(a), 1 << 40, 1 << 40, 0, 0, 0, None) == \
                _lib.KVQ_ERR_UNSUPPORTED, (fmt, D)
            assert L.kvq_quantize_append(ctypes.byref(a), 1 << 40, 1 << 40, 1 << 41, None) == \
                _lib.KVQ_ERR_UNSUPPORTED, (fmt, D)
            assert L.kvq_decode_split(ctypes.byref(a), 4, 16, op, lse, None) == \
                _lib.KVQ_ERR_UNSUPPORTED, (fmt, D)
        for D in (64, 128, 256):
            a = good_args()
            a.kv_format = fmt
            set_scale_pairs(a)
            a.head_dim = D
            assert L.kvq_quantize_cache(ctypes.byref(a), 0, 1 << 40, 0, 0, 0, None) == \
                _lib.KVQ_ERR_NULL_POINTER, (fmt, D)
    from kvq_decode_amd.quant import allocate_quantized_cache
    from kvq_decode_amd.ops import KvqArgumentError
    with pytest.raises(KvqArgumentError):
        allocate_quantized_cache(4, 16, 2, 32, "int8", "cpu")


def test_python_op_argument_errors_and_no_cpu_fallback():
    """The host op raises the reference's AssertionError family for its preconditions
    (triton_fp16.py:195-201) and refuses CPU tensors instead of falling back."""
    import torch

    from kvq_decode_amd import KvqArgumentError, paged_decode_attention
    q = torch.zeros(2, 32, 128, dtype=torch.float16)
    kc = torch.zeros(8, 16, 8, 128, dtype=torch.float16)
    bt = torch.zeros(2, 4, dtype=torch.int32)
    sl = torch.ones(2, dtype=torch.int32)
    with pytest.raises(AssertionError):
        paged_decode_attention(q.float(), kc, kc, bt, sl)
    with pytest.raises(KvqArgumentError):
        paged_decode_attention(q, kc, kc, bt.long(), sl)
    with pytest.raises(KvqArgumentError):
        paged_decode_attention(q[:, :30], kc, kc, bt, sl)
    with pytest.raises(KvqArgumentError, match="not both"):
        paged_decode_attention(q, kc, kc, bt, sl, num_splits=2, units=8)
    with pytest.raises(KvqArgumentError, match="GPU only"):
        paged_decode_attention(q, kc, kc, bt, sl)


def test_static_entry_point_rejects_on_the_host():
    """kvq_paged_decode_static refuses, before touching a GPU, a workspace beyond its
    KVQ_STATIC_SCRATCH_BYTES buffer (64 x 32 heads x 32 splits x 129 floats = 33.8 MB) and
    negative unit counts; the header and the Python mirror agree on the buffer size."""
    header = open(HEADER).read()
    m = re.search(r"#define KVQ_STATIC_SCRATCH_BYTES \((\d+) \* (\d+) \* (\d+)\)", header)
    assert m and int(m.group(1)) * int(m.group(2)) * int(m.group(3)) == _lib.STATIC_SCRATCH_BYTES
    L = _lib.lib()
    a = good_args()
    a.batch = 64
    assert L.kvq_paged_decode_static(ctypes.byref(a), 32, 0, None) == _lib.KVQ_ERR_SCRATCH
    units = _lib.STATIC_SCRATCH_BYTES // (4 * 32 * 129)
    assert L.kvq_paged_decode_static(ctypes.byref(a), 0, units, None) == _lib.KVQ_ERR_SCRATCH
    assert L.kvq_paged_decode_static(ctypes.byref(a), 0, -1, None) == _lib.KVQ_ERR_SPLITS
    assert L.kvq_paged_decode_static(None, 4, 0, None) == _lib.KVQ_ERR_NULL_POINTER
    assert L.kvq_status_string(_lib.KVQ_ERR_SCRATCH) == \
        b"workspace exceeds the static scratch buffer"
