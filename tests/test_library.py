"""torch.library registration and the fp16 append ABI, on the CPU (no GPU touched).

Covers: every kvq op is registered with the schema its mutations need, the fake kernels
propagate shapes (meta tensors), CPU tensors raise instead of falling back, and
kvq_append_kv / kvq_reshape_and_cache reject bad arguments with the documented status
before any HIP call."""
import ctypes

import pytest
import torch

import kvq_decode_amd  # noqa: F401  (registers torch.ops.kvq.*)
from kvq_decode_amd import KvqArgumentError, _lib
from kvq_decode_amd._lib import DecodeArgs

OPS = {
    "paged_decode": (),
    "paged_decode_out": ("out",),
    "append_kv": ("k_cache", "v_cache"),
    "reshape_and_cache": ("k_cache", "v_cache"),
    "quantize_append": ("k_codes", "v_codes", "k_sz", "v_sz", "k_resid"),
}


@pytest.mark.parametrize("name", sorted(OPS))
def test_ops_registered_with_mutations_in_schema(name):
    schema = getattr(torch.ops.kvq, name).default._schema
    written = tuple(a.name for a in schema.arguments
                    if a.alias_info is not None and a.alias_info.is_write)
    assert written == OPS[name], str(schema)


def meta_inputs(B=3, Hq=8, Hkv=2, D=128, nb=12, bs=16, mb=4):
    m = dict(device="meta")
    return (torch.empty(B, Hq, D, dtype=torch.float16, **m),
            torch.empty(nb, bs, Hkv, D, dtype=torch.float16, **m),
            torch.empty(nb, bs, Hkv, D, dtype=torch.float16, **m),
            torch.empty(B, mb, dtype=torch.int32, **m),
            torch.empty(B, dtype=torch.int32, **m))


def test_fake_kernels_propagate_shapes():
    q, kc, vc, bt, sl = meta_inputs()
    out = torch.ops.kvq.paged_decode(q, kc, vc, bt, sl, None, 4)
    assert out.shape == q.shape and out.dtype == torch.float16 and out.device.type == "meta"
    ksz = torch.empty(12, 2, 128, 2, dtype=torch.float16, device="meta")
    vsz = torch.empty(12, 2, 16, 2, dtype=torch.float16, device="meta")
    codes = torch.empty(12, 16, 2, 64, dtype=torch.uint8, device="meta")
    out = torch.ops.kvq.paged_decode(q, codes, codes, bt, sl, None, None, "int4", ksz, vsz)
    assert out.shape == q.shape
    assert torch.ops.kvq.paged_decode_out(q, kc, vc, bt, sl, torch.empty_like(q)) is None
    kn = torch.empty(3, 2, 128, dtype=torch.float16, device="meta")
    assert torch.ops.kvq.append_kv(kc, vc, kn, kn, bt, sl) is None


def test_cpu_tensors_raise():
    """No CPU kernel is registered: a CPU call fails loudly, it is never computed."""
    q = torch.zeros(2, 8, 128, dtype=torch.float16)
    kc = torch.zeros(4, 16, 2, 128, dtype=torch.float16)
    bt = torch.zeros(2, 4, dtype=torch.int32)
    sl = torch.ones(2, dtype=torch.int32)
    with pytest.raises(NotImplementedError):
        torch.ops.kvq.paged_decode(q, kc, kc, bt, sl)
    with pytest.raises(NotImplementedError):
        torch.ops.kvq.append_kv(kc, kc, q[:, :2], q[:, :2], bt, sl)
    from kvq_decode_amd.cache import append_kv, reshape_and_cache
    with pytest.raises(KvqArgumentError, match="GPU only"):
        append_kv(kc, kc, q[:, :2].contiguous(), q[:, :2].contiguous(), bt, sl)
    with pytest.raises(KvqArgumentError, match="GPU only"):
        reshape_and_cache(q[:, :2], q[:, :2], kc, kc, torch.zeros(2, dtype=torch.int64))


def cache_args():
    """Fake (never dereferenced) aligned pointers describing two fp16 caches."""
    a = DecodeArgs()
    base = 1 << 40
    a.k_cache, a.k_stride_blk, a.k_stride_tok, a.k_stride_head = base, 16 * 8 * 128, 8 * 128, 128
    a.v_cache, a.v_stride_blk, a.v_stride_tok, a.v_stride_head = base + (1 << 30), 16 * 8 * 128, 8 * 128, 128
    a.block_table, a.bt_stride_b = base + (2 << 30), 64
    a.seq_lens = base + (3 << 30)
    a.batch, a.kv_heads, a.head_dim = 2, 8, 128
    a.block_size, a.max_blocks, a.num_blocks = 16, 64, 128
    a.kv_format = 0
    return a


NEW = (1 << 40) + (4 << 30)

APPEND_BAD = [
    ("kv_format", 3, _lib.KVQ_ERR_FORMAT),       # quantized caches append via quantize_append
    ("k_cache", 0, _lib.KVQ_ERR_NULL_POINTER),
    ("block_table", 0, _lib.KVQ_ERR_NULL_POINTER),
    ("seq_lens", 0, _lib.KVQ_ERR_NULL_POINTER),
    ("batch", 0, _lib.KVQ_ERR_SHAPE),
    ("head_dim", 96, _lib.KVQ_ERR_SHAPE),
    ("block_size", 24, _lib.KVQ_ERR_SHAPE),
    ("bt_stride_b", 32, _lib.KVQ_ERR_SHAPE),     # rows overlap
    ("v_cache", (1 << 40) + (1 << 30) + 8, _lib.KVQ_ERR_ALIGNMENT),
    ("k_stride_tok", 8 * 128 + 4, _lib.KVQ_ERR_ALIGNMENT),
    ("v_stride_blk", -8, _lib.KVQ_ERR_SHAPE),
]


@pytest.mark.parametrize("field,value,status", APPEND_BAD)
def test_append_kv_rejects(field, value, status):
    a = cache_args()
    setattr(a, field, value)
    assert _lib.lib().kvq_append_kv(ctypes.byref(a), NEW, NEW + (1 << 20), None) == status


def test_append_kv_rejects_bad_new_rows():
    L = _lib.lib()
    a = cache_args()
    assert L.kvq_append_kv(ctypes.byref(a), 0, NEW, None) == _lib.KVQ_ERR_NULL_POINTER
    assert L.kvq_append_kv(ctypes.byref(a), NEW + 2, NEW, None) == _lib.KVQ_ERR_ALIGNMENT


def test_reshape_and_cache_rejects():
    L = _lib.lib()
    a = cache_args()
    slots = NEW + (2 << 20)
    call = lambda a, st, sh, sm, n: L.kvq_reshape_and_cache(  # noqa: E731
        ctypes.byref(a), NEW, NEW + (1 << 20), st, sh, sm, n, None)
    assert call(a, 3 * 8 * 128, 128, 0, 4) == _lib.KVQ_ERR_NULL_POINTER
    assert call(a, 3 * 8 * 128, 128, slots, -1) == _lib.KVQ_ERR_SHAPE
    assert call(a, 3 * 8 * 128 + 4, 128, slots, 4) == _lib.KVQ_ERR_ALIGNMENT
    assert call(a, 3 * 8 * 128, -128, slots, 4) == _lib.KVQ_ERR_SHAPE
    b = cache_args()
    b.kv_format = 1
    assert call(b, 3 * 8 * 128, 128, slots, 4) == _lib.KVQ_ERR_FORMAT
    # no rows: nothing to launch, success without touching the device
    assert call(a, 3 * 8 * 128, 128, slots, 0) == _lib.KVQ_OK
