"""kvq_paged_decode_static, the allocation-free entry point, through the C ABI. Needs a GPU.

Its output must equal, bit for bit, that of the entry point it stands in for -
kvq_paged_decode (splits) or kvq_decode_units (work units) with a caller-allocated
workspace - on two calls in a row, the second with a smaller batch, so that a stale
workspace from the first call cannot pass unnoticed. The same kernels run on the same
inputs, and they are deterministic, so equality is exact. fp16 and INT4 caches.
"""
import ctypes

import numpy as np
import pytest
import torch

from kvq_decode_amd import _lib, ops
from oracle.attention import build_paged_cache

pytestmark = pytest.mark.gpu

HQ, HKV, D, BS = 32, 8, 128, 16


def make(lens, seed):
    rng = np.random.default_rng(seed)
    B, S = len(lens), max(lens)
    q = rng.standard_normal((B, HQ, D)).astype(np.float16)
    k = rng.standard_normal((B, S, HKV, D)).astype(np.float16)
    v = rng.standard_normal((B, S, HKV, D)).astype(np.float16)
    sl = np.array(lens, np.int32)
    kc, vc, bt = build_paged_cache(k, v, sl, BS, rng)
    return [torch.from_numpy(np.ascontiguousarray(a)).cuda() for a in (q, kc, vc, bt, sl)]


def decode_both(q, kc, vc, bt, sl, num_splits, units, fmt):
    """(existing entry point's output, static entry point's output)."""
    L = _lib.lib()
    stream = torch.cuda.current_stream().cuda_stream
    B = q.shape[0]
    outs = []
    for static in (False, True):
        out = torch.full_like(q, float("nan"))
        args = ops.build_args(q, kc, vc, bt, sl, out, 1.0 / np.sqrt(D), **fmt)
        if static:
            st = L.kvq_paged_decode_static(ctypes.byref(args), num_splits, units, stream)
            _lib.check("kvq_paged_decode_static", st)
        elif units:
            o_shape, l_shape = ops.units_workspace_shapes(B, HQ, D, units)
            o = torch.empty(o_shape, dtype=torch.float32, device="cuda")
            lse = torch.empty(l_shape, dtype=torch.float32, device="cuda")
            _lib.check("kvq_decode_units", L.kvq_decode_units(ctypes.byref(args), units,
                                                              o.data_ptr(), lse.data_ptr(), stream))
        else:
            s = ops.normalize_splits(num_splits, bt.shape[1])[0]
            o_shape, l_shape = ops.workspace_shapes(B, HQ, D, s)
            o = torch.empty(o_shape, dtype=torch.float32, device="cuda")
            lse = torch.empty(l_shape, dtype=torch.float32, device="cuda")
            _lib.check("kvq_paged_decode", L.kvq_paged_decode(ctypes.byref(args), num_splits,
                                                              o.data_ptr(), lse.data_ptr(), stream))
        torch.cuda.synchronize()
        outs.append(out)
    return outs


CALLS = [[3000, 1200, 4096, 17, 900, 2500, 64, 4000], [700, 33, 1500]]  # the second smaller


@pytest.mark.parametrize("fmt_name", ["fp16", "int4"])
@pytest.mark.parametrize("num_splits,units", [(8, 0), (3, 0), (1, 0), (0, 32), (0, 5)])
def test_static_equals_existing_entry_point(fmt_name, num_splits, units):
    from kvq_decode_amd.quant import quantize_paged_cache
    for i, lens in enumerate(CALLS):
        q, kc, vc, bt, sl = make(lens, seed=10 + i)
        fmt = {}
        if fmt_name != "fp16":
            qc = quantize_paged_cache(kc, vc, bt, sl, fmt_name)
            kc, vc, fmt = qc.k_codes, qc.v_codes, qc.decode_kwargs()
        print(f"\n[static {fmt_name} splits={num_splits} units={units} call {i} B={len(lens)}]",
              flush=True)
        want, got = decode_both(q, kc, vc, bt, sl, num_splits, units, fmt)
        assert not torch.isnan(want).any()
        assert torch.equal(got, want), f"call {i}: {(got != want).sum().item()} elements differ"


def test_static_rejects_a_workspace_beyond_the_buffer(cuda):
    """64 sequences x 32 q heads x 32 splits x 129 floats is 33.8 MB > 16 MiB: the call
    returns KVQ_ERR_SCRATCH before any launch and leaves the output untouched."""
    q, kc, vc, bt, sl = make([600] * 64, seed=3)
    out = torch.full_like(q, 7.0)
    args = ops.build_args(q, kc, vc, bt, sl, out, 1.0 / np.sqrt(D))
    L = _lib.lib()
    stream = torch.cuda.current_stream().cuda_stream
    assert L.kvq_paged_decode_static(ctypes.byref(args), 32, 0, stream) == _lib.KVQ_ERR_SCRATCH
    units = _lib.STATIC_SCRATCH_BYTES // (4 * HQ * (D + 1))  # units + 64 rows too many
    assert L.kvq_paged_decode_static(ctypes.byref(args), 0, units, stream) == \
        _lib.KVQ_ERR_SCRATCH
    torch.cuda.synchronize()
    assert bool((out == 7.0).all())
