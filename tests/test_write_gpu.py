"""The KV write path and graph capture on the GPU. Needs a GPU.

  * kvq_append_kv: appending token n of every sequence to a cache that holds tokens
    0..n-1 gives exactly the cache the reference's builder (oracle build_paged_cache,
    reference.py:52-82) makes for tokens 0..n - every byte of both caches, garbage slots
    included, so nothing else is written;
  * kvq_reshape_and_cache: vLLM's slot-mapping scatter, padding rows (slot -1) and
    strided key/value views (slices of a fused qkv tensor) - bit-exact;
  * the torch.ops.kvq ops: opcheck (schema, fake kernel, tracing) and a decode step
    (append + decode, fp16 and INT4) captured in a torch.cuda.CUDAGraph and replayed
    several times with new inputs; every replay equals the same ops run eagerly on a
    mirror of the state, bit for bit, and the last one matches the oracle.
"""
import numpy as np
import pytest
import torch

from oracle import kivi
from oracle.attention import build_paged_cache, paged_decode_attention_ref

pytestmark = pytest.mark.gpu

ATOL, RTOL = 2e-3, 1e-2


def gpu(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def make(lens, Hq=8, Hkv=2, D=128, bs=16, seed=0, extra_blocks=0):
    """Builder caches for sequences of lengths `lens`; with extra_blocks > 0 every
    sequence's table row gets that many more (unused, in-pool) blocks to grow into."""
    rng = np.random.default_rng(seed)
    B, S = len(lens), max(lens) + extra_blocks * bs
    q = rng.standard_normal((B, Hq, D)).astype(np.float16)
    k = rng.standard_normal((B, S, Hkv, D)).astype(np.float16)
    v = rng.standard_normal((B, S, Hkv, D)).astype(np.float16)
    kc, vc, bt = build_paged_cache(k, v, np.array(lens, np.int32), bs, rng)
    return q, k, v, kc, vc, bt


def test_append_kv_matches_builder():
    from kvq_decode_amd.cache import append_kv
    lens = [1, 16, 17, 40, 100]  # after the append: page starts, page ends, mid-page
    q, k, v, kc, vc, bt = make(lens)
    kc0, vc0 = kc.copy(), vc.copy()
    B = len(lens)
    for b, n in enumerate(lens):  # the slot of token n-1 holds garbage before the append
        blk, off = bt[b, (n - 1) // 16], (n - 1) % 16
        kc0[blk, off] = 77.0
        vc0[blk, off] = -77.0
    kn = np.stack([k[b, n - 1] for b, n in enumerate(lens)])
    vn = np.stack([v[b, n - 1] for b, n in enumerate(lens)])
    kc_g, vc_g = gpu(kc0), gpu(vc0)
    append_kv(kc_g, vc_g, gpu(kn), gpu(vn), gpu(bt), gpu(np.array(lens, np.int32)))
    torch.cuda.synchronize()
    assert np.array_equal(kc_g.cpu().numpy().view(np.uint16), kc.view(np.uint16))
    assert np.array_equal(vc_g.cpu().numpy().view(np.uint16), vc.view(np.uint16))


def test_append_kv_out_of_range_writes_nothing():
    """A position past the block table, or a table entry outside the pool, is skipped by
    the kernel's own bounds checks."""
    from kvq_decode_amd.cache import append_kv
    q, k, v, kc, vc, bt = make([32, 20])
    bt = bt.copy()
    bt[1, 1] = kc.shape[0]  # sequence 1's second page points past the pool
    lens = np.array([bt.shape[1] * 16 + 1, 20], np.int32)  # sequence 0: past its table
    kc_g, vc_g = gpu(kc), gpu(vc)
    kn = torch.full((2, 2, 128), 5.0, dtype=torch.float16, device="cuda")
    append_kv(kc_g, vc_g, kn, kn, gpu(bt), gpu(lens))
    torch.cuda.synchronize()
    assert np.array_equal(kc_g.cpu().numpy().view(np.uint16), kc.view(np.uint16))
    assert np.array_equal(vc_g.cpu().numpy().view(np.uint16), vc.view(np.uint16))


def test_reshape_and_cache_slot_mapping():
    from kvq_decode_amd.cache import reshape_and_cache
    rng = np.random.default_rng(3)
    nb, bs, hkv, d, T = 20, 16, 2, 128, 37
    kc = rng.standard_normal((nb, bs, hkv, d)).astype(np.float16)
    vc = rng.standard_normal((nb, bs, hkv, d)).astype(np.float16)
    slots = rng.choice(nb * bs, T, replace=False).astype(np.int64)
    slots[[0, 5, 36]] = -1  # padding rows
    qkv = rng.standard_normal((T, 3 * hkv, d)).astype(np.float16)  # fused q | k | v
    qkv_g = gpu(qkv)
    key, value = qkv_g[:, hkv:2 * hkv], qkv_g[:, 2 * hkv:]
    assert not key.is_contiguous()
    kc_g, vc_g = gpu(kc), gpu(vc)
    reshape_and_cache(key, value, kc_g, vc_g, gpu(slots))
    torch.cuda.synchronize()
    want_k, want_v = kc.copy(), vc.copy()
    for t, s in enumerate(slots):
        if s >= 0:
            want_k[s // bs, s % bs] = qkv[t, hkv:2 * hkv]
            want_v[s // bs, s % bs] = qkv[t, 2 * hkv:]
    assert np.array_equal(kc_g.cpu().numpy().view(np.uint16), want_k.view(np.uint16))
    assert np.array_equal(vc_g.cpu().numpy().view(np.uint16), want_v.view(np.uint16))


def test_opcheck_paged_decode():
    import kvq_decode_amd  # noqa: F401
    q, k, v, kc, vc, bt = make([5, 70, 33])
    args = (gpu(q), gpu(kc), gpu(vc), gpu(bt), torch.tensor([5, 70, 33], dtype=torch.int32,
                                                            device="cuda"))
    for splits in (None, 1, 3):
        torch.library.opcheck(torch.ops.kvq.paged_decode.default, args + (None, splits))


def _graph_step(state, quant):
    """One decode step from torch.ops.kvq: append the new token, decode."""
    s = state
    if quant:
        torch.ops.kvq.quantize_append(s["kc"], s["vc"], s["ksz"], s["vsz"], s["kn"], s["vn"],
                                      s["bt"], s["sl"], s["resid"], "int4")
        return torch.ops.kvq.paged_decode(s["q"], s["kc"], s["vc"], s["bt"], s["sl"], None,
                                          None, "int4", s["ksz"], s["vsz"])
    torch.ops.kvq.append_kv(s["kc"], s["vc"], s["kn"], s["vn"], s["bt"], s["sl"])
    return torch.ops.kvq.paged_decode(s["q"], s["kc"], s["vc"], s["bt"], s["sl"])


@pytest.mark.parametrize("quant", [False, True], ids=["fp16", "int4"])
def test_graph_captured_decode_step(quant):
    import kvq_decode_amd  # noqa: F401
    from kvq_decode_amd.quant import (allocate_quantized_cache, init_k_residual,
                                      quantize_paged_cache)
    lens0 = [1, 127, 300, 1000]
    steps = 4
    Hq, Hkv, D, bs = 32, 8, 128, 16
    q, k, v, kc, vc, bt = make(lens0, Hq, Hkv, D, bs, seed=7, extra_blocks=1)
    rng = np.random.default_rng(11)
    sl0 = np.array(lens0, np.int32)
    kc_g, vc_g, bt_g = gpu(kc), gpu(vc), gpu(bt)

    def fresh_state():
        st = dict(q=gpu(q), bt=bt_g, sl=gpu(sl0),
                  kn=torch.zeros(len(lens0), Hkv, D, dtype=torch.float16, device="cuda"),
                  vn=torch.zeros(len(lens0), Hkv, D, dtype=torch.float16, device="cuda"))
        if quant:  # zeroed first: slots past the sequences compare equal too
            qc = allocate_quantized_cache(kc.shape[0], bs, Hkv, D, "int4", "cuda")
            for t in (qc.k_codes, qc.v_codes, qc.k_sz, qc.v_sz):
                t.zero_()
            qc = quantize_paged_cache(kc_g, vc_g, bt_g, st["sl"], "int4", out=qc)
            st.update(kc=qc.k_codes, vc=qc.v_codes, ksz=qc.k_sz, vsz=qc.v_sz,
                      resid=init_k_residual(kc_g, bt_g, st["sl"]))
        else:
            st.update(kc=kc_g.clone(), vc=vc_g.clone())
        return st

    graph_state, eager_state, warm_state = fresh_state(), fresh_state(), fresh_state()
    # warm-up outside capture (library load, device queries), then capture one step
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        warm_state["sl"] += 1
        _graph_step(warm_state, quant)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    graph_state["sl"] += 1  # the captured step appends token lens0[b]
    eager_state["sl"] += 1
    with torch.cuda.graph(g):
        out_static = _graph_step(graph_state, quant)
    torch.cuda.synchronize()
    # capture does not run the kernels: the first replay is the first real step
    for step in range(steps):
        if step:
            for st in (graph_state, eager_state):
                st["sl"] += 1
        qs = rng.standard_normal(q.shape).astype(np.float16)
        pos = sl0 + step  # position of the new token
        kn = np.stack([k[b, p] for b, p in enumerate(pos)])
        vn = np.stack([v[b, p] for b, p in enumerate(pos)])
        for st in (graph_state, eager_state):
            st["q"].copy_(gpu(qs))
            st["kn"].copy_(gpu(kn))
            st["vn"].copy_(gpu(vn))
        g.replay()
        torch.cuda.synchronize()
        want = _graph_step(eager_state, quant)
        torch.cuda.synchronize()
        print(f"\n[{'int4' if quant else 'fp16'} graph replay {step}]", flush=True)
        assert torch.equal(out_static, want), f"replay {step} differs from eager"
        for name in ("kc", "vc") + (("ksz", "vsz", "resid") if quant else ()):
            assert torch.equal(graph_state[name], eager_state[name]), (step, name)
    # the last state against the oracle
    lens = sl0 + steps
    if quant:
        host = {n: getattr(t, "cpu")().numpy() for n, t in (
            ("k_codes", graph_state["kc"]), ("v_codes", graph_state["vc"]),
            ("k_scale", graph_state["ksz"][..., 0]), ("k_zero", graph_state["ksz"][..., 1]),
            ("v_scale", graph_state["vsz"][..., 0]), ("v_zero", graph_state["vsz"][..., 1]))}
        kd, vd = kivi.dequantize_paged_cache(host, bt, lens, "int4")
    else:
        kd, vd = graph_state["kc"].cpu().numpy(), graph_state["vc"].cpu().numpy()
    ref = paged_decode_attention_ref(qs.astype(np.float32), kd.astype(np.float32),
                                     vd.astype(np.float32), bt, lens, out_dtype=np.float32)
    diff = np.abs(out_static.float().cpu().numpy() - ref)
    assert diff.max() < ATOL and np.all(diff <= ATOL + RTOL * np.abs(ref)), diff.max()
