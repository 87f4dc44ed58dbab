"""The whole-model decode step that `bench.py --layers` / `--model` times (the per-model,
all-layers step of the reference's byte model, src/bpt/roofline.py:42-63). Needs a GPU.

bench.build_layers makes one cache per layer, bench.run_model_step decodes every layer back
to back, and bench.capture_layers records that step in one HIP graph. Each replay of the
graph must give every layer's output bit for bit as the eager step did (the same kernels
on the same inputs; they are deterministic), with eager work and synchronizations between
the replays, and one layer must match the oracle within the north-star tolerance (fp16:
the paged fp32 reference; INT4 / INT8: fp32 attention over the dequantized cache). Besides
Llama-3-8B's 4 q heads per kv head, the quantized steps run Llama-3-70B's 8 (64 / 8 heads)
and Qwen2.5-7B's 7 (28 / 4 heads), which take the 5-8 head chunk-pair kernel.
"""
import numpy as np
import pytest
import torch

import bench
from oracle import kivi
from oracle.attention import paged_decode_attention_ref

pytestmark = pytest.mark.gpu

ATOL, RTOL = 2e-3, 1e-2


@pytest.mark.parametrize("fmt,shape", [("fp16", (32, 8, 128)), ("int4", (32, 8, 128)),
                                       ("int4", (64, 8, 128)), ("int8", (28, 4, 128))])
def test_captured_model_step_equals_eager_and_oracle(fmt, shape, cuda):
    layers = 3
    step_list, lens = bench.build_layers(4, 3000, None, fmt, layers, shape=shape)
    assert step_list[0].units > 0  # the default plan at this shape: work units + merge
    bench.run_model_step(step_list)
    torch.cuda.synchronize()
    eager = [st.out.clone() for st in step_list]
    assert all(not torch.isnan(o).any() for o in eager)
    graph = bench.capture_layers(step_list)
    for rep in range(3):
        for st in step_list:  # eager work between replays: poison every output
            st.out.fill_(float("nan"))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        print(f"\n[{fmt} {shape} model-step replay {rep}]", flush=True)
        for i, st in enumerate(step_list):
            assert torch.equal(st.out, eager[i]), f"replay {rep}, layer {i} differs from eager"
    # layer 1 against the oracle
    q, k, v, bt, sl, fmt_kw = step_list[1].inputs
    btn, sln = bt.cpu().numpy(), sl.cpu().numpy()
    qn = q.cpu().numpy().astype(np.float32)
    if fmt == "fp16":
        kd, vd = k.cpu().numpy(), v.cpu().numpy()
    else:
        host = {n: fmt_kw[n].cpu().numpy() for n in ("k_scale", "k_zero", "v_scale", "v_zero")}
        host.update(k_codes=k.cpu().numpy(), v_codes=v.cpu().numpy())
        kd, vd = kivi.dequantize_paged_cache(host, btn, sln, fmt)
    ref = paged_decode_attention_ref(qn, kd.astype(np.float32), vd.astype(np.float32), btn, sln,
                                     out_dtype=np.float32)
    diff = np.abs(step_list[1].out.float().cpu().numpy() - ref)
    print(f"[{fmt} {shape} layer 1 vs oracle] max_abs={diff.max():.3e}", flush=True)
    assert diff.max() < ATOL and np.all(diff <= ATOL + RTOL * np.abs(ref))
