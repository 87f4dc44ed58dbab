"""Decode-step benchmark on one MI355X: achieved KV-read bandwidth of the paged-KV GQA
decode path (split-KV stage 1 + merge) against the 8 TB/s HBM3E roofline.

    python bench.py [--steps K] [--warmup W] [--config C2] [--splits S]
    python bench.py --sweep            # split / workgroup sweep, table on stderr

Workload ("C2"): Llama-3-8B GQA layer (32 q heads, 8 kv heads,
head_dim 128), batch 8, every sequence 32768 tokens, block_size 16, q/K/V ~ N(0,1) fp16,
block table = a random permutation of a 16384-block pool; split count from the heuristic
(32 on 256 CUs). A step is one decode of the whole batch (stage 1 + stage 2), inputs
resident in HBM. Algorithmic bytes = KV reads only (reference src/bpt/roofline.py:1-4,
bench/bench_triton_fp16.py:58): B * ctx * Hkv * 2 * D * 2 bytes for fp16.

Prints progress on stderr and ONE JSON line on stdout.
"""
import argparse
import json
import math
import os
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
if REPO not in sys.path:
    sys.path.insert(0, REPO)

METRIC = ("achieved KV-read TB/s & % of 8 TB/s HBM peak; µs per decode step (1 layer)")
PEAK_GBPS = 8000.0
HQ, HKV, D, BS = 32, 8, 128, 16

# name -> (batch, ctx, pool blocks, description); BASELINE.json configs[0..2]
CONFIGS = {
    "C1": (1, 4096, 256, "C1: fp16 KV, batch 1, seq_len 4096, no split"),
    "C2": (8, 32768, 16384, "C2: fp16 KV, batch 8, seq_len 32768, split-KV + merge"),
    "C3": (1, 131072, 8192, "C3: fp16 KV, batch 1, seq_len 131072, split-KV + merge"),
    "B1_64K": (1, 65536, 4096, "fp16 KV, batch 1, seq_len 65536 (north-star 50% point)"),
}


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def make_inputs(B, ctx, pool, seed=0):
    import torch
    g = torch.Generator(device="cuda").manual_seed(seed)
    q = torch.randn(B, HQ, D, generator=g, device="cuda").half()
    k = torch.randn(pool, BS, HKV, D, generator=g, device="cuda").half()
    v = torch.randn(pool, BS, HKV, D, generator=g, device="cuda").half()
    nb = ctx // BS
    bt = torch.randperm(pool, generator=g, device="cuda")[: B * nb].view(B, nb).int().contiguous()
    sl = torch.full((B,), ctx, dtype=torch.int32, device="cuda")
    return q, k, v, bt, sl


class Step:
    """One decode step through the C ABI with prebuilt arguments and workspace, so the
    timed loop issues exactly the library's launches (split + merge, or single pass)."""

    def __init__(self, q, k, v, bt, sl, splits, waves=0, pipeline=0):
        import ctypes

        import torch

        from kvq_decode_amd import _lib, ops
        self.ctypes = ctypes
        self.L = _lib.lib()
        self.check = _lib.check
        B = q.shape[0]
        self.out = torch.empty_like(q)
        self.splits, self.pps = ops.normalize_splits(splits, bt.shape[1])
        self.args = ops.build_args(q, k, v, bt, sl, self.out, 1.0 / math.sqrt(D),
                                   waves_per_group=waves, pipeline=pipeline)
        self.o_part = torch.empty(B, HQ, self.splits, D, dtype=torch.float32, device="cuda")
        self.lse = torch.empty(B, HQ, self.splits, dtype=torch.float32, device="cuda")
        self.stream = torch.cuda.current_stream().cuda_stream
        self.B = B

    def stage1(self):
        a = self.ctypes.byref(self.args)
        if self.splits == 1:
            self.check("kvq_decode_single", self.L.kvq_decode_single(a, self.stream))
        else:
            self.check("kvq_decode_split",
                       self.L.kvq_decode_split(a, self.splits, self.pps, self.o_part.data_ptr(),
                                               self.lse.data_ptr(), self.stream))

    def stage2(self):
        if self.splits > 1:
            self.check("kvq_decode_merge",
                       self.L.kvq_decode_merge(self.o_part.data_ptr(), self.lse.data_ptr(),
                                               self.out.data_ptr(), self.out.stride(0),
                                               self.out.stride(1), self.B, HQ, D, self.splits,
                                               self.stream))

    def __call__(self):
        self.stage1()
        self.stage2()


def time_steps(step, steps, warmup):
    """Wall time of exactly `steps` back-to-back steps between synchronizes."""
    import torch
    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    ev0.record()
    for _ in range(steps):
        step()
    ev1.record()
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - t0) * 1e3 / steps
    return wall_ms, ev0.elapsed_time(ev1) / steps


def time_stage1(step, iters):
    """Average duration of the dominant kernel (stage 1) from HIP events recorded on the
    stream it is launched on, back to back."""
    import torch
    starts = [torch.cuda.Event(enable_timing=True) for _ in range(iters)]
    ends = [torch.cuda.Event(enable_timing=True) for _ in range(iters)]
    for i in range(iters):
        starts[i].record()
        step.stage1()
        ends[i].record()
        step.stage2()
    torch.cuda.synchronize()
    return sum(s.elapsed_time(e) for s, e in zip(starts, ends)) / iters


def time_flushed(step, iters):
    """Median step time with the 256 MB Infinity Cache flushed before each step (a 1 GiB
    scratch write), per-iteration events around the step only."""
    import torch
    scratch = torch.empty(1 << 28, dtype=torch.float32, device="cuda")
    ts = []
    for _ in range(iters):
        scratch.zero_()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        step()
        e1.record()
        torch.cuda.synchronize()
        ts.append(e0.elapsed_time(e1))
    del scratch
    ts.sort()
    return ts[len(ts) // 2]


def cpu_baseline(q, k, v, bt, sl):
    """The numpy oracle (oracle/attention.py, fp32) on the full workload on the host: one
    BLAS thread, 1 warmup + 3 timed reps. Checker code, timed only as the CPU baseline."""
    import numpy as np
    from threadpoolctl import threadpool_limits

    from oracle.attention import paged_decode_attention_ref
    qn, kn, vn, btn, sln = (t.cpu().numpy() for t in (q, k, v, bt, sl))
    nbytes = float(sum(int(x) for x in sln)) * HKV * 2 * D * 2
    with threadpool_limits(limits=1):
        paged_decode_attention_ref(qn, kn, vn, btn, sln)
        reps = 3
        t0 = time.perf_counter()
        for _ in range(reps):
            paged_decode_attention_ref(qn, kn, vn, btn, sln)
        sec = (time.perf_counter() - t0) / reps
    return {"value": nbytes / sec / 1e12, "unit": "TB/s", "cores": 1, "kind": "port",
            "sample": f"full workload step (B={qn.shape[0]}, ctx={int(sln[0])}), numpy fp32 "
                      f"oracle, 1 BLAS thread, 1 warmup + {reps} reps: {sec * 1e3:.0f} ms/step",
            "s_per_step": sec}


def read_traffic(workload, splits):
    """HBM bytes per stage-1 launch measured by rocprofv3 --pmc, if a summary for this
    workload and split count is committed under profiles/ (see DESIGN.md), else None."""
    path = os.path.join(REPO, "profiles", f"decode_split_{workload}_traffic.txt")
    if not os.path.exists(path):
        return None
    vals = {}
    with open(path) as f:
        for line in f:
            if "=" in line and not line.lstrip().startswith("#"):
                key, val = line.split("=", 1)
                vals[key.strip()] = val.strip()
    try:
        if int(vals.get("splits", -1)) != splits:
            return None
        return float(vals["hbm_bytes_per_launch"])
    except (KeyError, ValueError):
        return None


def sweep(args):
    import torch
    B, ctx, pool, _ = CONFIGS[args.config]
    q, k, v, bt, sl = make_inputs(B, ctx, pool)
    nbytes = B * ctx * HKV * 2 * D * 2
    log(f"{args.config}: B={B} ctx={ctx} kv={nbytes / 1e9:.3f} GB")
    log(f"{'splits':>6}{'waves':>6}{'pipe':>5}{'step_us':>10}{'stage1_us':>11}{'TB/s':>8}{'%peak':>7}")
    for splits in [int(s) for s in args.sweep_splits.split(",")]:
        for waves in [int(w) for w in args.sweep_waves.split(",")]:
            for pipe in (1, 2):
                try:
                    st = Step(q, k, v, bt, sl, splits, waves, pipe)
                except Exception as e:  # invalid combination for this config
                    log(f"{splits:>6}{waves:>6}{pipe:>5}  skipped: {e}")
                    continue
                _, ev_ms = time_steps(st, 20, 5)
                s1 = time_stage1(st, 20)
                tbs = nbytes / (ev_ms * 1e-3) / 1e12
                log(f"{st.splits:>6}{waves:>6}{pipe:>5}{ev_ms * 1e3:>10.1f}{s1 * 1e3:>11.1f}"
                    f"{tbs:>8.3f}{100 * tbs * 1e3 / PEAK_GBPS:>7.1f}")
                del st
                torch.cuda.synchronize()


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--config", default="C2", choices=sorted(CONFIGS))
    ap.add_argument("--splits", type=int, default=None, help="default: the heuristic")
    ap.add_argument("--waves", type=int, default=0)
    ap.add_argument("--pipeline", type=int, default=0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--sweep", action="store_true")
    ap.add_argument("--sweep-splits", default="8,16,32,64")
    ap.add_argument("--sweep-waves", default="1,2,4,8,16")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU only (asked for {args.gpus}); the "
              "multi-GPU sharding of the path is described in DESIGN.md", file=sys.stderr)
        sys.exit(2)

    import torch

    from kvq_decode_amd import _sm_count, choose_num_splits
    if args.sweep:
        sweep(args)
        return

    B, ctx, pool, desc = CONFIGS[args.config]
    log(f"bench {args.config}: {desc}")
    q, k, v, bt, sl = make_inputs(B, ctx, pool)
    cus = _sm_count(0)
    splits = args.splits if args.splits is not None else choose_num_splits(B, HKV, BS, ctx // BS, cus)
    if args.config == "C1" and args.splits is None:
        splits = 1
    step = Step(q, k, v, bt, sl, splits, args.waves, args.pipeline)
    nbytes = B * ctx * HKV * 2 * D * 2
    log(f"splits={step.splits} pages/split={step.pps} CUs={cus} KV bytes/step={nbytes}")

    wall_ms, ev_ms = time_steps(step, args.steps, args.warmup)
    log(f"timed {args.steps} steps: wall {wall_ms * 1e3:.1f} us/step, events {ev_ms * 1e3:.1f} us/step")
    stage1_ms = time_stage1(step, max(20, min(args.steps, 100)))
    log(f"stage-1 kernel average: {stage1_ms * 1e3:.1f} us")
    flushed_ms = time_flushed(step, 30)
    log(f"flushed-cache median step: {flushed_ms * 1e3:.1f} us")

    tbs = nbytes / (wall_ms * 1e-3) / 1e12
    achieved_gbps = nbytes / (stage1_ms * 1e-3) / 1e9
    traffic = read_traffic(args.config, step.splits)
    result = {
        "metric": METRIC,
        "value": round(tbs, 4),
        "unit": "TB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(wall_ms, 5),
        "us_per_step": round(wall_ms * 1e3, 2),
        "pct_of_hbm_peak": round(100 * tbs * 1e3 / PEAK_GBPS, 2),
        "us_per_step_flushed_median": round(flushed_ms * 1e3, 2),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16",
        "data": "synthetic: q, K, V ~ N(0,1) fp16, random-permutation block table, seed 0",
        "config": {"workload": desc, "batch": B, "seq_len": ctx, "q_heads": HQ, "kv_heads": HKV,
                   "head_dim": D, "block_size": BS, "pool_blocks": pool,
                   "num_splits": step.splits, "pages_per_split": step.pps,
                   "kv_bytes_per_step": nbytes, "kv_format": "fp16"},
        "roofline": {"bound": "hbm", "achieved": round(achieved_gbps, 1), "peak": PEAK_GBPS,
                     "unit": "GB/s", "frac": round(achieved_gbps / PEAK_GBPS, 4),
                     "traffic": traffic, "kernel": "decode_f16_kernel (stage 1)",
                     "kernel_us": round(stage1_ms * 1e3, 2)},
    }
    if not args.no_cpu_baseline:
        log("cpu baseline (numpy oracle) ...")
        cb = cpu_baseline(q, k, v, bt, sl)
        log(f"cpu baseline: {cb['s_per_step'] * 1e3:.0f} ms/step")
        cb.pop("s_per_step")
        result["cpu_baseline"] = cb
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
