"""Quantized-KV accuracy harness: how much INT8 / FP8-e4m3 / INT4 KIVI caches change what
decode attention retrieves (the reference asks for this evaluation and never built it,
README.md:90).

No model weights are available offline, so perplexity is out of reach; the harness uses
the attention-level test that drives it instead, a synthetic needle in a haystack:

  * every (sequence, kv head) gets a long haystack of K ~ N(0,1) with 4 outlier
    channels x10 per kv head (the distribution KIVI's per-channel K scales exist for) and
    V ~ N(0,1);
  * one needle token at a random position gets a key boosted along its q-head group's
    mean query direction, with a logit margin of ln(ctx) + delta, and a value drawn
    N(0, 9 I);
  * the truth is float32 attention over the fp16 cache (torch, dense); each format is
    decoded through the library (quantized with the library's own quantizer);
  * per q head, the needle weight a decode output o implies is w = <o, v_n> / <v_n, v_n>
    (the haystack's values are independent of v_n, so w estimates the needle's softmax
    weight). A head "retrieves" the needle when w > 1/2.

Reported per (format, delta): mean |w - w_true|, retrieval agreement with the float32
truth, mean cosine similarity and relative L2 error of the outputs against the fp16-cache
decode. Run `python -m kvq_decode_amd.accuracy` on a GPU; one JSON line per row.
"""
import json
import math
import sys

import torch

HQ, HKV, D, BS = 32, 8, 128, 16
FORMATS = ("fp16", "int8", "fp8_e4m3", "int4")


def _haystack(B, ctx, delta, gen):
    """Contiguous K/V [B, ctx, Hkv, D] fp16 with one needle per (sequence, kv head), the
    queries, and the needle positions and values."""
    g = HQ // HKV
    scale = 1.0 / math.sqrt(D)
    q = torch.randn(B, HQ, D, generator=gen, device="cuda")
    k = torch.randn(B, ctx, HKV, D, generator=gen, device="cuda")
    for h in range(HKV):
        k[:, :, h, torch.randperm(D, generator=gen, device="cuda")[:4]] *= 10
    v = torch.randn(B, ctx, HKV, D, generator=gen, device="cuda")
    pos = torch.randint(0, ctx, (B, HKV), generator=gen, device="cuda")
    vn = 3.0 * torch.randn(B, HKV, D, generator=gen, device="cuda")
    u = q.view(B, HKV, g, D).mean(2)
    u = u / u.norm(dim=-1, keepdim=True)
    # boost so that the group's mean q gains ln(ctx) + delta on the needle's logit
    proj = (q.view(B, HKV, g, D) * u[:, :, None]).sum(-1).mean(-1).clamp_min(0.5)
    gamma = (math.log(ctx) + delta) / (scale * proj)
    bi = torch.arange(B, device="cuda")[:, None].expand(B, HKV)
    hi = torch.arange(HKV, device="cuda")[None, :].expand(B, HKV)
    k[bi, pos, hi] = k[bi, pos, hi] + gamma[..., None] * u
    v[bi, pos, hi] = vn
    return q.half(), k.half(), v.half(), pos, vn.half()


def _paged(k, v, gen):
    """Scatter contiguous K/V into a randomly permuted paged cache (reference.py:52-82
    addressing) and return (k_cache, v_cache, block_table)."""
    B, ctx, hkv, d = k.shape
    mb = -(-ctx // BS)
    nb = B * mb
    bt = torch.randperm(nb, generator=gen, device="cuda").view(B, mb).int()
    kc = torch.zeros(nb, BS, hkv, d, dtype=torch.float16, device="cuda")
    vc = torch.zeros_like(kc)
    pad = mb * BS - ctx
    kp = torch.nn.functional.pad(k, (0, 0, 0, 0, 0, pad)).view(B, mb, BS, hkv, d)
    vp = torch.nn.functional.pad(v, (0, 0, 0, 0, 0, pad)).view(B, mb, BS, hkv, d)
    kc[bt.long()] = kp
    vc[bt.long()] = vp
    return kc, vc, bt


def _truth(q, k, v):
    """float32 attention over the fp16 K/V (dense) -> [B, Hq, D] float32."""
    B, ctx, hkv, d = k.shape
    g = HQ // hkv
    kf = k.float().permute(0, 2, 3, 1).contiguous()  # [B, Hkv, D, ctx]
    vf = v.float().permute(0, 2, 1, 3).contiguous()  # [B, Hkv, ctx, D]
    qf = q.float().view(B, hkv, g, d)
    s = torch.matmul(qf, kf) / math.sqrt(d)            # [B, Hkv, g, ctx]
    p = torch.softmax(s, dim=-1)
    return torch.matmul(p, vf).view(B, HQ, d)


def _needle_weight(o, vn):
    """w = <o, v_n> / <v_n, v_n> per q head (v_n of the head's kv head)."""
    B = o.shape[0]
    vq = vn.float().repeat_interleave(HQ // HKV, dim=1)  # [B, Hq, D]
    return (o.float() * vq).sum(-1) / (vq * vq).sum(-1)


def evaluate(B=4, ctx=16384, deltas=(-2.0, 0.0, 2.0, 4.0), seeds=(0, 1), formats=FORMATS):
    """Rows of accuracy metrics, one per (format, delta), aggregated over `seeds`."""
    from kvq_decode_amd import paged_decode_attention
    from kvq_decode_amd.quant import quantize_paged_cache
    rows = []
    for delta in deltas:
        acc = {f: {"dw": [], "agree": [], "cos": [], "rel": []} for f in formats}
        for seed in seeds:
            gen = torch.Generator(device="cuda").manual_seed(seed)
            q, k, v, pos, vn = _haystack(B, ctx, delta, gen)
            truth = _truth(q, k, v)
            w_true = _needle_weight(truth, vn)
            kc, vc, bt = _paged(k, v, gen)
            sl = torch.full((B,), ctx, dtype=torch.int32, device="cuda")
            outs = {}
            for f in formats:
                if f == "fp16":
                    outs[f] = paged_decode_attention(q, kc, vc, bt, sl)
                else:
                    qc = quantize_paged_cache(kc, vc, bt, sl, f)
                    outs[f] = paged_decode_attention(q, qc.k_codes, qc.v_codes, bt, sl,
                                                     **qc.decode_kwargs())
                    del qc
            base = outs["fp16"].float() if "fp16" in outs else truth
            for f, o in outs.items():
                w = _needle_weight(o, vn)
                of = o.float()
                a = acc[f]
                a["dw"].append((w - w_true).abs().mean().item())
                a["agree"].append(((w > 0.5) == (w_true > 0.5)).float().mean().item())
                a["cos"].append(torch.nn.functional.cosine_similarity(of, base, dim=-1)
                                .mean().item())
                a["rel"].append(((of - base).norm(dim=-1) / base.norm(dim=-1)).mean().item())
            w_frac = (w_true > 0.5).float().mean().item()
            del q, k, v, kc, vc, bt, outs
            torch.cuda.empty_cache()
        for f in formats:
            a = acc[f]
            n = len(a["dw"])
            rows.append({"format": f, "delta": delta, "ctx": ctx, "batch": B,
                         "trials": n * B * HQ, "retrieving_heads_true": round(w_frac, 3),
                         "mean_abs_needle_weight_err": round(sum(a["dw"]) / n, 5),
                         "retrieval_agreement": round(sum(a["agree"]) / n, 5),
                         "cos_vs_fp16": round(sum(a["cos"]) / n, 6),
                         "rel_l2_vs_fp16": round(sum(a["rel"]) / n, 6)})
    return rows


def main(argv=None):
    import argparse
    ap = argparse.ArgumentParser(description="needle-in-a-haystack accuracy of quantized KV")
    ap.add_argument("--batch", type=int, default=4)
    ap.add_argument("--ctx", type=int, default=16384)
    ap.add_argument("--seeds", type=int, default=2)
    args = ap.parse_args(argv)
    for row in evaluate(args.batch, args.ctx, seeds=tuple(range(args.seeds))):
        print(json.dumps(row), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
