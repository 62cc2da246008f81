"""Benchmark of the write-gated dual-cache decode path on one MI355X.

Workload (the ragged 128K decode the metric names):
one Llama-3.1-8B-shaped attention layer (32 q / 8 KV heads, head_dim 128),
batch 8, 128K context, local window 1024, per-(sequence, head) admitted
fraction U[2 %, 60 %] -> 2.6K..79K cached tokens per head, 16-token pages
in random physical order, bf16 K/V ~ N(0,1).  A step is one decode-attention
pass over the whole batch (one new token per sequence) through the HIP
kernels; inputs are resident in HBM before timing starts.

Prints one JSON line (rank 0) with the driver's fields plus ``roofline``
(HBM-bound: algorithmic bytes per launch / average launch time) and
``cpu_baseline`` (the CPU oracle on a bounded sample of the same workload).
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "wg-kv_amd"))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=50)
    p.add_argument("--warmup", type=int, default=10)
    p.add_argument("--cpu-seconds", type=float, default=12.0,
                   help="wall-time budget of the CPU-oracle baseline sample")
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--no-secondary", action="store_true")
    return p.parse_args()


def time_op(fn, steps, warmup):
    import torch
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record()  # torch's current stream: the stream the kernels are launched on
    for _ in range(steps):
        fn()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / steps


def cpu_baseline(w, budget_s):
    """Oracle decode of whole sequences of the workload on the host cores.

    The sequences' pages are copied to host memory once (not timed); then
    the oracle decodes one sequence after another, cycling over the batch,
    until ``budget_s`` seconds of CPU time have been spent (at least one pass).
    """
    import torch
    from oracle import attention

    torch.set_num_threads(os.cpu_count() or 1)
    B = w.q.shape[0]
    host = []
    for b in range(B):
        sl = w.cache_seqlens[b:b + 1].cpu()
        bt = w.block_table[b:b + 1].cpu()
        pages = bt[bt >= 0].long().unique()
        remap = torch.full((w.k_cache.shape[0],), -1, dtype=torch.int64)
        remap[pages] = torch.arange(pages.numel())
        idx = pages.to(w.k_cache.device)
        k = w.k_cache[idx].cpu()
        v = w.v_cache[idx].cpu()
        bt2 = torch.where(bt >= 0, remap[bt.clamp(min=0).long()], -1).to(torch.int32)
        host.append((w.q[b:b + 1].cpu(), k, v, sl, bt2))
    done = 0
    tokens = 0
    t_total = 0.0
    while t_total < budget_s or done < B:
        q, k, v, sl, bt2 = host[done % B]
        t0 = time.perf_counter()
        attention.paged_decode(q, k, v, sl, bt2, w.softmax_scale)
        t_total += time.perf_counter() - t0
        tokens += int(sl.sum())
        done += 1
    per_seq = t_total / done
    return {
        "value": round(1.0 / per_seq, 3),
        "unit": "tokens/s",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": (f"oracle.attention.paged_decode (torch fp32 CPU): {done} sequence decodes cycling over the "
                   f"batch of {B} ({tokens} cached tokens attended, {t_total:.1f} s); one decode token per "
                   "sequence, so tokens/s = sequences decoded / second"),
    }


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU; --gpus must be 1",
                          "n_gpus": args.gpus}))
        sys.exit(2)
    import torch
    import wgkv
    from wgkv import workloads

    assert torch.cuda.is_available(), "bench.py needs a GPU"
    dev = torch.device("cuda:0")
    w = workloads.decode_ragged(ctx=131072, batch=8, device=dev, seed=0)
    B = w.q.shape[0]
    out = torch.empty_like(w.q)

    def step():
        wgkv.paged_decode_attn(w.q, w.k_cache, w.v_cache, w.cache_seqlens, w.block_table,
                               w.softmax_scale, out=out)

    ms = time_op(step, args.steps, args.warmup)
    nbytes = w.algorithmic_bytes()
    achieved = nbytes / (ms * 1e-3) / 1e9
    result = {
        "metric": "decode tokens/s + attn HBM GB/s (ragged dual-cache, 128K ctx, ~20% admit)",
        "value": round(B / (ms * 1e-3), 2),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {
            "workload": "decode_ragged_b8_128k (BASELINE config 3): one layer's paged decode attention",
            "batch": B, "context": 131072, "local_window": 1024, "admit_frac": "U[0.02,0.60] per (seq,head)",
            "q_heads": 32, "kv_heads": 8, "head_dim": 128, "page": 16,
            "cached_tokens": w.total_tokens,
        },
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": None,
            "bytes_per_launch": nbytes,
            "launch": "wgkv_paged_decode_attn = decode_split_kernel + decode_merge_kernel",
        },
    }
    if not args.no_secondary:
        sec = []
        for name, mk in (("decode_beta_b1_32k", lambda: workloads.decode_beta(ctx=32768, device=dev)),
                         ("decode_beta_b1_128k", lambda: workloads.decode_beta(ctx=131072, device=dev))):
            ws = mk()
            o2 = torch.empty_like(ws.q)
            m2 = time_op(lambda: wgkv.paged_decode_attn(ws.q, ws.k_cache, ws.v_cache, ws.cache_seqlens,
                                                        ws.block_table, ws.softmax_scale, out=o2),
                         args.steps, args.warmup)
            b2 = ws.algorithmic_bytes()
            sec.append({"workload": name, "ms": round(m2, 5), "bytes": b2,
                        "GB/s": round(b2 / (m2 * 1e-3) / 1e9, 1), "cached_tokens": ws.total_tokens})
            del ws
        result["secondary"] = sec
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(w, args.cpu_seconds)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
