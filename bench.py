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
BF16_PEAK_TFLOPS = 2500.0   # dense MFMA
FP32_PEAK_TFLOPS = 157.3    # dense MFMA


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=50)
    p.add_argument("--warmup", type=int, default=10)
    p.add_argument("--cpu-seconds", type=float, default=12.0,
                   help="wall-time budget of the CPU-oracle baseline sample")
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--no-secondary", action="store_true")
    p.add_argument("--no-prefill", action="store_true")
    p.add_argument("--no-layer", action="store_true")
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


def prefill_section(dev, steps, warmup):
    """Config-4 shapes, one-shot over the 32K prompt: every kernel of the
    gated prefill timed on its own (gate, admission into the dual cache,
    metadata, sparse attention), with MFMA utilisation of the gate (fp32) and
    of the attention (bf16, FLOPs = sum over query heads and rows of
    4*D*|visible keys|).  The chunked per-4096 figure is the one-shot time
    divided by the 8 chunks (the visible (query, key) set is the same)."""
    import torch
    import wgkv
    from wgkv import ops, workloads
    from wgkv.cache import DualCache
    from wgkv.layers import WGKVConfig

    S, Hq, Hkv, D, W = 32768, 32, 8, 128, 1024
    w = workloads.prefill_llama(S=S, Hq=Hq, Hkv=Hkv, D=D, W=W, device=dev)
    pk, kk, vv = w.pre_k.transpose(1, 2), w.k.transpose(1, 2), w.v.transpose(1, 2)
    mask = torch.empty(1, Hkv, S, dtype=torch.bool, device=dev)
    scores = torch.empty(1, Hkv, S, dtype=torch.float32, device=dev)

    def gate():
        w.gate.scores_and_mask(pk, kk, None, w.threshold, scores_out=scores, mask_out=mask)

    t_gate = time_op(gate, steps, warmup)
    cfg = WGKVConfig(num_hidden_layers=1, num_attention_heads=Hq, num_key_value_heads=Hkv, head_dim=D,
                     hidden_size=Hq * D, local_window_size=W, max_tokens_per_head=S + W,
                     max_total_tokens=Hkv * (S + W) + 4096)
    cache = DualCache()
    cache.initialize(cfg, D, torch.bfloat16, dev)
    snap = (cache.block_table.clone(), cache.global_lengths.clone(), cache.next_free_block_dev.clone())

    def admit():
        cache.block_table.copy_(snap[0])
        cache.global_lengths.copy_(snap[1])
        cache.next_free_block_dev.copy_(snap[2])
        ops.prefill_admit(cache, 0, kk[0], vv[0], mask[0])

    t_admit = time_op(admit, steps, warmup)
    meta = [None]

    def build_meta():
        meta[0] = wgkv.generate_sparse_indices(mask, W, 1, Hkv, S)

    t_meta = time_op(build_meta, steps, warmup)
    out = torch.empty_like(w.q)

    def attn():
        wgkv.sparse_attn_func(w.q, w.k, w.v, *meta[0], out=out)

    t_attn = time_op(attn, steps, warmup)
    pairs = workloads.visible_pairs(mask[0], W)
    attn_flop = float((pairs * (Hq // Hkv)).sum().item()) * 4 * D
    gate_flop = 2.0 * 512 * 256 * S * Hkv
    admitted = mask.float().mean().item()
    total = t_gate + t_admit + t_meta + t_attn
    return {
        "workload": "prefill_llama_32k (BASELINE config 4 shapes, one-shot over the prompt)",
        "admitted_frac": round(admitted, 4),
        "ms": {"gate": round(t_gate, 4), "admit": round(t_admit, 4), "meta": round(t_meta, 4),
               "sparse_attn": round(t_attn, 4), "total": round(total, 4),
               "per_4096_chunk_equiv": round(total / 8, 4)},
        "sparse_attn": {"tflop": round(attn_flop / 1e12, 4), "tflops": round(attn_flop / t_attn / 1e9, 1),
                        "mfma_frac_bf16": round(attn_flop / t_attn / 1e9 / BF16_PEAK_TFLOPS, 4),
                        "dense_causal_tflop": round(4.0 * D * Hq * S * (S + 1) / 2 / 1e12, 3)},
        "gate": {"gflop": round(gate_flop / 1e9, 2), "tflops": round(gate_flop / t_gate / 1e9, 1),
                 "mfma_frac_fp32": round(gate_flop / t_gate / 1e9 / FP32_PEAK_TFLOPS, 4)},
    }


def layer_section(dev, cpu_budget):
    """the write-gated layer (2048 prefill + 32 decode
    steps) on the GPU through the HIP path, and the same layer as the CPU
    oracle in fp32 (the reference's CPU path) on the host cores."""
    import torch
    from oracle import gate as ogate
    from oracle.llama_layer import OracleLayer
    from wgkv import workloads
    from wgkv.attention import LlamaAttention, LlamaRotaryEmbedding
    from wgkv.cache import DualCache
    from wgkv.layers import WGKVConfig

    cfg, w, x, xs = workloads.config1_layer()
    probe = OracleLayer(w, 512, 8, 2, 64, 128, cfg["max_tokens_per_head"])
    _, pre_k, k, v = probe._project(x, torch.arange(x.shape[1]))
    w = workloads.shift_gate_bias(w, ogate.gate_logits(pre_k, k, v, probe.gp)[0], cfg["_frac"],
                                  cfg["_logit_threshold"])
    c = WGKVConfig(**{kk: vv for kk, vv in cfg.items() if not kk.startswith("_")})
    c.check_capacity = False
    layer = LlamaAttention(c, 0)
    layer.load_state_dict(w, strict=True)
    layer = layer.to(dev)
    rope = LlamaRotaryEmbedding(64).to(dev)
    S = x.shape[1]
    xg = x.to(dev)
    xsg = [xi.to(dev) for xi in xs]
    pos = torch.arange(S, device=dev)[None]
    emb = rope(xg, pos)
    embs = [rope(xsg[i], torch.tensor([[S + i]], device=dev)) for i in range(len(xs))]

    def gpu_run():
        cache = DualCache()
        t0 = torch.cuda.Event(enable_timing=True)
        t1 = torch.cuda.Event(enable_timing=True)
        t2 = torch.cuda.Event(enable_timing=True)
        with torch.no_grad():
            t0.record()
            layer(3, xg, emb, None, cache)
            t1.record()
            for xi, e in zip(xsg, embs):
                layer(3, xi, e, None, cache)
            t2.record()
        torch.cuda.synchronize()
        return t0.elapsed_time(t1), t1.elapsed_time(t2) / len(xs)

    for _ in range(2):
        gpu_run()
    runs = [gpu_run() for _ in range(5)]
    g_pre = sorted(r[0] for r in runs)[2]
    g_dec = sorted(r[1] for r in runs)[2]
    torch.set_num_threads(os.cpu_count() or 1)

    def cpu_run():
        o = OracleLayer(w, 512, 8, 2, 64, 128, cfg["max_tokens_per_head"])
        t0 = time.perf_counter()
        o.prefill(x, torch.arange(S))
        t1 = time.perf_counter()
        for i, xi in enumerate(xs):
            o.decode(xi, S + i)
        t2 = time.perf_counter()
        return (t1 - t0) * 1e3, (t2 - t1) * 1e3 / len(xs)

    cpu_run()
    cruns = []
    t_start = time.perf_counter()
    while len(cruns) < 5 and (time.perf_counter() - t_start < cpu_budget or len(cruns) < 1):
        cruns.append(cpu_run())
    c_pre = sorted(r[0] for r in cruns)[len(cruns) // 2]
    c_dec = sorted(r[1] for r in cruns)[len(cruns) // 2]
    return {
        "workload": "config1_layer (BASELINE config 1: hidden 512, 8q/2kv, D 64, W 128, 2048 prefill + 32 decode)",
        "gpu": {"prefill_ms": round(g_pre, 3), "decode_ms_per_step": round(g_dec, 4),
                "note": "whole layer incl. projections/RoPE/gate; includes host launch overhead"},
        "cpu_reference_path": {"prefill_ms": round(c_pre, 2), "decode_ms_per_step": round(c_dec, 3),
                               "decode_tokens_per_s": round(1e3 / c_dec, 1), "cores": torch.get_num_threads(),
                               "kind": "port", "runs": len(cruns),
                               "sample": "oracle.llama_layer.OracleLayer fp32 on the host cores; median of runs"},
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
    del w, out
    torch.cuda.empty_cache()
    if not args.no_prefill:
        result["prefill"] = prefill_section(dev, max(5, args.steps // 5), max(2, args.warmup // 5))
        torch.cuda.empty_cache()
    if not args.no_layer:
        result["layer_config1"] = layer_section(dev, args.cpu_seconds)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
