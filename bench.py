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


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=50)
    # untimed steps first: the GPU's clocks settle over ~0.1 s of sustained
    # work (config 3 at 10 warm-up steps 0.2210-0.2220 ms, at 400 0.2164-0.2173)
    p.add_argument("--warmup", type=int, default=400)
    p.add_argument("--cpu-seconds", type=float, default=12.0,
                   help="wall-time budget of the CPU-oracle baseline sample")
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--no-secondary", action="store_true")
    p.add_argument("--no-prefill", action="store_true")
    p.add_argument("--no-layer", action="store_true")
    p.add_argument("--e2e", action="store_true",
                   help="only the BASELINE config-5 end-to-end run: a 32-layer Llama-3.1-8B-shaped model, "
                        "chunked prefill of --e2e-prompt tokens then --e2e-steps greedy decode steps, "
                        "gated and all-admitted, on one GPU (about 1.5 minutes at 400K)")
    p.add_argument("--no-e2e", action="store_true",
                   help="leave the config-5 end-to-end run out of the default line")
    p.add_argument("--e2e-prompt", type=int, default=400000)
    p.add_argument("--e2e-chunk", type=int, default=4096, help="prompt tokens per prefill chunk")
    p.add_argument("--e2e-steps", type=int, default=256)
    p.add_argument("--e2e-layers", type=int, default=32)
    p.add_argument("--e2e-admit", type=float, default=0.30)
    p.add_argument("--e2e-model", choices=["llama3-8b", "qwen3-8b"], default="llama3-8b")
    p.add_argument("--e2e-profile", choices=["rms_linear_attn", "linear_attn", "attn", "wrapper", "kernel",
                                             "predictor"], default=None,
                   help="with --e2e: one more eager run per mode that times attention (at this granularity), "
                        "MLP and LM head per phase, as the reference's --profile_attn_mlp --attn_granularity")
    p.add_argument("--e2e-profile-steps", type=int, default=32)
    p.add_argument("--prefill-long-probe", action="store_true",
                   help="run only one Llama-8B layer prefilled to 409,600 tokens in 4096-token chunks (30 %% "
                        "admitted), time the last chunk's attention x5 and a 1 GiB torch copy, for rocprofv3 --pmc "
                        "FETCH_SIZE passes over a long-context chunk (the copy calibrates the counter)")
    p.add_argument("--traffic-probe", action="store_true",
                   help="run only a 1 GiB torch copy x5 and the config-3 decode x5, for rocprofv3 --pmc "
                        "FETCH_SIZE / WRITE_SIZE passes (the copy calibrates the counters)")
    return p.parse_args()


# HBM bytes per config-3 decode call, from rocprofv3 --pmc FETCH_SIZE and
# WRITE_SIZE passes over `bench.py --traffic-probe`, each scaled by what the
# counter reads for a 1 GiB device copy in the same program; the summary with
# the commands and raw counter values is DECODE_TRAFFIC_SOURCE
DECODE_TRAFFIC_BYTES = 1347606162
DECODE_TRAFFIC_SOURCE = "profiles/decode_attn_traffic_b8_128k.md"


def host_cpu():
    """The host's CPU model (from /proc/cpuinfo) and logical CPU count."""
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"cpu_model": model, "nproc": os.cpu_count()}


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


class DeviceEvent:
    """A HIP timing event without the system-scope fence
    (hipEventCreateWithFlags(hipEventDisableSystemFence), which HIP documents
    for events used only to measure time).  torch's events take the default
    system-scope release, which writes back the L2 when recorded and leaves
    the GPU idle for ~5.5 us between the two kernels an event separates -- a
    cost the pipeline itself never pays (hipEventReleaseToDevice still
    leaves ~5 us).  The AQL barrier bit still orders the event after the
    kernels before it; its times are read after torch.cuda.synchronize(),
    which waits for the device.  Recorded on torch's current stream, the
    stream the kernels are launched on."""
    FLAGS = 0x20000000  # hipEventDisableSystemFence
    _hip = None
    KIND = "hipEventDisableSystemFence"

    @classmethod
    def runtime(cls):
        if cls._hip is None:
            import ctypes
            import torch  # noqa: F401  (the HIP runtime torch loaded; same SONAME, so dlopen returns it)
            h = ctypes.CDLL("libamdhip64.so.7")
            h.hipEventCreateWithFlags.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_uint]
            h.hipEventRecord.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
            h.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_void_p, ctypes.c_void_p]
            h.hipEventDestroy.argtypes = [ctypes.c_void_p]
            cls._hip = h
        return cls._hip

    def __init__(self):
        import ctypes
        self.ev = ctypes.c_void_p()
        st = self.runtime().hipEventCreateWithFlags(ctypes.byref(self.ev), self.FLAGS)
        if st != 0:
            raise RuntimeError(f"hipEventCreateWithFlags({self.KIND}) failed: {st}")

    def record(self):
        import torch
        st = self.runtime().hipEventRecord(self.ev, torch.cuda.current_stream().cuda_stream)
        if st != 0:
            raise RuntimeError(f"hipEventRecord failed: {st}")

    def elapsed_time(self, end):
        import ctypes
        ms = ctypes.c_float()
        st = self.runtime().hipEventElapsedTime(ctypes.byref(ms), self.ev, end.ev)
        if st != 0:
            raise RuntimeError(f"hipEventElapsedTime failed: {st}")
        return ms.value

    def __del__(self):
        if getattr(self, "ev", None):
            self.runtime().hipEventDestroy(self.ev)
            self.ev = None


def time_graph(fn, calls=20, replays=10):
    """Average time of fn() per call with the host out of the way: `calls`
    calls captured in one HIP graph, replayed `replays` times between HIP
    events (a batch-1 decode call is shorter than its host-side launch
    path, so back-to-back stream launches measure the host)."""
    import torch
    fn()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for _ in range(calls):
            fn()
    g.replay()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < 0.15:  # untimed: the GPU's clocks settle under sustained work
        for _ in range(10):
            g.replay()
        torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(replays):
        g.replay()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / (calls * replays)


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
        **host_cpu(),
        "kind": "port",
        "sample": (f"oracle.attention.paged_decode (torch fp32 CPU): {done} sequence decodes cycling over the "
                   f"batch of {B} ({tokens} cached tokens attended, {t_total:.1f} s); one decode token per "
                   "sequence, so tokens/s = sequences decoded / second"),
    }


def prefill_section(dev, steps, warmup):
    """a 32K-token prompt in 4096-token chunks through one
    Llama-3.1-8B-shaped layer.  Per chunk: the write gate (fp32 scores and the
    admission mask), admission into the dual cache (compaction, page scatter,
    column counts), the chunk's sparse attention over admitted columns plus
    the local band, and the ring rewrite.  ms/chunk is the whole prompt's
    time / 8 between two HIP events; the phases come from timed runs with a
    HIP event between every two phases (timing-only events without the
    system-scope fence, DeviceEvent), alternating with the first kind;
    medians over the runs.
    MFMA utilisation: attention FLOPs = sum over query heads and rows of
    4*D*|visible keys| (the ideal mask), gate FLOPs = 2*(2D*inner + inner)
    per token and head, against the dense bf16 / fp32 peaks."""
    import torch
    import wgkv
    from wgkv import ops, workloads
    from wgkv.cache import DualCache
    from wgkv.layers import WGKVConfig

    S, Hq, Hkv, D, W, CH = 32768, 32, 8, 128, 1024, 4096
    w = workloads.prefill_llama(S=S, Hq=Hq, Hkv=Hkv, D=D, W=W, device=dev)
    pk, kk, vv = w.pre_k.transpose(1, 2), w.k.transpose(1, 2), w.v.transpose(1, 2)  # (1, H, S, D) views
    mask = torch.empty(1, Hkv, S, dtype=torch.bool, device=dev)
    scores = torch.empty(1, Hkv, S, dtype=torch.float32, device=dev)
    out = torch.empty(S, Hq, D, dtype=torch.bfloat16, device=dev)
    cfg = WGKVConfig(num_hidden_layers=1, num_attention_heads=Hq, num_key_value_heads=Hkv, head_dim=D,
                     hidden_size=Hq * D, local_window_size=W, max_tokens_per_head=S + W,
                     max_total_tokens=Hkv * (S + W) + 4096)
    cache = DualCache()
    cache.initialize(cfg, D, torch.bfloat16, dev)
    snap = (cache.block_table.clone(), cache.global_lengths.clone(), cache.next_free_block_dev.clone(),
            cache.local_is_global.clone())
    chunks = [(c0, min(CH, S - c0)) for c0 in range(0, S, CH)]
    phases = ("gate", "admit", "sparse_attn", "ring")
    # per timed run: the prompt between two events, the phase-timed prompt
    # (first to last event) and its phases, the host's enqueue time
    runs = {"total": [], "marked": [], "phases": [], "host": []}
    gate_mod = [w.gate]

    n_ev = 1 + len(phases) * len(chunks)
    try:  # created once, re-recorded
        pool = [DeviceEvent() for _ in range(n_ev)]
        ev_kind = DeviceEvent.KIND + " (timing-only events)"
    except (OSError, AttributeError, RuntimeError) as exc:  # the runtime's symbols not reachable: torch's events
        pool = [torch.cuda.Event(enable_timing=True) for _ in range(n_ev)]
        ev_kind = f"torch.cuda.Event (default release; {type(exc).__name__}: {exc})"

    def run(timed):
        """timed: None (warm-up), "total" (events around the prompt) or
        "phases" (an event between every two phases)."""
        cache.block_table.copy_(snap[0])
        cache.global_lengths.copy_(snap[1])
        cache.next_free_block_dev.copy_(snap[2])
        cache.local_is_global.copy_(snap[3])
        ev = []

        def mark(force=False):
            if timed == "phases" or (timed == "total" and force):
                e = pool[len(ev)]
                e.record()
                ev.append(e)

        mark(True)
        h0 = time.perf_counter()
        for c0, C in chunks:
            sl = slice(c0, c0 + C)
            gate_mod[0].scores_and_mask(pk[:, :, sl], kk[:, :, sl], None, w.threshold,
                                        scores_out=scores[:, :, sl], mask_out=mask[:, :, sl])
            mark()
            st = ops.ChunkStep(cache, 0, w.q[0, sl], w.k[0, sl], w.v[0, sl], mask[0, :, sl], c0,
                               softmax_scale=D ** -0.5, out=out[sl])
            st.admit()
            mark()
            st.attend()
            mark()
            st.ring()
            mark()
        if timed == "total":
            mark(True)
            runs["host"].append((time.perf_counter() - h0) * 1000)
        if timed:
            torch.cuda.synchronize()
        if timed == "phases":
            runs["phases"].append({p: sum(ev[4 * n + k].elapsed_time(ev[4 * n + k + 1]) for n in range(len(chunks)))
                                   for k, p in enumerate(phases)})
            runs["marked"].append(ev[0].elapsed_time(ev[-1]))
        elif timed == "total":
            runs["total"].append(ev[0].elapsed_time(ev[-1]))

    def timed_runs():
        """Medians over the timed runs (the two kinds alternate, so both see
        the same warm GPU)."""
        for v in runs.values():
            v.clear()
        for _ in range(warmup):
            run(None)
        torch.cuda.synchronize()
        for _ in range(steps):
            run("total")
            run("phases")
        med = lambda xs: sorted(xs)[len(xs) // 2]
        return (med(runs["total"]), med(runs["marked"]), {p: med([r[p] for r in runs["phases"]]) for p in phases},
                med(runs["host"]))

    t_total, t_marked, ms, t_host = timed_runs()
    if int(cache.status.item()) != 0:
        raise RuntimeError("config-4 prefill ran out of cache capacity")
    pairs = workloads.visible_pairs(mask[0], W)
    attn_flop = float((pairs * (Hq // Hkv)).sum().item()) * 4 * D
    inner = 4 * D
    gate_flop = 2.0 * (2 * D * inner + inner) * S * Hkv
    gate_l1_flop = 2.0 * 2 * D * inner * S * Hkv
    planes = 1 if w.gate.precision(torch.bfloat16) else 3
    admitted = mask.float().mean().item()
    # the same gate with fp32 parameters (fp32 arithmetic and scores), per chunk
    import copy
    g32 = copy.deepcopy(w.gate).float()
    sc32 = torch.empty_like(scores)
    mk32 = torch.empty_like(mask)

    def gate32():
        for c0, C in chunks:
            sl = slice(c0, c0 + C)
            g32.scores_and_mask(pk[:, :, sl], kk[:, :, sl], None, w.threshold, scores_out=sc32[:, :, sl],
                                mask_out=mk32[:, :, sl])

    t_gate32 = time_op(gate32, steps, warmup) / len(chunks)
    # BASELINE config 4 as stated ("fp32 scores"): the whole pipeline with the
    # fp32-parameter gate (its own admission mask, hence its own attention
    # work); run after the bf16 pipeline's figures and masks are taken
    bf16_mask = mask.clone()
    gate_mod[0] = g32
    t_total32, t_marked32, ms32, _ = timed_runs()
    if int(cache.status.item()) != 0:
        raise RuntimeError("config-4 prefill (fp32 scores) ran out of cache capacity")
    pairs32 = workloads.visible_pairs(mask[0], W)
    attn_flop32 = float((pairs32 * (Hq // Hkv)).sum().item()) * 4 * D
    as_stated = {"gate_parameters": "float32", "scores": "float32",
                 "admitted_frac": round(mask.float().mean().item(), 4),
                 "ms_per_chunk": round(t_total32 / len(chunks), 4),
                 "ms_per_chunk_phase_timed": round(t_marked32 / len(chunks), 4),
                 "ms_per_chunk_by_phase": {p: round(ms32[p] / len(chunks), 4) for p in phases},
                 "sparse_attn_tflop": round(attn_flop32 / 1e12, 4),
                 "sparse_attn_mfma_frac_bf16": round(attn_flop32 / ms32["sparse_attn"] / 1e9 / BF16_PEAK_TFLOPS, 4)}
    mask.copy_(bf16_mask)
    # the one-shot kernel over the whole prompt, for comparison (same visible set)
    md = wgkv.generate_sparse_indices(mask, W, 1, Hkv, S)
    out1 = torch.empty_like(w.q)
    t_one = time_op(lambda: wgkv.sparse_attn_func(w.q, w.k, w.v, *md, out=out1), steps, warmup)
    return {
        "workload": "prefill_llama_32k_chunked (BASELINE config 4: 32K prompt in 8 chunks of 4096, one layer)",
        "admitted_frac": round(admitted, 4),
        "ms_per_chunk": round(t_total / len(chunks), 4),
        "ms_prompt": round(t_total, 4),
        "ms_per_chunk_by_phase": {p: round(ms[p] / len(chunks), 4) for p in phases},
        "ms_per_chunk_phase_timed": round(t_marked / len(chunks), 4),
        "host_enqueue_ms_per_chunk": round(t_host / len(chunks), 4),
        "phase_events": ev_kind + ", one between every two phases",
        "gate_parameters": "bfloat16 (the reference's inference loads the gate in bf16)",
        "config4_as_stated": as_stated,
        "sparse_attn": {"tflop": round(attn_flop / 1e12, 4), "tflops": round(attn_flop / ms["sparse_attn"] / 1e9, 1),
                        "mfma_frac_bf16": round(attn_flop / ms["sparse_attn"] / 1e9 / BF16_PEAK_TFLOPS, 4),
                        "one_shot_ms": round(t_one, 4),
                        "one_shot_mfma_frac_bf16": round(attn_flop / t_one / 1e9 / BF16_PEAK_TFLOPS, 4),
                        "dense_causal_tflop": round(4.0 * D * Hq * S * (S + 1) / 2 / 1e12, 3)},
        # bf16 inputs: the first layer runs on the bf16 matrix core -- bf16
        # parameters (the reference's inference) over one weight plane at the
        # reference's bf16 rounding points, fp32 parameters over three planes
        # (3 bf16 products per fp32 multiply-add)
        "gate": {"gflop": round(gate_flop / 1e9, 2), "tflops": round(gate_flop / ms["gate"] / 1e9, 1),
                 "parameters": str(w.gate.conv1.weight.dtype).replace("torch.", ""),
                 "path": f"first layer on bf16 MFMA, weights in {planes} bf16 plane{'s' if planes > 1 else ''}",
                 "bf16_gflop_executed": round(planes * gate_l1_flop / 1e9, 2),
                 "mfma_frac_bf16": round(planes * gate_l1_flop / ms["gate"] / 1e9 / BF16_PEAK_TFLOPS, 4),
                 "fp32_parameters_ms_per_chunk": round(t_gate32, 4)},
    }


def quest_section(dev, steps, warmup):
    """QUEST page selection (the reference's comparison baseline) at Llama-8B
    decode shapes: one layer, batch 1, a 128K prompt with 20 % admitted
    (~27K cached tokens per KV head), token budget 4096.  Per decode step:
    the selection (page scores + top-k, one launch) and the decode attention
    over the selected pages, beside the attention over the whole cache."""
    import torch
    from wgkv import ops
    from wgkv.cache import DualCache
    from wgkv.layers import WGKVConfig

    S, H, G, D, W, budget = 131072, 8, 4, 128, 1024, 4096
    cfg = WGKVConfig(num_hidden_layers=1, num_attention_heads=H * G, num_key_value_heads=H, head_dim=D,
                     hidden_size=H * G * D, local_window_size=W, max_tokens_per_head=S + W,
                     max_total_tokens=H * (S + W), use_quest=True, quest_token_budget=budget)
    c = DualCache()
    c.initialize(cfg, D, torch.bfloat16, dev)
    g = torch.Generator(device=dev).manual_seed(0)
    k = torch.randn(H, S, D, generator=g, device=dev).to(torch.bfloat16)
    v = torch.randn(H, S, D, generator=g, device=dev).to(torch.bfloat16)
    m = torch.rand(H, S, generator=g, device=dev) < 0.2
    ops.prefill_admit(c, 0, k, v, m)
    ops.quest_update_bounds(c, 0)
    del k, v
    c.local_length = W
    seqlens = (W + c.global_lengths[0]).view(1, H).contiguous()
    q = torch.randn(1, 1, H * G, D, generator=g, device=dev).to(torch.bfloat16)  # (batch, 1, Hq, D)
    out = torch.empty_like(q)
    sel = {}

    def select():
        sel["r"] = ops.quest_select(c, 0, q[0, 0], W, budget)

    t_sel = time_op(select, steps, warmup)
    sl, bt = sel["r"]
    t_att_sel = time_op(lambda: ops.paged_decode_attn(q, c.k_cache(), c.v_cache(), sl, bt, D ** -0.5, out=out),
                        steps, warmup)
    t_att_full = time_op(lambda: ops.paged_decode_attn(q, c.k_cache(), c.v_cache(), seqlens,
                                                       c.block_table[0].unsqueeze(0), D ** -0.5, out=out),
                         steps, warmup)
    torch.cuda.synchronize()
    tok_full = int(seqlens.sum())
    tok_sel = int(sl.sum())
    return {"workload": "quest_b1_128k (one layer, 20 % admitted, budget 4096 tokens per head)",
            "cached_tokens": tok_full, "selected_tokens": tok_sel,
            "us": {"select": round(t_sel * 1e3, 1), "attention_selected": round(t_att_sel * 1e3, 1),
                   "attention_full_cache": round(t_att_full * 1e3, 1)},
            "bounds_bytes_read_per_step": int((c.global_lengths[0] // 16).sum()) * D * 2 * 2}


def snapkv_section(dev, runs=3):
    """SnapKV eviction (the reference's other comparison baseline) at config-5
    decode shapes: 32 layers x 8 KV heads of a Llama-3.1-8B cache, 80K-120K
    global tokens per head (~25.6M tokens, 13 GB of K+V in random page order), a full
    256-query window, ratio 0.2, max-pool 5.  Timed with HIP events around
    the four launches of wgkv_snapkv_evict; the cache state is restored
    between runs (not timed).  Also the cost of the call on a step that does
    not evict (the device trigger says no)."""
    import torch
    from wgkv import ops
    L, H, G, D, W, P, win = 32, 8, 4, 128, 1024, 16, 256
    g = torch.Generator(device=dev).manual_seed(0)
    lengths = torch.randint(80000, 120001, (L, H), generator=g, device=dev, dtype=torch.int32)
    lb = W // P
    mtph = W + 120064
    maxp = mtph // P
    gpages = (lengths + P - 1) // P
    total = L * H * lb + int(gpages.sum()) + 1
    i32 = dict(dtype=torch.int32, device=dev)
    table = torch.full((L, H, maxp), total - 1, **i32)
    table[:, :, :lb] = torch.arange(L * H * lb, **i32).view(L, H, lb)
    perm = (torch.randperm(total - 1 - L * H * lb, generator=g, device=dev) + L * H * lb).to(torch.int32)
    starts = torch.cumsum(gpages.flatten(), 0) - gpages.flatten()
    idx = torch.arange(maxp - lb, device=dev)[None, :]
    valid = idx < gpages.flatten()[:, None]
    src = (starts[:, None] + idx).clamp(max=perm.numel() - 1)
    table.view(L * H, maxp)[:, lb:] = torch.where(valid, perm[src], torch.full_like(src, total - 1, dtype=torch.int32))
    pool_k = torch.randn(total * P, D, generator=g, device=dev, dtype=torch.float32).to(torch.bfloat16)
    pool_v = torch.randn(total * P, D, generator=g, device=dev, dtype=torch.float32).to(torch.bfloat16)
    import types
    c = types.SimpleNamespace(
        num_layers=L, num_kv_heads=H, head_dim=D, block_size=P, local_window_size=W, max_tokens_per_head=mtph,
        total_blocks=total, block_pool_k=pool_k, block_pool_v=pool_v, block_table=table.clone(),
        global_lengths=lengths.clone(), free_block_ids_dev=torch.zeros(total, **i32),
        free_count_dev=torch.zeros(1, **i32),
        snapkv_query_buffer=torch.randn(L, win, H * G, D, generator=g, device=dev,
                                        dtype=torch.float32).to(torch.bfloat16),
        snapkv_state=torch.zeros(2, **i32))
    tokens = int(lengths.sum())

    def restore():
        c.block_table.copy_(table)
        c.global_lengths.copy_(lengths)
        c.free_count_dev.zero_()

    def evict(budget):
        ops.snapkv_evict(c, G, D ** -0.5, win, 5, 0.2, max_cached_tokens=budget)

    times = []
    for r in range(runs + 1):
        restore()
        torch.cuda.synchronize()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        evict(tokens - 1)
        end.record()
        torch.cuda.synchronize()
        if r:  # the first run loads the code objects and allocates the workspace
            times.append(start.elapsed_time(end))
    kept = int(c.global_lengths.sum())
    released = int(c.free_count_dev.item())
    t_idle = time_op(lambda: evict(1 << 40), 20, 5)
    flop = 2 * 2.0 * G * win * D * tokens
    return {"workload": "snapkv_llama8b_evict (32 layers x 8 KV heads, 80K-120K global tokens per head, window 256, "
                        "ratio 0.2, kernel 5)",
            "cached_tokens": tokens, "kept_tokens": kept, "released_pages": released,
            "ms_per_eviction": round(sum(times) / len(times), 3), "ms_runs": [round(t, 3) for t in times],
            "scoring_tflop": round(flop / 1e12, 3),
            "scoring_tflops": round(flop / (min(times) * 1e-3) / 1e12, 1),
            "us_per_step_without_eviction": round(t_idle * 1e3, 1)}


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
                               **host_cpu(), "kind": "port", "runs": len(cruns),
                               "sample": "oracle.llama_layer.OracleLayer fp32 on the host cores; median of runs"},
    }


def prefill_long_probe(dev):
    """The last 4096-token chunk of a 409,600-token prompt through one layer:
    every 64-row block streams its head's ~119K admitted K/V rows, so the
    chunk shows whether long-context chunks are bound by K/V re-reads (the
    FETCH_SIZE counter of its kernel, against the bytes the row blocks stream)
    or by the arithmetic."""
    import torch
    from wgkv import ops, workloads
    from wgkv.cache import DualCache
    from wgkv.layers import WGKVConfig

    S, Hq, Hkv, D, W, CH = 409600, 32, 8, 128, 1024, 4096
    w = workloads.prefill_llama(S=S, Hq=Hq, Hkv=Hkv, D=D, W=W, frac=0.3, device=dev)
    pk, kk = w.pre_k.transpose(1, 2), w.k.transpose(1, 2)
    mask = torch.empty(1, Hkv, S, dtype=torch.bool, device=dev)
    scores = torch.empty(1, Hkv, S, dtype=torch.float32, device=dev)
    out = torch.empty(S, Hq, D, dtype=torch.bfloat16, device=dev)
    cfg = WGKVConfig(num_hidden_layers=1, num_attention_heads=Hq, num_key_value_heads=Hkv, head_dim=D,
                     hidden_size=Hq * D, local_window_size=W, max_tokens_per_head=S + W,
                     max_total_tokens=Hkv * (S + W) + 4096)
    cache = DualCache()
    cache.initialize(cfg, D, torch.bfloat16, dev)
    last = None
    for c0 in range(0, S, CH):
        sl = slice(c0, c0 + CH)
        w.gate.scores_and_mask(pk[:, :, sl], kk[:, :, sl], None, w.threshold, scores_out=scores[:, :, sl],
                               mask_out=mask[:, :, sl])
        st = ops.ChunkStep(cache, 0, w.q[0, sl], w.k[0, sl], w.v[0, sl], mask[0, :, sl], c0,
                           softmax_scale=D ** -0.5, out=out[sl])
        st.admit()
        st.attend()
        st.ring()
        last = st
    torch.cuda.synchronize()
    # visible pairs of the last chunk's rows (the ideal mask, as workloads.visible_pairs)
    m = mask[0].to(torch.int64)
    cum = torch.cumsum(m, dim=1)
    i = torch.arange(S - CH, S, device=dev)
    start = torch.clamp((i // 64) * 64 - W + 1, min=0)
    before = cum[:, start - 1]
    pairs = float(((i - start + 1)[None, :] + before).sum().item())
    flop = pairs * (Hq // Hkv) * 4 * D
    streamed = 0.0  # K and V bytes the chunk's 64-row blocks stream (admitted columns + band, per block)
    for r0 in range(S - CH, S, 64):
        s0 = max(0, r0 - W + 1)
        streamed += float(((cum[:, s0 - 1] if s0 > 0 else torch.zeros_like(cum[:, 0])) + (r0 + 64 - s0)).sum().item())
    streamed *= D * 2 * 2
    ms = time_op(last.attend, 5, 2)
    src = torch.ones(1 << 29, dtype=torch.bfloat16, device=dev)  # 1 GiB
    dst = torch.empty_like(src)
    dst.copy_(src)
    torch.cuda.synchronize()
    return {"prefill_long_probe": {
        "workload": "last 4096-token chunk of a 409,600-token prompt, one Llama-8B layer (32 q / 8 KV heads, D 128, "
                    "W 1024, 30 % admitted)",
        "admitted_per_head_before_chunk": round(float(m[:, :S - CH].sum(dim=1).float().mean().item())),
        "attention_ms": round(ms, 4), "tflop": round(flop / 1e12, 3),
        "mfma_frac_bf16": round(flop / (ms * 1e-3) / 1e12 / BF16_PEAK_TFLOPS, 4),
        "kv_bytes_streamed_by_row_blocks": int(streamed),
        "copy_bytes_read": src.numel() * 2}}


def e2e_section(args):
    """BASELINE config 5 (the reference's scripts/profiling.py run): a random-
    initialised bf16 Llama-3.1-8B-shaped model, uniform random token ids, the
    prompt prefilled in 4096-token chunks, then greedy decode steps; once with
    the learned gate (bias calibrated to admit ``--e2e-admit`` of the first
    chunk per head and layer) and once with every token admitted (the
    reference's "full" recipe: g_expand 0, random_sparsity 0.0).  Prefill time (TTFT), mean decode step
    (TPOT; each step one replay of a captured HIP graph of the whole model's
    decode step), tokens/s, cached tokens per (layer, head) and KV memory."""
    import torch
    from wgkv import e2e

    dev = torch.device("cuda:0")
    if args.e2e_model == "qwen3-8b":
        ec = e2e.E2EConfig.qwen3_8b(**({} if args.e2e_layers == 32 else {"num_hidden_layers": args.e2e_layers}))
    else:
        ec = e2e.E2EConfig(num_hidden_layers=args.e2e_layers)
    S, steps, W = args.e2e_prompt, args.e2e_steps, ec.local_window_size
    torch.manual_seed(0)
    prev = torch.get_default_dtype()
    torch.set_default_dtype(torch.bfloat16)
    with torch.device(dev):
        model = e2e.LlamaLite(ec, gated=True, max_tokens_per_head=S + steps + 2 * W,
                              max_total_tokens=ec.num_hidden_layers * ec.num_key_value_heads * (S + steps + 2 * W))
    torch.set_default_dtype(prev)
    model.init_weights(seed=0)
    ids = torch.randint(0, ec.vocab_size, (1, S), generator=torch.Generator().manual_seed(0)).to(dev)

    def log(msg):
        print(f"[e2e] {msg}", file=sys.stderr, flush=True)

    tag = "qwen3_8b" if args.e2e_model == "qwen3-8b" else "llama8b"
    out = {"workload": f"e2e_{tag}_{S // 1000}k (BASELINE config 5): {ec.num_hidden_layers} layers, "
                       f"hidden {ec.hidden_size}, FFN {ec.intermediate_size}, vocab {ec.vocab_size}, "
                       f"prompt {S} in {args.e2e_chunk}-token chunks, {steps} greedy decode steps, W {W}",
           "data": "synthetic: random-init bf16 weights, uniform random token ids",
           "gating": ("deferred (g_defer, as scripts/profiling.py:212-213): decode steps re-gate the window "
                      "when its last slot is written" if ec.g_defer else "every token"),
           "full_run": "g_expand 0, random_sparsity 0.0 (README.md:128-136): every token admitted",
           "decode": "each step one replay of a captured HIP graph of the whole model's step"}
    log("calibrating the gates")
    e2e.calibrate_gates(model, ids, args.e2e_admit)
    # pass-through (phase "warmup") until a run switches them on; graph runs never do
    timers = e2e.install_timing(model, args.e2e_profile) if args.e2e_profile else None
    for name, gated in (("gated", True), ("full", False)):
        # the full run is the reference's own recipe (README.md:128-136:
        # --g_expand 0 --random_sparsity 0.0, with g_defer forced on by
        # profiling.py:211-213): every token admitted by the random rule
        model.cfg.g_expand = ec.g_expand if gated else 0.0
        model.cfg.random_sparsity = None if gated else 0.0
        # the gated pool holds the expected admitted share with margin; the full pool every token
        per_head = S + steps + 2 * W if not gated else int(S * min(1.0, 1.5 * args.e2e_admit)) + steps + 2 * W
        model.cfg.max_tokens_per_head = S + steps + 2 * W
        model.cfg.max_total_tokens = ec.num_hidden_layers * ec.num_key_value_heads * per_head
        log(f"{name}: prefill {S} tokens")
        r = e2e.run(model, ids, steps, chunk=args.e2e_chunk, progress=log, graph=True)
        torch.cuda.empty_cache()
        dm = sorted(r.decode_ms)
        tpot = sum(r.decode_ms) / len(r.decode_ms)
        out[name] = {"prefill_ms": round(r.prefill_ms, 1), "prefill_tokens_per_s": round(S / (r.prefill_ms / 1e3), 1),
                     "tpot_ms": round(tpot, 3), "tpot_median_ms": round(dm[len(dm) // 2], 3),
                     "decode_tokens_per_s": round(1000.0 / tpot, 2),
                     "avg_tokens_per_head_before_decode": round(r.tokens_before),
                     "avg_tokens_per_head_after_decode": round(r.tokens_after),
                     "model_gib": round(r.model_mib / 1024, 2), "kv_cache_gib": round(r.kv_mib / 1024, 2),
                     "first_tokens": r.tokens[:8]}
        log(f"{name}: {out[name]}")
        if timers is not None:
            log(f"{name}: eager run timing {args.e2e_profile}, MLP and LM head per phase")
            for key in timers.ms:
                timers.ms[key] = 0.0
            rp = e2e.run(model, ids, args.e2e_profile_steps, chunk=args.e2e_chunk, progress=log, timers=timers)
            torch.cuda.empty_cache()
            out[name]["profile"] = {"attn_granularity": args.e2e_profile, "decode_steps": args.e2e_profile_steps,
                                    "eager_prefill_ms": round(rp.prefill_ms, 1),
                                    "eager_tpot_ms": round(sum(rp.decode_ms) / len(rp.decode_ms), 3),
                                    **timers.report()}
            log(f"{name}: {out[name]['profile']}")
    out["gated_vs_full"] = {"prefill_speedup": round(out["full"]["prefill_ms"] / out["gated"]["prefill_ms"], 3),
                            "decode_speedup": round(out["full"]["tpot_ms"] / out["gated"]["tpot_ms"], 3),
                            "kv_ratio": round(out["gated"]["kv_cache_gib"] / out["full"]["kv_cache_gib"], 3)}
    return out


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU; --gpus must be 1",
                          "n_gpus": args.gpus}))
        sys.exit(2)
    if args.e2e:
        print(json.dumps({"e2e": e2e_section(args)}), flush=True)
        return
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

    if args.prefill_long_probe:
        print(json.dumps(prefill_long_probe(dev)), flush=True)
        return
    if args.traffic_probe:
        src = torch.ones(1 << 29, dtype=torch.bfloat16, device=dev)  # 1 GiB
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        for _ in range(5):
            step()
        torch.cuda.synchronize()
        print(json.dumps({"traffic_probe": {"copy_bytes_read": src.numel() * 2, "copy_bytes_written": dst.numel() * 2,
                                            "decode_algorithmic_bytes": w.algorithmic_bytes()}}), flush=True)
        return
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
            "traffic": DECODE_TRAFFIC_BYTES,
            "traffic_source": DECODE_TRAFFIC_SOURCE,
            "bytes_per_launch": nbytes,
            "launch": "wgkv_paged_decode_attn = decode_split_kernel + decode_merge_kernel (B*Hkv >= 32; fewer heads: one launch, the last chunk of a head merges)",
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
            mg = time_graph(lambda: wgkv.paged_decode_attn(ws.q, ws.k_cache, ws.v_cache, ws.cache_seqlens,
                                                           ws.block_table, ws.softmax_scale, out=o2))
            b2 = ws.algorithmic_bytes()
            line = {"workload": name, "ms": round(m2, 5), "bytes": b2,
                    "GB/s": round(b2 / (m2 * 1e-3) / 1e9, 1), "cached_tokens": ws.total_tokens,
                    "ms_graph": round(mg, 5), "GB/s_graph": round(b2 / (mg * 1e-3) / 1e9, 1),
                    "frac_graph": round(b2 / (mg * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}
            if name.endswith("128k"):
                # the same shape over 4 distinct caches in turn (~0.4 GB, more
                # than the 256 MB Infinity Cache), so that repeated calls
                # cannot be served from the last call's cached lines
                rot = [ws] + [workloads.decode_beta(ctx=131072, device=dev, seed=sd) for sd in (1, 2, 3)]
                outs = [o2] + [torch.empty_like(x.q) for x in rot[1:]]
                fns = [(lambda x=x, o=o: wgkv.paged_decode_attn(x.q, x.k_cache, x.v_cache, x.cache_seqlens,
                                                                 x.block_table, x.softmax_scale, out=o))
                       for x, o in zip(rot, outs)]
                mr = time_graph(lambda it=iter(range(1 << 30)): fns[next(it) % len(fns)]())
                br = sum(x.algorithmic_bytes() for x in rot) / len(rot)
                line["rotating_4_caches"] = {"ms_graph": round(mr, 5), "bytes_avg": int(br),
                                             "GB/s_graph": round(br / (mr * 1e-3) / 1e9, 1)}
                del rot, outs, fns
            sec.append(line)
            del ws
        result["secondary"] = sec
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(w, args.cpu_seconds)
    del w, out
    torch.cuda.empty_cache()
    if not args.no_prefill:
        result["prefill"] = prefill_section(dev, max(10, args.steps // 2), max(4, args.warmup // 2))
        torch.cuda.empty_cache()
    if not args.no_secondary:
        result["quest"] = quest_section(dev, args.steps, args.warmup)
        torch.cuda.empty_cache()
        result["snapkv"] = snapkv_section(dev)
        torch.cuda.empty_cache()
    if not args.no_layer:
        result["layer_config1"] = layer_section(dev, args.cpu_seconds)
    if not args.no_e2e:
        torch.cuda.empty_cache()
        try:
            result["e2e"] = e2e_section(args)
        except Exception as exc:  # the decode and prefill lines above stand on their own
            result["e2e"] = {"error": f"{type(exc).__name__}: {exc}"}
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
