"""Write golden vectors with the reference's own implementation.

Run once in the development container (the only place the reference
checkout exists):  ``python tests/golden/make_golden.py /path/to/WG-KV
[gate|gate_bf16|cache|quest|snapkv ...]`` (all when none is named).

Only functions that no closed form or reference test pins are run here:

* ``GatingPredictor.forward`` (src/modeling_layers.py:134-205), fast and conv
  paths -- float32 scores, and the same module converted to bf16 on bf16
  inputs (the inference scripts' configuration) -- bf16 scores;
* ``quest_select_blocks`` (:452-576) on seeded cache states, bf16 and fp32
  -- the selected tables and lengths and the page ranking it made;
* ``snapkv_evict`` (:595-671) on seeded cache states, bf16 and fp32 -- the
  pooled scores and dropped positions of every head, the resulting lengths,
  tables, free list and kept contents;
* the dual-cache state machine through ``self_attn_forward_patch_inference``
  (:1452-1509) -> ``prefill_wrapper`` (:1183-1376), ``decode_wrapper``
  (:1379-1449), ``migrate_local_kv_to_global`` (:674-763),
  ``refresh_local_is_global`` (:1169-1180).

The reference attention kernels are replaced by stubs that record the decode
metadata (``cache_seqlens``, ``block_table``) and return zeros: attention is
pinned separately.  Outputs are written as ``.npz`` data (no pickles) plus a
checksum of the inputs, which the tests regenerate from the same seeds.
"""
import importlib.util
import json
import os
import sys
import types

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)
import scenarios  # noqa: E402


def load_reference(root):
    import transformers  # noqa: F401  (the module uses relative imports inside it)
    path = os.path.join(root, "src", "modeling_layers.py")
    spec = importlib.util.spec_from_file_location("transformers._wgkv_reference_layers", path)
    mod = importlib.util.module_from_spec(spec)
    sys.modules[spec.name] = mod
    spec.loader.exec_module(mod)
    return mod


def make_gate(ref, H, D, g_expand, params, fast_path, g_inputs=("pre_k", "post_k"), act="gelu"):
    g = ref.GatingPredictor(D, H, list(g_inputs), act, g_expand, 1e-3, True, fast_path)
    sd = {k: v.clone() for k, v in params.items()}
    g.load_state_dict(sd, strict=True)
    return g.eval()


def gate_golden(ref):
    out = {}
    for name, sc in scenarios.GATE_SCENARIOS.items():
        params, pre_k, post_k, value = scenarios.gate_inputs(sc)
        with torch.no_grad():
            fast = make_gate(ref, sc["H"], sc["D"], sc["g_expand"], params, True)(pre_k, post_k, value)
            conv = make_gate(ref, sc["H"], sc["D"], sc["g_expand"], params, False)(pre_k, post_k, value)
        out[f"{name}.fast"] = fast.numpy()
        out[f"{name}.conv"] = conv.numpy()
        out[f"{name}.inputs_sha256"] = np.frombuffer(
            scenarios.checksum(pre_k, post_k, *params.values()).encode(), dtype=np.uint8)
    np.savez_compressed(os.path.join(HERE, "gate_golden.npz"), **out)
    print("gate:", {k: v.shape for k, v in out.items() if not k.endswith("sha256")})


def gate_bf16_golden(ref):
    """The reference's GatingPredictor converted to bf16 (as its inference
    scripts load the gate checkpoint) on bf16 inputs: bf16 scores, stored as
    their int16 bit patterns."""
    out = {}
    for name, sc in scenarios.GATE_BF16_SCENARIOS.items():
        params, pre_k, post_k, value = scenarios.gate_inputs_bf16(sc)
        for fast in (True, False):
            g = make_gate(ref, sc["H"], sc["D"], sc["g_expand"], {k: v.float() for k, v in params.items()},
                          fast, sc["g_inputs"], sc["act"]).to(torch.bfloat16)
            with torch.no_grad():
                s = g(pre_k, post_k, value)
            assert s.dtype == torch.bfloat16
            out[f"{name}.{'fast' if fast else 'conv'}"] = s.view(torch.int16).numpy()
        out[f"{name}.inputs_sha256"] = np.frombuffer(
            scenarios.checksum(pre_k, post_k, value, *params.values()).encode(), dtype=np.uint8)
    np.savez_compressed(os.path.join(HERE, "gate_bf16_golden.npz"), **out)
    print("gate bf16:", {k: v.shape for k, v in out.items() if not k.endswith("sha256")})


def fake_attention_module(ref, sc, layer_idx, record, gate):
    cfg = types.SimpleNamespace(
        num_hidden_layers=sc["L"], num_key_value_heads=sc["H"], local_window_size=sc["W"],
        block_size=16, max_total_tokens=sc["L"] * sc["H"] * sc["max_tokens_per_head"],
        max_tokens_per_head=sc["max_tokens_per_head"], use_quest=False, g_defer=sc["g_defer"],
        snapkv_enabled=False, use_baseline=False, g_expand=4.0, random_sparsity=None,
        g_threshold=0.1,
    )
    self = types.SimpleNamespace()
    self.config = cfg
    self.layer_idx = layer_idx
    self.head_dim = sc["D"]
    self.num_key_value_groups = sc["G"]
    self.scaling = sc["D"] ** -0.5
    self.prefill_wrapper = ref.prefill_wrapper
    self.decode_wrapper = ref.decode_wrapper

    def prefill_kernel(q, k, v, *meta, softmax_scale=None, causal=True, return_softmax_lse=False):
        return torch.zeros_like(q)

    def decode_kernel_handle(q, k_cache, v_cache, cache_seqlens, block_table, softmax_scale):
        record.append((cache_seqlens.clone(), block_table.clone()))
        return lambda: torch.zeros_like(q)

    self.prefill_kernel = prefill_kernel
    self.decode_kernel_handle = decode_kernel_handle
    self.decode_kernel_executor = lambda f: f()
    if gate is not None:
        self.g_predictors = gate
    return self


def logical_hash(cache, L, H, W, P, D, cur_len):
    parts = []
    kc = cache.block_pool_k.view(cache.total_blocks, P, D)
    vc = cache.block_pool_v.view(cache.total_blocks, P, D)
    for l in range(L):
        for h in range(H):
            T = cur_len + int(cache.global_lengths[l, h])
            n = (T + P - 1) // P
            ids = cache.block_table[l, h, :n].long()
            parts.append(kc[ids].reshape(-1, D)[:T])
            parts.append(vc[ids].reshape(-1, D)[:T])
    return scenarios.checksum(*parts)


def cache_golden(ref):
    out = {}
    meta = {}
    for name, sc in scenarios.CACHE_SCENARIOS.items():
        inp = scenarios.cache_inputs(sc)
        L, H, W, D = sc["L"], sc["H"], sc["W"], sc["D"]
        gates = None
        if sc["g_defer"]:
            gates = [make_gate(ref, H, D, 4.0, scenarios.defer_bias_shift(p), True) for p in inp["gates"]]
        record = []
        mods = [fake_attention_module(ref, sc, l, record, gates[l] if gates else None) for l in range(L)]
        cache = types.SimpleNamespace()
        with torch.no_grad():
            for l in range(L):
                q, pk, k, v, mask = inp["prompt"][l]
                ref.self_attn_forward_patch_inference(
                    mods[l], cache, (1, sc["S"]), q, pk, k, v, mask.to(torch.float32))
            out[f"{name}.after_prefill.block_table"] = cache.block_table.numpy().copy()
            out[f"{name}.after_prefill.global_lengths"] = cache.global_lengths.numpy().copy()
            out[f"{name}.after_prefill.local_is_global"] = cache.local_is_global.numpy().copy()
            meta[f"{name}.after_prefill"] = dict(next_free_block=int(cache.next_free_block),
                                                 local_ptr=int(cache.local_ptr),
                                                 local_length=int(cache.local_length))
            for step in inp["steps"]:
                for l in range(L):
                    q, pk, k, v, mask = step[l]
                    g = None if mask is None else mask.to(torch.float32)
                    ref.self_attn_forward_patch_inference(mods[l], cache, (1, 1), q, pk, k, v, g)
        cur_len = cache.local_length
        out[f"{name}.final.block_table"] = cache.block_table.numpy().copy()
        out[f"{name}.final.global_lengths"] = cache.global_lengths.numpy().copy()
        out[f"{name}.final.local_is_global"] = cache.local_is_global.numpy().copy()
        out[f"{name}.decode_seqlens"] = torch.stack([r[0].reshape(-1) for r in record]).numpy()
        out[f"{name}.decode_block_table_sha256"] = np.frombuffer(
            scenarios.checksum(*[r[1] for r in record]).encode(), dtype=np.uint8)
        meta[name] = dict(next_free_block=int(cache.next_free_block), local_ptr=int(cache.local_ptr),
                          local_length=int(cache.local_length),
                          logical_sha256=logical_hash(cache, L, H, W, 16, D, cur_len),
                          inputs_sha256=scenarios.checksum(
                              *[t for lay in inp["prompt"] for t in lay],
                              *[t for st in inp["steps"] for lay in st for t in lay if t is not None]))
        print(name, meta[name])
    # capacity error: one head admits more than max_tokens_per_head allows
    sc = dict(scenarios.CACHE_SCENARIOS["long_prompt"], max_tokens_per_head=256)
    inp = scenarios.cache_inputs(sc)
    cache = types.SimpleNamespace()
    mod = fake_attention_module(ref, sc, 0, [], None)
    q, pk, k, v, mask = inp["prompt"][0]
    try:
        ref.self_attn_forward_patch_inference(mod, cache, (1, sc["S"]), q, pk, k, v, mask.to(torch.float32))
        meta["capacity_error_raises"] = False
    except AssertionError:
        meta["capacity_error_raises"] = True
    np.savez_compressed(os.path.join(HERE, "cache_golden.npz"), **out)
    with open(os.path.join(HERE, "cache_golden.json"), "w") as f:
        json.dump(meta, f, indent=1, sort_keys=True)


def snapkv_golden(ref):
    """The reference's snapkv_evict (src/modeling_layers.py:595-671) on the
    seeded states of scenarios.SNAPKV_SCENARIOS, in bf16 and in fp32: per
    evicted head (call order) its pooled scores (the input of its
    torch.topk) and dropped positions, then the lengths, tables, free list
    and a checksum of every head's kept tokens in order."""
    out, meta = {}, {}
    for name, sc in scenarios.SNAPKV_SCENARIOS.items():
        st = scenarios.snapkv_state(sc)
        L, H, G, D, W = sc["L"], sc["H"], sc["G"], sc["D"], sc["W"]
        lb = W // 16
        cfg = types.SimpleNamespace(num_hidden_layers=L, num_key_value_heads=H, snapkv_evict_ratio=sc["ratio"],
                                    snapkv_kernel_size=sc["ksz"], block_size=16, snapkv_window_size=sc["win"])
        mod = types.SimpleNamespace(config=cfg, num_key_value_groups=G, head_dim=D, scaling=D ** -0.5,
                                    layer_idx=L - 1)
        pkv = types.SimpleNamespace(block_pool_k=st["pool_k"].clone(), block_pool_v=st["pool_v"].clone(),
                                    block_table=st["block_table"].clone(),
                                    global_lengths=st["global_lengths"].clone(), free_block_ids=list(st["free_ids"]),
                                    total_blocks=st["total_blocks"], snapkv_query_buffer=st["qbuf"].clone(),
                                    snapkv_query_length=sc["win"])
        calls = []
        orig = torch.topk

        def recording_topk(*args, **kwargs):
            r = orig(*args, **kwargs)
            calls.append((args[0].detach().float().clone(), r.indices.clone()))
            return r

        torch.topk = recording_topk
        try:
            with torch.no_grad():
                ref.snapkv_evict(mod, pkv, torch.device("cpu"), lb)
        finally:
            torch.topk = orig
        heads = [(l, h) for l in range(L) for h in range(H)
                 if int(int(st["global_lengths"][l, h]) * sc["ratio"]) > 0]
        assert len(heads) == len(calls)
        out[f"{name}.heads"] = np.array(heads, dtype=np.int32).reshape(-1, 2)
        out[f"{name}.scores"] = torch.cat([c[0] for c in calls]).numpy()
        out[f"{name}.evicted"] = torch.cat([torch.sort(c[1]).values for c in calls]).to(torch.int32).numpy()
        out[f"{name}.global_lengths"] = pkv.global_lengths.numpy().copy()
        out[f"{name}.block_table"] = pkv.block_table.numpy().copy()
        out[f"{name}.free_ids"] = np.array(pkv.free_block_ids, dtype=np.int32)
        kept_k = scenarios.logical_tokens(pkv.block_pool_k, pkv.block_table, pkv.global_lengths, lb)
        kept_v = scenarios.logical_tokens(pkv.block_pool_v, pkv.block_table, pkv.global_lengths, lb)
        meta[name] = dict(
            inputs_sha256=scenarios.checksum(st["pool_k"], st["pool_v"], st["qbuf"], st["block_table"]),
            kept_sha256=scenarios.checksum(*[kept_k[k] for k in sorted(kept_k)], *[kept_v[k] for k in sorted(kept_v)]))
        print(name, meta[name], "evicted heads", heads)
    np.savez_compressed(os.path.join(HERE, "snapkv_golden.npz"), **out)
    with open(os.path.join(HERE, "snapkv_golden.json"), "w") as f:
        json.dump(meta, f, indent=1, sort_keys=True)


def quest_golden(ref):
    """The reference's quest_select_blocks (src/modeling_layers.py:452-576)
    at each step of scenarios.QUEST_SCENARIOS: the returned cache_seqlens and
    block_table, and per head that ranks its full pages the page scores and
    the chosen positions (the input and output of its torch.topk)."""
    out, meta = {}, {}
    for name, sc in scenarios.QUEST_SCENARIOS.items():
        st = scenarios.quest_state(sc)
        H, G, D, W = sc["H"], sc["G"], sc["D"], sc["W"]
        pkv = types.SimpleNamespace(block_table=st["block_table"], global_lengths=st["global_lengths"],
                                    quest_block_key_min=st["key_min"], quest_block_key_max=st["key_max"])
        meta[name] = dict(inputs_sha256=scenarios.checksum(st["pool_k"], st["key_min"], st["key_max"],
                                                           st["block_table"], *st["qs"]))
        for i, (local, budget) in enumerate(sc["steps"]):
            cfg = types.SimpleNamespace(num_key_value_heads=H, block_size=16, quest_token_budget=budget)
            mod = types.SimpleNamespace(config=cfg, num_key_value_groups=G, head_dim=D, layer_idx=0)
            calls = []
            orig = torch.topk

            def recording_topk(*args, **kwargs):
                r = orig(*args, **kwargs)
                calls.append((args[0].detach().float().clone(), r.indices.clone()))
                return r

            torch.topk = recording_topk
            try:
                with torch.no_grad():
                    seqlens, table = ref.quest_select_blocks(mod, st["qs"][i].view(1, H * G, 1, D), pkv, W // 16,
                                                             torch.device("cpu"), local)
            finally:
                torch.topk = orig
            out[f"{name}.{i}.seqlens"] = seqlens.numpy().copy()
            out[f"{name}.{i}.block_table"] = table.numpy().copy()
            out[f"{name}.{i}.ranked_scores"] = (torch.cat([c[0] for c in calls]).numpy() if calls
                                                else np.zeros(0, np.float32))
            out[f"{name}.{i}.ranked_choice"] = (torch.cat([c[1] for c in calls]).to(torch.int32).numpy() if calls
                                                else np.zeros(0, np.int32))
            print(name, i, (local, budget), "seqlens", seqlens.tolist(), "ranked heads", len(calls))
    np.savez_compressed(os.path.join(HERE, "quest_golden.npz"), **out)
    with open(os.path.join(HERE, "quest_golden.json"), "w") as f:
        json.dump(meta, f, indent=1, sort_keys=True)


def main():
    root = sys.argv[1] if len(sys.argv) > 1 else "/root/reference"
    ref = load_reference(root)
    torch.set_num_threads(4)
    only = sys.argv[2:] or ["gate", "gate_bf16", "cache", "snapkv", "quest"]
    if "gate" in only:
        gate_golden(ref)
    if "gate_bf16" in only:
        gate_bf16_golden(ref)
    if "cache" in only:
        cache_golden(ref)
    if "snapkv" in only:
        snapkv_golden(ref)
    if "quest" in only:
        quest_golden(ref)


if __name__ == "__main__":
    main()
