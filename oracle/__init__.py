"""CPU oracle for the write-gated dual-cache KV path.

TEST INFRASTRUCTURE ONLY.  Nothing in the product package imports this
package: only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may use it, and only as the checker (or
as the timed CPU baseline), never as the thing that produces product results.

Every function restates the reference's algorithm from its source text and
cites the reference file:line it follows (paths relative to the reference
checkout ``EMCLab-Sinica/WG-KV``).  Integer and byte work (metadata, page
allocation, compaction) is plain numpy; floating-point work (gate MLP,
attention) is torch on the CPU in float32/float64.

Pinning (what checks each function besides its own formula):

* ``meta``      -- the reference's brute-force builder
                   (src/modeling_layers.py:274-318, restated independently in
                   ``meta.sparse_indices_bruteforce``) and the "ideal mask"
                   identity of utils/test_sparse_attn.py:78-93.
* ``decode``    -- a float64 per-token loop, closed forms (equal keys give the
                   mean of V, one token gives that V row) and page-permutation
                   invariance.
* ``prefill``   -- float64 SDPA and a per-row float64 loop under the mask.
* ``gate``      -- a float64 loop with math.erf, a closed form with W1 = 0, and
                   golden vectors written by the reference's own
                   GatingPredictor (tests/golden/).
* ``dualcache`` -- invariants (position-sorted global cache, T = local+global,
                   page accounting) and golden vectors written by the
                   reference's own prefill_wrapper / decode_wrapper /
                   migrate_local_kv_to_global (tests/golden/).
"""
