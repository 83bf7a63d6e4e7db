"""CPU oracle for the abridged-KV hot path.

TEST INFRASTRUCTURE ONLY. Nothing in ``abridgekv_amd`` imports this package; only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` use it, and only as the checker
(or as the timed CPU baseline), never as the product path.

Modules (each function cites the reference file:line it restates):

* ``layout``     -- bitrev code offsets, bitrev RoPE positions, NeoX RoPE, quota grouping, per-layer row counts.
* ``decode``     -- fp64 closed-form decode attention (+ natural-log LSE) over a paged cache, and the reference's
                    own torch arithmetic (bf16 scores, fp32 softmax, bf16 probabilities) used as the CPU baseline.
* ``compaction`` -- line-by-line restatement of the serving-side compaction planner: free-block queue, block pool,
                    per-group page lists, compacted-span index, ``mask_token_span``, copy-op execution with
                    gather-then-scatter semantics, block-table truncation and slot mapping.
* ``prefill``    -- the teacher-forced compression mask in its two reference forms (role/block dense mask and the
                    closed-form arithmetic mask) and an fp64 masked attention.
* ``trace``      -- the block state machine that decides which spans are compacted when (processor semantics),
                    producing planner-agnostic event traces.

Pinning status of every function is listed in each module's header.
"""
