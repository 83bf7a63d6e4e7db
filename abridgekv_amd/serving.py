"""Serving stress loop over the abridged cache: decode steps with block-boundary code steps and compaction
interleaved, as the saturated serving workload runs (every request decodes one token per step; a request whose open
block fills runs its K code rows in the next step, then its block is compacted).

Host side: the block state machine (``CompressLMProcessor``, the reference's
third_party/vllm_overlay/vllm/v1/core/compresslm/processor.py) decides every request's next run
(``limit_num_new_tokens``, ``should_skip_sampling``), and after the step ``update_after_step`` settles it with
``KVPlanner.mask_token_span`` as its ``mask_span`` callback: the compaction of a block whose code run ended is exactly
the processor's ``_finish_block`` (processor.py:419-557), and the planner turns it into fused row moves.

Device side, per step: the previous step's compaction moves (``abkv_kv_move_mixed``); the slot of every new row per
KV-cache group (``abkv_slot_mapping``: logical position minus the group's compacted count through the group's page
table, gpu_model_runner.py:1579-1661 + block_table.py:186-197); then for every layer the fused RoPE + KV append
(``abkv_rope_kv_append``, bitrev RoPE positions of the abridged layout computed on the device,
config/compresslm.py:208-216), decode attention for decoding requests (``abkv_decode_attn``) and code-step attention for
coding requests (``abkv_paged_prefill_attn``, non-causal, key limit ``code_start + quota`` per group). The decoding
and the coding requests of a step are disjoint and attention reads only a request's own rows, so the two are
independent sub-batches through all layers: the code rows' appends and attention run on a second stream of the same
priority, forked once after the slot mapping and joined once at the end of the step, beside the decode layers on the
first. The host work and metadata of step s+1 are prepared while step s runs: the metadata travels in one pinned,
asynchronous host-to-device copy per step.

Queries, keys and values are synthetic (N(0,1) bf16 pools from the seed): the loop measures the attention path,
not a model.
"""
from __future__ import annotations

import ctypes as C

import numpy as np
import torch

from . import ops
from ._lib import check, lib
from .backend import code_step_key_limits
from .worker import device_move_lists, launch_moves, take_step_move_lists
from .workloads import (BLOCK_C, CODES_K_MAX, MAX_MODEL_LEN, QWEN3_4B_LAYER_QUOTAS, SAMPLED_TOKEN,
                        build_decode_state)

PAGE = ops.PAGE


def _ptr(t):
    return C.c_void_p(t.data_ptr())


class ServingPlan:
    """Host half of the loop: the state machine and request objects, the planner, the page tables and the per-step
    metadata."""

    def __init__(self, T, P, layer_quotas=QWEN3_4B_LAYER_QUOTAS, seed=0, growth_tokens=2048, C=BLOCK_C,
                 K=CODES_K_MAX, max_coding=64):
        self.C, self.K = C, K
        n_groups = len(set(layer_quotas))
        # pool slack for the run: every request's growth by growth_tokens rows per group, plus the code rows of up
        # to max_coding requests coding at once (compaction returns pages to the pool)
        slack = 1024 + len(T) * n_groups * (-(-growth_tokens // PAGE) + 2) + max_coding * n_groups * (K // PAGE + 2)
        st = build_decode_state(T, P, layer_quotas, seed=seed, slack_pages=slack, C=C, K=K, op_rows=False)
        self.st = st
        self.planner = st.planner
        self.proc = st.processor
        self.reqs = st.requests
        for req in self.reqs:                              # per-group logical -> physical maps of the planner
            req.planner = self.planner
        # the replayed histories leave their last compaction's outputs pending; the synthetic cache already stands
        # for the compacted layout, so they are dropped rather than executed
        self.planner.take_step_outputs(as_arrays=True)
        self.B, self.L, self.G = len(T), st.num_layers, len(st.groups)
        self.gq = list(st.group_quotas)
        B, G = self.B, self.G
        self.compacted = np.array([self.planner.compacted_counts(r) for r in range(B)], np.int64).T.copy()  # [G, B]
        self.pending_rows = np.zeros(0, np.int64)         # page-table / compacted rows changed since the last prepare
        self.W = int(max(-(-(sl.max() + growth_tokens + 2 * K) // PAGE) for sl in st.seq_lens)) + 2
        self.tables = np.stack([self.planner.fill_block_table(list(range(B)), g, self.W) for g in range(G)])
        self.stats = {"decode_tokens": 0, "code_steps": 0, "moved_rows": 0, "steps": 0}
        # the query step is already allocated in the planner (build_decode_state scheduled it): only the state
        # machine's side of scheduling runs for it
        self._schedule(allocate=False)
        self.start_logical = self.logical.copy()

    # -- scheduler side ---------------------------------------------------------------------------------------
    def _schedule(self, allocate=True) -> None:
        """The state machine picks every request's next run (one decode token, or the K-row code run of a full
        block); the planner allocates its slots (requests in batch order)."""
        B, K = self.B, self.K
        start = np.empty(B, np.int64)
        n_new = np.empty(B, np.int64)
        skip = np.empty(B, bool)
        code = np.empty(B, bool)
        proc = self.proc
        for r, req in enumerate(self.reqs):
            s0 = req.num_computed_tokens
            n = proc.limit_num_new_tokens(req, req.num_tokens - s0)
            code[r] = proc.is_code_ready(req)
            if n != (K if code[r] else 1):
                raise RuntimeError(f"request {r}: unexpected run of {n} tokens (code={bool(code[r])})")
            skip[r] = proc.should_skip_sampling(req, n)
            start[r], n_new[r] = s0, n
            req.num_computed_tokens = s0 + n
        if allocate:
            ev = np.zeros((B, 6), np.int64)
            ev[:, 0], ev[:, 1], ev[:, 2] = 1, np.arange(B), n_new
            self.planner.apply_events(ev)
        self.tok_start, self.n_new, self.skip, self.code = start, n_new, skip, code
        self.logical = start + n_new
        self.seq_lens = self.logical[None, :] - self.compacted            # [G, B] rows incl. the step's tokens

    def prepare(self) -> dict:
        """Metadata (numpy) of the scheduled step: tokens are the decodes (one each) then K code rows per coding
        request, each with its request and logical position (the device maps them to slots and RoPE positions);
        decode lengths; code-step starts / key limits / tiles per group; changed table rows."""
        G, K = self.G, self.K
        dec = np.flatnonzero(~self.code)
        cod = np.flatnonzero(self.code)
        nd, nc = dec.size, cod.size
        n_tok = nd + nc * K
        tok_req = np.concatenate([dec, np.repeat(cod, K)]).astype(np.int64)
        tok_pos = np.concatenate([self.tok_start[dec],
                                  (self.tok_start[cod][:, None] + np.arange(K)[None, :]).reshape(-1)])
        q_start = np.arange(nc + 1, dtype=np.int64) * K
        kv_start = np.zeros((G, nc), np.int64)
        limits = np.zeros((G, nc), np.int64)
        if nc:
            for g in range(G):
                # the staged code span of the block being closed, in the group's physical layout: the code step sees
                # every row before it and the first min(q_g, K) rows of it (gpu_model_runner.py:2042-2107)
                spans = [self.proc.code_physical_spans(self.reqs[r], g)[-1] for r in cod.tolist()]
                kv_start[g] = [s for s, _ in spans]
                limits[g] = code_step_key_limits(q_start, self.seq_lens[g][cod], spans, self.gq[g], K)
        tiles = np.array([(r, q0) for r in range(nc) for q0 in range(0, K, 64)], np.int64).reshape(-1, 2)
        dec_lens = self.seq_lens[:, dec]
        max_pages = [max(1, int(-(-dec_lens[g].max() // PAGE))) if nd else 1 for g in range(G)]
        split = [ops.auto_split_pages(dec_lens[g]) if nd else ops.DEFAULT_SPLIT_PAGES for g in range(G)]
        rows = self.pending_rows
        self.pending_rows = np.zeros(0, np.int64)
        return dict(dec=dec, cod=cod, nd=nd, nc=nc, n_tok=n_tok, dec_lens=dec_lens, q_start=q_start,
                    kv_start=kv_start, limits=limits, tiles=tiles, max_pages=max_pages, split=split, upd_rows=rows,
                    upd_tables=self.tables[:, rows], upd_compacted=self.compacted[:, rows], tok_req=tok_req,
                    tok_pos=tok_pos, max_pos=int(tok_pos.max()) if n_tok else 0)

    def advance(self, m):
        """Settle the step described by ``m`` in the state machine (compaction of the blocks whose code run ended, via
        the planner), then schedule the next step. Returns the step's fused moves (``worker.take_step_move_lists``:
        the planner's run descriptors for the device to expand, or its host-written move lists when it refuses
        descriptors for the step; valid until the next step) for the device to execute after the step's attention,
        before the next step's appends, or None."""
        B, G = self.B, self.G
        touched: set[int] = set()
        planner = self.planner

        def mask_span(request_id, start, end, groups=None):
            touched.add(request_id)
            return planner.mask_token_span(request_id, start, end, groups)

        for r, req in enumerate(self.reqs):
            _, stopped = self.proc.update_after_step(req, int(self.n_new[r]),
                                                     [] if self.skip[r] else [SAMPLED_TOKEN], mask_span,
                                                     MAX_MODEL_LEN)
            if stopped:
                raise RuntimeError(f"request {r} stopped; the stress loop keeps every request decoding")
        moves = None
        if touched:
            moves = take_step_move_lists(planner)
            self.stats["moved_rows"] += sum(n for _, _, n, _, _, _ in moves[3])
            for r in touched:
                self.compacted[:, r] = planner.compacted_counts(r)
        self.stats["decode_tokens"] += int(m["nd"])
        self.stats["code_steps"] += int(m["nc"])
        self.stats["steps"] += 1
        old_pages = -(-self.seq_lens // PAGE)
        self._schedule()
        if int(self.seq_lens.max()) > self.W * PAGE:
            raise RuntimeError("page-table width exhausted; raise growth_tokens")
        changed = set(touched)
        changed.update(np.flatnonzero((-(-self.seq_lens // PAGE) != old_pages).any(axis=0)).tolist())
        if changed:
            rows = np.asarray(sorted(changed), np.int64)
            for g in range(G):
                self.tables[g][rows] = planner.fill_block_table(rows.tolist(), g, self.W)
            self.pending_rows = np.union1d(self.pending_rows, rows)
        return moves


class ServingStress:
    """Device half: caches, synthetic q/k/v pools, and the per-step launches of a :class:`ServingPlan`."""

    def __init__(self, T, P, layer_quotas=QWEN3_4B_LAYER_QUOTAS, seed=0, device="cuda", split_pages=None,
                 growth_tokens=2048, C=BLOCK_C, K=CODES_K_MAX, tag=False, concurrent_code_step=True,
                 code_target_blocks=None):
        plan = ServingPlan(T, P, layer_quotas, seed=seed, growth_tokens=growth_tokens, C=C, K=K)
        self.plan = plan
        self.C, self.K, self.B, self.L, self.G, self.W = C, K, plan.B, plan.L, plan.G, plan.W
        self.st = plan.st
        self.dev = torch.device(device)
        self.split_pages = split_pages
        # Pages per decode split when split_pages is None: the plan's ops.auto_split_pages, capped at 40 while code
        # steps run beside the decode. The B=256 stress (T ~ U[2048, 32768]) over 300 steps, interleaved runs on two
        # boxes, tokens/s: 40 pages 7466 / 7490 / 7440 / 7513 against 7415 / 7401 / 7414 / 7390 for the automatic
        # choice (48 at B=256); 36 pages 7282 / 7286, 44 pages 7002 / 7002, 56 pages 7305 / 7301. Alone on the GPU
        # (the saturated decode steps) 48 pages stay faster: 7599 / 7612 against 7531 / 7488 at 40.
        self.split_cap = 40 if concurrent_code_step else None
        # Workgroups a code step's key splits aim at. None: a quarter of the CUs when the code step runs beside the
        # decode (2 key splits for one request: fewer, longer workgroups leave more of the GPU to the memory-bound
        # decode; the B=256 stress over 300 steps, two boxes, interleaved runs: 7369 -> 7429 and 7381 -> 7401 tokens/s
        # against one workgroup per CU), all of them when it runs alone after the decode (serial order).
        if code_target_blocks is None:
            code_target_blocks = max(ops._num_cus() // 4, 1) if concurrent_code_step else ops._num_cus()
        self.code_target_blocks = int(code_target_blocks)
        self.tag = tag
        B = self.B
        n_tensors = max(len(g) for g in self.st.groups)
        gen = torch.Generator(device=self.dev).manual_seed(seed)
        self.caches = []
        for _ in range(n_tensors):
            c = torch.empty(ops.kv_cache_shape(self.st.num_pages), dtype=torch.bfloat16, device=self.dev)
            c.normal_(generator=gen)
            self.caches.append(c)
        self.by_group = [[self.caches[i] for i in range(len(layers))] for layers in self.st.groups]
        self.q_pool = torch.randn((B * K, 32, 128), generator=gen, device=self.dev).to(torch.bfloat16)
        self.k_pool = torch.randn((B * K, 8, 128), generator=gen, device=self.dev).to(torch.bfloat16)
        self.v_pool = torch.randn((B * K, 8, 128), generator=gen, device=self.dev).to(torch.bfloat16)
        self.out = torch.empty((B * K, 32, 128), dtype=torch.bfloat16, device=self.dev)
        self.slots = torch.empty((self.G, B * K), dtype=torch.int64, device=self.dev)
        self.bt_dev = torch.from_numpy(plan.tables).to(self.dev)                       # [G, B, W]
        self.comp_dev = torch.from_numpy(plan.compacted.astype(np.int32)).to(self.dev)  # [G, B]
        # RoPE table for every position the run can reach: in growth_tokens steps a request decodes at most
        # growth_tokens tokens and runs at most growth_tokens // C + 2 code runs of K rows
        max_logical = int(plan.logical.max()) + growth_tokens + (growth_tokens // C + 2) * K
        self.cos_sin = ops.rope_cos_sin_cache(ops.rope_bound(max_logical, C, K) + 1, device=self.dev)
        # split_pages None: per step and group the plan's ops.auto_split_pages (never below 32, so this workspace fits)
        self.ws = ops.decode_workspace(B, self.W, min(split_pages or ops.DEFAULT_SPLIT_PAGES, ops.DEFAULT_SPLIT_PAGES),
                                       device=self.dev)
        self.ws_bytes = 0 if self.ws is None else self.ws.numel()
        # pinned staging ring for the per-step metadata
        self._pinned = [torch.empty(1 << 22, dtype=torch.int32, pin_memory=True) for _ in range(2)]
        self._staged = [torch.empty(1 << 22, dtype=torch.int32, device=self.dev) for _ in range(2)]
        self._copy_done = [None, None]
        self._ring = 0
        self.scale = ops.default_scale()
        self.decode_events = None          # a list: (start, end) events around every decode launch are appended
        # the code rows of a step on a side stream (default priority, as every stream here): one fork and one join
        # event, created once and re-recorded every step
        self._code_stream = torch.cuda.Stream(device=self.dev) if concurrent_code_step else None
        self._fork = [torch.cuda.Event()] if concurrent_code_step else None
        self._join = [torch.cuda.Event()] if concurrent_code_step else None
        self._code_ws = torch.empty(0, dtype=torch.uint8, device=self.dev)
        # move lists of the staged compaction: written by abkv_moves_expand after the step's upload and read by the
        # next launch's moves, both on the one stream, so one buffer serves every step
        self._moves_out = torch.empty(1 << 20, dtype=torch.int32, device=self.dev)
        self._meta = self._stage(plan.prepare())

    @property
    def stats(self):
        return self.plan.stats

    @property
    def seq_lens(self):
        return self.plan.seq_lens

    @property
    def tables(self):
        return self.plan.tables

    def _stage(self, m, moves=None):
        """Pack the step metadata (and the previous step's compaction moves) into one pinned buffer and start its
        asynchronous copy to the device."""
        G, W = self.G, self.W
        nd, nc, n_tok = m["nd"], m["nc"], m["n_tok"]
        rows = m["upd_rows"]
        if ops.rope_bound(m["max_pos"], self.C, self.K) >= self.cos_sin.shape[0]:
            raise RuntimeError("RoPE table exhausted; raise growth_tokens")
        parts = {
            "upd_rows": rows.astype(np.int32),
            "upd_tables": m["upd_tables"].astype(np.int32).reshape(-1),
            "upd_comp": m["upd_compacted"].astype(np.int32).reshape(-1),
            "tok_req": m["tok_req"].astype(np.int32),
            "tok_pos": m["tok_pos"].astype(np.int64).view(np.int32),
            "dec_lens": m["dec_lens"].astype(np.int32).reshape(-1),
            "dec_idx": m["dec"].astype(np.int32),
            "cod_idx": m["cod"].astype(np.int32),
            "q_start": m["q_start"].astype(np.int32),
            "kv_start": m["kv_start"].astype(np.int32).reshape(-1),
            "limits": m["limits"].astype(np.int32).reshape(-1),
            "tile_req": m["tiles"][:, 0].astype(np.int32).copy(),
            "tile_q0": m["tiles"][:, 1].astype(np.int32).copy(),
        }
        mv_kind, mv_desc, mv_layout, mv_parts, mv_elems = moves if moves else (None, None, None, [], 0)
        if mv_parts:
            # run descriptors (records, page windows, group table; 16-byte aligned sections), or the move lists
            parts["move_runs" if mv_kind == "runs" else "move_lists"] = mv_desc
        if self.tag:                                       # (request, logical position) of every new row
            tp = m["tok_pos"]
            parts["tags"] = np.stack([m["tok_req"], tp // 256, tp % 256], axis=1).astype(np.int32).reshape(-1)
        i = self._ring
        if self._copy_done[i] is not None:
            self._copy_done[i].synchronize()                 # the copy that last read this pinned buffer is done
        buf = self._pinned[i].numpy()
        off, where = 0, {}
        for name, arr in parts.items():
            off = (off + 3) & ~3                             # 16-byte aligned sections
            if off + arr.size > buf.size:
                raise RuntimeError("per-step metadata exceeds the staging buffer")
            buf[off: off + arr.size] = arr
            where[name] = (off, arr.size)
            off += arr.size
        dev = self._staged[i]
        dev[:off].copy_(self._pinned[i][:off], non_blocking=True)
        ev = torch.cuda.Event()
        ev.record()
        self._copy_done[i] = ev
        self._ring ^= 1
        v = {name: dev[o: o + n] for name, (o, n) in where.items()}
        v["tok_pos"] = v["tok_pos"].view(torch.int64)
        v["dec_lens"] = v["dec_lens"].view(G, nd)
        v["kv_start"] = v["kv_start"].view(G, nc)
        v["limits"] = v["limits"].view(G, nc)
        v["upd_tables"] = v["upd_tables"].view(G, rows.size, W)
        v["upd_comp"] = v["upd_comp"].view(G, rows.size)
        if self.tag:
            v["tags"] = v["tags"].view(n_tok, 3)
        mv = []
        if mv_parts and mv_kind == "packed":
            mv = device_move_lists(v["move_lists"], mv_parts)
        elif mv_parts:                                     # the move lists, written on the device from the descriptors
            if mv_elems > self._moves_out.numel():
                self._moves_out = torch.empty(2 * mv_elems, dtype=torch.int32, device=self.dev)
            base = v["move_runs"].data_ptr()
            runs_at, n_runs, pages_at, groups_at = mv_layout
            check(lib().abkv_moves_expand(C.c_void_p(base + 4 * runs_at), n_runs, C.c_void_p(base + 4 * pages_at),
                                          groups_at - pages_at, C.c_void_p(base + 4 * groups_at), G,
                                          PAGE.bit_length() - 1,
                                          C.c_void_p(self._moves_out.data_ptr()), mv_elems,
                                          C.c_void_p(torch.cuda.current_stream().cuda_stream)), "abkv_moves_expand")
            mv = device_move_lists(self._moves_out[:mv_elems], mv_parts)
        # key splits of the code step per group (its few query tiles cannot fill the GPU on their own)
        n_tiles = int(m["tiles"].shape[0])
        code_split = [ops.paged_split_plan(n_tiles, int(m["limits"][g].max()), self.code_target_blocks) if nc
                      else (1, 0) for g in range(G)]
        need = max((lib().abkv_paged_prefill_workspace_size(nc * self.K, n) for n, _ in code_split if n > 1),
                   default=0)
        if need > self._code_ws.numel():
            self._code_ws = torch.empty(need, dtype=torch.uint8, device=self.dev)
        return dict(m, view=v, n_tiles=n_tiles, n_upd=int(rows.size), moves=mv, code_split=code_split)

    # -- device: one step ---------------------------------------------------------------------------------------
    def _split(self, m, g):
        """Pages per decode split of group g in the step whose metadata is m."""
        if self.split_pages:
            return self.split_pages
        sp = m["split"][g]
        return sp if self.split_cap is None else min(sp, self.split_cap)

    def _layer_out(self, layer):
        """Output rows of a layer's attention (one buffer shared by every layer: the loop measures attention, and the
        next layer's queries come from the synthetic pool, not from this output)."""
        return self.out

    def _launch_step(self, m):
        v, nd, nc, n_tok = m["view"], m["nd"], m["nc"], m["n_tok"]
        main = torch.cuda.current_stream()
        stream = C.c_void_p(main.cuda_stream)
        side = self._code_stream if nc and nd else None
        L = lib()
        q, k, val = self.q_pool, self.k_pool, self.v_pool
        if m["moves"]:
            launch_moves(m["moves"], self.by_group)
        if m["n_upd"]:
            rows = v["upd_rows"].long()
            self.bt_dev[:, rows] = v["upd_tables"]
            self.comp_dev[:, rows] = v["upd_comp"]
        if self.tag:
            val[:n_tok, 0, :3] = v["tags"].to(torch.bfloat16)
        # slots of the step's new rows per group: logical position - the group's compacted count -> page table
        for g in range(self.G):
            check(L.abkv_slot_mapping(_ptr(v["tok_req"]), _ptr(v["tok_pos"]), n_tok, _ptr(self.bt_dev[g]), self.B,
                                      self.W, PAGE, _ptr(self.comp_dev[g]), _ptr(self.slots[g]), stream),
                  "abkv_slot_mapping")
        dec_bt = [self.bt_dev[g].index_select(0, v["dec_idx"].long()) if nd else None for g in range(self.G)]
        m["cod_bt"] = [self.bt_dev[g].index_select(0, v["cod_idx"].long()) if nc else None for g in range(self.G)]
        code_stream = C.c_void_p(side.cuda_stream) if side is not None else stream
        if side is not None:
            # The decoding and the coding requests of a step are disjoint, and attention reads only a request's own
            # rows: the two are independent sub-batches through every layer. The code rows' appends and attention of
            # all layers run on the side stream, forked once here and joined once at the end of the step; layer by
            # layer, the decode launches are issued first.
            self._fork[0].record(main)
            side.wait_event(self._fork[0])
        for layer in range(self.L):
            g = int(self.st.layer_group[layer])
            cache = self.caches[int(self.st.layer_slot[layer])]
            out = self._layer_out(layer)
            # RoPE of q and k at the bitrev positions of the abridged layout + KV append, one launch (the decode rows
            # only when the code rows run on the side stream)
            self._append(layer, g, cache, 0, nd if side is not None else n_tok, v, stream)
            if nd:
                if self.decode_events is not None:
                    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                    e0.record()
                check(L.abkv_decode_attn(_ptr(q), q.stride(0), q.stride(1), _ptr(cache), cache.shape[0],
                                         _ptr(dec_bt[g]), self.W, _ptr(v["dec_lens"][g]), nd, m["max_pages"][g],
                                         self._split(m, g), C.c_float(self.scale), _ptr(out),
                                         out.stride(0),
                                         out.stride(1), None, None if self.ws is None else _ptr(self.ws),
                                         C.c_size_t(self.ws_bytes), stream), "abkv_decode_attn")
                if self.decode_events is not None:
                    e1.record()
                    self.decode_events.append((e0, e1))
            if nc:
                if side is not None:
                    self._append(layer, g, cache, nd, n_tok, v, code_stream)
                self._code_step(m, g, cache, out, code_stream)
        if side is not None:
            self._join[0].record(side)
            main.wait_event(self._join[0])               # the next step's moves and appends follow the code rows

    def _append(self, layer, g, cache, t0, t1, v, stream):
        """RoPE of the q and k rows [t0, t1) of the step at the bitrev positions of the abridged layout, and their K/V
        rows appended at their slots of group g."""
        if t1 <= t0:
            return
        q, k, val, cs = self.q_pool, self.k_pool, self.v_pool, self.cos_sin
        check(lib().abkv_rope_kv_append(C.c_void_p(q.data_ptr() + t0 * q.stride(0) * 2), q.stride(0), q.stride(1),
                                        C.c_void_p(k.data_ptr() + t0 * k.stride(0) * 2), k.stride(0),
                                        C.c_void_p(val.data_ptr() + t0 * val.stride(0) * 2), val.stride(0),
                                        C.c_void_p(v["tok_pos"].data_ptr() + 8 * t0), t1 - t0, self.C, self.K, 0,
                                        _ptr(cs), cs.shape[0], C.c_void_p(self.slots[g].data_ptr() + 8 * t0),
                                        _ptr(cache), cache.shape[0], stream), "abkv_rope_kv_append")

    def _code_step(self, m, g, cache, out, stream):
        """Code-step attention of the step's coding requests over one layer of group g (non-causal, per-request key
        limit code_start + quota)."""
        v, nd, nc = m["view"], m["nd"], m["nc"]
        qc, oc = self.q_pool[nd:], out[nd:]
        n_sp, sp_tiles = m["code_split"][g]
        check(lib().abkv_paged_prefill_attn(_ptr(qc), qc.stride(0), qc.stride(1), _ptr(cache), cache.shape[0],
                                            _ptr(m["cod_bt"][g]), self.W, self.W, _ptr(v["q_start"]),
                                            _ptr(v["kv_start"][g]), _ptr(v["limits"][g]), None, _ptr(v["tile_req"]),
                                            _ptr(v["tile_q0"]), m["n_tiles"], None, 0, C.c_float(self.scale),
                                            _ptr(oc), oc.stride(0), oc.stride(1), None, nc * self.K, n_sp,
                                            sp_tiles, _ptr(self._code_ws) if n_sp > 1 else None,
                                            C.c_size_t(self._code_ws.numel() if n_sp > 1 else 0), stream),
              "abkv_paged_prefill_attn")

    def flush(self) -> None:
        """Execute the compaction moves staged for the next step now (e.g. before reading the cache)."""
        if self._meta["moves"]:
            launch_moves(self._meta["moves"], self.by_group)
            self._meta["moves"] = []

    def check_layout(self, requests=None):
        """With ``tag=True``: read every group's physical rows written during the run back from the cache and check
        that row p of request r holds logical position planner.physical_to_logical(r, p, g) (the tag is in the V
        row, which RoPE leaves alone; rows of tokens scheduled for the next step are not written yet and are
        skipped). Returns rows checked."""
        if not self.tag:
            raise RuntimeError("construct with tag=True")
        self.flush()
        torch.cuda.synchronize()
        checked = 0
        plan = self.plan
        for g in range(self.G):
            cache = self.by_group[g][0]
            for r in (range(self.B) if requests is None else requests):
                n = int(self.seq_lens[g, r])
                pos = np.arange(n)
                logical = np.array([plan.planner.physical_to_logical(r, int(p), g) for p in pos])
                # rows written during the run; the tokens already scheduled for the next step are not written yet
                keep = (logical >= plan.start_logical[r] - 1) & (logical < plan.tok_start[r])
                if not keep.any():
                    continue
                pp = pos[keep]
                pages = torch.from_numpy(self.tables[g][r, pp // PAGE].astype(np.int64)).to(self.dev)
                offs = torch.from_numpy(pp % PAGE).to(self.dev)
                tags = cache[pages, 1, offs, 0, :3].float().cpu().numpy().astype(np.int64)
                if not (np.all(tags[:, 0] == r) and np.array_equal(tags[:, 1] * 256 + tags[:, 2], logical[keep])):
                    raise AssertionError(f"request {r} group {g}: rows do not hold their logical positions")
                checked += int(keep.sum())
        return checked

    def decode_bytes(self, m) -> int:
        """Algorithmic bytes of the step's decode launches: K+V rows (4096 B per row per layer) plus q and out."""
        per_group = m["dec_lens"].astype(np.int64).sum(axis=1) * 4096 + m["nd"] * 16384
        return int(sum(per_group[int(self.st.layer_group[l])] for l in range(self.L)))

    def step(self):
        """Launch the staged step; settle it in the plan; stage the next step (with this step's compaction moves,
        which run first in the next launch: after this step's attention, before the next step's appends)."""
        m = self._meta
        self._launch_step(m)
        moves = self.plan.advance(m)                       # staged (copied) before the planner's next step
        self._meta = self._stage(self.plan.prepare(), moves)
        return m

    def run(self, steps):
        for _ in range(steps):
            self.step()
