"""Serving stress loop over the abridged cache: decode steps with block-boundary code steps and compaction
interleaved, as the saturated serving workload runs (every request decodes one token per step; a request whose open
block fills runs its K code rows in the next step, then its block is compacted).

Per step, on one HIP stream: for every layer the new K/V rows are appended (``abkv_kv_append``), decoding requests
attend with ``abkv_decode_attn`` over their group page table and coding requests with ``abkv_paged_prefill_attn``
(non-causal, key limit ``code_start + quota`` per group); then the planner's removals of the finished blocks
(``_finish_block`` order: response content in every group, code rows >= q in groups of quota q < K;
third_party/vllm_overlay/vllm/v1/core/compresslm/processor.py:467-557) become fused row moves
(``abkv_kv_move_segments``). The host planner work and metadata of step s+1 are prepared while step s runs: the
metadata travels in one pinned, asynchronous host-to-device copy per step.

Queries, keys and values are synthetic (N(0,1) bf16 pools from the seed): the loop measures the attention path,
not a model.
"""
from __future__ import annotations

import ctypes as C

import numpy as np
import torch

from . import ops
from ._lib import check, lib
from .worker import launch_moves, split_fused_moves
from .workloads import BLOCK_C, CODES_K_MAX, QWEN3_4B_LAYER_QUOTAS, build_decode_state

PAGE = ops.PAGE


def _ptr(t):
    return C.c_void_p(t.data_ptr())


class ServingPlan:
    """Host half of the loop: the planner, every request's state, the page tables and the per-step metadata."""

    def __init__(self, T, P, layer_quotas=QWEN3_4B_LAYER_QUOTAS, seed=0, growth_tokens=2048, C=BLOCK_C,
                 K=CODES_K_MAX, max_coding=64):
        self.C, self.K = C, K
        n_groups = len(set(layer_quotas))
        # pool slack for the run: every request's growth by growth_tokens rows per group, plus the code rows of up
        # to max_coding requests coding at once (compaction returns pages to the pool)
        slack = 1024 + len(T) * n_groups * (-(-growth_tokens // PAGE) + 2) + max_coding * n_groups * (K // PAGE + 2)
        st = build_decode_state(T, P, layer_quotas, seed=seed, slack_pages=slack, C=C, K=K)
        self.st = st
        self.planner = st.planner
        # the replayed histories leave their last compaction's outputs pending; the synthetic cache already stands
        # for the compacted layout, so they are dropped rather than executed
        self.planner.take_step_outputs(as_arrays=True)
        self.B, self.L, self.G = len(T), st.num_layers, len(st.groups)
        self.gq = list(st.group_quotas)
        B, G = self.B, self.G
        # request state: content tokens incl. the step's query, logical length, phase (0 decode, 1 code)
        self.T = np.asarray(st.T, np.int64).copy()
        self.P = np.asarray(st.P, np.int64).copy()
        self.logical = np.array([self.planner.num_computed_tokens(r) for r in range(B)], np.int64)
        self.phase = np.zeros(B, np.int64)
        self.code_block = np.zeros(B, np.int64)          # block being coded (phase 1)
        self.start_logical = self.logical.copy()
        self.pending_rows = np.zeros(0, np.int64)         # page-table rows changed since the last prepare
        self.seq_lens = np.stack([sl.astype(np.int64) for sl in st.seq_lens])         # [G, B] rows incl. the step
        self.W = int(max(-(-(sl.max() + growth_tokens + 2 * K) // PAGE) for sl in self.seq_lens)) + 2
        self.tables = np.stack([self.planner.fill_block_table(list(range(B)), g, self.W) for g in range(G)])
        self.stats = {"decode_tokens": 0, "code_steps": 0, "moved_rows": 0, "steps": 0}

    def prepare(self) -> dict:
        """Metadata (numpy) of the step about to run: tokens are the decodes (one each) then K code rows per coding
        request; per-group slots, decode lengths, code-step starts / key limits / tiles, changed table rows."""
        G, K = self.G, self.K
        dec = np.flatnonzero(self.phase == 0)
        cod = np.flatnonzero(self.phase == 1)
        nd, nc = dec.size, cod.size
        n_tok = nd + nc * K
        slots = np.empty((G, n_tok), np.int64)
        for g in range(G):
            sl, tab = self.seq_lens[g], self.tables[g]
            pos_d = sl[dec] - 1
            slots[g, :nd] = tab[dec, pos_d // PAGE].astype(np.int64) * PAGE + pos_d % PAGE
            if nc:
                pos_c = ((sl[cod] - K)[:, None] + np.arange(K)[None, :]).reshape(-1)
                req_c = np.repeat(cod, K)
                slots[g, nd:] = tab[req_c, pos_c // PAGE].astype(np.int64) * PAGE + pos_c % PAGE
        kv_start = (np.stack([self.seq_lens[g][cod] - K for g in range(G)]) if nc
                    else np.zeros((G, 0), np.int64))
        limits = kv_start + np.minimum(np.asarray(self.gq)[:, None], K)
        tiles = np.array([(r, q0) for r in range(nc) for q0 in range(0, K, 64)], np.int64).reshape(-1, 2)
        dec_lens = self.seq_lens[:, dec]
        max_pages = [max(1, int(-(-dec_lens[g].max() // PAGE))) if nd else 1 for g in range(G)]
        split = [ops.auto_split_pages(dec_lens[g]) if nd else ops.DEFAULT_SPLIT_PAGES for g in range(G)]
        rows = self.pending_rows
        self.pending_rows = np.zeros(0, np.int64)
        tok_req = np.concatenate([dec, np.repeat(cod, K)]).astype(np.int64)
        tok_pos = np.concatenate([self.logical[dec] - 1,
                                  ((self.logical[cod] - K)[:, None] + np.arange(K)[None, :]).reshape(-1)])
        return dict(dec=dec, cod=cod, nd=nd, nc=nc, n_tok=n_tok, slots=slots, dec_lens=dec_lens,
                    q_start=np.arange(nc + 1, dtype=np.int64) * K, kv_start=kv_start, limits=limits, tiles=tiles,
                    max_pages=max_pages, split=split, upd_rows=rows, upd_tables=self.tables[:, rows], tok_req=tok_req,
                    tok_pos=tok_pos)

    def advance(self, m) -> np.ndarray:
        """Account for the step described by ``m``: compact the blocks whose code step ran (the planner's removals),
        move decoders on, schedule the next step's tokens. Returns the fused move rows to execute on the device
        (after the step's attention, before the next step's appends)."""
        B, G, K, Cb = self.B, self.G, self.K, self.C
        dec, cod = m["dec"], m["cod"]
        events = []
        for r in cod.tolist():
            code_start = int(self.logical[r]) - K
            block_start = code_start - Cb
            b = int(self.code_block[r])
            resp_from = block_start + min(max(int(self.P[r]) - b * Cb, 0), Cb)
            if resp_from < code_start:
                events.append((2, r, resp_from, code_start, -1, 0))
                self.seq_lens[:, r] -= code_start - resp_from
            for qv in sorted({q for q in self.gq if q < K}):
                mask = sum(1 << g for g, gq in enumerate(self.gq) if gq == qv)
                events.append((2, r, code_start + qv, code_start + K, mask, 0))
                for g, gq in enumerate(self.gq):
                    if gq == qv:
                        self.seq_lens[g, r] -= K - qv
        changed = set(cod.tolist())
        fused = np.zeros((0, 6), np.int64)
        if events:
            self.planner.apply_events(np.asarray(events, np.int64))
            _, _, fu = self.planner.take_step_outputs(as_arrays=True)
            fused = fu.copy()
            self.stats["moved_rows"] += int(fused.shape[0])
        self.stats["decode_tokens"] += int(dec.size)
        self.stats["code_steps"] += int(cod.size)
        self.stats["steps"] += 1
        finished = dec[(self.T[dec] % Cb) == 0]          # the decoded token closed its block: code it next step
        self.code_block[finished] = (self.T[finished] - 1) // Cb
        self.T[dec] += 1
        self.phase[:] = 0
        self.phase[finished] = 1
        n_new = np.where(self.phase == 1, K, 1)
        ev = np.zeros((B, 6), np.int64)
        ev[:, 0], ev[:, 1], ev[:, 2] = 1, np.arange(B), n_new
        old_pages = -(-self.seq_lens // PAGE)
        self.planner.apply_events(ev)
        self.logical += n_new
        self.seq_lens += n_new[None, :]
        if int(self.seq_lens.max()) > self.W * PAGE:
            raise RuntimeError("page-table width exhausted; raise growth_tokens")
        grew = np.flatnonzero((-(-self.seq_lens // PAGE) != old_pages).any(axis=0))
        changed.update(grew.tolist())
        if changed:
            rows = np.asarray(sorted(changed), np.int64)
            for g in range(G):
                self.tables[g][rows] = self.planner.fill_block_table(rows.tolist(), g, self.W)
            self.pending_rows = np.union1d(self.pending_rows, rows)
        return fused


class ServingStress:
    """Device half: caches, synthetic q/k/v pools, and the per-step launches of a :class:`ServingPlan`."""

    def __init__(self, T, P, layer_quotas=QWEN3_4B_LAYER_QUOTAS, seed=0, device="cuda", split_pages=None,
                 growth_tokens=2048, C=BLOCK_C, K=CODES_K_MAX, tag=False):
        plan = ServingPlan(T, P, layer_quotas, seed=seed, growth_tokens=growth_tokens, C=C, K=K)
        self.plan = plan
        self.C, self.K, self.B, self.L, self.G, self.W = C, K, plan.B, plan.L, plan.G, plan.W
        self.st = plan.st
        self.dev = torch.device(device)
        self.split_pages = split_pages
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
        self.bt_dev = torch.from_numpy(plan.tables).to(self.dev)                       # [G, B, W]
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
        self._code_ws = torch.empty(0, dtype=torch.uint8, device=self.dev)
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

    def _stage(self, m, moves=()):
        """Pack the step metadata (and the previous step's compaction moves) into one pinned buffer and start its
        asynchronous copy to the device."""
        G, W = self.G, self.W
        nd, nc, n_tok = m["nd"], m["nc"], m["n_tok"]
        rows = m["upd_rows"]
        parts = {
            "upd_rows": rows.astype(np.int32),
            "upd_tables": m["upd_tables"].astype(np.int32).reshape(-1),
            "slots": m["slots"].view(np.int32).reshape(-1),
            "dec_lens": m["dec_lens"].astype(np.int32).reshape(-1),
            "dec_idx": m["dec"].astype(np.int32),
            "cod_idx": m["cod"].astype(np.int32),
            "q_start": m["q_start"].astype(np.int32),
            "kv_start": m["kv_start"].astype(np.int32).reshape(-1),
            "limits": m["limits"].astype(np.int32).reshape(-1),
            "tile_req": m["tiles"][:, 0].astype(np.int32).copy(),
            "tile_q0": m["tiles"][:, 1].astype(np.int32).copy(),
        }
        for j, (gid, ops_h, offs) in enumerate(moves):
            parts[f"mv_ops{j}"] = ops_h.reshape(-1)
            parts[f"mv_offs{j}"] = offs
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
        v["slots"] = v["slots"].view(torch.int64).view(G, n_tok)
        v["dec_lens"] = v["dec_lens"].view(G, nd)
        v["kv_start"] = v["kv_start"].view(G, nc)
        v["limits"] = v["limits"].view(G, nc)
        v["upd_tables"] = v["upd_tables"].view(G, rows.size, W)
        if self.tag:
            v["tags"] = v["tags"].view(n_tok, 3)
        mv = [(gid, v[f"mv_ops{j}"].view(-1, 4), v[f"mv_offs{j}"]) for j, (gid, _, _) in enumerate(moves)]
        # key splits of the code step per group (its few query tiles cannot fill the GPU on their own)
        n_tiles = int(m["tiles"].shape[0])
        code_split = [ops.paged_split_plan(n_tiles, int(m["limits"][g].max())) if nc else (1, 0) for g in range(G)]
        need = max((lib().abkv_paged_prefill_workspace_size(nc * self.K, n) for n, _ in code_split if n > 1),
                   default=0)
        if need > self._code_ws.numel():
            self._code_ws = torch.empty(need, dtype=torch.uint8, device=self.dev)
        return dict(m, view=v, n_tiles=n_tiles, n_upd=int(rows.size), moves=mv, code_split=code_split)

    # -- device: one step ---------------------------------------------------------------------------------------
    def _launch_step(self, m):
        v, nd, nc, n_tok = m["view"], m["nd"], m["nc"], m["n_tok"]
        stream = C.c_void_p(torch.cuda.current_stream().cuda_stream)
        L = lib()
        q, k, val, out = self.q_pool, self.k_pool, self.v_pool, self.out
        if m["moves"]:
            launch_moves(m["moves"], self.by_group)
        if m["n_upd"]:
            self.bt_dev[:, v["upd_rows"].long()] = v["upd_tables"]
        if self.tag:
            k[:n_tok, 0, :3] = v["tags"].to(torch.bfloat16)
        dec_bt = [self.bt_dev[g].index_select(0, v["dec_idx"].long()) if nd else None for g in range(self.G)]
        cod_bt = [self.bt_dev[g].index_select(0, v["cod_idx"].long()) if nc else None for g in range(self.G)]
        for layer in range(self.L):
            g = int(self.st.layer_group[layer])
            cache = self.caches[int(self.st.layer_slot[layer])]
            check(L.abkv_kv_append(_ptr(k), k.stride(0) * 2, _ptr(val), val.stride(0) * 2, _ptr(v["slots"][g]), n_tok,
                                   _ptr(cache), cache.shape[0], ops.PAGE_BYTES, ops.HALF_BYTES, ops.SLOT_BYTES, PAGE,
                                   stream), "abkv_kv_append")
            if nd:
                if self.decode_events is not None:
                    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                    e0.record()
                check(L.abkv_decode_attn(_ptr(q), q.stride(0), q.stride(1), _ptr(cache), cache.shape[0],
                                         _ptr(dec_bt[g]), self.W, _ptr(v["dec_lens"][g]), nd, m["max_pages"][g],
                                         self.split_pages or m["split"][g], C.c_float(self.scale), _ptr(out),
                                         out.stride(0),
                                         out.stride(1), None, None if self.ws is None else _ptr(self.ws),
                                         C.c_size_t(self.ws_bytes), stream), "abkv_decode_attn")
                if self.decode_events is not None:
                    e1.record()
                    self.decode_events.append((e0, e1))
            if nc:
                qc, oc = q[nd:], out[nd:]
                n_sp, sp_tiles = m["code_split"][g]
                check(L.abkv_paged_prefill_attn(_ptr(qc), qc.stride(0), qc.stride(1), _ptr(cache), cache.shape[0],
                                                _ptr(cod_bt[g]), self.W, self.W, _ptr(v["q_start"]),
                                                _ptr(v["kv_start"][g]), _ptr(v["limits"][g]), _ptr(v["tile_req"]),
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
        that row p of request r holds logical position planner.physical_to_logical(r, p, g) (rows of tokens
        scheduled for the next step are not written yet and are skipped). Returns rows checked."""
        if not self.tag:
            raise RuntimeError("construct with tag=True")
        self.flush()
        torch.cuda.synchronize()
        checked = 0
        for g in range(self.G):
            cache = self.by_group[g][0]
            for r in (range(self.B) if requests is None else requests):
                n = int(self.seq_lens[g, r])
                pos = np.arange(n)
                logical = np.array([self.plan.planner.physical_to_logical(r, int(p), g) for p in pos])
                # rows written during the run; the tokens already scheduled for the next step are not written yet
                pending = self.K if self.plan.phase[r] == 1 else 1
                keep = (logical >= self.plan.start_logical[r] - 1) & (logical < self.plan.logical[r] - pending)
                if not keep.any():
                    continue
                pp = pos[keep]
                pages = torch.from_numpy(self.tables[g][r, pp // PAGE].astype(np.int64)).to(self.dev)
                offs = torch.from_numpy(pp % PAGE).to(self.dev)
                tags = cache[pages, 0, offs, 0, :3].float().cpu().numpy().astype(np.int64)
                if not (np.all(tags[:, 0] == r) and np.array_equal(tags[:, 1] * 256 + tags[:, 2], logical[keep])):
                    raise AssertionError(f"request {r} group {g}: rows do not hold their logical positions")
                checked += int(keep.sum())
        return checked

    def decode_bytes(self, m) -> int:
        """Algorithmic bytes of the step's decode launches: K+V rows (4096 B per row per layer) plus q and out."""
        per_group = m["dec_lens"].astype(np.int64).sum(axis=1) * 4096 + m["nd"] * 16384
        return int(sum(per_group[int(self.st.layer_group[l])] for l in range(self.L)))

    def step(self):
        """Launch the staged step; advance the plan; stage the next step (with this step's compaction moves, which
        run first in the next launch: after this step's attention, before the next step's appends)."""
        m = self._meta
        self._launch_step(m)
        moves = split_fused_moves(self.plan.advance(m), self.st.num_pages, check=False)
        self._meta = self._stage(self.plan.prepare(), moves)
        return m

    def run(self, steps):
        for _ in range(steps):
            self.step()
