"""Incremental CompressLM generator over the paged abridged cache (the serving path for one sequence).

Mirrors the public surface of abridgekv/gen_compress.py:85-1052 (``CompressGen``: ``feed_content``, ``compress``,
``step``, ``prefill``, ``generate``, ``cache_kv_stats``) for the served configuration (L=1, raw prompt, per-layer code
quotas, an optional retained or replay tail, no raw tail) with bidirectional, causal or no code<->code attention in a
code step (``pause_xattn``; only bidirectional with per-head packed pages). The reference keeps a
dense per-layer store and masks it; here every layer's rows live in paged caches, quotas are physical, and the block
boundary is a compaction:

* content chunks rotate q/k and append K/V at the group's next physical slots in one launch
  (``abkv_rope_kv_append``: the kernel maps the rows' logical positions to RoPE positions, and the slots come from
  ``abkv_slot_mapping`` -- logical position minus the group's compacted count through its page table -- both on the
  device) and attend over every resident row: one token -> ``abkv_decode_attn``, several -> causal
  ``abkv_paged_prefill_attn``. Resident rows are exactly the reference's visible set (codes of earlier blocks, raw
  prompt, the current block's content; gen_compress.py:667-707).
* ``compress`` runs the K code rows of the block non-causally with the key limit ``code_start + q_layer`` (the
  code visibility of gen_compress.py:328-358, 709-745), then compacts the block with the removals the block state
  machine prescribes (``CompressLMProcessor.block_removal_spans``: response content in every group, then code rows
  ``>= q`` in groups of quota ``q < K``; processor.py:467-557) through the native planner (``mask_token_span``) and
  moves the surviving rows with the HIP mover. The generator's API hands over the next token only after
  ``compress()``, so it runs the processor's block compaction directly rather than through ``update_after_step``
  (which needs that token to open the next block).
* a retained tail of T rows (``retain_tail_kv``): the block's last T content rows survive its compaction; the code
  step hides them from the block's own codes (an excluded key range) and the bitrev code positions spread over the
  first C - T offsets. ``retain_tail_policy="static"`` keeps them for every later row. The window policies keep a
  block's response tail rows for the next block's content only, as the serving state machine does
  (compresslm/processor.py:318-353, 559-646): "sticky" removes them all before that block's code step; "rolling"
  removes tail row i once content token i of the next block has run, and a content chunk ends at every such token
  so that each removal follows that token's query (processor.py:123-151). Raw-prompt rows never leave.
* a raw tail of W rows (``raw_tail``, or ``raw_tail_override``; gen_compress.py:118-137, 445-470, 980-1000): the
  rolling window over the block's last W content rows (W <= C), which the block's own codes see like the rest of
  their block.

Layers with equal quota form one KV-cache group (one page table); tensor i holds the i-th layer of every group, as
the serving worker shares them (kv_cache_utils.py:1110-1127).

A replay tail of R rows (appended code positions): after its code step a block runs its last R tokens again as a
causal chunk (they see the prompt, the codes the quotas leave -- the code part of the block's removals runs first --
and the block's content, which leaves after them); content token i of the next block expires replay row i, a chunk
ending at each such token (gen_compress.py:900-916, processor.py:336-345, 594-618).

Code-step inputs follow the model's seed pools (``seg_pool``, ``gated_seg_pool``, ``pool_init`` or
``code_init_override="segment_mean"``: gen_compress.py:867-898). A model trained with code-row projections
(``query_residual``, ``code_q_heads``, ``code_kv_heads``) runs its code rows through them here too, as its
teacher-forced forward does; the reference's generator leaves them to the layer's own weights
(compress_forward.py:203-207 notes the step "would need the same swap"), which would not reproduce that forward.

Per-head quotas (a layer whose KV heads keep different numbers of codes) use the per-head packed pages of the
serving sidecar (compresslm_packed_kv.py): one KV-cache group; the code step hides paged code rows ``>= q_h`` per KV
head (``abkv_paged_prefill_attn_packed``); ``compress`` then copies the block's code rows into one packed page per
layer (``abkv_packed_capture``) and removes the response content and all K codes as one span; content steps attend
over the packed pages plus the paged rows (``abkv_decode_attn_packed`` / ``abkv_paged_prefill_attn_packed``).
"""
from __future__ import annotations

import numpy as np
import torch
import torch.nn.functional as F

from . import backend as bk
from . import ops
from .compress_forward import _QProjCode, _QProjQRes, code_seeds
from .config import CompressLMConfig, bitrev_offsets
from .packed_kv import PackedKVLayout, PackedKVSidecar
from .planner import KVPlanner
from .processor import CompressLMBlock, CompressLMProcessor
from .worker import execute_fused_moves

_UNSUPPORTED = ("capture_hidden", "capture_attention",
                "oracle_full_history", "oracle_history_layers", "preserve_full_history", "retain_full_history_layers",
                "history_replaces_codes_layers", "capture_content_attention", "content_attention_offsets",
                "content_head_callback", "evict_policy", "keep_per_block", "evict_seed", "skip_unused_codes")


def _layer_quotas(head_code_quotas, num_layers, num_kv_heads, K):
    if head_code_quotas is None:
        return [K] * num_layers
    q = torch.as_tensor(head_code_quotas, dtype=torch.long).cpu()
    if tuple(q.shape) != (num_layers, num_kv_heads):
        raise ValueError(f"head_code_quotas must have shape [{num_layers}, {num_kv_heads}], got {tuple(q.shape)}")
    if bool(((q <= 0) | (q > K)).any()):
        raise ValueError(f"head_code_quotas must be in [1, {K}]")
    return [int(x) for x in q[:, 0]]


def _per_head(head_code_quotas) -> bool:
    """Whether some layer's KV heads have different quotas (served through per-head packed pages)."""
    if head_code_quotas is None:
        return False
    q = torch.as_tensor(head_code_quotas, dtype=torch.long)
    return bool((q != q[:, :1]).any())


def _project(proj, x, code_step):
    """A layer projection of the generator's rows x [1, n, d]. Code steps (n = K code rows, slots 0..K-1) take the
    code rows' own weights (code_q_heads / code_kv_heads) or the query residual of their slot (query_residual), as
    the teacher-forced forward does at its code rows (compress_forward.py:181-222); content rows and plain
    projections run the layer's own weights."""
    if isinstance(proj, _QProjCode):
        return (proj.code if code_step else proj.orig)(x)
    if isinstance(proj, _QProjQRes):
        out = proj.orig(x)
        return out + proj.qres[: x.size(1)].to(out.dtype) if code_step else out
    return proj(x)


class CompressGen:
    """One sequence's incremental generator. ``clm`` is a :class:`abridgekv_amd.compress_forward.CompressLM` (or any
    object with ``model``, ``C``, ``K``, ``pause``, ``code_positions``); ``max_tokens`` bounds the logical length the
    page pool must hold."""

    def __init__(self, clm, device, raw_prompt_len=0, head_code_quotas=None, code_attend_current_content=True,
                 code_init_override=None, raw_tail_override=None, max_tokens: int = 1 << 15, **options):
        bad = sorted(name for name in options if name not in _UNSUPPORTED)
        if bad:
            raise TypeError(f"unexpected CompressGen options {bad}")
        used = sorted(name for name, value in options.items() if value)
        if used:
            raise NotImplementedError(f"CompressGen options {used} are not supported on the paged path")
        if not code_attend_current_content:
            raise NotImplementedError("code rows always attend the current block's content on the paged path")
        if getattr(clm, "L", 1) != 1:
            raise NotImplementedError("the paged path serves one pause pass (L=1)")
        if code_init_override not in (None, "segment_mean"):
            raise ValueError(f"unsupported code_init_override={code_init_override!r}")
        # code seeds of a code step: the generic seeds or the block's segment means / learned pool (gen_compress.py:
        # 867-898; "segment_mean" forces the segment means, :194-200)
        self.code_init_override = code_init_override
        # code <-> code attention of a code step (gen_compress.py:953-959): bidirectional, causal, or none
        self.xattn = getattr(clm, "pause_xattn", "full")
        if self.xattn not in ("full", "causal", "none"):
            raise ValueError(f"pause_xattn must be 'none', 'causal' or 'full', got {self.xattn!r}")
        # raw tail (gen_compress.py:118-137): the next block's i-th content row sees the block's last W - i content
        # rows (a rolling window that its own codes also see); raw_tail_override replaces the model's W
        retain = int(getattr(clm, "retain_tail_kv", 0) or 0)
        if raw_tail_override is not None and retain:
            raise ValueError("raw_tail_override cannot be combined with retain_tail_kv")
        self.raw = int(getattr(clm, "raw_tail", 0) or 0) if raw_tail_override is None else int(raw_tail_override)
        if not 0 <= self.raw <= int(clm.C):
            raise ValueError(f"raw_tail must be in [0, C={clm.C}], got {self.raw}")
        if self.raw and getattr(clm, "replay_tail", 0):
            raise NotImplementedError("the paged path takes a raw tail or a replay tail, not both")
        self.T = self.raw or retain
        self.policy = "rolling" if self.raw else getattr(clm, "retain_tail_policy", "rolling") if self.T else "static"
        # replay tail (gen_compress.py:900-916): R rows after each block's codes, fed its last R content tokens; the
        # next block's content token i expires replay row i (processor.py:336-345, 594-618)
        self.R = int(getattr(clm, "replay_tail", 0) or 0)
        if self.R and self.code_positions_of(clm) == "bitrev":
            raise ValueError("a replay tail needs appended code positions")
        # the block's last content rows its own codes do not see: the retained tail, or the replayed rows with
        # code_exclude_replay_tail (compress_forward.py:298-300)
        self.X = self.R if getattr(clm, "code_exclude_replay_tail", False) else retain
        self.clm = clm
        self.inner = clm.model.model
        self.layers = self.inner.layers
        self.num_layers = len(self.layers)
        self.lm_head = clm.model.lm_head
        self.device = torch.device(device)
        self.dtype = next(clm.model.parameters()).dtype
        if self.dtype != torch.bfloat16:
            raise NotImplementedError("the paged kernels run bf16 models")
        self.C, self.K = int(clm.C), int(clm.K)
        self.code_positions = getattr(clm, "code_positions", "appended")
        self.raw_prompt_len = int(raw_prompt_len)
        self.d = clm.model.config.hidden_size
        cfg = clm.model.config
        self.quotas = _layer_quotas(head_code_quotas, self.num_layers, int(cfg.num_key_value_heads), self.K)
        self.head_code_quotas = None if head_code_quotas is None else torch.as_tensor(head_code_quotas)
        # Per-head quotas (rows not uniform): closed blocks' code rows move to per-head packed pages and leave the
        # paged cache with the summarised content (one KV-cache group, every layer its own tensor); per-layer quotas:
        # one group per distinct quota, code rows >= quota removed from the group's layout.
        self.packed = _per_head(head_code_quotas)
        if self.packed:
            self.quotas = [self.K] * self.num_layers
        if self.packed and self.policy != "static":
            raise NotImplementedError("per-head packed pages take the static retained tail only "
                                      "(config/compresslm.py:160-167)")
        if self.packed and self.xattn != "full":
            raise NotImplementedError("per-head packed pages serve bidirectional code steps (pause_xattn='full')")

        # KV-cache groups: layers of equal quota, in order of first appearance; tensor i = i-th layer of each group
        distinct = list(dict.fromkeys(self.quotas))
        self.group_quotas = distinct
        self.group_of = [distinct.index(q) for q in self.quotas]
        self.tensor_of = [self.group_of[:li].count(self.group_of[li]) for li in range(self.num_layers)]
        n_tensors = max(self.tensor_of) + 1
        G = len(distinct)
        pages_per_group = -(-int(max_tokens) // ops.PAGE) + 2
        self.num_pages = G * pages_per_group + 1
        self.caches = [torch.zeros(ops.kv_cache_shape(self.num_pages), dtype=torch.bfloat16, device=self.device)
                       for _ in range(n_tensors)]
        self.caches_by_group = [[self.caches[self.tensor_of[li]] for li in range(self.num_layers)
                                 if self.group_of[li] == g] for g in range(G)]
        self.planner = KVPlanner(self.num_pages, G, ops.PAGE)
        self.rid = 0
        self.planner.add_request(self.rid)
        # the block state machine's compaction rule for these groups (the serving validation of an enabled config --
        # bitrev positions, power-of-two sizes -- is the vLLM path's; the generator also runs appended positions)
        # (a raw tail is kept out of the block's response content by the generator itself, so it may span the block)
        pcfg = CompressLMConfig(replay_tail=0, code_positions="bitrev",
                                block_size=self.C, num_code_tokens=self.K, packed_kv=self.packed,
                                packed_kv_k_max=self.K, retain_tail_kv=retain,
                                retain_tail_policy=self.policy if retain else "rolling")
        pcfg.set_code_token_ids(range(1 << 20, (1 << 20) + self.K))
        self.proc = CompressLMProcessor(pcfg)
        if not self.packed:
            self.proc.set_group_quotas(self.group_quotas)
        self.impl = bk.AbridgeAttentionImpl(scale=getattr(self.layers[0].self_attn, "scaling", None))
        self.builder = bk.AbridgeMetadataBuilder(max_num_seqs=1, max_pages=pages_per_group, device=self.device)
        self.sidecar = None
        if self.packed:
            layout = PackedKVLayout.from_schedule(self.head_code_quotas.tolist(), num_layers=self.num_layers,
                                                  num_kv_heads=int(cfg.num_key_value_heads), k_max=self.K)
            blocks = int(max_tokens) // self.C + 2
            self.sidecar = PackedKVSidecar(layout, self.caches_by_group[0], pool_pages=blocks,
                                           max_pages_per_request=min(blocks, 2048), device=self.device)
        self.b = 0                      # current block index
        self.f = 0                      # content tokens committed in the current block
        # window tails: the previous block's tail rows still resident, by tail index (None: raw prompt or gone)
        self._window: list[int | None] = []
        self.logical_len = 0            # tokens in the planner's logical sequence (content + code rows)
        self._cur_ids: list[int] = []
        self._code_offsets = (torch.from_numpy(bitrev_offsets(self.K, self.C - self.X)).to(self.device)
                              if self.code_positions == "bitrev" else None)
        # fp32 cos/sin of the model's rotary embedding for every position this sequence can reach (RoPE positions
        # never exceed logical positions); the fused kernel rotates q/k and appends K/V in one launch per layer
        self._cos_sin = ops.rotary_cos_sin_from_model(self.inner.rotary_emb, int(max_tokens) + 1, self.device)

    # -- positions ------------------------------------------------------------------------------------------------
    def _content_pos(self, n):
        """RoPE positions of the next n content tokens of block b (gen_compress.py:789-795)."""
        base = self.b * self.C if self.code_positions == "bitrev" else self.b * (self.C + self.K + self.R)
        return torch.arange(base + self.f, base + self.f + n, device=self.device)

    def _code_pos(self):
        """RoPE positions of the K code rows of block b (gen_compress.py:797-804)."""
        if self.code_positions == "bitrev":
            return self.b * self.C + self._code_offsets
        base = self.b * (self.C + self.K + self.R)
        return torch.arange(base + self.C, base + self.C + self.K, device=self.device)

    # -- one step over all layers ---------------------------------------------------------------------------------
    def _group_metadata(self, n, code_step, logical):
        """Per-group metadata for n new rows appended after each group's resident rows; the slots of the new rows are
        computed on the device from their logical positions and the group's compacted count."""
        blocks = self.planner.get_blocks(self.rid)
        comp = self.planner.compacted_counts(self.rid)
        comp_dev = torch.tensor(comp, dtype=torch.int32).to(self.device)
        out = []
        for g, q in enumerate(self.group_quotas):
            start = self.logical_len - comp[g]
            seq_len = start + n
            table = torch.from_numpy(np.asarray(blocks[g], dtype=np.int32)).view(1, -1).to(self.device)
            # the block's own code rows a code row sees: the first q (bidirectional or causal) or none
            own = min(q, self.K) if self.xattn != "none" else 0
            limit = [start + own] if code_step else None
            # the block's own retained tail: its last T content rows, just before the code rows in every group
            excluded = [[start - self.X, start]] if code_step and self.X else None
            causal = [self.xattn == "causal"] if code_step else None
            out.append(self.builder.build([0, n], [seq_len], table, code_key_limit=limit, positions=logical,
                                          compacted=comp_dev[g:g + 1], code_excluded=excluded, code_causal=causal))
        return out

    @torch.no_grad()
    def _forward_rows(self, hidden, code_step):
        """Run every decoder layer over hidden [1, n, d]; new K/V rows are committed to the caches. The rows take the
        next n logical positions; the fused kernel maps them to RoPE positions on the device (bitrev layout:
        block * C + in-block offset, config/compresslm.py:208-216; appended layout: the logical position itself)."""
        n = hidden.shape[1]
        if self.planner.allocate_slots(self.rid, n) is None:
            raise RuntimeError("page pool exhausted; raise max_tokens")
        logical = torch.arange(self.logical_len, self.logical_len + n, dtype=torch.int64, device=self.device)
        mds = self._group_metadata(n, code_step, logical)
        bc, bk = (self.C, self.K) if self.code_positions == "bitrev" else (0, 0)
        last = self.logical_len + n - 1
        for li, layer in enumerate(self.layers):
            attn = layer.self_attn
            md = mds[self.group_of[li]]
            cache = self.caches[self.tensor_of[li]]
            normed = layer.input_layernorm(hidden)
            q = _project(attn.q_proj, normed, code_step).view(1, n, -1, attn.head_dim)
            k = _project(attn.k_proj, normed, code_step).view(1, n, -1, attn.head_dim)
            if getattr(attn, "q_norm", None) is not None:
                q = attn.q_norm(q)
            if getattr(attn, "k_norm", None) is not None:
                k = attn.k_norm(k)
            q = q[0].to(self.dtype).contiguous()
            k = k[0].to(self.dtype).contiguous()
            v = _project(attn.v_proj, normed, code_step).view(n, -1, attn.head_dim).contiguous()
            ops.rope_kv_append(q, k, v, logical, self._cos_sin, slot_mapping=md.slot_mapping, kv_cache=cache,
                               block_c=bc, codes_k=bk, max_position=last, code_span=bc - self.X if bc else 0)
            o = torch.empty((n, ops.HEADS_Q, ops.HEAD_DIM), dtype=self.dtype, device=self.device)
            if self.sidecar is not None:
                # paged rows + this layer's per-head packed pages; a code step's paged keys stop at the block's
                # first q_h code rows for KV head h
                ex = None if md.code_excluded is None else [tuple(md.code_excluded[0])]
                self.sidecar.attend(li, q, cache, md.block_table, md.query_start_loc, md.seq_lens, not code_step, o,
                                    request_ids=(self.rid,), seq_lens_dev=md.seq_lens_dev, scale=self.impl.scale,
                                    excluded=ex)
            else:
                self.impl.attend(q, cache, md, o)
            h = hidden + attn.o_proj(o.view(1, n, -1))
            hidden = h + layer.mlp(layer.post_attention_layernorm(h))
        self.logical_len += n
        self.planner.set_num_computed_tokens(self.rid, self.logical_len)
        return hidden

    @staticmethod
    def code_positions_of(clm):
        return getattr(clm, "code_positions", "appended")

    def _code_seeds(self):
        """Inputs [K, d] of the block's code rows (the content embeddings feed the seed pools)."""
        tok_e = self.inner.embed_tokens(torch.tensor([self._cur_ids], device=self.device))
        return code_seeds(self.clm, tok_e, self.code_init_override == "segment_mean")[0].to(self.dtype)

    # -- reference surface ----------------------------------------------------------------------------------------
    def _remove(self, spans):
        """Run span removals (logical [start, end) in every group, or (start, end, groups)) through the planner and
        move the rows."""
        for span in spans:
            start, end, groups = span if len(span) == 3 else (*span, None)
            CompressLMProcessor._mask_or_raise(self.planner.mask_token_span, self.rid, start, end, groups)
        _, _, fused = self.planner.take_step_outputs(as_arrays=True)
        execute_fused_moves(fused.copy(), self.caches_by_group)

    def feed_content(self, ids):
        """Feed <= C - f content tokens as one chunk (split where a rolling tail row expires); returns the final-normed
        hidden states (n, d)."""
        n = len(ids)
        if n == 0 or self.f + n > self.C:
            raise ValueError(f"chunk of {n} tokens does not fit the block ({self.f}/{self.C} used)")
        outs, i = [], 0
        while i < n:
            take = n - i
            if self.policy == "rolling" or self.R:
                # the chunk ends at the first content token whose tail row of the previous block expires
                for j in range(self.f, min(self.f + take, len(self._window))):
                    if self._window[j] is not None:
                        take = j - self.f + 1
                        break
            part = ids[i:i + take]
            hidden = self.inner.embed_tokens(torch.tensor([list(part)], device=self.device))
            outs.append(self._forward_rows(hidden, code_step=False))
            if (self.policy == "rolling" or self.R) and self.f + take - 1 < len(self._window) and \
                    self._window[self.f + take - 1] is not None:
                row, self._window[self.f + take - 1] = self._window[self.f + take - 1], None
                self._remove([(row, row + 1)])
            self.f += take
            self._cur_ids += [int(t) for t in part]
            i += take
        return self.inner.norm(torch.cat(outs, dim=1))[0]

    def compress(self):
        """Code step of the full block, then compaction of its response content and of code rows >= quota."""
        if self.f != self.C:
            raise RuntimeError("compress() needs a full block")
        K, C = self.K, self.C
        if self.policy == "sticky":
            # the previous block's response tail leaves after this block's last content row, before its codes
            rows = [r for r in self._window if r is not None]
            self._window = []
            if rows:
                self._remove([(rows[0], rows[-1] + 1)])
        hidden = self._code_seeds().view(1, K, self.d)
        code_start = self.logical_len
        self._forward_rows(hidden, code_step=True)
        block_start = code_start - C
        resp_from = block_start + min(max(self.raw_prompt_len - self.b * C, 0), C)
        # the block as the state machine sees it; its removals (and their order) are the processor's
        tail = list(range(code_start - self.T, code_start)) if self.T else []
        response = list(range(resp_from, code_start - self.T if self.raw else code_start))
        block = CompressLMBlock(self.b, content_positions=list(range(block_start, code_start)),
                                prompt_content_positions=list(range(block_start, resp_from)),
                                response_content_positions=response, code_span=(code_start, code_start + K),
                                retained_tail_positions=[] if self.raw else tail)
        spans = self.proc.block_removal_spans(block)
        if self.sidecar is not None:
            # archive the code rows into packed pages before the span that removes them runs
            # (compresslm/processor.py:484-520)
            phys = code_start - self.planner.compacted_counts(self.rid)[0]
            table = self.planner.get_blocks(self.rid)[0]
            self.sidecar.capture(self.rid, physical_start=phys, physical_end=phys + K, block_ids=table)
        if self.R:
            # The replay rows (the block's last R tokens again, after its codes) run while the block's content is
            # resident but must see only the code rows the quotas leave: the code part of the removals goes first
            # (code slots >= q per group; with packed pages every paged code row, the sidecar now holding them),
            # then the replay chunk, then the content part. The kept rows are those of the processor's order.
            code_part = [(max(a, code_start), e, g) for a, e, g in spans if e > code_start]
            content_part = [(a, min(e, code_start), g) for a, e, g in spans if a < code_start]
            self._remove(code_part)
            replay_ids = self._cur_ids[-self.R:]
            self._forward_rows(self.inner.embed_tokens(torch.tensor([replay_ids], device=self.device)),
                               code_step=False)
            spans = content_part
        for start, end, groups in spans:
            CompressLMProcessor._mask_or_raise(self.planner.mask_token_span, self.rid, start, end, groups)
        _, _, fused = self.planner.take_step_outputs(as_arrays=True)
        execute_fused_moves(fused.copy(), self.caches_by_group)
        if self.policy != "static":
            # this block's tail rows, by tail index, that the next block's content may still expire (response rows)
            self._window = [p if p >= resp_from else None for p in range(code_start - self.T, code_start)]
        if self.R:
            # every replay row expires, prompt blocks' too (processor.py:336-345)
            self._window = list(range(code_start + K, code_start + K + self.R))
        self.b += 1
        self.f = 0
        self._cur_ids = []

    def step(self, token_id):
        """Feed one content token (compressing when it completes the block); returns its next-token logits."""
        h = self.feed_content([int(token_id)])
        logits = self.lm_head(h[-1:]).float()[0]
        if self.f == self.C:
            self.compress()
        return logits

    def prefill(self, prompt_ids):
        """Feed the prompt in block-aligned chunks (compressing full blocks); returns the last token's logits."""
        ids = list(prompt_ids)
        last, i = None, 0
        while i < len(ids):
            take = min(self.C - self.f, len(ids) - i)
            h = self.feed_content(ids[i:i + take])
            last = self.lm_head(h[-1:]).float()[0]
            i += take
            if self.f == self.C:
                self.compress()
        return last

    @torch.no_grad()
    def generate(self, prompt_ids, max_new_tokens, eos_id=None, temperature=0.0, top_p=1.0, top_k=0, gen=None):
        logits = self.prefill(prompt_ids)
        out = []
        for _ in range(max_new_tokens):
            nxt = sample(logits, temperature, top_p, top_k, gen)
            out.append(nxt)
            if eos_id is not None and nxt == eos_id:
                break
            logits = self.step(nxt)
        return out

    def resident_rows(self) -> list[int]:
        """Paged rows held per layer (its group's length)."""
        comp = self.planner.compacted_counts(self.rid)
        return [self.logical_len - comp[g] for g in self.group_of]

    def packed_rows(self) -> list[int]:
        """Rows held per layer in per-head packed pages (summed over the KV heads, so a row here is one head's
        K/V; zero without per-head quotas)."""
        if self.sidecar is None:
            return [0] * self.num_layers
        n = len(self.sidecar.request_pages(self.rid))
        return [n * r for r in self.sidecar.layout.packed_slots_per_layer]

    def cache_kv_stats(self):
        main = self.resident_rows()
        total = sum(main)
        elements = total * 2 * ops.HEADS_KV * ops.HEAD_DIM + sum(self.packed_rows()) * 2 * ops.HEAD_DIM
        return {"main_columns_by_layer": main, "history_columns_by_layer": [0] * self.num_layers,
                "packed_head_rows_by_layer": self.packed_rows(), "total_columns": total,
                "total_kv_elements": elements}


def sample(logits, temperature, top_p, top_k, gen):
    """Greedy for temperature <= 0, else temperature / top-k / top-p sampling (gen_compress.py:1035-1052)."""
    if temperature is None or temperature <= 0:
        return int(logits.argmax())
    logits = logits / temperature
    if top_k and top_k > 0:
        kth = torch.topk(logits, min(top_k, logits.numel())).values[-1]
        logits = logits.masked_fill(logits < kth, float("-inf"))
    probs = F.softmax(logits, dim=-1)
    if top_p and top_p < 1.0:
        sp, si = torch.sort(probs, descending=True)
        cut = torch.cumsum(sp, dim=-1) > top_p
        cut[..., 1:] = cut[..., :-1].clone()
        cut[..., 0] = False
        probs = torch.zeros_like(probs).scatter_(-1, si, sp.masked_fill(cut, 0.0))
        probs = probs / probs.sum()
    return int(torch.multinomial(probs, 1, generator=gen))
