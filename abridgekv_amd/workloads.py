"""Synthetic serving states of the abridged cache, built through the compaction planner.

A request with prompt length P that has produced content tokens up to T-1 (the decode query is content token T-1)
went through this history, every step decided by the block state machine (abridgekv_amd.processor, the reference's
third_party/vllm_overlay/vllm/v1/core/compresslm/processor.py): one prefill step per prompt chunk (a chunk ends at a
block boundary), one decode step per response token, and after every full block of C=512 content tokens one code step
of K_max=256 rows followed by the compaction the processor issues for that block. The builder replays every
request's history through the native planner as scheduler events -- all requests interleaved step by step,
allocations of a step in request order before its compactions -- so page tables, free-queue order and compacted
counts are exactly what the reference's scheduler would produce for that arrival pattern, and the processor states
are left at the query for the serving loop to continue. Steps where no group needs a new page and nothing is
compacted are folded into the next event (allocation depends only on the token totals), which keeps 256 x 32K-token
histories cheap to replay.
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np

from .config import CompressLMConfig
from .planner import KVPlanner, SpanRemovalResult
from .processor import CODE, CompressLMProcessor, SamplingSpec, ServingRequest

BLOCK_C = 512
CODES_K_MAX = 256
PAGE = 16

# Per-layer code quotas of the per-layer arm (results/schedules/sched_trunc_perlayer_mean128.json, one quota per
# layer: every head of a layer carries the same value).
QWEN3_4B_LAYER_QUOTAS = (
    256, 64, 64, 64, 64, 64, 64, 128, 64, 128, 64, 128, 128, 128, 128, 256, 128, 128,
    256, 128, 256, 256, 128, 128, 256, 128, 128, 128, 128, 128, 64, 64, 64, 128, 128, 64,
)


def quota_groups(layer_quotas):
    """KV-cache groups of a per-layer quota model: layers bucketed by quota in first-appearance order, each bucket
    split into equal groups with layers[i::n] (third_party/vllm_overlay/vllm/v1/core/kv_cache_utils.py:1001-1052,
    1216-1226). Returns (layers per group, quota per group)."""
    buckets: dict[int, list[int]] = {}
    for layer, q in enumerate(layer_quotas):
        buckets.setdefault(int(q), []).append(layer)
    sizes = [len(v) for v in buckets.values()]
    group_size = max(sizes) if max(sizes) < min(sizes) * 1.25 else min(sizes)
    groups, quotas = [], []
    for q, layers in buckets.items():
        n = -(-len(layers) // group_size)
        for i in range(n):
            groups.append(layers[i::n])
            quotas.append(q)
    return groups, quotas


def rows_per_group(T, P, quota, C=BLOCK_C):
    """Physical rows of a group at the decode query (content token T-1, counted): prompt rows, q rows per closed
    block, the open block."""
    nb = (T - 1) // C
    return min(P, nb * C) + nb * quota + (T - nb * C)


PROMPT_TOKEN = 3                  # synthetic token ids of the replayed histories
SAMPLED_TOKEN = 11
CODE_TOKEN_BASE = 1 << 20
MAX_MODEL_LEN = 1 << 30


def serving_processor(group_quotas, C=BLOCK_C, K=CODES_K_MAX) -> CompressLMProcessor:
    """The block state machine of a served model with these per-group code quotas (synthetic code token ids)."""
    cfg = CompressLMConfig(replay_tail=0, enable=True, block_size=C, num_code_tokens=K, code_positions="bitrev")
    cfg.set_code_token_ids(range(CODE_TOKEN_BASE, CODE_TOKEN_BASE + K))
    proc = CompressLMProcessor(cfg)
    proc.set_group_quotas(group_quotas)
    return proc


def new_request(proc: CompressLMProcessor, rid, P: int) -> ServingRequest:
    """A request with a P-token synthetic prompt, prepared by the state machine (code tokens banned, no EOS)."""
    ids = proc.config.code_token_ids
    req = ServingRequest(rid, [PROMPT_TOKEN] * int(P), SamplingSpec(ignore_eos=True,
                                                                   bad_words_token_ids=[[i] for i in ids]))
    req.compresslm_state = proc.prepare_request(req)
    return req


def request_history(T, P, proc: CompressLMProcessor, rid=0, C=BLOCK_C, K=CODES_K_MAX):
    """Scheduler events of one request up to (excluding) the decode step of content token T-1, in its own step
    numbering, with the state machine deciding every step: one prefill step per prompt chunk, one decode step per
    response token, a code step of K rows after each full block, and that block's compaction -- the removals are the
    ones the processor issues through its ``mask_span`` callback, recorded here as events.

    Returns (events [(step, kind, a, b, group_mask)], number of steps, the request with its processor state at the
    query). Decode steps in which no group needs a new page are folded into the next allocation event (allocation
    depends only on token totals), and a stretch of decode steps that does not reach the block end is replayed
    through the processor at once (``update_after_decode_steps``)."""
    req = new_request(proc, rid, P)
    state = req.compresslm_state
    G = len(proc.group_quotas)
    compacted = [0] * G                  # tokens removed per group (the planner's tokens_removed of each span)
    events = []
    pending = 0                          # tokens scheduled since the last emitted allocation
    step = 0
    c = 0                                # content tokens computed
    target = T - 1

    def recorder(at):
        def mask_span(request_id, start, end, groups=None):
            for g in (range(G) if groups is None else groups):
                compacted[g] += end - start
            events.append((at, "mask", start, end, -1 if groups is None else sum(1 << g for g in groups)))
            return SpanRemovalResult(True, end - start, 0)
        return mask_span

    while True:
        start = req.num_computed_tokens
        avail = req.num_tokens - start
        if state.roles[start] == CODE:   # the code run of a full block, then its compaction
            n = proc.limit_num_new_tokens(req, avail)
            events.append((step, "alloc", pending + n, 0, 0))
            pending = 0
            req.num_computed_tokens += n
            proc.update_after_step(req, n, [], recorder(step), MAX_MODEL_LEN)
            step += 1
            continue
        if c >= target:
            break
        if avail > 1:                    # one prefill step: a prompt chunk (it ends at a block boundary)
            n = proc.limit_num_new_tokens(req, min(avail, target - c))
            skip = proc.should_skip_sampling(req, n)
            events.append((step, "alloc", pending + n, 0, 0))
            pending = 0
            req.num_computed_tokens += n
            c += n
            proc.update_after_step(req, n, [] if skip else [SAMPLED_TOKEN], recorder(step), MAX_MODEL_LEN)
            step += 1
            continue
        m = min(C - len(state.current_block.content_positions), target - c)
        if m > 0:                        # decode steps that do not compute the block's last content token
            # step i computes logical position start + i; group g needs a new page when its physical position
            # start + i - compacted_g starts one
            i = np.arange(m)
            need = np.zeros(m, bool)
            for g in range(G):
                need |= (start + i - compacted[g]) % PAGE == 0
            for off in np.flatnonzero(need).tolist():
                events.append((step + off, "alloc", pending + off + 1, 0, 0))
                pending = -(off + 1)
            pending += m
            req.num_computed_tokens += m
            c += m
            proc.update_after_decode_steps(req, [SAMPLED_TOKEN] * m, MAX_MODEL_LEN)
            step += m
        else:                            # the step computing the block's last content token stages the codes
            events.append((step, "alloc", pending + 1, 0, 0))
            pending = 0
            req.num_computed_tokens += 1
            c += 1
            proc.update_after_step(req, 1, [SAMPLED_TOKEN], recorder(step), MAX_MODEL_LEN)
            step += 1
    if pending:
        events.append((step - 1, "tail", pending, 0, 0))
    return events, step, req


def _schedule_rows(rows):
    """Order (global step, phase, request, index, event) rows as the scheduler runs them: per step, arrivals and
    allocations in request order, then the previous step's outputs are taken (they ride on this step's
    SchedulerOutput), then the step's compactions in request order."""
    rows = sorted(rows, key=lambda x: x[:4])
    out, last_step = [], None
    for step, phase, *_rest in rows:
        if phase == 1 and step != last_step:
            out.append((4, 0, 0, 0, 0, 0))
            last_step = step
        out.append(_rest[-1])
    return np.asarray(out, np.int64)


@dataclass
class DecodeState:
    """Per-group decode metadata of a batch at its next decode step (query = content token T-1 of every request)."""
    T: np.ndarray                    # [B] content tokens incl. the query
    P: np.ndarray                    # [B] prompt lengths
    groups: list                     # layers per group
    group_quotas: list               # quota per group
    layer_group: np.ndarray          # [num_layers] group of each layer
    layer_slot: np.ndarray           # [num_layers] index of the layer inside its group (= shared tensor index)
    block_tables: list               # per group [B, W] int32
    seq_lens: list                   # per group [B] int32 (rows incl. the query)
    slots: list                      # per group [B] int64: slot of the query token
    num_pages: int
    planner: KVPlanner
    processor: CompressLMProcessor   # the block state machine the histories ran through
    requests: list                   # its request objects (rid = batch index), at the decode query

    @property
    def num_layers(self):
        return len(self.layer_group)

    def rows(self, layer):
        return self.seq_lens[self.layer_group[layer]]

    def kv_bytes_per_step(self):
        """Algorithmic K+V bytes one decode step streams over all layers (4096 B per row per layer)."""
        return int(sum(int(self.rows(l).astype(np.int64).sum()) for l in range(self.num_layers)) * 4096)


def build_decode_state(T, P, layer_quotas=QWEN3_4B_LAYER_QUOTAS, seed=0, slack_pages=1024, C=BLOCK_C,
                       K=CODES_K_MAX, op_rows: bool = True) -> DecodeState:
    """Replay every request's history through a planner over a pool sized for the batch, then schedule the decode
    step (one token per request). Requests arrive staggered so that all reach their query at the same step.
    ``op_rows=False``: a planner that emits the fused moves only."""
    T = np.asarray(T, np.int64)
    P = np.minimum(np.asarray(P, np.int64), T - 1)
    B = T.size
    groups, gq = quota_groups(layer_quotas)
    G = len(groups)
    proc = serving_processor(gq, C, K)
    histories = [request_history(int(t), int(p), proc, r, C, K) for r, (t, p) in enumerate(zip(T, P))]
    S = max(h[1] for h in histories)
    pages_needed = 0
    for t, p in zip(T, P):
        for q in gq:
            # peak pages of a group: the open block's rows plus one code run before compaction
            pages_needed += -(-(rows_per_group(int(t), int(p), q, C) + K) // PAGE) + 1
    num_pages = pages_needed + slack_pages + 1
    free_order = np.random.default_rng(seed).permutation(np.arange(1, num_pages)).astype(np.int32)
    planner = KVPlanner(num_pages, G, PAGE, free_order=free_order, op_rows=op_rows)
    rows = []
    for r, (evs, n_steps, _) in enumerate(histories):
        start = S - n_steps
        rows.append((start, -1, r, -1, (0, r, 0, 0, 0, 0)))            # the request arrives
        for k, (st, kind, a, b, m) in enumerate(evs):
            if kind == "mask":
                rows.append((start + st, 1, r, k, (2, r, a, b, m, 0)))
            else:                                                       # "alloc" or the folded "tail" tokens
                rows.append((start + st, 0, r, k, (1, r, a, 0, 0, 0)))
    planner.apply_events(_schedule_rows(rows))
    # the decode step itself: one token per request
    step_ev = np.array([(1, r, 1, 0, 0, 0) for r in range(B)], np.int64)
    planner.apply_events(step_ev)
    W = 0
    seq_lens, tables, slots = [], [], []
    for g in range(G):
        sl = np.array([planner.num_computed_tokens(r) - planner.compacted_counts(r)[g] for r in range(B)], np.int32)
        seq_lens.append(sl)
    W = int(max(-(-s.max() // PAGE) for s in seq_lens))
    for g in range(G):
        tab = planner.fill_block_table(list(range(B)), g, W)
        tables.append(tab)
        pos = seq_lens[g].astype(np.int64) - 1
        slots.append(tab[np.arange(B), pos // PAGE].astype(np.int64) * PAGE + pos % PAGE)
    layer_group = np.zeros(len(layer_quotas), np.int64)
    layer_slot = np.zeros(len(layer_quotas), np.int64)
    for g, layers in enumerate(groups):
        for i, l in enumerate(layers):
            layer_group[l], layer_slot[l] = g, i
    return DecodeState(T, P, groups, gq, layer_group, layer_slot, tables, seq_lens, slots, num_pages, planner, proc,
                       [h[2] for h in histories])


def saturated_decode_lengths(B=256, seed=0, t_range=(2048, 32768), p_range=(128, 1024)):
    """Config of the saturated serving stress: total lengths T ~ U[2048, 32768] (32K cap), prompts ~ U[128, 1024]."""
    rng = np.random.default_rng(seed)
    T = rng.integers(t_range[0], t_range[1] + 1, B)
    P = np.minimum(rng.integers(p_range[0], p_range[1] + 1, B), T - 1)
    return T, P


def full_model_decode_lengths(B=64, seed=0, prompt=512, closed_generated=32):
    """Full-model decode: 512-token prompt, 32 generated closed blocks, open block of U[1, 511] tokens."""
    rng = np.random.default_rng(seed)
    L = rng.integers(1, 512, B)
    T = prompt + closed_generated * BLOCK_C + L
    return T, np.full(B, prompt)


def visible_pairs_prompt_block(C, K, N, T=0, policy="static"):
    """Visible (query, key) pairs per head of the teacher-forced mask when block 0 is the raw prompt: block-b content
    queries see their block's content causally, b*K earlier codes and (b > 0) the C prompt rows; block-b code queries
    see their block's C content and K codes, b*K earlier codes and (b > 0) the prompt rows. A retained tail of T rows
    hides a block's own last T content rows from its codes, and adds the last T content rows of earlier non-prompt
    blocks (blocks 1 ..): static, those of blocks 1 .. b-1 for every query of block b; sticky, those of block b-1 for
    its content queries; rolling, T - i of them for its i-th content query (i < T)."""
    n = 0
    for b in range(N):
        if policy == "static":
            tail_c, tail_k = C * max(0, b - 1) * T, K * max(0, b - 1) * T
        elif policy == "sticky":
            tail_c, tail_k = (C * T if b >= 2 else 0), 0
        elif policy == "rolling":
            tail_c, tail_k = (T * (T + 1) // 2 if b >= 2 else 0), 0
        else:
            raise ValueError(f"unknown tail policy {policy!r}")
        n += C * (C + 1) // 2 + C * b * K + (C * C if b else 0) + tail_c
        n += K * (C - T) + K * K + K * b * K + (K * C if b else 0) + tail_k
    return n


@dataclass
class CompactionState:
    """A batch whose requests all finished the code step of their current block and await its compaction."""
    planner: KVPlanner
    groups: list
    group_quotas: list
    num_pages: int
    pending: np.ndarray              # the compaction calls of the step, abkv_planner_apply_events rows
    prompt_lens: np.ndarray
    closed_blocks: np.ndarray
    history: np.ndarray              # the scheduler events replayed before the step (abkv_planner_apply_events rows)
    free_order: np.ndarray           # the pool's initial free-queue order

    def compact(self, as_arrays: bool = False):
        """Run the step's span removals (processor order per request: response content in every group, then code
        slots >= q per quota) and return the step outputs."""
        self.planner.apply_events(self.pending)
        return self.planner.take_step_outputs(as_arrays=as_arrays)


def build_compaction_state(B=64, seed=0, layer_quotas=QWEN3_4B_LAYER_QUOTAS, C=BLOCK_C, K=CODES_K_MAX,
                           max_prior_blocks=3, p_range=(128, 1024), slack_pages=1024,
                           op_rows: bool = True) -> CompactionState:
    """Config of the compaction benchmark: every request has closed ``nb`` earlier blocks (seeded in
    [0, max_prior_blocks]) and has just computed the K code rows of block ``nb``; prompts P ~ U[p_range] (capped so the
    closing block holds at least one response row). ``op_rows=False``: a planner that emits the fused moves only."""
    rng = np.random.default_rng(seed)
    nb = rng.integers(0, max_prior_blocks + 1, B)
    P = rng.integers(p_range[0], p_range[1] + 1, B)
    P = np.minimum(P, (nb + 1) * C - 1)
    T = (nb + 1) * C + 1
    groups, gq = quota_groups(layer_quotas)
    G = len(groups)
    proc = serving_processor(gq, C, K)
    histories = [request_history(int(t), int(p), proc, r, C, K) for r, (t, p) in enumerate(zip(T, P))]
    S = max(h[1] for h in histories)
    pages_needed = sum(-(-(int(t) + K) // PAGE) + 1 for t in T) * G
    num_pages = pages_needed + slack_pages + 1
    free_order = rng.permutation(np.arange(1, num_pages)).astype(np.int32)
    planner = KVPlanner(num_pages, G, PAGE, free_order=free_order, op_rows=op_rows)
    rows, pending = [], []
    for r, (evs, n_steps, _) in enumerate(histories):
        start = S - n_steps
        rows.append((start, -1, r, -1, (0, r, 0, 0, 0, 0)))
        for k, (st, kind, a, b, m) in enumerate(evs):
            if kind == "mask":
                if st == n_steps - 1:
                    pending.append((2, r, a, b, m, 0))
                else:
                    rows.append((start + st, 1, r, k, (2, r, a, b, m, 0)))
            else:
                rows.append((start + st, 0, r, k, (1, r, a, 0, 0, 0)))
    history = _schedule_rows(rows)
    planner.apply_events(history)
    planner.take_step_outputs()                              # earlier steps' outputs were executed long ago
    return CompactionState(planner, groups, gq, num_pages, np.asarray(pending, np.int64), P, nb, history, free_order)
