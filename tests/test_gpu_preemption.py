"""Preemption replay through the device path. A request is preempted (its pages freed in reverse group order, its
step outputs dropped, num_computed_tokens = 0, the state machine's compaction progress reset: scheduler.py:1098-1130,
processor.py:259-260) and re-prefilled from token 0 beside a request that keeps decoding: prompt chunks and response
content as causal chunks, the staged code runs again as code steps over code_physical_spans(logical_limit=) (codes
are not restaged), each closed block compacted again by the planner and its rows moved, and no block reopened while
later tokens exist (processor.py:276-316, 419-465; gpu_model_runner.py:888-930). K/V rows are a fixed function of
(request, logical position), so once the replay has caught up every kept row must sit where it sat before the
preemption and hold that token's bytes exactly; every replayed chunk and code step, and the first decode after the
catch-up, must match fp64 attention under the reference's masks (2e-2, bf16). With a retained tail (rolling or sticky
window, T=12) the code steps hide their block's tail (an excluded physical range, sched/scheduler.py:979-991) and the
previous block's tail leaves through one-row (rolling) or one-span (sticky) removals, replayed after the preemption;
the kept rows must then be the oracle trace's (oracle.trace.RequestTrace, stepped in lockstep). With a replay tail
(R=8 rows after each block's codes, appended code positions, one group at quota K: the reference's default layout)
the replay chunk runs causally after the code step, the block closes after it (so "at block close" preempts in the
replay step), the next block's content expires the replay rows one by one, and with code_exclude_replay_tail the code
step hides the replayed content rows."""
import numpy as np
import pytest
import torch

from abridgekv_amd import backend as bk
from abridgekv_amd import worker
from abridgekv_amd.config import CompressLMConfig
from abridgekv_amd.planner import KVPlanner
from abridgekv_amd.processor import REPLAY, CompressLMProcessor, SamplingSpec, ServingRequest
from oracle import masks as om
from oracle import trace as ot

pytestmark = pytest.mark.gpu
TOL = 2e-2
C, K = 64, 16
QUOTAS = (16, 4, 8)                 # one layer per KV-cache group
CODES = list(range(900, 900 + K))
TOKEN = 7                           # every sampled token (any id that is not a code)
MAX_LEN = 1024
PAGE = 16


class Engine:
    """Scheduler + worker loop over the real state machine, native planner, attention backend and mover, one
    layer per KV-cache group."""

    def __init__(self, num_pages=600, seed=0, tail=0, policy="static", replay=0, exclude=False):
        self.dev = torch.device("cuda")
        self.T, self.policy, self.R = tail, policy, replay
        self.X = tail or (replay if exclude else 0)          # rows a code step hides
        self.quotas = (K,) if replay else QUOTAS
        cfg = CompressLMConfig(replay_tail=replay, code_exclude_replay_tail=exclude, enable=True, block_size=C,
                               num_code_tokens=K, code_positions="appended" if replay else "bitrev",
                               layer_code_quotas=self.quotas, physical_layer_quotas=True, retain_tail_kv=tail,
                               retain_tail_policy=policy)
        cfg.set_code_token_ids(CODES)
        self.proc = CompressLMProcessor(cfg)
        self.proc.set_group_quotas(self.quotas)
        self.G = len(self.quotas)
        rng = np.random.default_rng(seed)
        self.planner = KVPlanner(num_pages, self.G, PAGE,
                                 free_order=rng.permutation(np.arange(1, num_pages)).astype(np.int32))
        g = torch.Generator().manual_seed(seed)
        self.caches = [torch.randn((num_pages, 2, PAGE, 8, 128), generator=g).to(torch.bfloat16).to(self.dev)
                       for _ in range(self.G)]
        # the rows of every (request, logical position): q [32, 128], k and v [8, 128] per layer (group)
        self.qtab = torch.randn((2, MAX_LEN, self.G, 32, 128), generator=g).to(torch.bfloat16)
        self.ktab = torch.randn((2, MAX_LEN, self.G, 8, 128), generator=g).to(torch.bfloat16)
        self.vtab = torch.randn((2, MAX_LEN, self.G, 8, 128), generator=g).to(torch.bfloat16)
        self.builder = bk.AbridgeMetadataBuilder(max_num_seqs=4, max_pages=MAX_LEN // PAGE, device=self.dev)
        self.impl = bk.AbridgeAttentionImpl()
        self.reqs = []
        self.traces = {}
        self.checks = 0

    def add(self, rid, prompt_len):
        req = ServingRequest(rid, list(range(1, prompt_len + 1)), SamplingSpec(bad_words_token_ids=[[c] for c in CODES]),
                             planner=self.planner)
        req.compresslm_state = self.proc.prepare_request(req)
        self.planner.add_request(rid)
        self.reqs.append(req)
        self.traces[rid] = ot.RequestTrace(prompt_len, 1 << 30, C, K, self.quotas, retain_tail=self.T,
                                           tail_policy=self.policy, replay=self.R)
        return req

    def preempt(self, req):
        """scheduler.py:1098-1130: free the pages (and the request's pending step outputs), restart at token 0 with
        no compacted spans, reset the state machine's compaction progress; the logical stream is kept."""
        self.planner.free(req.request_id)
        req.num_computed_tokens = 0
        self.proc.reset_for_preemption(req.compresslm_state)
        self.planner.add_request(req.request_id)
        self.traces[req.request_id].preempt()

    def step(self, check_rids=(), preempt_after=None):
        """One scheduler step over every request (each runs its whole next role run), the worker's appends and
        attention per group, the state machine's update (compaction through the planner); ``preempt_after`` is
        preempted before the step's outputs are taken, so its moves of this step are dropped as the worker drops
        those of preempted requests. Launches of requests in ``check_rids`` are checked against fp64."""
        sched, excluded = [], {}
        for req in self.reqs:
            start = req.num_computed_tokens
            n = self.proc.limit_num_new_tokens(req, req.num_tokens - start)
            if n <= 0:
                continue
            code = self.proc.is_code_ready(req)
            skip = self.proc.should_skip_sampling(req, n)
            assert n == self.traces[req.request_id].next_chunk()
            # a code step hides its block's retained tail: the physical range in each group's layout, taken at
            # scheduling time (sched/scheduler.py:979-991)
            excluded[req.request_id] = self.proc.code_excluded_physical_ranges(req, self.G) if code and self.X \
                else [(0, 0)] * self.G
            assert self.planner.allocate_slots(req.request_id, n) is not None, "pool exhausted"
            self.planner.set_num_computed_tokens(req.request_id, start + n)
            req.num_computed_tokens = start + n
            sched.append((req, start, n, code, skip))
        sched.sort(key=lambda e: not (e[2] == 1 and not e[3]))          # decodes first
        rids = [e[0].request_id for e in sched]
        qsl = np.concatenate([[0], np.cumsum([e[2] for e in sched])])
        positions = torch.from_numpy(np.concatenate([np.arange(s, s + n) for _, s, n, _, _ in sched])).to(self.dev)
        width = MAX_LEN // PAGE
        for g in range(self.G):
            comp = np.array([self.planner.compacted_counts(r)[g] for r in rids], np.int64)
            seq_lens = np.array([s + n for _, s, n, _, _ in sched]) - comp
            spans = [self.proc.code_physical_spans(req, g, s + n) if code else [] for req, s, n, code, _ in sched]
            limits = bk.code_step_key_limits(qsl, seq_lens, [sp[-1] if sp else None for sp in spans],
                                             self.quotas[g], K)
            excl = np.array([excluded[req.request_id][g] for req, _, _, _, _ in sched], dtype=np.int64)
            table = self.planner.fill_block_table(rids, g, width)
            md = self.builder.build(qsl, seq_lens, torch.from_numpy(table).to(self.dev), positions=positions,
                                    compacted=torch.from_numpy(comp.astype(np.int32)).to(self.dev),
                                    code_key_limit=limits, code_excluded=excl if self.X else None)
            idx = [(int(req.request_id), s, n) for req, s, n, _, _ in sched]
            q = torch.cat([self.qtab[r, s: s + n, g] for r, s, n in idx]).to(self.dev)
            k = torch.cat([self.ktab[r, s: s + n, g] for r, s, n in idx]).to(self.dev)
            v = torch.cat([self.vtab[r, s: s + n, g] for r, s, n in idx]).to(self.dev)
            out = torch.empty_like(q)
            self.impl.forward(None, q.view(-1, 32 * 128), k.view(-1, 8 * 128), v.view(-1, 8 * 128), self.caches[g],
                              md, out.view(-1, 32 * 128))
            torch.cuda.synchronize()
            for i, (req, s, n, code, _) in enumerate(sched):
                if req.request_id not in check_rids:
                    continue
                sl = int(seq_lens[i])
                ex = tuple(excl[i]) if excl[i, 1] > excl[i, 0] else None
                mask = om.request_mask(n, sl, spans[i], ex, self.quotas[g], K, causal=not code)
                ref, _ = om.masked_paged_attention_fp64(q[qsl[i]: qsl[i + 1]].float().cpu().numpy(),
                                                        self.caches[g].float().cpu().numpy(), table[i], sl, mask,
                                                        128 ** -0.5)
                got = out[qsl[i]: qsl[i + 1]].float().cpu().numpy()
                assert np.abs(got - ref).max() <= TOL, (req.request_id, g, s, n, code)
                self.checks += 1
        for req, s, n, code, skip in sched:
            _, stopped = self.proc.update_after_step(req, n, [] if skip else [TOKEN], self.planner.mask_token_span,
                                                     MAX_LEN)
            assert not stopped
            tr = self.traces[req.request_id]
            tr.num_computed_tokens += n
            tr.after_step(n)
        if preempt_after is not None:
            self.preempt(preempt_after)
        out = self.planner.take_step_outputs()
        worker.execute_fused_moves(out.fused_moves, [[c] for c in self.caches])
        return {e[0].request_id: e for e in sched}

    def layout(self, req):
        """Per group: the logical position of every physical row the request holds, and those rows' K/V bytes."""
        res = []
        for g in range(self.G):
            n = req.num_computed_tokens - self.planner.compacted_counts(req.request_id)[g]
            logical = np.array([self.planner.physical_to_logical(req.request_id, p, g) for p in range(n)])
            table = self.planner.fill_block_table([req.request_id], g, MAX_LEN // PAGE)[0]
            slots = table[np.arange(n) // PAGE].astype(np.int64) * PAGE + np.arange(n) % PAGE
            rows = self.caches[g][torch.from_numpy(slots // PAGE).to(self.dev), :,
                                  torch.from_numpy(slots % PAGE).to(self.dev)].cpu()
            res.append((logical, rows))
        return res


def _closed_blocks(req):
    return len(req.compresslm_state.compacted_block_ids)


CASES = [("mid_block", 0, "static", 0, False), ("at_block_close", 0, "static", 0, False),
         ("mid_block", 12, "rolling", 0, False), ("at_block_close", 12, "rolling", 0, False),
         ("mid_block", 12, "sticky", 0, False), ("at_block_close", 12, "sticky", 0, False),
         ("mid_block", 0, "static", 8, False), ("at_block_close", 0, "static", 8, True)]


def _case_id(w, t, p, r, x):
    return f"{w}-" + (f"replay{r}{'-excl' if x else ''}" if r else (p if t else "no_tail"))


@pytest.mark.parametrize("where,tail,policy,replay,exclude", CASES, ids=[_case_id(*c) for c in CASES])
def test_preempted_request_replays_to_the_same_layout(where, tail, policy, replay, exclude):
    print(f"case: {where} tail={tail} {policy} replay={replay} exclude={exclude}", flush=True)
    eng = Engine(seed=3 if where == "mid_block" else 4, tail=tail, policy=policy, replay=replay, exclude=exclude)
    r0 = eng.add(0, 100)                       # prompt spans block 0 and part of block 1
    r1 = eng.add(1, 30)
    # run until r0 has closed two blocks (then, mid-block: 20 more decode steps)
    while _closed_blocks(r0) < 2:
        eng.step()
    if where == "mid_block":
        for _ in range(20):
            eng.step()
    else:
        # run until r0's next code step (with a replay tail: its replay step) is the one scheduled, and preempt in
        # the step that closes its block
        while not eng.proc.is_code_ready(r0):
            eng.step()
        if replay:
            eng.step()
            assert r0.compresslm_state.roles[r0.num_computed_tokens] == REPLAY
    before_closed = _closed_blocks(r0)
    if where == "at_block_close":
        eng.step(preempt_after=r0)
        before_closed += 1                      # that block closed in the state machine, its moves dropped
    else:
        eng.step()
        eng.preempt(r0)
    target = r0.num_tokens                      # the logical stream the re-prefill replays
    assert r0.compresslm_state.compacted_block_ids == set()
    steps, replay_chunks, replay_codes = 0, 0, 0
    while r0.num_computed_tokens < target - 1:
        sched = eng.step(check_rids=(0,))
        if 0 in sched:
            _, s, n, code, _ = sched[0]
            replay_codes += int(code)
            replay_chunks += int(not code and n > 1)
        steps += 1
        assert steps < 200
    # the replay ran the closed blocks' code steps and compactions again, and reopened no block
    assert replay_codes >= before_closed and replay_chunks >= before_closed
    assert _closed_blocks(r0) == before_closed
    assert len(r0.compresslm_state.blocks) == before_closed + 1
    # every kept row sits at the logical position the planner maps it to and holds that token's bytes
    for g, (logical, rows) in enumerate(eng.layout(r0)):
        assert np.all(np.diff(logical) > 0)
        assert logical.tolist() == eng.traces[0].kept_positions(g)
        want_k = eng.ktab[0, torch.from_numpy(logical), g]
        want_v = eng.vtab[0, torch.from_numpy(logical), g]
        assert torch.equal(rows[:, 0], want_k) and torch.equal(rows[:, 1], want_v), g
        # the kept positions are the closed-form layout: prompt rows of block 0 (raw prompt) and every closed
        # block's first QUOTAS[g] codes, then the open block's content
        closed = [b for b in r0.compresslm_state.blocks if b.block_id in r0.compresslm_state.compacted_block_ids]
        kept_codes = {p for b in closed for p in range(b.code_span[0], b.code_span[0] + eng.quotas[g])}
        assert kept_codes <= set(logical.tolist())
        assert not any(p in set(logical.tolist()) for b in closed for p in range(b.code_span[0] + eng.quotas[g],
                                                                               b.code_span[1]))
    # decoding resumes over the rebuilt cache (the first decode step is checked against fp64)
    for _ in range(3):
        eng.step(check_rids=(0,))
    assert eng.checks >= 3 * replay_codes
