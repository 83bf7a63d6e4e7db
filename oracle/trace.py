"""Block state machine of one request: which tokens are scheduled when and which spans are compacted
(oracle; test infrastructure only).

Restates, for the served configuration of the per-layer arm (C=512 content tokens per block, K_max code rows,
raw prompt, bitrev positions, no replay/retained tails, physical per-layer quotas), the role bookkeeping of
third_party/vllm_overlay/vllm/v1/core/compresslm/processor.py:
  prepare_request :42-105 (first prompt chunk), limit_num_new_tokens :123-151 (a CODE run is scheduled whole,
  a CONTENT run up to its end), should_skip_sampling :153-168, update_after_step :170-257 (a full block stages
  its K codes and holds the sampled token), _stage_codes :369-400, _finish_block :419-465 (compact, then open the
  next block with the next prompt chunk or the held token), _compact_response_content :467-557 (response content
  in every group, then code slots [q, K) per distinct quota q < K in ascending order). With a retained tail
  (``retain_tail`` = T, compresslm.py:22-26) the block's last T content rows are not removed with the block
  (:480-482): the response content before them goes. Their fate is the tail policy's:
    "static"  -- they stay for the rest of the request;
    "rolling" -- the i-th content token of the next block expires the tail's i-th row once it has run (a one-row
                 removal of a response row; :320-353 maps it, :123-151 ends a chunk at every such token so each
                 expiry has a query of its own, :614-646 removes it);
    "sticky"  -- the tail's response rows go as one span after the next block's last content token has run,
                 before that block's codes (:559-592, called from :215-224 and again, as a no-op, from :427-430).
  With a replay tail (``replay`` = R, appended positions) a block's code run is followed by R replay tokens (its last
  R content tokens again, role REPLAY, :236-240, :402-417); the block is compacted after them (:253-259), and the
  next block's i-th content token expires replay row i once it has run (a one-row removal of any replay row, prompt
  blocks' too; :336-345 maps it, :123-151 ends a chunk at each, :594-618 removes it, before any tail expiry).
  Preemption (``preempt``) restarts the request at token 0 with its logical stream and block structure kept and
  its compaction progress cleared (state.py:46-50); the replay compacts every closed block again and opens no block
  that already exists (:429-431).

The machine is planner-agnostic: it emits the scheduler-visible events (allocate ``n`` new tokens, then compact
spans) and is shared by the oracle planner and the product planner so that both see identical event streams.

Pinning: tests/test_oracle_compaction.py checks the reference's invariants (scripts/test_compresslm_physical_quotas.py:
68-138): every compacted block keeps exactly codes[:q_g] and no response content in group g; removed rows per
group differ from group 0 by (K - q_g) per compacted block; and the closed form of oracle.layout.rows_per_layer.
The static tail: tests/test_static_tail.py checks the kept rows against their closed form (prompt content, the last T
content rows and q codes per closed block) and the reference's own static-tail scenarios through the product machine,
which must issue this trace's calls.
"""
from __future__ import annotations

from dataclasses import dataclass, field

CONTENT, CODE, REPLAY = 0, 1, 2


@dataclass
class Block:
    block_id: int
    content_positions: list = field(default_factory=list)
    prompt_positions: list = field(default_factory=list)
    response_positions: list = field(default_factory=list)
    code_span: tuple | None = None
    replay_positions: list = field(default_factory=list)


class RequestTrace:
    """Logical token stream of one request and its block structure."""

    def __init__(self, prompt_len, max_tokens, C, K, group_quotas, retain_tail=0, tail_policy="static", replay=0):
        if prompt_len <= 0:
            raise ValueError("CompressLM decoding requires a non-empty prompt")
        if tail_policy not in ("static", "rolling", "sticky"):
            raise ValueError(f"unknown tail policy {tail_policy!r}")
        self.C, self.K = C, K
        self.T = retain_tail
        self.R = replay
        if replay and retain_tail:
            raise ValueError("replay and retained tails are mutually exclusive")
        self.policy = tail_policy
        self.replay_expire_at: dict[int, int] = {}   # content position -> previous block's replay row it expires
        self.replay_expired: set[int] = set()
        self.expire_at: dict[int, int] = {}     # rolling: content position -> previous block's tail row it expires
        self.expired: set[int] = set()          # rolling tail rows removed so far
        self.sticky_done: set[int] = set()      # blocks whose tail the sticky policy has removed
        self.group_quotas = tuple(group_quotas)
        self.prompt_len = prompt_len
        self.max_tokens = max_tokens
        self.roles: list[int] = []
        self.kind: list[str] = []               # "prompt" | "response" | "code" per logical position
        self.blocks = [Block(0)]
        self.compacted_block_ids: set[int] = set()
        self.num_computed_tokens = 0
        self.pending_prompt = 0
        self.held = False
        self.visible = 0
        self.finished = False
        first = min(prompt_len, C)                # processor.py:90-104
        self.pending_prompt = first
        self._record_content(first, is_prompt=True)

    @property
    def num_tokens(self):
        return len(self.roles)

    @property
    def current_block(self):
        return self.blocks[-1]

    def _tail_rows(self, block):
        """The block's retained tail (its last T content rows) once its codes are staged."""
        return block.content_positions[-self.T:] if self.T and block.code_span else []

    def _record_content(self, n, is_prompt):       # processor.py:318-353
        block = self.current_block
        prev = self.blocks[-2] if len(self.blocks) > 1 else None
        for _ in range(n):
            pos = len(self.roles)
            within = len(block.content_positions)
            block.content_positions.append(pos)
            (block.prompt_positions if is_prompt else block.response_positions).append(pos)
            self.roles.append(CONTENT)
            self.kind.append("prompt" if is_prompt else "response")
            if prev is not None and within < len(prev.replay_positions):
                self.replay_expire_at[pos] = prev.replay_positions[within]
            if self.policy == "rolling" and prev is not None and within < len(self._tail_rows(prev)):
                row = self._tail_rows(prev)[within]
                if self.kind[row] == "response":   # raw-prompt rows never leave
                    self.expire_at[pos] = row

    def next_chunk(self):
        """Tokens the scheduler runs next for this request (limit_num_new_tokens with an unbounded budget)."""
        start = self.num_computed_tokens
        if self.finished or start >= self.num_tokens:
            return 0
        role = self.roles[start]
        end = start + 1
        while end < self.num_tokens and self.roles[end] == role:
            end += 1
        if role == CONTENT:
            for pos in range(start, end):          # a replay or rolling-tail expiry ends the chunk
                if pos in self.expire_at or pos in self.replay_expire_at:
                    return pos - start + 1
        return end - start

    def preempt(self):
        """Restart at token 0 with the logical stream kept and the compaction progress cleared."""
        self.num_computed_tokens = 0
        self.compacted_block_ids.clear()
        self.expired.clear()
        self.sticky_done.clear()
        self.replay_expired.clear()

    def should_skip_sampling(self, n):             # processor.py:153-168
        start = self.num_computed_tokens - n
        end = self.num_computed_tokens
        if self.roles[start] != CONTENT:
            return True
        if end < self.num_tokens:
            return True
        return self.pending_prompt < self.prompt_len

    def after_step(self, n):
        """update_after_step for a step that ran ``n`` tokens (num_computed_tokens already advanced).
        Returns the compaction calls as (start, end, groups-or-None) in call order."""
        end = self.num_computed_tokens
        start = end - n
        role = self.roles[start]
        sampled = not self.should_skip_sampling(n)
        calls = []
        if role == CONTENT:                            # replay expiries of the rows this step's queries saw last
            for pos in range(start, end):
                row = self.replay_expire_at.get(pos)
                if row is not None and row not in self.replay_expired:
                    calls.append((row, row + 1, None))
                    self.replay_expired.add(row)
        if role == CONTENT:                            # rolling expiries of the rows this step's queries saw last
            for pos in range(start, end):
                row = self.expire_at.get(pos)
                if row is not None and row not in self.expired:
                    calls.append((row, row + 1, None))
                    self.expired.add(row)
        if sampled:
            self.visible += 1
            if self.visible >= self.max_tokens:        # _check_stop (processor.py:663-685), length cap
                self.finished = True
                return calls
        block = self.blocks[self._block_of(start)]
        role_end = end == self.num_tokens or self.roles[end] != role
        if role == CONTENT:
            if len(block.content_positions) == self.C and end == block.content_positions[-1] + 1:
                calls += self._sticky_expire(block)
                if block.code_span is None:
                    self.held = sampled
                    cs = self.num_tokens                    # _stage_codes (processor.py:369-400)
                    self.roles.extend([CODE] * self.K)
                    self.kind.extend(["code"] * self.K)
                    block.code_span = (cs, cs + self.K)
            elif sampled:
                self._record_content(1, is_prompt=False)
        elif role == CODE and role_end:
            if self.R and not block.replay_positions:    # _stage_replay: the block's last R tokens after its codes
                rs = self.num_tokens
                self.roles.extend([REPLAY] * self.R)
                self.kind.extend(["replay"] * self.R)
                block.replay_positions = list(range(rs, rs + self.R))
            elif not block.replay_positions:
                calls = self._finish_block(block)
        elif role == REPLAY and role_end:
            calls = self._finish_block(block)
        return calls

    def _block_of(self, pos):
        for b in self.blocks:
            if b.content_positions and b.content_positions[0] <= pos:
                last = (b.replay_positions[-1] + 1 if b.replay_positions else
                        b.code_span[1] if b.code_span else b.content_positions[-1] + 1)
                if pos < last:
                    return b.block_id
        raise RuntimeError(f"position {pos} outside every block")

    def _sticky_expire(self, block):               # processor.py:559-592
        """Sticky policy: the previous block's tail response rows as one removal, once."""
        if self.policy != "sticky" or not block.block_id or block.block_id - 1 in self.sticky_done:
            return []
        prev = self.blocks[block.block_id - 1]
        self.sticky_done.add(prev.block_id)
        rows = [p for p in self._tail_rows(prev) if self.kind[p] == "response"]
        if not rows:
            return []
        if rows != list(range(rows[0], rows[-1] + 1)):
            raise RuntimeError("sticky retained response tail must be contiguous")
        return [(rows[0], rows[-1] + 1, None)]

    def _finish_block(self, block):                # processor.py:419-465, :467-557
        calls = self._sticky_expire(block)
        if block.block_id not in self.compacted_block_ids:
            tail = set(block.content_positions[-self.T:]) if self.T else set()
            pos = [p for p in block.response_positions if p not in tail]
            if pos:
                if pos != list(range(pos[0], pos[-1] + 1)):
                    raise RuntimeError("CompressLM response content must be contiguous")
                calls.append((pos[0], pos[-1] + 1, None))
            cs, ce = block.code_span
            for q in sorted(set(self.group_quotas)):
                if q >= self.K:
                    continue
                calls.append((cs + q, ce, [g for g, gq in enumerate(self.group_quotas) if gq == q]))
            self.compacted_block_ids.add(block.block_id)
        last = block.replay_positions[-1] + 1 if block.replay_positions else block.code_span[1]
        if last < self.num_tokens:                     # a preemption replay: the next block exists
            return calls
        nxt = Block(len(self.blocks))
        self.blocks.append(nxt)
        if self.pending_prompt < self.prompt_len:
            chunk = min(self.C, self.prompt_len - self.pending_prompt)
            self.pending_prompt += chunk
            self._record_content(chunk, is_prompt=True)
            return calls
        if not self.held:
            raise RuntimeError("CompressLM block completed without continuation token")
        self.held = False
        self._record_content(1, is_prompt=False)
        return calls

    def kept_positions(self, group):
        """Brute-force physical stream of ``group``: every logical position not removed from that group."""
        q = self.group_quotas[group]
        keep = []
        for b in self.blocks:
            compacted = b.block_id in self.compacted_block_ids
            tail = set(b.content_positions[-self.T:]) if self.T else set()
            for p in b.content_positions:
                if p >= self.num_computed_tokens:
                    continue
                if self.kind[p] == "response":
                    if compacted and p not in tail:
                        continue                       # summarized response content
                    if p in self.expired or (p in tail and b.block_id in self.sticky_done):
                        continue                       # an expired window-tail row
                keep.append(p)
            if b.code_span:
                cs, ce = b.code_span
                for p in range(cs, min(ce, self.num_computed_tokens)):
                    if not (compacted and p - cs >= q):
                        keep.append(p)
            for p in b.replay_positions:              # replay rows until the next block's content expires them
                if p < self.num_computed_tokens and p not in self.replay_expired:
                    keep.append(p)
        return sorted(keep)


def build_schedule(prompt_lens, max_tokens, start_steps, num_steps, C, K, group_quotas):
    """Planner-agnostic event stream of several requests served together.

    Every step first schedules each running request in request order (allocate ``n`` new tokens), then, after the
    model step, runs each request's update in request order (compaction calls), as the reference scheduler does
    (schedule(): scheduler.py:300-1061, then update_from_output -> update_after_step: scheduler.py:1512-1532).
    Returns (events, traces): events are ("alloc", rid, n) / ("mask", rid, start, end, groups) tuples grouped per
    step as a list of lists; traces are the final RequestTrace objects.
    """
    traces = [RequestTrace(p, m, C, K, group_quotas) for p, m in zip(prompt_lens, max_tokens)]
    steps = []
    for step in range(num_steps):
        events, ran = [], []
        for rid, tr in enumerate(traces):
            if step < start_steps[rid] or tr.finished:
                continue
            n = tr.next_chunk()
            if n == 0:
                continue
            events.append(("alloc", rid, n))
            tr.num_computed_tokens += n
            ran.append((rid, n))
        for rid, n in ran:
            for s, e, g in traces[rid].after_step(n):
                events.append(("mask", rid, s, e, g))
        steps.append(events)
    return steps, traces


def steps_until_closed(prompt_len, num_closed, C, K, group_quotas):
    """Number of steps a request needs, from its first prefill step, until ``num_closed`` blocks are compacted."""
    tr = RequestTrace(prompt_len, 1 << 30, C, K, group_quotas)
    steps = 0
    while len(tr.compacted_block_ids) < num_closed:
        n = tr.next_chunk()
        tr.num_computed_tokens += n
        tr.after_step(n)
        steps += 1
    return steps
