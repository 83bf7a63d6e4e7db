"""Scheduler-side block state machine: which tokens run when, and which spans are compacted.

API-compatible with the reference's CompressLMProcessor (third_party/vllm_overlay/vllm/v1/core/compresslm/
processor.py) for the served configuration (one pause pass, raw prompt, appended or bitrev positions, a replay tail or
a retained tail under the static, rolling or sticky policy, physical per-layer quotas or per-head packed KV pages):
prepare_request :42-105, is_code_ready / num_code_rows_pending :106-121, limit_num_new_tokens :123-151,
should_skip_sampling :153-168, update_after_step :170-257, reset_for_preemption :259-260 (state.py:46-50),
code_excluded_logical_range :262-274, code_physical_spans :276-316, _record_content :318-353, _stage_codes :369-400,
_stage_replay :402-417, _finish_block :419-465, _compact_response_content :467-557,
_expire_sticky_retained_tail_at_boundary :559-592, _expire_replay_after_content :594-618,
_expire_retained_tail_after_content :614-646, _mask_or_raise :648-661, _check_stop :663-685; the physical exclusion
ranges of a code step restate sched/scheduler.py:979-991. The compaction callback
``mask_span(request_id, start, end, groups=None)`` is KVPlanner.mask_token_span.

Replay tail: after a block's code run its last R content tokens are appended again (role REPLAY) and run as
ordinary chunks while the block's content is still resident; the block is compacted after them; the next block's
i-th content token removes replay row i after its step (prompt blocks' too), a content chunk ending at each such
token.

Window tails: a block's last T content rows survive its compaction; under "rolling" the i-th content token of the
next block removes the tail's i-th row (a response row; raw-prompt rows stay) after its step, and a content chunk
ends at every such token so each removal follows a query of its own; under "sticky" the tail's response rows go as
one span after the next block's last content token and before its codes.
"""
from __future__ import annotations

import enum
from collections.abc import Callable, Sequence
from dataclasses import dataclass, field

from .config import CompressLMConfig

CONTENT, CODE, REPLAY = 0, 1, 2

MaskSpan = Callable[..., object]


class RequestStatus(enum.IntEnum):
    RUNNING = 0
    FINISHED_STOPPED = 1
    FINISHED_LENGTH_CAPPED = 2


@dataclass
class SamplingSpec:
    """The sampling fields the state machine reads, and those prepare_request refuses to see changed from their
    defaults (vllm SamplingParams names)."""
    max_tokens: int = 1 << 30
    ignore_eos: bool = False
    stop_token_ids: tuple[int, ...] = ()
    min_tokens: int = 0
    bad_words_token_ids: list = field(default_factory=list)
    frequency_penalty: float = 0.0
    presence_penalty: float = 0.0
    repetition_penalty: float = 1.0
    stop: list | None = None
    logprobs: int | None = None
    prompt_logprobs: int | None = None


@dataclass
class CompressLMBlock:
    block_id: int
    content_positions: list[int] = field(default_factory=list)
    content_token_ids: list[int] = field(default_factory=list)
    prompt_content_positions: list[int] = field(default_factory=list)
    response_content_positions: list[int] = field(default_factory=list)
    code_span: tuple[int, int] | None = None
    replay_positions: list[int] = field(default_factory=list)
    retained_tail_positions: list[int] = field(default_factory=list)
    code_excluded_content_span: tuple[int, int] | None = None


@dataclass
class CompressLMState:
    original_prompt_token_ids: list[int]
    pending_prompt_index: int
    blocks: list[CompressLMBlock]
    roles: list[int] = field(default_factory=list)
    position_to_block: list[int] = field(default_factory=list)
    visible_output_token_ids: list[int] = field(default_factory=list)
    held_sampled_token: int | None = None
    compacted_block_ids: set[int] = field(default_factory=set)
    current_block_id: int = 0
    worker_token_ids_dirty: bool = False
    content_to_expired_replay: dict[int, int] = field(default_factory=dict)
    expired_replay_positions: set[int] = field(default_factory=set)
    content_to_expired_retained_tail: dict[int, int] = field(default_factory=dict)
    expired_retained_tail_positions: set[int] = field(default_factory=set)
    expired_sticky_retained_block_ids: set[int] = field(default_factory=set)

    @property
    def current_block(self) -> CompressLMBlock:
        return self.blocks[self.current_block_id]

    def reset_compaction_progress(self) -> None:
        self.expired_replay_positions.clear()
        self.expired_retained_tail_positions.clear()
        self.expired_sticky_retained_block_ids.clear()
        self.compacted_block_ids.clear()


class ServingRequest:
    """Minimal request object with the fields the state machine and the planner read (vllm.v1.request.Request)."""

    def __init__(self, request_id, prompt_token_ids, sampling: SamplingSpec | None = None, eos_token_id=None,
                 planner=None, prompt_embeds=None, pooling_params=None, use_structured_output=False):
        self.request_id = request_id
        self.prompt_token_ids = None if prompt_token_ids is None else list(prompt_token_ids)
        self.prompt_embeds = prompt_embeds
        self.pooling_params = pooling_params
        self.use_structured_output = use_structured_output
        if self.prompt_token_ids is None:
            self.num_prompt_tokens = 0
            self._all_token_ids: list[int] = []
            self._output_token_ids: list[int] = []
            self.num_computed_tokens = 0
            self.sampling_params = sampling or SamplingSpec()
            self.max_tokens = self.sampling_params.max_tokens
            self.eos_token_id = eos_token_id
            self.status = RequestStatus.RUNNING
            self.stop_reason = None
            self.compresslm_state = None
            self.planner = planner
            return
        self.num_prompt_tokens = len(self.prompt_token_ids)
        self._all_token_ids = list(self.prompt_token_ids)
        self._output_token_ids: list[int] = []
        self.num_computed_tokens = 0
        self.sampling_params = sampling or SamplingSpec()
        self.max_tokens = self.sampling_params.max_tokens
        self.eos_token_id = eos_token_id
        self.status = RequestStatus.RUNNING
        self.stop_reason = None
        self.compresslm_state: CompressLMState | None = None
        self.planner = planner

    @property
    def num_tokens(self) -> int:
        return len(self._all_token_ids)

    @property
    def all_token_ids(self) -> list[int]:
        return self._all_token_ids

    def append_output_token_ids(self, ids: Sequence[int]) -> None:
        self._output_token_ids.extend(ids)
        self._all_token_ids.extend(ids)

    def logical_to_physical(self, pos: int, group: int = 0) -> int:
        return pos if self.planner is None else self.planner.logical_to_physical(self.request_id, pos, group)


def _run_end(roles: list[int], start: int, stop: int) -> int:
    """End of the run of equal roles that begins at ``start`` (scanning no further than ``stop``)."""
    end = max(stop, start + 1)
    for other in (CONTENT, CODE, REPLAY):
        if other != roles[start]:
            try:
                end = min(end, roles.index(other, start + 1, stop))
            except ValueError:
                pass
    return end


def _no_mask(*_args, **_kwargs):
    raise RuntimeError("a replayed decode step cannot compact a block or expire a retained tail")


class CompressLMProcessor:
    def __init__(self, config: CompressLMConfig) -> None:
        if not config._initialized:
            raise ValueError("CompressLMConfig token IDs are not initialized")
        self.config = config
        self.group_quotas: tuple[int, ...] | None = None
        self._code_removals: list[tuple[int, list[int]]] = []
        T = config.retain_tail_kv
        self._rolling = T if config.retain_tail_policy == "rolling" else 0
        self._sticky = bool(T) and config.retain_tail_policy == "sticky"

    def set_group_quotas(self, group_quotas: Sequence[int] | None) -> None:
        if group_quotas is None:
            self.group_quotas = None
            self._code_removals = []
            return
        K = self.config.num_code_tokens
        for q in group_quotas:
            if not 0 < q <= K:
                raise ValueError(f"KV cache group quota {q} outside [1, {K}]")
        self.group_quotas = tuple(int(q) for q in group_quotas)
        # code slots [q, K) leave the groups of quota q, for each quota q < K in ascending order
        self._code_removals = [(q, [g for g, gq in enumerate(self.group_quotas) if gq == q])
                               for q in sorted(set(self.group_quotas)) if q < K]

    # -- request set-up -------------------------------------------------------------------------------------------
    def prepare_request(self, request) -> CompressLMState:
        """Validate a new request and open its first block (processor.py:42-105): the requests CompressLM decoding
        cannot serve are refused with the reference's messages, in its order."""
        sampling = request.sampling_params
        ga = getattr
        refusals = (
            (request.prompt_token_ids is None, "CompressLM decoding requires prompt token IDs"),
            (ga(request, "prompt_embeds", None) is not None, "CompressLM decoding does not support prompt_embeds"),
            (ga(request, "pooling_params", None) is not None, "CompressLM decoding only supports generation requests"),
            (sampling is None, "CompressLM decoding requires sampling parameters"),
        )
        for refused, message in refusals:
            if refused:
                raise ValueError(message)
        refusals = (
            (ga(sampling, "frequency_penalty", 0.0) != 0.0, "CompressLM decoding requires frequency_penalty=0"),
            (ga(sampling, "presence_penalty", 0.0) != 0.0, "CompressLM decoding requires presence_penalty=0"),
            (ga(sampling, "repetition_penalty", 1.0) != 1.0, "CompressLM decoding requires repetition_penalty=1"),
            (bool(ga(sampling, "stop", None)),
             "CompressLM decoding currently supports token/EOS stops, not stop strings"),
            (ga(sampling, "min_tokens", 0) != 0, "CompressLM decoding currently requires min_tokens=0"),
            (ga(sampling, "logprobs", None) is not None and not self.config.debug,
             "CompressLM output logprobs are only available in debug mode"),
            (ga(sampling, "prompt_logprobs", None) is not None, "CompressLM decoding does not support prompt logprobs"),
            (bool(ga(request, "use_structured_output", False)),
             "CompressLM decoding does not support structured output"),
        )
        for refused, message in refusals:
            if refused:
                raise ValueError(message)
        banned = {ids[0] for ids in (getattr(sampling, "bad_words_token_ids", None) or []) if len(ids) == 1}
        missing = set(self.config.code_token_ids) - banned
        if missing:
            raise ValueError("CompressLM code tokens must be passed as bad_words so internal IDs cannot be sampled; "
                             f"missing {len(missing)} IDs")
        prompt = list(request.prompt_token_ids)
        if not prompt:
            raise ValueError("CompressLM decoding requires a non-empty prompt")
        first = prompt[: self.config.block_size]
        state = CompressLMState(original_prompt_token_ids=prompt, pending_prompt_index=len(first),
                                blocks=[CompressLMBlock(block_id=0)])
        request.prompt_token_ids = first
        request.num_prompt_tokens = len(first)
        request._all_token_ids.clear()
        request._all_token_ids.extend(first)
        request._output_token_ids.clear()
        self._record_content(state, 0, first, is_prompt=True)
        return state

    # -- scheduling queries ---------------------------------------------------------------------------------------
    def is_code_ready(self, request) -> bool:
        state = request.compresslm_state
        if state is None or request.num_computed_tokens >= request.num_tokens:
            return False
        return state.roles[request.num_computed_tokens] == CODE

    def num_code_rows_pending(self, request) -> int:
        if not self.is_code_ready(request):
            return 0
        start = request.num_computed_tokens
        return _run_end(request.compresslm_state.roles, start, request.num_tokens) - start

    def limit_num_new_tokens(self, request, proposed: int) -> int:
        """A CODE run is scheduled whole (or not at all); a CONTENT run up to its end."""
        state = request.compresslm_state
        if state is None or proposed <= 0:
            return proposed
        start = request.num_computed_tokens
        if start >= request.num_tokens:
            return proposed
        role = state.roles[start]
        remaining = _run_end(state.roles, start, request.num_tokens) - start
        if role == CODE:
            return remaining if proposed >= remaining else 0
        limit = min(proposed, remaining)
        if role == CONTENT:                               # a replay or rolling-tail expiry ends the chunk
            replay, tail = state.content_to_expired_replay, state.content_to_expired_retained_tail
            if replay or tail:
                for pos in range(start, start + limit):
                    if pos in replay or pos in tail:
                        return pos - start + 1
        return limit

    def should_skip_sampling(self, request, num_scheduled_tokens: int) -> bool:
        state = request.compresslm_state
        if state is None:
            return False
        start = request.num_computed_tokens
        end = start + num_scheduled_tokens
        if state.roles[start] != CONTENT:
            return True
        if end < request.num_tokens:
            return True
        return state.pending_prompt_index < len(state.original_prompt_token_ids)

    # -- after a model step ---------------------------------------------------------------------------------------
    def update_after_step(self, request, num_scheduled_tokens: int, sampled_token_ids: list[int],
                          mask_span: MaskSpan, max_model_len: int, pack_code_span=None) -> tuple[list[int], bool]:
        """``request.num_computed_tokens`` already includes the step. Returns (visible sampled tokens, stopped)."""
        state = request.compresslm_state
        if state is None:
            return sampled_token_ids, False
        if len(sampled_token_ids) > 1:
            raise RuntimeError("CompressLM decoding is incompatible with speculative multi-token output")
        end = request.num_computed_tokens
        start = end - num_scheduled_tokens
        role = state.roles[start]
        if _run_end(state.roles, start, end) != end:
            raise RuntimeError("CompressLM scheduled a mixed-role model step")
        if role == CONTENT and state.content_to_expired_replay:
            self._expire_replay_after_content(state, request, start, end, mask_span)
        if role == CONTENT and state.content_to_expired_retained_tail:
            self._expire_retained_tail_after_content(state, request, start, end, mask_span)
        sampled = sampled_token_ids[0] if sampled_token_ids else None
        visible: list[int] = []
        if sampled is not None:
            state.visible_output_token_ids.append(sampled)
            visible.append(sampled)
            if self._check_stop(request, state, sampled, max_model_len):
                return visible, True
        block = state.blocks[state.position_to_block[start]]
        role_end = end == request.num_tokens or state.roles[end] != role
        if role == CONTENT:
            if len(block.content_positions) == self.config.block_size and end == block.content_positions[-1] + 1:
                if self._sticky:
                    # after the block's last content query, before its codes (also in a preemption replay, where
                    # the codes exist already)
                    self._expire_sticky_retained_tail_at_boundary(request, state, block, mask_span)
                if block.code_span is None:
                    if end + self.config.num_code_tokens + self.config.replay_tail >= max_model_len:
                        request.status = RequestStatus.FINISHED_LENGTH_CAPPED
                        return visible, True
                    state.held_sampled_token = sampled
                    self._stage_codes(request, state, block)
            elif sampled is not None:
                self._append_content(request, state, [sampled], is_prompt=False)
        elif role == CODE and role_end:
            if not block.replay_positions:
                self._stage_replay(request, state, block)
                if not block.replay_positions:
                    self._finish_block(request, state, block, mask_span, pack_code_span)
        elif role == REPLAY and role_end:
            self._finish_block(request, state, block, mask_span, pack_code_span)
        return visible, False

    def update_after_decode_steps(self, request, sampled_token_ids: Sequence[int], max_model_len: int) -> None:
        """``len(sampled_token_ids)`` consecutive one-token decode steps of one request at once, for replaying a known
        history: the same state as calling :meth:`update_after_step` once per step with ``num_scheduled_tokens=1``
        and the i-th sampled token, for a stretch in which no step computes the block's last content token (that step
        stages the codes), expires a replay row or a retained tail row (those steps issue removals) and no sampled
        token stops the request. ``request.num_computed_tokens`` already includes
        the steps. Anything else (a stretch reaching the block end, a possible stop) is stepped one by one."""
        ids = list(sampled_token_ids)
        m = len(ids)
        state = request.compresslm_state
        if m == 0:
            return
        end = request.num_computed_tokens
        start = end - m
        sampling = request.sampling_params
        stops = set(getattr(sampling, "stop_token_ids", None) or ())
        if not getattr(sampling, "ignore_eos", False) and request.eos_token_id is not None:
            stops.add(request.eos_token_id)
        block = state.blocks[state.position_to_block[start]] if start < len(state.position_to_block) else None
        fast = (state is not None and block is not None and request.num_tokens == start + 1
                and state.roles[start] == CONTENT and block is state.current_block
                and len(block.content_positions) + m <= self.config.block_size
                and block.content_positions[-1] == start and (not stops or stops.isdisjoint(ids))
                and (not self._rolling or not block.block_id or len(block.content_positions) > self._rolling)
                and (not block.block_id or len(block.content_positions) >
                     len(state.blocks[block.block_id - 1].replay_positions))
                and request.num_tokens + m < max_model_len
                and len(state.visible_output_token_ids) + m < request.max_tokens)
        if not fast:
            request.num_computed_tokens = start
            for tok in ids:
                request.num_computed_tokens += 1
                _, stopped = self.update_after_step(request, 1, [tok], _no_mask, max_model_len)
                if stopped:
                    raise RuntimeError("a replayed decode step stopped the request")
            return
        state.visible_output_token_ids.extend(ids)
        self._append_content(request, state, ids, is_prompt=False)

    def reset_for_preemption(self, state: CompressLMState) -> None:
        state.reset_compaction_progress()

    def code_excluded_logical_range(self, request) -> tuple[int, int] | None:
        """Logical [start, end) of the content rows the scheduled code step's codes must not see (their block's
        retained tail), or None without a tail. The block is the one whose code rows are scheduled: the current
        block, except in a preemption replay, where earlier blocks' code steps run again (the reference reads the
        current block there, processor.py:262-274, which fails or names the wrong rows in a replay)."""
        if not self.config.code_excluded_tail:
            return None
        state = request.compresslm_state
        if state is None:
            raise RuntimeError("CompressLM request has no state")
        start = request.num_computed_tokens
        if start < len(state.roles) and state.roles[start] == CODE:
            block = state.blocks[state.position_to_block[start]]
        else:
            block = state.current_block
        if block.code_excluded_content_span is None:
            raise RuntimeError("tail-exclusive code block has no source span")
        return block.code_excluded_content_span

    def code_excluded_physical_ranges(self, request, num_groups: int) -> list[tuple[int, int]] | None:
        """Physical [start, end) of the excluded range in each KV-cache group's layout during the block's code step
        (sched/scheduler.py:979-991), or None without a tail."""
        logical = self.code_excluded_logical_range(request)
        if logical is None:
            return None
        ls, le = logical
        ranges = []
        for g in range(num_groups):
            ps = request.logical_to_physical(ls, g)
            pe = request.logical_to_physical(le - 1, g) + 1
            if pe - ps != self.config.code_excluded_tail:
                raise RuntimeError("exact tail source is not contiguous after KV compaction")
            ranges.append((ps, pe))
        return ranges

    def code_physical_spans(self, request, group: int = 0, logical_limit: int | None = None):
        """Physical [start, end) of every staged code span still holding all K rows in ``group``'s layout."""
        state = request.compresslm_state
        if state is None:
            raise RuntimeError("CompressLM request has no state")
        K = self.config.num_code_tokens
        spans = []
        for block in state.blocks:
            if block.code_span is None:
                continue
            if (self.group_quotas is not None or self.config.uses_packed_kv) and \
                    block.block_id in state.compacted_block_ids:
                continue
            start, end = block.code_span
            if logical_limit is not None and end > logical_limit:
                continue
            ps = request.logical_to_physical(start, group)
            pe = request.logical_to_physical(end - 1, group) + 1
            if pe - ps != K:
                raise RuntimeError("code span is not contiguous after KV compaction")
            spans.append((ps, pe))
        return spans

    # -- internals ------------------------------------------------------------------------------------------------
    def _record_content(self, state: CompressLMState, start: int, token_ids, is_prompt: bool) -> None:
        block = state.current_block
        n = len(token_ids)
        within = len(block.content_positions)
        positions = range(start, start + n)
        block.content_positions.extend(positions)
        block.content_token_ids.extend(token_ids)
        (block.prompt_content_positions if is_prompt else block.response_content_positions).extend(positions)
        state.roles.extend([CONTENT] * n)
        state.position_to_block.extend([block.block_id] * n)
        if block.block_id:
            # the i-th content token of the block expires the previous block's i-th replay row
            rep = state.blocks[block.block_id - 1].replay_positions
            for i in range(within, min(within + n, len(rep))):
                state.content_to_expired_replay[start + i - within] = rep[i]
        if self._rolling and block.block_id and within < self._rolling:
            # the i-th content token of the block expires the previous block's i-th tail row if it is a response
            # row (a block's response rows are one contiguous run after its prompt rows)
            prev = state.blocks[block.block_id - 1]
            tail, resp = prev.retained_tail_positions, prev.response_content_positions
            for i in range(within, min(within + n, len(tail))):
                row = tail[i]
                if resp and resp[0] <= row <= resp[-1]:
                    state.content_to_expired_retained_tail[start + i - within] = row

    def _append_content(self, request, state, token_ids, is_prompt: bool) -> None:
        if not token_ids:
            return
        start = request.num_tokens
        request.append_output_token_ids(token_ids)
        self._record_content(state, start, token_ids, is_prompt)

    def _stage_codes(self, request, state, block) -> None:
        start = request.num_tokens
        ids = self.config.code_token_ids
        request.append_output_token_ids(ids)
        block.code_span = (start, request.num_tokens)
        T = self.config.retain_tail_kv
        if T:
            block.retained_tail_positions = block.content_positions[-T:]
        X = self.config.code_excluded_tail
        if X:
            tail = block.content_positions[-X:]
            if tail != list(range(tail[0], tail[-1] + 1)):
                raise RuntimeError("exact tail source positions must be contiguous")
            block.code_excluded_content_span = (tail[0], tail[-1] + 1)
        state.roles.extend([CODE] * len(ids))
        state.position_to_block.extend([block.block_id] * len(ids))
        state.worker_token_ids_dirty = True

    def _stage_replay(self, request, state, block) -> None:
        """Append the block's last R content tokens after its codes as replay tokens (processor.py:402-417)."""
        R = self.config.replay_tail
        if not R:
            return
        ids = block.content_token_ids[-R:]
        start = request.num_tokens
        request.append_output_token_ids(ids)
        block.replay_positions = list(range(start, start + len(ids)))
        state.roles.extend([REPLAY] * len(ids))
        state.position_to_block.extend([block.block_id] * len(ids))
        state.worker_token_ids_dirty = True

    def _finish_block(self, request, state, block, mask_span, pack_code_span=None) -> None:
        if self._sticky:                                      # done at the block's last content step already
            self._expire_sticky_retained_tail_at_boundary(request, state, block, mask_span)
        self._compact_response_content(request, state, block, mask_span, pack_code_span)
        last = block.replay_positions[-1] + 1 if block.replay_positions else block.code_span[1]
        if last < request.num_tokens:                        # preemption replay: later tokens already exist
            return
        nxt = CompressLMBlock(block_id=len(state.blocks))
        state.blocks.append(nxt)
        state.current_block_id = nxt.block_id
        if state.pending_prompt_index < len(state.original_prompt_token_ids):
            chunk = state.original_prompt_token_ids[state.pending_prompt_index:][: self.config.block_size]
            state.pending_prompt_index += len(chunk)
            self._append_content(request, state, chunk, is_prompt=True)
            state.worker_token_ids_dirty = True
            return
        if state.held_sampled_token is None:
            raise RuntimeError("CompressLM block completed without continuation token")
        held, state.held_sampled_token = state.held_sampled_token, None
        self._append_content(request, state, [held], is_prompt=False)
        state.worker_token_ids_dirty = True

    def block_removal_spans(self, block: CompressLMBlock) -> list[tuple[int, int, list[int] | None]]:
        """The span removals that compact a closed block, in the order they must run: ``(start, end, groups)`` with
        ``groups`` None for every KV-cache group (compresslm/processor.py:467-557). Response content goes from every
        group, then (physical quotas) code slots [q, K) from the groups of each quota q < K, ascending q, each on the
        layout the previous removal left. Packed KV: the response content and the codes as one span (the codes are
        archived into packed pages before it runs). A retained tail (the block's last T content rows) is not removed
        with the block: the response content before it goes, and with packed KV (static tail only) the codes go as a
        span of their own; the window policies remove the tail later (``_expire_*``)."""
        pos = block.response_content_positions
        if self.config.retain_tail_kv:
            kept = set(block.retained_tail_positions)
            pos = [p for p in pos if p not in kept]
        if pos and pos[-1] - pos[0] + 1 != len(pos):
            raise RuntimeError("packed KV response content must be contiguous" if self.config.uses_packed_kv
                               else "CompressLM response content must be contiguous")
        if self.config.uses_packed_kv:
            if block.code_span is None:
                raise RuntimeError("packed KV block has no completed code span")
            cs, ce = block.code_span
            if self.config.retain_tail_kv:
                return ([(pos[0], pos[-1] + 1, None)] if pos else []) + [(cs, ce, None)]
            if pos and pos[-1] + 1 != cs:
                raise RuntimeError("packed KV response content and code span are not contiguous")
            return [(pos[0] if pos else cs, ce, None)]
        spans: list[tuple[int, int, list[int] | None]] = []
        if pos:
            spans.append((pos[0], pos[-1] + 1, None))
        if self.group_quotas is not None:
            if block.code_span is None:
                raise RuntimeError("physical per-layer quotas need a completed code span")
            cs, ce = block.code_span
            for q, groups in self._code_removals:
                spans.append((cs + q, ce, list(groups)))
        return spans

    def _compact_response_content(self, request, state, block, mask_span, pack_code_span=None) -> None:
        """Run :meth:`block_removal_spans` of the block through ``mask_span``. Packed KV: archive the code span first
        (``pack_code_span(request_id, start, end)``), then remove the response content and the codes as one span
        (compresslm/processor.py:484-520)."""
        if block.block_id in state.compacted_block_ids:
            return
        spans = self.block_removal_spans(block)
        if self.config.uses_packed_kv:
            if pack_code_span is None:
                raise RuntimeError("packed KV decoding has no code capture callback")
            pack_code_span(request.request_id, *block.code_span)
        for start, end, groups in spans:
            self._mask_or_raise(mask_span, request.request_id, start, end, groups=groups)
        state.compacted_block_ids.add(block.block_id)

    def _expire_sticky_retained_tail_at_boundary(self, request, state, block, mask_span) -> None:
        """Sticky policy: remove the previous block's retained response rows as one span, once per block
        (processor.py:559-592)."""
        if not block.block_id:
            return
        prev = state.blocks[block.block_id - 1]
        if prev.block_id in state.expired_sticky_retained_block_ids:
            return
        resp = prev.response_content_positions
        rows = [p for p in prev.retained_tail_positions if resp and resp[0] <= p <= resp[-1]]
        if rows:
            if rows[-1] - rows[0] + 1 != len(rows):
                raise RuntimeError("sticky retained response tail must be contiguous")
            self._mask_or_raise(mask_span, request.request_id, rows[0], rows[-1] + 1)
        state.expired_sticky_retained_block_ids.add(prev.block_id)

    def _expire_replay_after_content(self, state, request, start, end, mask_span) -> None:
        """Remove each previous-block replay row whose expiring content token ran in [start, end)
        (processor.py:594-618)."""
        expiring, expired = state.content_to_expired_replay, state.expired_replay_positions
        for pos in range(start, end):
            row = expiring.get(pos)
            if row is None or row in expired:
                continue
            self._mask_or_raise(mask_span, request.request_id, row, row + 1)
            expired.add(row)

    def _expire_retained_tail_after_content(self, state, request, start, end, mask_span) -> None:
        """Rolling policy: remove each previous-block tail row whose expiring content token ran in [start, end)
        (processor.py:614-646)."""
        expiring, expired = state.content_to_expired_retained_tail, state.expired_retained_tail_positions
        for pos in range(start, end):
            row = expiring.get(pos)
            if row is None or row in expired:
                continue
            self._mask_or_raise(mask_span, request.request_id, row, row + 1)
            expired.add(row)

    @staticmethod
    def _mask_or_raise(mask_span, request_id, start, end, groups=None) -> None:
        """Run one removal; a failed SpanRemovalResult becomes RuntimeError (processor.py:648-661)."""
        res = mask_span(request_id, start, end) if groups is None else mask_span(request_id, start, end, groups=groups)
        if not res.success:
            raise RuntimeError(f"CompressLM KV compaction failed for [{start}, {end}): {res.error_message}")

    @staticmethod
    def _check_stop(request, state, token_id, max_model_len) -> bool:
        sampling = request.sampling_params
        visible = len(state.visible_output_token_ids)
        if visible < getattr(sampling, "min_tokens", 0):
            return False
        if not getattr(sampling, "ignore_eos", False) and token_id == request.eos_token_id:
            request.status = RequestStatus.FINISHED_STOPPED
            return True
        if token_id in (getattr(sampling, "stop_token_ids", None) or ()):
            request.status = RequestStatus.FINISHED_STOPPED
            request.stop_reason = token_id
            return True
        if request.num_tokens >= max_model_len or visible >= request.max_tokens:
            request.status = RequestStatus.FINISHED_LENGTH_CAPPED
            return True
        return False
