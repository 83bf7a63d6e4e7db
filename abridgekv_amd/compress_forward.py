"""Teacher-forced CompressLM forward over the masked-prefill kernel (the training/evaluation entry point).

Mirrors abridgekv/compress_forward.py:240-1230 (``CompressLM``): L pause passes (pass l of a block refines pass
l - 1; later blocks read the final pass, :566-649), code<->code attention within a pass bidirectional
(``pause_xattn="full"``, the served setting), causal or absent (``"causal"``, ``"none"``: :313-314, 622-625),
optional raw prompt, optional fixed per-(layer, KV head) code quotas, ``active_code_rows``, ``appended`` /
``bitrev`` code positions and the retained tail (``retain_tail_kv`` = T: a block's codes do not see or summarize its
last T content rows, bitrev codes spread over the first C - T; by ``retain_tail_policy`` those rows stay visible to
every later row ("static"), to the next block's content rows ("sticky"), or to the next block's i-th content row
from tail row i on ("rolling"), compress_forward.py:99-124); the replay tail (``replay_tail`` = R rows after a
block's codes replaying its last R content tokens, seen by the next block's content as a rolling window;
``code_exclude_replay_tail`` hides those content rows from the codes, :139-178, 594-603); the code-seed pools
(``seg_pool``, ``gated_seg_pool``, ``pool_init``, :315-343, 1147-1178) and the code-row projections
(``query_residual``, ``code_q_heads``, ``code_kv_heads``, :181-222, 397-432). The sequence layout, RoPE positions,
loss positions and
loss reductions follow the reference (compress_forward.py:20-88, 1044-1071, 957-1042, 1134-1230); the attention of
every decoder layer runs ``abkv_prefill_masked_attn`` through a HuggingFace attention function registered as
``"abridgekv_hip"`` in place of FlexAttention with a BlockMask (``_arith_mask_mod`` / ``_mask_mod`` /
``_mask_rawprompt_mod`` / ``_quota_key_allowed``, compress_forward.py:230-236, 566-649, 695-727, 815-894). The mask
is never materialised: the kernel evaluates it from (C, K, L, R, N, prompt_len, head quota, tail, xattn); layouts off
the 64-row tile grid, L > 1, replay rows, the raw tail and non-full xattn take its per-element walk.

The raw tail (``raw_tail`` = W, a training ablation the reference's serving refuses, compress_forward.py:89-96):
content row i of the next block sees the block's last W - i content rows (the rolling window of a retained tail),
and the block's codes see their whole block.
Gradients flow through the attention by the kernel's HIP backward (dq, dk, dv under the same mask), so the module
trains.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch
import torch.nn.functional as F
from torch import nn

from . import ops
from .config import bitrev_offsets

ATTN_IMPLEMENTATION = "abridgekv_hip"


@dataclass(frozen=True)
class CompressMask:
    """What the kernel needs to evaluate the compression mask (the analogue of the reference's BlockMask):
    N blocks of [C content | ``passes`` passes of K code rows] and ``copy_rows`` copy-region rows (codes_k = 0: causal
    attention within blocks of C rows); ``prompt_len`` [B] int32 raw-prompt content tokens (None: no raw prompt);
    ``head_quota`` [layers, 32] int32 code rows visible per query head (None: all K); ``retain_tail`` T of a retained
    tail (0: none) under ``tail_policy`` ("static", "rolling", "sticky", or "raw" for the raw tail: the rolling
    window, seen by the codes too)."""
    block_c: int
    codes_k: int
    num_blocks: int
    prompt_len: torch.Tensor | None = None
    head_quota: torch.Tensor | None = None
    retain_tail: int = 0
    tail_policy: str = "static"
    pause_xattn: str = "full"
    passes: int = 1
    copy_rows: int = 0
    replay_rows: int = 0
    replay_exclude: bool = False


class _MaskedPrefill(torch.autograd.Function):
    """The masked-prefill kernel and its backward (abkv_prefill_masked_attn / _bwd), the FlexAttention
    forward + backward the reference trains through (compress_forward.py:1134-1230, :1329)."""

    @staticmethod
    def forward(ctx, q, k, v, mask: CompressMask, layer_idx: int, scale: float):
        hq = None if mask.head_quota is None else mask.head_quota[layer_idx]
        need_grad = any(ctx.needs_input_grad[:3])
        lse = None
        if need_grad:
            if q.dtype != torch.bfloat16:
                raise NotImplementedError("the masked-prefill backward runs bf16 inputs")
            lse = torch.empty((q.shape[0], ops.HEADS_Q, q.shape[1]), dtype=torch.float32, device=q.device)
        out, _ = ops.prefill_masked_attention(q, k, v, mask.block_c, mask.codes_k, mask.num_blocks,
                                              prompt_len=mask.prompt_len, head_quota=hq, scale=scale, lse=lse,
                                              retain_tail=mask.retain_tail, tail_policy=mask.tail_policy,
                                              pause_xattn=mask.pause_xattn, pause_passes=mask.passes,
                                              copy_rows=mask.copy_rows, replay_rows=mask.replay_rows,
                                              replay_exclude=mask.replay_exclude)
        if need_grad:
            ctx.save_for_backward(q, k, v, out, lse)
            ctx.mask, ctx.hq, ctx.scale = mask, hq, scale
        return out

    @staticmethod
    def backward(ctx, grad_out):
        q, k, v, out, lse = ctx.saved_tensors
        m = ctx.mask
        g = grad_out if grad_out.stride(-1) == 1 else grad_out.contiguous()
        dq, dk, dv = ops.prefill_masked_attention_backward(q, k, v, out, lse, g, m.block_c, m.codes_k, m.num_blocks,
                                                           prompt_len=m.prompt_len, head_quota=ctx.hq,
                                                           scale=ctx.scale, retain_tail=m.retain_tail,
                                                           tail_policy=m.tail_policy, pause_xattn=m.pause_xattn,
                                                           pause_passes=m.passes, copy_rows=m.copy_rows,
                                                           replay_rows=m.replay_rows,
                                                           replay_exclude=m.replay_exclude)
        return dq, dk, dv, None, None, None


def masked_attention_forward(module, query, key, value, attention_mask, scaling=None, dropout=0.0, **kwargs):
    """HuggingFace attention function: query [B, 32, S, 128], key/value [B, 8, S, 128] bf16 ->
    (out [B, S, 32, 128], None). ``attention_mask`` is a :class:`CompressMask`, or None for a plain causal forward
    of the model (the full-context baseline and teacher, compress_forward.py:952-956, 1095-1105), which runs the
    same kernel without code rows."""
    if attention_mask is None:
        attention_mask = CompressMask(query.shape[2], 0, 1)
    if not isinstance(attention_mask, CompressMask):
        raise TypeError(f"{ATTN_IMPLEMENTATION} attention needs a CompressMask or None, got "
                        f"{type(attention_mask).__name__}")
    if dropout:
        raise NotImplementedError("attention dropout is not supported")
    if kwargs.get("sliding_window"):
        raise NotImplementedError("sliding-window attention is not supported")
    scale = ops.default_scale() if scaling is None else float(scaling)
    out = _MaskedPrefill.apply(query.transpose(1, 2), key.transpose(1, 2), value.transpose(1, 2), attention_mask,
                               int(module.layer_idx), scale)
    return out, None


def register_attention() -> None:
    """Register ``"abridgekv_hip"`` with transformers' attention interface (idempotent)."""
    from transformers import AttentionInterface
    AttentionInterface.register(ATTN_IMPLEMENTATION, masked_attention_forward)


def roles(C: int, N: int, K: int, device=None, L: int = 1, R: int = 0):
    """(blk, role) per row of the layout of N blocks of [C content | L passes of K codes | R replay rows]: role 0 =
    content, 1..L = pause pass, L + 1 = replay (compress_forward.py:20-31)."""
    per = C + L * K + R
    within = torch.arange(per, device=device).repeat(N)
    blk = torch.arange(N, device=device).repeat_interleave(per)
    code = torch.div(within - C, max(K, 1), rounding_mode="floor") + 1
    role = torch.where(within < C, torch.zeros_like(within), torch.where(within < C + L * K, code,
                                                                         torch.full_like(within, L + 1)))
    return blk, role


def content_abs_pos(C: int, N: int, K: int, device=None, L: int = 1, R: int = 0) -> torch.Tensor:
    """Absolute content index b*C + j of content rows, of the replayed token for replay rows; N*C for code rows
    (compress_forward.py:72-88)."""
    per = C + L * K + R
    within = torch.arange(per, device=device).repeat(N)
    blk = torch.arange(N, device=device).repeat_interleave(per)
    pos = torch.where(within < C, blk * C + within, torch.full_like(within, N * C))
    return torch.where(within >= C + L * K, blk * C + (C - R) + (within - C - L * K), pos)


def rope_position_ids(C: int, N: int, K: int, K_act: int, code_positions: str, device=None,
                      code_excluded_tail: int = 0, L: int = 1, R: int = 0) -> torch.Tensor:
    """(1, N*(C+L*K_act+R)) RoPE positions numbered as in the full-K layout (compress_forward.py:1044-1071, no copy
    rows): appended code row p of a block sits at C + (p // K_act) K + p % K_act of the full layout and replay row r
    at C + L K + r; bitrev code rows (L = 1, no replay rows) spread over the first C - code_excluded_tail in-block
    offsets."""
    per_full, per_act = C + L * K + R, C + L * K_act + R
    idx = torch.arange(N * per_act, device=device)
    within, blk = idx % per_act, idx // per_act
    is_code = (within >= C) & (within < C + L * K_act)
    p = (within - C).clamp_min(0)
    if code_positions == "bitrev":
        offs = torch.from_numpy(bitrev_offsets(K, C - code_excluded_tail)).to(device)
        pos = torch.where(is_code, blk * C + offs[p.clamp_max(K - 1)], blk * C + within)
    else:
        slot = torch.div(p, K_act, rounding_mode="floor") * K + p % K_act
        pos = torch.where(is_code, blk * per_full + C + slot, blk * per_full + within)
        replay = within >= C + L * K_act
        pos = torch.where(replay, blk * per_full + C + L * K + (within - C - L * K_act), pos)
    return pos.view(1, -1)


class _CodeRows:
    """The code rows of the current teacher-forced layout (sequence indices and slot 0..L*K_act-1 within the block),
    shared by the code-row projections and kept current by :meth:`CompressLM.set_N`."""

    def __init__(self):
        self.rows = self.slots = None
        self.S0 = -1
        self.lengths = ()           # sequence lengths of the layout: S0, and S0 + 1 + C with the copy region
        self._copies = {}

    def at(self, device):
        """(rows, slots) on ``device`` (the module may have been moved after the layout was built); copies are kept
        per device, the layout's own tensors stay where it built them."""
        if self.rows.device == device:
            return self.rows, self.slots
        key = (str(device), self.S0)
        if key not in self._copies:
            self._copies[key] = (self.rows.to(device), self.slots.to(device))
        return self._copies[key]


class _QProjQRes(nn.Module):
    """q_proj of one layer plus a learned query residual per code slot, added at the code rows of the compressed
    layout (``query_residual``, compress_forward.py:181-199, 397-413). ``qres`` starts at zero (an exact no-op) and
    sequences of another length than the layout's pass through unchanged. Names ``orig`` / ``qres`` as in the
    reference's state dict."""

    def __init__(self, orig: nn.Linear, num_slots: int, code_rows: _CodeRows):
        super().__init__()
        self.orig = orig
        self.qres = nn.Parameter(torch.zeros(num_slots, orig.out_features, device=orig.weight.device))
        self._code_rows = code_rows

    def forward(self, x):
        out = self.orig(x)
        cr = self._code_rows
        if out.size(1) not in cr.lengths:
            return out
        rows, slots = cr.at(out.device)
        res = self.qres.index_select(0, slots).to(out.dtype)
        return out.index_add(1, rows, res.unsqueeze(0).expand(out.size(0), -1, -1))


class _QProjCode(nn.Module):
    """A projection (q_proj, or k_proj / v_proj) of one layer whose code rows go through their own copy of the
    weights (``code_q_heads`` / ``code_kv_heads``, compress_forward.py:202-222, 414-432): ``code`` starts as a copy of
    ``orig`` (an exact no-op), content rows and sequences of another length keep ``orig``."""

    def __init__(self, orig: nn.Linear, code_rows: _CodeRows):
        super().__init__()
        self.orig = orig
        self.code = nn.Linear(orig.in_features, orig.out_features, bias=orig.bias is not None,
                              device=orig.weight.device, dtype=orig.weight.dtype)
        with torch.no_grad():
            self.code.weight.copy_(orig.weight)
            if orig.bias is not None:
                self.code.bias.copy_(orig.bias)
        self._code_rows = code_rows

    def forward(self, x):
        out = self.orig(x)
        cr = self._code_rows
        if out.size(1) not in cr.lengths:
            return out
        rows, _ = cr.at(out.device)
        return out.index_copy(1, rows, self.code(x.index_select(1, rows)).to(out.dtype))


def code_seeds(clm, tok_e: torch.Tensor, segment_mean: bool = False) -> torch.Tensor:
    """Input embeddings [..., K, d] of one pass of code rows for blocks whose content embeddings are tok_e
    [..., C, d] (compress_forward.py:1147-1178, gen_compress.py:867-898): the learned seeds ``pause``, plus the
    mean of K contiguous segments of the block's content (``seg_pool``, ``gated_seg_pool`` times a learned per-slot
    gate; ``segment_mean`` forces it) or a learned softmax pooling of the content (``pool_init``). Both pools read
    the content rows the codes summarise (the first C - T under a retained tail)."""
    K = getattr(clm, "K_act", clm.K)
    mdt = tok_e.dtype
    d = tok_e.size(-1)
    lead = tok_e.shape[:-2]
    T = getattr(clm, "code_excluded_tail", 0)
    src = tok_e[..., : tok_e.size(-2) - T, :] if T else tok_e
    n = src.size(-2)
    pause = clm.pause[:K].to(mdt)
    gated = getattr(clm, "gated_seg_pool", False)
    if segment_mean or gated or getattr(clm, "seg_pool", False):
        seg = n // K
        if seg >= 1:
            tm = src[..., : K * seg, :].reshape(*lead, K, seg, d).mean(-2)
        else:                                                      # fewer content rows than codes: the block mean
            tm = src.mean(-2, keepdim=True).expand(*lead, K, d)
        if gated:
            tm = tm * clm.seg_pool_gate.to(mdt).view(K, 1)
        return pause + tm.to(mdt)
    if getattr(clm, "pool_init", False):
        keys = F.linear(src, clm.pool_k.weight.to(mdt))
        vals = F.linear(src, clm.pool_v.weight.to(mdt))
        sc = torch.matmul(keys, clm.pool_q.to(mdt).t()).transpose(-1, -2) * (d ** -0.5)      # [..., K, n]
        return pause + torch.matmul(sc.float().softmax(-1).to(mdt), vals)
    return pause.expand(*lead, K, d)




class CompressLM(nn.Module):
    """API-compatible ``CompressLM(base_model, C, N, K, ...)`` (compress_forward.py:239-433), same positional order.

    ``base_model`` is a HuggingFace causal LM with 32 query heads, 8 KV heads and head size 128 in bf16 (e.g.
    Qwen3-4B or a random model of that attention shape); its attention implementation is switched to
    ``"abridgekv_hip"``.
    """

    def __init__(self, base_model, C, N, K, L=1, pause_xattn="full", pool_init=False, query_residual=False,
                 code_q_heads=False, code_kv_heads=False, seg_pool=False, gated_seg_pool=False, raw_tail=0,
                 replay_tail=0, code_exclude_replay_tail=False, retain_tail_kv=0, retain_tail_policy="rolling",
                 head_code_quotas=None, active_code_rows=None, code_positions="appended"):
        super().__init__()
        if int(L) != L or L < 1:
            raise ValueError(f"L must be a positive integer, got {L}")
        if pause_xattn not in ("none", "causal", "full"):
            raise ValueError(f"pause_xattn must be 'none', 'causal' or 'full', got {pause_xattn!r}")
        if not 0 <= replay_tail <= C:
            raise ValueError(f"replay_tail must be in [0, C={C}], got {replay_tail}")
        if not 0 <= raw_tail <= C:
            raise ValueError(f"raw_tail must be in [0, C={C}], got {raw_tail}")
        if not 0 <= retain_tail_kv < C:
            raise ValueError(f"retain_tail_kv must be in [0, C={C}), got {retain_tail_kv}")
        if sum(bool(value) for value in (raw_tail, replay_tail, retain_tail_kv)) > 1:
            raise ValueError("raw_tail, replay_tail, and retain_tail_kv are mutually exclusive")
        if retain_tail_policy not in ("rolling", "sticky", "static"):
            raise ValueError(f"retain_tail_policy must be 'rolling', 'sticky' or 'static', got {retain_tail_policy!r}")
        if retain_tail_policy != "rolling" and not retain_tail_kv:
            raise ValueError(f"retain_tail_policy={retain_tail_policy!r} requires retain_tail_kv > 0")
        if code_exclude_replay_tail and not 0 < replay_tail < C:
            raise ValueError("code_exclude_replay_tail requires replay_tail in [1, C)")
        if code_positions not in ("appended", "bitrev"):
            raise ValueError(f"code_positions must be 'appended' or 'bitrev', got {code_positions!r}")
        if code_positions == "bitrev" and (K & (K - 1) or C & (C - 1) or L != 1 or replay_tail or raw_tail):
            raise ValueError("code_positions='bitrev' needs power-of-two C and K, L=1 and no tails")
        if query_residual and code_q_heads:
            raise ValueError("query_residual and code_q_heads both replace q_proj; enable one of them")
        cfg = base_model.config
        heads, kv_heads = int(cfg.num_attention_heads), int(getattr(cfg, "num_key_value_heads", cfg.num_attention_heads))
        head_dim = int(getattr(cfg, "head_dim", None) or cfg.hidden_size // heads)
        if (heads, kv_heads, head_dim) != (ops.HEADS_Q, ops.HEADS_KV, ops.HEAD_DIM):
            raise NotImplementedError(f"the kernels need {ops.HEADS_Q} query heads, {ops.HEADS_KV} KV heads and "
                                      f"head size {ops.HEAD_DIM}; got {(heads, kv_heads, head_dim)}")
        register_attention()
        self.model = base_model
        self.model.config._attn_implementation = ATTN_IMPLEMENTATION
        self.C, self.N, self.K, self.L = int(C), int(N), int(K), int(L)
        self.pause_xattn, self.code_positions = pause_xattn, code_positions
        self.raw_tail = int(raw_tail)
        self.replay_tail = int(replay_tail)
        self.code_exclude_replay_tail = bool(code_exclude_replay_tail)
        self.retain_tail_kv = int(retain_tail_kv)
        # the content rows a block's codes neither see nor summarise (compress_forward.py:298-300)
        self.code_excluded_tail = self.replay_tail if self.code_exclude_replay_tail else self.retain_tail_kv
        self.retain_tail_policy = retain_tail_policy
        if code_positions == "bitrev" and C - self.code_excluded_tail < K:
            raise ValueError(f"bitrev code span {C - self.code_excluded_tail} < num_code_tokens {K}")
        self.K_act = int(active_code_rows) if active_code_rows else self.K
        if not 1 <= self.K_act <= self.K:
            raise ValueError(f"active_code_rows must be in [1, K={K}], got {active_code_rows}")
        if self.K_act != self.K and (pool_init or seg_pool or gated_seg_pool):
            raise ValueError("active_code_rows < K is not supported with pool_init/seg_pool")
        d = int(cfg.hidden_size)
        std = getattr(cfg, "initializer_range", 0.02)
        dev = next(base_model.parameters()).device
        self.pause = nn.Parameter(torch.empty(self.K, d, device=dev).normal_(0, std))
        self.copy_token = nn.Parameter(torch.empty(d, device=dev).normal_(0, std))   # heads the copy region
        # code-seed pools (compress_forward.py:315-343): a per-slot gate on the segment means (zero: the generic
        # seeds), or K learned queries over the content with a zero value map (likewise an exact no-op at first)
        self.pool_init, self.seg_pool, self.gated_seg_pool = bool(pool_init), bool(seg_pool), bool(gated_seg_pool)
        if gated_seg_pool:
            self.seg_pool_gate = nn.Parameter(torch.zeros(self.K, device=dev))
        if pool_init:
            self.pool_q = nn.Parameter(torch.empty(self.K, d, device=dev).normal_(0, std))
            self.pool_k = nn.Linear(d, d, bias=False, device=dev)
            self.pool_v = nn.Linear(d, d, bias=False, device=dev)
            nn.init.zeros_(self.pool_v.weight)
        self.num_layers = len(self.model.model.layers)
        self.num_attention_heads, self.num_kv_heads = heads, kv_heads
        self.num_key_value_groups = heads // kv_heads
        # projections of the code rows (compress_forward.py:397-432)
        self.query_residual, self.code_q_heads, self.code_kv_heads = (bool(query_residual), bool(code_q_heads),
                                                                       bool(code_kv_heads))
        self._code_rows = _CodeRows()
        for layer in self.model.model.layers:
            attn = layer.self_attn
            if query_residual:
                attn.q_proj = _QProjQRes(attn.q_proj, self.L * self.K_act, self._code_rows)
            if code_q_heads:
                attn.q_proj = _QProjCode(attn.q_proj, self._code_rows)
            if code_kv_heads:
                attn.k_proj = _QProjCode(attn.k_proj, self._code_rows)
                attn.v_proj = _QProjCode(attn.v_proj, self._code_rows)
        self._set_layout(self.N)
        self.set_head_code_quotas(head_code_quotas)

    def _set_layout(self, N):
        dev = self.pause.device
        C, Ka, L, R = self.C, self.K_act, self.L, self.replay_tail
        blk, role = roles(C, N, Ka, dev, L, R)
        content = role == 0
        pf = torch.tensor([k for k in range(N * C) if k % C != C - 1], device=dev, dtype=torch.long)
        layout = {"blk": blk, "role": role, "content_abs_pos": content_abs_pos(C, N, Ka, dev, L, R),
                  "loss_pos": content & torch.roll(content, -1), "content_pos": content.nonzero(as_tuple=True)[0],
                  "predict_flat": pf, "predict_block": pf // C,
                  "_pos_ids": rope_position_ids(C, N, self.K, Ka, self.code_positions, dev,
                                                self.code_excluded_tail, L, R)}
        for name, value in layout.items():
            self.register_buffer(name, value, persistent=False)
        code = ((role > 0) & (role <= L)).nonzero(as_tuple=True)[0]
        self._code_rows.rows = code
        self._code_rows.slots = code % (C + L * Ka + R) - C
        self._code_rows.S0 = N * (C + L * Ka + R)
        self._code_rows.lengths = (self._code_rows.S0, self._code_rows.S0 + 1 + C)
        self._code_rows._copies = {}

    def set_N(self, N):
        """Rebuild the N-dependent layout for a new block count (compress_forward.py set_N)."""
        self.N = int(N)
        self._set_layout(self.N)

    def set_head_code_quotas(self, head_code_quotas):
        """Fixed per-(layer, KV head) code quotas in [1, K_act] (compress_forward.py:516-575); None clears them."""
        dev = self.pause.device
        if head_code_quotas is None:
            self.register_buffer("head_code_quotas", torch.empty((0, 0), dtype=torch.long, device=dev), False)
            self.register_buffer("query_head_code_quotas", torch.empty((0, 0), dtype=torch.long, device=dev), False)
            self.register_buffer("_head_quota_i32", None, False)
            return
        try:
            raw = torch.as_tensor(head_code_quotas, device=dev)
        except (TypeError, ValueError, RuntimeError) as exc:
            raise ValueError("head_code_quotas must be a rectangular 2D integer array") from exc
        expected = (self.num_layers, self.num_kv_heads)
        if tuple(raw.shape) != expected:
            raise ValueError(f"head_code_quotas must have shape {expected}, got {tuple(raw.shape)}")
        if raw.dtype == torch.bool or (raw.is_floating_point() and bool((raw != raw.round()).any())):
            raise ValueError("head_code_quotas must contain integers")
        physical = raw.to(torch.long)
        if bool(((physical <= 0) | (physical > self.K)).any()):
            raise ValueError(f"head_code_quotas must be in [1, {self.K}]")
        if bool((physical > self.K_act).any()):
            raise ValueError(f"head_code_quotas exceed active_code_rows={self.K_act}")
        expanded = physical.repeat_interleave(self.num_key_value_groups, dim=1)
        self.register_buffer("head_code_quotas", physical, False)
        self.register_buffer("query_head_code_quotas", expanded, False)
        self.register_buffer("_head_quota_i32", expanded.to(torch.int32).contiguous(), False)

    @property
    def has_head_code_quotas(self) -> bool:
        return self.head_code_quotas.numel() > 0

    def compress_mask(self, batch: int, prompt_len: torch.Tensor | None = None, N: int | None = None,
                      copy_rows: int = 0) -> CompressMask:
        N = self.N if N is None else int(N)
        if prompt_len is not None:
            prompt_len = prompt_len.to(device=self.pause.device, dtype=torch.int32).contiguous()
            if prompt_len.numel() != batch:
                raise ValueError("prompt_len must hold one length per sequence")
        # the raw tail is the kernels' "raw" policy: the rolling window, not hidden from the codes
        policy = "raw" if self.raw_tail else self.retain_tail_policy if self.retain_tail_kv else "static"
        return CompressMask(self.C, self.K_act, N, prompt_len, self._head_quota_i32,
                            self.raw_tail or self.retain_tail_kv, policy, self.pause_xattn, self.L,
                            copy_rows, self.replay_tail, self.code_exclude_replay_tail)

    def _lm_ce(self, hid, tgt, chunk):
        if chunk <= 0:
            return F.cross_entropy(self.model.lm_head(hid).float(), tgt)
        tot = hid.new_zeros((), dtype=torch.float32)
        for i in range(0, hid.size(0), chunk):
            tot = tot + F.cross_entropy(self.model.lm_head(hid[i:i + chunk]).float(), tgt[i:i + chunk],
                                        reduction="sum")
        return tot / hid.size(0)

    def _per_token_lm_ce(self, hid, tgt, chunk):
        step = hid.size(0) if chunk <= 0 else chunk
        return torch.cat([F.cross_entropy(self.model.lm_head(hid[i:i + step]).float(), tgt[i:i + step],
                                          reduction="none") for i in range(0, hid.size(0), step)])

    def _masked_lm_ce(self, hid, tgt, mask, chunk):
        den = mask.sum().clamp_min(1.0)
        return (self._per_token_lm_ce(hid, tgt, chunk) * mask).sum() / den

    def _perblock_ce(self, hid, tgt, blk_idx, nblk, reps):
        ce = F.cross_entropy(self.model.lm_head(hid).float(), tgt, reduction="none")
        blk = blk_idx.repeat(reps)
        s = ce.new_zeros(nblk).scatter_add_(0, blk, ce)
        c = ce.new_zeros(nblk).scatter_add_(0, blk, torch.ones_like(ce))
        return ce.mean(), s / c.clamp_min(1.0)

    def _compressed_forward(self, content_ids, prompt_len=None, with_copy=False, mask=None, need_rep=False):
        """The decoder over the compressed layout (compress_forward.py:1146-1229): content embeddings, L passes of
        code seeds per block, then with ``with_copy`` the copy region [copy_token | last block's content]; returns
        the HF model output (``hidden_states`` with ``need_rep``)."""
        B, N, C = content_ids.shape
        if C != self.C:
            raise ValueError(f"content_ids block size {C} != C={self.C}")
        if N != self.N:
            self.set_N(N)
        K, L, R = self.K_act, self.L, self.replay_tail
        emb = self.model.model.embed_tokens
        tok_e = emb(content_ids)
        d = tok_e.size(-1)
        pause_e = code_seeds(self, tok_e).expand(B, N, K, d)
        if L > 1:
            pause_e = pause_e.repeat(1, 1, L, 1)                      # every pass starts from the same seeds
        parts = [tok_e, pause_e] + ([tok_e[:, :, C - R:, :]] if R else [])   # the replay rows: the last R tokens
        x = torch.cat(parts, dim=2).reshape(B, N * (C + L * K + R), d)
        pos = self._pos_ids
        if with_copy:
            copy_in = torch.cat([self.copy_token.to(tok_e.dtype).view(1, 1, d).expand(B, 1, d),
                                 emb(content_ids[:, -1, :])], dim=1)
            x = torch.cat([x, copy_in], dim=1)
            start = N * C if self.code_positions == "bitrev" else N * (C + L * self.K + R)
            pos = torch.cat([pos, start + torch.arange(1 + C, device=pos.device).view(1, -1)], dim=1)
        if torch.is_autocast_enabled(x.device.type):
            x = x.to(torch.get_autocast_dtype(x.device.type))
        if mask is None:
            mask = self.compress_mask(B, prompt_len, N, copy_rows=1 + C if with_copy else 0)
        return self.model.model(inputs_embeds=x, attention_mask={"full_attention": mask}, position_ids=pos,
                                use_cache=False, output_hidden_states=need_rep)

    def hidden_states(self, content_ids, prompt_len=None):
        """Final-normed hidden states [B, S0, d] of the compressed teacher-forced layout."""
        return self._compressed_forward(content_ids, prompt_len).last_hidden_state

    def _embed_for_plain_forward(self, ids):
        """Token embeddings for a plain (uncompressed) forward, in the active autocast dtype (compress_forward.py:
        940-950)."""
        e = self.model.model.embed_tokens(ids)
        if torch.is_autocast_enabled(e.device.type):
            e = e.to(torch.get_autocast_dtype(e.device.type))
        return e

    @torch.no_grad()
    def full_ctx_logits(self, content_ids):
        """Logits of the plain causal forward over all N * C content tokens (the full-context teacher,
        compress_forward.py:952-956); the attention runs the masked-prefill kernel without code rows."""
        B, N, C = content_ids.shape
        return self.model(inputs_embeds=self._embed_for_plain_forward(content_ids.reshape(B, N * C)),
                          use_cache=False).logits

    def baseline_loss(self, content_ids, ce_chunk=0, ctx_blocks=0, block_ce=False, resp_mask=None, per_token=False,
                      include_cross_block=False):
        """Plain causal LM without compression on the same predict positions (compress_forward.py:1095-1132):
        sequences of ``ctx_blocks`` contiguous blocks (0: all N, the full-context ceiling; 1: the floor)."""
        B, N, C = content_ids.shape
        G = ctx_blocks if ctx_blocks else N
        if N % G:
            raise ValueError(f"ctx_blocks={G} must divide N={N}")
        flat = content_ids.reshape(B * (N // G), G * C)
        out = self.model.model(inputs_embeds=self._embed_for_plain_forward(flat), use_cache=False).last_hidden_state
        ar = torch.arange(G * C, device=flat.device)
        pos = ar[:-1] if include_cross_block else ar[(ar % C) != (C - 1)]
        hid = out[:, pos, :].reshape(-1, out.size(-1))
        tgt = flat[:, pos + 1].reshape(-1)
        if block_ce:
            m, bc = self._perblock_ce(hid, tgt, pos // C, G, flat.size(0))
            return {"ce": m, "block_ce": bc}
        if resp_mask is not None:
            rm = resp_mask.reshape(flat.shape)[:, pos + 1].reshape(-1).float()
            if per_token:
                ce = self._per_token_lm_ce(hid, tgt, ce_chunk)
                reps = flat.size(0)
                if include_cross_block:
                    target = pos + 1
                    return {"ce_pt": ce, "tmask": rm, "blk": (target // C).repeat(reps),
                            "pos": (target % C).repeat(reps), "supervised": ((pos % C) != C - 1).repeat(reps)}
                return {"ce_pt": ce, "tmask": rm, "blk": (pos // C).repeat(reps), "pos": (pos % C).repeat(reps)}
            return {"ce": self._masked_lm_ce(hid, tgt, rm, ce_chunk)}
        return {"ce": self._lm_ce(hid, tgt, ce_chunk)}

    def _masked_ce_kl_chunked(self, hid, tgt, mask, teacher_rows, teacher_head, temp, chunk):
        """Response-masked CE and KL(teacher || student) at temperature ``temp`` from a frozen teacher's final
        hidden rows, chunked over rows with activation checkpointing (compress_forward.py:978-1020)."""
        import torch.utils.checkpoint as ckpt
        if teacher_rows.shape[0] != hid.shape[0]:
            raise ValueError(f"teacher_rows {tuple(teacher_rows.shape)} misaligned with student rows "
                             f"{tuple(hid.shape)}")
        den = mask.sum().clamp_min(1.0)
        T = float(temp)
        lm_head = self.model.lm_head

        def part(h, t, m, tr):
            logits = lm_head(h).float()
            ce = F.cross_entropy(logits, t, reduction="none")
            with torch.no_grad():
                tl = teacher_head(tr).float()
                tp, tlp = F.softmax(tl / T, -1), F.log_softmax(tl / T, -1)
            kl = (tp * (tlp - F.log_softmax(logits / T, -1))).sum(-1) * (T * T)
            return (ce * m).sum(), (kl * m).sum()

        step = hid.size(0) if chunk <= 0 else chunk
        ce_tot = hid.new_zeros((), dtype=torch.float32)
        kl_tot = hid.new_zeros((), dtype=torch.float32)
        for i in range(0, hid.size(0), step):
            sl = slice(i, i + step)
            args = (hid[sl], tgt[sl], mask[sl], teacher_rows[sl])
            c, k = ckpt.checkpoint(part, *args, use_reentrant=False) if torch.is_grad_enabled() else part(*args)
            ce_tot, kl_tot = ce_tot + c, kl_tot + k
        return ce_tot / den, kl_tot / den

    def forward(self, content_ids, distill_lambda=0.0, copy_lambda=0.0, distill_temp=1.0, ce_chunk=0, baseline=False,
                ctx_blocks=0, teacher_logits=None, teacher_hidden=None, block_ce=False, resp_mask=None,
                raw_prompt=False, blockmask=None, per_token=False, include_cross_block=False,
                boundary_recovery_width=0, boundary_recovery_weight=1.0, teacher_rows=None, teacher_head=None):
        """Losses of the compressed teacher-forced forward, same signature, control flow and return dicts as
        compress_forward.py:1134-1315: the full-context baseline, CE (masked by ``resp_mask``, per block, per
        token), self- or teacher distillation (KL at ``distill_temp``), the chunked frozen-teacher KD
        (``teacher_rows`` / ``teacher_head``), the copy loss (``copy_lambda``: the copy region reproduces the last
        block from its codes) and the representation loss (``teacher_hidden``). ``blockmask``: a prebuilt
        :class:`CompressMask` (the analogue of the reference's prebuilt BlockMask)."""
        if baseline:
            return self.baseline_loss(content_ids, ce_chunk, ctx_blocks, block_ce=block_ce, resp_mask=resp_mask,
                                      per_token=per_token, include_cross_block=include_cross_block)
        B, N, C = content_ids.shape
        dev = content_ids.device
        with_copy = copy_lambda > 0
        need_rep = teacher_hidden is not None
        prompt_len, mask = None, None
        if blockmask is not None:
            if self.has_head_code_quotas:
                raise ValueError("an external blockmask cannot encode layer/head quotas; "
                                 "omit blockmask when head_code_quotas are enabled")
            if not isinstance(blockmask, CompressMask):
                raise TypeError(f"blockmask must be a CompressMask, got {type(blockmask).__name__}")
            mask = blockmask
        elif raw_prompt and resp_mask is not None and not with_copy:
            rmf = resp_mask.reshape(B, N * C)
            prompt_len = (rmf.cumsum(1) == 0).sum(1).to(torch.int32)      # leading zeros = prompt length
        mo = self._compressed_forward(content_ids, prompt_len, with_copy, mask, need_rep)
        out = mo.last_hidden_state
        d = out.size(-1)
        S0 = N * (C + self.L * self.K_act + self.replay_tail)
        if include_cross_block:
            pred_flat = torch.arange(N * C - 1, device=dev)
            hid = out[:, :S0, :][:, self.content_pos, :][:, :-1, :].reshape(-1, d)
        else:
            pred_flat = self.predict_flat
            hid = out[:, :S0, :][:, self.loss_pos, :].reshape(-1, d)
        tgt = content_ids.reshape(B, N * C)[:, pred_flat + 1].reshape(-1)
        if block_ce:
            m, bc = self._perblock_ce(hid, tgt, pred_flat // C, N, B)
            return {"ce": m, "block_ce": bc}
        if resp_mask is not None:
            tmask = resp_mask.reshape(B, N * C)[:, pred_flat + 1].reshape(-1).float()
            target = pred_flat + 1
            if per_token and include_cross_block:
                return {"ce_pt": self._per_token_lm_ce(hid, tgt, ce_chunk), "tmask": tmask,
                        "blk": (target // C).repeat(B), "pos": (target % C).repeat(B),
                        "supervised": ((pred_flat % C) != C - 1).repeat(B)}
            if boundary_recovery_width > 0 and boundary_recovery_weight != 1.0:
                recovery = ((target // C > 0) & (target % C >= 1) & (target % C <= boundary_recovery_width)).repeat(B)
                tmask = tmask * torch.where(recovery, tmask.new_tensor(boundary_recovery_weight),
                                            tmask.new_tensor(1.0))
            if teacher_rows is not None and not per_token:
                ce, kl = self._masked_ce_kl_chunked(hid, tgt, tmask, teacher_rows, teacher_head, distill_temp, ce_chunk)
                return {"ce": ce, "distill": kl}
            if not per_token and teacher_logits is None:
                return {"ce": self._masked_lm_ce(hid, tgt, tmask, ce_chunk)}
            logits = self.model.lm_head(hid).float()
            ce = F.cross_entropy(logits, tgt, reduction="none")
            if per_token:
                return {"ce_pt": ce, "tmask": tmask, "blk": self.predict_block.repeat(B),
                        "pos": (self.predict_flat % C).repeat(B)}
            den = tmask.sum().clamp_min(1.0)
            outd = {"ce": (ce * tmask).sum() / den}
            if teacher_logits is not None:
                T = distill_temp
                kl = F.kl_div(F.log_softmax(logits / T, -1), F.softmax(teacher_logits.float() / T, -1),
                              reduction="none").sum(-1) * (T * T)
                outd["distill"] = (kl * tmask).sum() / den
            return outd
        if distill_lambda > 0:
            logits = self.model.lm_head(hid).float()
            losses = {"ce": F.cross_entropy(logits, tgt)}
            if teacher_logits is None:                                     # self-teacher: the full-context forward
                with torch.no_grad():
                    teacher_logits = self.full_ctx_logits(content_ids)[:, pred_flat, :].reshape(-1, logits.size(-1))
            T = distill_temp
            losses["distill"] = F.kl_div(F.log_softmax(logits / T, -1), F.softmax(teacher_logits.float() / T, -1),
                                         reduction="batchmean") * (T * T)
        else:
            losses = {"ce": self._lm_ce(hid, tgt, ce_chunk)}
        if with_copy:
            losses["copy"] = self._lm_ce(out[:, S0:S0 + C, :].reshape(-1, d), content_ids[:, -1, :].reshape(-1),
                                         ce_chunk)
        if need_rep:
            rep = out.new_zeros((), dtype=torch.float32)
            for li in range(teacher_hidden.shape[0]):
                hs = mo.hidden_states[li + 1][:, self.content_pos, :].float()
                ht = teacher_hidden[li].float()
                hs = hs / hs.pow(2).mean(-1, keepdim=True).clamp_min(1e-12).sqrt()
                ht = ht / ht.pow(2).mean(-1, keepdim=True).clamp_min(1e-12).sqrt()
                rep = rep + (hs - ht).pow(2).mean()
            losses["rep"] = rep / teacher_hidden.shape[0]
        return losses

    @torch.no_grad()
    def loss_logits(self, content_ids, prompt_len=None):
        """fp32 logits at the loss positions (block-major, within-block 0..C-2), as the reference's gate compares."""
        out = self.hidden_states(content_ids, prompt_len)
        hid = out[:, self.loss_pos, :].reshape(-1, out.size(-1))
        return self.model.lm_head(hid).float()
