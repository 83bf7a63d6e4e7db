"""Teacher-forced CompressLM forward with materialised dense masks (oracle; test infrastructure only).

Restates abridgekv/gen_compress.py:1143-1182 (``_dense_ref_logits``): the compressed layout [C content | K codes]
per block with the code rows seeded by ``pause``, RoPE positions of compress_forward.py:1044-1071, and for every
decoder layer manual attention under the dense boolean mask of ``oracle.prefill.arith_mask`` (the reference's
``_dense_mask`` / ``_arith_mask_mod``), with the per-layer query-head quota of compress_forward.py:230-236. Runs the
HuggingFace layer modules of ``model`` in whatever dtype the model is in (float64 on the CPU for a tight bound).

With a retained tail of T rows the mask is ``arith_mask(..., retain_tail=T, tail_policy=...)`` and the bitrev code
rows spread over the first C - T in-block offsets (compress_forward.py:1059).

With L = ``passes`` pause passes every block is [C content | L passes of K code rows], each pass fed the same seeds
(compress_forward.py:1179, ``pause_base.repeat(1, 1, L, 1)``), appended positions. ``seeds`` replaces the generic
seeds by per-block code inputs (:func:`code_seeds`, the pools of compress_forward.py:1147-1178); ``code_proj``
gives per layer the code rows' own projections (compress_forward.py:181-222): a query residual per code slot
("qres"), or separate (weight, bias) for q / k / v at the code rows.

Pinning: tests/test_oracle_model.py checks that with one block the content logits equal the model's own causal
forward (code rows come after the content and are invisible to it, whatever their seeds, passes and projections),
that all-K quotas equal no quotas, that zero residuals and copied projections change nothing while a changed code
projection moves the later blocks' logits only, and that ``rope_positions`` matches the closed-form bitrev /
appended layout (with and without a code span, with passes); :func:`code_seeds` against explicit segment sums, the
block-mean fallback, a zero value map and a one-hot pooling.
"""
from __future__ import annotations

import numpy as np
import torch
import torch.nn.functional as F

from . import layout as ol
from . import prefill as op


def rope_positions(C, N, K, code_positions, span=None, passes=1, replay=0):
    """RoPE position of every row of the full-K layout (compress_forward.py:1044-1071); bitrev code rows (one pass,
    no replay rows) spread over in-block offsets [0, span) (span None: C); appended rows keep their index."""
    per = C + passes * K + replay
    pos = np.zeros(N * per, dtype=np.int64)
    offs = ol.bitrev_code_offsets(K, C, span) if code_positions == "bitrev" else None
    for b in range(N):
        for j in range(per):
            if code_positions == "bitrev":
                pos[b * per + j] = b * C + (j if j < C else int(offs[j - C]))
            else:
                pos[b * per + j] = b * per + j
    return pos


def loss_rows(C, N, K, passes=1, replay=0):
    """Rows whose hidden state predicts the next content token of the same block (content j = 0..C-2)."""
    per = C + passes * K + replay
    return np.array([b * per + j for b in range(N) for j in range(C - 1)], dtype=np.int64)


def code_seeds(tok_e, pause, K, excluded_tail=0, segment_mean=False, seg_gate=None, pool=None):
    """Code-row inputs [B, N, K, d] of blocks with content embeddings tok_e [B, N, C, d] (compress_forward.py:
    1147-1178): ``pause`` [K, d] plus, with ``segment_mean`` (seg_pool), the mean of segment k of the first
    C - excluded_tail content rows split into K runs of (C - T) // K (the block mean when that is 0), times
    ``seg_gate`` [K] when given (gated_seg_pool); with ``pool`` = (pool_q [K, d], W_k [d, d], W_v [d, d])
    (pool_init) the softmax over the content of pool_q[k] . (W_k x) / sqrt(d) weighting W_v x. Loops, float64."""
    tok_e = torch.as_tensor(tok_e, dtype=torch.float64)
    pause = torch.as_tensor(pause, dtype=torch.float64)
    B, N, C, d = tok_e.shape
    n = C - excluded_tail
    out = torch.zeros(B, N, K, d, dtype=torch.float64)
    for b in range(B):
        for blk in range(N):
            rows = tok_e[b, blk, :n]
            for k in range(K):
                extra = torch.zeros(d, dtype=torch.float64)
                if segment_mean:
                    seg = n // K
                    part = rows[k * seg:(k + 1) * seg] if seg >= 1 else rows
                    extra = sum(part[i] for i in range(part.shape[0])) / part.shape[0]
                    if seg_gate is not None:
                        extra = extra * torch.as_tensor(seg_gate, dtype=torch.float64)[k]
                elif pool is not None:
                    pq, wk, wv = (torch.as_tensor(t, dtype=torch.float64) for t in pool)
                    scores = [pq[k] @ (wk @ rows[i]) / d ** 0.5 for i in range(n)]
                    top = max(float(x) for x in scores)
                    w = [torch.exp(x - top) for x in scores]
                    z = sum(w)
                    extra = sum((w[i] / z) * (wv @ rows[i]) for i in range(n))
                out[b, blk, k] = pause[k] + extra
    return out


def _rotate_half(x):
    h = x.shape[-1] // 2
    return torch.cat((-x[..., h:], x[..., :h]), dim=-1)


def dense_hidden(model, pause, content_ids, C, N, K, code_positions="appended", prompt_len=None,
                 layer_head_quota=None, retain_tail=0, tail_policy="static", pause_xattn="full", passes=1,
                 seeds=None, code_proj=None, copy_token=None, output_layers=False, replay=0, replay_exclude=False,
                 raw_tail=0):
    """Final-normed hidden states [B, S, d]. ``layer_head_quota``: [layers, Hq] code rows visible per query head
    (None: all K); ``prompt_len``: [B] raw-prompt content tokens (None: no raw prompt); ``retain_tail``: T of a
    retained tail under ``tail_policy``; ``pause_xattn``: code rows' attention to their own pass's codes;
    ``passes``: pause passes per block; ``seeds`` [B, N, K, d] code inputs (None: ``pause``); ``code_proj``: per
    layer a dict of the code rows' projections ("qres" [passes * K, dq]; "q" / "k" / "v": (weight, bias or None));
    ``copy_token`` [d]: append the copy region [copy_token | last block's content] (compress_forward.py:1185-1189),
    at positions after the layout's; ``output_layers``: also return every layer's output hidden states;
    ``replay``: R replay rows after each block's codes, fed the block's last R content tokens (compress_forward.py:
    1180-1183), ``replay_exclude`` hiding those content rows from the codes; ``raw_tail``: W of a raw tail (the next
    block's content rows see the block's last rows in a rolling window; the codes see their whole block)."""
    inner = model.model
    B = content_ids.shape[0]
    dt = next(model.parameters()).dtype
    tok_e = inner.embed_tokens(content_ids)
    d = tok_e.shape[-1]
    L = int(passes)
    R = int(replay)
    per = C + L * K + R
    code_in = pause.to(dt).view(1, 1, K, d).expand(B, N, K, d) if seeds is None else seeds.to(dt)
    x = torch.cat([tok_e] + [code_in] * L + ([tok_e[:, :, C - R:]] if R else []), dim=2).reshape(B, N * per, d)
    S0 = x.shape[1]
    code_rows = torch.from_numpy(np.array([r for r in range(S0) if C <= r % per < C + L * K], dtype=np.int64))
    slots = code_rows % per - C
    span = C - (R if replay_exclude else retain_tail)
    pos = torch.from_numpy(rope_positions(C, N, K, code_positions, span, L, R)).view(1, -1)
    copy = 0
    if copy_token is not None:
        copy = 1 + C
        x = torch.cat([x, copy_token.to(dt).view(1, 1, d).expand(B, 1, d), tok_e[:, -1]], dim=1)
        start = N * C if code_positions == "bitrev" else S0
        pos = torch.cat([pos, start + torch.arange(copy).view(1, -1)], dim=1)
        S0 = x.shape[1]
    cos, sin = inner.rotary_emb(x, pos)
    cos, sin = cos.unsqueeze(1), sin.unsqueeze(1)
    pl = None if prompt_len is None else np.asarray(prompt_len, dtype=np.int64)
    h = x
    layers_out = []
    for li, layer in enumerate(inner.layers):
        attn = layer.self_attn
        hq = None if layer_head_quota is None else np.asarray(layer_head_quota[li], dtype=np.int64)
        vis = op.arith_mask(C, K, N, pl, hq, retain_tail, tail_policy, pause_xattn, L, copy, R,
                            replay_exclude, raw_tail)                                                   # [B?, H?, S, S]
        vis = torch.from_numpy(np.ascontiguousarray(vis))
        if pl is None:
            vis = vis.unsqueeze(0)                              # [1, H?, S0, S0]
        if hq is None:
            vis = vis.unsqueeze(1)                              # [B?, 1, S0, S0]
        add = torch.zeros(vis.shape, dtype=dt).masked_fill(~vis, torch.finfo(dt).min)
        normed = layer.input_layernorm(h)
        hs = (B, S0, -1, attn.head_dim)
        cp = {} if code_proj is None else code_proj[li]

        def project(base, name):
            out = base(normed)
            if name in cp:                                      # the code rows' own (weight, bias)
                w, bias = cp[name]
                out[:, code_rows] = F.linear(normed[:, code_rows], w.to(dt), None if bias is None else bias.to(dt))
            if name == "q" and "qres" in cp:                    # plus the residual of the row's slot
                out[:, code_rows] = out[:, code_rows] + cp["qres"].to(dt)[slots]
            return out

        q = project(attn.q_proj, "q").view(hs)
        k = project(attn.k_proj, "k").view(hs)
        if getattr(attn, "q_norm", None) is not None:
            q = attn.q_norm(q)
        if getattr(attn, "k_norm", None) is not None:
            k = attn.k_norm(k)
        q, k = q.transpose(1, 2), k.transpose(1, 2)
        v = project(attn.v_proj, "v").view(hs).transpose(1, 2)
        q = q * cos + _rotate_half(q) * sin
        k = k * cos + _rotate_half(k) * sin
        rep = q.shape[1] // k.shape[1]
        kr = k.repeat_interleave(rep, dim=1)
        vr = v.repeat_interleave(rep, dim=1)
        w = torch.matmul(q, kr.transpose(2, 3).contiguous()) * attn.scaling + add
        w = F.softmax(w, dim=-1, dtype=torch.float32 if dt != torch.float64 else torch.float64).to(dt)
        o = torch.matmul(w, vr).transpose(1, 2).reshape(B, S0, -1)
        h = h + attn.o_proj(o)
        h = h + layer.mlp(layer.post_attention_layernorm(h))
        layers_out.append(h)
    return (inner.norm(h), layers_out) if output_layers else inner.norm(h)


def dense_loss_logits(model, pause, content_ids, C, N, K, code_positions="appended", prompt_len=None,
                      layer_head_quota=None, retain_tail=0, tail_policy="static", pause_xattn="full", passes=1,
                      seeds=None, code_proj=None, replay=0, replay_exclude=False, raw_tail=0):
    """Logits [B * N * (C-1), V] at the loss rows (block-major, within-block 0..C-2)."""
    h = dense_hidden(model, pause, content_ids, C, N, K, code_positions, prompt_len, layer_head_quota, retain_tail,
                     tail_policy, pause_xattn, passes, seeds, code_proj, replay=replay, replay_exclude=replay_exclude,
                     raw_tail=raw_tail)
    rows = torch.from_numpy(loss_rows(C, N, K, passes, replay))
    return model.lm_head(h[:, rows, :].reshape(-1, h.shape[-1])).double()
