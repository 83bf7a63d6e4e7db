"""Teacher-forced CompressLM forward with materialised dense masks (oracle; test infrastructure only).

Restates abridgekv/gen_compress.py:1143-1182 (``_dense_ref_logits``): the compressed layout [C content | K codes]
per block with the code rows seeded by ``pause``, RoPE positions of compress_forward.py:1044-1071, and for every
decoder layer manual attention under the dense boolean mask of ``oracle.prefill.arith_mask`` (the reference's
``_dense_mask`` / ``_arith_mask_mod``), with the per-layer query-head quota of compress_forward.py:230-236. Runs the
HuggingFace layer modules of ``model`` in whatever dtype the model is in (float64 on the CPU for a tight bound).

With a retained tail of T rows the mask is ``arith_mask(..., retain_tail=T, tail_policy=...)`` and the bitrev code
rows spread over the first C - T in-block offsets (compress_forward.py:1059).

Pinning: tests/test_oracle_model.py checks that with one block the content logits equal the model's own causal
forward (code rows come after the content and are invisible to it), that all-K quotas equal no quotas, and that
``rope_positions`` matches the closed-form bitrev / appended layout (with and without a code span).
"""
from __future__ import annotations

import numpy as np
import torch
import torch.nn.functional as F

from . import layout as ol
from . import prefill as op


def rope_positions(C, N, K, code_positions, span=None):
    """RoPE position of every row of the full-K layout (compress_forward.py:1044-1071, L=1, no replay tail); bitrev
    code rows spread over in-block offsets [0, span) (span None: C)."""
    pos = np.zeros(N * (C + K), dtype=np.int64)
    offs = ol.bitrev_code_offsets(K, C, span) if code_positions == "bitrev" else None
    for b in range(N):
        for j in range(C + K):
            if code_positions == "bitrev":
                pos[b * (C + K) + j] = b * C + (j if j < C else int(offs[j - C]))
            else:
                pos[b * (C + K) + j] = b * (C + K) + j
    return pos


def loss_rows(C, N, K):
    """Rows whose hidden state predicts the next content token of the same block (content j = 0..C-2)."""
    return np.array([b * (C + K) + j for b in range(N) for j in range(C - 1)], dtype=np.int64)


def _rotate_half(x):
    h = x.shape[-1] // 2
    return torch.cat((-x[..., h:], x[..., :h]), dim=-1)


def dense_hidden(model, pause, content_ids, C, N, K, code_positions="appended", prompt_len=None,
                 layer_head_quota=None, retain_tail=0, tail_policy="static", pause_xattn="full"):
    """Final-normed hidden states [B, S0, d]. ``layer_head_quota``: [layers, Hq] code rows visible per query head
    (None: all K); ``prompt_len``: [B] raw-prompt content tokens (None: no raw prompt); ``retain_tail``: T of a
    retained tail under ``tail_policy``; ``pause_xattn``: code rows' attention to their own block's codes."""
    inner = model.model
    B = content_ids.shape[0]
    dt = next(model.parameters()).dtype
    tok_e = inner.embed_tokens(content_ids)
    d = tok_e.shape[-1]
    x = torch.cat([tok_e, pause.to(dt).view(1, 1, K, d).expand(B, N, K, d)], dim=2).reshape(B, N * (C + K), d)
    S0 = x.shape[1]
    pos = torch.from_numpy(rope_positions(C, N, K, code_positions, C - retain_tail)).view(1, -1)
    cos, sin = inner.rotary_emb(x, pos)
    cos, sin = cos.unsqueeze(1), sin.unsqueeze(1)
    pl = None if prompt_len is None else np.asarray(prompt_len, dtype=np.int64)
    h = x
    for li, layer in enumerate(inner.layers):
        attn = layer.self_attn
        hq = None if layer_head_quota is None else np.asarray(layer_head_quota[li], dtype=np.int64)
        vis = op.arith_mask(C, K, N, pl, hq, retain_tail, tail_policy, pause_xattn)     # [B?, H?, S0, S0]
        vis = torch.from_numpy(np.ascontiguousarray(vis))
        if pl is None:
            vis = vis.unsqueeze(0)                              # [1, H?, S0, S0]
        if hq is None:
            vis = vis.unsqueeze(1)                              # [B?, 1, S0, S0]
        add = torch.zeros(vis.shape, dtype=dt).masked_fill(~vis, torch.finfo(dt).min)
        normed = layer.input_layernorm(h)
        hs = (B, S0, -1, attn.head_dim)
        q = attn.q_proj(normed).view(hs)
        k = attn.k_proj(normed).view(hs)
        if getattr(attn, "q_norm", None) is not None:
            q = attn.q_norm(q)
        if getattr(attn, "k_norm", None) is not None:
            k = attn.k_norm(k)
        q, k = q.transpose(1, 2), k.transpose(1, 2)
        v = attn.v_proj(normed).view(hs).transpose(1, 2)
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
    return inner.norm(h)


def dense_loss_logits(model, pause, content_ids, C, N, K, code_positions="appended", prompt_len=None,
                      layer_head_quota=None, retain_tail=0, tail_policy="static", pause_xattn="full"):
    """Logits [B * N * (C-1), V] at the loss rows (block-major, within-block 0..C-2)."""
    h = dense_hidden(model, pause, content_ids, C, N, K, code_positions, prompt_len, layer_head_quota, retain_tail,
                     tail_policy, pause_xattn)
    rows = torch.from_numpy(loss_rows(C, N, K))
    return model.lm_head(h[:, rows, :].reshape(-1, h.shape[-1])).double()
