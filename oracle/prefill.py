"""Teacher-forced attention under the compression mask (oracle; test infrastructure only).

Layout of one sequence: N blocks of [C content | K codes] (S0 = N * (C + K)), content tokens numbered block-major.
Visibility (L=1, full code<->code attention, no replay / raw / retained tails, raw prompt of ``prompt_len`` content
tokens, optional per-query-head code quota):
  causal & (own-block content | earlier blocks' codes | raw-prompt content)  |  (code query & code key & same block)
  and, with a quota, a code key is visible to head h only if its slot < quota[h].

With L = ``passes`` > 1 pause passes a block is [C content | L passes of K code rows] (per = C + L K,
compress_forward.py:20-31): pass l >= 1 reads its block's content and its pass l - 1 ("refine"), its own pass by
``pause_xattn``, and later blocks read only the final pass L ("earlier_final", compress_forward.py:594-600); the
quota counts a code row's slot within its pass ((within - C) % K, :576-577).

``replay`` = R rows after a block's codes replay its last R content tokens (replay_tail, compress_forward.py:20-31,
139-178, 594-603): a replay row sees its block's content, final-pass codes and replay rows (causally) besides what
every row sees, and content row i of the next block sees the previous block's replay rows from row i on (a rolling
window, _replay_tail_visible); with ``replay_exclude`` (code_exclude_replay_tail) a block's codes do not see its last
R content rows. Replay and retained tails are mutually exclusive.

``raw_tail`` = W (CompressLM(raw_tail=W), compress_forward.py:89-96, _raw_tail_visible): content query i of block b
sees content row j of block b - 1 iff (b C + i) - ((b - 1) C + j) <= W; unlike a retained tail the codes still see
their whole block (code_excluded_tail = retain_tail_kv = 0, :309-311). Exclusive with replay and retained tails.

``copy_rows`` rows after the N blocks form the copy region (copy_lambda, compress_forward.py:631-633): a copy row
sees the last block's final-pass codes (slot < quota) and the copy rows up to itself; no other row sees it. K = 0
(no codes) leaves causal attention within blocks of C rows (the plain forward).

With a retained tail of T rows (retain_tail_kv = T) a block's codes never see its own last T content rows, and the
last T content rows of an earlier block are visible, by ``tail_policy``
(abridgekv/compress_forward.py:99-124, _retained_tail_visible):
  "static"  -- to every later query (content and codes);
  "sticky"  -- to the content queries of the next block only;
  "rolling" -- to the content queries of the next block through a sliding window: content query i of block b sees
               row j of block b - 1 iff (b C + i) - ((b - 1) C + j) <= T, i.e. j >= C - T + i.

Code rows attend their own block's code rows by ``pause_xattn`` (compress_forward.py:622-625, 871-874,
gen_compress.py:1121-1123): "full" all of them (bidirectional, the served setting), "causal" those at or before their own position,
"none" none (not even themselves).

Two independent restatements of the reference are kept and cross-checked:
* ``arith_mask``  -- closed-form integer arithmetic: abridgekv/compress_forward.py:695-727 (_arith_mask_mod) with
                     the quota term of :725-726 and the static-tail terms of :714-715, :721-722; the window policies
                     (which the reference sends to its gather-based _mask_mod, :566-649) as the same integer terms.
* ``role_mask``   -- role/block/content-position gathers: abridgekv/gen_compress.py:1062-1140 (_dense_mask, the
                     reference's own dense oracle) restricted to L=1, no replay / raw tail, with its
                     ``retained_tail`` term for the three policies (:1088-1112) and the own-tail exclusion of
                     compress_forward.py:139-155 (_code_content_tail_excluded), plus the quota rule of
                     abridgekv/compress_forward.py:230-236 (_quota_key_allowed).
Pinning: the two agree element by element on every tested shape; brute-force per-element predicates written from
the prose rule (tests/test_oracle_prefill.py); N=1 without codes reduces to the causal mask; masked_attention_fp64
reduces to textbook causal attention under the causal mask and to per-row softmax identities (rows sum to one,
single visible key -> that key's value).
"""
from __future__ import annotations

import numpy as np


TAIL_POLICIES = ("static", "rolling", "sticky")


XATTN = ("full", "causal", "none")


def arith_mask(C, K, N, prompt_len=None, head_quota=None, retain_tail=0, tail_policy="static", pause_xattn="full",
               passes=1, copy_rows=0, replay=0, replay_exclude=False, raw_tail=0):
    """Boolean visibility [B?, H?, S, S] (leading dims only when prompt_len / head_quota are given),
    S = N * (C + passes * K + replay) + copy_rows."""
    S = N * (C + passes * K + replay) + copy_rows
    return arith_mask_block(C, K, N, np.arange(S), np.arange(S), prompt_len, head_quota, retain_tail, tail_policy,
                            pause_xattn, passes, copy_rows, replay, replay_exclude, raw_tail)


def arith_mask_block(C, K, N, rows, cols, prompt_len=None, head_quota=None, retain_tail=0, tail_policy="static",
                     pause_xattn="full", passes=1, copy_rows=0, replay=0, replay_exclude=False, raw_tail=0):
    """The rows x cols sub-block of :func:`arith_mask` ([B?, H?, len(rows), len(cols)]) without building the whole
    S0 x S0 mask: the sampled-row / sampled-key checks at full sequence lengths use it."""
    L, R, W = int(passes), int(replay), int(raw_tail)
    if sum(bool(x) for x in (R, retain_tail, W)) > 1:
        raise ValueError("raw, replay and retained tails are mutually exclusive")
    LK = L * K
    per = C + LK + R
    q = np.asarray(rows, dtype=np.int64).reshape(-1, 1)
    kv = np.asarray(cols, dtype=np.int64).reshape(1, -1)
    qb, kb = q // per, kv // per
    qw, kw = q - qb * per, kv - kb * per
    k_content = kw < C
    k_code = (kw >= C) & (kw < C + LK)
    q_code = (qw >= C) & (qw < C + LK)
    same_blk = kb == qb
    Kd = max(K, 1)
    kp = np.where(k_code, (kw - C) // Kd + 1, 0)                           # pause pass of a code key (1..L)
    qp = np.where(q_code, (qw - C) // Kd + 1, 0)
    T = int(retain_tail)
    if tail_policy not in TAIL_POLICIES:
        raise ValueError(f"unknown tail policy {tail_policy!r}")
    vis = (k_content & same_blk) | (k_code & (kp == L) & (kb < qb))
    if R:
        q_rep, k_rep = qw >= C + LK, kw >= C + LK
        vis = vis | (q_rep & k_code & (kp == L) & same_blk)                # a replay row: its block's final codes
        vis = vis | (q_rep & k_rep & same_blk)                              # ... and replay rows (causal below)
        vis = vis | ((qw < C) & k_rep & (kb + 1 == qb) & (kw - C - LK >= qw))   # rolling window of the next block
    if T and tail_policy == "static":
        vis = vis | (k_content & (kb < qb) & (kw >= C - T))                 # earlier blocks' static tails
    elif T:
        nxt = (qw < C) & k_content & (kb + 1 == qb)                         # next block's content queries
        if tail_policy == "sticky":
            vis = vis | (nxt & (kw >= C - T))
        else:
            vis = vis | (nxt & (C + qw - kw <= T))                          # sliding window
    if W:
        vis = vis | ((qw < C) & k_content & (kb + 1 == qb) & (C + qw - kw <= W))   # raw tail, the codes' too
    if prompt_len is not None:
        pl = np.asarray(prompt_len, dtype=np.int64).reshape(-1, 1, 1)
        vis = vis[None] | (k_content & (kb * C + kw < pl))[...]
    vis = (kv <= q) & vis
    if pause_xattn not in XATTN:
        raise ValueError(f"unknown pause_xattn {pause_xattn!r}")
    own = q_code & k_code & same_blk                                        # code query, code key, same block
    if L > 1:
        vis = vis | (own & (kp == qp - 1))                                  # pass l reads pass l - 1
    if pause_xattn != "none":                                               # code <-> code, same pass
        vis = vis | (own & (kp == qp) & ((kv <= q) if pause_xattn == "causal" else True))
    X = R if (R and replay_exclude) else T
    if X:
        vis = vis & ~(q_code & same_blk & k_content & (kw >= C - X))       # codes never see their own tail
    if head_quota is not None:
        hq = np.asarray(head_quota, dtype=np.int64).reshape(-1, 1, 1)
        quota_ok = ~k_code | ((kw - C) % Kd < hq)                 # [H, 1, S0]: the slot within its pass
        if vis.ndim == 3:
            vis = vis[:, None] & quota_ok[None]
        else:
            vis = vis[None] & quota_ok
    if copy_rows:
        S0 = N * per
        q_copy, k_copy = q >= S0, kv >= S0
        lo = S0 - per + C + (L - 1) * K                                     # the last block's final pass
        final = (kv >= lo) & (kv < lo + K)
        if head_quota is not None:
            final = final[None] & (kv - lo < hq)                            # [H, R, S]
        vis = np.where(q_copy, (k_copy & (kv <= q)) | final, vis & ~k_copy)
    return vis


def role_mask(C, K, N, prompt_len=None, head_quota=None, retain_tail=0, tail_policy="static", pause_xattn="full",
              passes=1, copy_rows=0, replay=0, replay_exclude=False, raw_tail=0):
    """Same visibility from per-position role / block / content-position tables (the _dense_mask form, with its
    replay terms and _mask_mod's raw-tail term, compress_forward.py:601-603); the copy region as _mask_mod's ``copy``
    term (compress_forward.py:627-633)."""
    L, R, W = int(passes), int(replay), int(raw_tail)
    per = C + L * K + R
    S0 = N * per
    idx = np.arange(S0)
    within, blk = idx % per, idx // per
    # 0 content, 1..L pause pass, L + 1 replay (_roles)
    role = np.where(within < C, 0, np.where(within < C + L * K, (within - C) // max(K, 1) + 1, L + 1))
    # content_abs of a replay row: the content position it replays (_content_abs_pos)
    content_abs = np.where(role == 0, blk * C + within,
                           np.where(role == L + 1, blk * C + (C - R) + (within - C - L * K), -1))
    code_slot = np.where((role > 0) & (role <= L), (within - C) % max(K, 1), -1)
    qr, kr = role.reshape(S0, 1), role.reshape(1, S0)
    qb, kb = blk.reshape(S0, 1), blk.reshape(1, S0)
    causal = idx.reshape(1, S0) <= idx.reshape(S0, 1)
    content_vis = (kr == 0) & (kb == qb)
    earlier_final = (kr == L) & (kb < qb)
    pause_q = (qr > 0) & (qr <= L)
    refine = pause_q & (kr == qr - 1) & (kb == qb)
    replay_q = qr == L + 1
    replay_own_final = replay_q & (kr == L) & (kb == qb)
    replay_causal = replay_q & (kr == L + 1) & (kb == qb)
    samepass = pause_q & (kr == qr) & (kb == qb)
    if pause_xattn not in XATTN:
        raise ValueError(f"unknown pause_xattn {pause_xattn!r}")
    if pause_xattn == "causal":
        samepass = samepass & causal
    elif pause_xattn == "none":
        samepass = np.zeros_like(samepass)
    T = int(retain_tail)
    qa, ka = content_abs.reshape(S0, 1), content_abs.reshape(1, S0)
    if tail_policy == "static":
        retained = (kr == 0) & (kb < qb) & (ka % C >= C - T) & (T > 0)
    elif tail_policy in ("rolling", "sticky"):
        window = (ka % C >= C - T) if tail_policy == "sticky" else (qa - ka <= T)
        retained = (qr == 0) & (kr == 0) & (kb + 1 == qb) & window & (T > 0)
    else:
        raise ValueError(f"unknown tail policy {tail_policy!r}")
    replay_tail = (qr == 0) & (kr == L + 1) & (kb + 1 == qb) & (qa - ka <= R) & (R > 0)
    raw_tail_vis = (qr == 0) & (kr == 0) & (kb + 1 == qb) & (qa - ka <= W) & (W > 0)      # _raw_tail_visible
    base = (causal & (content_vis | earlier_final | refine | retained | replay_own_final | replay_causal
                      | replay_tail | raw_tail_vis)) | samepass
    if prompt_len is not None:
        pl = np.asarray(prompt_len).reshape(-1, 1, 1)
        prompt_raw = (kr == 0)[None] & (content_abs.reshape(1, 1, S0) < pl) & (content_abs.reshape(1, 1, S0) >= 0)
        base = base[None] | (causal[None] & prompt_raw)
    X = R if replay_exclude else T                                 # code_excluded_tail
    if X:
        own_tail = pause_q & (kr == 0) & (kb == qb) & (content_abs.reshape(1, S0) % C >= C - X)
        base = base & ~own_tail
    if head_quota is not None:
        hq = np.asarray(head_quota).reshape(-1, 1, 1)
        slot = code_slot.reshape(1, 1, S0)
        allowed = (slot < 0) | (slot < hq)                          # _quota_key_allowed
        if base.ndim == 3:
            base = base[:, None] & allowed[None]
        else:
            base = base[None] & allowed
    if copy_rows:
        S = S0 + copy_rows
        full = np.zeros(base.shape[:-2] + (S, S), dtype=bool)
        full[..., :S0, :S0] = base
        q, kv = np.arange(S).reshape(S, 1), np.arange(S).reshape(1, S)
        in_cq, in_ck = q >= S0, kv >= S0
        last_final_lo = (N - 1) * per + C + (L - 1) * K
        code_kv = (kv >= last_final_lo) & (kv < last_final_lo + K) & ~in_ck
        copy = in_cq & (code_kv | (in_ck & (kv <= q)))
        if head_quota is not None:
            slot = np.full(S, -1)
            slot[:S0] = code_slot
            copy = copy[None] & ((kv >= S0) | (slot.reshape(1, 1, S) < 0) | (slot.reshape(1, 1, S) < hq))
            if full.ndim == 4:
                copy = copy[None]
        full = full | copy
        base = full
    return base


def masked_attention_fp64(q, k, v, mask, scale):
    """softmax(scale * q k^T, masked) v per head in float64, GQA by head // (Hq / Hkv).

    q: [S, Hq, D]; k, v: [S, Hkv, D]; mask: [S, S] or [Hq, S, S] bool. Returns out [S, Hq, D], lse [S, Hq]
    (natural log). Same arithmetic as the reference's dense path (gen_compress.py:1177-1179) in float64.
    """
    q = np.asarray(q, np.float64)
    k = np.asarray(k, np.float64)
    v = np.asarray(v, np.float64)
    S, Hq, D = q.shape
    Hkv = k.shape[1]
    g = Hq // Hkv
    out = np.zeros((S, Hq, D))
    lse = np.zeros((S, Hq))
    for h in range(Hq):
        m = mask if mask.ndim == 2 else mask[h]
        s = (q[:, h] @ k[:, h // g].T) * scale
        s = np.where(m, s, -np.inf)
        mx = s.max(axis=1, keepdims=True)
        e = np.exp(s - mx)
        z = e.sum(axis=1, keepdims=True)
        out[:, h] = (e / z) @ v[:, h // g]
        lse[:, h] = (mx + np.log(z))[:, 0]
    return out, lse


def masked_attention_rows_fp64(q, k, v, mask_rows, rows, scale):
    """:func:`masked_attention_fp64` restricted to query ``rows`` (every key is still considered).

    mask_rows: [len(rows), S] or [Hq, len(rows), S] (``arith_mask_block(.., rows, all keys, ..)``). Returns
    out [R, Hq, D], lse [R, Hq]. Costs R x S per head instead of S x S, so full-length sequences can be sampled."""
    rows = np.asarray(rows, dtype=np.int64)
    return masked_attention_fp64_qk(np.asarray(q)[rows], k, v, mask_rows, scale)


def masked_attention_fp64_qk(q_rows, k, v, mask_rows, scale):
    """Attention of the given query rows [R, Hq, D] over all keys [S, Hkv, D] under mask_rows ([R, S] or
    [Hq, R, S]); float64, GQA by head // (Hq / Hkv). Returns out [R, Hq, D], lse [R, Hq]."""
    q = np.asarray(q_rows, np.float64)
    k = np.asarray(k, np.float64)
    v = np.asarray(v, np.float64)
    R, Hq, D = q.shape
    g = Hq // k.shape[1]
    out = np.zeros((R, Hq, D))
    lse = np.zeros((R, Hq))
    for h in range(Hq):
        m = mask_rows if mask_rows.ndim == 2 else mask_rows[h]
        s = np.where(m, (q[:, h] @ k[:, h // g].T) * scale, -np.inf)
        mx = s.max(axis=1, keepdims=True)
        e = np.exp(s - mx)
        z = e.sum(axis=1, keepdims=True)
        out[:, h] = (e / z) @ v[:, h // g]
        lse[:, h] = (mx + np.log(z))[:, 0]
    return out, lse


def masked_attention_query_grads_fp64(q, k, v, dout, mask_rows, rows, scale):
    """dq of :func:`masked_attention_grads_fp64` for query ``rows`` only: row i's gradient needs only row i's own
    softmax (dq_i = scale * sum_j P_ij (dP_ij - D_i) k_j with D_i = sum_j P_ij dP_ij). Returns dq [R, Hq, D]."""
    rows = np.asarray(rows, dtype=np.int64)
    qr = np.asarray(q, np.float64)[rows]
    dr = np.asarray(dout, np.float64)[rows]
    k = np.asarray(k, np.float64)
    v = np.asarray(v, np.float64)
    R, Hq, D = qr.shape
    g = Hq // k.shape[1]
    dq = np.zeros((R, Hq, D))
    for h in range(Hq):
        hk = h // g
        m = mask_rows if mask_rows.ndim == 2 else mask_rows[h]
        p = _softmax_rows(np.where(m, (qr[:, h] @ k[:, hk].T) * scale, -np.inf))
        dp = dr[:, h] @ v[:, hk].T
        ds = p * (dp - (p * dp).sum(axis=1, keepdims=True))
        dq[:, h] = scale * ds @ k[:, hk]
    return dq


def masked_attention_key_grads_fp64(q, k, v, dout, mask_fn, keys, scale):
    """dk, dv of :func:`masked_attention_grads_fp64` for the key rows ``keys`` only.

    ``mask_fn(rows, cols)`` returns the mask block ([R, Cc] or [Hq, R, Cc]). Only the queries that see one of the keys
    contribute; each of them needs its whole softmax row (for P and D_i), so the cost is (#such queries) x S per head:
    cheap for keys late in the sequence. Returns dk, dv [len(keys), Hkv, D]."""
    keys = np.asarray(keys, dtype=np.int64)
    q = np.asarray(q, np.float64)
    k = np.asarray(k, np.float64)
    v = np.asarray(v, np.float64)
    dout = np.asarray(dout, np.float64)
    S, Hq, D = q.shape
    Hkv = k.shape[1]
    g = Hq // Hkv
    cols = mask_fn(np.arange(S), keys)
    seen = cols.any(axis=-1) if cols.ndim == 2 else cols.any(axis=(0, 2))
    qi = np.flatnonzero(seen)
    dk = np.zeros((keys.size, Hkv, D))
    dv = np.zeros((keys.size, Hkv, D))
    if qi.size == 0:
        return dk, dv
    m_all = mask_fn(qi, np.arange(S))
    for h in range(Hq):
        hk = h // g
        m = m_all if m_all.ndim == 2 else m_all[h]
        p = _softmax_rows(np.where(m, (q[qi, h] @ k[:, hk].T) * scale, -np.inf))
        dp = dout[qi, h] @ v[:, hk].T
        ds = p * (dp - (p * dp).sum(axis=1, keepdims=True))
        dk[:, hk] += scale * ds[:, keys].T @ q[qi, h]
        dv[:, hk] += p[:, keys].T @ dout[qi, h]
    return dk, dv


def _softmax_rows(s):
    """Row softmax of masked scores (-inf = hidden); an all-hidden row gives zeros."""
    mx = s.max(axis=1, keepdims=True)
    ok = np.isfinite(mx)
    e = np.where(ok, np.exp(s - np.where(ok, mx, 0.0)), 0.0)
    z = e.sum(axis=1, keepdims=True)
    return e / np.where(z > 0, z, 1.0)


def dense_masked_attention_ref_torch(q, k, v, mask, scale):
    """The reference's dense teacher-forced attention on CPU torch (the timed CPU baseline of the masked prefill):
    abridgekv/gen_compress.py:1158-1160, 1176-1179 -- an additive mask of finfo(dtype).min on hidden pairs, scores
    ``q @ repeat_kv(k)^T * scale + add`` in the input dtype, softmax in float32 cast back, ``@ repeat_kv(v)``.

    q [B, Hq, S, D], k / v [B, Hkv, S, D] torch tensors (bf16 as the reference's model runs); mask [S, S] or
    [B, 1, S, S] bool. Returns out [B, Hq, S, D] in q's dtype."""
    import torch

    g = q.shape[1] // k.shape[1]
    m = torch.as_tensor(mask)
    if m.ndim == 2:
        m = m[None, None]
    add = torch.zeros(m.shape, dtype=q.dtype).masked_fill(~m, torch.finfo(q.dtype).min)
    kk = k.repeat_interleave(g, dim=1)
    vv = v.repeat_interleave(g, dim=1)
    w = torch.matmul(q, kk.transpose(2, 3)) * scale + add
    w = torch.softmax(w, dim=-1, dtype=torch.float32).to(q.dtype)
    return torch.matmul(w, vv)


def visible_pairs(C, K, N, prompt_len=None, retain_tail=0, tail_policy="static", pause_xattn="full"):
    """Number of visible (query, key) pairs of one sequence (FLOP accounting: 4 * D * pairs per head)."""
    m = arith_mask(C, K, N, None if prompt_len is None else [prompt_len], retain_tail=retain_tail,
                   tail_policy=tail_policy, pause_xattn=pause_xattn)
    return int(m.sum())


def masked_attention_grads_fp64(q, k, v, mask, scale, dout):
    """Gradients (dq, dk, dv) of sum(dout * masked_attention_fp64(q, k, v, mask, scale)[0]) in float64.

    The softmax backward in closed form: P = softmax(scale * q k^T) over the visible keys, dP = dout v^T,
    dS = P * (dP - rowsum(dP * P)), dq = scale * dS k, dk = scale * dS^T q, dv = P^T dout, dk / dv summed over the
    query heads of each KV head. (The reference trains through FlexAttention's autograd of this attention,
    abridgekv/compress_forward.py:1134-1230, :1329.) Rows with no visible key have P = 0 and contribute nothing.
    """
    q = np.asarray(q, np.float64)
    k = np.asarray(k, np.float64)
    v = np.asarray(v, np.float64)
    dout = np.asarray(dout, np.float64)
    S, Hq, D = q.shape
    Hkv = k.shape[1]
    g = Hq // Hkv
    dq = np.zeros_like(q)
    dk = np.zeros_like(k)
    dv = np.zeros_like(v)
    for h in range(Hq):
        hk = h // g
        m = mask if mask.ndim == 2 else mask[h]
        s = np.where(m, (q[:, h] @ k[:, hk].T) * scale, -np.inf)
        mx = s.max(axis=1, keepdims=True)
        ok = np.isfinite(mx)
        e = np.where(ok, np.exp(s - np.where(ok, mx, 0.0)), 0.0)
        z = e.sum(axis=1, keepdims=True)
        p = e / np.where(z > 0, z, 1.0)
        dp = dout[:, h] @ v[:, hk].T
        ds = p * (dp - (p * dp).sum(axis=1, keepdims=True))
        dq[:, h] = scale * ds @ k[:, hk]
        dk[:, hk] += scale * ds.T @ q[:, h]
        dv[:, hk] += p.T @ dout[:, h]
    return dq, dk, dv

