"""Pins of oracle.prefill: the two reference mask forms agree, a per-element predicate written from the prose rule
agrees, L=1 analogues of the reference's spot checks hold, and the fp64 attention reduces to textbook cases."""
import json
from pathlib import Path

import numpy as np
import pytest
import scipy.special as sp

from oracle import prefill as op

GOLDEN = Path(__file__).resolve().parent / "golden"


def brute(C, K, N, prompt_len=None, quota=None, tail=0, policy="static", xattn="full", passes=1, copy_rows=0,
          replay=0, replay_exclude=False, raw=0):
    """Element-by-element rule: causal & (own-block content | earlier blocks' codes | raw-prompt content), or
    (code query & code key & same block); a code key with slot >= quota is hidden. Static retained tail (the config's
    prose, compresslm.py:22-25): "the final T content KVs of every completed block stay resident forever, visible to
    all later queries (content and code rows), and the codes summarize only the first block_size - T tokens".
    Window tails (compresslm.py:23, "window tails of the previous block (content queries only, expire)"): sticky
    keeps the previous block's whole tail for every content query of the block; rolling lets the i-th content token
    of the block see the previous block's tail rows from the i-th on (one tail row expires per content token).
    pause_xattn (compress_forward.py:313-314, "within-pass code<->code attention"): "full" every code row of the
    block, "causal" the ones up to the query, "none" no code row of its own block.
    L = passes pause passes (compress_forward.py:594-600, "pause^l <- own pause^{l-1}", "earlier blocks' final
    codes"): a code row of pass l also reads its block's pass l - 1, the xattn rule speaks of its own pass, later
    blocks read the final pass only, and a quota counts a row's slot within its pass.
    Copy region (compress_forward.py:631, "copy region q>=S0: attend ONLY last block's K final codes + causal within
    copy"): copy_rows rows after the blocks; the quota still hides code slots >= quota.
    Replay rows (compress_forward.py:20-31, 139-178, "post-summary tail replay", "pause^l <- own pause^{l-1}";
    _replay_tail_visible "Whether content query q may see a post-summary replay row from the preceding block"): the
    R rows after a block's codes replay its last R content tokens; a replay row reads its block's content, final
    codes and replay rows up to itself; content row i of the next block reads the previous block's replay rows whose
    replayed position is within R of its own (replay row r with r >= i); with replay_exclude the codes do not read the
    block's last R content rows.
    Raw tail (_raw_tail_visible, compress_forward.py:90-93: "Whether content query q may see a raw token from the
    immediately preceding block. The tail is a rolling window: at position j in a new block, only the final
    raw_tail-j tokens from the previous block remain visible"); nothing hides it from the codes."""
    LK = passes * K
    per = C + LK + replay
    S0 = N * per
    S = S0 + copy_rows
    m = np.zeros((S, S), bool)
    for q in range(S):
        if q >= S0:                              # a copy row
            lo = S0 - replay - K                 # the last block's final pass (before its replay rows)
            for k in range(q + 1):
                m[q, k] = k >= S0 or (lo <= k < lo + K and (quota is None or k - lo < quota))
            continue
        qb, qw = divmod(q, per)
        q_rep = qw >= C + LK
        q_pass = 0 if (qw < C or q_rep) else (qw - C) // K + 1
        for k in range(S0):
            kb, kw = divmod(k, per)
            k_content = kw < C
            k_rep = kw >= C + LK
            k_pass = 0 if (k_content or k_rep) else (kw - C) // K + 1
            vis = (k_content and kb == qb) or (k_pass == passes and kb < qb)
            if q_rep and kb == qb and (k_pass == passes or k_rep):
                vis = True                       # a replay row: its block's final codes and replay rows
            if replay and qw < C and k_rep and kb == qb - 1 and kw - C - LK >= qw:
                vis = True                       # the previous block's replay rows, a rolling window
            if prompt_len is not None and k_content and kb * C + kw < prompt_len:
                vis = True
            if raw and qw < C and k_content and kb == qb - 1 and kw >= C - (raw - qw):
                vis = True                       # the previous block's final raw - j rows, j = the query's offset
            if tail and policy == "static" and k_content and kb < qb and kw >= C - tail:
                vis = True                       # an earlier block's tail row: resident, seen by every later query
            if tail and policy != "static" and qw < C and k_content and kb == qb - 1:
                row = kw - (C - tail)            # index of the key in the previous block's tail (< 0: not in it)
                if row >= 0 and (policy == "sticky" or row >= qw):
                    vis = True
            vis = vis and k <= q
            same_pass = q_pass == k_pass
            q_code, k_code = q_pass > 0, k_pass > 0
            if q_code and k_code and kb == qb and same_pass and (xattn == "full" or (xattn == "causal" and k <= q)):
                vis = True
            if q_code and k_code and kb == qb and k_pass == q_pass - 1:
                vis = True                       # the previous pass of the same block
            if tail and q_code and k_content and kb == qb and kw >= C - tail:
                vis = False                      # a code row does not summarize its own block's tail
            if replay_exclude and q_code and k_content and kb == qb and kw >= C - replay:
                vis = False
            if quota is not None and k_code and (kw - C) % K >= quota:
                vis = False
            m[q, k] = vis
    return m


@pytest.mark.parametrize("C,K,N", [(4, 4, 3), (8, 2, 2), (4, 1, 4), (2, 4, 3)])
def test_arith_equals_role_equals_brute(C, K, N):
    a = op.arith_mask(C, K, N)
    r = op.role_mask(C, K, N)
    assert np.array_equal(a, r)
    assert np.array_equal(a, brute(C, K, N))
    pl = [0, 3, C + 1, N * C]
    ap = op.arith_mask(C, K, N, prompt_len=pl)
    assert np.array_equal(ap, op.role_mask(C, K, N, prompt_len=pl))
    for b, p in enumerate(pl):
        assert np.array_equal(ap[b], brute(C, K, N, prompt_len=p))


@pytest.mark.parametrize("C,K,N,T", [(4, 2, 3, 2), (8, 4, 3, 3), (8, 2, 4, 1), (6, 4, 3, 2)])
def test_static_tail_arith_equals_role_equals_brute(C, K, N, T):
    a = op.arith_mask(C, K, N, retain_tail=T)
    assert np.array_equal(a, op.role_mask(C, K, N, retain_tail=T))
    assert np.array_equal(a, brute(C, K, N, tail=T))
    assert not np.array_equal(a, op.arith_mask(C, K, N))                    # the tail changes the mask
    pl = [0, 3, C + 1, N * C]
    hq = [1, K, 2, K]
    ap = op.arith_mask(C, K, N, prompt_len=pl, head_quota=hq, retain_tail=T)
    assert np.array_equal(ap, op.role_mask(C, K, N, prompt_len=pl, head_quota=hq, retain_tail=T))
    for b, p in enumerate(pl):
        for h, q in enumerate(hq):
            assert np.array_equal(ap[b, h], brute(C, K, N, prompt_len=p, quota=q, tail=T))


@pytest.mark.parametrize("policy", ["rolling", "sticky"])
@pytest.mark.parametrize("C,K,N,T", [(4, 2, 3, 2), (8, 4, 3, 3), (8, 2, 4, 1), (6, 4, 3, 5)])
def test_window_tail_arith_equals_role_equals_brute(C, K, N, T, policy):
    a = op.arith_mask(C, K, N, retain_tail=T, tail_policy=policy)
    assert np.array_equal(a, op.role_mask(C, K, N, retain_tail=T, tail_policy=policy))
    assert np.array_equal(a, brute(C, K, N, tail=T, policy=policy))
    assert not np.array_equal(a, op.arith_mask(C, K, N, retain_tail=T))       # not the static mask
    pl = [0, 3, C + 1, N * C]
    hq = [1, K, 2, K]
    ap = op.arith_mask(C, K, N, prompt_len=pl, head_quota=hq, retain_tail=T, tail_policy=policy)
    assert np.array_equal(ap, op.role_mask(C, K, N, prompt_len=pl, head_quota=hq, retain_tail=T, tail_policy=policy))
    for b, p in enumerate(pl):
        for h, q in enumerate(hq):
            assert np.array_equal(ap[b, h], brute(C, K, N, prompt_len=p, quota=q, tail=T, policy=policy))


@pytest.mark.parametrize("xattn", ["causal", "none"])
@pytest.mark.parametrize("C,K,N,T", [(4, 2, 3, 0), (8, 4, 3, 3), (6, 4, 3, 2)])
def test_pause_xattn_arith_equals_role_equals_brute(C, K, N, T, xattn):
    for policy in ("static", "rolling"):
        kw = dict(retain_tail=T, tail_policy=policy, pause_xattn=xattn)
        a = op.arith_mask(C, K, N, **kw)
        assert np.array_equal(a, op.role_mask(C, K, N, **kw))
        assert np.array_equal(a, brute(C, K, N, tail=T, policy=policy, xattn=xattn))
        assert not np.array_equal(a, op.arith_mask(C, K, N, retain_tail=T, tail_policy=policy))
        pl, hq = [0, C + 1], [1, K, 2, K]
        ap = op.arith_mask(C, K, N, prompt_len=pl, head_quota=hq, **kw)
        assert np.array_equal(ap, op.role_mask(C, K, N, prompt_len=pl, head_quota=hq, **kw))
        for b, p in enumerate(pl):
            for h, q in enumerate(hq):
                assert np.array_equal(ap[b, h], brute(C, K, N, prompt_len=p, quota=q, tail=T, policy=policy,
                                                      xattn=xattn))
    per = C + K
    m = op.arith_mask(C, K, N, pause_xattn=xattn)
    assert m[C, C] == (xattn == "causal") and not m[C, C + 1]          # a code row and the next code row
    assert m[C + 1, C] == (xattn == "causal") and m[per + C, C]        # earlier codes stay visible


@pytest.mark.parametrize("C,K,N,L", [(4, 2, 3, 2), (4, 2, 2, 3), (6, 4, 3, 2), (2, 3, 3, 3)])
def test_pause_passes_arith_equals_role_equals_brute(C, K, N, L):
    for T, policy, xattn in ((0, "static", "full"), (1, "static", "causal"), (2 if C > 2 else 1, "rolling", "none"),
                             (1, "sticky", "full")):
        kw = dict(retain_tail=T, tail_policy=policy, pause_xattn=xattn, passes=L)
        a = op.arith_mask(C, K, N, **kw)
        assert np.array_equal(a, op.role_mask(C, K, N, **kw))
        assert np.array_equal(a, brute(C, K, N, tail=T, policy=policy, xattn=xattn, passes=L))
        pl, hq = [0, C + 1], [1, K, 2, K]
        ap = op.arith_mask(C, K, N, prompt_len=pl, head_quota=hq, **kw)
        assert np.array_equal(ap, op.role_mask(C, K, N, prompt_len=pl, head_quota=hq, **kw))
        for b, p in enumerate(pl):
            for h, q in enumerate(hq):
                assert np.array_equal(ap[b, h], brute(C, K, N, prompt_len=p, quota=q, tail=T, policy=policy,
                                                      xattn=xattn, passes=L))
    per = C + L * K
    m = op.arith_mask(C, K, N, passes=L)
    first, final = C, C + (L - 1) * K                        # the first rows of pass 1 and of the final pass
    assert m[per + C, final] and not m[per + C, first]       # a later block reads the final pass only
    assert m[C + K, first] and m[C + K, first + K - 1]       # pass 2 reads all of pass 1 (after it)
    assert not m[C, C + K] and m[C + K, C + K + K - 1]       # pass 1 does not read pass 2; pass 2 reads itself
    assert L < 3 or not m[C + 2 * K, first]                  # pass 3 does not read pass 1
    assert np.array_equal(op.arith_mask(C, K, N, passes=1), op.arith_mask(C, K, N))


@pytest.mark.parametrize("C,K,N,L", [(4, 2, 3, 1), (4, 2, 2, 2), (6, 4, 2, 1), (3, 2, 3, 3)])
def test_copy_region_arith_equals_role_equals_brute(C, K, N, L):
    cr = C + 1                                               # the copy token and the last block's content
    for T, policy, xattn in ((0, "static", "full"), (1, "static", "causal"), (2, "rolling", "full")):
        kw = dict(retain_tail=T, tail_policy=policy, pause_xattn=xattn, passes=L, copy_rows=cr)
        a = op.arith_mask(C, K, N, **kw)
        assert np.array_equal(a, op.role_mask(C, K, N, **kw))
        assert np.array_equal(a, brute(C, K, N, tail=T, policy=policy, xattn=xattn, passes=L, copy_rows=cr))
        S0 = N * (C + L * K)
        assert np.array_equal(a[:S0, :S0], op.arith_mask(C, K, N, retain_tail=T, tail_policy=policy,
                                                         pause_xattn=xattn, passes=L))
        hq = [1, K, 2, K]
        ah = op.arith_mask(C, K, N, head_quota=hq, **kw)
        assert np.array_equal(ah, op.role_mask(C, K, N, head_quota=hq, **kw))
        for h, q in enumerate(hq):
            assert np.array_equal(ah[h], brute(C, K, N, quota=q, tail=T, policy=policy, xattn=xattn, passes=L,
                                               copy_rows=cr))
    # a block-local causal mask without codes
    plain = op.arith_mask(C, 0, N)
    blk = np.arange(N * C) // C
    assert np.array_equal(plain, np.tril(np.ones((N * C, N * C), bool)) & (blk[:, None] == blk[None, :]))
    assert np.array_equal(plain, op.role_mask(C, 0, N))


@pytest.mark.parametrize("C,K,N,L,R", [(4, 2, 3, 1, 2), (6, 2, 3, 2, 3), (4, 3, 3, 1, 4), (3, 2, 4, 1, 1)])
def test_replay_rows_arith_equals_role_equals_brute(C, K, N, L, R):
    for exclude, xattn in ((False, "full"), (True, "full"), (False, "causal"), (True, "none")):
        kw = dict(passes=L, replay=R, replay_exclude=exclude, pause_xattn=xattn)
        a = op.arith_mask(C, K, N, **kw)
        assert np.array_equal(a, op.role_mask(C, K, N, **kw))
        assert np.array_equal(a, brute(C, K, N, xattn=xattn, passes=L, replay=R, replay_exclude=exclude))
        pl, hq = [0, C + 1], [1, K, 2, K]
        ap = op.arith_mask(C, K, N, prompt_len=pl, head_quota=hq, copy_rows=C + 1, **kw)
        assert np.array_equal(ap, op.role_mask(C, K, N, prompt_len=pl, head_quota=hq, copy_rows=C + 1, **kw))
        for b, p in enumerate(pl):
            for h, q in enumerate(hq):
                assert np.array_equal(ap[b, h], brute(C, K, N, prompt_len=p, quota=q, xattn=xattn, passes=L,
                                                      copy_rows=C + 1, replay=R, replay_exclude=exclude))
    per = C + L * K + R
    m = op.arith_mask(C, K, N, passes=L, replay=R)
    rep0 = C + L * K                                          # block 0's first replay row
    assert m[rep0, 0] and m[rep0, rep0 - 1] and not m[rep0, rep0 + 1]      # content, final codes; causal replay
    assert m[per, rep0] and m[per + 1, rep0 + 1] and not m[per + 1, rep0]  # content row i reads replay rows >= i
    assert not m[2 * per, rep0]                                             # two blocks later: expired
    assert not m[rep0, per]                                                 # the next block is hidden
    with pytest.raises(ValueError):
        op.arith_mask(C, K, N, replay=R, retain_tail=1)


def test_window_tail_spot_checks():
    """Rolling: block 1's i-th content row sees block 0's tail rows i.. only, block 2 sees none of block 0's tail,
    codes see no earlier tail. Sticky: all of block 0's tail for every content row of block 1, none for its codes.
    Both: a raw-prompt tail row stays visible to everyone."""
    C, K, N, T = 8, 4, 3, 3
    per = C + K
    r = op.arith_mask(C, K, N, retain_tail=T, tail_policy="rolling")
    assert r[per, C - T] and r[per, C - 1] and not r[per, C - T - 1]
    assert not r[per + 1, C - T] and r[per + 1, C - T + 1] and r[per + 2, C - 1] and not r[per + 3, C - 1]
    assert not r[2 * per, C - 1] and not r[per + C, C - 1] and not r[2 * per + C, per + C - 1]
    assert r[2 * per, per + C - 1] and r[C, 0] and not r[C, C - T]          # own-tail exclusion kept
    s = op.arith_mask(C, K, N, retain_tail=T, tail_policy="sticky")
    assert all(s[per + i, C - T] and s[per + i, C - 1] for i in range(C)) and not s[per, C - T - 1]
    assert not s[per + C, C - 1] and not s[2 * per, C - 1]
    for pol in ("rolling", "sticky"):
        m = op.arith_mask(C, K, N, prompt_len=[C], retain_tail=T, tail_policy=pol)[0]
        assert m[2 * per + C, C - 1] and m[per + C, C - T]                   # prompt rows: raw prompt
        assert not m[C, C - 1]                                               # but not for their own block's codes


def test_static_tail_spot_checks():
    """Block 1's content sees block 0's last T rows but not the rows before them; block 0's codes do not see its own
    tail; a tail row inside the raw prompt is still hidden from its own block's codes."""
    C, K, N, T = 8, 4, 3, 3
    per = C + K
    m = op.arith_mask(C, K, N, retain_tail=T)
    assert m[per, C - T] and m[per, C - 1] and not m[per, C - T - 1]
    assert m[2 * per + C, C - 1]                        # codes of a later block see earlier tails
    assert m[C, 0] and m[C, C - T - 1] and not m[C, C - T] and not m[C, C - 1]
    assert m[C - 1, C - T]                              # content sees its own block causally, tail included
    mp = op.arith_mask(C, K, N, prompt_len=[2 * C], retain_tail=T)[0]
    assert mp[per, 0] and not mp[C, C - 1] and not mp[per + C, per + C - 1]


def test_head_quotas_compose_with_base_mask():
    """scripts/test_sft_head_code_quotas.py:175-197 rule (L=1): masked(h) == base & key_allowed(h), with per-query-head
    quotas from the 2x2 fixture expanded over the GQA group (kv head quota repeated for its query heads)."""
    quotas = json.loads((GOLDEN / "head_code_quotas_2x2.json").read_text())["head_code_quotas"]
    C, K, N = 4, 4, 3
    base = op.arith_mask(C, K, N)
    for layer_q in quotas:
        per_q_head = np.repeat(layer_q, 2)                          # 2 KV heads -> 4 query heads
        got = op.arith_mask(C, K, N, head_quota=per_q_head)
        assert np.array_equal(got, op.role_mask(C, K, N, head_quota=per_q_head))
        for h, q in enumerate(per_q_head):
            assert np.array_equal(got[h], brute(C, K, N, quota=q))
            assert np.array_equal(got[h] & ~base, np.zeros_like(base))
    pl = [5, 2]
    got = op.arith_mask(C, K, N, prompt_len=pl, head_quota=[1, 1, 3, 3])
    assert got.shape == (2, 4, N * (C + K), N * (C + K))
    assert np.array_equal(got, op.role_mask(C, K, N, prompt_len=pl, head_quota=[1, 1, 3, 3]))


def test_spot_checks_l1():
    """L=1 analogues of the reference's point checks (scripts/test_sft_head_code_quotas.py:201-260)."""
    C, K, N = 4, 4, 3
    per = C + K
    m = op.arith_mask(C, K, N, head_quota=[1, 1, 3, 3])[0]      # head 0, quota 1
    assert m[per, C]                         # block-1 content sees block-0 code slot 0
    assert not m[per, C + 1]                 # ... but not slot 1 (quota 1)
    assert m[2 * per, C] and m[2 * per, per + C]
    assert not m[2 * per, per + C + 1]
    assert not m[C - 1, C]                   # content never sees its own block's codes
    full = op.arith_mask(C, K, N)
    assert full[C, C + 3]                    # codes attend to later codes of their block (bidirectional)
    assert full[C + 3, 0]                    # codes see their own block's content
    assert not full[per + C, 0]              # ... but not earlier blocks' content (no raw prompt)
    assert op.arith_mask(C, K, N, prompt_len=[5])[0][per + C, 3]    # raw prompt is visible to everyone later


def test_single_block_without_quota_is_causal_on_content():
    m = op.arith_mask(6, 2, 1)
    assert np.array_equal(m[:6, :6], np.tril(np.ones((6, 6), bool)))


def test_masked_attention_textbook_cases():
    rng = np.random.default_rng(0)
    S, D = 12, 16
    q = rng.standard_normal((S, 4, D))
    k = rng.standard_normal((S, 2, D))
    v = rng.standard_normal((S, 2, D))
    causal = np.tril(np.ones((S, S), bool))
    out, lse = op.masked_attention_fp64(q, k, v, causal, 0.25)
    for h in range(4):
        for i in range(S):
            s = 0.25 * k[: i + 1, h // 2] @ q[i, h]
            assert np.isclose(lse[i, h], sp.logsumexp(s))
            assert np.allclose(out[i, h], sp.softmax(s) @ v[: i + 1, h // 2])
    eye = np.eye(S, dtype=bool)                                     # one visible key -> its value
    out, lse = op.masked_attention_fp64(q, k, v, eye, 0.25)
    assert np.allclose(out[:, 1], v[:, 0]) and np.allclose(out[:, 3], v[:, 1])


def closed_form_pairs(C, K, N):
    """Visible pairs per head when block 0 is the raw prompt: block-b content queries see their block's content
    causally, b*K earlier codes and (b > 0) the C prompt rows; block-b code queries see their block's C content and K
    codes, b*K earlier codes and (b > 0) the prompt rows."""
    n = 0
    for b in range(N):
        n += C * (C + 1) // 2 + C * b * K + (C * C if b else 0)
        n += K * C + K * K + K * b * K + (K * C if b else 0)
    return n


@pytest.mark.parametrize("C,K,N", [(8, 4, 3), (16, 4, 5), (512, 128, 16)])
def test_visible_pair_count(C, K, N):
    """FLOP accounting of the masked prefill (B=4 workload: N=16 blocks of [512 | 128], 512-token raw prompt)."""
    assert op.visible_pairs(C, K, N, prompt_len=C) == closed_form_pairs(C, K, N)


@pytest.mark.parametrize("C,K,N,T", [(8, 4, 3, 0), (8, 4, 4, 3), (16, 8, 5, 5), (64, 16, 6, 16), (512, 128, 16, 32)])
def test_benchmark_pair_count_matches_the_mask(C, K, N, T):
    """The masked-prefill bench's FLOP accounting (workloads.visible_pairs_prompt_block, with a retained tail of T
    rows under each policy) counts exactly the pairs the oracle mask shows, raw prompt = block 0."""
    from abridgekv_amd.workloads import visible_pairs_prompt_block
    for policy in ("static", "rolling", "sticky"):
        assert visible_pairs_prompt_block(C, K, N, T, policy) == op.visible_pairs(C, K, N, prompt_len=C,
                                                                                  retain_tail=T, tail_policy=policy)


def test_masked_attention_grads_match_autograd_and_finite_differences():
    """The closed-form softmax backward against torch autograd of the fp64 forward (an independent derivation) on the
    compression mask with prompt and per-head quotas, and against central differences on a tiny case."""
    import torch

    rng = np.random.default_rng(7)
    C, K, N, Hq, Hkv, D = 6, 3, 3, 4, 2, 5
    S = N * (C + K)
    mask = op.arith_mask(C, K, N, [4], [3, 1, 2, 3])[0]           # [Hq, S, S]
    q, k, v, dout = (rng.standard_normal(sh) for sh in ((S, Hq, D), (S, Hkv, D), (S, Hkv, D), (S, Hq, D)))
    scale = 0.7
    dq, dk, dv = op.masked_attention_grads_fp64(q, k, v, mask, scale, dout)

    tq, tk, tv = (torch.tensor(x, dtype=torch.float64, requires_grad=True) for x in (q, k, v))
    outs = []
    for h in range(Hq):
        s = (tq[:, h] @ tk[:, h // 2].T) * scale
        s = s.masked_fill(~torch.from_numpy(mask[h]), float("-inf"))
        outs.append(torch.softmax(s, dim=1) @ tv[:, h // 2])
    (torch.stack(outs, 1) * torch.from_numpy(dout)).sum().backward()
    for mine, ref in ((dq, tq.grad), (dk, tk.grad), (dv, tv.grad)):
        np.testing.assert_allclose(mine, ref.numpy(), rtol=1e-10, atol=1e-12)

    def loss(qq, kk, vv):
        return float((op.masked_attention_fp64(qq, kk, vv, mask, scale)[0] * dout).sum())

    eps = 1e-6
    for arr, grad in ((q, dq), (k, dk), (v, dv)):
        for idx in [(0, 0, 0), (S - 1, arr.shape[1] - 1, D - 1), (C + 1, 1, 2)]:
            a1, a2 = arr.copy(), arr.copy()
            a1[idx] += eps
            a2[idx] -= eps
            args1 = [a1 if arr is x else x for x in (q, k, v)]
            args2 = [a2 if arr is x else x for x in (q, k, v)]
            fd = (loss(*args1) - loss(*args2)) / (2 * eps)
            assert abs(fd - grad[idx]) <= 1e-6 * max(1.0, abs(fd)), (idx, fd, grad[idx])


@pytest.mark.parametrize("seed", range(3))
def test_mask_block_equals_role_mask_slices(seed):
    """arith_mask_block (sampled rows x sampled keys) against the independent role/table restatement, with a raw
    prompt and per-head quotas, on unsorted and repeated index sets."""
    rng = np.random.default_rng(seed)
    C, K, N = 8, 4, 4
    S = N * (C + K)
    rows = rng.integers(0, S, 17)
    cols = rng.integers(0, S, 23)
    pl, hq = [int(rng.integers(0, 2 * C))], rng.integers(1, K + 1, 4).tolist()
    got = op.arith_mask_block(C, K, N, rows, cols, pl, hq)[0]
    ref = op.role_mask(C, K, N, pl, hq)[0][:, rows][:, :, cols]
    assert np.array_equal(got, ref)
    assert np.array_equal(op.arith_mask_block(C, K, N, rows, cols), op.role_mask(C, K, N)[rows][:, cols])


def test_row_and_key_restricted_attention_equal_the_full_forms():
    """The sampled-row forward, the sampled-row dq and the sampled-key dk/dv equal the corresponding rows of the full
    fp64 forms (which are pinned against autograd and central differences above)."""
    rng = np.random.default_rng(11)
    C, K, N, Hq, Hkv, D = 6, 3, 4, 4, 2, 5
    S = N * (C + K)
    pl, hq = [5], [3, 1, 2, 3]
    mask = op.arith_mask(C, K, N, pl, hq)[0]
    q, k, v, dout = (rng.standard_normal(sh) for sh in ((S, Hq, D), (S, Hkv, D), (S, Hkv, D), (S, Hq, D)))
    scale = 0.6
    out, lse = op.masked_attention_fp64(q, k, v, mask, scale)
    dq, dk, dv = op.masked_attention_grads_fp64(q, k, v, mask, scale, dout)
    rows = np.array([0, 3, C, C + K - 1, S - 1, 2 * (C + K) + 1])
    mrows = op.arith_mask_block(C, K, N, rows, np.arange(S), pl, hq)[0]
    o_r, l_r = op.masked_attention_rows_fp64(q, k, v, mrows, rows, scale)
    np.testing.assert_allclose(o_r, out[rows], rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(l_r, lse[rows], rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(op.masked_attention_query_grads_fp64(q, k, v, dout, mrows, rows, scale), dq[rows],
                               rtol=1e-10, atol=1e-12)
    keys = np.array([0, 4, C, S - K - 1, S - 1, S - K])

    def mask_fn(r, c):
        return op.arith_mask_block(C, K, N, r, c, pl, hq)[0]

    dk_r, dv_r = op.masked_attention_key_grads_fp64(q, k, v, dout, mask_fn, keys, scale)
    np.testing.assert_allclose(dk_r, dk[keys], rtol=1e-10, atol=1e-12)
    np.testing.assert_allclose(dv_r, dv[keys], rtol=1e-10, atol=1e-12)


def test_dense_reference_torch_matches_fp64_within_bf16():
    """The CPU baseline's dense bf16 attention (the reference's gen_compress.py arithmetic) against the fp64 oracle on
    the same bf16 inputs: within 3e-2 (that arithmetic rounds scores and probabilities to bf16 itself), and a key
    hidden from a row cannot move that row's output by a single bit."""
    import torch

    C, K, N = 16, 8, 3
    S = N * (C + K)
    rng = np.random.default_rng(2)
    q, k, v = (rng.standard_normal(sh) for sh in ((S, 4, 32), (S, 2, 32), (S, 2, 32)))
    t = [torch.from_numpy(x).permute(1, 0, 2)[None].to(torch.bfloat16) for x in (q, k, v)]
    q, k, v = (x[0].permute(1, 0, 2).double().numpy() for x in t)
    mask = op.arith_mask(C, K, N, [10])[0]
    ref, _ = op.masked_attention_fp64(q, k, v, mask, 0.3)
    got = op.dense_masked_attention_ref_torch(*t, torch.from_numpy(mask), 0.3)[0].permute(1, 0, 2).float().numpy()
    assert np.abs(got - ref).max() <= 3e-2
    t2 = [x.clone() for x in t]
    t2[1][0, :, S - 1] = 100.0                 # the last key is visible only to the last block's code rows
    got2 = op.dense_masked_attention_ref_torch(*t2, torch.from_numpy(mask), 0.3)[0].permute(1, 0, 2)
    hidden_rows = ~mask[:, S - 1]
    assert torch.equal(got2[torch.from_numpy(hidden_rows)], torch.from_numpy(got)[torch.from_numpy(hidden_rows)].to(
        torch.bfloat16))


@pytest.mark.parametrize("C,K,N,L,W", [(4, 2, 3, 1, 2), (6, 2, 3, 2, 3), (4, 3, 3, 1, 4), (3, 2, 4, 1, 1),
                                       (8, 4, 3, 1, 5)])
def test_raw_tail_arith_equals_role_equals_brute(C, K, N, L, W):
    for xattn in ("full", "causal", "none"):
        kw = dict(passes=L, raw_tail=W, pause_xattn=xattn)
        a = op.arith_mask(C, K, N, **kw)
        assert np.array_equal(a, op.role_mask(C, K, N, **kw))
        assert np.array_equal(a, brute(C, K, N, xattn=xattn, passes=L, raw=W))
        pl, hq = [0, C + 1], [1, K, 2, K]
        ap = op.arith_mask(C, K, N, prompt_len=pl, head_quota=hq, copy_rows=C + 1, **kw)
        assert np.array_equal(ap, op.role_mask(C, K, N, prompt_len=pl, head_quota=hq, copy_rows=C + 1, **kw))
        for b, p in enumerate(pl):
            for h, q in enumerate(hq):
                assert np.array_equal(ap[b, h], brute(C, K, N, prompt_len=p, quota=q, xattn=xattn, passes=L,
                                                      copy_rows=C + 1, raw=W))
    per = C + L * K
    m = op.arith_mask(C, K, N, passes=L, raw_tail=W)
    assert m[C, C - 1] and m[C, 0]                              # a code row sees its whole block, tail included
    assert m[per, C - W] and (W == 1 or not m[per, C - W - 1])  # content row 0 of block 1: block 0's last W rows
    assert not m[per + W, C - 1] if W < C else True             # row W: the window has passed
    assert not m[2 * per, C - 1]                                # two blocks later: gone
    # the retained rolling tail is the same window with the codes kept off the block's tail
    if W < C:
        rolling = op.arith_mask(C, K, N, passes=L, retain_tail=W, tail_policy="rolling")
        code = np.zeros(m.shape[0], bool)
        code[[b * per + C + i for b in range(N) for i in range(L * K)]] = True
        assert np.array_equal(rolling[~code], m[~code])
        assert not np.array_equal(rolling[code], m[code])
    with pytest.raises(ValueError):
        op.arith_mask(C, K, N, raw_tail=W, retain_tail=1)
    with pytest.raises(ValueError):
        op.arith_mask(C, K, N, raw_tail=W, replay=1)
