"""Block-masked teacher-forced attention on the GPU vs the fp64 oracle under the arithmetic compression mask
(tolerance: max-abs <= 2e-2 for bf16 outputs and LSE)."""
import numpy as np
import pytest
import torch

from oracle import prefill as op

pytestmark = pytest.mark.gpu
TOL = 2e-2


def _bf16(x):
    return torch.from_numpy(np.asarray(x, np.float32)).to(torch.bfloat16)


def _check(C, K, N, B, prompt_len=None, head_quota=None, seed=0, rows=None, tail=0, policy="static", xattn="full",
           passes=1, copy_rows=0, replay=0, replay_exclude=False):
    from abridgekv_amd import ops
    S0 = N * (C + passes * K + replay) + copy_rows
    g = torch.Generator().manual_seed(seed)
    q = torch.randn((B, S0, 32, 128), generator=g).to(torch.bfloat16)
    k = torch.randn((B, S0, 8, 128), generator=g).to(torch.bfloat16)
    v = torch.randn((B, S0, 8, 128), generator=g).to(torch.bfloat16)
    dev = torch.device("cuda")
    pl = None if prompt_len is None else torch.tensor(prompt_len, dtype=torch.int32, device=dev)
    hq = None if head_quota is None else torch.tensor(head_quota, dtype=torch.int32, device=dev)
    lse = torch.empty((B, 32, S0), dtype=torch.float32, device=dev)
    out, _ = ops.prefill_masked_attention(q.to(dev), k.to(dev), v.to(dev), C, K, N, prompt_len=pl, head_quota=hq,
                                          lse=lse, retain_tail=tail, tail_policy=policy, pause_xattn=xattn,
                                          pause_passes=passes, copy_rows=copy_rows, replay_rows=replay,
                                          replay_exclude=replay_exclude)
    torch.cuda.synchronize()
    out = out.float().cpu().numpy()
    lse = lse.cpu().numpy()
    worst = 0.0
    for b in range(B):
        raw = policy == "raw"                   # the kernels' raw policy is the oracle's separate raw-tail term
        mask = op.arith_mask(C, K, N, None if prompt_len is None else [prompt_len[b]], head_quota,
                             retain_tail=0 if raw else tail, tail_policy="static" if raw else policy,
                             pause_xattn=xattn, passes=passes, copy_rows=copy_rows, replay=replay,
                             replay_exclude=replay_exclude, raw_tail=tail if raw else 0)
        if prompt_len is not None:
            mask = mask[0]
        sel = slice(None) if rows is None else rows
        ref_o, ref_l = op.masked_attention_fp64(q[b].float().numpy(), k[b].float().numpy(), v[b].float().numpy(),
                                                mask, 128 ** -0.5)
        worst = max(worst, float(np.abs(out[b][sel] - ref_o[sel]).max()),
                    float(np.abs(lse[b].T[sel] - ref_l[sel]).max()))
    assert worst <= TOL, worst


def test_aligned_tiles_no_prompt():
    _check(C=128, K=64, N=3, B=1)


def test_aligned_tiles_prompt_straddles_tiles():
    _check(C=128, K=64, N=4, B=3, prompt_len=[0, 150, 320], seed=1)


def test_aligned_tiles_head_quotas():
    quota = np.repeat([64, 16, 40, 64, 1, 33, 64, 8], 4).tolist()       # per KV head, expanded to its 4 q heads
    _check(C=128, K=64, N=3, B=2, prompt_len=[100, 0], head_quota=quota, seed=2)


def test_unaligned_small_blocks():
    """C=8, K=4: every tile takes the per-element mask path; S0=60 leaves a partial query and key tile."""
    quota = [4, 4, 4, 4, 1, 1, 1, 1, 2, 2, 2, 2, 3, 3, 3, 3] * 2
    _check(C=8, K=4, N=5, B=2, prompt_len=[5, 13], head_quota=quota, seed=3)


def test_config4_shape_sampled_rows():
    """Config-4 block geometry (C=512, K=128) with 4 blocks; rows sampled across blocks and regions."""
    rows = np.r_[0:70, 500:700, 1250:1300, 2400:2560]
    _check(C=512, K=128, N=4, B=1, prompt_len=[512], rows=rows, seed=4)


def test_static_tail_aligned_blocks():
    """Static retained tail T=32 on 64-aligned blocks (the tail forces the per-element mask path): earlier blocks'
    last 32 content rows visible to every later row, hidden from their own block's codes; raw prompt and quotas."""
    quota = np.repeat([64, 16, 40, 64, 1, 33, 64, 8], 4).tolist()
    _check(C=128, K=64, N=4, B=2, prompt_len=[100, 0], head_quota=quota, seed=6, tail=32)


def test_static_tail_unaligned_blocks():
    """C=8, K=4, T=3 with a partial last tile; a raw prompt that covers a tail."""
    quota = [4, 4, 4, 4, 1, 1, 1, 1, 2, 2, 2, 2, 3, 3, 3, 3] * 2
    _check(C=8, K=4, N=5, B=2, prompt_len=[8, 13], head_quota=quota, seed=7, tail=3)


def test_static_tail_served_block_geometry():
    """C=512, K=128, T=64 (span 448 for the codes) with 4 blocks; rows sampled across blocks and regions."""
    rows = np.r_[0:70, 440:520, 600:700, 1250:1300, 2400:2560]
    _check(C=512, K=128, N=4, B=1, prompt_len=[512], rows=rows, seed=8, tail=64)


@pytest.mark.parametrize("policy", ["rolling", "sticky"])
@pytest.mark.parametrize("tail", [32, 100])
def test_window_tail_aligned_blocks(policy, tail):
    """Window tails on 64-aligned blocks: the previous block's last T content rows for the block's content rows only
    (rolling: content row i from tail row i on, a band across one or two key tiles); a raw prompt that covers part of
    block 0's tail; per-head quotas."""
    quota = np.repeat([64, 16, 40, 64, 1, 33, 64, 8], 4).tolist()
    print(f"case: {policy} T={tail}", flush=True)
    _check(C=128, K=64, N=4, B=2, prompt_len=[100, 0], head_quota=quota, seed=16, tail=tail, policy=policy)


@pytest.mark.parametrize("policy", ["rolling", "sticky"])
def test_window_tail_unaligned_blocks(policy):
    """C=8, K=4, T=3 (the per-element predicate) with a partial last tile."""
    quota = [4, 4, 4, 4, 1, 1, 1, 1, 2, 2, 2, 2, 3, 3, 3, 3] * 2
    _check(C=8, K=4, N=5, B=2, prompt_len=[8, 13], head_quota=quota, seed=17, tail=3, policy=policy)


@pytest.mark.parametrize("policy", ["rolling", "sticky"])
def test_window_tail_served_block_geometry(policy):
    """C=512, K=128, T=200 (a rolling band over four key tiles) with 4 blocks; rows sampled where the window acts."""
    rows = np.r_[0:70, 600:780, 1200:1300, 1900:1990, 2400:2560]
    _check(C=512, K=128, N=4, B=1, prompt_len=[300], rows=rows, seed=18, tail=200, policy=policy)


@pytest.mark.parametrize("xattn", ["causal", "none"])
@pytest.mark.parametrize("shape", ["aligned", "unaligned"])
def test_pause_xattn(xattn, shape):
    """Code rows attending their own block's codes causally or not at all (the per-element walk), with a raw prompt,
    per-head quotas and a rolling tail."""
    if shape == "aligned":
        quota = np.repeat([64, 16, 40, 64, 1, 33, 64, 8], 4).tolist()
        _check(C=128, K=64, N=3, B=2, prompt_len=[100, 0], head_quota=quota, seed=19, tail=20, policy="rolling",
               xattn=xattn)
    else:
        quota = [4, 4, 4, 4, 1, 1, 1, 1, 2, 2, 2, 2, 3, 3, 3, 3] * 2
        _check(C=8, K=4, N=5, B=2, prompt_len=[5, 13], head_quota=quota, seed=20, xattn=xattn)


@pytest.mark.parametrize("passes,shape", [(2, "aligned"), (3, "unaligned"), (2, "unaligned")])
def test_pause_passes(passes, shape):
    """L pause passes per block (pass l reads pass l - 1, later blocks the final pass; the per-element walk), with a
    raw prompt, per-head quotas (a slot within its pass), a tail and non-full xattn."""
    if shape == "aligned":
        quota = np.repeat([64, 16, 40, 64, 1, 33, 64, 8], 4).tolist()
        _check(C=128, K=64, N=3, B=2, prompt_len=[100, 0], head_quota=quota, seed=21, tail=20, policy="static",
               passes=passes)
    else:
        quota = [4, 4, 4, 4, 1, 1, 1, 1, 2, 2, 2, 2, 3, 3, 3, 3] * 2
        _check(C=8, K=4, N=5, B=2, prompt_len=[5, 13], head_quota=quota, seed=22 + passes, tail=3,
               policy="rolling", xattn="causal" if passes == 3 else "none", passes=passes)


@pytest.mark.parametrize("shape", ["aligned", "unaligned"])
def test_copy_region(shape):
    """A copy region of 1 + C rows after the blocks (it reads the last block's final pass and itself causally),
    with per-head quotas, one and two passes."""
    if shape == "aligned":
        quota = np.repeat([64, 16, 40, 64, 1, 33, 64, 8], 4).tolist()
        _check(C=128, K=64, N=3, B=2, head_quota=quota, seed=31, copy_rows=129)
        _check(C=128, K=64, N=2, B=1, seed=32, passes=2, copy_rows=129)
    else:
        quota = [4, 4, 4, 4, 1, 1, 1, 1, 2, 2, 2, 2, 3, 3, 3, 3] * 2
        _check(C=8, K=4, N=5, B=2, head_quota=quota, seed=33, tail=2, policy="static", copy_rows=9)


@pytest.mark.parametrize("shape", ["aligned", "unaligned"])
def test_replay_rows(shape):
    """Replay rows after each block's codes (the last R content tokens again; the next block's content reads them
    as a rolling window), with and without hiding the replayed rows from the codes, quotas, a raw prompt, passes and
    a copy region."""
    if shape == "aligned":
        quota = np.repeat([64, 16, 40, 64, 1, 33, 64, 8], 4).tolist()
        _check(C=128, K=64, N=3, B=2, prompt_len=[100, 0], head_quota=quota, seed=37, replay=16)
        _check(C=128, K=64, N=3, B=1, seed=38, replay=64, replay_exclude=True, passes=2, copy_rows=129)
    else:
        quota = [4, 4, 4, 4, 1, 1, 1, 1, 2, 2, 2, 2, 3, 3, 3, 3] * 2
        _check(C=8, K=4, N=5, B=2, prompt_len=[5, 13], head_quota=quota, seed=39, replay=3, replay_exclude=True,
               xattn="causal")


@pytest.mark.parametrize("shape", ["aligned", "unaligned"])
def test_raw_tail(shape):
    """The raw tail (CompressLM(raw_tail=W)): the next block's content rows see the block's last W - i rows and the
    block's codes see their whole block; W up to C, with quotas, a raw prompt, passes, a copy region and xattn."""
    if shape == "aligned":
        quota = np.repeat([64, 16, 40, 64, 1, 33, 64, 8], 4).tolist()
        _check(C=128, K=64, N=3, B=2, prompt_len=[100, 0], head_quota=quota, seed=42, tail=20, policy="raw")
        _check(C=128, K=64, N=3, B=1, seed=43, tail=128, policy="raw", passes=2, copy_rows=129)
    else:
        quota = [4, 4, 4, 4, 1, 1, 1, 1, 2, 2, 2, 2, 3, 3, 3, 3] * 2
        _check(C=8, K=4, N=5, B=2, prompt_len=[5, 13], head_quota=quota, seed=44, tail=3, policy="raw")
        _check(C=8, K=4, N=5, B=1, seed=45, tail=8, policy="raw", xattn="causal")


@pytest.mark.parametrize("C,N", [(512, 1), (256, 3), (200, 2)])
def test_plain_causal_without_codes(C, N):
    """codes_k = 0: causal attention within blocks of C rows (the model's plain forward), aligned and not."""
    _check(C=C, K=0, N=N, B=2, seed=34)


def test_strided_hf_layout():
    """Inputs as HF hands them to an attention function: [B, H, S, D] views of [B, S, H, D] storage, passed back as
    [B, S, H, D] permutations (non-contiguous strides)."""
    from abridgekv_amd import ops
    C, K, N, B = 64, 64, 2, 2
    S0 = N * (C + K)
    dev = torch.device("cuda")
    g = torch.Generator(device=dev).manual_seed(5)
    q_bhsd = torch.randn((B, 32, S0, 128), generator=g, device=dev).to(torch.bfloat16)
    k_bhsd = torch.randn((B, 8, S0, 128), generator=g, device=dev).to(torch.bfloat16)
    v_bhsd = torch.randn((B, 8, S0, 128), generator=g, device=dev).to(torch.bfloat16)
    out, _ = ops.prefill_masked_attention(q_bhsd.transpose(1, 2), k_bhsd.transpose(1, 2), v_bhsd.transpose(1, 2),
                                          C, K, N)
    ref, _ = ops.prefill_masked_attention(q_bhsd.transpose(1, 2).contiguous(), k_bhsd.transpose(1, 2).contiguous(),
                                          v_bhsd.transpose(1, 2).contiguous(), C, K, N)
    torch.cuda.synchronize()
    assert torch.equal(out, ref)


def config4_sample_rows(C, K, N, rng, extra=24):
    """Query rows of the config-4 layout worth checking: the first and last tiles, tile-diagonal rows (first / last
    row of a 64-row tile), the content / code boundary, code rows, in an early, a middle and the last block, plus
    seeded random rows."""
    per = C + K
    picks = set()
    for b in (0, 1, N // 2, N - 1):
        base = b * per
        picks.update(base + x for x in (0, 1, 62, 63, 64, 65, 255, 256, C - 1, C, C + 1, C + 63, C + 64, per - 1))
    picks.update(rng.integers(0, N * per, extra).tolist())
    return np.array(sorted(p for p in picks if p < N * per))


# per-KV-head code quotas (each KV head's 4 query heads share one), aligned and unaligned, for the full-size cases
CONFIG4_QUOTAS = np.repeat([128, 64, 100, 32, 1, 47, 8, 16], 4).tolist()


@pytest.mark.parametrize("prompts,quota", [([512] * 4, None), ([512, 300, 0, 640], CONFIG4_QUOTAS)],
                         ids=["benched", "prompts_and_head_quotas"])
def test_config4_full_size_sampled_rows(prompts, quota):
    """The benched launch itself: B=4, N=16 blocks of [512 content | 128 codes] (S0=10240, 160 query tiles per
    sequence), 512-token raw prompts; and the same size with a different raw prompt per sequence and per-head code
    quotas. Every output and LSE is finite; sampled rows of every sequence match the float64 oracle evaluated on those
    rows over all 10240 keys."""
    from abridgekv_amd import ops
    B, C, K, N = 4, 512, 128, 16
    S0 = N * (C + K)
    dev = torch.device("cuda")
    g = torch.Generator(device=dev).manual_seed(40)
    q = torch.randn((B, S0, 32, 128), generator=g, device=dev).to(torch.bfloat16)
    k = torch.randn((B, S0, 8, 128), generator=g, device=dev).to(torch.bfloat16)
    v = torch.randn((B, S0, 8, 128), generator=g, device=dev).to(torch.bfloat16)
    pl = torch.tensor(prompts, dtype=torch.int32, device=dev)
    hq = None if quota is None else torch.tensor(quota, dtype=torch.int32, device=dev)
    lse = torch.empty((B, 32, S0), dtype=torch.float32, device=dev)
    out, _ = ops.prefill_masked_attention(q, k, v, C, K, N, prompt_len=pl, head_quota=hq, lse=lse)
    torch.cuda.synchronize()
    assert torch.isfinite(out).all() and torch.isfinite(lse).all()
    rng = np.random.default_rng(4)
    worst = 0.0
    for b in range(B):
        rows = config4_sample_rows(C, K, N, rng)
        mask = op.arith_mask_block(C, K, N, rows, np.arange(S0), [prompts[b]], quota)[0]
        qb, kb, vb = (t[b].float().cpu().numpy() for t in (q, k, v))
        ref_o, ref_l = op.masked_attention_rows_fp64(qb, kb, vb, mask, rows, 128 ** -0.5)
        got_o = out[b].float().cpu().numpy()[rows]
        got_l = lse[b].cpu().numpy().T[rows]
        worst = max(worst, float(np.abs(got_o - ref_o).max()), float(np.abs(got_l - ref_l).max()))
    assert worst <= TOL, worst


@pytest.mark.parametrize("seed", range(6))
def test_seeded_random_layouts(seed):
    """Seeded random layouts: block sizes aligned to the 64-row tiles or not, raw prompts anywhere in the first blocks,
    per-KV-head code quotas in [1, K], and (for odd seeds) a retained tail under one of the three policies; against
    the fp64 oracle."""
    rng = np.random.default_rng(2000 + seed)
    C = int(rng.choice([64, 128, 40, 24]))
    K = int(rng.choice([64, 16, 8]))
    N = int(rng.integers(2, 4))
    B = int(rng.integers(1, 3))
    prompt = [int(x) for x in rng.integers(0, N * C // 2 + 1, B)]
    quota = np.repeat(rng.integers(1, K + 1, 8), 4).tolist()
    tail = int(rng.integers(1, max(2, C - K))) if seed % 2 and C > K else 0
    policy = ("static", "rolling", "sticky")[seed % 3] if tail else "static"
    print(f"case: seed {seed} C={C} K={K} N={N} B={B} prompt={prompt} tail={tail} {policy}", flush=True)
    _check(C=C, K=K, N=N, B=B, prompt_len=prompt, head_quota=quota, seed=10 + seed, tail=tail, policy=policy)
