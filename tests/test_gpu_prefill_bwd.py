"""Backward of the block-masked teacher-forced attention on the GPU vs the fp64 closed-form gradients of the oracle
(bf16 inputs; tolerance: max-abs error <= 2e-2 x the largest |gradient| of each tensor, plus 2e-3)."""
import numpy as np
import pytest
import torch

from oracle import prefill as op

pytestmark = pytest.mark.gpu


def _check(C, K, N, B, prompt_len=None, head_quota=None, seed=0, tail=0, policy="static", xattn="full", passes=1,
           copy_rows=0, replay=0, replay_exclude=False):
    from abridgekv_amd import ops
    S0 = N * (C + passes * K + replay) + copy_rows
    g = torch.Generator().manual_seed(seed)
    q = torch.randn((B, S0, 32, 128), generator=g).to(torch.bfloat16)
    k = torch.randn((B, S0, 8, 128), generator=g).to(torch.bfloat16)
    v = torch.randn((B, S0, 8, 128), generator=g).to(torch.bfloat16)
    dout = torch.randn((B, S0, 32, 128), generator=g).to(torch.bfloat16)
    dev = torch.device("cuda")
    pl = None if prompt_len is None else torch.tensor(prompt_len, dtype=torch.int32, device=dev)
    hq = None if head_quota is None else torch.tensor(head_quota, dtype=torch.int32, device=dev)
    qd, kd, vd, gd = (t.to(dev) for t in (q, k, v, dout))
    lse = torch.empty((B, 32, S0), dtype=torch.float32, device=dev)
    out, _ = ops.prefill_masked_attention(qd, kd, vd, C, K, N, prompt_len=pl, head_quota=hq, lse=lse,
                                          retain_tail=tail, tail_policy=policy, pause_xattn=xattn,
                                          pause_passes=passes, copy_rows=copy_rows, replay_rows=replay,
                                          replay_exclude=replay_exclude)
    dq, dk, dv = ops.prefill_masked_attention_backward(qd, kd, vd, out, lse, gd, C, K, N, prompt_len=pl,
                                                       head_quota=hq, retain_tail=tail, tail_policy=policy,
                                                       pause_xattn=xattn, pause_passes=passes, copy_rows=copy_rows,
                                                       replay_rows=replay, replay_exclude=replay_exclude)
    torch.cuda.synchronize()
    got = [t.float().cpu().numpy() for t in (dq, dk, dv)]
    worst = 0.0
    for b in range(B):
        raw = policy == "raw"                   # the kernels' raw policy is the oracle's separate raw-tail term
        mask = op.arith_mask(C, K, N, None if prompt_len is None else [prompt_len[b]], head_quota,
                             retain_tail=0 if raw else tail, tail_policy="static" if raw else policy,
                             pause_xattn=xattn, passes=passes, copy_rows=copy_rows, replay=replay,
                             replay_exclude=replay_exclude, raw_tail=tail if raw else 0)
        if prompt_len is not None:
            mask = mask[0]
        ref = op.masked_attention_grads_fp64(q[b].float().numpy(), k[b].float().numpy(), v[b].float().numpy(), mask,
                                             128 ** -0.5, dout[b].float().numpy())
        for name, mine, r in zip("qkv", got, ref):
            assert np.isfinite(mine[b]).all(), name
            err = float(np.abs(mine[b] - r).max())
            bound = 2e-2 * float(np.abs(r).max()) + 2e-3
            print(f"d{name} b{b}: max err {err:.3e}, bound {bound:.3e}")
            assert err <= bound, (name, b, err, bound)
            worst = max(worst, err / bound)
    return worst


def test_aligned_no_prompt():
    _check(C=128, K=64, N=3, B=1)


def test_aligned_prompt_straddles_tiles():
    _check(C=128, K=64, N=3, B=2, prompt_len=[150, 320], seed=1)


def test_aligned_head_quotas():
    quota = np.repeat([64, 16, 40, 64, 1, 33, 64, 8], 4).tolist()
    _check(C=128, K=64, N=3, B=2, prompt_len=[100, 0], head_quota=quota, seed=2)


def test_unaligned_small_blocks_partial_tiles():
    """C=40, K=12: the per-element mask path; S0=208 leaves a partial query and key tile."""
    quota = np.repeat([12, 3, 7, 12, 1, 5, 9, 12], 4).tolist()
    _check(C=40, K=12, N=4, B=2, prompt_len=[50, 0], head_quota=quota, seed=3)


def test_static_tail_aligned_blocks():
    """Static retained tail T=32 on 64-aligned blocks: the dK/dV pair walk must reach every later query tile of an
    earlier block's tail keys, and a block's codes must give its own tail keys no gradient."""
    quota = np.repeat([64, 16, 40, 64, 1, 33, 64, 8], 4).tolist()
    _check(C=128, K=64, N=3, B=2, prompt_len=[100, 0], head_quota=quota, seed=5, tail=32)


def test_static_tail_unaligned_blocks():
    quota = np.repeat([12, 3, 7, 12, 1, 5, 9, 12], 4).tolist()
    _check(C=40, K=12, N=4, B=1, prompt_len=[45], head_quota=quota, seed=6, tail=7)


@pytest.mark.parametrize("policy", ["rolling", "sticky"])
@pytest.mark.parametrize("tail", [32, 100])
def test_window_tail_aligned_blocks(policy, tail):
    """Window tails on 64-aligned blocks: a block's tail keys get gradient from the next block's content rows only
    (rolling: from content row i for tail row >= i), and none from its own codes."""
    quota = np.repeat([64, 16, 40, 64, 1, 33, 64, 8], 4).tolist()
    print(f"case: {policy} T={tail}", flush=True)
    _check(C=128, K=64, N=3, B=2, prompt_len=[100, 0], head_quota=quota, seed=25, tail=tail, policy=policy)


@pytest.mark.parametrize("policy", ["rolling", "sticky"])
def test_window_tail_unaligned_blocks(policy):
    quota = np.repeat([12, 3, 7, 12, 1, 5, 9, 12], 4).tolist()
    _check(C=40, K=12, N=4, B=1, prompt_len=[45], head_quota=quota, seed=26, tail=7, policy=policy)


@pytest.mark.parametrize("xattn", ["causal", "none"])
def test_pause_xattn(xattn):
    quota = np.repeat([64, 16, 40, 64, 1, 33, 64, 8], 4).tolist()
    _check(C=128, K=64, N=3, B=2, prompt_len=[100, 0], head_quota=quota, seed=27, tail=20, policy="sticky",
           xattn=xattn)


@pytest.mark.parametrize("passes", [2, 3])
def test_pause_passes(passes):
    quota = np.repeat([64, 16, 40, 64, 1, 33, 64, 8], 4).tolist()
    _check(C=128, K=64, N=3, B=2, prompt_len=[100, 0], head_quota=quota, seed=28 + passes, tail=20,
           policy="rolling" if passes == 2 else "static", xattn="full" if passes == 2 else "causal", passes=passes)


def test_copy_region():
    quota = np.repeat([64, 16, 40, 64, 1, 33, 64, 8], 4).tolist()
    _check(C=128, K=64, N=3, B=2, head_quota=quota, seed=35, passes=2, copy_rows=129)


@pytest.mark.parametrize("exclude", [False, True])
def test_replay_rows(exclude):
    quota = np.repeat([64, 16, 40, 64, 1, 33, 64, 8], 4).tolist()
    _check(C=128, K=64, N=3, B=2, prompt_len=[100, 0], head_quota=quota, seed=40, replay=16, replay_exclude=exclude)


@pytest.mark.parametrize("W", [20, 128])
def test_raw_tail(W):
    """The raw tail (the rolling window that the codes also see), up to the whole block."""
    quota = np.repeat([64, 16, 40, 64, 1, 33, 64, 8], 4).tolist()
    print(f"case: raw W={W}", flush=True)
    _check(C=128, K=64, N=3, B=2, prompt_len=[100, 0], head_quota=quota, seed=41, tail=W, policy="raw")


@pytest.mark.parametrize("C,N", [(512, 1), (200, 2)])
def test_plain_causal_without_codes(C, N):
    _check(C=C, K=0, N=N, B=2, seed=36)


def test_autograd_through_hf_attention_layout():
    """The autograd function CompressLM's attention uses: [B, H, S, D] views in, gradients out in the same views."""
    from abridgekv_amd import compress_forward as cf
    from abridgekv_amd import ops
    C, K, N, B = 64, 64, 2, 1
    S0 = N * (C + K)
    dev = torch.device("cuda")
    g = torch.Generator(device=dev).manual_seed(4)
    q = torch.randn((B, 32, S0, 128), generator=g, device=dev).to(torch.bfloat16).requires_grad_()
    k = torch.randn((B, 8, S0, 128), generator=g, device=dev).to(torch.bfloat16).requires_grad_()
    v = torch.randn((B, 8, S0, 128), generator=g, device=dev).to(torch.bfloat16).requires_grad_()
    mask = cf.CompressMask(block_c=C, codes_k=K, num_blocks=N)
    module = type("M", (), {"layer_idx": 0})()
    out, _ = cf.masked_attention_forward(module, q, k, v, mask, scaling=ops.default_scale())
    dout = torch.randn(out.shape, generator=g, device=dev).to(torch.bfloat16)
    (out.float() * dout.float()).sum().backward()
    ref = op.masked_attention_grads_fp64(q.detach()[0].transpose(0, 1).float().cpu().numpy(),
                                         k.detach()[0].transpose(0, 1).float().cpu().numpy(),
                                         v.detach()[0].transpose(0, 1).float().cpu().numpy(),
                                         op.arith_mask(C, K, N), ops.default_scale(), dout[0].float().cpu().numpy())
    for t, r in zip((q, k, v), ref):
        mine = t.grad[0].transpose(0, 1).float().cpu().numpy()
        assert np.abs(mine - r).max() <= 2e-2 * np.abs(r).max() + 2e-3


def test_config4_geometry_full_oracle():
    """C=512 / K=128 blocks (tiles of the benched geometry), N=4, two sequences with different raw prompts; every
    gradient element against the full float64 oracle."""
    _check(C=512, K=128, N=4, B=2, prompt_len=[512, 300], seed=5)


@pytest.mark.parametrize("case", ["benched", "prompts_and_head_quotas"])
def test_config4_full_size_sampled(case):
    """The benched backward launch: B=4, N=16 blocks of [512 | 128] (S0=10240), 512-token raw prompts; and the same
    size with a different raw prompt per sequence and per-head code quotas. dq, dk, dv are finite everywhere; dq of
    sampled query rows (every sequence) and dk / dv of sampled keys of the last block (first and last sequence) match
    the float64 oracle (tolerance 2e-2 x the largest |reference| + 2e-3 per tensor)."""
    from abridgekv_amd import ops
    from tests.test_gpu_prefill import CONFIG4_QUOTAS, config4_sample_rows
    prompts, quota = ([512] * 4, None) if case == "benched" else ([512, 300, 0, 640], CONFIG4_QUOTAS)
    B, C, K, N = 4, 512, 128, 16
    S0 = N * (C + K)
    dev = torch.device("cuda")
    g = torch.Generator(device=dev).manual_seed(41)
    q = torch.randn((B, S0, 32, 128), generator=g, device=dev).to(torch.bfloat16)
    k = torch.randn((B, S0, 8, 128), generator=g, device=dev).to(torch.bfloat16)
    v = torch.randn((B, S0, 8, 128), generator=g, device=dev).to(torch.bfloat16)
    dout = torch.randn((B, S0, 32, 128), generator=g, device=dev).to(torch.bfloat16)
    pl = torch.tensor(prompts, dtype=torch.int32, device=dev)
    hq = None if quota is None else torch.tensor(quota, dtype=torch.int32, device=dev)
    lse = torch.empty((B, 32, S0), dtype=torch.float32, device=dev)
    out, _ = ops.prefill_masked_attention(q, k, v, C, K, N, prompt_len=pl, head_quota=hq, lse=lse)
    dq, dk, dv = ops.prefill_masked_attention_backward(q, k, v, out, lse, dout, C, K, N, prompt_len=pl,
                                                       head_quota=hq)
    torch.cuda.synchronize()
    for name, t in (("dq", dq), ("dk", dk), ("dv", dv)):
        assert torch.isfinite(t).all(), name
    rng = np.random.default_rng(5)
    scale = 128 ** -0.5
    last = (N - 1) * (C + K)
    keys = np.array([last, last + 1, last + 63, last + 64, last + 300, last + C - 1, last + C, last + C + 1,
                     last + C + 64, S0 - 1])

    def close(name, got, ref):
        err = float(np.abs(got - ref).max())
        bound = 2e-2 * float(np.abs(ref).max()) + 2e-3
        print(f"{name}: max err {err:.3e}, bound {bound:.3e}")
        assert err <= bound, (name, err, bound)

    for b in range(B):
        qb, kb, vb, gb = (t[b].float().cpu().numpy() for t in (q, k, v, dout))
        rows = config4_sample_rows(C, K, N, rng, extra=8)
        mrows = op.arith_mask_block(C, K, N, rows, np.arange(S0), [prompts[b]], quota)[0]
        close(f"dq b{b}", dq[b].float().cpu().numpy()[rows],
              op.masked_attention_query_grads_fp64(qb, kb, vb, gb, mrows, rows, scale))
        if b in (0, B - 1):
            def mask_fn(r, c, b=b):
                return op.arith_mask_block(C, K, N, r, c, [prompts[b]], quota)[0]
            ref_k, ref_v = op.masked_attention_key_grads_fp64(qb, kb, vb, gb, mask_fn, keys, scale)
            close(f"dk b{b}", dk[b].float().cpu().numpy()[keys], ref_k)
            close(f"dv b{b}", dv[b].float().cpu().numpy()[keys], ref_v)
