"""End-to-end gate on a random model with Qwen3-4B's attention shape (32 query heads, 8 KV heads, head size 128):
the teacher-forced forward (masked-prefill kernel) and the incremental paged generator (decode / chunk / code-step
kernels, planner compaction, row mover) must both reproduce the dense float64 teacher-forced forward, as the
reference's gate requires of its generator (gen_compress.py:1189-1378).

Tolerance: our bf16 paths may differ from the float64 oracle by at most 2x what the same model in plain PyTorch
bf16 (dense masks, CPU) differs by, plus 2e-3 (logits here are O(0.3))."""
import copy

import numpy as np
import pytest
import torch

from oracle import model as om

pytestmark = pytest.mark.gpu
transformers = pytest.importorskip("transformers")

CASES = [
    # C, N, K, code positions, prompt lengths, quota per layer (an int, or 8 per KV head; None: all K),
    # token-by-token sequences
    (64, 4, 16, "bitrev", [40, 100], [16, 4], [1]),
    (32, 3, 8, "appended", None, None, [0]),
    (64, 3, 32, "bitrev", [64, 0], [8, 32], [0, 1]),
    # per-head quotas: closed blocks' codes live in per-head packed pages
    (64, 3, 16, "bitrev", [40, 100], [[1, 16, 3, 5, 2, 7, 4, 16], [8, 8, 1, 1, 12, 3, 9, 2]], [1]),
    # a static retained tail of 12 rows with per-layer quotas (and one with per-head packed pages): every closed
    # block's last 12 content rows stay resident; the codes neither see nor span them
    (64, 4, 16, "bitrev", [40, 100], [16, 4], [1], 12),
    (64, 3, 16, "bitrev", [70, 0], [[1, 16, 3, 5, 2, 7, 4, 16], [8, 8, 1, 1, 12, 3, 9, 2]], [0], 12),
    # window tails (per-layer quotas): the previous block's last 12 content rows for the block's content only --
    # rolling (content token i sees tail rows i..; fed token by token and as whole blocks split at each expiry) and
    # sticky (all 12 until the block's codes)
    (64, 4, 16, "bitrev", [40, 100], [16, 4], [1], 12, "rolling"),
    (64, 4, 16, "bitrev", [40, 100], [16, 4], [0], 12, "sticky"),
    # code rows attending their own block's codes causally, or not at all (gen_compress.py:953-959, the reference
    # gate's xattn="causal" case), the second with a rolling tail
    (64, 3, 16, "bitrev", [40, 100], [16, 4], [1], 0, "static", "causal"),
    (64, 3, 16, "bitrev", [70, 0], [8, 16], [0], 12, "rolling", "none"),
]


def _model(seed):
    torch.manual_seed(seed)
    cfg = transformers.Qwen3Config(vocab_size=257, hidden_size=256, intermediate_size=512, num_hidden_layers=2,
                                   num_attention_heads=32, num_key_value_heads=8, head_dim=128,
                                   max_position_embeddings=4096,
                                   rope_parameters={"rope_theta": 1e6, "rope_type": "default"})
    cfg._attn_implementation = "eager"
    return transformers.Qwen3ForCausalLM(cfg).to(torch.bfloat16).eval()


@pytest.mark.parametrize("case", range(len(CASES)))
def test_generator_and_teacher_forced_match_dense_forward(case):
    from abridgekv_amd.compress_forward import CompressLM
    from abridgekv_amd.gen_compress import CompressGen

    C, N, K, code_positions, prompt, quota, stepwise = CASES[case][:7]
    T = CASES[case][7] if len(CASES[case]) > 7 else 0
    policy = CASES[case][8] if len(CASES[case]) > 8 else "static"
    xattn = CASES[case][9] if len(CASES[case]) > 9 else "full"
    hcq = None if quota is None else [list(q) if isinstance(q, list) else [q] * 8 for q in quota]
    per_head = hcq is not None and any(len(set(row)) > 1 for row in hcq)
    base = _model(case)
    dev = torch.device("cuda")
    tail = dict(retain_tail_kv=T, retain_tail_policy=policy) if T else {}
    clm = CompressLM(copy.deepcopy(base).to(dev), C, N, K, code_positions=code_positions,
                     head_code_quotas=hcq, pause_xattn=xattn, **tail).eval()
    torch.manual_seed(100 + case)
    with torch.no_grad():
        clm.pause.normal_(0, 0.05)
    ids = torch.randint(0, 257, (2, N, C))
    lhq = None if hcq is None else np.repeat(np.asarray(hcq), 4, axis=1)
    pause = clm.pause.detach().cpu()

    ref = om.dense_loss_logits(copy.deepcopy(base).double(), pause.double(), ids, C, N, K, code_positions, prompt,
                               lhq, retain_tail=T, tail_policy=policy, pause_xattn=xattn)
    eager = om.dense_loss_logits(base, pause.to(torch.bfloat16), ids, C, N, K, code_positions, prompt, lhq,
                                 retain_tail=T, tail_policy=policy, pause_xattn=xattn)
    tol = 2 * (eager - ref).abs().max().item() + 2e-3

    pl = None if prompt is None else torch.tensor(prompt, dtype=torch.int32, device=dev)
    tf = clm.loss_logits(ids.to(dev), pl).double().cpu()
    err_tf = (tf - ref).abs().max().item()
    print(f"case {case}: eager-bf16 {(eager - ref).abs().max().item():.3e}  teacher-forced {err_tf:.3e}")
    assert err_tf <= tol

    rows_per_seq = N * (C - 1)
    for bi in range(2):
        p = 0 if prompt is None else prompt[bi]
        g = CompressGen(clm, dev, raw_prompt_len=p, head_code_quotas=hcq, max_tokens=N * (C + K) + 16)
        got = []
        for blk in range(N):
            toks = ids[bi, blk].tolist()
            if bi in stepwise:
                hs = torch.cat([g.feed_content([t]) for t in toks])
            else:
                hs = g.feed_content(toks)
            got.append(clm.model.lm_head(hs).float()[: C - 1].double().cpu())
            g.compress()
            kept_prompt = min(p, (blk + 1) * C)
            # each closed block also keeps the part of its last T content rows that lies past the raw prompt (a
            # window tail: the last closed block only)
            first = 0 if policy == "static" else blk
            tails = sum(min(T, (b + 1) * C - max(p, b * C)) for b in range(first, blk + 1) if (b + 1) * C > p) \
                if T else 0
            if per_head:
                assert g.resident_rows() == [kept_prompt + tails] * 2
                assert g.packed_rows() == [(blk + 1) * sum(row) for row in hcq]
            else:
                assert g.resident_rows() == [kept_prompt + tails + (blk + 1) * row[0]
                                             for row in (hcq or [[K], [K]])]
        err = (torch.cat(got) - ref[bi * rows_per_seq: (bi + 1) * rows_per_seq]).abs().max().item()
        print(f"case {case} seq {bi}: generator {err:.3e}")
        assert err <= tol


def test_forward_losses_match_dense_cross_entropy():
    from abridgekv_amd.compress_forward import CompressLM

    C, N, K = 64, 3, 16
    base = _model(7)
    dev = torch.device("cuda")
    clm = CompressLM(copy.deepcopy(base).to(dev), C, N, K, code_positions="bitrev").eval()
    ids = torch.randint(0, 257, (2, N, C))
    resp = torch.ones((2, N, C), dtype=torch.long)
    resp.view(2, -1)[0, :70] = 0
    resp.view(2, -1)[1, :5] = 0
    pause = clm.pause.detach().cpu().double()
    ref = om.dense_loss_logits(copy.deepcopy(base).double(), pause, ids, C, N, K, "bitrev", [70, 5])
    tgt = ids.view(2, -1)[:, torch.from_numpy(np.array([k for k in range(N * C) if k % C != C - 1])) + 1]
    ce = torch.nn.functional.cross_entropy(ref, tgt.reshape(-1), reduction="none")
    tm = resp.view(2, -1)[:, torch.from_numpy(np.array([k for k in range(N * C) if k % C != C - 1])) + 1]
    tm = tm.reshape(-1).double()
    want = (ce * tm).sum() / tm.sum()
    with torch.no_grad():
        got = clm(ids.to(dev), resp_mask=resp.to(dev), raw_prompt=True)["ce"].item()
        blk = clm(ids.to(dev), resp_mask=resp.to(dev), raw_prompt=True, block_ce=True)
    assert abs(got - want.item()) <= 1e-2
    assert blk["block_ce"].shape == (N,)


@pytest.mark.parametrize("tail,policy", [(0, "static"), (12, "static"), (12, "rolling"), (12, "sticky")])
def test_training_gradients_match_dense_float64(tail, policy):
    """CompressLM trains through the kernels: the CE loss's gradients (attention and MLP weights, the pause rows)
    through the masked-prefill forward + backward kernels match the dense float64 model's autograd, within 2x the
    error of the same dense model run in bf16 autograd (plus 1e-3 of the gradient's scale); also with a retained
    tail under each policy."""
    from abridgekv_amd.compress_forward import CompressLM

    C, N, K = 64, 3, 32 if tail else 64
    quota = [[32] * 8, [32, 16, 24, 32, 8, 32, 32, 24]] if tail else [[32] * 8, [64, 16, 48, 64, 8, 32, 64, 24]]
    base = _model(11)
    dev = torch.device("cuda")
    extra = dict(retain_tail_kv=tail, retain_tail_policy=policy) if tail else {}
    clm = CompressLM(copy.deepcopy(base).to(dev), C, N, K, code_positions="bitrev", head_code_quotas=quota,
                     **extra).eval()
    torch.manual_seed(12)
    with torch.no_grad():
        clm.pause.normal_(0, 0.05)
    ids = torch.randint(0, 257, (2, N, C))
    resp = torch.ones((2, N, C), dtype=torch.long)
    resp.view(2, -1)[0, :70] = 0
    resp.view(2, -1)[1, :5] = 0
    loss = clm(ids.to(dev), resp_mask=resp.to(dev), raw_prompt=True)["ce"]
    loss.backward()
    names = ["model.layers.0.self_attn.q_proj.weight", "model.layers.0.self_attn.k_proj.weight",
             "model.layers.1.self_attn.v_proj.weight", "model.layers.1.self_attn.o_proj.weight",
             "model.layers.0.mlp.up_proj.weight"]
    ours = dict(clm.model.named_parameters())
    got = {n: ours[n].grad.double().cpu() for n in names}
    got["pause"] = clm.pause.grad.double().cpu()

    lhq = np.repeat(np.asarray(quota), 4, axis=1)
    keep = torch.from_numpy(np.array([k for k in range(N * C) if k % C != C - 1]))
    tgt = ids.view(2, -1)[:, keep + 1].reshape(-1)
    tm = resp.view(2, -1)[:, keep + 1].reshape(-1).double()

    def dense_grads(dtype):
        m = copy.deepcopy(base).to(dtype)
        pause = clm.pause.detach().cpu().to(dtype).requires_grad_()
        logits = om.dense_loss_logits(m, pause, ids, C, N, K, "bitrev", [70, 5], lhq, retain_tail=tail,
                                      tail_policy=policy)
        ce = torch.nn.functional.cross_entropy(logits.double(), tgt, reduction="none")
        ((ce * tm).sum() / tm.sum()).backward()
        params = dict(m.named_parameters())
        out = {n: params[n].grad.double() for n in names}
        out["pause"] = pause.grad.double()
        return out

    ref = dense_grads(torch.float64)
    eager = dense_grads(torch.bfloat16)
    for n in got:
        e_ours = (got[n] - ref[n]).abs().max().item()
        e_eager = (eager[n] - ref[n]).abs().max().item()
        scale = ref[n].abs().max().item()
        print(f"{n}: ours {e_ours:.3e}  eager-bf16 {e_eager:.3e}  scale {scale:.3e}")
        assert e_ours <= 2 * e_eager + 1e-3 * scale, n
