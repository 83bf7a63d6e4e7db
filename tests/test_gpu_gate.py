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
import torch.nn.functional as F

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


def _code_options(clm):
    """The oracle's view of a CompressLM's code-row projections (per layer), float64; None without any."""
    if not (clm.query_residual or clm.code_q_heads or clm.code_kv_heads):
        return None
    out = []
    for layer in clm.model.model.layers:
        a, cp = layer.self_attn, {}
        if clm.query_residual:
            cp["qres"] = a.q_proj.qres.detach().double().cpu()
        for name in ("q", "k", "v"):
            proj = getattr(a, name + "_proj")
            if hasattr(proj, "code"):
                cp[name] = (proj.code.weight.detach().double().cpu(),
                            None if proj.code.bias is None else proj.code.bias.detach().double().cpu())
        out.append(cp)
    return out


def _seeds(clm, base, ids, segment_mean=False):
    """The oracle's code inputs of every block, or None for the generic seeds."""
    if not (segment_mean or clm.seg_pool or clm.gated_seg_pool or clm.pool_init):
        return None
    tok = copy.deepcopy(base).double().model.embed_tokens(ids).detach()
    pool = None
    if clm.pool_init:
        pool = tuple(t.detach().double().cpu() for t in (clm.pool_q, clm.pool_k.weight, clm.pool_v.weight))
    gate = clm.seg_pool_gate.detach().double().cpu() if clm.gated_seg_pool else None
    return om.code_seeds(tok, clm.pause.detach().double().cpu(), clm.K, clm.code_excluded_tail,
                         segment_mean or clm.seg_pool or clm.gated_seg_pool, gate, pool)


def _gate(case, C, N, K, code_positions, prompt, quota, stepwise, T=0, policy="static", xattn="full", options=None,
          perturb=None, generator=True, teacher_forced=True, gen_options=None):
    from abridgekv_amd.compress_forward import CompressLM
    from abridgekv_amd.gen_compress import CompressGen

    hcq = None if quota is None else [list(q) if isinstance(q, list) else [q] * 8 for q in quota]
    per_head = hcq is not None and any(len(set(row)) > 1 for row in hcq)
    base = _model(case)
    dev = torch.device("cuda")
    tail = dict(retain_tail_kv=T, retain_tail_policy=policy) if T else {}
    clm = CompressLM(copy.deepcopy(base).to(dev), C, N, K, code_positions=code_positions,
                     head_code_quotas=hcq, pause_xattn=xattn, **tail, **(options or {})).eval()
    L = clm.L
    torch.manual_seed(100 + case)
    with torch.no_grad():
        clm.pause.normal_(0, 0.05)
        if perturb is not None:
            perturb(clm)
    ids = torch.randint(0, 257, (2, N, C))
    lhq = None if hcq is None else np.repeat(np.asarray(hcq), 4, axis=1)
    pause = clm.pause.detach().cpu()
    seg_mean = (gen_options or {}).get("code_init_override") == "segment_mean"
    seeds, proj = _seeds(clm, base, ids, seg_mean), _code_options(clm)
    # a raw tail: the model's, or the generator's override (then the generator alone is compared)
    W = (gen_options or {}).get("raw_tail_override", clm.raw_tail)
    kw = dict(retain_tail=T, tail_policy=policy, pause_xattn=xattn, passes=L, replay=clm.replay_tail,
              replay_exclude=clm.code_exclude_replay_tail, raw_tail=W)
    ref = om.dense_loss_logits(copy.deepcopy(base).double(), pause.double(), ids, C, N, K, code_positions, prompt,
                               lhq, seeds=seeds, code_proj=proj, **kw)
    eager = om.dense_loss_logits(base, pause.to(torch.bfloat16), ids, C, N, K, code_positions, prompt, lhq,
                                 seeds=seeds, code_proj=proj, **kw)
    tol = 2 * (eager - ref).abs().max().item() + 2e-3

    pl = None if prompt is None else torch.tensor(prompt, dtype=torch.int32, device=dev)
    if teacher_forced:
        tf = clm.loss_logits(ids.to(dev), pl).double().cpu()
        err_tf = (tf - ref).abs().max().item()
        print(f"case {case}: eager-bf16 {(eager - ref).abs().max().item():.3e}  teacher-forced {err_tf:.3e}")
        assert err_tf <= tol
    if not generator:
        return

    rows_per_seq = N * (C - 1)
    for bi in range(2):
        p = 0 if prompt is None else prompt[bi]
        g = CompressGen(clm, dev, raw_prompt_len=p, head_code_quotas=hcq,
                        max_tokens=N * (C + K + clm.replay_tail) + 16, **(gen_options or {}))
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
            # window tail, the raw tail's too: the last closed block only)
            first = 0 if policy == "static" and not W else blk
            tails = sum(min(T or W, (b + 1) * C - max(p, b * C)) for b in range(first, blk + 1) if (b + 1) * C > p) \
                if T or W else 0
            # the closed block's replay rows stay until the next block's content expires them
            tails += clm.replay_tail
            if per_head:
                assert g.resident_rows() == [kept_prompt + tails] * 2
                assert g.packed_rows() == [(blk + 1) * sum(row) for row in hcq]
            else:
                assert g.resident_rows() == [kept_prompt + tails + (blk + 1) * row[0]
                                             for row in (hcq or [[K], [K]])]
        err = (torch.cat(got) - ref[bi * rows_per_seq: (bi + 1) * rows_per_seq]).abs().max().item()
        print(f"case {case} seq {bi}: generator {err:.3e}")
        assert err <= tol


@pytest.mark.parametrize("case", range(len(CASES)))
def test_generator_and_teacher_forced_match_dense_forward(case):
    C, N, K, code_positions, prompt, quota, stepwise = CASES[case][:7]
    T = CASES[case][7] if len(CASES[case]) > 7 else 0
    policy = CASES[case][8] if len(CASES[case]) > 8 else "static"
    xattn = CASES[case][9] if len(CASES[case]) > 9 else "full"
    _gate(case, C, N, K, code_positions, prompt, quota, stepwise, T, policy, xattn)


def _perturb(**scales):
    """Move the options' parameters off their no-op initial values (zero gate / value map / residual, copied
    projections), so that each option changes the logits."""
    def apply(clm):
        for name, module in clm.named_modules():
            if name.endswith("_proj") and hasattr(module, "qres"):
                module.qres.normal_(0, scales.get("qres", 0.3))
            if name.endswith("_proj") and hasattr(module, "code"):
                module.code.weight.add_(torch.randn_like(module.code.weight) * scales.get("code", 0.02))
        if clm.gated_seg_pool:
            clm.seg_pool_gate.normal_(0, 1.0)
        if clm.pool_init:
            clm.pool_v.weight.normal_(0, 0.05)
    return apply


# the training options beyond the served configuration: (name, C, N, K, code positions, CompressLM options, prompt,
# quota per layer, whether the paged generator runs it too (it serves one pause pass), generator options)
OPTION_CASES = [
    ("two pause passes", 64, 3, 16, "appended", dict(L=2), [40, 100], [16, 4], False, None),
    ("three passes, causal codes, static tail", 64, 3, 16, "appended",
     dict(L=3, pause_xattn="causal", retain_tail_kv=12, retain_tail_policy="static"), [70, 0], None, False, None),
    ("segment-mean seeds, static tail", 64, 3, 16, "bitrev",
     dict(seg_pool=True, retain_tail_kv=12, retain_tail_policy="static"), [40, 100], [16, 4], True, None),
    ("gated segment means", 64, 3, 16, "bitrev", dict(gated_seg_pool=True), [40, 0], [16, 8], True, None),
    ("learned pooled seeds", 64, 3, 16, "bitrev", dict(pool_init=True), [40, 100], None, True, None),
    ("query residual", 64, 3, 16, "bitrev", dict(query_residual=True), [40, 100], [16, 4], True, None),
    ("code-row query projection", 64, 3, 16, "bitrev", dict(code_q_heads=True), [70, 0], [16, 4], True, None),
    ("code-row key/value projections, rolling tail", 64, 3, 16, "bitrev",
     dict(code_kv_heads=True, retain_tail_kv=12, retain_tail_policy="rolling"), [40, 100], [16, 4], True, None),
    ("segment-mean override of the generator", 64, 3, 16, "bitrev", {}, [40, 100], [16, 4], True,
     {"code_init_override": "segment_mean"}),
    ("replay tail", 64, 3, 16, "appended", dict(replay_tail=16), [40, 100], None, True, None),
    ("replay tail hidden from the codes, per-layer quotas", 64, 4, 16, "appended",
     dict(replay_tail=12, code_exclude_replay_tail=True), [70, 0], [16, 4], True, None),
    ("replay tail with per-head packed pages", 64, 3, 16, "appended", dict(replay_tail=16), [40, 100],
     [[1, 16, 3, 5, 2, 7, 4, 16], [8, 8, 1, 1, 12, 3, 9, 2]], True, None),
    ("replay tail hidden from the codes, two passes", 64, 3, 16, "appended",
     dict(replay_tail=12, code_exclude_replay_tail=True, L=2, seg_pool=True), [70, 0], [16, 4], False, None),
    ("raw tail", 64, 3, 16, "appended", dict(raw_tail=12, seg_pool=True), [40, 100], [16, 4], True, None),
    ("raw tail of the whole block", 64, 3, 16, "appended", dict(raw_tail=64), [70, 0], [16, 8], True, None),
    ("raw tail, two passes, causal codes", 64, 3, 16, "appended", dict(raw_tail=20, L=2, pause_xattn="causal"),
     [40, 100], None, False, None),
    ("raw-tail override of the generator", 64, 3, 16, "appended", {}, [40, 100], [16, 4], True,
     {"raw_tail_override": 20}),
]


@pytest.mark.parametrize("case", range(len(OPTION_CASES)), ids=[c[0] for c in OPTION_CASES])
def test_training_options_match_dense_forward(case):
    name, C, N, K, code_positions, options, prompt, quota, generator, gen_options = OPTION_CASES[case]
    options = dict(options)
    xattn = options.pop("pause_xattn", "full")
    T = options.pop("retain_tail_kv", 0)
    policy = options.pop("retain_tail_policy", "static")
    _gate(200 + case, C, N, K, code_positions, prompt, quota, [1], T, policy, xattn, options, _perturb(),
          generator=generator, teacher_forced=gen_options is None, gen_options=gen_options)


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


@pytest.mark.parametrize("tail,policy", [(0, "static"), (12, "static"), (12, "rolling"), (12, "sticky"),
                                         (12, "raw")])
def test_training_gradients_match_dense_float64(tail, policy):
    """CompressLM trains through the kernels: the CE loss's gradients (attention and MLP weights, the pause rows)
    through the masked-prefill forward + backward kernels match the dense float64 model's autograd, within 2x the
    error of the same dense model run in bf16 autograd (plus 1e-3 of the gradient's scale); also with a retained
    tail under each policy and with a raw tail (appended code positions)."""
    from abridgekv_amd.compress_forward import CompressLM

    C, N, K = 64, 3, 32 if tail else 64
    quota = [[32] * 8, [32, 16, 24, 32, 8, 32, 32, 24]] if tail else [[32] * 8, [64, 16, 48, 64, 8, 32, 64, 24]]
    base = _model(11)
    dev = torch.device("cuda")
    raw = policy == "raw"
    positions = "appended" if raw else "bitrev"
    extra = dict(raw_tail=tail) if raw else dict(retain_tail_kv=tail, retain_tail_policy=policy) if tail else {}
    clm = CompressLM(copy.deepcopy(base).to(dev), C, N, K, code_positions=positions, head_code_quotas=quota,
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
        logits = om.dense_loss_logits(m, pause, ids, C, N, K, positions, [70, 5], lhq,
                                      retain_tail=0 if raw else tail, tail_policy="static" if raw else policy,
                                      raw_tail=tail if raw else 0)
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


def test_training_option_gradients_match_dense_float64():
    """Gradients through two pause passes, a query residual, code-row key/value projections and gated segment-mean
    seeds (the kernels' per-element walk and the host-side option modules) against the dense float64 model's
    autograd, as test_training_gradients_match_dense_float64 bounds them."""
    from abridgekv_amd.compress_forward import CompressLM

    C, N, K, L = 64, 3, 16, 2
    quota = [[16] * 8, [16, 4, 8, 16, 2, 16, 12, 16]]
    base = _model(13)
    dev = torch.device("cuda")
    clm = CompressLM(copy.deepcopy(base).to(dev), C, N, K, L=L, head_code_quotas=quota, query_residual=True,
                     code_kv_heads=True, gated_seg_pool=True).eval()
    torch.manual_seed(14)
    with torch.no_grad():
        clm.pause.normal_(0, 0.05)
        _perturb()(clm)
    ids = torch.randint(0, 257, (2, N, C))
    resp = torch.ones((2, N, C), dtype=torch.long)
    resp.view(2, -1)[0, :70] = 0
    loss = clm(ids.to(dev), resp_mask=resp.to(dev), raw_prompt=True)["ce"]
    loss.backward()
    layers = clm.model.model.layers
    got = {"q0": layers[0].self_attn.q_proj.orig.weight.grad, "qres0": layers[0].self_attn.q_proj.qres.grad,
           "kcode1": layers[1].self_attn.k_proj.code.weight.grad, "vcode0": layers[0].self_attn.v_proj.code.weight.grad,
           "gate": clm.seg_pool_gate.grad, "pause": clm.pause.grad}
    got = {n: g.double().cpu() for n, g in got.items()}

    lhq = np.repeat(np.asarray(quota), 4, axis=1)
    keep = torch.from_numpy(np.array([k for k in range(N * C) if k % C != C - 1]))
    tgt = ids.view(2, -1)[:, keep + 1].reshape(-1)
    tm = resp.view(2, -1)[:, keep + 1].reshape(-1).double()

    def dense_grads(dtype):
        m = copy.deepcopy(base).to(dtype)
        leaf = lambda t: t.detach().cpu().to(dtype).requires_grad_()
        pause, gate = leaf(clm.pause), leaf(clm.seg_pool_gate)
        proj = []
        for layer in layers:
            a = layer.self_attn
            proj.append({"qres": leaf(a.q_proj.qres), "k": (leaf(a.k_proj.code.weight), None),
                         "v": (leaf(a.v_proj.code.weight), None)})
        tok = m.model.embed_tokens(ids)
        seeds = om.code_seeds(tok, pause, K, segment_mean=True, seg_gate=gate)
        logits = om.dense_loss_logits(m, pause, ids, C, N, K, "appended", [70, 0], lhq, passes=L, seeds=seeds,
                                      code_proj=proj)
        ce = torch.nn.functional.cross_entropy(logits.double(), tgt, reduction="none")
        ((ce * tm).sum() / tm.sum()).backward()
        params = dict(m.named_parameters())
        return {"q0": params["model.layers.0.self_attn.q_proj.weight"].grad.double(),
                "qres0": proj[0]["qres"].grad.double(), "kcode1": proj[1]["k"][0].grad.double(),
                "vcode0": proj[0]["v"][0].grad.double(), "gate": gate.grad.double(), "pause": pause.grad.double()}

    ref = dense_grads(torch.float64)
    eager = dense_grads(torch.bfloat16)
    for n in got:
        e_ours = (got[n] - ref[n]).abs().max().item()
        e_eager = (eager[n] - ref[n]).abs().max().item()
        scale = ref[n].abs().max().item()
        print(f"{n}: ours {e_ours:.3e}  eager-bf16 {e_eager:.3e}  scale {scale:.3e}")
        assert scale > 0, n
        assert e_ours <= 2 * e_eager + 1e-3 * scale, n


def _dense_plain_hidden(model, ids_flat):
    """Final-normed hidden states of the model's plain causal forward (eager attention), any dtype."""
    m = copy.deepcopy(model)
    m.config._attn_implementation = "eager"
    with torch.no_grad():
        return m.model(input_ids=ids_flat, use_cache=False).last_hidden_state


@pytest.mark.parametrize("L", [1, 2])
def test_forward_training_losses_match_dense(L):
    """CompressLM.forward's training losses beyond the plain CE against the dense model: the reference's own
    self-test call (distill_lambda=1, copy_lambda=1, distill_temp=2; compress_forward.py:1320-1329) with one and two
    passes, the full-context baseline (ceiling and floor), response-masked distillation from teacher logits, the
    chunked frozen-teacher KD, the representation loss and a prebuilt mask. Each loss within 2x the float64 error of
    the same dense computation in bf16, plus 1e-3."""
    from abridgekv_amd.compress_forward import CompressLM

    C, N, K, B = 64, 3, 16, 2
    base = _model(40 + L)
    dev = torch.device("cuda")
    clm = CompressLM(copy.deepcopy(base).to(dev), C, N, K, L=L).eval()
    torch.manual_seed(41)
    with torch.no_grad():
        clm.pause.normal_(0, 0.05)
        clm.copy_token.normal_(0, 0.05)
    ids = torch.randint(0, 257, (B, N, C))
    resp = torch.ones((B, N, C), dtype=torch.long)
    resp.view(B, -1)[0, :70] = 0
    pf = torch.from_numpy(np.array([k for k in range(N * C) if k % C != C - 1]))
    tgt = ids.view(B, -1)[:, pf + 1].reshape(-1)
    tm = resp.view(B, -1)[:, pf + 1].reshape(-1).double()
    teacher_hidden = torch.randn(2, B, N * C, 256) * 0.5
    g = torch.Generator().manual_seed(42)
    teacher_logits = torch.randn(B * (N * C - N), 257, generator=g, dtype=torch.float64)
    teacher_head = torch.nn.Linear(256, 257, bias=False).double()
    teacher_rows = torch.randn(B * (N * C - N), 256, generator=g, dtype=torch.float64)

    def dense(dtype):
        m = copy.deepcopy(base).to(dtype)
        pause, ctok = clm.pause.detach().cpu().to(dtype), clm.copy_token.detach().cpu().to(dtype)
        with torch.no_grad():
            h, layers = om.dense_hidden(m, pause, ids, C, N, K, passes=L, copy_token=ctok, output_layers=True)
            S0 = N * (C + L * K)
            logits = m.lm_head(h[:, om.loss_rows(C, N, K, L)].reshape(-1, 256)).double()
            full = m.lm_head(_dense_plain_hidden(m, ids.view(B, N * C))).double()[:, pf].reshape(-1, 257)
            out = {"ce": F.cross_entropy(logits, tgt),
                   "distill": F.kl_div(F.log_softmax(logits / 2, -1), F.softmax(full / 2, -1),
                                       reduction="batchmean") * 4,
                   "copy": F.cross_entropy(m.lm_head(h[:, S0:S0 + C]).double().reshape(-1, 257),
                                           ids[:, -1].reshape(-1))}
            ce_rows = F.cross_entropy(logits, tgt, reduction="none")
            kl_rows = F.kl_div(F.log_softmax(logits, -1), F.softmax(teacher_logits, -1), reduction="none").sum(-1)
            out["masked_ce"] = (ce_rows * tm).sum() / tm.sum()
            out["masked_distill"] = (kl_rows * tm).sum() / tm.sum()
            tl = teacher_head(teacher_rows)
            kd = (F.softmax(tl, -1) * (F.log_softmax(tl, -1) - F.log_softmax(logits, -1))).sum(-1)
            out["kd"] = (kd * tm).sum() / tm.sum()
            # representation loss on the content rows: layer 1's output and the final (normed) hidden state
            content = torch.from_numpy(np.array([r for r in range(S0) if r % (C + L * K) < C]))
            rep = 0.0
            for li, hs in enumerate([layers[0], h]):
                hs = hs[:, content].double()
                ht = teacher_hidden[li].double()
                hs = hs / hs.pow(2).mean(-1, keepdim=True).clamp_min(1e-12).sqrt()
                ht = ht / ht.pow(2).mean(-1, keepdim=True).clamp_min(1e-12).sqrt()
                rep = rep + (hs - ht).pow(2).mean()
            out["rep"] = rep / 2
            for G, name in ((N, "ceiling"), (1, "floor")):
                flat = ids.reshape(B * (N // G), G * C)
                ar = torch.arange(G * C)
                pos = ar[(ar % C) != C - 1]
                hb = _dense_plain_hidden(m, flat)[:, pos].reshape(-1, 256)
                out[name] = F.cross_entropy(m.lm_head(hb).double(), flat[:, pos + 1].reshape(-1))
        return out

    ref, eager = dense(torch.float64), dense(torch.bfloat16)
    idd = ids.to(dev)
    with torch.no_grad():
        main = clm(idd, distill_lambda=1.0, copy_lambda=1.0, distill_temp=2.0)
        masked = clm(idd, resp_mask=resp.to(dev), teacher_logits=teacher_logits.to(dev))
        kd = clm(idd, resp_mask=resp.to(dev), teacher_rows=teacher_rows.to(dev).float(),
                 teacher_head=copy.deepcopy(teacher_head).to(dev).float(), ce_chunk=50)
        rep = clm(idd, teacher_hidden=teacher_hidden.to(dev))
        ceiling = clm(idd, baseline=True)
        floor = clm(idd, baseline=True, ctx_blocks=1)
        prebuilt = clm(idd, blockmask=clm.compress_mask(B))
    got = {"ce": main["ce"], "distill": main["distill"], "copy": main["copy"], "masked_ce": masked["ce"],
           "masked_distill": masked["distill"], "kd": kd["distill"], "rep": rep["rep"], "ceiling": ceiling["ce"],
           "floor": floor["ce"]}
    for name, value in got.items():
        e_ours, e_eager = abs(float(value) - float(ref[name])), abs(float(eager[name]) - float(ref[name]))
        print(f"L={L} {name}: ours {float(value):.5f} ref {float(ref[name]):.5f} err {e_ours:.2e} eager {e_eager:.2e}")
        assert e_ours <= 2 * e_eager + 1e-3, name
    bound = 2 * abs(float(eager["masked_ce"] - ref["masked_ce"])) + 1e-3
    assert abs(float(kd["ce"]) - float(ref["masked_ce"])) <= bound
    assert float(prebuilt["ce"]) == float(rep["ce"])                       # the same mask, the same kernels
    # the reference's self-test step: the three losses train the codes
    clm.train()
    losses = clm(idd, distill_lambda=1.0, copy_lambda=1.0, distill_temp=2.0)
    (losses["ce"] + losses["distill"] + losses["copy"]).backward()
    assert torch.isfinite(clm.pause.grad).all() and clm.pause.grad.norm() > 0
    assert torch.isfinite(clm.copy_token.grad).all() and clm.copy_token.grad.norm() > 0
