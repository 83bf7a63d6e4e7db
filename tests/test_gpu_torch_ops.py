"""The torch custom ops on the GPU: a caller compiled with torch.compile(fullgraph=True) and the same calls recorded
into a HIP graph and replayed compute bit-identically to the direct (ctypes) calls of abridgekv_amd.ops.

The compiled caller uses the aot_eager backend: dynamo traces the whole caller as one graph (fullgraph) and AOT
autograd functionalises the in-place ops, with no generated kernels around ours. Graph replays run with eager work and
synchronisations between them, each against a fresh eager result."""
import ctypes as C

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _inputs(seed=0):
    from abridgekv_amd import ops
    dev = torch.device("cuda")
    g = torch.Generator(device=dev).manual_seed(seed)
    rng = np.random.default_rng(seed)
    B, W, P = 6, 40, 400
    cache = torch.empty(ops.kv_cache_shape(P), dtype=torch.bfloat16, device=dev).normal_(generator=g)
    pages = torch.from_numpy(rng.permutation(np.arange(1, P))[:B * W].astype(np.int32).reshape(B, W)).to(dev)
    lens_h = rng.integers(100, W * 16 - 64, B).astype(np.int32)
    lens_h[0] = 500                                       # the code-step request: 372 rows + its 128 code rows
    lens = torch.from_numpy(lens_h).to(dev)
    d = dict(cache=cache, bt=pages, lens=lens,
             q=torch.randn((B, 32, 128), generator=g, device=dev).to(torch.bfloat16),
             key=torch.randn((B, 8, 128), generator=g, device=dev).to(torch.bfloat16),
             val=torch.randn((B, 8, 128), generator=g, device=dev).to(torch.bfloat16),
             pos=(lens.long() - 1).contiguous(), req=torch.arange(B, dtype=torch.int32, device=dev),
             comp=torch.zeros(B, dtype=torch.int32, device=dev),
             cos_sin=ops.rope_cos_sin_cache(W * 16, device=dev), ws=ops.decode_workspace(B, W, 8, device=dev))
    # a code step of one request (128 queries, key limit = start + 64) split over 3 key ranges
    Tq = 128
    d["cq"] = torch.randn((Tq, 32, 128), generator=g, device=dev).to(torch.bfloat16)
    kv0 = int(lens[0]) - Tq
    d["meta"] = torch.tensor([0, Tq, kv0, kv0 + 64, 0], dtype=torch.int32, device=dev)
    d["tiles"] = torch.tensor([[0, 0], [0, 64]], dtype=torch.int32, device=dev).T.contiguous()
    n_split, split_tiles = 3, -(-(-(-(kv0 + 64) // 64)) // 3)
    d["split"] = (n_split, split_tiles)
    d["cws"] = torch.empty(ops.lib().abkv_paged_prefill_workspace_size(Tq, n_split), dtype=torch.uint8, device=dev)
    # compaction moves: shift rows 64..95 of request 1 down by 32, as a compaction of [32, 64) does
    src = np.arange(64, 96)
    dst = src - 32
    bt1 = pages[1].cpu().numpy()
    mv = np.stack([bt1[src // 16], src % 16, bt1[dst // 16], dst % 16], 1).astype(np.int32)
    d["mv"] = torch.from_numpy(mv).to(dev)
    d["offs"] = torch.tensor([0, 32], dtype=torch.int32, device=dev)
    # a mixed move list: request 3 shifts rows 100..131 down by 16 (sources and destinations overlap: one ordered
    # segment), request 4 shifts rows 200..231 down by 64 (no overlap: 32 independent ops)
    def run(r, lo, shift):
        s_ = np.arange(lo, lo + 32)
        t_ = s_ - shift
        b = pages[r].cpu().numpy()
        return np.stack([b[s_ // 16], s_ % 16, b[t_ // 16], t_ % 16], 1)
    d["mx"] = torch.from_numpy(run(3, 100, 16).astype(np.int32)).to(dev)
    d["mx_free"] = torch.from_numpy(run(4, 200, 64).astype(np.int32)).to(dev)
    d["mx_offs"] = torch.tensor([0, 32], dtype=torch.int32, device=dev)
    # the planner's run descriptors of a step with two span removals (the device expansion of its move lists)
    from abridgekv_amd.planner import KVPlanner
    plan = KVPlanner(200, 1, 16, op_rows=False)
    plan.add_request(7)
    assert plan.allocate_slots(7, 1000) is not None
    plan.set_num_computed_tokens(7, 1000)
    assert plan.mask_token_span(7, 300, 340).success and plan.mask_token_span(7, 100, 164).success
    _, desc, (r_at, n_runs, p_at, g_at), _, n_el = plan.take_step_move_runs()
    dd = torch.from_numpy(desc.copy()).to(dev)
    d["mr_runs"], d["mr_pages"], d["mr_groups"] = dd[r_at: r_at + 30 * n_runs], dd[p_at: g_at], dd[g_at: g_at + 4]
    d["mr_n"] = n_el
    # masked prefill (C=64, K=16, N=3), 2 sequences, raw prompt 40 / 0
    S0 = 3 * 80
    d["pq"] = torch.randn((2, S0, 32, 128), generator=g, device=dev).to(torch.bfloat16)
    d["pk"] = torch.randn((2, S0, 8, 128), generator=g, device=dev).to(torch.bfloat16)
    d["pv"] = torch.randn((2, S0, 8, 128), generator=g, device=dev).to(torch.bfloat16)
    d["pl"] = torch.tensor([40, 0], dtype=torch.int32, device=dev)
    return d


def _outputs(d):
    dev = d["q"].device
    B = d["q"].shape[0]
    return dict(slots=torch.empty(B, dtype=torch.int64, device=dev), out=torch.empty_like(d["q"]),
                lse=torch.empty((B, 32), dtype=torch.float32, device=dev), cout=torch.empty_like(d["cq"]),
                clse=torch.empty((d["cq"].shape[0], 32), dtype=torch.float32, device=dev),
                pout=torch.empty_like(d["pq"]), plse=torch.empty((2, 32, d["pq"].shape[1]), device=dev),
                mvout=torch.empty(d["mr_n"], dtype=torch.int32, device=dev))


def _via_torch_ops(d, o):
    A = torch.ops.abridgekv
    scale = 128 ** -0.5
    A.slot_mapping(d["req"], d["pos"], d["bt"], d["comp"], o["slots"])
    A.rope_kv_append(d["q"], d["key"], d["val"], d["pos"], d["cos_sin"], o["slots"], d["cache"], 0, 0,
                     d["bt"].shape[1] * 16 - 1)
    A.kv_move_segments([d["cache"]], d["mv"], d["offs"])
    A.kv_move_mixed([d["cache"]], d["mx"], d["mx_offs"], d["mx_free"])
    A.moves_expand(d["mr_runs"], d["mr_runs"].numel() // 30, d["mr_pages"], d["mr_groups"], 4, o["mvout"], d["mr_n"])
    A.decode_attn(d["q"], d["cache"], d["bt"], d["lens"], scale, d["bt"].shape[1], 8, o["out"], o["lse"], d["ws"])
    m = d["meta"]
    A.paged_prefill_attn(d["cq"], d["cache"], d["bt"], m[0:2], m[2:3], m[3:4], d["tiles"][0], d["tiles"][1], m[4:5],
                         scale, d["cq"].shape[0], d["split"][0], d["split"][1], o["cout"], o["clse"], d["cws"])
    A.prefill_masked_attn(d["pq"], d["pk"], d["pv"], 64, 16, 3, d["pl"], None, scale, o["pout"], o["plse"])


def _via_ctypes(d, o):
    from abridgekv_amd import ops
    scale = 128 ** -0.5
    ops.slot_mapping(d["req"], d["pos"], d["bt"], out=o["slots"], compacted=d["comp"])
    ops.rope_kv_append(d["q"], d["key"], d["val"], d["pos"], d["cos_sin"], slot_mapping=o["slots"],
                       kv_cache=d["cache"], max_position=d["bt"].shape[1] * 16 - 1)
    ops.kv_move_segments([d["cache"]], d["mv"], d["offs"])
    ops.kv_move_mixed([d["cache"]], d["mx"], d["mx_offs"], d["mx_free"])
    r = d["mr_runs"]
    assert ops.lib().abkv_moves_expand(C.c_void_p(r.data_ptr()), r.numel() // 30, C.c_void_p(d["mr_pages"].data_ptr()),
                                       d["mr_pages"].numel(), C.c_void_p(d["mr_groups"].data_ptr()), 1, 4,
                                       C.c_void_p(o["mvout"].data_ptr()),
                                       d["mr_n"], C.c_void_p(torch.cuda.current_stream().cuda_stream)) == 0
    ops.decode_attention(d["q"], d["cache"], d["bt"], d["lens"], scale, out=o["out"], lse=o["lse"], split_pages=8,
                         workspace=d["ws"])
    m = d["meta"].cpu().numpy()
    ops.paged_prefill_attention(d["cq"], d["cache"], d["bt"], m[0:2], m[2:3], m[3:4], False, scale, out=o["cout"],
                                lse=o["clse"], split=d["split"][0])
    ops.prefill_masked_attention(d["pq"], d["pk"], d["pv"], 64, 16, 3, prompt_len=d["pl"], scale=scale,
                                 out=o["pout"], lse=o["plse"])


def _same(a, b):
    for k in a:
        assert torch.equal(a[k], b[k]), k


def _clone(d):
    return {k: (v.clone() if isinstance(v, torch.Tensor) else v) for k, v in d.items()}


def test_compiled_caller_matches_ctypes_bitwise():
    import abridgekv_amd  # noqa: F401  (registers the ops)
    d = _inputs(0)
    ref_d, got_d = _clone(d), _clone(d)
    ref_o, got_o = _outputs(d), _outputs(d)
    _via_ctypes(ref_d, ref_o)
    compiled = torch.compile(_via_torch_ops, fullgraph=True, backend="aot_eager")
    compiled(got_d, got_o)
    torch.cuda.synchronize()
    _same(ref_o, got_o)
    for k in ("cache", "q", "key"):                       # in-place results (cache rows, rotated q / key)
        assert torch.equal(ref_d[k], got_d[k]), k


def test_hip_graph_replays_match_ctypes_bitwise():
    import abridgekv_amd  # noqa: F401
    d = _inputs(1)
    snapshot = _clone(d)
    o = _outputs(d)
    _via_torch_ops(_clone(snapshot), _outputs(d))         # warm-up outside the capture
    torch.cuda.synchronize()
    stream = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        with torch.cuda.graph(graph, stream=stream):
            _via_torch_ops(d, o)
    torch.cuda.synchronize()
    gen = torch.Generator(device="cuda").manual_seed(5)
    for rep in range(3):
        # eager work between replays: fresh inputs into the captured buffers (new queries each time)
        for k in ("cache", "key", "val", "pq", "pk", "pv"):
            d[k].copy_(snapshot[k])
        for k in ("q", "cq"):
            d[k].copy_(torch.randn(d[k].shape, generator=gen, device="cuda").to(torch.bfloat16))
        ref_d = _clone(d)
        ref_o = _outputs(d)
        _via_ctypes(ref_d, ref_o)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        _same(ref_o, o)
        assert torch.equal(ref_d["cache"], d["cache"]), rep
