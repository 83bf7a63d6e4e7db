"""The kernels' torch custom-op registrations (namespace ``abridgekv``), without a GPU: every op exists with the
mutation schema its in-place convention needs, and tracing a caller with fake CUDA tensors keeps each op as one
graph node (what torch.compile(fullgraph=True) needs; no kernel runs)."""
import torch
from torch._subclasses.fake_tensor import FakeTensorMode
from torch.fx.experimental.proxy_tensor import make_fx

from abridgekv_amd import torch_ops

MUTATES = {
    "decode_attn": {"out", "lse", "workspace"},
    "kv_append": {"kv_cache"},
    "rope_kv_append": {"q", "key", "kv_cache"},
    "slot_mapping": {"out"},
    "kv_move_segments": {"layer_caches"},
    "kv_move_mixed": {"layer_caches"},
    "moves_expand": {"out"},
    "paged_prefill_attn": {"out", "lse", "workspace"},
    "prefill_masked_attn": {"out", "lse"},
    "prefill_masked_attn_bwd": set(),
}


def test_every_op_is_registered_with_its_mutations():
    assert set(torch_ops.OPS) == set(MUTATES)
    for name, muts in MUTATES.items():
        schema = getattr(torch.ops.abridgekv, name).default._schema
        got = {a.name for a in schema.arguments if a.alias_info is not None and a.alias_info.is_write}
        assert got == muts, (name, got)
        assert (len(schema.returns) == 0) == (name != "prefill_masked_attn_bwd"), name


def test_fake_tracing_keeps_each_op_as_one_node():
    def caller(q, cache, bt, sl, out, lse, ws, key, val, slots, pos, cos_sin, req, comp, mv_ops, offs, tq0, tr,
               meta, pq, pk, pv, pout, plse):
        torch.ops.abridgekv.slot_mapping(req, pos, bt, comp, slots)
        torch.ops.abridgekv.rope_kv_append(q, key, val, pos, cos_sin, slots, cache, 64, 16, 500)
        torch.ops.abridgekv.kv_append(key, val, slots, cache)
        torch.ops.abridgekv.decode_attn(q, cache, bt, sl, 0.088, 8, 4, out, lse, ws)
        torch.ops.abridgekv.paged_prefill_attn(q, cache, bt, meta[:3], meta[3:5], meta[5:7], tr, tq0, meta[7:9],
                                               0.088, 4, 2, 1, out, lse, ws)
        torch.ops.abridgekv.kv_move_segments([cache], mv_ops, offs)
        torch.ops.abridgekv.kv_move_mixed([cache], mv_ops, offs, mv_ops)
        torch.ops.abridgekv.moves_expand(meta[:0], 0, meta, meta[:4], 4, offs, 2)
        torch.ops.abridgekv.prefill_masked_attn(pq, pk, pv, 8, 4, 2, None, None, 0.088, pout, plse)
        dq, dk, dv = torch.ops.abridgekv.prefill_masked_attn_bwd(pq, pk, pv, pout, plse, pout, 8, 4, 2, None, None,
                                                                0.088)
        return out.sum() + dq.float().sum() + dk.float().sum()

    with FakeTensorMode():
        d, bf, i32, i64 = "cuda", torch.bfloat16, torch.int32, torch.int64
        args = (torch.empty(2, 32, 128, device=d, dtype=bf), torch.empty(40, 2, 16, 8, 128, device=d, dtype=bf),
                torch.empty(2, 8, device=d, dtype=i32), torch.empty(2, device=d, dtype=i32),
                torch.empty(2, 32, 128, device=d, dtype=bf), torch.empty(2, 32, device=d),
                torch.empty(1 << 16, device=d, dtype=torch.uint8), torch.empty(2, 8, 128, device=d, dtype=bf),
                torch.empty(2, 8, 128, device=d, dtype=bf), torch.empty(2, device=d, dtype=i64),
                torch.empty(2, device=d, dtype=i64), torch.empty(600, 128, device=d),
                torch.empty(2, device=d, dtype=i32), torch.empty(2, device=d, dtype=i32),
                torch.empty(3, 4, device=d, dtype=i32), torch.empty(2, device=d, dtype=i32),
                torch.empty(1, device=d, dtype=i32), torch.empty(1, device=d, dtype=i32),
                torch.empty(9, device=d, dtype=i32), torch.empty(1, 24, 32, 128, device=d, dtype=bf),
                torch.empty(1, 24, 8, 128, device=d, dtype=bf), torch.empty(1, 24, 8, 128, device=d, dtype=bf),
                torch.empty(1, 24, 32, 128, device=d, dtype=bf), torch.empty(1, 32, 24, device=d))
        gm = make_fx(caller, tracing_mode="fake")(*args)
    targets = [str(n.target) for n in gm.graph.nodes if n.op == "call_function"]
    for name in torch_ops.OPS:
        assert sum(t.startswith(f"abridgekv.{name}.") for t in targets) == 1, (name, targets)
