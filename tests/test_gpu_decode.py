"""Decode attention on the GPU vs the fp64 oracle (tolerance: max-abs <= 2e-2 for bf16 outputs and for LSE)."""
import numpy as np
import pytest
import torch

from oracle import decode as od
from oracle import layout as ol

pytestmark = pytest.mark.gpu
TOL = 2e-2


def _bf16_round(x: np.ndarray) -> np.ndarray:
    return torch.from_numpy(np.asarray(x, np.float32)).to(torch.bfloat16).float().numpy()


def _paged_cache(rows_k, rows_v, num_pages, rng, garbage=50.0):
    """Place each sequence's rows at randomly chosen pages. Returns (cache [P,2,16,8,128] f32, tables, seq_lens)."""
    B = len(rows_k)
    seq_lens = [r.shape[0] for r in rows_k]
    need = [-(-n // 16) for n in seq_lens]
    pages = rng.permutation(np.arange(1, num_pages))[: sum(need)]
    W = max(max(need), 1)
    tables = np.zeros((B, W), np.int32)
    cache = rng.standard_normal((num_pages, 2, 16, 8, 128)).astype(np.float32) * garbage   # stale rows
    at = 0
    for b in range(B):
        tables[b, : need[b]] = pages[at: at + need[b]]
        at += need[b]
        pos = np.arange(seq_lens[b])
        cache[tables[b, pos // 16], 0, pos % 16] = rows_k[b]
        cache[tables[b, pos // 16], 1, pos % 16] = rows_v[b]
    return cache, tables, np.asarray(seq_lens, np.int32)


def _run(q, cache, tables, seq_lens, split_pages=32, max_pages=None):
    from abridgekv_amd import ops
    dev = torch.device("cuda")
    qd = torch.from_numpy(q).to(dev, torch.bfloat16)
    kvd = torch.from_numpy(cache).to(dev, torch.bfloat16)
    bt = torch.from_numpy(tables).to(dev)
    sl = torch.from_numpy(seq_lens).to(dev)
    lse = torch.empty((q.shape[0], 32), dtype=torch.float32, device=dev)
    out, _ = ops.decode_attention(qd, kvd, bt, sl, 128 ** -0.5, lse=lse,
                                  split_pages=split_pages, max_pages=max_pages)
    torch.cuda.synchronize()
    return out.float().cpu().numpy(), lse.cpu().numpy()


def _oracle(q, cache, tables, seq_lens):
    qb = _bf16_round(q)
    cb = _bf16_round(cache)
    return od.decode_paged_fp64(qb, cb, tables, seq_lens, 128 ** -0.5)


def config1_rows(seed=0, with_prompt=True):
    """Single-layer abridged decode, quota K=128: prompt 256 rows at 0..255, 4 closed blocks of C=512 starting at 256
    each keeping 128 code rows at 256 + 512 b + 4 * bitrev7(k), open block of 300 rows at 2304..2603, query at 2603.
    K/V/Q ~ N(0,1) from the seed, RoPE theta 1e6 at those positions."""
    rng = np.random.default_rng(seed)
    offs = ol.bitrev_code_offsets(128, 512)
    pos = list(range(256)) if with_prompt else []
    for b in range(4):
        pos += (256 + 512 * b + offs).tolist()
    pos += list(range(2304, 2604))
    pos = np.asarray(pos)
    n = pos.size
    k = rng.standard_normal((n, 8, 128))
    v = rng.standard_normal((n, 8, 128))
    q = rng.standard_normal((1, 32, 128))
    k = ol.rope_neox(k, pos)
    q = ol.rope_neox(q, np.array([2603]))
    return q, k, v


@pytest.mark.parametrize("with_prompt,rows", [(True, 1068), (False, 812)])
def test_config1_single_layer(with_prompt, rows):
    q, k, v = config1_rows(0, with_prompt)
    assert k.shape[0] == rows
    rng = np.random.default_rng(1)
    cache, tables, sl = _paged_cache([k], [v], 200, rng)
    out, lse = _run(q.astype(np.float32), cache, tables, sl)
    ref_out, ref_lse = _oracle(q, cache, tables, sl)
    assert np.abs(out - ref_out).max() <= TOL
    assert np.abs(lse - ref_lse).max() <= TOL


@pytest.mark.parametrize("split_pages", [2, 4, 32])
def test_ragged_batch_edges(split_pages):
    rng = np.random.default_rng(split_pages)
    lens = [1, 2, 15, 16, 17, 31, 32, 33, 63, 64, 65, 511, 512, 513, 1000, 2049]
    ks = [rng.standard_normal((n, 8, 128)) for n in lens]
    vs = [rng.standard_normal((n, 8, 128)) for n in lens]
    q = rng.standard_normal((len(lens), 32, 128)).astype(np.float32)
    cache, tables, sl = _paged_cache(ks, vs, 400, rng, garbage=np.nan)   # stale rows are NaN
    out, lse = _run(q, cache, tables, sl, split_pages=split_pages)
    ref_out, ref_lse = _oracle(q, cache, tables, sl)
    assert np.abs(out - ref_out).max() <= TOL
    assert np.abs(lse - ref_lse).max() <= TOL


def test_peaked_scores_and_large_magnitudes():
    """Scores spread over a wide range (online-softmax rescaling across chunks and splits)."""
    rng = np.random.default_rng(5)
    lens = [700, 1500, 40]
    ks = [rng.standard_normal((n, 8, 128)) * 4 for n in lens]
    for k in ks:
        k[-1] *= 3                              # the last row dominates late
    vs = [rng.standard_normal((n, 8, 128)) * 3 for n in lens]
    q = rng.standard_normal((3, 32, 128)).astype(np.float32)
    cache, tables, sl = _paged_cache(ks, vs, 300, rng)
    out, lse = _run(q, cache, tables, sl, split_pages=4)
    ref_out, ref_lse = _oracle(q, cache, tables, sl)
    assert np.abs(out - ref_out).max() <= 3 * TOL   # |v| up to ~12: bf16 output rounding scales with |out|
    assert np.abs(lse - ref_lse).max() <= TOL * 4


def test_values_beyond_fp16_range_in_split_partials():
    """Split partials are stored in fp16 divided by a per-(split, head) scale; V rows of magnitude ~1e6 (beyond fp16's
    65504, representable in bf16) must come out finite and as accurate, relative to that magnitude, as unit rows."""
    rng = np.random.default_rng(11)
    lens = [1500, 700, 64]
    big = 1.0e6
    ks = [rng.standard_normal((n, 8, 128)) for n in lens]
    vs = [rng.standard_normal((n, 8, 128)) * big for n in lens]
    vs[1][:, :4] /= big                         # KV heads 0-3 of the second sequence stay at unit scale
    q = rng.standard_normal((3, 32, 128)).astype(np.float32)
    cache, tables, sl = _paged_cache(ks, vs, 300, rng)
    out, lse = _run(q, cache, tables, sl, split_pages=4)
    ref_out, ref_lse = _oracle(q, cache, tables, sl)
    assert np.isfinite(out).all()
    err = np.abs(out - ref_out)
    assert err[1, :16].max() <= TOL                       # the unit-scale heads (query heads 0-15)
    assert err.max() <= TOL * big
    assert np.abs(lse - ref_lse).max() <= TOL


def test_zero_length_sequence_writes_zeros():
    rng = np.random.default_rng(2)
    ks = [rng.standard_normal((n, 8, 128)) for n in (0, 20)]
    vs = [rng.standard_normal((n, 8, 128)) for n in (0, 20)]
    q = rng.standard_normal((2, 32, 128)).astype(np.float32)
    cache, tables, sl = _paged_cache(ks, vs, 10, rng)
    out, lse = _run(q, cache, tables, sl, max_pages=2)
    assert np.all(out[0] == 0) and np.all(np.isneginf(lse[0]))
    ref_out, _ = _oracle(q[1:], cache, tables[1:], sl[1:])
    assert np.abs(out[1] - ref_out[0]).max() <= TOL


def test_strided_q_and_out():
    from abridgekv_amd import ops
    rng = np.random.default_rng(3)
    ks = [rng.standard_normal((n, 8, 128)) for n in (100, 300)]
    vs = [rng.standard_normal((n, 8, 128)) for n in (100, 300)]
    q = rng.standard_normal((2, 32, 128)).astype(np.float32)
    cache, tables, sl = _paged_cache(ks, vs, 40, rng)
    dev = torch.device("cuda")
    big = torch.zeros((2, 48, 128), dtype=torch.bfloat16, device=dev)
    big[:, 8:40] = torch.from_numpy(q).to(dev, torch.bfloat16)
    qv = big[:, 8:40]
    outbig = torch.zeros((2, 40, 128), dtype=torch.bfloat16, device=dev)
    ov = outbig[:, 4:36]
    ops.decode_attention(qv, torch.from_numpy(cache).to(dev, torch.bfloat16), torch.from_numpy(tables).to(dev),
                         torch.from_numpy(sl).to(dev), 128 ** -0.5, out=ov, split_pages=2)
    torch.cuda.synchronize()
    ref_out, _ = _oracle(q, cache, tables, sl)
    assert np.abs(ov.float().cpu().numpy() - ref_out).max() <= TOL
    assert torch.all(outbig[:, :4] == 0) and torch.all(outbig[:, 36:] == 0)


def test_single_row_table_with_zero_row_stride():
    """A one-row page table made as a numpy ``table[None]`` view has row stride 0 in torch; it must decode the same."""
    rng = np.random.default_rng(4)
    ks, vs = [rng.standard_normal((700, 8, 128))], [rng.standard_normal((700, 8, 128))]
    q = rng.standard_normal((1, 32, 128)).astype(np.float32)
    cache, tables, sl = _paged_cache(ks, vs, 80, rng)
    row = np.ascontiguousarray(tables[0])
    bt0 = torch.from_numpy(row[None])
    assert bt0.stride(0) == 0
    from abridgekv_amd import ops
    dev = torch.device("cuda")
    out, _ = ops.decode_attention(torch.from_numpy(q).to(dev, torch.bfloat16), torch.from_numpy(cache).to(dev, torch.bfloat16),
                                  bt0.to(dev), torch.from_numpy(sl).to(dev), 128 ** -0.5, split_pages=8)
    torch.cuda.synchronize()
    ref_out, _ = _oracle(q, cache, tables, sl)
    assert np.abs(out.float().cpu().numpy() - ref_out).max() <= TOL


def test_shape_errors_raise_before_launch():
    from abridgekv_amd import ops
    dev = torch.device("cuda")
    kv = torch.zeros((4, 2, 16, 8, 128), dtype=torch.bfloat16, device=dev)
    with pytest.raises(ValueError):
        ops.decode_attention(torch.zeros((1, 16, 128), dtype=torch.bfloat16, device=dev), kv,
                             torch.zeros((1, 2), dtype=torch.int32, device=dev),
                             torch.ones(1, dtype=torch.int32, device=dev), 0.1)
    with pytest.raises(ValueError):
        ops.decode_attention(torch.zeros((1, 32, 128), dtype=torch.bfloat16, device=dev), kv.float(),
                             torch.zeros((1, 2), dtype=torch.int32, device=dev),
                             torch.ones(1, dtype=torch.int32, device=dev), 0.1)


@pytest.mark.parametrize("seed", range(6))
def test_seeded_random_batches(seed):
    """Seeded random batches: sizes 1..40, lengths log-uniform in [1, 6000], split sizes of 2..48 pages, query scales
    0.1..4 (flat to peaked softmax), stale rows garbage; every sequence against the fp64 oracle."""
    rng = np.random.default_rng(1000 + seed)
    B = int(rng.integers(1, 41))
    lens = np.exp(rng.uniform(0, np.log(6000), B)).astype(int).clip(1, 6000).tolist()
    split = [2, 4, 6, 8, 16, 48, 64][seed % 7]
    scale = float(rng.choice([0.1, 1.0, 4.0]))
    ks = [rng.standard_normal((n, 8, 128)) for n in lens]
    vs = [rng.standard_normal((n, 8, 128)) for n in lens]
    q = (rng.standard_normal((B, 32, 128)) * scale).astype(np.float32)
    pages = sum(-(-n // 16) for n in lens) + 8
    cache, tables, sl = _paged_cache(ks, vs, pages, rng, garbage=30.0)
    print(f"case: seed {seed} B={B} max_len={max(lens)} split={split} q_scale={scale}", flush=True)
    out, lse = _run(q, cache, tables, sl, split_pages=split)
    ref_out, ref_lse = _oracle(q, cache, tables, sl)
    assert np.abs(out - ref_out).max() <= TOL
    assert np.abs(lse - ref_lse).max() <= TOL
