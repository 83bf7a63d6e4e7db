"""Attention backend host logic (no GPU): the code-step mask restatement, its conversion into per-request key
limits, and metadata validation."""
from types import SimpleNamespace

import numpy as np
import pytest
import torch

from abridgekv_amd import backend as bk
from oracle import masks as om


def test_oracle_causal_mask_is_shifted_tril():
    for ql, sl in [(1, 1), (5, 5), (3, 9), (7, 40)]:
        m = om.request_mask(ql, sl, [], None, 256, 256, causal=True)
        assert np.array_equal(m, np.tril(np.ones((ql, sl), bool), k=sl - ql))


@pytest.mark.parametrize("quota", [1, 2, 64, 128, 255, 256])
def test_oracle_code_mask_is_prefix_below_code_start_plus_quota(quota):
    """Physical quotas on the code step: queries = the block's K=256 code rows at the end; keys < start + q."""
    K, resident = 256, 700
    sl = resident + K
    m = om.request_mask(K, sl, [(resident, sl)], None, quota, K, causal=False)
    expect = np.broadcast_to(np.arange(sl) < resident + min(quota, K), (K, sl))
    assert np.array_equal(m, expect)


def test_oracle_mask_exclusion_and_several_spans_brute_force():
    rng = np.random.default_rng(0)
    for _ in range(20):
        sl = int(rng.integers(20, 60))
        ql = int(rng.integers(1, 8))
        causal = bool(rng.integers(2))
        cuts = np.sort(rng.choice(np.arange(sl - ql), 4, replace=False))
        spans = [(int(cuts[0]), int(cuts[1])), (int(cuts[2]), int(cuts[3]))]
        ex = (1, 3) if rng.integers(2) else None
        q, K = int(rng.integers(0, 6)), 4
        hidden = set()
        if q < K:
            for s, e in spans:
                hidden |= set(range(s + q, e))
        if ex is not None:
            hidden |= set(range(*ex))
        m = om.request_mask(ql, sl, spans, ex, q, K, causal)
        for i in range(ql):
            vis = {c for c in range(sl) if (c <= sl - ql + i or not causal)} - hidden
            assert set(np.flatnonzero(m[i]).tolist()) == vis


def _mixed_batch(rng):
    """Requests (query_len, seq_len, code_span or None, causal) of one group in one step."""
    reqs = []
    for _ in range(int(rng.integers(1, 6))):
        kind = int(rng.integers(3))
        if kind == 0:                          # code step: 16 code rows after a resident prefix
            res = int(rng.integers(0, 90))
            reqs.append((16, res + 16, (res, res + 16), False))
        elif kind == 1:                        # causal chunk after some context
            ql = int(rng.integers(1, 30))
            reqs.append((ql, ql + int(rng.integers(0, 50)), None, True))
        else:                                  # decode
            reqs.append((1, int(rng.integers(1, 80)), None, True))
    return reqs


@pytest.mark.parametrize("quota", [1, 5, 16, 40])
def test_custom_mask_converts_to_code_step_limits(quota):
    K = 16
    rng = np.random.default_rng(quota)
    for _ in range(10):
        reqs = _mixed_batch(rng)
        flat = np.concatenate([om.request_mask(ql, sl, [span] if span else [], None, quota, K, causal).reshape(-1)
                               for ql, sl, span, causal in reqs])
        qsl = np.concatenate([[0], np.cumsum([r[0] for r in reqs])])
        sls = [r[1] for r in reqs]
        limits, causal = bk.limits_from_custom_mask(torch.from_numpy(flat), qsl, sls)
        expect = bk.code_step_key_limits(qsl, sls, [r[2] for r in reqs], quota, K)
        for r, (ql, sl, span, c) in enumerate(reqs):
            if span is not None:
                assert limits[r] == expect[r] and not causal[r]
            elif ql > 1:
                assert causal[r] and limits[r] == sl
            else:                              # one query row: the causal row is the full prefix
                assert limits[r] == sl


@pytest.mark.parametrize("quota", [1, 5, 16])
def test_custom_mask_with_static_tail_converts_to_limits_and_excluded_ranges(quota):
    """The reference's code-step mask with a static retained tail (compresslm_masks.py:206-213: the block's own tail
    rows hidden from its codes) converts to the same key limit plus an excluded range, and code_step_excluded_ranges
    accepts exactly the ranges the worker accepts (gpu_model_runner.py:2086-2091)."""
    K, T = 16, 6
    rng = np.random.default_rng(10 + quota)
    for _ in range(10):
        reqs = _mixed_batch(rng)
        ex = [(span[0] - T, span[0]) if span is not None and span[0] >= T + 2 else None
              for _, _, span, _ in reqs]
        flat = np.concatenate([om.request_mask(ql, sl, [span] if span else [], e, quota, K, causal).reshape(-1)
                               for (ql, sl, span, causal), e in zip(reqs, ex)])
        qsl = np.concatenate([[0], np.cumsum([r[0] for r in reqs])])
        sls = [r[1] for r in reqs]
        limits, causal, excluded = bk.key_ranges_from_custom_mask(torch.from_numpy(flat), qsl, sls)
        expect = bk.code_step_key_limits(qsl, sls, [r[2] for r in reqs], quota, K)
        expect_ex = bk.code_step_excluded_ranges([r[2] for r in reqs], ex, qsl, sls)
        for r, (ql, sl, span, c) in enumerate(reqs):
            if span is not None:
                assert limits[r] == expect[r] and not causal[r]
                got = None if excluded is None or excluded[r, 1] == 0 else tuple(excluded[r])
                assert got == ex[r]
                if ex[r] is not None:
                    assert tuple(expect_ex[r]) == ex[r]
        if any(e is not None for e in ex):
            with pytest.raises(RuntimeError, match="prefix"):
                bk.limits_from_custom_mask(torch.from_numpy(flat), qsl, sls)
    with pytest.raises(RuntimeError, match="exclusion"):           # must end before the query rows
        bk.code_step_excluded_ranges([(16, 20)], [(14, 17)], [0, 4], [20])
    with pytest.raises(RuntimeError, match="not coding"):
        bk.code_step_excluded_ranges([None], [(2, 4)], [0, 1], [9])
    m = np.ones((2, 9), bool)
    m[:, 1] = m[:, 4] = False                                        # two hidden ranges: not runnable
    with pytest.raises(RuntimeError, match="more than one"):
        bk.key_ranges_from_custom_mask(torch.from_numpy(m.reshape(-1)), [0, 2], [9])


def test_custom_mask_rejects_non_prefix_masks():
    m = np.ones((2, 5), bool)
    m[0, 2] = False
    with pytest.raises(RuntimeError):
        bk.limits_from_custom_mask(torch.from_numpy(m.reshape(-1)), [0, 2], [5])
    m = np.zeros((3, 5), bool)
    m[0, :1], m[1, :3], m[2, :2] = True, True, True
    with pytest.raises(RuntimeError):
        bk.limits_from_custom_mask(torch.from_numpy(m.reshape(-1)), [0, 3], [5])
    with pytest.raises(RuntimeError):
        bk.limits_from_custom_mask(torch.ones(9, dtype=torch.bool), [0, 2], [5])


def test_code_step_limits_validate_spans():
    assert list(bk.code_step_key_limits([0, 1, 5], [9, 20], [None, (16, 20)], 2, 4)) == [bk.NOT_CODE, 18]
    assert list(bk.code_step_key_limits([0, 4], [20], [(16, 20)], 256, 4)) == [20]
    with pytest.raises(RuntimeError):
        bk.code_step_key_limits([0, 4], [20], [(15, 19)], 2, 4)      # not the request's own query rows
    with pytest.raises(RuntimeError):
        bk.code_step_key_limits([0, 4], [20], [(18, 22)], 2, 4)


def test_metadata_builder_validation():
    b = bk.AbridgeMetadataBuilder(max_num_seqs=4, max_pages=8, device="cpu")
    b._workspace = torch.empty(0)                      # keep the CPU test off the native library
    bt = torch.zeros((4, 8), dtype=torch.int32)
    sm = torch.zeros(8, dtype=torch.int64)
    md = b.build([0, 1, 2, 6], [10, 30, 40], bt, sm, seq_lens_dev=torch.zeros(3, dtype=torch.int32))
    assert (md.num_decodes, md.num_decode_tokens, md.num_actual_tokens, md.max_decode_pages) == (2, 2, 6, 2)
    with pytest.raises(RuntimeError):                  # a decode after a chunk
        b.build([0, 4, 5], [10, 30], bt, sm, seq_lens_dev=torch.zeros(2, dtype=torch.int32))
    with pytest.raises(RuntimeError):                  # past the table width
        b.build([0, 1], [129], bt, sm, seq_lens_dev=torch.zeros(1, dtype=torch.int32))
    with pytest.raises(RuntimeError):                  # code limit outside the query rows
        b.build([0, 4], [20], bt, sm, code_key_limit=[10], seq_lens_dev=torch.zeros(1, dtype=torch.int32))
    with pytest.raises(RuntimeError):
        b.build([0] * 6, [1] * 5, bt, sm)
    md = b.build([0, 4], [20], bt, sm, code_key_limit=[18], seq_lens_dev=torch.zeros(1, dtype=torch.int32))
    assert md.num_decodes == 0 and md.workspace is None and md.code_excluded is None
    md = b.build([0, 4], [20], bt, sm, code_key_limit=[18], seq_lens_dev=torch.zeros(1, dtype=torch.int32),
                 code_excluded=[[10, 16]])
    assert md.code_excluded.tolist() == [[10, 16]]
    with pytest.raises(RuntimeError):                  # the excluded range reaches into the query rows
        b.build([0, 4], [20], bt, sm, code_key_limit=[18], seq_lens_dev=torch.zeros(1, dtype=torch.int32),
                code_excluded=[[10, 17]])
    with pytest.raises(RuntimeError):                  # only code-step requests carry one
        b.build([0, 4], [20], bt, sm, seq_lens_dev=torch.zeros(1, dtype=torch.int32), code_excluded=[[10, 12]])
    md = b.build([0, 4], [20], bt, sm, code_key_limit=[18], seq_lens_dev=torch.zeros(1, dtype=torch.int32),
                 code_causal=[True])                   # a causal code step (pause_xattn="causal" of the generator)
    assert md.code_causal.tolist() == [True]
    with pytest.raises(RuntimeError):                  # only code-step requests may be causal code steps
        b.build([0, 4], [20], bt, sm, seq_lens_dev=torch.zeros(1, dtype=torch.int32), code_causal=[True])


def test_backend_surface_and_hook_is_inert_without_impl():
    assert bk.AbridgeAttentionBackend.get_kv_cache_shape(10) == (10, 2, 16, 8, 128)
    with pytest.raises(NotImplementedError):
        bk.AbridgeAttentionBackend.get_kv_cache_shape(10, block_size=32)
    with pytest.raises(NotImplementedError):
        bk.AbridgeAttentionImpl(num_heads=16)
    out = torch.full((2, 32 * 128), 3.0)
    bk.maybe_override_attention(SimpleNamespace(), torch.zeros(2, 32 * 128), torch.zeros(1), object(), out)
    assert bool((out == 3.0).all())


def test_auto_split_pages_fills_the_gpu_with_the_longest_split():
    from abridgekv_amd import ops
    rng = np.random.default_rng(0)
    assert ops.auto_split_pages(rng.integers(2000, 17000, 256), num_cus=256) == 48       # saturated-like batch
    assert ops.auto_split_pages(np.full(64, 5000), num_cus=256) == 40                    # 48 would leave CUs idle
    assert ops.auto_split_pages([1068], num_cus=256) == ops.DEFAULT_SPLIT_PAGES          # tiny batch: the default
    assert ops.auto_split_pages(np.full(64, 5000), num_cus=64) == 48
