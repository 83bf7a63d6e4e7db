"""Pins of oracle.layout: closed forms, brute force and the reference's own test invariants."""
from pathlib import Path

import numpy as np
import pytest

from abridgekv_amd import workloads
from oracle import layout as ol

GOLDEN = Path(__file__).resolve().parent / "golden"


def _bitrev(k, bits):
    return int(format(k, f"0{bits}b")[::-1], 2) if bits else 0


def test_bitrev_offsets_closed_form_k256():
    offs = ol.bitrev_code_offsets(256, 512)
    assert offs.tolist() == [2 * _bitrev(k, 8) for k in range(256)]


@pytest.mark.parametrize("K", [1, 2, 4, 8, 64, 128, 256])
def test_bitrev_offsets_prefix_independent_distinct_in_range(K):
    """scripts/test_compresslm_vllm_state.py:349-353: distinct offsets, max < span, and the first K' rows of any
    larger K use the same offsets (a quota's prefix is K-independent)."""
    offs = ol.bitrev_code_offsets(K, 512)
    assert len(set(offs.tolist())) == K and offs.max() < 512 and offs.min() >= 0
    big = ol.bitrev_code_offsets(256, 512)
    assert np.array_equal(big[:K], offs)


def test_bitrev_offsets_with_span_tail():
    """compress_forward.py:47-51 docstring case: C=512, T=16, K=256 -> floor(1.9375 * rev), max 494."""
    offs = ol.bitrev_code_offsets(256, 512, span=512 - 16)
    assert offs.max() == 494
    assert offs.tolist() == [int(1.9375 * _bitrev(k, 8)) for k in range(256)]
    with pytest.raises(ValueError):
        ol.bitrev_code_offsets(256, 200)


def test_bitrev_rope_positions_brute_force():
    C, K = 16, 8
    offs = [(_bitrev(k, 3) * C) // K for k in range(K)]
    expect = []
    for b in range(5):
        expect += [b * C + j for j in range(C)] + [b * C + o for o in offs]
    got = ol.bitrev_rope_positions(np.arange(len(expect)), C, K)
    assert got.tolist() == expect
    assert np.array_equal(ol.training_rope_positions(5, C, K), got)


def test_rope_neox_matches_pairwise_rotation():
    rng = np.random.default_rng(0)
    x = rng.standard_normal((7, 3, 128))
    pos = np.array([0, 1, 5, 100, 2603, 32767, 123456])
    got = ol.rope_neox(x, pos)
    inv = 1e6 ** (-np.arange(64) * 2 / 128)
    expect = np.empty_like(x)
    for s, p in enumerate(pos):
        for i in range(64):
            c, sn = np.cos(p * inv[i]), np.sin(p * inv[i])
            a, b = x[s, :, i], x[s, :, i + 64]
            expect[s, :, i] = a * c - b * sn
            expect[s, :, i + 64] = b * c + a * sn
    assert np.allclose(got, expect, atol=1e-12)
    assert np.allclose(got[0], x[0])                                  # position 0 is the identity
    assert np.allclose(np.linalg.norm(got, axis=-1), np.linalg.norm(x, axis=-1))


def test_rope_relative_position_property():
    """<R(p) q, R(p') k> depends on p - p' only (catches a sign or a swapped half)."""
    rng = np.random.default_rng(1)
    q, k = rng.standard_normal((1, 1, 128)), rng.standard_normal((1, 1, 128))
    d1 = (ol.rope_neox(q, [1000]) * ol.rope_neox(k, [990])).sum()
    d2 = (ol.rope_neox(q, [20]) * ol.rope_neox(k, [10])).sum()
    d3 = (ol.rope_neox(q, [20]) * ol.rope_neox(k, [30])).sum()
    assert abs(d1 - d2) < 1e-9 and abs(d1 - d3) > 1e-6


def test_quota_groups_match_reference_grouping():
    """scripts/test_compresslm_physical_quotas.py:141-167 asserts 6 groups of 6 with quotas [64,64,128,128,128,256]
    for the 6 x 256 / 18 x 128 / 12 x 64 layer split."""
    quotas = ol.load_schedule_quotas(GOLDEN / "sched_trunc_perlayer_mean128.json")
    assert quotas == ol.PERLAYER_MEAN128_QUOTAS == workloads.QWEN3_4B_LAYER_QUOTAS
    assert sum(quotas) == 4608 and len(quotas) == 36
    groups, gq = ol.quota_groups(quotas)
    assert sorted(len(g) for g in groups) == [6] * 6
    assert sorted(gq) == [64, 64, 128, 128, 128, 256]
    assert groups == [[0, 15, 18, 20, 21, 24], [1, 3, 5, 8, 30, 32], [2, 4, 6, 10, 31, 35],
                      [7, 12, 16, 22, 26, 29], [9, 13, 17, 23, 27, 33], [11, 14, 19, 25, 28, 34]]
    for g, layers in enumerate(groups):
        assert {quotas[l] for l in layers} == {gq[g]}
    assert workloads.quota_groups(quotas) == (groups, gq)


def test_quota_groups_uniform_and_near_equal_buckets():
    groups, gq = ol.quota_groups([128] * 36)
    assert groups == [list(range(36))] and gq == [128]
    # 12 x a + 13 x b: max < 1.25 * min -> group size 13, the smaller bucket is one padded group
    groups, gq = ol.quota_groups([64] * 12 + [128] * 13)
    assert [len(g) for g in groups] == [12, 13] and gq == [64, 128]


def test_rows_per_layer_closed_form_cases():
    # T content tokens incl. the query
    assert ol.rows_per_layer(1, 1, 64) == 1
    assert ol.rows_per_layer(512, 100, 64) == 512                    # block 0 still open (query is token 511)
    assert ol.rows_per_layer(513, 100, 64) == 100 + 64 + 1           # block 0 closed, query opens block 1
    assert ol.rows_per_layer(513, 600, 64) == 512 + 64 + 1           # all-prompt block keeps its rows
    assert ol.rows_per_layer(512 + 16384 + 7, 512, 256) == 512 + 33 * 256 + 7
