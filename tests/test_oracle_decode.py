"""Pins of oracle.decode: closed-form special cases of softmax attention and the paged gather."""
import numpy as np
import pytest
import scipy.special as sp
import torch

from oracle import decode as od


def test_single_row_returns_value_and_score():
    rng = np.random.default_rng(0)
    q = rng.standard_normal((32, 128))
    k = rng.standard_normal((1, 8, 128))
    v = rng.standard_normal((1, 8, 128))
    out, lse = od.decode_fp64(q, k, v, 0.1)
    for h in range(32):
        assert np.allclose(out[h], v[0, h // 4])
        assert np.isclose(lse[h], 0.1 * q[h] @ k[0, h // 4])


def test_identical_rows_add_log_n():
    rng = np.random.default_rng(1)
    q = rng.standard_normal((32, 128))
    k1 = rng.standard_normal((1, 8, 128))
    v1 = rng.standard_normal((1, 8, 128))
    n = 37
    out, lse = od.decode_fp64(q, np.repeat(k1, n, 0), np.repeat(v1, n, 0), 0.3)
    o1, l1 = od.decode_fp64(q, k1, v1, 0.3)
    assert np.allclose(out, o1) and np.allclose(lse, l1 + np.log(n))


def test_two_rows_logistic_weights():
    rng = np.random.default_rng(2)
    q = rng.standard_normal((32, 128))
    k = rng.standard_normal((2, 8, 128))
    v = rng.standard_normal((2, 8, 128))
    out, _ = od.decode_fp64(q, k, v, 0.05)
    for h in range(32):
        s = 0.05 * (k[:, h // 4] @ q[h])
        w0 = 1 / (1 + np.exp(s[1] - s[0]))
        assert np.allclose(out[h], w0 * v[0, h // 4] + (1 - w0) * v[1, h // 4])


def test_matches_scipy_and_is_row_permutation_invariant():
    rng = np.random.default_rng(3)
    n = 300
    q = rng.standard_normal((32, 128))
    k = rng.standard_normal((n, 8, 128))
    v = rng.standard_normal((n, 8, 128))
    out, lse = od.decode_fp64(q, k, v, 128 ** -0.5)
    for h in (0, 5, 31):
        s = (k[:, h // 4] @ q[h]) * 128 ** -0.5
        assert np.isclose(lse[h], sp.logsumexp(s))
        assert np.allclose(out[h], sp.softmax(s) @ v[:, h // 4])
    perm = rng.permutation(n)
    o2, l2 = od.decode_fp64(q, k[perm], v[perm], 128 ** -0.5)
    assert np.allclose(out, o2) and np.allclose(lse, l2)


def test_empty_sequence():
    out, lse = od.decode_fp64(np.ones((32, 128)), np.zeros((0, 8, 128)), np.zeros((0, 8, 128)), 1.0)
    assert np.all(out == 0) and np.all(np.isneginf(lse))


def test_paged_rows_walks_pages_in_table_order():
    rng = np.random.default_rng(4)
    cache = rng.standard_normal((10, 2, 16, 8, 128))
    table = np.array([7, 2, 9])
    k, v = od.paged_rows(cache, table, 40)
    assert k.shape == (40, 8, 128)
    for pos in range(40):
        assert np.array_equal(k[pos], cache[table[pos // 16], 0, pos % 16])
        assert np.array_equal(v[pos], cache[table[pos // 16], 1, pos % 16])


def test_reference_arithmetic_within_bf16_bound():
    """The reference's torch arithmetic (bf16 scores, fp32 softmax, bf16 probabilities) stays within the 2e-2 bf16
    bound of the fp64 closed form: it is a measurement baseline, not the parity target."""
    rng = np.random.default_rng(5)
    cache = torch.randn((40, 2, 16, 8, 128), generator=torch.Generator().manual_seed(0)).to(torch.bfloat16)
    lens = np.array([1, 200, 513], np.int32)
    table = np.stack([rng.permutation(np.arange(1, 40))[:33] for _ in range(3)]).astype(np.int32)
    q = torch.randn((3, 32, 128), generator=torch.Generator().manual_seed(1)).to(torch.bfloat16)
    got = od.decode_ref_torch(q, cache, torch.from_numpy(table), torch.from_numpy(lens.astype(np.int64)),
                              128 ** -0.5).float().numpy()
    ref, _ = od.decode_paged_fp64(q.float().numpy(), cache.float().numpy(), table, lens, 128 ** -0.5)
    assert np.abs(got - ref).max() <= 2e-2


def test_request_arithmetic_within_bf16_bound_and_limit_exact():
    """The reference's per-request multi-query arithmetic (code step: non-causal, keys < limit; prompt chunk: causal
    after a prefix) row by row against the fp64 closed form. The key row just past each query's visible range carries
    values of 100: reading it would move that query's output far beyond the 2e-2 bound."""
    g = torch.Generator().manual_seed(3)
    S, n = 90, 12
    key = torch.randn((8, S, 128), generator=g).to(torch.bfloat16)
    value = torch.randn((8, S, 128), generator=g).to(torch.bfloat16)
    q = torch.randn((n, 32, 128), generator=g).to(torch.bfloat16)
    kf, vf, qf = (t.float().numpy() for t in (key, value, q))
    # non-causal, keys < 70: row 70 planted
    v_pl = value.clone()
    v_pl[:, 70] = 100.0
    got = od.request_ref_torch(q, key, v_pl, 128 ** -0.5, limit=70).float().numpy()
    for i in range(n):
        ref, _ = od.decode_fp64(qf[i], kf[:, :70].transpose(1, 0, 2), vf[:, :70].transpose(1, 0, 2), 128 ** -0.5)
        assert np.abs(got[i] - ref).max() <= 2e-2
    # causal after a prefix of 60: query i sees keys <= 60 + i; the planted row is the first one it must not see
    for i in (0, 5, 11):
        v_pl = value.clone()
        v_pl[:, 61 + i] = 100.0
        got = od.request_ref_torch(q, key, v_pl, 128 ** -0.5, limit=S, causal=True, prefix_len=60).float().numpy()
        m = 61 + i
        ref, _ = od.decode_fp64(qf[i], kf[:, :m].transpose(1, 0, 2), vf[:, :m].transpose(1, 0, 2), 128 ** -0.5)
        assert np.abs(got[i] - ref).max() <= 2e-2
