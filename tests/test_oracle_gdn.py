"""Pins of the Gated DeltaNet oracle (oracle.gdn_scan, restating crates/ops/src/gdn.rs:83-150).

The reference ships no vectors for this op (its tests only check the stub error,
crates/attention/tests/gdn.rs), so the oracle is pinned by what the delta rule fixes:
read-after-write returns the written value, the g = 0 and beta = 0 reductions, linearity
in v from a zero state, the key-head mapping of the head expansion, and chunking
invariance. A swapped state axis, a decay applied after the write, a wrong sign in delta,
or q and k exchanged each fail at least one of them.
"""
import numpy as np
import pytest

import oracle


def _inputs(rng, B, T, Hk, Hv, Dk, Dv, unit_k=True):
    q = rng.standard_normal((B, T, Hk, Dk)).astype(np.float32)
    k = rng.standard_normal((B, T, Hk, Dk)).astype(np.float32)
    if unit_k:
        k = (k / np.linalg.norm(k, axis=-1, keepdims=True)).astype(np.float32)
    v = rng.standard_normal((B, T, Hv, Dv)).astype(np.float32)
    g = rng.uniform(0.5, 1.0, (B, T, Hv)).astype(np.float32)
    beta = rng.uniform(0.05, 0.95, (B, T, Hv)).astype(np.float32)
    return q, k, v, g, beta


def test_read_after_write_returns_v():
    # beta = 1: after the write, S k = kv + |k|^2 (v - kv), which is v for a unit key;
    # with g != 1 it also fixes the decay before the recall (decaying after the write
    # would give g v instead).
    rng = np.random.default_rng(1)
    B, T, Hk, Hv, Dk, Dv = 2, 1, 2, 4, 16, 8
    q, k, v, g, beta = _inputs(rng, B, T, Hk, Hv, Dk, Dv)
    beta[:] = 1.0
    S0 = rng.standard_normal((B, Hv, Dv, Dk))
    _, S = oracle.gdn_scan(q, k, v, g, beta, S0)
    for b in range(B):
        for h in range(Hv):
            kk = k[b, 0, h // (Hv // Hk)].astype(np.float64)
            kv_old = (g[b, 0, h] * S0[b, h]) @ kk
            expect = kv_old + (kk @ kk) * (v[b, 0, h] - kv_old)
            np.testing.assert_allclose(S[b, h] @ kk, expect, rtol=0, atol=1e-12)
            np.testing.assert_allclose(S[b, h] @ kk, v[b, 0, h], rtol=0, atol=1e-6)


def test_zero_decay_writes_outer_product():
    # g = 0 clears the state: kv = 0, delta = beta v, S = delta k^T, y = delta (k . q)
    rng = np.random.default_rng(2)
    B, T, Hk, Hv, Dk, Dv = 1, 1, 1, 2, 8, 16
    q, k, v, g, beta = _inputs(rng, B, T, Hk, Hv, Dk, Dv, unit_k=False)
    g[:] = 0.0
    S0 = rng.standard_normal((B, Hv, Dv, Dk))
    y, S = oracle.gdn_scan(q, k, v, g, beta, S0)
    for h in range(Hv):
        delta = beta[0, 0, h].astype(np.float64) * v[0, 0, h].astype(np.float64)
        kk, qq = k[0, 0, 0].astype(np.float64), q[0, 0, 0].astype(np.float64)
        np.testing.assert_allclose(S[0, h], np.outer(delta, kk), rtol=1e-15, atol=1e-15)
        np.testing.assert_allclose(y[0, 0, h], delta * (kk @ qq), rtol=1e-12, atol=1e-12)


def test_zero_beta_only_decays():
    rng = np.random.default_rng(3)
    B, T, Hk, Hv, Dk, Dv = 1, 1, 2, 2, 8, 8
    q, k, v, g, beta = _inputs(rng, B, T, Hk, Hv, Dk, Dv)
    beta[:] = 0.0
    S0 = rng.standard_normal((B, Hv, Dv, Dk))
    y, S = oracle.gdn_scan(q, k, v, g, beta, S0)
    for h in range(Hv):
        np.testing.assert_allclose(S[0, h], g[0, 0, h] * S0[0, h], rtol=1e-15)
        np.testing.assert_allclose(y[0, 0, h], (g[0, 0, h] * S0[0, h]) @ q[0, 0, h].astype(np.float64),
                                   rtol=1e-12, atol=1e-12)


def test_linear_in_v_from_zero_state():
    rng = np.random.default_rng(4)
    B, T, Hk, Hv, Dk, Dv = 1, 6, 1, 2, 16, 16
    q, k, v1, g, beta = _inputs(rng, B, T, Hk, Hv, Dk, Dv)
    v2 = rng.standard_normal(v1.shape).astype(np.float32)
    Z = np.zeros((B, Hv, Dv, Dk))
    y1, S1 = oracle.gdn_scan(q, k, v1, g, beta, Z)
    y2, S2 = oracle.gdn_scan(q, k, v2, g, beta, Z)
    y3, S3 = oracle.gdn_scan(q, k, (v1 + 2 * v2).astype(np.float64).astype(np.float32), g, beta, Z)
    np.testing.assert_allclose(y3, y1 + 2 * y2, rtol=1e-6, atol=1e-6)
    np.testing.assert_allclose(S3, S1 + 2 * S2, rtol=1e-6, atol=1e-6)


def test_key_head_mapping():
    # value head h reads key head h // (Hv / Hk): the same result as a single-head scan fed
    # that key head, and different from the neighbouring key head
    rng = np.random.default_rng(5)
    B, T, Hk, Hv, Dk, Dv = 1, 3, 2, 6, 8, 8
    q, k, v, g, beta = _inputs(rng, B, T, Hk, Hv, Dk, Dv)
    S0 = rng.standard_normal((B, Hv, Dv, Dk))
    y, S = oracle.gdn_scan(q, k, v, g, beta, S0)
    rep = Hv // Hk
    for h in range(Hv):
        kh = h // rep
        ys, Ss = oracle.gdn_scan(q[:, :, kh:kh + 1], k[:, :, kh:kh + 1], v[:, :, h:h + 1], g[:, :, h:h + 1],
                                 beta[:, :, h:h + 1], S0[:, h:h + 1])
        assert np.array_equal(ys[:, :, 0], y[:, :, h]) and np.array_equal(Ss[:, 0], S[:, h])
        other = (kh + 1) % Hk
        yo, _ = oracle.gdn_scan(q[:, :, other:other + 1], k[:, :, other:other + 1], v[:, :, h:h + 1],
                                g[:, :, h:h + 1], beta[:, :, h:h + 1], S0[:, h:h + 1])
        assert not np.allclose(yo[:, :, 0], y[:, :, h])


def test_chunked_scan_equals_one_scan():
    rng = np.random.default_rng(6)
    B, T, Hk, Hv, Dk, Dv = 2, 9, 1, 2, 8, 16
    q, k, v, g, beta = _inputs(rng, B, T, Hk, Hv, Dk, Dv)
    S0 = rng.standard_normal((B, Hv, Dv, Dk))
    y, S = oracle.gdn_scan(q, k, v, g, beta, S0)
    ya, Sa = oracle.gdn_scan(q[:, :4], k[:, :4], v[:, :4], g[:, :4], beta[:, :4], S0)
    yb, Sb = oracle.gdn_scan(q[:, 4:], k[:, 4:], v[:, 4:], g[:, 4:], beta[:, 4:], Sa)
    assert np.array_equal(np.concatenate([ya, yb], axis=1), y) and np.array_equal(Sb, S)


def test_output_reads_updated_state_with_q():
    # y uses the state after the write and the query (not the key): with q orthogonal to k
    # and a zero state, y = 0 although S != 0
    rng = np.random.default_rng(7)
    B, T, Hk, Hv, Dk, Dv = 1, 1, 1, 1, 8, 8
    q, k, v, g, beta = _inputs(rng, B, T, Hk, Hv, Dk, Dv)
    kk = k[0, 0, 0].astype(np.float64)
    qq = rng.standard_normal(Dk)
    qq -= (qq @ kk) / (kk @ kk) * kk
    q[0, 0, 0] = qq.astype(np.float32)
    y, S = oracle.gdn_scan(q, k, v, g, beta, np.zeros((B, Hv, Dv, Dk)))
    assert np.abs(S).max() > 0.01
    np.testing.assert_allclose(y, 0.0, atol=1e-6)
    y2, _ = oracle.gdn_scan(k, k, v, g, beta, np.zeros((B, Hv, Dv, Dk)))
    np.testing.assert_allclose(y2[0, 0, 0], beta[0, 0, 0] * v[0, 0, 0] * (kk @ kk), rtol=1e-6)


@pytest.mark.parametrize("T", [1, 5])
def test_row_norm_bounded_for_unit_keys(T):
    # with |k| = 1, beta in [0, 1] and g in [0, 1], a row's component along k becomes a
    # convex combination of its decayed value and v, and the rest only decays, so
    # |S_T[r]|^2 <= |S_0[r]|^2 + sum_t v_t[r]^2
    rng = np.random.default_rng(8)
    B, Hk, Hv, Dk, Dv = 1, 1, 1, 16, 4
    q, k, v, g, beta = _inputs(rng, B, T, Hk, Hv, Dk, Dv)
    S0 = rng.standard_normal((B, Hv, Dv, Dk))
    _, S = oracle.gdn_scan(q, k, v, g, beta, S0)
    lhs = (S[0, 0] ** 2).sum(axis=-1)
    rhs = (S0[0, 0] ** 2).sum(axis=-1) + (v[0, :, 0].astype(np.float64) ** 2).sum(axis=0)
    assert np.all(lhs <= rhs * (1 + 1e-6))
