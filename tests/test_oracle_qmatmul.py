"""Pins of the affine quantized-matmul oracle (oracle.qmatmul / oracle.dequantize, restating
MLX quantized_matmul with transpose=true as called by crates/ops/src/quant.rs:57-76).

The reference holds no packed-weight vectors (its quantized tests run only on the MLX
backend, absent here: crates/serve/tests/forward_separate.rs), so the oracle is pinned by
what the format and the arithmetic fix: hand-built words read back field by field in
MLX's lowest-bits-first order, the per-group affine map on constant fields, an
independent numpy unpack-and-matmul, the transpose convention (y = x W^T), and the
reference's own separate-vs-fused projection property (forward_separate.rs:80-91).
Whether MLX's own kernels agree bit for bit is parity unpinned: only its published
packing is restated. A field order reversed within a word, a group index taken modulo
the wrong count, swapped scales and biases, or W used untransposed each fail a check.
"""
import numpy as np
import pytest

import oracle


def _rand_q(rng, N, K, gs, bits):
    q = rng.integers(0, 1 << bits, (N, K), dtype=np.uint32)
    s = oracle.f32_from_bf16(oracle.bf16_from_f32(rng.uniform(0.002, 0.02, (N, K // gs)).astype(np.float32)))
    b = oracle.f32_from_bf16(oracle.bf16_from_f32(rng.uniform(-0.1, 0.1, (N, K // gs)).astype(np.float32)))
    return q, oracle.pack_bits(q, bits), s, b


def test_hand_built_words_read_lowest_bits_first():
    # 4-bit: word 0x76543210 holds fields 0, 1, ..., 7; 8-bit: 0x03020100 holds 0, 1, 2, 3
    K = 32
    w4 = np.array([[0x76543210, 0xFEDCBA98, 0x01234567, 0x89ABCDEF]], np.uint32)
    ones = np.ones((1, 1), np.float32)
    W = oracle.dequantize(w4, ones, np.zeros((1, 1), np.float32), 32, 4)
    expect = list(range(16)) + [7, 6, 5, 4, 3, 2, 1, 0, 15, 14, 13, 12, 11, 10, 9, 8]
    assert W[0].tolist() == expect
    # one-hot activations read the same fields through the matmul
    y = oracle.qmatmul(np.eye(K, dtype=np.float32), w4, ones, np.zeros((1, 1), np.float32), 32, 4)
    assert y[:, 0].tolist() == expect
    w8 = np.array([[0x03020100, 0x07060504, 0xFF80407F, 0, 0, 0, 0, 0]], np.uint32)
    W8 = oracle.dequantize(w8, ones, np.zeros((1, 1), np.float32), 32, 8)
    assert W8[0, :12].tolist() == [0, 1, 2, 3, 4, 5, 6, 7, 0x7F, 0x40, 0x80, 0xFF]
    assert np.array_equal(oracle.pack_bits(np.array([expect]), 4), w4)
    assert np.array_equal(oracle.unpack_bits(w8, 8)[0, :12], W8[0, :12].astype(np.uint32))


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("gs", [32, 64, 128])
def test_group_affine_map_on_constant_fields(bits, gs):
    # every field = c: W[n, k] = s[n, g] c + b[n, g]; with x = 1 the row sums are
    # gs * sum_g (s c + b); swapping scales and biases changes them
    rng = np.random.default_rng(bits * 1000 + gs)
    N, K, c = 3, 4 * gs, (1 << bits) - 3
    wq = oracle.pack_bits(np.full((N, K), c), bits)
    s = rng.uniform(0.01, 0.1, (N, K // gs)).astype(np.float32)
    b = rng.uniform(-1, 1, (N, K // gs)).astype(np.float32)
    y = oracle.qmatmul(np.ones((1, K), np.float32), wq, s, b, gs, bits)
    expect = gs * (s.astype(np.float64) * c + b).sum(axis=1)
    np.testing.assert_allclose(y[0], expect, rtol=1e-12)
    ys = oracle.qmatmul(np.ones((1, K), np.float32), wq, b, s, gs, bits)
    assert not np.allclose(ys, y)
    # group g covers k in [g gs, (g + 1) gs): a one-hot x at k picks group k // gs
    for k in (0, gs - 1, gs, K - 1):
        e = np.zeros((1, K), np.float32)
        e[0, k] = 1
        y1 = oracle.qmatmul(e, wq, s, b, gs, bits)[0]
        np.testing.assert_allclose(y1, s[:, k // gs].astype(np.float64) * c + b[:, k // gs], rtol=1e-12)


@pytest.mark.parametrize("bits,gs", [(4, 64), (4, 32), (8, 64), (8, 128)])
def test_matches_independent_numpy_path(bits, gs):
    rng = np.random.default_rng(7 + bits + gs)
    M, N, K = 5, 48, 512
    q, wq, s, b = _rand_q(rng, N, K, gs, bits)
    x = oracle.f32_from_bf16(oracle.normal_bf16((M, K), seed=bits + gs))
    # numpy: unpack with shifts over a uint8 view (a different route than the oracle's
    # word/field indexing), dequantise per group, then x @ W^T
    if bits == 8:
        fields = wq.view(np.uint8).reshape(N, K).astype(np.float64)
    else:
        by = wq.view(np.uint8).reshape(N, K // 2)
        fields = np.stack([by & 15, by >> 4], axis=-1).reshape(N, K).astype(np.float64)
    assert np.array_equal(fields, q)
    W = fields * np.repeat(s, gs, axis=1) + np.repeat(b, gs, axis=1)
    np.testing.assert_allclose(oracle.dequantize(wq, s, b, gs, bits), W, rtol=0, atol=0)
    np.testing.assert_allclose(oracle.qmatmul(x, wq, s, b, gs, bits), x.astype(np.float64) @ W.T, rtol=1e-12, atol=1e-12)


def test_transpose_convention():
    # y = x W^T with W [N, K]: a W with one nonzero row n puts output only in column n
    rng = np.random.default_rng(3)
    N, K, gs = 6, 64, 64
    q = np.zeros((N, K), np.uint32)
    q[4] = rng.integers(1, 16, K)
    s = np.ones((N, 1), np.float32)
    y = oracle.qmatmul(rng.standard_normal((3, K)).astype(np.float32), oracle.pack_bits(q, 4), s,
                       np.zeros((N, 1), np.float32), gs, 4)
    assert np.count_nonzero(y[:, [0, 1, 2, 3, 5]]) == 0 and np.all(y[:, 4] != 0)


def test_separate_projections_equal_the_fused_one():
    # run_qkv's two paths (crates/serve/src/forward/projection.rs:105-128): three quantized
    # matmuls concatenated on the feature axis equal one over the row-concatenated weights
    # (the reference checks this at max-abs 1e-3, forward_separate.rs:80-91; here exact)
    rng = np.random.default_rng(11)
    K, gs, bits = 256, 64, 4
    parts = [_rand_q(rng, n, K, gs, bits) for n in (64, 32, 32)]
    x = rng.standard_normal((3, K)).astype(np.float32)
    sep = np.concatenate([oracle.qmatmul(x, p[1], p[2], p[3], gs, bits) for p in parts], axis=1)
    fused = oracle.qmatmul(x, np.concatenate([p[1] for p in parts]), np.concatenate([p[2] for p in parts]),
                           np.concatenate([p[3] for p in parts]), gs, bits)
    assert np.array_equal(sep, fused)


@pytest.mark.parametrize("bits", [4, 8])
def test_minmax_quantize_round_trip(bits):
    # the test-data generator: every weight within half a step of its dequantised value,
    # plus the bf16 roundings of the group's minimum and of the step (at most 2^-8 of it,
    # times the largest field)
    rng = np.random.default_rng(bits)
    N, K, gs = 16, 256, 64
    w = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    wq, sb, bb = oracle.minmax_quantize(w, gs, bits)
    s, b = oracle.f32_from_bf16(sb), oracle.f32_from_bf16(bb)
    W = oracle.dequantize(wq, s, b, gs, bits)
    lo = w.reshape(N, K // gs, gs).min(-1)
    slack = np.repeat(s * (0.5 + ((1 << bits) - 1) * 2.0**-8) + np.abs(lo - b) + 1e-7, gs, axis=1)
    assert np.all(np.abs(W - w) <= slack)


def test_dequantize_act_rounds_each_weight_once_to_nearest_even():
    # the large-M weights: round_T(s q + b). Pinned against torch's own bf16 / f16 rounding
    # of the exact value (exact in f64 for bf16 s and b and fields below 256), ties to even
    # at hand-built halfway points, and exactness where the value is representable
    import torch

    rng = np.random.default_rng(7)
    for bits in (4, 8):
        N, K, gs = 6, 128, 32
        q, wq, s, b = _rand_q(rng, N, K, gs, bits)
        exact = oracle.dequantize(wq, s, b, gs, bits)  # f64, exact here
        for dtype, td in (("bf16", torch.bfloat16), ("f16", torch.float16)):
            got = oracle.dequantize_act(wq, s, b, gs, bits, dtype)
            want = torch.from_numpy(exact.astype(np.float32)).to(td).float().numpy()
            assert np.array_equal(got, want), (bits, dtype)
    one = np.ones((1, 1), np.float32)
    # 1 + 2^-8 is halfway between bf16 1 and 1 + 2^-7: even is 1; 1 + 3 2^-8 rounds up to
    # 1 + 2^-6; f16 (10 fraction bits) keeps both
    w = oracle.pack_bits(np.array([[1, 3] + [0] * 30], np.uint32), 4)
    s = np.full((1, 1), 2.0**-8, np.float32)
    assert oracle.dequantize_act(w, s, one, 32, 4, "bf16")[0, :2].tolist() == [1.0, 1.0 + 2.0**-6]
    assert oracle.dequantize_act(w, s, one, 32, 4, "f16")[0, :2].tolist() == [1.0 + 2.0**-8, 1.0 + 3 * 2.0**-8]
    # representable values pass unchanged
    q = np.arange(16, dtype=np.uint32)[None, :].repeat(2, axis=1)
    w = oracle.pack_bits(q, 4)
    got = oracle.dequantize_act(w, np.full((1, 1), 0.5, np.float32), np.full((1, 1), -3.0, np.float32), 32, 4)
    assert got[0].tolist() == (0.5 * q[0] - 3.0).tolist()
