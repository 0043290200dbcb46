"""CPU pins of the oracle's 4-bit affine KV format (MLX "affine" quantisation, group 64).

MLX is not available here and the reference holds no int4 vectors, so parity with MLX's
own kernels is unpinned; these checks pin what the algorithm fixes: the larger-magnitude
end of each group is reproduced exactly, every value within half a step (plus the bf16
rounding of the parameters), codes ordered like the values, the sign symmetry
quantize(-x) = (codes, -scale, -bias), ties rounded away from zero, the word layout, and
constant groups.
"""
import numpy as np
import pytest


@pytest.fixture(scope="module")
def O(ora):
    return ora


def _groups(x):
    return x.reshape(-1, 64)


def test_edge_value_reproduced_exactly_and_round_trip_bound(O):
    x = O.f32_from_bf16(O.normal_bf16((64, 256), 11, std=1.5))
    w, s, b = O.int4_quantize(x)
    d = O.int4_dequantize(w, s, b)
    codes = O.unpack_bits(w, 4)
    sf = np.repeat(O.f32_from_bf16(s), 64, axis=-1).astype(np.float64)
    bf = np.repeat(O.f32_from_bf16(b), 64, axis=-1).astype(np.float64)
    u = 2.0 ** -8  # bf16 unit roundoff
    err = np.abs(d.astype(np.float64) - x)
    bound = (0.5 + 16 * u) * np.abs(sf) * (1 + u) + 2 * u * (np.abs(bf) + np.abs(d)) + 15 * u * np.abs(sf)
    inner = codes < 15
    assert (err[inner] <= bound[inner]).all(), float((err - bound)[inner].max())
    # code 15 also takes the values past the grid's far end (the edge moved onto the grid can
    # shrink the step): those lie at or beyond step 14.5
    t = (x - bf) / sf
    assert (t[~inner] >= 14.5 - 0.1).all()
    # the larger-magnitude end is the bias: code 0, reproduced bit-exactly
    for g, (xg, dg, cg) in enumerate(zip(_groups(x), _groups(d), _groups(codes))):
        edge_i = int(np.argmin(xg)) if abs(xg.min()) > abs(xg.max()) else int(np.argmax(xg))
        assert cg[edge_i] == 0 and dg[edge_i] == xg[edge_i], g
        assert cg.max() >= 14  # the range spans the grid


def test_codes_follow_value_order_and_sign_symmetry(O):
    x = O.f32_from_bf16(O.normal_bf16((32, 128), 12))
    w, s, b = O.int4_quantize(x)
    codes = _groups(O.unpack_bits(w, 4))
    sf = O.f32_from_bf16(s).reshape(-1)
    for xg, cg, sg in zip(_groups(x), codes, sf):
        order = np.argsort(xg, kind="stable")
        c_sorted = cg[order].astype(int)
        assert (np.diff(c_sorted) >= 0).all() if sg > 0 else (np.diff(c_sorted) <= 0).all()
    # away from ties |min| = |max| (where both signs pick the maximum as the edge), negating the
    # values negates scale and bias and keeps the codes
    wn, sn, bn = O.int4_quantize(-x)
    xg = _groups(x)
    untied = np.abs(xg.min(1)) != np.abs(xg.max(1))
    assert untied.sum() > 0.8 * len(untied)
    assert (wn.reshape(-1, 8)[untied] == w.reshape(-1, 8)[untied]).all()
    assert (O.f32_from_bf16(sn).reshape(-1)[untied] == -O.f32_from_bf16(s).reshape(-1)[untied]).all()
    assert (O.f32_from_bf16(bn).reshape(-1)[untied] == -O.f32_from_bf16(b).reshape(-1)[untied]).all()


def test_ties_round_away_from_zero_and_word_layout(O):
    # group 0..15 then 6.5: min 0, max 15 -> scale -1, bias 15, code = 15 - x;
    # (6.5 - 15) / -1 = 8.5 rounds to 9 (half away from zero; half-to-even would give 8)
    g = np.zeros(64, dtype=np.float32)
    g[:16] = np.arange(16)
    g[16:] = 6.5
    w, s, b = O.int4_quantize(g[None, :])
    assert O.f32_from_bf16(s)[0, 0] == -1.0 and O.f32_from_bf16(b)[0, 0] == 15.0
    codes = O.unpack_bits(w, 4)[0]
    assert (codes[:16] == 15 - np.arange(16)).all() and (codes[16:] == 9).all()
    # value i at bits 4 (i % 8) of word i / 8
    assert int(w[0, 0]) == 0x89ABCDEF and int(w[0, 1]) == 0x01234567


@pytest.mark.parametrize("c", [0.0, 1.0, -3.5, 1e-3])
def test_constant_group(O, c):
    x = np.full((1, 128), c, dtype=np.float32)
    x = O.f32_from_bf16(O.bf16_from_f32(x))
    w, s, b = O.int4_quantize(x)
    assert (O.unpack_bits(w, 4) == 0).all()
    assert (O.int4_dequantize(w, s, b) == x).all()


def test_dequantize_rounds_once(O):
    # code 15, scale 1.0078125 (bf16 1 + 2^-7), bias -15: the exact value 15.1171875 - 15 =
    # 0.1171875 is a bf16 value and is kept (rounding the product to bf16 first would give
    # 15.125 - 15 = 0.125); with bias 0 the one rounding takes 15.1171875 to 15.125
    w = np.full((1, 16), 0xFFFFFFFF, dtype=np.uint32)
    s = O.bf16_from_f32(np.full((1, 2), 1.0078125, dtype=np.float32))
    for bias, want in ((-15.0, 0.1171875), (0.0, 15.125)):
        b = O.bf16_from_f32(np.full((1, 2), bias, dtype=np.float32))
        assert (O.int4_dequantize(w, s, b) == want).all()
        assert (O.int4_affine_values(w, s, b) == 15.1171875 + bias).all()
