"""Pins for the oracle's FP8 E4M3FN quantiser (runs without a GPU).

The oracle restates crates/ops/src/fp8.rs (the quantiser of the reference's
FP8 KV cache, crates/kvcache/src/fp8.rs). It is checked against:
  - the reference's own unit tests (crates/ops/tests/fp8.rs), same inputs and
    the same assertions;
  - torch's float8_e4m3fn cast, an independent round-to-nearest-even
    implementation of the same OCP E4M3FN format, on every finite bf16 value;
  - the format itself: each of the 253 finite codes maps to itself, midpoints
    between neighbours round to the even mantissa, 448 saturates;
  - the two forms of the block exponent (the reference's f32 log2 and the
    kernels' double log2 rounded to f32) on every f32 near a power of two;
  - scale invariants of the block quantisation.
"""
import numpy as np
import pytest


def finite_bf16_as_f32():
    h = np.arange(65536, dtype=np.uint32)
    x = (h << 16).view(np.float32)
    return x[np.isfinite(x)]


# ---------------------------------------------------- crates/ops/tests/fp8.rs
def test_reference_unit_tests(ora):
    # e4m3fn_roundtrip_zero / _one / _negative / _small
    assert ora.e4m3fn_round(0.0)[0] == 0.0
    assert abs(ora.e4m3fn_round(1.0)[0] - 1.0) < 0.01
    assert abs(ora.e4m3fn_round(-2.5)[0] - (-2.5)) < 0.1
    v = ora.e4m3fn_round(0.001)[0]
    assert 0.0 <= v <= 0.01
    # fp8_round_trip_slice_basic
    data = [0.5, -0.5, 1.0, -1.0, 2.0, -2.0, 0.0, 0.25]
    out = ora.fp8_round_trip(data, 8, 0)
    assert np.all(np.abs(out - np.float32(data)) < 0.1)
    # fp8_round_trip_slice_with_rope: the RoPE tail passes through
    out = ora.fp8_round_trip([1.0, 2.0, 3.0, 4.0, 5.0, 6.0, 999.0, 888.0], 8, 2)
    assert out[6] == 999.0 and out[7] == 888.0
    # fp8_round_trip_multiple_rows
    out = ora.fp8_round_trip([1.0, -1.0, 2.0, -2.0, 0.5, -0.5, 3.0, -3.0], 4, 0)
    assert abs(out[0] - 1.0) < 0.1 and abs(out[1] + 1.0) < 0.1 and abs(out[4] - 0.5) < 0.1
    # fp8_roundtrip_preserves_sign
    for x in [-100.0, -10.0, -1.0, -0.1, 0.1, 1.0, 10.0, 100.0]:
        assert (ora.e4m3fn_round(x)[0] < 0.0) == (x < 0.0)


# ---------------------------------------------------------- the E4M3FN format
def test_code_table_is_e4m3fn(ora):
    vals = np.array([ora.e4m3_value(c) for c in range(256)], np.float64)
    assert np.isnan(vals[0x7F]) and np.isnan(vals[0xFF])
    pos = vals[:0x7F]
    assert pos[0] == 0.0 and pos[1] == 2.0 ** -9 and pos[0x7E] == 448.0
    assert np.all(np.diff(pos) > 0), "codes 0..126 increase"
    assert np.array_equal(vals[0x80:0xFF], -pos)
    # normal codes: (1 + m/8) 2^(e-7); subnormal: m 2^-9
    for c in range(0x7F):
        e, m = c >> 3, c & 7
        want = m * 2.0 ** -9 if e == 0 else (1 + m / 8) * 2.0 ** (e - 7)
        assert pos[c] == want


def test_every_code_maps_to_itself_and_midpoints_go_even(ora):
    pos = np.array([ora.e4m3_value(c) for c in range(0x7F)], np.float64)
    for c in range(0x7F):
        v, code = ora.e4m3fn_round(pos[c])
        assert v == pos[c] and code == c
        v, code = ora.e4m3fn_round(-pos[c]) if c else (0.0, 0)
        assert v == -pos[c] and (code == (0x80 | c) or c == 0)
    for c in range(0x7E):
        mid = np.float32((pos[c] + pos[c + 1]) / 2)  # exact in f32
        assert float(mid) == (pos[c] + pos[c + 1]) / 2
        v, code = ora.e4m3fn_round(mid)
        assert code == (c if c % 2 == 0 else c + 1), (c, mid, code)
    assert ora.e4m3fn_round(460.0) == (448.0, 0x7E)
    assert ora.e4m3fn_round(1e30) == (448.0, 0x7E)
    assert ora.e4m3fn_round(float("nan")) == (448.0, 0x7E)  # f32::min(NaN, 448) = 448


def test_rounding_matches_torch_float8_on_every_bf16(ora):
    torch = pytest.importorskip("torch")
    if not hasattr(torch, "float8_e4m3fn"):
        pytest.skip("torch without float8_e4m3fn")
    x = finite_bf16_as_f32()
    x = np.clip(x, -448.0, 448.0).astype(np.float32)
    ours = ora.e4m3fn_round_array(x)
    theirs = torch.from_numpy(x).to(torch.float8_e4m3fn).to(torch.float32).numpy()
    assert np.array_equal(ours, theirs)  # -0.0 == 0.0 here; signs checked below
    nz = ours != 0
    assert np.array_equal(np.signbit(ours[nz]), np.signbit(theirs[nz]))


# ------------------------------------------------------------ block exponent
def test_exponent_forms_agree_near_powers_of_two(ora):
    """ceil(f32 log2(r)) (the reference) == ceil(f32(double log2(r))) (the kernels)."""
    assert ora.fp8_exp_mismatches(-40, 126, 4096) == 0


def test_exponent_exact_cases(ora):
    assert ora.fp8_exp_of(1.0) == 0
    assert ora.fp8_exp_of(0.5) == -1
    assert ora.fp8_exp_of(0.75) == 0
    assert ora.fp8_exp_of(2.0 ** -20) == -20
    # one ulp above 2^-20 the f32 log2 is exactly -20.0 (the true value is within half an
    # ulp of it), so the reference's exponent stays -20 and that element saturates at 448;
    # both forms agree on this
    r = np.nextafter(np.float32(2.0 ** -20), np.float32(1))
    assert ora.fp8_exp_of(r) == -20 and ora.fp8_exp_of(r, ref=False) == -20
    assert ora.fp8_exp_of(np.float32(2.0 ** -20 * 1.001)) == -19
    # amax floor 1e-4: an all-zero block gets ceil(log2(1e-4 / 448)) = -22
    codes, exps = ora.fp8_quantize(np.zeros((1, 128), np.float32))
    assert np.all(codes == 0) and np.all(exps == -22)


def test_block_scale_invariants(ora):
    rng = np.random.default_rng(3)
    rows = (rng.standard_normal((512, 128)) * np.exp(rng.uniform(-12, 12, (512, 1)))).astype(np.float32)
    rows = ora.f32_from_bf16(ora.bf16_from_f32(rows))
    codes, exps = ora.fp8_quantize(rows)
    deq = ora.fp8_dequantize(codes, exps)
    # the stored form equals the reference's in-place round trip
    assert np.array_equal(deq, ora.fp8_round_trip(rows, 128, 0))
    # idempotent: quantising the decoded rows changes nothing
    c2, e2 = ora.fp8_quantize(deq)
    assert np.array_equal(ora.fp8_dequantize(c2, e2), deq)
    blocks = np.abs(rows.reshape(-1, 64))
    amax = np.maximum(blocks.max(axis=1), np.float32(1e-4))
    s = np.ldexp(1.0, exps.reshape(-1).astype(np.int32))
    r = amax / s
    # amax / scale lands in (224, 448] (a few ulps above 448 in the band where the f32 log2
    # rounds to the integer below; that element then saturates)
    assert np.all(r <= 448.0 * (1 + 2 ** -18)) and np.all(r > 224.0), "amax lands in the top binade"
    # relative error of normal-range codes <= 2^-4 (3 mantissa bits, round to nearest)
    d = deq.reshape(-1, 64)
    xs = rows.reshape(-1, 64)
    normal = np.abs(xs) >= (s[:, None] * 2.0 ** -6)
    rel = np.abs(d - xs)[normal] / np.abs(xs)[normal]
    assert rel.max() <= 2.0 ** -4
    # decoded values are exactly representable in bf16 (what the GPU decoder produces)
    assert np.array_equal(ora.f32_from_bf16(ora.bf16_from_f32(deq)), deq)
