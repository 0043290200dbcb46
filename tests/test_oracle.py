"""Pins for the CPU oracle (runs without a GPU).

Each oracle function is checked against something other than a retyping of
its own formula: the reference's own test data (RMSNorm closed forms,
crates/mlx-ffi/tests/grouped_rms_norm.rs; the KV-write pattern,
crates/serve/tests/profile_decode.rs:222-260), closed forms, invariants, and a
numpy brute force written in a different form (whole-matrix softmax with the
reference's additive -1e9 mask instead of the oracle's streaming exclusion).
"""
import json
import math
import os

import numpy as np
import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
FIX = json.load(open(os.path.join(HERE, "golden", "reference_fixtures.json")))


def np_bf16(x):
    """Independent RNE float32 -> bf16 bits (numpy integer ops)."""
    u = np.asarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    r = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    return r.astype(np.uint16)


def np_f32(h):
    return (np.asarray(h, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


# ---------------------------------------------------------------- bf16
def test_bf16_roundtrip_matches_independent_rne(ora):
    rng = np.random.default_rng(0)
    x = rng.standard_normal(100000).astype(np.float32) * np.float32(1e3)
    # exact ties: values halfway between two bf16 numbers
    ties = (np.arange(1, 2000, dtype=np.uint32) << 16 | 0x8000).view(np.float32)
    x = np.concatenate([x, ties, -ties, np.float32([0.0, -0.0, 1.0, np.inf, -np.inf])])
    assert np.array_equal(ora.bf16_from_f32(x), np_bf16(x))
    h = np.arange(0, 65536, dtype=np.uint16)
    finite = np.isfinite(np_f32(h))
    assert np.array_equal(ora.f32_from_bf16(h)[finite], np_f32(h)[finite])


def test_bf16_known_answers(ora):
    m = FIX["mask"]
    b = ora.bf16_from_f32(np.float32([1.0, 1.00390625, 1.01171875, m["masked_value"]]))
    # 1+2^-8 is a tie -> even (1.0); 1+3*2^-8 is a tie -> even (1+2^-6)
    assert list(b[:3]) == [0x3F80, 0x3F80, 0x3F82]
    assert int(b[3]) == m["masked_value_bf16_bits"]
    assert float(ora.f32_from_bf16(b[3:4])[0]) == m["masked_value_bf16"]
    # the additive mask underflows exp to exactly zero in f32 (exclusion == mask)
    assert np.exp(np.float32(m["masked_value_bf16"]) - np.float32(10.0)) == 0.0


def test_generator_is_counter_based_and_normal(ora):
    a = ora.normal_f32(200000, seed=7)
    b = ora.normal_f32(1000, seed=7)
    assert np.array_equal(a[:1000], b)
    assert abs(a.mean()) < 0.01 and abs(a.std() - 1.0) < 0.01
    assert not np.array_equal(a[:1000], ora.normal_f32(1000, seed=8))


# ------------------------------------------------------------- RMSNorm
def _reference_groups(x, w, eps, groups):
    """crates/mlx-ffi/tests/grouped_rms_norm.rs:27-44 (f32 closed form)."""
    x = np.asarray(x, np.float32)
    w = np.asarray(w, np.float32)
    dims = x.shape[-1]
    per = dims // groups
    out = np.zeros_like(x)
    for g in range(groups):
        s = slice(g * per, (g + 1) * per)
        ms = np.float32(np.sum(x[..., s] * x[..., s], axis=-1, keepdims=True, dtype=np.float32) / np.float32(per))
        out[..., s] = w[s] * (x[..., s] / np.sqrt(ms + np.float32(eps)))
    return out


@pytest.mark.parametrize("case", FIX["rms_norm"], ids=lambda c: c["source"].split(":")[-1])
def test_rms_norm_reference_fixtures(ora, case):
    shape = case["shape"]
    x = np.full(shape, case["x_fill"], np.float32) if "x_fill" in case else np.asarray(case["x"], np.float32).reshape(shape)
    w = np.asarray(case["w"], np.float32)
    expected = _reference_groups(x, w, case["eps"], 1)
    got = np_f32(ora.rms_norm(np_bf16(x), np_bf16(w), case["eps"]))
    tol = case["bf16_rel_tol"]
    assert np.all(np.abs(got - expected) <= tol * (1.0 + np.abs(expected))), (got, expected)


def test_rms_norm_invariants(ora):
    rng = np.random.default_rng(1)
    D = 128
    x = np_bf16(rng.standard_normal((64, D)))
    ones = np_bf16(np.ones(D))
    y = np_f32(ora.rms_norm(x, ones, 1e-6))
    # unit weight -> unit RMS (up to bf16 rounding of each element)
    rms = np.sqrt(np.mean(y.astype(np.float64) ** 2, axis=1))
    assert np.all(np.abs(rms - 1.0) < 4e-3)
    # scale invariance: a power-of-two scale is exact in bf16
    x4 = np_bf16(np_f32(x) * 4.0)
    assert np.array_equal(ora.rms_norm(x4, ones, 0.0), ora.rms_norm(x, ones, 0.0))
    # weight applies per column after the normalised value is rounded
    w = np_bf16(1.0 + 0.02 * rng.standard_normal(D))
    yw = np_f32(ora.rms_norm(x, w, 1e-6))
    assert np.array_equal(yw, np_f32(np_bf16(y * np_f32(w))))
    # a dropped eps is visible on a tiny row
    small = np_bf16(np.full((1, D), 1e-4))
    assert np_f32(ora.rms_norm(small, ones, 1e-6))[0, 0] < 0.2


# ---------------------------------------------------------------- RoPE
def test_rope_closed_form_unit_vectors(ora):
    """e_i -> (cos, sin) at (i, i+D/2); e_{i+D/2} -> (-sin, cos): split-half pairs,
    angle pos * theta^(-2i/D)."""
    D, theta = 128, 1e6
    half = D // 2
    for pos in (0, 1, 7, 1023, 14336):
        for i in (0, 1, 5, 31, 63):
            e = np.zeros((2, D), np.float32)
            e[0, i] = 1.0
            e[1, i + half] = 1.0
            y = np_f32(ora.rope(np_bf16(e), np.array([pos, pos], np.int32), theta))
            ang = pos * theta ** (-2.0 * i / D)
            c, s = math.cos(ang), math.sin(ang)
            tol = 4e-3 + 2e-7 * pos  # bf16 output + f32 angle formation
            assert abs(y[0, i] - c) < tol and abs(y[0, i + half] - s) < tol
            assert abs(y[1, i] + s) < tol and abs(y[1, i + half] - c) < tol
            others = np.delete(y, [i, i + half], axis=1)
            assert np.all(others == 0.0)


def test_rope_position_zero_is_identity(ora):
    x = ora.normal_bf16((16, 128), seed=3)
    assert np.array_equal(ora.rope(x, np.zeros(16, np.int32), 1e6), x)


def test_rope_preserves_pair_norms_and_composes(ora):
    rng = np.random.default_rng(2)
    D, theta = 128, 1e4
    x = np_bf16(rng.standard_normal((8, D)))
    pa, pb = 37, 91
    ya = np_f32(ora.rope(x, np.full(8, pa, np.int32), theta))
    xf = np_f32(x)
    n0 = xf[:, :64] ** 2 + xf[:, 64:] ** 2
    n1 = ya[:, :64] ** 2 + ya[:, 64:] ** 2
    assert np.allclose(n0, n1, rtol=2e-2, atol=2e-2)
    yab = np_f32(ora.rope(np_bf16(ya), np.full(8, pb, np.int32), theta))
    ysum = np_f32(ora.rope(x, np.full(8, pa + pb, np.int32), theta))
    assert np.max(np.abs(yab - ysum)) < 5e-2


def test_rope_relative_position(ora):
    """<R(p)q, R(p')k> depends only on p - p'."""
    rng = np.random.default_rng(3)
    q = np_bf16(rng.standard_normal((1, 128)))
    k = np_bf16(rng.standard_normal((1, 128)))
    dots = []
    for p in (10, 500, 3000):
        rq = np_f32(ora.rope(q, np.array([p + 5], np.int32), 1e6)).astype(np.float64)
        rk = np_f32(ora.rope(k, np.array([p], np.int32), 1e6)).astype(np.float64)
        dots.append(float((rq @ rk.T)[0, 0]))
    assert max(dots) - min(dots) < 0.25


# ---------------------------------------------------------- KV write
def test_kv_write_reference_pattern(ora):
    """crates/serve/tests/profile_decode.rs:222-260: a 999.0 update at offset 7
    lands in row 7 of every kv head; every other element keeps its bits."""
    f = FIX["kv_write"]
    Hkv, D, cap, off = f["n_kv_heads"], f["head_dim"], f["capacity"], f["offset"]
    base = np_bf16(np.arange(Hkv * cap * D, dtype=np.float32) * 0.5 + 1.0).reshape(1, Hkv, cap, D)
    kc, vc = base.copy(), base.copy()
    Hq = Hkv
    qkv = np.zeros((1, 1, (Hq + 2 * Hkv) * D), np.uint16)
    qkv[..., Hq * D:] = np_bf16(np.float32(f["update_value"]))
    ora.pre_attention(qkv, None, None, 1e-6, 1e6, [off], Hq, Hkv, kc, vc,
                      flags=ora.FLAG_NO_NORM | ora.FLAG_NO_ROPE)
    for c in (kc, vc):
        assert np.all(c[:, :, off, :] == np_bf16(np.float32(f["update_value"])))
        keep = np.ones(cap, bool)
        keep[off] = False
        assert np.array_equal(c[:, :, keep, :], base[:, :, keep, :])


def test_pre_attention_prefill_equals_token_by_token(ora):
    """A T-token write at off equals T single-token writes (prefill slice_update
    vs decode scatter_single, crates/serve/src/forward_qwen3.rs:124-142 and
    crates/serve/src/compiled.rs:157-161)."""
    B, T, Hq, Hkv, D, cap = 2, 5, 4, 2, 128, 16
    qkv = ora.normal_bf16((B, T, (Hq + 2 * Hkv) * D), seed=11)
    qw = ora.normal_bf16(D, seed=12, mean=1.0, std=0.02)
    kw = ora.normal_bf16(D, seed=13, mean=1.0, std=0.02)
    off = np.array([3, 9], np.int32)
    junk = ora.normal_bf16((B, Hkv, cap, D), seed=14)
    k1, v1 = junk.copy(), junk.copy()
    q1 = ora.pre_attention(qkv, qw, kw, 1e-6, 1e6, off, Hq, Hkv, k1, v1)
    k2, v2 = junk.copy(), junk.copy()
    q2 = np.empty_like(q1)
    for t in range(T):
        q2[:, :, t:t + 1] = ora.pre_attention(qkv[:, t:t + 1].copy(), qw, kw, 1e-6, 1e6, off + t, Hq, Hkv, k2, v2)
    assert np.array_equal(q1, q2) and np.array_equal(k1, k2) and np.array_equal(v1, v2)
    # rows outside [off, off+T) untouched
    for b in range(B):
        rows = np.r_[0:off[b], off[b] + T:cap]
        assert np.array_equal(k1[b][:, rows], junk[b][:, rows])
    # v is a bit copy of the v slice; k is rope(norm(k))
    vsrc = qkv[:, :, (Hq + Hkv) * D:].reshape(B, T, Hkv, D).transpose(0, 2, 1, 3)
    for b in range(B):
        assert np.array_equal(v1[b, :, off[b]:off[b] + T], vsrc[b])
    ksrc = qkv[0, :, Hq * D:(Hq + Hkv) * D].reshape(T, Hkv, D).transpose(1, 0, 2)
    kref = ora.rope(ora.rms_norm(ksrc.copy(), kw, 1e-6).reshape(-1, D),
                    np.tile(off[0] + np.arange(T, dtype=np.int32), Hkv), 1e6).reshape(Hkv, T, D)
    assert np.array_equal(k1[0, :, off[0]:off[0] + T], kref)


@pytest.mark.parametrize("one_sided", ["q", "k"])
def test_pre_attention_one_sided_norm(ora, one_sided):
    """optional_qk_norm (crates/ops/src/attention.rs:57-76) normalises q and k each on its
    own: with only k_norm given, q is the un-normalised (rotated) q of the NO_NORM call and
    k the normalised k of the full call; and the other way round."""
    B, T, Hq, Hkv, D, cap = 2, 3, 4, 2, 128, 16
    qkv = ora.normal_bf16((B, T, (Hq + 2 * Hkv) * D), seed=21)
    qw = ora.normal_bf16(D, seed=22, mean=1.0, std=0.02)
    kw = ora.normal_bf16(D, seed=23, mean=1.0, std=0.02)
    off = np.array([2, 7], np.int32)
    junk = ora.normal_bf16((B, Hkv, cap, D), seed=24)
    runs = {}
    for name, flags in (("both", 0), ("none", ora.FLAG_NO_NORM),
                        ("q", ora.FLAG_NO_Q_NORM), ("k", ora.FLAG_NO_K_NORM)):
        kc, vc = junk.copy(), junk.copy()
        q = ora.pre_attention(qkv, None if name in ("none", "q") else qw, None if name in ("none", "k") else kw,
                              1e-6, 1e6, off, Hq, Hkv, kc, vc, flags=flags)
        runs[name] = (q, kc, vc)
    q1, k1, v1 = runs[one_sided]
    q_src = runs["none"] if one_sided == "q" else runs["both"]
    k_src = runs["both"] if one_sided == "q" else runs["none"]
    assert np.array_equal(q1, q_src[0]) and np.array_equal(k1, k_src[1]) and np.array_equal(v1, junk_v(runs))
    assert not np.array_equal(q1, runs["both" if one_sided == "q" else "none"][0])


def junk_v(runs):
    v = runs["both"][2]
    assert all(np.array_equal(r[2], v) for r in runs.values())  # v never normalised
    return v


def test_pre_attention_overflow_raises(ora):
    kc = np.zeros((1, 1, 8, 128), np.uint16)
    qkv = np.zeros((1, 2, 3 * 128), np.uint16)
    with pytest.raises(ValueError, match="overflow"):
        ora.pre_attention(qkv, None, None, 1e-6, 1e6, [7], 1, 1, kc, kc.copy())


# ---------------------------------------------------------------- SDPA
def _np_sdpa(q, kc, vc, kv_len, scale, causal):
    """Brute force: whole-matrix scores plus the reference's additive mask
    (0 / -1e9 rounded to bf16, crates/serve/src/engine_ext.rs:237-260), f64."""
    B, Hq, Tq, D = q.shape
    Hkv, cap = kc.shape[1], kc.shape[2]
    G = Hq // Hkv
    neg = float(np_f32(np_bf16(np.float32(-1e9))))
    out = np.zeros((B, Tq, Hq, D))
    for b in range(B):
        L = int(kv_len[b])
        pos = np.arange(cap)
        for h in range(Hq):
            K = np_f32(kc[b, h // G]).astype(np.float64)
            V = np_f32(vc[b, h // G]).astype(np.float64)
            Q = np_f32(q[b, h]).astype(np.float64)
            S = scale * Q @ K.T
            lim = (L - Tq + np.arange(Tq))[:, None] if causal else np.full((Tq, 1), L - 1)
            mask = np.where(pos[None, :] <= lim, 0.0, neg)
            S = S + mask
            S = np.where(np.isfinite(S), S, neg)  # stale NaN rows are masked
            P = np.exp(S - S.max(axis=1, keepdims=True))
            P = P / P.sum(axis=1, keepdims=True)
            Vz = np.where(pos[:, None] < L, V, 0.0)
            out[b, :, h] = P @ Vz
    return out.reshape(B, Tq, Hq * D)


@pytest.mark.parametrize("G", [1, 2, 4, 8])
@pytest.mark.parametrize("causal,Tq", [(False, 1), (True, 1), (True, 5)])
def test_sdpa_brute_force(ora, G, causal, Tq):
    B, Hkv, D, cap = 2, 2, 64, 40
    Hq = Hkv * G
    q = ora.normal_bf16((B, Hq, Tq, D), seed=21 + G)
    kc = ora.normal_bf16((B, Hkv, cap, D), seed=22 + G)
    vc = ora.normal_bf16((B, Hkv, cap, D), seed=23 + G)
    kv_len = np.array([17, 33], np.int32)
    scale = 1.0 / math.sqrt(D)
    got = np_f32(ora.sdpa(q, kc, vc, kv_len, scale, causal))
    ref = _np_sdpa(q, kc, vc, kv_len, scale, causal)
    assert np.max(np.abs(got - ref)) <= 2.0 ** -8 * np.max(np.abs(ref)) + 1e-6


def test_sdpa_invariants(ora):
    B, Hq, Hkv, D, cap = 1, 8, 2, 128, 64
    G = Hq // Hkv
    q = ora.normal_bf16((B, Hq, 1, D), seed=31)
    kc = ora.normal_bf16((B, Hkv, cap, D), seed=32)
    L = np.array([50], np.int32)
    s = 1.0 / math.sqrt(D)
    # constant V per kv head -> each q head returns its group's constant (GQA map h -> h/G)
    vc = np.zeros((B, Hkv, cap, D), np.uint16)
    for kh in range(Hkv):
        vc[0, kh] = np_bf16(np.float32(kh + 1.5))
    out = np_f32(ora.sdpa(q, kc, vc, L, s, False)).reshape(Hq, D)
    for h in range(Hq):
        assert np.all(out[h] == h // G + 1.5)
    # one dominant key -> its value
    vr = ora.normal_bf16((B, Hkv, cap, D), seed=33)
    kd = kc.copy()
    kd[0, :, 20] = np_bf16(np_f32(q[0, ::G, 0]) * 64.0)
    out = np_f32(ora.sdpa(q[:, ::G].copy(), kd, vr, L, s, False)).reshape(Hkv, D)
    assert np.max(np.abs(out - np_f32(vr[0, :, 20]))) < 1e-2
    # key permutation invariance (same permutation on K and V)
    perm = np.random.default_rng(4).permutation(50)
    kp, vp = kc.copy(), vr.copy()
    kp[:, :, :50] = kc[:, :, perm]
    vp[:, :, :50] = vr[:, :, perm]
    a = np_f32(ora.sdpa(q, kc, vr, L, s, False))
    b = np_f32(ora.sdpa(q, kp, vp, L, s, False))
    assert np.max(np.abs(a - b)) <= 2.0 ** -8 * np.max(np.abs(a))


def test_sdpa_stale_tail_and_capacity_independence(ora):
    """Rows >= kv_len never matter: NaN/inf poison and a larger cap give bit-identical output."""
    B, Hq, Hkv, D, cap = 2, 4, 2, 128, 48
    q = ora.normal_bf16((B, Hq, 1, D), seed=41)
    kc = ora.normal_bf16((B, Hkv, cap, D), seed=42)
    vc = ora.normal_bf16((B, Hkv, cap, D), seed=43)
    L = np.array([19, 31], np.int32)
    ref = ora.sdpa(q, kc, vc, L, 0.088, False)
    kp, vp = kc.copy(), vc.copy()
    for b in range(B):
        kp[b, :, L[b]:] = 0x7FC0  # NaN
        vp[b, :, L[b]:] = 0x7F80  # +inf
    assert np.array_equal(ora.sdpa(q, kp, vp, L, 0.088, False), ref)
    big_k = np.full((B, Hkv, 4 * cap, D), 0x7FC0, np.uint16)
    big_v = big_k.copy()
    big_k[:, :, :cap] = kc
    big_v[:, :, :cap] = vc
    assert np.array_equal(ora.sdpa(q, big_k, big_v, L, 0.088, False), ref)


def test_prefill_rows_equal_decode(ora):
    """Causal row i over kv_len = off+T equals decode with kv_len = off+i+1."""
    B, Hq, Hkv, D, cap, T, off = 1, 4, 2, 128, 64, 6, 20
    q = ora.normal_bf16((B, Hq, T, D), seed=51)
    kc = ora.normal_bf16((B, Hkv, cap, D), seed=52)
    vc = ora.normal_bf16((B, Hkv, cap, D), seed=53)
    pre = ora.sdpa(q, kc, vc, [off + T], 0.1, True)
    for i in range(T):
        dec = ora.sdpa(q[:, :, i:i + 1].copy(), kc, vc, [off + i + 1], 0.1, False)
        assert np.array_equal(pre[:, i], dec[:, 0])
    # chunk-only window (kv_begin = off) equals attention over the chunk alone
    chunk = ora.sdpa(q, kc, vc, [off + T], 0.1, True, kv_begin=[off])
    alone = ora.sdpa(q, kc[:, :, off:off + T].copy(), vc[:, :, off:off + T].copy(), [T], 0.1, True)
    assert np.array_equal(chunk, alone)


def test_split_k_lse_merge_equals_unsplit(ora):
    D, n = 128, 300
    q = ora.normal_bf16(D, seed=61)
    k = ora.normal_bf16((n, D), seed=62)
    v = ora.normal_bf16((n, D), seed=63)
    k[::37] = np_bf16(np_f32(k[::37]) * 8.0)  # outliers stress the running max
    m, l, acc = ora.sdpa_partial(q, k, v, 0.088)
    whole = acc / l
    for parts in (1, 2, 3, 7, 16, 300):
        cuts = np.linspace(0, n, parts + 1).astype(int)
        ms, ls, accs = [], [], []
        for a, b in zip(cuts[:-1], cuts[1:]):
            mm, ll, aa = ora.sdpa_partial(q, k[a:b].copy(), v[a:b].copy(), 0.088)
            ms.append(mm)
            ls.append(ll)
            accs.append(aa)
        merged = ora.lse_merge(ms, ls, np.array(accs))
        assert np.allclose(merged, whole, rtol=1e-12, atol=1e-13)
    # merge matches the full sdpa oracle after bf16 rounding
    kc = k.reshape(1, 1, n, D)
    vc = v.reshape(1, 1, n, D)
    o = ora.sdpa(q.reshape(1, 1, 1, D), kc, vc, [n], 0.088, False)
    assert np.array_equal(o.reshape(D), np_bf16(whole.astype(np.float32)))


def test_f32_mode_within_tolerance(ora):
    B, Hq, Hkv, D, cap = 2, 8, 2, 128, 256
    q = ora.normal_bf16((B, Hq, 1, D), seed=71)
    kc = ora.normal_bf16((B, Hkv, cap, D), seed=72)
    vc = ora.normal_bf16((B, Hkv, cap, D), seed=73)
    L = np.array([200, 256], np.int32)
    a = np_f32(ora.sdpa(q, kc, vc, L, 0.088, False, precision=0))
    b = np_f32(ora.sdpa(q, kc, vc, L, 0.088, False, precision=1))
    assert np.max(np.abs(a - b)) < 2e-2 and np.mean(np.abs(a - b)) < 2e-3


def test_empty_window_gives_zeros(ora):
    q = ora.normal_bf16((1, 2, 1, 128), seed=81)
    kc = ora.normal_bf16((1, 1, 8, 128), seed=82)
    out = ora.sdpa(q, kc, kc, [0], 0.1, False)
    assert np.all(out == 0)
