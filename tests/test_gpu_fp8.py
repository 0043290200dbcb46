"""GPU parity of the FP8 E4M3FN KV cache (the stored form of the reference's
Fp8Cache, crates/kvcache/src/fp8.rs over crates/ops/src/fp8.rs), through the C ABI.

Bars:
  - written rows: codes and block exponents bit-exact against the oracle's
    quantisation of the same bf16 row (every finite bf16 value is exercised);
  - decode over an FP8 cache matches decode over a bf16 cache that holds the
    decoded values to max-abs 2e-3 / mean-abs 1e-5 (the decoder is exact; only
    the dot product's summation order differs), and is within the bf16
    tolerance (max-abs 2e-2, mean-abs 2e-3) of the f64 oracle;
  - the fused step writes the same codes as the oracle and attends within the
    same tolerance.
"""
import numpy as np
import pytest

from gpu_util import assert_close, dev, host, say, scale_of

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ema():
    import torch

    if not torch.cuda.is_available():
        pytest.fail("GPU tests need a ROCm GPU")
    import ema_attn

    ema_attn.lib()
    return ema_attn


def fp8_cache(ema, codes_k, exps_k, codes_v, exps_v):
    B, Hkv, cap, D = codes_k.shape
    return ema.StaticCache(B, Hkv, cap, D, dtype="fp8", k=dev(codes_k), v=dev(codes_v), k_exp=dev(exps_k),
                           v_exp=dev(exps_v))


def quantized_pair(ora, shape, seed, outliers=False):
    """Random bf16 K/V rows quantised by the oracle: (codes, exps, decoded bf16) for K and V."""
    out = []
    for i in range(2):
        x = ora.normal_f32(shape, seed=seed + i)
        if outliers and i == 0:  # 1% of K entries x8
            sel = np.random.default_rng(seed).random(shape, dtype=np.float32) < 0.01
            x[sel] *= 8.0
        x = ora.f32_from_bf16(ora.bf16_from_f32(x))
        codes, exps = ora.fp8_quantize(x)
        deq = ora.bf16_from_f32(ora.fp8_dequantize(codes, exps))
        out.append((codes, exps, deq))
    return out


def random_fp8_pair(ora, shape, seed):
    """Random finite E4M3FN codes with block exponents in {-8, -7} (values of N(0,1) size):
    (codes, exps, decoded bf16) for K and V, decoded through the oracle's code table."""
    rng = np.random.default_rng(seed)
    table = np.array([ora.e4m3_value(c) for c in range(256)], np.float32)
    out = []
    for _ in range(2):
        codes = rng.integers(0, 254, size=shape, dtype=np.uint8)
        codes = codes + (codes >= 0x7F)  # skip the NaN code 0x7F (and 0xFF: max 254 + 1)
        exps = rng.integers(-8, -6, size=shape[:-1] + (shape[-1] // 64,), dtype=np.int8)
        vals = table[codes] * np.ldexp(np.float32(1), np.repeat(exps, 64, axis=-1).astype(np.int32))
        out.append((codes, exps, ora.bf16_from_f32(vals)))
    return out


def canon(codes):
    """-0 (0x80) and +0 (0x00) are the same value."""
    c = np.asarray(codes).copy()
    c[c == 0x80] = 0
    return c


# ------------------------------------------------------------------ writes
def test_fp8_write_every_bf16_value(ema, ora):
    """pre_attention without norm/RoPE writes k, v as given: their codes must be the
    oracle's for all 65536 bf16 bit patterns (non-finite ones replaced by 0)."""
    import torch

    B, T, Hq, Hkv, D, cap = 1, 64, 8, 8, 128, 80
    say("fp8 write: every bf16 pattern")
    pats = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    f = (pats.astype(np.uint32) << 16).view(np.float32)
    pats[~np.isfinite(f)] = 0
    k = pats.reshape(T, Hkv, D)
    v = pats[::-1].copy().reshape(T, Hkv, D)  # other block compositions
    qkv = np.zeros((B, T, (Hq + 2 * Hkv) * D), np.uint16)
    qkv[0, :, Hq * D:(Hq + Hkv) * D] = k.reshape(T, -1)
    qkv[0, :, (Hq + Hkv) * D:] = v.reshape(T, -1)
    off = np.array([9], np.int32)
    cache = ema.StaticCache(B, Hkv, cap, D, dtype="fp8")
    ema.pre_attention(dev(qkv), None, None, 1e-6, 1e6, dev(off), Hq, cache, flags=3)
    torch.cuda.synchronize()
    for name, src, codes, exps in (("k", k, cache.k, cache.k_exp), ("v", v, cache.v, cache.v_exp)):
        rows = ora.f32_from_bf16(np.ascontiguousarray(src.transpose(1, 0, 2)))  # [Hkv, T, D]
        rc, re = ora.fp8_quantize(rows)
        gc, ge = host(codes)[0], host(exps)[0]
        assert np.array_equal(canon(gc[:, 9:9 + T]), canon(rc)), f"{name} codes"
        assert np.array_equal(ge[:, 9:9 + T], re), f"{name} exponents"
        assert np.all(gc[:, :9] == 0) and np.all(gc[:, 9 + T:] == 0) and np.all(ge[:, :9] == 0)


@pytest.mark.parametrize("flags", [0, 2])
def test_fp8_write_after_norm_rope(ema, ora, flags):
    """With norm and RoPE the written codes are the oracle's quantisation of the bf16 k
    the same kernel writes into a bf16 cache (which the bf16 tests hold to the oracle)."""
    import torch

    B, T, Hq, Hkv, D, cap = 2, 7, 16, 8, 128, 64
    say(f"fp8 write after norm/rope flags={flags}")
    qkv = ora.normal_bf16((B, T, (Hq + 2 * Hkv) * D), seed=700 + flags)
    qw = ora.normal_bf16(D, seed=701, mean=1.0, std=0.02)
    kw = ora.normal_bf16(D, seed=702, mean=1.0, std=0.02)
    off = np.array([0, 40], np.int32)
    c16 = ema.StaticCache(B, Hkv, cap, D)
    c8 = ema.StaticCache(B, Hkv, cap, D, dtype="fp8")
    q16 = ema.pre_attention(dev(qkv), dev(qw), dev(kw), 1e-6, 1e6, dev(off), Hq, c16, flags=flags)
    q8 = ema.pre_attention(dev(qkv), dev(qw), dev(kw), 1e-6, 1e6, dev(off), Hq, c8, flags=flags)
    torch.cuda.synchronize()
    assert np.array_equal(host(q16), host(q8)), "q does not depend on the cache format"
    for src, codes, exps in ((c16.k, c8.k, c8.k_exp), (c16.v, c8.v, c8.v_exp)):
        rows = ora.f32_from_bf16(host(src))
        rc, re = ora.fp8_quantize(rows)
        for b in range(B):
            sl = slice(off[b], off[b] + T)
            assert np.array_equal(canon(host(codes)[b][:, sl]), canon(rc[b][:, sl]))
            assert np.array_equal(host(exps)[b][:, sl], re[b][:, sl])


# ------------------------------------------------------------------ decode
@pytest.mark.parametrize("G,lengths,cap", [
    (4, [1, 31, 32, 33, 100, 1000, 1024], 1024),
    (8, [4096, 17, 2500], 4096),
    (1, [64, 65, 3], 96),
    (2, [203, 1, 150, 97], 203),  # capacity not a multiple of 8: exponents loaded row by row
    (5, [256, 77, 1, 200], 256),  # 5 query heads per kv head (Qwen3-14B)
])
def test_fp8_decode_equals_bf16_decode_of_decoded_cache(ema, ora, G, lengths, cap):
    import torch

    Hkv, D = 4, 128
    B, Hq = len(lengths), 4 * G
    say(f"fp8 decode == bf16 decode G={G} lengths={lengths}")
    (kc, ke, kd), (vc, ve, vd) = quantized_pair(ora, (B, Hkv, cap, D), seed=710 + G, outliers=True)
    q = ora.normal_bf16((B, Hq, 1, D), seed=715)
    L = np.asarray(lengths, np.int32)
    c8 = fp8_cache(ema, kc, ke, vc, ve)
    c16 = ema.StaticCache(B, Hkv, cap, D, k=dev(kd), v=dev(vd))
    o8 = ema.decode_attention(dev(q), c8, dev(L), int(L.max()))
    o16 = ema.decode_attention(dev(q), c16, dev(L), int(L.max()))
    torch.cuda.synchronize()
    # same values, same arithmetic; only the order in which the QK dot product visits the
    # head dims differs (the fp8 layout reads 16 contiguous codes per lane), so outputs
    # differ by f32 summation order only: a bf16 ulp here and there
    assert_close(host(o8), host(o16), "fp8 vs bf16 decode of the decoded cache", max_abs=2e-3, mean_abs=1e-5)
    assert_close(host(o8), ora.sdpa(q, kd, vd, L, scale_of(D), False), "fp8 decode vs oracle")


@pytest.mark.parametrize("cap,lengths", [(1024, [1, 31, 33, 700, 1000]), (203, [1, 33, 150, 202])])
def test_fp8_decode_stale_rows_are_never_used(ema, ora, cap, lengths):
    """Rows at or past each length hold NaN codes and the largest exponent: the output is
    bit-identical to that of a clean cache (16-byte exponent groups with a capacity that is
    a multiple of 8; row-by-row exponents otherwise)."""
    import torch

    Hkv, D, G = 2, 128, 4
    B, Hq = len(lengths), Hkv * G
    say(f"fp8 decode stale-row poison cap={cap} lengths={lengths}")
    (kc, ke, _), (vc, ve, _) = quantized_pair(ora, (B, Hkv, cap, D), seed=741)
    q = ora.normal_bf16((B, Hq, 1, D), seed=742)
    L = np.asarray(lengths, np.int32)
    outs = []
    for poison in (False, True):
        k2, e2, v2, f2 = kc.copy(), ke.copy(), vc.copy(), ve.copy()
        if poison:
            for b in range(B):
                k2[b, :, L[b]:] = 0x7F  # E4M3FN NaN
                v2[b, :, L[b]:] = 0x7F
                e2[b, :, L[b]:] = 127
                f2[b, :, L[b]:] = 127
        c8 = fp8_cache(ema, k2, e2, v2, f2)
        outs.append(host(ema.decode_attention(dev(q), c8, dev(L), cap)))
        torch.cuda.synchronize()
    assert np.array_equal(outs[0], outs[1]), "stale rows changed the output"
    assert np.all(np.isfinite(ora.f32_from_bf16(outs[1])))


def test_fp8_decode_qwen3_8b_batched_shape(ema, ora):
    """Batch 32, 32q/8kv, cap 8192, lengths U[512, 8192] (the benchmark workload)."""
    import torch

    B, Hq, Hkv, D, cap = 32, 32, 8, 128, 8192
    L = np.random.default_rng(1234).integers(512, 8193, size=B).astype(np.int32)
    say("fp8 decode B32 32q/8kv cap 8192")
    (kc, ke, kd), (vc, ve, vd) = random_fp8_pair(ora, (B, Hkv, cap, D), seed=720)
    q = ora.normal_bf16((B, Hq, 1, D), seed=722)
    c8 = fp8_cache(ema, kc, ke, vc, ve)
    del kc, vc
    o8 = ema.decode_attention(dev(q), c8, dev(L), cap)
    torch.cuda.synchronize()
    assert_close(host(o8), ora.sdpa(q, kd, vd, L, scale_of(D), False), "fp8 decode 8B batched")


# ------------------------------------------------------------------ fused step
@pytest.mark.parametrize("flags", [0, 3])
def test_fp8_fused_step(ema, ora, flags):
    """decode_step on an fp8 cache: the new row is quantised like pre_attention's and
    attended in its decoded form; rows elsewhere stay untouched."""
    import torch

    B, Hq, Hkv, D, cap = 6, 16, 4, 128, 200
    off = np.array([0, 31, 32, 100, 199, 63], np.int32)
    say(f"fp8 fused step flags={flags}")
    (kc, ke, kd), (vc, ve, vd) = quantized_pair(ora, (B, Hkv, cap, D), seed=730)
    qkv = ora.normal_bf16((B, (Hq + 2 * Hkv) * D), seed=733)
    qw = ora.normal_bf16(D, seed=734, mean=1.0, std=0.02)
    kw = ora.normal_bf16(D, seed=735, mean=1.0, std=0.02)
    # the same step through the separate kernels (pre_attention writes the row)
    c_pair = fp8_cache(ema, kc, ke, vc, ve)
    q = ema.pre_attention(dev(qkv.reshape(B, 1, -1)), dev(qw), dev(kw), 1e-6, 1e6, dev(off), Hq, c_pair,
                          flags=flags)
    pair = ema.decode_attention(q, c_pair, dev(off + 1), cap)
    c_f = fp8_cache(ema, kc, ke, vc, ve)
    fused = ema.decode_step(dev(qkv), dev(qw), dev(kw), 1e-6, 1e6, dev(off), Hq, c_f, cap, flags=flags)
    torch.cuda.synchronize()
    gk, gke, gv, gve = host(c_f.k), host(c_f.k_exp), host(c_f.v), host(c_f.v_exp)
    pk, pke = host(c_pair.k), host(c_pair.k_exp)
    assert np.array_equal(canon(gv), canon(host(c_pair.v))) and np.array_equal(gve, host(c_pair.v_exp))
    for b in range(B):
        others = np.r_[0:off[b], off[b] + 1:cap]
        assert np.array_equal(gk[b][:, others], kc[b][:, others]) and np.array_equal(gke[b][:, others],
                                                                                     ke[b][:, others])
    # k rows: same quantisation of a bf16 k that may differ from pre_attention's by the last
    # bit (f32 sum order), so compare the decoded rows
    dk_f = ora.bf16_from_f32(ora.fp8_dequantize(gk, gke))
    dk_p = ora.bf16_from_f32(ora.fp8_dequantize(pk, pke))
    assert_close(dk_f, dk_p, "fused vs pair decoded k rows", max_abs=2e-2, mean_abs=1e-5)
    assert_close(host(fused), host(pair), "fp8 fused vs pair", max_abs=1e-2, mean_abs=1e-4)
    # oracle: attend the decoded cache the fused step left behind
    q_ref = host(q)
    L = np.clip(off + 1, 0, cap).astype(np.int32)
    dv = ora.bf16_from_f32(ora.fp8_dequantize(gv, gve))
    assert_close(host(fused), ora.sdpa(q_ref, dk_f, dv, L, scale_of(D), False), "fp8 fused vs oracle")


def test_fp8_fused_step_out_of_capacity(ema, ora):
    """An offset at or past the capacity writes nothing and attends the full (stale) cache."""
    import torch

    B, Hq, Hkv, D, cap = 3, 8, 2, 128, 64
    off = np.array([64, 10, 200], np.int32)
    (kc, ke, kd), (vc, ve, vd) = quantized_pair(ora, (B, Hkv, cap, D), seed=740)
    qkv = ora.normal_bf16((B, (Hq + 2 * Hkv) * D), seed=742)
    cache = fp8_cache(ema, kc, ke, vc, ve)
    out = ema.decode_step(dev(qkv), None, None, 1e-6, 1e6, dev(off), Hq, cache, cap, flags=3)
    torch.cuda.synchronize()
    for b in (0, 2):
        assert np.array_equal(host(cache.k)[b], kc[b]) and np.array_equal(host(cache.k_exp)[b], ke[b])
        assert np.array_equal(host(cache.v)[b], vc[b]) and np.array_equal(host(cache.v_exp)[b], ve[b])
    # flags 3: q is the raw q row; sequence 1 also wrote row 10 (checked by the fused tests)
    q = qkv[:, :Hq * D].reshape(B, Hq, 1, D).copy()
    L = np.clip(off + 1, 0, cap).astype(np.int32)
    dk = ora.bf16_from_f32(ora.fp8_dequantize(host(cache.k), host(cache.k_exp)))
    dv = ora.bf16_from_f32(ora.fp8_dequantize(host(cache.v), host(cache.v_exp)))
    assert_close(host(out), ora.sdpa(q, dk, dv, L, scale_of(D), False), "fp8 fused out of capacity")


@pytest.mark.parametrize("B,G,L,max_len", [(1, 4, [1024], 4096), (2, 16, [777, 1], 2048), (3, 2, [5, 300, 64], 300)])
def test_fp8_decode_shapes(ema, ora, B, G, L, max_len):
    """Batch 1, 16 query heads per kv head, a split sized for more rows than are valid."""
    import torch

    Hkv, D, cap = 2, 128, 4096
    Hq = G * Hkv
    say(f"fp8 decode B={B} G={G} L={L} max_len={max_len}")
    (kc, ke, kd), (vc, ve, vd) = quantized_pair(ora, (B, Hkv, cap, D), seed=750 + G)
    q = ora.normal_bf16((B, Hq, 1, D), seed=753)
    L = np.asarray(L, np.int32)
    out = ema.decode_attention(dev(q), fp8_cache(ema, kc, ke, vc, ve), dev(L), max_len)
    torch.cuda.synchronize()
    assert_close(host(out), ora.sdpa(q, kd, vd, L, scale_of(D), False), "fp8 decode shapes")


@pytest.mark.parametrize("B,cap", [(64, 96), (65, 96), (130, 203)])
def test_fp8_decode_batch_sizes_around_64(ema, ora, B, cap):
    """Both sides of the 64-sequence edge between the per-wave length table and the
    workgroup's, with empty sequences, over whole-8-row exponent groups (96) and row by
    row (203)."""
    import torch

    Hkv, G, D = 2, 4, 128
    Hq = G * Hkv
    rng = np.random.default_rng(780 + B)
    L = rng.integers(1, cap + 1, size=B).astype(np.int32)
    L[::9] = 0
    L[1] = cap
    say(f"fp8 decode B={B} cap={cap} sum(L)={int(L.sum())}")
    (kc, ke, kd), (vc, ve, vd) = quantized_pair(ora, (B, Hkv, cap, D), seed=780 + B)
    q = ora.normal_bf16((B, Hq, 1, D), seed=783)
    out = host(ema.decode_attention(dev(q), fp8_cache(ema, kc, ke, vc, ve), dev(L), cap))
    torch.cuda.synchronize()
    assert_close(out, ora.sdpa(q, kd, vd, L, scale_of(D), False), f"fp8 decode B={B}")
    assert not out[::9].any()


def test_fp8_graph_replay_matches_eager(ema, ora):
    """The fused fp8 step captured in a HIP graph: every replay, with eager work and
    synchronisation in between, equals the eager result (and rewrites the same row)."""
    import torch

    B, Hq, Hkv, D, cap = 4, 16, 8, 128, 1024
    off = np.array([100, 1023, 0, 512], np.int32)
    (kc, ke, _), (vc, ve, _) = quantized_pair(ora, (B, Hkv, cap, D), seed=760)
    qkv = dev(ora.normal_bf16((B, (Hq + 2 * Hkv) * D), seed=762))
    qw = dev(ora.normal_bf16(D, seed=763, mean=1.0, std=0.02))
    kw = dev(ora.normal_bf16(D, seed=764, mean=1.0, std=0.02))
    cache = fp8_cache(ema, kc, ke, vc, ve)
    off_d = dev(off)
    out = torch.empty((B, Hq * D), dtype=torch.bfloat16, device="cuda")
    ws = ema.decode_workspace(B, Hq, Hkv, D, cap)

    def step():
        ema.decode_step(qkv, qw, kw, 1e-6, 1e6, off_d, Hq, cache, cap, out=out, workspace=ws)

    step()
    torch.cuda.synchronize()
    eager, k_eager = host(out).copy(), host(cache.k).copy()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            step()
    torch.cuda.synchronize()
    for i in range(4):
        out.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert np.array_equal(host(out), eager), f"replay {i}"
        assert np.array_equal(host(cache.k), k_eager)
        step()
        torch.cuda.synchronize()


# ------------------------------------------------------------------ prefill
@pytest.mark.parametrize("T,q_off,causal,chunk,G,max_kv", [
    (300, 0, True, False, 4, None),
    (257, 1000, True, True, 8, 1500),
    (128, 700, True, False, 2, None),
    (64, 33, False, False, 1, 97),
])
def test_fp8_prefill_equals_bf16_prefill_of_decoded_cache(ema, ora, T, q_off, causal, chunk, G, max_kv):
    """Prefill over an FP8 cache (ema_prefill_attention_ws) is the bf16 prefill over the
    decoded rows: bit-identical to a bf16 cache holding them, and within the bf16
    tolerance of the f64 oracle."""
    import torch

    B, Hkv, D, cap = 2, 2, 128, 2048
    Hq = G * Hkv
    say(f"fp8 prefill T={T} q_off={q_off} causal={causal} chunk={chunk} G={G} max_kv={max_kv}")
    (kc, ke, kd), (vc, ve, vd) = quantized_pair(ora, (B, Hkv, cap, D), seed=770 + G)
    q = ora.normal_bf16((B, Hq, T, D), seed=773)
    qo = np.array([q_off, q_off // 2], np.int32)
    c8 = fp8_cache(ema, kc, ke, vc, ve)
    c16 = ema.StaticCache(B, Hkv, cap, D, k=dev(kd), v=dev(vd))
    o8 = ema.prefill_attention(dev(q), c8, dev(qo), causal=causal, chunk_only=chunk, max_kv_len=max_kv)
    o16 = ema.prefill_attention(dev(q), c16, dev(qo), causal=causal, chunk_only=chunk)
    torch.cuda.synchronize()
    assert np.array_equal(host(o8), host(o16)), "decoded fp8 rows == the bf16 cache"
    kv_len = np.minimum(qo + T, cap).astype(np.int32)
    kb = qo if chunk else None
    ref = ora.sdpa(q, kd, vd, kv_len, scale_of(D), causal, kv_begin=kb)
    assert_close(host(o8), ref, "fp8 prefill vs oracle")


def test_fp8_prefill_paired(ema, ora):
    """The FP8 prefill at a paired grid (B 4 x 16 query heads x 8 query blocks = 512 blocks,
    two per CU on MI355X): the paired kernel over the decoded rows in the workspace, whose
    row count (max_kv_len) differs from the cache's capacity. Bit-identical to the bf16
    cache of the decoded values, within the bf16 tolerance of the oracle."""
    import torch

    B, Hkv, G, D, cap, T = 4, 4, 4, 128, 2048, 1000
    Hq = G * Hkv
    qo = np.array([0, 300, 48, 1000], np.int32)
    say(f"fp8 paired prefill B={B} Hq={Hq} T={T} q_off={qo.tolist()}")
    (kc, ke, kd), (vc, ve, vd) = quantized_pair(ora, (B, Hkv, cap, D), seed=881)
    q = ora.normal_bf16((B, Hq, T, D), seed=883)
    c8 = fp8_cache(ema, kc, ke, vc, ve)
    c16 = ema.StaticCache(B, Hkv, cap, D, k=dev(kd), v=dev(vd))
    o8 = ema.prefill_attention(dev(q), c8, dev(qo), causal=True, max_kv_len=int((qo + T).max()))
    o16 = ema.prefill_attention(dev(q), c16, dev(qo), causal=True)
    torch.cuda.synchronize()
    assert np.array_equal(host(o8), host(o16)), "decoded fp8 rows == the bf16 cache"
    ref = ora.sdpa(q, kd, vd, (qo + T).astype(np.int32), scale_of(D), True)
    assert_close(host(o8), ref, "fp8 paired prefill vs oracle")


# ------------------------------------------------------------------ row conversion
def test_fp8_convert_quantises_and_decodes_rows(ema, ora):
    """ema_kvcache_convert bf16 -> FP8 writes the oracle's codes and exponents for the
    copied rows only (Fp8Cache::append, crates/kvcache/src/fp8.rs:47-68); FP8 -> bf16
    gives the exact decoded values (what Fp8Cache::get hands SDPA)."""
    import torch

    B, Hkv, D = 2, 3, 128
    say("fp8 convert: bf16 rows [5, 38) -> fp8 rows [20, 53), then back")
    x = ora.normal_f32((B, Hkv, 40, D), seed=901, std=4.0)
    x[0, 1, 7, :64] *= 1e-3  # one small block
    xb = ora.bf16_from_f32(x)
    src = ema.StaticCache(B, Hkv, 40, D, k=dev(xb), v=dev(xb[:, ::-1].copy()))
    dst = ema.StaticCache(B, Hkv, 64, D, dtype="fp8")
    ema.kvcache_convert(src, dst, 33, src_row=5, dst_row=20)
    torch.cuda.synchronize()
    for name, rows, codes, exps in (("k", xb, dst.k, dst.k_exp), ("v", xb[:, ::-1], dst.v, dst.v_exp)):
        rc, re = ora.fp8_quantize(ora.f32_from_bf16(np.ascontiguousarray(rows[:, :, 5:38])))
        gc, ge = host(codes), host(exps)
        assert np.array_equal(canon(gc[:, :, 20:53]), canon(rc)), f"{name} codes"
        assert np.array_equal(ge[:, :, 20:53], re), f"{name} exponents"
        assert not gc[:, :, :20].any() and not gc[:, :, 53:].any() and not ge[:, :, 53:].any()
    # FP8 -> bf16 of random codes (every finite code, exponents -8 / -7) into rows [3, 51)
    (kc, ke, kd), (vc, ve, vd) = random_fp8_pair(ora, (B, Hkv, 64, D), seed=907)
    c8 = fp8_cache(ema, kc, ke, vc, ve)
    out = ema.StaticCache(B, Hkv, 56, D)
    ema.kvcache_convert(c8, out, 48, src_row=10, dst_row=3)
    torch.cuda.synchronize()
    for name, got, want in (("k", out.k, kd), ("v", out.v, vd)):
        g = ora.f32_from_bf16(host(got))
        assert np.array_equal(g[:, :, 3:51], ora.f32_from_bf16(want[:, :, 10:58])), f"{name} decoded"
        assert not g[:, :, :3].any() and not g[:, :, 51:].any()


def test_position_write_is_stream_ordered(ema):
    import torch

    say("position_write")
    t = torch.full((4,), -1, dtype=torch.int32, device="cuda")
    s = torch.cuda.current_stream()
    for v in (7, 11, 123456):
        ema.position_write(t[2:], v, stream=s)
        t[0] = t[2]  # a later op on the same stream reads the written value
    torch.cuda.synchronize()
    assert t.cpu().tolist() == [123456, -1, 123456, -1]


@pytest.mark.parametrize("rotating,n_rot,first,T,chunk", [
    (False, 0, 0, 300, False),    # a fresh prefill: the chunk's rows are all it attends
    (False, 0, 0, 300, True),     # ... with chunk-only keys: no decode pass runs
    (False, 0, 200, 300, False),  # a second chunk: rows [0, 200) decoded by the pass
    (False, 0, 200, 300, True),
    (False, 64, 200, 300, False),  # the RoPE tail kept as bf16
    (True, 0, 200, 300, False),   # a ring of 384 rows that the second chunk wraps
    (True, 0, 200, 300, True),
])
def test_fp8_prefill_with_rows_from_pre_attention(ema, ora, rotating, n_rot, first, T, chunk):
    """ema_pre_attention_ws writes the chunk's rows, decoded, into the prefill workspace, and
    ema_prefill_attention_ws with EMA_PREFILL_ROWS_DECODED then decodes only the other
    rows: q, the cache and the output are bit-identical to ema_pre_attention followed by
    the plain FP8 prefill. The workspace starts as NaN, so a row neither writes would show."""
    import torch

    B, Hq, Hkv, D = 2, 8, 2, 128
    cap = 384 if rotating else 1024
    say(f"fp8 prefill rows from pre-attention rot={rotating} n_rot={n_rot} first={first} T={T} chunk={chunk}")
    qw = ora.normal_bf16(D, seed=901, mean=1.0, std=0.02)
    kw = ora.normal_bf16(D, seed=902, mean=1.0, std=0.02)
    F = (Hq + 2 * Hkv) * D
    c_a = ema.StaticCache(B, Hkv, cap, D, dtype="fp8", rotating=rotating, n_rot=n_rot)
    c_b = ema.StaticCache(B, Hkv, cap, D, dtype="fp8", rotating=rotating, n_rot=n_rot)
    if first:  # earlier tokens, written the same way into both caches
        qkv0 = dev(ora.normal_bf16((B, first, F), seed=903))
        off0 = dev(np.zeros(B, np.int32))
        for c in (c_a, c_b):
            ema.pre_attention(qkv0, dev(qw), dev(kw), 1e-6, 1e6, off0, Hq, c)
    qkv = dev(ora.normal_bf16((B, T, F), seed=904))
    off = dev(np.full(B, first, np.int32))
    mk = cap if rotating else first + T
    n = ema.prefill_workspace_size(c_a, mk)
    ws_a = torch.empty(n, dtype=torch.uint8, device="cuda")
    ws_b = torch.full((n // 2,), 0x7FC0, dtype=torch.int16, device="cuda").view(torch.uint8)  # bf16 NaN
    q_a = ema.pre_attention(qkv, dev(qw), dev(kw), 1e-6, 1e6, off, Hq, c_a)
    o_a = ema.prefill_attention(q_a, c_a, off, chunk_only=chunk, max_kv_len=mk, workspace=ws_a)
    q_b = ema.pre_attention(qkv, dev(qw), dev(kw), 1e-6, 1e6, off, Hq, c_b, prefill_workspace=ws_b, max_kv_len=mk)
    o_b = ema.prefill_attention(q_b, c_b, off, chunk_only=chunk, max_kv_len=mk, workspace=ws_b, rows_decoded=True)
    torch.cuda.synchronize()
    assert np.array_equal(host(q_a), host(q_b))
    for t_a, t_b in ((c_a.k, c_b.k), (c_a.v, c_b.v), (c_a.k_exp, c_b.k_exp), (c_a.v_exp, c_b.v_exp)):
        assert torch.equal(t_a, t_b)
    got = host(o_b)
    assert np.all(np.isfinite(ora.f32_from_bf16(got))), "a row of the copy was never written"
    assert np.array_equal(host(o_a), got), "rows from pre-attention == rows from the decode pass"
