"""GPU parity of the FP8 cache with an unquantised RoPE tail: the reference's
Fp8Cache::new(128, 64) (crates/kvcache/src/fp8.rs:38-54), whose round trip
(crates/ops/src/fp8.rs:69-92) quantises dims 0..63 of each K/V row in one 64-value block
and leaves dims 64..127 as they are. Stored here as 64 codes + 64 bf16 values per row
(n_rot = 64 in the descriptor), through the C ABI.

Bars:
  - written rows: block 0's codes and exponent bit-exact against the oracle's
    quantisation, the tail bit-exact against the written bf16 values, and the decoded
    row equal to the oracle's fp8_round_trip(row, 128, 64);
  - decode and prefill over the cache equal decode and prefill over a bf16 cache that
    holds the decoded values (decode: f32 summation order only, max-abs 2e-3; prefill
    bit-identical), and are within the bf16 tolerance of the f64 oracle;
  - the fused step writes the same rows as the separate pre-attention kernel.
"""
import numpy as np
import pytest

from gpu_util import assert_close, dev, host, say, scale_of

pytestmark = pytest.mark.gpu

D, NROT = 128, 64


@pytest.fixture(scope="module")
def ema():
    import torch

    if not torch.cuda.is_available():
        pytest.fail("GPU tests need a ROCm GPU")
    import ema_attn

    ema_attn.lib()
    return ema_attn


def canon(codes):
    """-0 (0x80) and +0 (0x00) are the same value."""
    c = np.asarray(codes).copy()
    c[c == 0x80] = 0
    return c


def tail_form(ora, x_bf16):
    """bf16 rows [..., 128] -> the stored form with n_rot = 64: rows uint8 [..., 192]
    (64 codes, then the 64 tail values' bf16 bytes), exponents int8 [..., 2] (block 1's 0)
    and the decoded bf16 rows."""
    x_bf16 = np.ascontiguousarray(x_bf16)
    head = ora.f32_from_bf16(np.ascontiguousarray(x_bf16[..., :NROT]))
    codes, exps = ora.fp8_quantize(head)
    tail = np.ascontiguousarray(x_bf16[..., NROT:])
    rows = np.concatenate([codes, tail.view(np.uint8)], axis=-1)
    e2 = np.zeros(x_bf16.shape[:-1] + (2,), np.int8)
    e2[..., 0] = exps[..., 0]
    dec = np.concatenate([ora.bf16_from_f32(ora.fp8_dequantize(codes, exps)), tail], axis=-1)
    return rows, e2, dec


def decoded(ora, rows, exps):
    """Decoded bf16 rows [..., 128] of stored rows [..., 192] (the reader's view)."""
    rows = np.ascontiguousarray(rows)
    head = ora.bf16_from_f32(ora.fp8_dequantize(np.ascontiguousarray(rows[..., :NROT]),
                                                np.ascontiguousarray(exps[..., :1])))
    tail = np.ascontiguousarray(rows[..., NROT:]).view(np.uint16)
    return np.concatenate([head, tail], axis=-1)


def tail_pair(ora, shape, seed):
    """Random K/V caches [B, Hkv, cap, 128] in the tail form: (rows, exps, decoded) each."""
    out = []
    for i in range(2):
        x = ora.bf16_from_f32(ora.normal_f32(shape, seed=seed + i))
        out.append(tail_form(ora, x))
    return out


def tail_cache(ema, kr, ke, vr, ve):
    B, Hkv, cap, _ = kr.shape
    return ema.StaticCache(B, Hkv, cap, D, dtype="fp8", n_rot=NROT, k=dev(kr), v=dev(vr), k_exp=dev(ke),
                           v_exp=dev(ve))


def test_tail_form_is_the_reference_round_trip(ora):
    """The stored form decodes to fp8_round_trip(row, 128, 64) (fp8.rs:69-92) exactly, and
    differs from the whole-head round trip only in the tail (the reference's n_rot)."""
    x = ora.bf16_from_f32(ora.normal_f32((5, 3, 40, D), seed=11, std=3.0))
    _, _, dec = tail_form(ora, x)
    ref = ora.bf16_from_f32(ora.fp8_round_trip(ora.f32_from_bf16(x), D, NROT))
    assert np.array_equal(ora.f32_from_bf16(dec), ora.f32_from_bf16(ref))
    assert np.array_equal(dec[..., NROT:], x[..., NROT:])
    whole = ora.bf16_from_f32(ora.fp8_round_trip(ora.f32_from_bf16(x), D, 0))
    assert np.array_equal(ora.f32_from_bf16(whole[..., :NROT]), ora.f32_from_bf16(dec[..., :NROT]))
    assert not np.array_equal(whole[..., NROT:], dec[..., NROT:])


# ------------------------------------------------------------------ writes
def test_tail_write_every_bf16_value(ema, ora):
    """pre_attention without norm/RoPE: every finite bf16 pattern as k and v."""
    import torch

    B, T, Hq, Hkv, cap = 1, 64, 8, 8, 80
    say("fp8 n_rot=64 write: every bf16 pattern")
    pats = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    f = (pats.astype(np.uint32) << 16).view(np.float32)
    pats[~np.isfinite(f)] = 0
    k = pats.reshape(T, Hkv, D)
    v = pats[::-1].copy().reshape(T, Hkv, D)
    qkv = np.zeros((B, T, (Hq + 2 * Hkv) * D), np.uint16)
    qkv[0, :, Hq * D:(Hq + Hkv) * D] = k.reshape(T, -1)
    qkv[0, :, (Hq + Hkv) * D:] = v.reshape(T, -1)
    off = np.array([9], np.int32)
    cache = ema.StaticCache(B, Hkv, cap, D, dtype="fp8", n_rot=NROT)
    ema.pre_attention(dev(qkv), None, None, 1e-6, 1e6, dev(off), Hq, cache, flags=3)
    torch.cuda.synchronize()
    for name, src, rows, exps in (("k", k, cache.k, cache.k_exp), ("v", v, cache.v, cache.v_exp)):
        want_rows, want_exps, _ = tail_form(ora, np.ascontiguousarray(src.transpose(1, 0, 2)))  # [Hkv, T, ...]
        gr, ge = host(rows)[0], host(exps)[0]
        assert np.array_equal(canon(gr[:, 9:9 + T, :NROT]), canon(want_rows[..., :NROT])), f"{name} codes"
        assert np.array_equal(gr[:, 9:9 + T, NROT:], want_rows[..., NROT:]), f"{name} tail"
        assert np.array_equal(ge[:, 9:9 + T], want_exps), f"{name} exponents"
        assert not gr[:, :9].any() and not gr[:, 9 + T:].any() and not ge[:, :9].any()


@pytest.mark.parametrize("flags", [0, 2])
def test_tail_write_after_norm_rope(ema, ora, flags):
    """With norm and RoPE: the rows are the tail form of the bf16 k / v the same kernel
    writes into a bf16 cache."""
    import torch

    B, T, Hq, Hkv, cap = 2, 7, 16, 8, 64
    say(f"fp8 n_rot=64 write after norm/rope flags={flags}")
    qkv = ora.normal_bf16((B, T, (Hq + 2 * Hkv) * D), seed=800 + flags)
    qw = ora.normal_bf16(D, seed=801, mean=1.0, std=0.02)
    kw = ora.normal_bf16(D, seed=802, mean=1.0, std=0.02)
    off = np.array([0, 40], np.int32)
    c16 = ema.StaticCache(B, Hkv, cap, D)
    c8 = ema.StaticCache(B, Hkv, cap, D, dtype="fp8", n_rot=NROT)
    q16 = ema.pre_attention(dev(qkv), dev(qw), dev(kw), 1e-6, 1e6, dev(off), Hq, c16, flags=flags)
    q8 = ema.pre_attention(dev(qkv), dev(qw), dev(kw), 1e-6, 1e6, dev(off), Hq, c8, flags=flags)
    torch.cuda.synchronize()
    assert np.array_equal(host(q16), host(q8))
    for src, rows, exps in ((c16.k, c8.k, c8.k_exp), (c16.v, c8.v, c8.v_exp)):
        wr, we, _ = tail_form(ora, host(src))
        gr, ge = host(rows), host(exps)
        for b in range(B):
            sl = slice(off[b], off[b] + T)
            assert np.array_equal(canon(gr[b][:, sl, :NROT]), canon(wr[b][:, sl, :NROT]))
            assert np.array_equal(gr[b][:, sl, NROT:], wr[b][:, sl, NROT:])
            assert np.array_equal(ge[b][:, sl], we[b][:, sl])


# ------------------------------------------------------------------ decode
@pytest.mark.parametrize("G,lengths,cap", [
    (4, [1, 31, 32, 33, 100, 1000, 1024], 1024),
    (1, [64, 65, 3], 96),
    (16, [777, 1], 2048),
])
def test_tail_decode_equals_bf16_decode_of_decoded_cache(ema, ora, G, lengths, cap):
    import torch

    Hkv = 2
    B, Hq = len(lengths), Hkv * G
    say(f"fp8 n_rot=64 decode G={G} lengths={lengths}")
    (kr, ke, kd), (vr, ve, vd) = tail_pair(ora, (B, Hkv, cap, D), seed=810 + G)
    q = ora.normal_bf16((B, Hq, 1, D), seed=815)
    L = np.asarray(lengths, np.int32)
    c8 = tail_cache(ema, kr, ke, vr, ve)
    c16 = ema.StaticCache(B, Hkv, cap, D, k=dev(kd), v=dev(vd))
    o8 = ema.decode_attention(dev(q), c8, dev(L), int(L.max()))
    o16 = ema.decode_attention(dev(q), c16, dev(L), int(L.max()))
    torch.cuda.synchronize()
    assert_close(host(o8), host(o16), "fp8 n_rot=64 vs bf16 decode of the decoded cache", max_abs=2e-3,
                 mean_abs=1e-5)
    assert_close(host(o8), ora.sdpa(q, kd, vd, L, scale_of(D), False), "fp8 n_rot=64 decode vs oracle")


def test_tail_decode_qwen3_8b_batched_shape(ema, ora):
    """Fp8Cache::new(128, 64) at the batch-32 decode shape: 32q/8kv, cap 8192, lengths
    U[512, 8192]; the cache holds the round trip of random rows."""
    import torch

    B, Hq, Hkv, cap = 32, 32, 8, 8192
    L = np.random.default_rng(1234).integers(512, 8193, size=B).astype(np.int32)
    say("fp8 n_rot=64 decode B32 32q/8kv cap 8192")
    (kr, ke, kd), (vr, ve, vd) = tail_pair(ora, (B, Hkv, cap, D), seed=820)
    q = ora.normal_bf16((B, Hq, 1, D), seed=822)
    c8 = tail_cache(ema, kr, ke, vr, ve)
    del kr, vr
    o8 = ema.decode_attention(dev(q), c8, dev(L), cap)
    torch.cuda.synchronize()
    assert_close(host(o8), ora.sdpa(q, kd, vd, L, scale_of(D), False), "fp8 n_rot=64 decode 8B batched")


@pytest.mark.parametrize("flags", [0, 3])
def test_tail_fused_step(ema, ora, flags):
    """decode_step over the tail cache writes the rows pre_attention writes (the k row up
    to the last bit of its f32 norm sum) and attends them in decoded form."""
    import torch

    B, Hq, Hkv, cap = 6, 16, 4, 200
    off = np.array([0, 31, 32, 100, 199, 63], np.int32)
    say(f"fp8 n_rot=64 fused step flags={flags}")
    (kr, ke, kd), (vr, ve, vd) = tail_pair(ora, (B, Hkv, cap, D), seed=830)
    qkv = ora.normal_bf16((B, (Hq + 2 * Hkv) * D), seed=833)
    qw = ora.normal_bf16(D, seed=834, mean=1.0, std=0.02)
    kw = ora.normal_bf16(D, seed=835, mean=1.0, std=0.02)
    c_pair = tail_cache(ema, kr, ke, vr, ve)
    q = ema.pre_attention(dev(qkv.reshape(B, 1, -1)), dev(qw), dev(kw), 1e-6, 1e6, dev(off), Hq, c_pair,
                          flags=flags)
    pair = ema.decode_attention(q, c_pair, dev(off + 1), cap)
    c_f = tail_cache(ema, kr, ke, vr, ve)
    fused = ema.decode_step(dev(qkv), dev(qw), dev(kw), 1e-6, 1e6, dev(off), Hq, c_f, cap, flags=flags)
    torch.cuda.synchronize()
    gk, gke, gv, gve = host(c_f.k), host(c_f.k_exp), host(c_f.v), host(c_f.v_exp)
    assert np.array_equal(canon(gv), canon(host(c_pair.v))) and np.array_equal(gve, host(c_pair.v_exp))
    for b in range(B):
        others = np.r_[0:off[b], off[b] + 1:cap]
        assert np.array_equal(gk[b][:, others], kr[b][:, others])
        assert np.array_equal(gke[b][:, others], ke[b][:, others])
        assert not gke[b][:, off[b], 1].any() and not gve[b][:, off[b], 1].any()
    dk_f = decoded(ora, gk, gke)
    dk_p = decoded(ora, host(c_pair.k), host(c_pair.k_exp))
    assert_close(dk_f, dk_p, "fused vs pair decoded k rows", max_abs=2e-2, mean_abs=1e-5)
    assert_close(host(fused), host(pair), "fp8 n_rot=64 fused vs pair", max_abs=1e-2, mean_abs=1e-4)
    L = np.clip(off + 1, 0, cap).astype(np.int32)
    dv = decoded(ora, gv, gve)
    assert_close(host(fused), ora.sdpa(host(q), dk_f, dv, L, scale_of(D), False), "fp8 n_rot=64 fused vs oracle")


def test_tail_rotating_fused_step(ema, ora):
    """A ring (EMA_KV_ROTATING) in the tail form: the fused step writes row off % cap."""
    import torch

    B, Hq, Hkv, cap = 3, 8, 2, 96
    off = np.array([95, 96, 500], np.int32)
    say("fp8 n_rot=64 rotating fused step")
    (kr, ke, kd), (vr, ve, vd) = tail_pair(ora, (B, Hkv, cap, D), seed=840)
    qkv = ora.normal_bf16((B, (Hq + 2 * Hkv) * D), seed=842)
    c_pair = tail_cache(ema, kr, ke, vr, ve)
    c_pair.desc.flags = ema.EMA_KV_ROTATING
    q = ema.pre_attention(dev(qkv.reshape(B, 1, -1)), None, None, 1e-6, 1e6, dev(off), Hq, c_pair, flags=3)
    c_f = tail_cache(ema, kr, ke, vr, ve)
    c_f.desc.flags = ema.EMA_KV_ROTATING
    out = ema.decode_step(dev(qkv), None, None, 1e-6, 1e6, dev(off), Hq, c_f, cap, flags=3)
    torch.cuda.synchronize()
    assert np.array_equal(canon(host(c_f.k)), canon(host(c_pair.k)))
    assert np.array_equal(canon(host(c_f.v)), canon(host(c_pair.v)))
    assert np.array_equal(host(c_f.k_exp), host(c_pair.k_exp))
    L = np.minimum(off + 1, cap).astype(np.int32)
    dk, dv = decoded(ora, host(c_f.k), host(c_f.k_exp)), decoded(ora, host(c_f.v), host(c_f.v_exp))
    assert_close(host(out), ora.sdpa(host(q), dk, dv, L, scale_of(D), False), "fp8 n_rot=64 ring step vs oracle")


# ------------------------------------------------------------------ prefill
@pytest.mark.parametrize("T,q_off,chunk,G,max_kv", [
    (300, 0, False, 4, None),
    (257, 1000, True, 8, 1500),
    (64, 33, False, 1, 97),
])
def test_tail_prefill_equals_bf16_prefill_of_decoded_cache(ema, ora, T, q_off, chunk, G, max_kv):
    import torch

    B, Hkv, cap = 2, 2, 2048
    Hq = G * Hkv
    say(f"fp8 n_rot=64 prefill T={T} q_off={q_off} chunk={chunk} G={G}")
    (kr, ke, kd), (vr, ve, vd) = tail_pair(ora, (B, Hkv, cap, D), seed=850 + G)
    q = ora.normal_bf16((B, Hq, T, D), seed=853)
    qo = np.array([q_off, q_off // 2], np.int32)
    c8 = tail_cache(ema, kr, ke, vr, ve)
    c16 = ema.StaticCache(B, Hkv, cap, D, k=dev(kd), v=dev(vd))
    o8 = ema.prefill_attention(dev(q), c8, dev(qo), causal=True, chunk_only=chunk, max_kv_len=max_kv)
    o16 = ema.prefill_attention(dev(q), c16, dev(qo), causal=True, chunk_only=chunk)
    torch.cuda.synchronize()
    assert np.array_equal(host(o8), host(o16)), "decoded rows == the bf16 cache"
    kv_len = np.minimum(qo + T, cap).astype(np.int32)
    ref = ora.sdpa(q, kd, vd, kv_len, scale_of(D), True, kv_begin=qo if chunk else None)
    assert_close(host(o8), ref, "fp8 n_rot=64 prefill vs oracle")


# ------------------------------------------------------------------ conversion
def test_tail_convert_both_ways(ema, ora):
    """ema_kvcache_convert into and out of the tail form (Fp8Cache::append / get)."""
    import torch

    B, Hkv = 2, 3
    say("fp8 n_rot=64 convert")
    x = ora.bf16_from_f32(ora.normal_f32((B, Hkv, 40, D), seed=861, std=4.0))
    src = ema.StaticCache(B, Hkv, 40, D, k=dev(x), v=dev(x[:, ::-1].copy()))
    dst = ema.StaticCache(B, Hkv, 64, D, dtype="fp8", n_rot=NROT)
    ema.kvcache_convert(src, dst, 33, src_row=5, dst_row=20)
    back = ema.StaticCache(B, Hkv, 64, D)
    ema.kvcache_convert(dst, back, 64)
    torch.cuda.synchronize()
    for name, rows, got, exps in (("k", x, dst.k, dst.k_exp), ("v", x[:, ::-1], dst.v, dst.v_exp)):
        wr, we, wd = tail_form(ora, np.ascontiguousarray(rows[:, :, 5:38]))
        gr, ge = host(got), host(exps)
        assert np.array_equal(canon(gr[:, :, 20:53, :NROT]), canon(wr[..., :NROT])), f"{name} codes"
        assert np.array_equal(gr[:, :, 20:53, NROT:], wr[..., NROT:]), f"{name} tail"
        assert np.array_equal(ge[:, :, 20:53], we), f"{name} exponents"
        gb = host(back.k if name == "k" else back.v)
        assert np.array_equal(ora.f32_from_bf16(gb[:, :, 20:53]), ora.f32_from_bf16(wd)), f"{name} decoded"
        assert not gb[:, :, :20].any() and not gb[:, :, 53:].any()


def test_tail_graph_loop_advances(ema, ora):
    """Four fused steps with EMA_STEP_ADVANCE over the tail cache captured in one HIP graph
    (each step is two kernels here): every replay, restarted from the same cache and
    offsets, equals the same four steps run eagerly, and the offsets advance by four
    (one sequence stops at the capacity)."""
    import torch

    B, Hq, Hkv, cap, n = 4, 16, 4, 256, 4
    off0 = np.array([0, 100, cap - 2, 37], np.int32)
    say("fp8 n_rot=64 graph loop with EMA_STEP_ADVANCE")
    (kr, ke, _), (vr, ve, _) = tail_pair(ora, (B, Hkv, cap, D), seed=870)
    qkvs = dev(np.stack([ora.normal_bf16((B, (Hq + 2 * Hkv) * D), seed=871 + i) for i in range(n)]))
    qw = dev(ora.normal_bf16(D, seed=876, mean=1.0, std=0.02))
    kw = dev(ora.normal_bf16(D, seed=877, mean=1.0, std=0.02))
    cache = tail_cache(ema, kr, ke, vr, ve)
    off_d = dev(off0)
    outs = torch.zeros((n, B, Hq * D), dtype=torch.bfloat16, device="cuda")
    ws = ema.decode_workspace(B, Hq, Hkv, D, cap)

    def restart():
        for t, h in ((cache.k, kr), (cache.v, vr), (cache.k_exp, ke), (cache.v_exp, ve), (off_d, off0)):
            t.copy_(torch.from_numpy(h).to("cuda"))
        outs.zero_()
        torch.cuda.synchronize()

    def steps():
        for i in range(n):
            ema.decode_step(qkvs[i], qw, kw, 1e-6, 1e6, off_d, Hq, cache, cap, out=outs[i], workspace=ws,
                            flags=ema.EMA_STEP_ADVANCE)

    restart()
    steps()
    torch.cuda.synchronize()
    eager, k_eager, off_eager = host(outs).copy(), host(cache.k).copy(), host(off_d).copy()
    assert off_eager.tolist() == [4, 104, cap, 41]
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    restart()
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            steps()
    torch.cuda.synchronize()
    for i in range(3):
        restart()
        g.replay()
        torch.cuda.synchronize()
        assert np.array_equal(host(outs), eager), f"replay {i}"
        assert np.array_equal(host(cache.k), k_eager) and np.array_equal(host(off_d), off_eager)


def test_tail_noalloc_step_equals_workspace_step(ema, ora):
    """ema_decode_step_noalloc over the tail cache equals ema_decode_step (both run the
    pre-attention kernel, then the tail decode kernel)."""
    import torch

    B, Hq, Hkv, cap = 3, 8, 2, 512
    off = np.array([5, 300, 511], np.int32)
    (kr, ke, _), (vr, ve, _) = tail_pair(ora, (B, Hkv, cap, D), seed=880)
    qkv = dev(ora.normal_bf16((B, (Hq + 2 * Hkv) * D), seed=882))
    ca, cb = tail_cache(ema, kr, ke, vr, ve), tail_cache(ema, kr, ke, vr, ve)
    out_a = ema.decode_step(qkv, None, None, 1e-6, 1e6, dev(off), Hq, ca, cap, flags=3)
    out_b = torch.empty_like(out_a)
    ema.decode_step_noalloc(qkv, None, None, 1e-6, 1e6, dev(off), Hq, cb, cap, out_b, flags=3)
    torch.cuda.synchronize()
    assert np.array_equal(host(out_a), host(out_b))
    assert np.array_equal(host(ca.k), host(cb.k)) and np.array_equal(host(ca.v), host(cb.v))
