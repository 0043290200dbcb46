"""GPU parity of the rotating (sliding-window) cache, EMA_KV_ROTATING: the reference's
RotatingCache (crates/kvcache/src/rotating.rs:56-122) as a ring in which position p lives
in row p % capacity.

Each case builds the whole sequence in a chronological cache `big` and the ring from the
positions the reference's cache would hold (oracle.ring_rows, pinned against a
restatement of RotatingCache::append in tests/test_oracle_rotating.py); ring rows holding
no position are NaN, so any read of them shows. Expected outputs are the oracle's SDPA
over `big` restricted to that window (kv_begin = max(0, L - capacity)); written rows are
compared with the oracle's pre-attention into `big`. Tolerance as in the other parity
tests: max-abs 2e-2, mean-abs 2e-3; V rows bit-exact.
"""
import numpy as np
import pytest

from gpu_util import assert_close, dev, f32, host, say, scale_of

pytestmark = pytest.mark.gpu

NAN = 0x7FC0


@pytest.fixture(scope="module")
def ema():
    import torch

    if not torch.cuda.is_available():
        pytest.fail("GPU tests need a ROCm GPU")
    import ema_attn

    ema_attn.lib()
    return ema_attn


def ring_from(ora, big, totals, window):
    """Ring [B, Hkv, window, D] holding, per sequence b, the window of totals[b] positions."""
    B, Hkv, _, D = big.shape
    ring = np.full((B, Hkv, window, D), NAN, np.uint16)
    for b in range(B):
        for r, p in ora.ring_rows(int(totals[b]), window).items():
            ring[b, :, r] = big[b, :, p]
    return ring


def ring_cache(ema, kr, vr):
    B, Hkv, W, D = kr.shape
    return ema.StaticCache(B, Hkv, W, D, k=dev(kr), v=dev(vr), rotating=True)


@pytest.mark.parametrize("W", [64, 100, 256])
def test_rotating_decode_attends_the_window(ema, ora, W):
    import torch

    B, Hq, Hkv, D = 4, 8, 2, 128
    N = np.array([W - 5, W, W + 1, 3 * W + 7], np.int32)  # tokens seen per sequence
    say(f"rotating decode W={W} N={N.tolist()}")
    big_k = ora.normal_bf16((B, Hkv, int(N.max()), D), seed=W)
    big_v = ora.normal_bf16((B, Hkv, int(N.max()), D), seed=W + 1)
    q = ora.normal_bf16((B, Hq, 1, D), seed=W + 2)
    cache = ring_cache(ema, ring_from(ora, big_k, N, W), ring_from(ora, big_v, N, W))
    out = ema.decode_attention(dev(q), cache, dev(N), W)
    torch.cuda.synchronize()
    ref = ora.sdpa(q, big_k, big_v, N, scale_of(D), False, kv_begin=np.maximum(N - W, 0))
    assert_close(host(out), ref, f"decode W={W}")


@pytest.mark.parametrize("off,T", [(30, 25), (10, 50), (0, 40), (77, 1)])
def test_rotating_pre_attention_writes_ring_rows(ema, ora, off, T):
    import torch

    B, Hq, Hkv, D, W = 1, 4, 2, 128, 40
    say(f"rotating pre-attention W={W} off={off} T={T}")
    qkv = ora.normal_bf16((B, T, (Hq + 2 * Hkv) * D), seed=off + T)
    qw = ora.normal_bf16(D, seed=5, mean=1.0, std=0.02)
    kw = ora.normal_bf16(D, seed=6, mean=1.0, std=0.02)
    big_k = np.zeros((B, Hkv, off + T, D), np.uint16)
    big_v = np.zeros((B, Hkv, off + T, D), np.uint16)
    q_ref = ora.pre_attention(qkv, qw, kw, 1e-6, 1e6, np.array([off], np.int32), Hq, Hkv, big_k, big_v)
    ring_k = np.full((B, Hkv, W, D), NAN, np.uint16)
    ring_v = ring_k.copy()
    cache = ring_cache(ema, ring_k, ring_v)
    q = ema.pre_attention(dev(qkv), dev(qw), dev(kw), 1e-6, 1e6, dev(np.array([off], np.int32)), Hq, cache)
    torch.cuda.synchronize()
    assert_close(host(q), q_ref, "q")
    got_k, got_v = host(cache.k), host(cache.v)
    written = {p % W: p for p in range(max(off, off + T - W), off + T)}  # the call's last W tokens
    for r in range(W):
        if r in written:
            p = written[r]
            assert np.array_equal(got_v[:, :, r], big_v[:, :, p]), (r, p)
            assert_close(got_k[:, :, r], big_k[:, :, p], f"k row {r} <- position {p}")
        else:
            assert np.all(got_k[:, :, r] == NAN) and np.all(got_v[:, :, r] == NAN), f"row {r} touched"


@pytest.mark.parametrize("W", [100, 128])
def test_rotating_fused_decode_step(ema, ora, W):
    import torch

    B, Hq, Hkv, D = 3, 8, 2, 128
    off = np.array([W - 1, W, 2 * W + 3], np.int32)  # position of the new token
    say(f"rotating fused step W={W} off={off.tolist()}")
    qkv = ora.normal_bf16((B, (Hq + 2 * Hkv) * D), seed=W)
    qw = ora.normal_bf16(D, seed=1, mean=1.0, std=0.02)
    kw = ora.normal_bf16(D, seed=2, mean=1.0, std=0.02)
    n = int(off.max()) + 1
    big_k = ora.normal_bf16((B, Hkv, n, D), seed=W + 3)
    big_v = ora.normal_bf16((B, Hkv, n, D), seed=W + 4)
    ring_k = ring_from(ora, big_k, off, W)  # the window before the new token
    ring_v = ring_from(ora, big_v, off, W)
    q_ref = np.zeros((B, Hq, 1, D), np.uint16)
    for b in range(B):
        kb, vb = big_k[b:b + 1].copy(), big_v[b:b + 1].copy()
        q_ref[b:b + 1] = ora.pre_attention(qkv[b:b + 1, None].copy(), qw, kw, 1e-6, 1e6, off[b:b + 1], Hq, Hkv, kb, vb)
        big_k[b], big_v[b] = kb[0], vb[0]
    L = off + 1
    ref = ora.sdpa(q_ref, big_k, big_v, L, scale_of(D), False, kv_begin=np.maximum(L - W, 0))
    cache = ring_cache(ema, ring_k, ring_v)
    out = ema.decode_step(dev(qkv), dev(qw), dev(kw), 1e-6, 1e6, dev(off), Hq, cache, W)
    torch.cuda.synchronize()
    assert_close(host(out), ref, f"fused step W={W}")
    got_k, got_v = host(cache.k), host(cache.v)
    for b in range(B):
        r = int(off[b]) % W
        assert np.array_equal(got_v[b, :, r], big_v[b, :, off[b]])
        assert_close(got_k[b, :, r], big_k[b, :, off[b]], f"new k row b={b}")


@pytest.mark.parametrize("q_off,T,W,chunk", [
    ((0, 37), 100, 256, False),    # no wrap
    ((200, 150), 100, 256, False),  # ends past the ring: key base 44 / 0
    ((500, 433), 128, 192, False),  # several wraps, ring not a multiple of the key block
    ((500, 433), 128, 200, True),   # chunk-only keys within the window
    ((1000, 3), 64, 64, False),     # chunk as long as the ring
])
def test_rotating_prefill_window(ema, ora, q_off, T, W, chunk):
    import torch

    B, Hq, Hkv, D = 2, 8, 2, 128
    qo = np.asarray(q_off, np.int32)
    L = qo + T
    say(f"rotating prefill W={W} q_off={qo.tolist()} T={T} chunk_only={chunk}")
    big_k = ora.normal_bf16((B, Hkv, int(L.max()), D), seed=W + T)
    big_v = ora.normal_bf16((B, Hkv, int(L.max()), D), seed=W + T + 1)
    q = ora.normal_bf16((B, Hq, T, D), seed=W + T + 2)
    cache = ring_cache(ema, ring_from(ora, big_k, L, W), ring_from(ora, big_v, L, W))
    out = ema.prefill_attention(dev(q), cache, dev(qo), causal=True, chunk_only=chunk)
    torch.cuda.synchronize()
    lo = np.maximum(L - W, 0)
    if chunk:
        lo = np.maximum(lo, qo)
    ref = ora.sdpa(q, big_k, big_v, L, scale_of(D), True, kv_begin=lo)
    assert_close(host(out), ref, f"prefill W={W}")


@pytest.mark.parametrize("q_off,chunk", [
    ((0, 300, 1500, 2100), False),  # one sequence without a wrap, three wrapping
    ((100, 1200, 40, 2500), True),  # chunk-only keys
])
def test_rotating_prefill_paired(ema, ora, q_off, chunk):
    """A rotating-cache prefill large enough for the paired grid (B 4 x 16 query heads x 8
    query blocks = 512 blocks, two per CU on MI355X): each workgroup streams a light and a
    heavy query block over ring rows."""
    import torch

    B, Hq, Hkv, D, T, W = 4, 16, 4, 128, 1000, 1024
    qo = np.asarray(q_off, np.int32)
    L = qo + T
    say(f"rotating paired prefill W={W} q_off={qo.tolist()} T={T} chunk_only={chunk}")
    big_k = ora.normal_bf16((B, Hkv, int(L.max()), D), seed=71)
    big_v = ora.normal_bf16((B, Hkv, int(L.max()), D), seed=72)
    q = ora.normal_bf16((B, Hq, T, D), seed=73)
    cache = ring_cache(ema, ring_from(ora, big_k, L, W), ring_from(ora, big_v, L, W))
    out = ema.prefill_attention(dev(q), cache, dev(qo), causal=True, chunk_only=chunk)
    torch.cuda.synchronize()
    lo = np.maximum(L - W, 0)
    if chunk:
        lo = np.maximum(lo, qo)
    ref = ora.sdpa(q, big_k, big_v, L, scale_of(D), True, kv_begin=lo)
    assert_close(host(out), ref, f"paired rotating prefill chunk_only={chunk}")


def test_rotating_prefill_without_wrap_equals_static(ema, ora):
    import torch

    B, Hq, Hkv, D, cap, T = 2, 16, 4, 128, 512, 200
    qo = np.array([0, 300], np.int32)
    kc = ora.normal_bf16((B, Hkv, cap, D), seed=71)
    vc = ora.normal_bf16((B, Hkv, cap, D), seed=72)
    q = ora.normal_bf16((B, Hq, T, D), seed=73)
    a = ema.prefill_attention(dev(q), ema.StaticCache(B, Hkv, cap, D, k=dev(kc), v=dev(vc)), dev(qo))
    b = ema.prefill_attention(dev(q), ring_cache(ema, kc, vc), dev(qo))
    torch.cuda.synchronize()
    assert np.array_equal(host(a), host(b))


def ring_any(ora, big, totals, window, fill):
    """ring_from for any element type and trailing shape: unheld rows hold `fill`."""
    B, Hkv = big.shape[:2]
    ring = np.empty((B, Hkv, window) + big.shape[3:], big.dtype)
    ring[...] = fill
    for b in range(B):
        for r, p in ora.ring_rows(int(totals[b]), window).items():
            ring[b, :, r] = big[b, :, p]
    return ring


@pytest.mark.parametrize("q_off,T,W,chunk", [
    ((200, 150), 100, 256, False),  # ends past the ring
    ((500, 433), 128, 192, True),   # several wraps, chunk-only keys
    ((0, 37), 100, 256, False),     # no wrap
])
def test_rotating_fp8_prefill_equals_bf16_ring(ema, ora, q_off, T, W, chunk):
    """Prefill over a rotating FP8 cache: its held rows decoded into a ring-shaped bf16
    copy, then the ring prefill. Bit-identical to a bf16 ring holding the decoded values;
    within the bf16 tolerance of the oracle over the window."""
    import torch
    from test_gpu_fp8 import quantized_pair

    B, Hq, Hkv, D = 2, 8, 2, 128
    qo = np.asarray(q_off, np.int32)
    L = qo + T
    n = int(L.max())
    say(f"rotating fp8 prefill W={W} q_off={qo.tolist()} T={T} chunk_only={chunk}")
    (kc, ke, kd), (vc, ve, vd) = quantized_pair(ora, (B, Hkv, n, D), seed=W + 7)
    q = ora.normal_bf16((B, Hq, T, D), seed=W + 9)
    c8 = ema.StaticCache(B, Hkv, W, D, dtype="fp8", rotating=True,
                         k=dev(ring_any(ora, kc, L, W, 0x7F)), v=dev(ring_any(ora, vc, L, W, 0x7F)),
                         k_exp=dev(ring_any(ora, ke, L, W, 0)), v_exp=dev(ring_any(ora, ve, L, W, 0)))
    c16 = ring_cache(ema, ring_from(ora, kd, L, W), ring_from(ora, vd, L, W))
    max_kv = W if n > W else n
    o8 = ema.prefill_attention(dev(q), c8, dev(qo), causal=True, chunk_only=chunk, max_kv_len=max_kv)
    o16 = ema.prefill_attention(dev(q), c16, dev(qo), causal=True, chunk_only=chunk)
    torch.cuda.synchronize()
    assert np.array_equal(host(o8), host(o16)), "decoded ring == the bf16 ring"
    lo = np.maximum(L - W, 0)
    if chunk:
        lo = np.maximum(lo, qo)
    assert_close(host(o8), ora.sdpa(q, kd, vd, L, scale_of(D), True, kv_begin=lo), f"rotating fp8 prefill W={W}")


def _fp8_ring(ema, ora, totals, W, D, seed, B=3, Hkv=4):
    """FP8 ring over the oracle's quantisation of a chronological cache of totals.max()
    positions; unheld rows hold code 0x7F (NaN in E4M3FN). Returns (cache, decoded K, V)."""
    from test_gpu_fp8 import quantized_pair

    (kc, ke, kd), (vc, ve, vd) = quantized_pair(ora, (B, Hkv, int(totals.max()), D), seed=seed)
    cache = ema.StaticCache(B, Hkv, W, D, dtype="fp8", rotating=True,
                            k=dev(ring_any(ora, kc, totals, W, 0x7F)), v=dev(ring_any(ora, vc, totals, W, 0x7F)),
                            k_exp=dev(ring_any(ora, ke, totals, W, 0)), v_exp=dev(ring_any(ora, ve, totals, W, 0)))
    return cache, kd, vd


@pytest.mark.parametrize("W", [64, 96])
def test_rotating_fp8_decode_attends_the_window(ema, ora, W):
    """Decode over a rotating FP8 cache attends its min(length, W) held rows, decoded
    exactly; a read of an unheld row (NaN codes) would show."""
    import torch

    B, Hq, Hkv, D = 3, 16, 4, 128
    N = np.array([W - 5, W + 37, 3 * W + 1], np.int32)  # tokens seen
    say(f"rotating fp8 decode W={W} N={N.tolist()}")
    cache, kd, vd = _fp8_ring(ema, ora, N, W, D, seed=W + 40, B=B, Hkv=Hkv)
    q = ora.normal_bf16((B, Hq, 1, D), seed=W + 42)
    out = ema.decode_attention(dev(q), cache, dev(N), W)
    torch.cuda.synchronize()
    ref = ora.sdpa(q, kd, vd, N, scale_of(D), False, kv_begin=np.maximum(N - W, 0))
    assert_close(host(out), ref, f"rotating fp8 decode W={W}")


def test_rotating_fp8_fused_step_writes_the_ring_row(ema, ora):
    """The fused step on an FP8 ring writes row offset % W (quantised as pre-attention's)
    and attends the window: it equals pre-attention + decode attention on the same ring,
    and only that row changes."""
    import torch

    B, Hq, Hkv, D, W = 3, 16, 4, 128, 64
    off = np.array([W - 1, W + 10, 2 * W + 63], np.int32)
    say(f"rotating fp8 fused step W={W} off={off.tolist()}")
    qkv = ora.normal_bf16((B, (Hq + 2 * Hkv) * D), seed=53)
    qw = ora.normal_bf16(D, seed=54, mean=1.0, std=0.02)
    kw = ora.normal_bf16(D, seed=55, mean=1.0, std=0.02)
    c_f, _, _ = _fp8_ring(ema, ora, off, W, D, seed=51, B=B, Hkv=Hkv)
    c_p, _, _ = _fp8_ring(ema, ora, off, W, D, seed=51, B=B, Hkv=Hkv)
    before = [host(t).copy() for t in (c_f.k, c_f.k_exp, c_f.v, c_f.v_exp)]
    fused = ema.decode_step(dev(qkv), dev(qw), dev(kw), 1e-6, 1e6, dev(off), Hq, c_f, W)
    q = ema.pre_attention(dev(qkv.reshape(B, 1, -1)), dev(qw), dev(kw), 1e-6, 1e6, dev(off), Hq, c_p)
    pair = ema.decode_attention(q, c_p, dev(off + 1), W)
    torch.cuda.synchronize()
    after = [host(t) for t in (c_f.k, c_f.k_exp, c_f.v, c_f.v_exp)]
    for x, y in zip(after, [host(t) for t in (c_p.k, c_p.k_exp, c_p.v, c_p.v_exp)]):
        assert np.array_equal(x, y), "fused and pre-attention write the same ring rows"
    assert_close(host(fused), host(pair), "fp8 ring fused vs pair", max_abs=1e-2, mean_abs=1e-4)
    for b in range(B):
        r = int(off[b]) % W
        others = np.r_[0:r, r + 1:W]
        for x, y in zip(before, after):
            assert np.array_equal(x[b][:, others], y[b][:, others]), "rows other than offset % W"
        assert not np.array_equal(before[2][b][:, r], after[2][b][:, r]), "the ring row was written"


def _int4_ring(ema, ora, big_bf16, totals, W):
    """int4 ring over the oracle's quantisation of a chronological bf16 cache; unheld rows
    hold all-ones code words, NaN scales and +inf biases. Returns (cache, MLX-dequantized
    chronological values)."""
    out, deq = [], []
    for x in big_bf16:
        w, s, bias = ora.int4_quantize(ora.f32_from_bf16(x))
        out.append((ring_any(ora, w, totals, W, 0xFFFFFFFF), ring_any(ora, s, totals, W, 0x7FC0),
                    ring_any(ora, bias, totals, W, 0x7F80)))
        deq.append(ora.bf16_from_f32(ora.int4_dequantize(w, s, bias)))
    (kw, ks, kb), (vw, vs, vb) = out
    B, Hkv = kw.shape[:2]
    cache = ema.StaticCache(B, Hkv, W, kw.shape[3] * 8, dtype="int4", rotating=True, k=dev(kw.view(np.int32)),
                            v=dev(vw.view(np.int32)), k_scales=dev(ks), k_biases=dev(kb), v_scales=dev(vs),
                            v_biases=dev(vb))
    return cache, deq[0], deq[1]


@pytest.mark.parametrize("W", [64, 96])
def test_rotating_int4_decode_attends_the_window(ema, ora, W):
    import torch

    B, Hq, Hkv, D = 3, 16, 4, 128
    N = np.array([W - 5, W + 37, 3 * W + 1], np.int32)  # tokens seen
    say(f"rotating int4 decode W={W} N={N.tolist()}")
    big_k = ora.normal_bf16((B, Hkv, int(N.max()), D), seed=W + 20)
    big_v = ora.normal_bf16((B, Hkv, int(N.max()), D), seed=W + 21)
    cache, kd, vd = _int4_ring(ema, ora, (big_k, big_v), N, W)
    q = ora.normal_bf16((B, Hq, 1, D), seed=W + 22)
    out = ema.decode_attention(dev(q), cache, dev(N), W)
    torch.cuda.synchronize()
    ref = ora.sdpa(q, kd, vd, N, scale_of(D), False, kv_begin=np.maximum(N - W, 0))
    assert_close(host(out), ref, f"rotating int4 decode W={W}")


def test_rotating_int4_fused_step_writes_the_ring_row(ema, ora):
    """The fused step on an int4 ring writes row offset % W (quantised as pre-attention's)
    and attends the window: it equals pre-attention + decode attention on the same ring,
    and only that row changes."""
    import torch

    B, Hq, Hkv, D, W = 3, 16, 4, 128, 64
    off = np.array([W - 1, W + 10, 2 * W + 63], np.int32)
    say(f"rotating int4 fused step W={W} off={off.tolist()}")
    big_k = ora.normal_bf16((B, Hkv, int(off.max()), D), seed=31)
    big_v = ora.normal_bf16((B, Hkv, int(off.max()), D), seed=32)
    qkv = ora.normal_bf16((B, (Hq + 2 * Hkv) * D), seed=33)
    qw = ora.normal_bf16(D, seed=34, mean=1.0, std=0.02)
    kw = ora.normal_bf16(D, seed=35, mean=1.0, std=0.02)
    c_f, _, _ = _int4_ring(ema, ora, (big_k, big_v), off, W)
    c_p, _, _ = _int4_ring(ema, ora, (big_k, big_v), off, W)
    before = [host(t).copy() for t in (c_f.k, c_f.k_scales, c_f.v, c_f.v_biases)]
    fused = ema.decode_step(dev(qkv), dev(qw), dev(kw), 1e-6, 1e6, dev(off), Hq, c_f, W)
    q = ema.pre_attention(dev(qkv.reshape(B, 1, -1)), dev(qw), dev(kw), 1e-6, 1e6, dev(off), Hq, c_p)
    pair = ema.decode_attention(q, c_p, dev(off + 1), W)
    torch.cuda.synchronize()
    assert np.array_equal(host(c_f.v), host(c_p.v)) and np.array_equal(host(c_f.v_scales), host(c_p.v_scales))
    assert_close(host(fused), host(pair), "int4 ring fused vs pair", max_abs=1e-2, mean_abs=1e-4)
    after = [host(t) for t in (c_f.k, c_f.k_scales, c_f.v, c_f.v_biases)]
    for b in range(B):
        r = int(off[b]) % W
        others = np.r_[0:r, r + 1:W]
        for x, y in zip(before, after):
            assert np.array_equal(x[b][:, others], y[b][:, others]), "rows other than offset % W"
        assert not np.array_equal(before[2][b][:, r], after[2][b][:, r]), "the ring row was written"
