"""GPU parity of the 4-bit affine KV cache (the reference's int4 KV buffers,
crates/serve/src/engine_ext.rs:92-157: MLX affine quantisation, group 64), through the C ABI.

Bars:
  - written rows (pre_attention, the fused step, the bf16 -> int4 converter): words, scales
    and biases bit-exact against the oracle's quantisation of the same bf16 rows;
  - decode over an int4 cache: within the bf16 tolerance (max-abs 2e-2, mean-abs 2e-3) of
    the f64 oracle over MLX's dequantized bf16 values (what the reference attends), and
    within one bf16 step (2^-7 |ref|) + 6e-3 per element, mean-abs 1e-3, of an f64
    attention over the exact affine values scale * code + bias (what the kernel attends: it
    skips the bf16 rounding of MLX's dequantize). What remains is the bf16 rounding of the
    PV operand P * scale (relative 2^-9 of scale * code, which can exceed the value itself
    where code and bias cancel) and f32 sums.
"""
import numpy as np
import pytest

from gpu_util import assert_close, dev, f32, host, say, scale_of

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ema():
    import torch

    if not torch.cuda.is_available():
        pytest.fail("GPU tests need a ROCm GPU")
    import ema_attn

    ema_attn.lib()
    return ema_attn


def int4_cache(ema, k, v):
    """StaticCache over oracle-quantised (words, scales, biases) for K and V."""
    (kw, ks, kb), (vw, vs, vb) = k, v
    B, Hkv, cap, W = kw.shape
    return ema.StaticCache(B, Hkv, cap, W * 8, dtype="int4", k=dev(kw.view(np.int32)), v=dev(vw.view(np.int32)),
                           k_scales=dev(ks), k_biases=dev(kb), v_scales=dev(vs), v_biases=dev(vb))


def quantized_kv(ora, shape, seed, outliers=False):
    """Random bf16 K/V rows quantised by the oracle: ((words, scales, biases), MLX-dequantized bf16)."""
    out = []
    for i in range(2):
        x = ora.normal_f32(shape, seed=seed + i)
        if outliers and i == 0:
            sel = np.random.default_rng(seed).random(shape, dtype=np.float32) < 0.01
            x[sel] *= 8.0
        x = ora.f32_from_bf16(ora.bf16_from_f32(x))
        q = ora.int4_quantize(x)
        out.append((q, ora.bf16_from_f32(ora.int4_dequantize(*q))))
    return out


def sdpa_affine(ora, q, kq, vq, L, scale):
    """f64 decode attention over the exact affine values; q [B, Hq, 1, D] bf16 -> [B, Hq*D] f64."""
    K = ora.int4_affine_values(*kq)
    V = ora.int4_affine_values(*vq)
    B, Hq, _, D = q.shape
    Hkv = K.shape[1]
    G = Hq // Hkv
    out = np.zeros((B, Hq, D))
    qf = f32(q).astype(np.float64)
    for b in range(B):
        for h in range(Hq):
            if L[b] == 0:
                continue
            s = K[b, h // G, :L[b]] @ qf[b, h, 0] * scale
            p = np.exp(s - s.max())
            out[b, h] = p @ V[b, h // G, :L[b]] / p.sum()
    return out.reshape(B, Hq * D)


def close_f64(got, ref, what, rel=2.0 ** -7, abs_=6e-3, mean_abs=1e-3):
    """Per element |got - ref| <= rel |ref| + abs_ (one bf16 step of the output plus the
    rounding of the PV operand), and the mean below mean_abs."""
    g = f32(got).astype(np.float64).reshape(ref.shape)
    d = np.abs(g - ref)
    excess = d - (rel * np.abs(ref) + abs_)
    say(f"  {what}: max_abs={d.max():.3e} mean_abs={d.mean():.3e} worst excess={excess.max():.3e}")
    assert np.isfinite(g).all() and excess.max() <= 0 and d.mean() <= mean_abs, what


# ------------------------------------------------------------------ writes
@pytest.mark.parametrize("flags", [0, 2, 3])
def test_int4_write_after_norm_rope(ema, ora, flags):
    """pre_attention into an int4 cache writes the oracle's quantisation of the bf16 k, v rows
    the same kernel writes into a bf16 cache (which the bf16 tests hold to the oracle)."""
    import torch

    B, T, Hq, Hkv, D, cap = 2, 7, 16, 8, 128, 64
    say(f"int4 write after norm/rope flags={flags}")
    qkv = ora.normal_bf16((B, T, (Hq + 2 * Hkv) * D), seed=800 + flags, std=2.0)
    qw = ora.normal_bf16(D, seed=801, mean=1.0, std=0.02)
    kw = ora.normal_bf16(D, seed=802, mean=1.0, std=0.02)
    off = np.array([0, 40], np.int32)
    c16 = ema.StaticCache(B, Hkv, cap, D)
    c4 = ema.StaticCache(B, Hkv, cap, D, dtype="int4")
    q16 = ema.pre_attention(dev(qkv), dev(qw), dev(kw), 1e-6, 1e6, dev(off), Hq, c16, flags=flags)
    q4 = ema.pre_attention(dev(qkv), dev(qw), dev(kw), 1e-6, 1e6, dev(off), Hq, c4, flags=flags)
    torch.cuda.synchronize()
    assert np.array_equal(host(q16), host(q4)), "q does not depend on the cache format"
    for src, words, sc, bi in ((c16.k, c4.k, c4.k_scales, c4.k_biases), (c16.v, c4.v, c4.v_scales, c4.v_biases)):
        rw, rs, rb = ora.int4_quantize(ora.f32_from_bf16(host(src)))
        gw, gs, gb = host(words).view(np.uint32), host(sc), host(bi)
        for b in range(B):
            sl = slice(off[b], off[b] + T)
            assert np.array_equal(gw[b][:, sl], rw[b][:, sl])
            assert np.array_equal(gs[b][:, sl], rs[b][:, sl]) and np.array_equal(gb[b][:, sl], rb[b][:, sl])
            rest = np.r_[0:off[b], off[b] + T:cap]
            assert not gw[b][:, rest].any() and not gs[b][:, rest].any()


def special_rows(ora, n, D=128):
    """Rows that exercise the quantiser's cases: zeros, constants, ties at half steps, both
    signs of edge, tiny and large ranges, single outliers, a wide exponent range."""
    rng = np.random.default_rng(5)
    rows = []
    rows.append(np.zeros(D))
    rows.append(np.full(D, -3.5))
    r = np.zeros(D)
    r[:16] = np.arange(16)
    r[16:64] = 6.5
    r[64:] = -np.arange(64) / 4
    rows.append(r)
    rows.append(rng.normal(size=D) * 1e-6)
    rows.append(rng.normal(size=D) * 1e4)
    r = rng.normal(size=D)
    r[3], r[70] = 50.0, -50.0
    rows.append(r)
    r = np.abs(rng.normal(size=D)) + 2.0  # one sign only
    rows.append(r)
    rows.append(-r)
    e = rng.integers(-60, 60, size=(n, D))
    m = rng.uniform(-2, 2, size=(n, D))
    rows.extend(list(m * np.exp2(e)))
    while len(rows) < n:
        rows.append(rng.normal(size=D) * rng.uniform(0.01, 100))
    x = np.asarray(rows[:n], dtype=np.float32)
    return ora.f32_from_bf16(ora.bf16_from_f32(x))


@pytest.mark.parametrize("src_row,dst_row,n", [(0, 0, 96), (5, 32, 40), (0, 95, 1)])
def test_int4_converter(ema, ora, src_row, dst_row, n):
    """ema_kvcache_quantize_int4 (convert_kv_to_int4) writes the oracle's quantisation of the
    bf16 rows, for special and random rows, and nothing else."""
    import torch

    B, Hkv, D, cap16, cap4 = 2, 3, 128, 100, 128
    say(f"int4 converter rows {src_row} -> {dst_row} x {n}")
    x = special_rows(ora, B * Hkv * cap16 * 2).reshape(2, B, Hkv, cap16, D)
    kb16, vb16 = ora.bf16_from_f32(x[0]), ora.bf16_from_f32(x[1])
    src = ema.StaticCache(B, Hkv, cap16, D, k=dev(kb16), v=dev(vb16))
    dst = ema.StaticCache(B, Hkv, cap4, D, dtype="int4")
    ema.quantize_int4(src, dst, n, src_row=src_row, dst_row=dst_row)
    torch.cuda.synchronize()
    for xs, words, sc, bi in ((x[0], dst.k, dst.k_scales, dst.k_biases), (x[1], dst.v, dst.v_scales, dst.v_biases)):
        rw, rs, rb = ora.int4_quantize(xs[:, :, src_row:src_row + n])
        gw, gs, gb = host(words).view(np.uint32), host(sc), host(bi)
        sl = slice(dst_row, dst_row + n)
        assert np.array_equal(gw[:, :, sl], rw), "words"
        assert np.array_equal(gs[:, :, sl], rs) and np.array_equal(gb[:, :, sl], rb), "scales/biases"
        rest = np.r_[0:dst_row, dst_row + n:cap4]
        assert not gw[:, :, rest].any() and not gs[:, :, rest].any() and not gb[:, :, rest].any()


# ------------------------------------------------------------------ decode
@pytest.mark.parametrize("G,lengths,cap", [
    (4, [1, 31, 32, 33, 100, 1000, 1024], 1024),
    (8, [4096, 17, 2500], 4096),
    (1, [64, 65, 3, 0], 96),
    (16, [300, 1], 320),
    (5, [320, 33, 1, 250], 320),  # 5 query heads per kv head (Qwen3-14B)
    (2, [0, 96] + [int(x) for x in np.random.default_rng(820).integers(0, 97, size=68)], 96),  # B 70
])
def test_int4_decode(ema, ora, G, lengths, cap):
    import torch

    Hkv, D = 4, 128
    B, Hq = len(lengths), 4 * G
    say(f"int4 decode G={G} lengths={lengths} cap={cap}")
    (kq, kd), (vq, vd) = quantized_kv(ora, (B, Hkv, cap, D), seed=810 + G, outliers=True)
    q = ora.normal_bf16((B, Hq, 1, D), seed=815)
    L = np.asarray(lengths, np.int32)
    c4 = int4_cache(ema, kq, vq)
    o4 = ema.decode_attention(dev(q), c4, dev(L), int(L.max()))
    torch.cuda.synchronize()
    assert_close(host(o4), ora.sdpa(q, kd, vd, L, scale_of(D), False), "int4 decode vs oracle (MLX values)")
    if cap <= 1024:
        close_f64(host(o4), sdpa_affine(ora, q, kq, vq, L, scale_of(D)), "int4 decode vs exact affine values")
    if (L == 0).any():
        assert not host(o4)[L == 0].any()


def test_int4_decode_qwen3_8b_batched_shape(ema, ora):
    """Batch 32, 32q/8kv, cap 8192, lengths U[512, 8192] (the benchmark workload)."""
    import torch

    B, Hq, Hkv, D, cap = 32, 32, 8, 128, 8192
    L = np.random.default_rng(1234).integers(512, 8193, size=B).astype(np.int32)
    say("int4 decode B32 32q/8kv cap 8192")
    (kq, kd), (vq, vd) = quantized_kv(ora, (B, Hkv, cap, D), seed=820)
    q = ora.normal_bf16((B, Hq, 1, D), seed=822)
    c4 = int4_cache(ema, kq, vq)
    del kq, vq
    o4 = ema.decode_attention(dev(q), c4, dev(L), cap)
    torch.cuda.synchronize()
    assert_close(host(o4), ora.sdpa(q, kd, vd, L, scale_of(D), False), "int4 decode 8B batched")


def _poison_rows(qkv_parts, lengths):
    """Copy of (words, scales, biases) whose rows >= lengths[b] hold all-ones code words,
    NaN scales and +inf biases (bf16 0x7FC0 / 0x7F80)."""
    w, sc, bi = (a.copy() for a in qkv_parts)
    for b, L in enumerate(lengths):
        w.view(np.uint32)[b, :, L:] = 0xFFFFFFFF
        sc.view(np.uint16)[b, :, L:] = 0x7FC0
        bi.view(np.uint16)[b, :, L:] = 0x7F80
    return w, sc, bi


def test_int4_decode_ignores_poisoned_rows_past_the_length(ema, ora):
    """Rows at or past a sequence's length never reach the output: codes, scales and biases
    set to garbage / NaN / inf there give a bit-identical result (lengths not multiples of
    the 32-row tile; a 1000-row segment split over several workers)."""
    import torch

    B, Hq, Hkv, D, cap = 3, 16, 4, 128, 4096
    L = np.array([37, 1000, 2017], np.int32)
    say(f"int4 decode NaN poison past lengths {L.tolist()}")
    (kq, _), (vq, _) = quantized_kv(ora, (B, Hkv, cap, D), seed=870)
    q = dev(ora.normal_bf16((B, Hq, 1, D), seed=872))
    clean = ema.decode_attention(q, int4_cache(ema, kq, vq), dev(L), cap)
    poisoned = ema.decode_attention(q, int4_cache(ema, _poison_rows(kq, L), _poison_rows(vq, L)), dev(L), cap)
    torch.cuda.synchronize()
    assert np.array_equal(host(clean), host(poisoned))
    assert np.isfinite(f32(host(clean))).all()


def test_int4_fused_step_ignores_poisoned_rows_past_the_offset(ema, ora):
    """The fused step writes row offset (poisoned beforehand too) and attends offset + 1 rows:
    poisoned rows after it leave the output and the written row bit-identical."""
    import torch

    B, Hq, Hkv, D, cap = 3, 16, 4, 128, 4096
    off = np.array([36, 999, 2016], np.int32)
    say(f"int4 fused step NaN poison past offsets {off.tolist()}")
    (kq, _), (vq, _) = quantized_kv(ora, (B, Hkv, cap, D), seed=880)
    qkv = dev(ora.normal_bf16((B, (Hq + 2 * Hkv) * D), seed=882))
    qw = dev(ora.normal_bf16(D, seed=883, mean=1.0, std=0.02))
    kw = dev(ora.normal_bf16(D, seed=884, mean=1.0, std=0.02))
    c_clean = int4_cache(ema, kq, vq)
    c_pois = int4_cache(ema, _poison_rows(kq, off), _poison_rows(vq, off))
    clean = ema.decode_step(qkv, qw, kw, 1e-6, 1e6, dev(off), Hq, c_clean, cap)
    poisoned = ema.decode_step(qkv, qw, kw, 1e-6, 1e6, dev(off), Hq, c_pois, cap)
    torch.cuda.synchronize()
    assert np.array_equal(host(clean), host(poisoned))
    assert np.isfinite(f32(host(clean))).all()
    for a, b in ((c_clean.k, c_pois.k), (c_clean.k_scales, c_pois.k_scales), (c_clean.v_biases, c_pois.v_biases)):
        ha, hb = host(a), host(b)
        for s in range(B):
            assert np.array_equal(ha[s, :, off[s]], hb[s, :, off[s]]), "the written row"


# ------------------------------------------------------------------ fused step
@pytest.mark.parametrize("flags", [0, 3])
def test_int4_fused_step(ema, ora, flags):
    """decode_step on an int4 cache: the new row is quantised as pre_attention's and attended
    in its stored form; rows elsewhere stay untouched."""
    import torch

    B, Hq, Hkv, D, cap = 6, 16, 4, 128, 224
    off = np.array([0, 31, 32, 100, 223, 63], np.int32)
    say(f"int4 fused step flags={flags}")
    (kq, kd), (vq, vd) = quantized_kv(ora, (B, Hkv, cap, D), seed=830)
    qkv = ora.normal_bf16((B, (Hq + 2 * Hkv) * D), seed=833)
    qw = ora.normal_bf16(D, seed=834, mean=1.0, std=0.02)
    kw = ora.normal_bf16(D, seed=835, mean=1.0, std=0.02)
    c_pair = int4_cache(ema, kq, vq)
    q = ema.pre_attention(dev(qkv.reshape(B, 1, -1)), dev(qw), dev(kw), 1e-6, 1e6, dev(off), Hq, c_pair,
                          flags=flags)
    pair = ema.decode_attention(q, c_pair, dev(off + 1), cap)
    c_f = int4_cache(ema, kq, vq)
    fused = ema.decode_step(dev(qkv), dev(qw), dev(kw), 1e-6, 1e6, dev(off), Hq, c_f, cap, flags=flags)
    torch.cuda.synchronize()
    g = [host(t) for t in (c_f.k, c_f.k_scales, c_f.k_biases, c_f.v, c_f.v_scales, c_f.v_biases)]
    p = [host(t) for t in (c_pair.k, c_pair.k_scales, c_pair.k_biases, c_pair.v, c_pair.v_scales, c_pair.v_biases)]
    for i in (3, 4, 5):  # v rows: a bit copy of the input, quantised identically
        assert np.array_equal(g[i], p[i]), f"v buffer {i}"
    ref = (kq[0], kq[1], kq[2])
    for b in range(B):
        others = np.r_[0:off[b], off[b] + 1:cap]
        for i in range(3):
            assert np.array_equal(g[i][b][:, others], ref[i].view(g[i].dtype)[b][:, others]), f"k buffer {i}"
    # k rows: the same quantisation of a bf16 k that may differ from pre_attention's in the
    # last bit (f32 sum order), so compare the dequantized rows
    dk_f = ora.int4_dequantize(g[0].view(np.uint32), g[1].view(np.uint16), g[2].view(np.uint16))
    dk_p = ora.int4_dequantize(p[0].view(np.uint32), p[1].view(np.uint16), p[2].view(np.uint16))
    assert_close(ora.bf16_from_f32(dk_f), ora.bf16_from_f32(dk_p), "fused vs pair dequantized k", max_abs=0.3,
                 mean_abs=1e-4)
    assert_close(host(fused), host(pair), "int4 fused vs pair", max_abs=1e-2, mean_abs=1e-4)
    L = np.clip(off + 1, 0, cap).astype(np.int32)
    dv = ora.bf16_from_f32(ora.int4_dequantize(g[3].view(np.uint32), g[4].view(np.uint16), g[5].view(np.uint16)))
    assert_close(host(fused), ora.sdpa(host(q), ora.bf16_from_f32(dk_f), dv, L, scale_of(D), False),
                 "int4 fused vs oracle")


def test_int4_graph_replay_matches_eager(ema, ora):
    """The fused int4 step captured in a HIP graph: every replay, with eager work and
    synchronisation in between, equals the eager result (and rewrites the same row)."""
    import torch

    B, Hq, Hkv, D, cap = 4, 16, 8, 128, 1024
    off = np.array([100, 1023, 0, 512], np.int32)
    (kq, _), (vq, _) = quantized_kv(ora, (B, Hkv, cap, D), seed=860)
    qkv = dev(ora.normal_bf16((B, (Hq + 2 * Hkv) * D), seed=862))
    qw = dev(ora.normal_bf16(D, seed=863, mean=1.0, std=0.02))
    kw = dev(ora.normal_bf16(D, seed=864, mean=1.0, std=0.02))
    cache = int4_cache(ema, kq, vq)
    off_d = dev(off)
    out = torch.empty((B, Hq * D), dtype=torch.bfloat16, device="cuda")
    ws = ema.decode_workspace(B, Hq, Hkv, D, cap)

    def step():
        ema.decode_step(qkv, qw, kw, 1e-6, 1e6, off_d, Hq, cache, cap, out=out, workspace=ws)

    say("int4 fused step graph replay")
    step()
    torch.cuda.synchronize()
    eager = host(out).copy()
    stored = [host(t).copy() for t in (cache.k, cache.k_scales, cache.k_biases, cache.v_scales)]
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
        for t, ref in zip((cache.k, cache.k_scales, cache.k_biases, cache.v_scales), stored):
            assert np.array_equal(host(t), ref)
        step()
        torch.cuda.synchronize()
