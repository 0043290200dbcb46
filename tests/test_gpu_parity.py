"""GPU parity of the HIP path against the CPU oracle, through the C ABI.

Tolerance (bf16 outputs vs the f64 oracle): max-abs 2e-2, mean-abs 2e-3.
KV-cache write positions, V rows and masking are bit-exact; post-RoPE K rows
may differ from the oracle by the last bf16 bit (f32 op order, sincos ulp) and
are held to the same 2e-2 / 2e-3 bound.
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


def make_cache(ema, kc: np.ndarray, vc: np.ndarray):
    B, Hkv, cap, D = kc.shape
    return ema.StaticCache(B, Hkv, cap, D, k=dev(kc), v=dev(vc))


# ------------------------------------------------------------ pre-attention
@pytest.mark.parametrize("D", [64, 128, 256])
@pytest.mark.parametrize("flags", [0, 1, 2, 3, 8, 16, 10])
def test_pre_attention_small(ema, ora, D, flags):
    """flags: 1 no norms, 2 no RoPE, 8 no q norm, 16 no k norm (each norm is optional on
    its own, crates/ops/src/attention.rs:57-76); the absent weights are passed as null."""
    import torch

    B, T, Hq, Hkv, cap = 2, 5, 4, 2, 16
    say(f"pre_attention small D={D} flags={flags}")
    qkv = ora.normal_bf16((B, T, (Hq + 2 * Hkv) * D), seed=100 + D + flags)
    qw = ora.normal_bf16(D, seed=101, mean=1.0, std=0.02)
    kw = ora.normal_bf16(D, seed=102, mean=1.0, std=0.02)
    off = np.array([3, 9], np.int32)
    junk = ora.normal_bf16((B, Hkv, cap, D), seed=103)
    kr, vr = junk.copy(), junk.copy()
    q_ref = ora.pre_attention(qkv, qw, kw, 1e-6, 1e6, off, Hq, Hkv, kr, vr, flags=flags)
    cache = make_cache(ema, junk, junk)
    qw_d = None if flags & (1 | 8) else dev(qw)
    kw_d = None if flags & (1 | 16) else dev(kw)
    q = ema.pre_attention(dev(qkv), qw_d, kw_d, 1e-6, 1e6, dev(off), Hq, cache, flags=flags)
    torch.cuda.synchronize()
    kg, vg = host(cache.k), host(cache.v)
    assert np.array_equal(vg, vr), "V rows must be a bit copy at [off, off+T)"
    for b in range(B):
        rows = np.r_[0:off[b], off[b] + T:cap]
        assert np.array_equal(kg[b][:, rows], junk[b][:, rows]), "rows outside the write changed"
    assert_close(host(q), q_ref, "q_out")
    assert_close(kg, kr, "k cache")
    if flags & 2 and flags & 1:  # pure copy: bit exact
        assert np.array_equal(kg, kr) and np.array_equal(host(q), q_ref)


def test_pre_attention_prefill_shape(ema, ora):
    """2048 tokens, 16q/8kv, written at offset 0 of a 4096-capacity cache."""
    import torch

    B, T, Hq, Hkv, D, cap = 1, 2048, 16, 8, 128, 4096
    say("pre_attention T=2048 16q/8kv cap 4096")
    qkv = ora.normal_bf16((B, T, (Hq + 2 * Hkv) * D), seed=110)
    qw = ora.normal_bf16(D, seed=111, mean=1.0, std=0.02)
    kw = ora.normal_bf16(D, seed=112, mean=1.0, std=0.02)
    off = np.zeros(B, np.int32)
    kr = np.zeros((B, Hkv, cap, D), np.uint16)
    vr = kr.copy()
    q_ref = ora.pre_attention(qkv, qw, kw, 1e-6, 1e6, off, Hq, Hkv, kr, vr)
    cache = ema.StaticCache(B, Hkv, cap, D)
    q = ema.pre_attention(dev(qkv), dev(qw), dev(kw), 1e-6, 1e6, dev(off), Hq, cache)
    torch.cuda.synchronize()
    assert np.array_equal(host(cache.v), vr)
    assert np.all(host(cache.k)[:, :, T:] == 0)
    assert_close(host(q), q_ref, "q_out")
    assert_close(host(cache.k)[:, :, :T], kr[:, :, :T], "k cache")
    # A bf16 flip of the normalised value (f32 vs f64 rsqrt) moves both outputs of its
    # RoPE pair by up to one ulp of the pair's magnitude; bound each element by that.
    g, r = f32(host(cache.k)).astype(np.float64), f32(kr).astype(np.float64)
    half = D // 2
    pair = np.sqrt(r[..., :half] ** 2 + r[..., half:] ** 2)
    pair = np.concatenate([pair, pair], axis=-1)
    ulp = np.exp2(np.floor(np.log2(np.maximum(pair, 2.0 ** -126))) - 7)
    diff = np.abs(g - r)
    say(f"  k elements differing from the oracle: {np.count_nonzero(diff)} of {diff.size}, "
        f"max {float(np.max(diff / ulp)):.2f} pair-ulp")
    assert np.all(diff <= 2 * ulp + 2.0 ** -11)


def test_pre_attention_decode_positions(ema, ora):
    """Decode write: one token per sequence at its own offset (scatter_single)."""
    import torch

    B, Hq, Hkv, D, cap = 32, 32, 8, 128, 512
    rng = np.random.default_rng(5)
    off = rng.integers(0, cap, size=B).astype(np.int32)
    off[0], off[1] = 0, cap - 1
    say("pre_attention decode B=32 ragged offsets")
    qkv = ora.normal_bf16((B, 1, (Hq + 2 * Hkv) * D), seed=120)
    qw = ora.normal_bf16(D, seed=121, mean=1.0, std=0.02)
    kw = ora.normal_bf16(D, seed=122, mean=1.0, std=0.02)
    base = ora.normal_bf16((B, Hkv, cap, D), seed=123)
    kr, vr = base.copy(), base.copy()
    q_ref = ora.pre_attention(qkv, qw, kw, 1e-6, 1e6, off, Hq, Hkv, kr, vr)
    cache = make_cache(ema, base, base)
    q = ema.pre_attention(dev(qkv), dev(qw), dev(kw), 1e-6, 1e6, dev(off), Hq, cache)
    torch.cuda.synchronize()
    kg = host(cache.k)
    assert np.array_equal(host(cache.v), vr)
    changed = np.any(kg != base, axis=(1, 3))
    for b in range(B):
        rows = np.nonzero(changed[b])[0]
        assert set(rows.tolist()) <= {int(off[b])}
    assert_close(host(q), q_ref, "q_out")
    assert_close(kg, kr, "k cache")


def test_pre_attention_overflow_writes_nothing(ema, ora):
    import torch

    B, T, Hq, Hkv, D, cap = 2, 4, 2, 1, 128, 8
    qkv = ora.normal_bf16((B, T, (Hq + 2 * Hkv) * D), seed=130)
    base = ora.normal_bf16((B, Hkv, cap, D), seed=131)
    cache = make_cache(ema, base, base)
    off = np.array([5, 2], np.int32)  # sequence 0 would overflow (5 + 4 > 8)
    ema.pre_attention(dev(qkv), None, None, 1e-6, 1e6, dev(off), Hq, cache, flags=3)
    torch.cuda.synchronize()
    kg = host(cache.k)
    assert np.array_equal(kg[0], base[0])
    assert not np.array_equal(kg[1], base[1])


# ------------------------------------------------------------------ decode
def _decode_case(ema, ora, B, Hq, Hkv, D, cap, lengths, seed, outliers=False, poison=False, max_len=None):
    import torch

    q = ora.normal_bf16((B, Hq, 1, D), seed=seed)
    kc = ora.normal_bf16((B, Hkv, cap, D), seed=seed + 1)
    vc = ora.normal_bf16((B, Hkv, cap, D), seed=seed + 2)
    if outliers:  # 1% of K entries x8 before bf16 rounding
        kf = ora.normal_f32((B, Hkv, cap, D), seed=seed + 1)
        sel = np.random.default_rng(seed).random(kf.shape, dtype=np.float32) < 0.01
        kf[sel] *= 8.0
        kc = ora.bf16_from_f32(kf)
        del kf, sel
    L = np.asarray(lengths, np.int32)
    ref = ora.sdpa(q, kc, vc, L, scale_of(D), False)
    if poison:
        for b in range(B):
            kc[b, :, L[b]:] = 0x7FC0
            vc[b, :, L[b]:] = 0x7FC0
    cache = make_cache(ema, kc, vc)
    out = ema.decode_attention(dev(q), cache, dev(L), int(max_len or L.max()))
    torch.cuda.synchronize()
    return host(out), ref


@pytest.mark.parametrize("G", [1, 2, 3, 4, 5, 6, 8, 12, 16])
def test_decode_small(ema, ora, G):
    B, Hkv, D, cap = 6, 2, 128, 160
    lengths = [1, 31, 32, 33, 100, 160]
    say(f"decode small G={G} lengths={lengths}")
    got, ref = _decode_case(ema, ora, B, Hkv * G, Hkv, D, cap, lengths, seed=200 + G)
    assert_close(got, ref, f"decode G={G}")


def test_decode_stale_tail_is_bit_exact(ema, ora):
    """Rows >= len poisoned with NaN give bit-identical output (mask exactness)."""
    B, Hq, Hkv, D, cap = 4, 8, 2, 128, 256
    lengths = [7, 64, 65, 200]
    say("decode stale-tail NaN poison")
    clean, ref = _decode_case(ema, ora, B, Hq, Hkv, D, cap, lengths, seed=210)
    dirty, _ = _decode_case(ema, ora, B, Hq, Hkv, D, cap, lengths, seed=210, poison=True)
    assert np.array_equal(clean, dirty)
    assert_close(clean, ref, "decode clean")


def test_decode_zero_length_gives_zeros(ema, ora):
    got, _ = _decode_case(ema, ora, 3, 4, 2, 128, 64, [0, 10, 0], seed=220, max_len=64)
    assert np.all(got[0] == 0) and np.all(got[2] == 0) and np.any(got[1] != 0)


@pytest.mark.parametrize("B,Hkv,G,L,cap", [(1, 8, 2, 1024, 4096), (1, 8, 2, 1, 64), (1, 1, 16, 4096, 4096),
                                            (2, 2, 4, 33, 64), (7, 2, 8, 100, 128), (64, 1, 4, 32, 32),
                                            (3, 8, 1, 777, 1024)])
def test_decode_lengths_at_the_bound(ema, ora, B, Hkv, G, L, cap):
    """Every length equal to the host's bound (the split the plan sized is the one the
    kernels take), over small grids of one to 64 sequences. Rows past the lengths poisoned
    with NaN leave the result bit-identical."""
    lengths = [L] * B
    say(f"decode at the bound B={B} {Hkv * G}q/{Hkv}kv L={L} cap={cap}")
    clean, ref = _decode_case(ema, ora, B, Hkv * G, Hkv, 128, cap, lengths, seed=280 + B + L)
    dirty, _ = _decode_case(ema, ora, B, Hkv * G, Hkv, 128, cap, lengths, seed=280 + B + L, poison=True)
    assert np.array_equal(clean, dirty)
    assert_close(clean, ref, f"decode at the bound B={B} L={L}")


@pytest.mark.parametrize("bound", [40, 1024])
def test_decode_equal_lengths_below_the_bound(ema, ora, bound):
    """Equal lengths below the host's bound: the kernels take the split from the actual tile
    count, not from the bound (NaN tails stay masked)."""
    B, Hkv, G, L, cap = 2, 8, 2, 33, 1024
    say(f"decode, lengths {L} under the bound {bound}")
    clean, ref = _decode_case(ema, ora, B, Hkv * G, Hkv, 128, cap, [L] * B, seed=290, max_len=bound)
    dirty, _ = _decode_case(ema, ora, B, Hkv * G, Hkv, 128, cap, [L] * B, seed=290, poison=True, max_len=bound)
    assert np.array_equal(clean, dirty)
    assert_close(clean, ref, f"decode, lengths under the bound {bound}")


@pytest.mark.parametrize("max_len", [33, 100, 1000, 4096])
def test_decode_split_invariance(ema, ora, max_len):
    """Different max_len hints change the worker split; results stay within tolerance."""
    B, Hq, Hkv, D, cap = 3, 16, 8, 128, 4096
    lengths = [33, 1, 29]
    say(f"decode split max_len={max_len}")
    got, ref = _decode_case(ema, ora, B, Hq, Hkv, D, cap, lengths, seed=230, max_len=max_len)
    assert_close(got, ref, f"decode max_len={max_len}")


def test_decode_lengths_are_clamped_to_the_cache(ema, ora):
    """Lengths past the capacity attend the whole cache; negative ones give zeros."""
    import torch

    B, Hq, Hkv, D, cap = 4, 8, 2, 128, 256
    q = ora.normal_bf16((B, Hq, 1, D), seed=233)
    kc = ora.normal_bf16((B, Hkv, cap, D), seed=234)
    vc = ora.normal_bf16((B, Hkv, cap, D), seed=235)
    given = np.array([cap + 100, -5, cap, 37], np.int32)
    clamped = np.clip(given, 0, cap).astype(np.int32)
    say(f"decode lengths {given.tolist()} over capacity {cap}")
    got = host(ema.decode_attention(dev(q), make_cache(ema, kc, vc), dev(given), cap))
    torch.cuda.synchronize()
    assert_close(got, ora.sdpa(q, kc, vc, clamped, scale_of(D), False), "clamped lengths")
    assert not got[1].any()


@pytest.mark.parametrize("max_len", [1, 100])
def test_decode_max_len_below_the_lengths(ema, ora, max_len):
    """A host bound below the true lengths sizes the grid and workspace for fewer tiles; the
    kernels take the split from the actual tile count (at most the planned workers, each
    with a longer slice), so the result is still exact."""
    B, Hq, Hkv, D, cap = 2, 8, 2, 128, 4096
    lengths = [4000, 3001]
    say(f"decode with max_len {max_len} below lengths {lengths}")
    got, ref = _decode_case(ema, ora, B, Hq, Hkv, D, cap, lengths, seed=232, max_len=max_len)
    assert_close(got, ref, f"decode, max_len {max_len}")


def test_decode_workspace_reuse_is_clean(ema, ora):
    """Reusing one workspace across calls with different lengths (stale partial
    slots from earlier calls) gives the same bits as fresh workspaces."""
    import torch

    B, Hq, Hkv, D, cap = 4, 32, 8, 128, 2048
    q = ora.normal_bf16((B, Hq, 1, D), seed=235)
    kc = ora.normal_bf16((B, Hkv, cap, D), seed=236)
    vc = ora.normal_bf16((B, Hkv, cap, D), seed=237)
    cache = make_cache(ema, kc, vc)
    ws = ema.decode_workspace(B, Hq, Hkv, D, cap)
    qd = dev(q)
    for lengths in ([2048, 1, 700, 1500], [64, 2048, 2048, 3], [2048] * 4, [1500, 900, 33, 1]):
        L = np.asarray(lengths, np.int32)
        say(f"decode workspace reuse lengths={lengths}")
        shared = host(ema.decode_attention(qd, cache, dev(L), cap, workspace=ws))
        fresh = host(ema.decode_attention(qd, cache, dev(L), cap))
        torch.cuda.synchronize()
        assert np.array_equal(shared, fresh)
        assert_close(shared, ora.sdpa(q, kc, vc, L, scale_of(D), False), "reused workspace")


def test_decode_workspace_reuse_across_shapes(ema, ora):
    """One workspace shared by calls of different batch sizes and head counts: its arrival
    counters are left at zero by every call, whatever partial states a call of another
    shape wrote next to them, so each call gives the bits of a fresh workspace."""
    import torch

    D = 128
    ws = ema.decode_workspace(64, 32, 8, D, 8192)  # large enough for every shape below
    for step, (B, Hq, Hkv, cap, seed) in enumerate([(32, 32, 8, 4096, 240), (1, 16, 8, 4096, 241),
                                                      (3, 64, 4, 1024, 242), (32, 32, 8, 4096, 243),
                                                      (64, 8, 8, 512, 244)]):
        rng = np.random.default_rng(seed)
        L = rng.integers(1, cap + 1, size=B).astype(np.int32)
        q = ora.normal_bf16((B, Hq, 1, D), seed=seed)
        kc = ora.normal_bf16((B, Hkv, cap, D), seed=seed + 1)
        vc = ora.normal_bf16((B, Hkv, cap, D), seed=seed + 2)
        cache = make_cache(ema, kc, vc)
        say(f"decode workspace reuse across shapes: step {step} B={B} {Hq}q/{Hkv}kv cap={cap}")
        shared = host(ema.decode_attention(dev(q), cache, dev(L), cap, workspace=ws))
        fresh = host(ema.decode_attention(dev(q), cache, dev(L), cap))
        torch.cuda.synchronize()
        assert np.array_equal(shared, fresh), f"step {step}"
        if step < 3:
            assert_close(shared, ora.sdpa(q, kc, vc, L, scale_of(D), False), f"step {step}")
    assert not host(ws)[:ema.EMA_DECODE_COUNTER_BYTES].any(), "counters left at zero"


def test_decode_merge_in_kernel_and_after_agree(ema, ora):
    """The split's merge runs inside the decode kernel for grids of at most one workgroup
    per CU and in a second kernel for fuller ones; the host's bound of the lengths picks
    the grid. The same inputs through both (bound = the true maximum: 252 workgroups;
    bound = the capacity: 512) match the oracle, for attention and for the fused step with
    the device-side offset advance."""
    import torch

    B, Hq, Hkv, D, cap = 2, 16, 8, 128, 8192
    L = np.array([1000, 2000], np.int32)
    q = ora.normal_bf16((B, Hq, 1, D), seed=250)
    kc = ora.normal_bf16((B, Hkv, cap, D), seed=251)
    vc = ora.normal_bf16((B, Hkv, cap, D), seed=252)
    ref = ora.sdpa(q, kc, vc, L, scale_of(D), False)
    cache = make_cache(ema, kc, vc)
    outs = {}
    for bound in (int(L.max()), cap):
        say(f"decode merge paths: max_len bound {bound}")
        outs[bound] = host(ema.decode_attention(dev(q), cache, dev(L), bound))
        torch.cuda.synchronize()
        assert_close(outs[bound], ref, f"decode, bound {bound}")
    assert_close(outs[cap], outs[int(L.max())], "the two merge paths", max_abs=1e-2, mean_abs=1e-4)
    # fused step with EMA_STEP_ADVANCE through both paths, on _fused_case's inputs (its
    # seeds) against its oracle result
    seed = 253
    got, ref_s, _, _, _, vr, _ = _fused_case(ema, ora, B, Hq, Hkv, D, cap, L - 1, seed=seed)
    assert_close(got, ref_s, "fused step, bound = capacity")
    qkv = ora.normal_bf16((B, (Hq + 2 * Hkv) * D), seed=seed)
    qw = ora.normal_bf16(D, seed=seed + 1, mean=1.0, std=0.02)
    kw = ora.normal_bf16(D, seed=seed + 2, mean=1.0, std=0.02)
    kc2 = ora.normal_bf16((B, Hkv, cap, D), seed=seed + 3)
    vc2 = ora.normal_bf16((B, Hkv, cap, D), seed=seed + 4)
    for bound in (int(L.max()), cap):
        c = make_cache(ema, kc2, vc2)
        off = dev(L - 1)
        out = ema.decode_step(dev(qkv), dev(qw), dev(kw), 1e-6, 1e6, off, Hq, c, bound, flags=ema.EMA_STEP_ADVANCE)
        torch.cuda.synchronize()
        assert_close(host(out), ref_s, f"fused step with advance, bound {bound}")
        assert np.array_equal(host(c.v), vr)
        assert np.array_equal(host(off), L), f"offsets advanced, bound {bound}"


def test_decode_qwen3_1p7b_shape(ema, ora):
    """batch 1, 16q/8kv, D 128, cap 4096, 1024 valid positions."""
    say("decode B1 16q/8kv cap 4096 L 1024")
    got, ref = _decode_case(ema, ora, 1, 16, 8, 128, 4096, [1024], seed=240, poison=True)
    assert_close(got, ref, "decode 1.7B shape")


def test_decode_qwen3_8b_batched_shape(ema, ora):
    """batch 32, 32q/8kv, cap 8192, lengths uniform in [512, 8192]."""
    L = np.random.default_rng(1234).integers(512, 8193, size=32)
    say(f"decode B32 32q/8kv cap 8192 ragged sum(L)={int(L.sum())}")
    got, ref = _decode_case(ema, ora, 32, 32, 8, 128, 8192, L, seed=250, max_len=8192)
    assert_close(got, ref, "decode 8B batched")


def test_decode_qwen3_30b_long_context_shape(ema, ora):
    """batch 8, 32q/4kv (G 8), cap = len = 32768, 1% of K entries x8."""
    say("decode B8 32q/4kv L 32768 outliers")
    got, ref = _decode_case(ema, ora, 8, 32, 4, 128, 32768, [32768] * 8, seed=260, outliers=True)
    assert_close(got, ref, "decode 30B long context")


def test_decode_merge_of_many_pieces(ema, ora):
    """Two long sequences over a full grid: each (sequence, kv head) segment is cut into
    about 100-160 pieces, which the merge kernel folds 16 at a time (and a remainder)."""
    B, Hq, Hkv, D, cap = 2, 8, 2, 128, 32768
    L = [32768, 20001]
    say(f"decode merge of many pieces L={L}")
    got, ref = _decode_case(ema, ora, B, Hq, Hkv, D, cap, L, seed=265, max_len=cap)
    assert_close(got, ref, "decode, many pieces")


@pytest.mark.parametrize("B,cap,bound", [(63, 160, None), (64, 160, None), (65, 160, None), (64, 2048, 2048),
                                         (200, 160, None), (100, 2048, 2048), (1024, 64, None)])
def test_decode_batch_sizes_around_64(ema, ora, B, cap, bound):
    """Up to 64 sequences each wave holds the lengths and tile prefix in its own lanes;
    larger batches scan them into the workgroup's table (at most 1024 rows). Both sides of
    that edge, ragged lengths with empty sequences among them, small grids (the merge inside
    the decode kernel) and full ones (the merge kernel)."""
    Hq, Hkv, D = 8, 2, 128
    rng = np.random.default_rng(270 + B + cap)
    L = rng.integers(1, cap + 1, size=B).astype(np.int32)
    L[::9] = 0
    L[1] = cap
    say(f"decode B={B} cap={cap} bound={bound} sum(L)={int(L.sum())}")
    got, ref = _decode_case(ema, ora, B, Hq, Hkv, D, cap, L, seed=270 + B, poison=True, max_len=bound)
    assert_close(got, ref, f"decode B={B}")
    assert not got[::9].any(), "empty sequences give zeros"


# ----------------------------------------------------------------- prefill
def _prefill_case(ema, ora, B, Hq, Hkv, D, cap, T, q_off, causal, chunk_only, seed, heads=None):
    import torch

    q = ora.normal_bf16((B, Hq, T, D), seed=seed)
    kc = ora.normal_bf16((B, Hkv, cap, D), seed=seed + 1)
    vc = ora.normal_bf16((B, Hkv, cap, D), seed=seed + 2)
    qo = np.asarray(q_off, np.int32)
    cache = make_cache(ema, kc, vc)
    out = host(ema.prefill_attention(dev(q), cache, dev(qo), causal=causal, chunk_only=chunk_only))
    torch.cuda.synchronize()
    kv_len = qo + T
    kv_begin = qo if chunk_only else None
    if heads is None:
        ref = ora.sdpa(q, kc, vc, kv_len, scale_of(D), causal, kv_begin=kv_begin)
        return out, ref
    G = Hq // Hkv
    kvh = sorted({h // G for h in heads})
    sel = [h for kh in kvh for h in range(kh * G, kh * G + G)]
    ref = ora.sdpa(q[:, sel].copy(), kc[:, kvh].copy(), vc[:, kvh].copy(), kv_len, scale_of(D), causal,
                   kv_begin=kv_begin)
    o = out.reshape(B, T, Hq, D)[:, :, sel].reshape(B, T, len(sel) * D)
    return o, ref


@pytest.mark.parametrize("T,q_off,causal,chunk", [
    (1, 0, True, False), (5, 0, True, False), (64, 0, True, False), (128, 0, True, False),
    (200, 0, True, False), (200, 37, True, False), (77, 100, True, True), (130, 50, False, False),
    (300, 0, False, True),
])
@pytest.mark.parametrize("G", [1, 2, 5, 8])
def test_prefill_small(ema, ora, T, q_off, causal, chunk, G):
    B, Hkv, D, cap = 2, 2, 128, 512
    say(f"prefill small T={T} q_off={q_off} causal={causal} chunk={chunk} G={G}")
    got, ref = _prefill_case(ema, ora, B, Hkv * G, Hkv, D, cap, T, [q_off, q_off // 2], causal, chunk,
                             seed=300 + T + G)
    assert_close(got, ref, f"prefill T={T}")


@pytest.mark.parametrize("causal,chunk", [(True, False), (False, False), (True, True)])
def test_prefill_xcd_grid_mapping(ema, ora, causal, chunk):
    """batch x kv heads a multiple of 8 (the XCD-grouped grid order), ragged offsets."""
    B, Hq, Hkv, D, cap, T = 4, 8, 2, 128, 640, 300
    say(f"prefill xcd mapping causal={causal} chunk={chunk}")
    got, ref = _prefill_case(ema, ora, B, Hq, Hkv, D, cap, T, [0, 37, 300, 129], causal, chunk, seed=340)
    assert_close(got, ref, "prefill xcd mapping")


def test_prefill_qwen3_1p7b_2k(ema, ora):
    """1 x 2048 tokens, 16q/8kv, causal from offset 0: every head and row."""
    say("prefill T=2048 16q/8kv causal, all heads")
    got, ref = _prefill_case(ema, ora, 1, 16, 8, 128, 4096, 2048, [0], True, False, seed=310)
    assert_close(got, ref, "prefill 2k 16q")


def test_prefill_qwen3_8b_2k_all_heads(ema, ora):
    """The benchmarked prefill shape: 1 x 2048 tokens, 32q/8kv, causal from offset 0, every
    head and row. With 16 query blocks x 32 heads = 512 items the launch pairs query blocks
    (a workgroup runs block 15-p, then block p)."""
    say("prefill T=2048 32q/8kv causal, all heads (paired blocks)")
    got, ref = _prefill_case(ema, ora, 1, 32, 8, 128, 4096, 2048, [0], True, False, seed=315)
    assert_close(got, ref, "prefill 2k 32q")


# Shapes with at least 2 x 256 query-block items, so the launch pairs query blocks, checked
# in full: odd block counts (the middle block paired with itself), ragged offsets, chunk-only
# windows, non-causal attention, and batch x kv heads not a multiple of the 8 XCDs.
@pytest.mark.parametrize("B,Hq,Hkv,T,q_off,causal,chunk", [
    (4, 16, 4, 1000, [0, 0, 0, 0], True, False),
    (4, 16, 4, 1100, [0, 37, 300, 129], True, False),
    (4, 16, 4, 1100, [64, 0, 250, 7], True, True),
    (4, 16, 4, 1000, [0, 100, 3, 400], False, False),
    (4, 16, 4, 1100, [10, 0, 128, 33], False, True),
    (3, 24, 3, 900, [0, 17, 200], True, False),
])
def test_prefill_paired_blocks(ema, ora, B, Hq, Hkv, T, q_off, causal, chunk):
    say(f"prefill paired B={B} Hq={Hq} Hkv={Hkv} T={T} q_off={q_off} causal={causal} chunk={chunk}")
    got, ref = _prefill_case(ema, ora, B, Hq, Hkv, 128, 1536, T, q_off, causal, chunk, seed=370 + T + B)
    assert_close(got, ref, "prefill paired")


def test_prefill_chunk_on_existing_cache_every_block(ema, ora):
    """64q/8kv, 14336 cached + 2048 new (16384 capacity): all 64 heads at the first and
    last four rows of every 128-row query block, and every row of the first, a middle and
    the last query block."""
    import torch

    B, Hq, Hkv, D, cap, T, off = 1, 64, 8, 128, 16384, 2048, 14336
    say("prefill chunked 64q/8kv off 14336 T 2048, every query block")
    q = ora.normal_bf16((B, Hq, T, D), seed=320)
    kc = ora.normal_bf16((B, Hkv, cap, D), seed=321)
    vc = ora.normal_bf16((B, Hkv, cap, D), seed=322)
    cache = make_cache(ema, kc, vc)
    out = host(ema.prefill_attention(dev(q), cache, dev(np.array([off], np.int32)), causal=True))
    torch.cuda.synchronize()
    out = out.reshape(T, Hq * D)
    for qb in range(T // 128):
        for r0 in (qb * 128, qb * 128 + 124):
            # four consecutive rows: end-aligned causal over kv_len = off + r0 + 4 gives row
            # r0 + i the keys <= off + r0 + i
            ref = ora.sdpa(q[:, :, r0:r0 + 4].copy(), kc, vc, [off + r0 + 4], scale_of(D), True)
            assert_close(out[r0:r0 + 4][None], ref, f"rows {r0}..{r0 + 3}")
    for qb in (0, 8, 15):  # whole query blocks: the pair partners 0/15 and a middle one
        r0 = qb * 128
        say(f"prefill chunked: every row of query block {qb}")
        ref = ora.sdpa(q[:, :, r0:r0 + 128].copy(), kc, vc, [off + r0 + 128], scale_of(D), True)
        assert_close(out[r0:r0 + 128][None], ref, f"query block {qb}")


@pytest.mark.parametrize("causal,chunk,q_off", [(True, True, 100), (True, True, 64), (False, True, 37),
                                                (True, False, 150), (False, False, 0)])
def test_prefill_ignores_cache_rows_outside_the_window(ema, ora, causal, chunk, q_off):
    """NaN in every cache row outside [kv_begin, kv_len) (before a chunk-only window and
    past the valid length) gives bit-identical output to finite data there: the
    reference attends over a slice of the cache (crates/serve/src/forward_qwen3.rs:150),
    so those rows are never read."""
    import torch

    B, Hq, Hkv, D, cap, T = 1, 4, 2, 128, 512, 120
    say(f"prefill NaN outside window causal={causal} chunk={chunk} q_off={q_off}")
    q = ora.normal_bf16((B, Hq, T, D), seed=360)
    kc = ora.normal_bf16((B, Hkv, cap, D), seed=361)
    vc = ora.normal_bf16((B, Hkv, cap, D), seed=362)
    kv_len = q_off + T
    lo = q_off if chunk else 0
    qo = np.asarray([q_off], np.int32)

    def run(k, v):
        out = host(ema.prefill_attention(dev(q), make_cache(ema, k, v), dev(qo), causal=causal, chunk_only=chunk))
        torch.cuda.synchronize()
        return out

    clean = run(kc, vc)
    kp, vp = kc.copy(), vc.copy()
    for a in (kp, vp):  # bf16 quiet NaN bits
        a[:, :, kv_len:] = 0x7FC0
        a[:, :, :lo] = 0x7FC0
    dirty = run(kp, vp)
    assert np.array_equal(clean, dirty)
    ref = ora.sdpa(q, kc, vc, np.asarray([kv_len]), scale_of(D), causal, kv_begin=np.asarray([lo]) if chunk else None)
    assert_close(clean, ref, "prefill window")


def test_prefill_rows_match_decode_on_gpu(ema, ora):
    """Causal prefill row i equals decode with len = off + i + 1 on the same cache."""
    import torch

    B, Hq, Hkv, D, cap, T, off = 1, 8, 2, 128, 1024, 96, 500
    q = ora.normal_bf16((B, Hq, T, D), seed=330)
    kc = ora.normal_bf16((B, Hkv, cap, D), seed=331)
    vc = ora.normal_bf16((B, Hkv, cap, D), seed=332)
    cache = make_cache(ema, kc, vc)
    pre = host(ema.prefill_attention(dev(q), cache, dev(np.array([off], np.int32)), causal=True))
    for i in (0, 17, 95):
        dec = host(ema.decode_attention(dev(q[:, :, i].copy()), cache, dev(np.array([off + i + 1], np.int32)),
                                        off + i + 1))
        torch.cuda.synchronize()
        assert_close(pre[:, i], dec, f"row {i}", max_abs=1e-2, mean_abs=1e-3)


# --------------------------------------------------------------- full step
def test_decode_step_pre_attention_then_attention(ema, ora):
    """The decode step: write one token per sequence, then attend over len = off + 1."""
    import torch

    B, Hq, Hkv, D, cap = 8, 32, 8, 128, 2048
    rng = np.random.default_rng(77)
    off = rng.integers(0, cap, size=B).astype(np.int32)
    say("decode step B=8 pre-attention + attention")
    qkv = ora.normal_bf16((B, 1, (Hq + 2 * Hkv) * D), seed=400)
    qw = ora.normal_bf16(D, seed=401, mean=1.0, std=0.02)
    kw = ora.normal_bf16(D, seed=402, mean=1.0, std=0.02)
    kc = ora.normal_bf16((B, Hkv, cap, D), seed=403)
    vc = ora.normal_bf16((B, Hkv, cap, D), seed=404)
    kr, vr = kc.copy(), vc.copy()
    q_ref = ora.pre_attention(qkv, qw, kw, 1e-6, 1e6, off, Hq, Hkv, kr, vr)
    ref = ora.sdpa(q_ref, kr, vr, off + 1, scale_of(D), False)
    cache = make_cache(ema, kc, vc)
    q = ema.pre_attention(dev(qkv), dev(qw), dev(kw), 1e-6, 1e6, dev(off), Hq, cache)
    out = ema.decode_attention(q, cache, dev(off + 1), cap)
    torch.cuda.synchronize()
    assert_close(host(out), ref, "decode step")


def test_graph_replay_matches_eager(ema, ora):
    """The decode step (pre-attention + decode) captured in a HIP graph: every
    replay, with eager work and synchronisation in between, equals the eager result."""
    import torch

    B, Hq, Hkv, D, cap = 4, 16, 8, 128, 1024
    off = np.array([100, 1023, 0, 512], np.int32)
    qkv = dev(ora.normal_bf16((B, 1, (Hq + 2 * Hkv) * D), seed=500))
    qw = dev(ora.normal_bf16(D, seed=501, mean=1.0, std=0.02))
    kw = dev(ora.normal_bf16(D, seed=502, mean=1.0, std=0.02))
    kc = ora.normal_bf16((B, Hkv, cap, D), seed=503)
    vc = ora.normal_bf16((B, Hkv, cap, D), seed=504)
    cache = make_cache(ema, kc, vc)
    off_d, len_d = dev(off), dev(off + 1)
    q = torch.empty((B, Hq, 1, D), dtype=torch.bfloat16, device="cuda")
    out = torch.empty((B, Hq * D), dtype=torch.bfloat16, device="cuda")
    ws = ema.decode_workspace(B, Hq, Hkv, D, cap)

    def step():
        ema.pre_attention(qkv, qw, kw, 1e-6, 1e6, off_d, Hq, cache, q_out=q)
        ema.decode_attention(q, cache, len_d, cap, out=out, workspace=ws)

    step()
    torch.cuda.synchronize()
    eager = host(out).copy()
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
        step()  # eager work between replays
        torch.cuda.synchronize()


# ------------------------------------------------------------ fused step
def _fused_case(ema, ora, B, Hq, Hkv, D, cap, off, seed, flags=0):
    import torch

    qkv = ora.normal_bf16((B, (Hq + 2 * Hkv) * D), seed=seed)
    qw = ora.normal_bf16(D, seed=seed + 1, mean=1.0, std=0.02)
    kw = ora.normal_bf16(D, seed=seed + 2, mean=1.0, std=0.02)
    kc = ora.normal_bf16((B, Hkv, cap, D), seed=seed + 3)
    vc = ora.normal_bf16((B, Hkv, cap, D), seed=seed + 4)
    off = np.asarray(off, np.int32)
    # oracle: write (where it fits), then attend over clamp(off + 1)
    kr, vr = kc.copy(), vc.copy()
    q_ref = np.zeros((B, Hq, 1, D), np.uint16)
    for bb in range(B):
        if 0 <= off[bb] < cap:
            kb, vb = kr[bb:bb + 1].copy(), vr[bb:bb + 1].copy()
            q_ref[bb:bb + 1] = ora.pre_attention(qkv[bb:bb + 1, None].copy(), qw, kw, 1e-6, 1e6, off[bb:bb + 1],
                                                 Hq, Hkv, kb, vb, flags=flags)
            kr[bb], vr[bb] = kb[0], vb[0]
        else:  # nothing is written; q is still normalised and rotated at the offset
            x = qkv[bb, :Hq * D].reshape(Hq, D).copy()
            if not flags & (1 | 8):
                x = ora.rms_norm(x, qw, 1e-6)
            if not flags & 2:
                x = ora.rope(x, np.full(Hq, off[bb], np.int32), 1e6)
            q_ref[bb] = x.reshape(Hq, 1, D)
    L = np.clip(off + 1, 0, cap).astype(np.int32)
    ref = ora.sdpa(q_ref, kr, vr, L, scale_of(D), False)
    cache = make_cache(ema, kc, vc)
    out = ema.decode_step(dev(qkv), dev(qw), dev(kw), 1e-6, 1e6, dev(off), Hq, cache, cap, flags=flags)
    torch.cuda.synchronize()
    return host(out), ref, host(cache.k), host(cache.v), kr, vr, kc


@pytest.mark.parametrize("flags", [0, 1, 2, 3, 8, 16, 18])
def test_decode_step_fused_small(ema, ora, flags):
    B, Hq, Hkv, D, cap = 6, 16, 4, 128, 200
    off = [0, 31, 32, 100, 199, 63]
    say(f"fused decode step flags={flags} offsets={off}")
    got, ref, kg, vg, kr, vr, _ = _fused_case(ema, ora, B, Hq, Hkv, D, cap, off, seed=600 + flags, flags=flags)
    assert np.array_equal(vg, vr), "V rows: bit copy at the offset, untouched elsewhere"
    assert_close(kg, kr, "fused k cache")
    assert_close(got, ref, "fused decode step")


def test_decode_step_fused_batch_above_64(ema, ora):
    """80 sequences (the workgroup-wide length table), offsets from 0 to past the capacity."""
    B, Hq, Hkv, D, cap = 80, 8, 2, 128, 96
    off = np.random.default_rng(630).integers(0, cap, size=B).astype(np.int32)
    off[:4] = [0, cap - 1, cap, cap + 7]
    say(f"fused decode step B={B} cap={cap}")
    got, ref, kg, vg, kr, vr, _ = _fused_case(ema, ora, B, Hq, Hkv, D, cap, off, seed=630)
    assert np.array_equal(vg, vr)
    assert_close(kg, kr, "fused k cache, B 80")
    assert_close(got, ref, "fused decode step, B 80")


def test_decode_step_fused_qwen3_14b_heads(ema, ora):
    """40 query / 8 kv heads (G = 5, Qwen3-14B): the zero-padded query columns of the QK
    operand, the fused norm/RoPE of five heads per kv head, ragged offsets."""
    B, Hq, Hkv, D, cap = 4, 40, 8, 128, 384
    off = [0, 131, 383, 257]
    say(f"fused decode step 40q/8kv offsets={off}")
    got, ref, kg, vg, kr, vr, _ = _fused_case(ema, ora, B, Hq, Hkv, D, cap, off, seed=640)
    assert np.array_equal(vg, vr)
    assert_close(kg, kr, "fused k cache, 40q/8kv")
    assert_close(got, ref, "fused decode step, 40q/8kv")


def test_prefill_qwen3_14b_heads_paired(ema, ora):
    """40 query / 8 kv heads (G = 5) over 2048 tokens: 640 query-block items, so the launch
    pairs blocks; heads of the first and the last kv group, every row."""
    say("prefill T=2048 40q/8kv causal (paired), heads 0-4 and 35-39")
    got, ref = _prefill_case(ema, ora, 1, 40, 8, 128, 2048, 2048, [0], True, False, seed=320,
                             heads=list(range(5)) + list(range(35, 40)))
    assert_close(got, ref, "prefill 2k 40q")


def test_decode_step_fused_out_of_capacity(ema, ora):
    """An offset at or past the capacity writes nothing and attends the (stale) full cache."""
    B, Hq, Hkv, D, cap = 3, 8, 2, 128, 64
    got, ref, kg, vg, kr, vr, kc = _fused_case(ema, ora, B, Hq, Hkv, D, cap, [64, 10, 200], seed=620, flags=3)
    assert np.array_equal(kg[0], kc[0]) and np.array_equal(kg[2], kc[2])
    assert_close(got, ref, "fused out of capacity")


@pytest.mark.parametrize("flags", [1, 3, 8, 16])
def test_decode_step_fused_null_norm_weights(ema, ora, flags):
    """With EMA_PRE_NO_NORM the norm weights may be null (they are never read): the result
    equals the call that passes (unused) weights, bit for bit."""
    import torch

    B, Hq, Hkv, D, cap = 4, 16, 4, 128, 256
    off = np.array([0, 100, 255, 300], np.int32)
    qkv = dev(ora.normal_bf16((B, (Hq + 2 * Hkv) * D), seed=660))
    w = dev(ora.normal_bf16(D, seed=661, mean=1.0, std=0.02))
    kc = ora.normal_bf16((B, Hkv, cap, D), seed=662)
    vc = ora.normal_bf16((B, Hkv, cap, D), seed=663)
    c1, c2 = make_cache(ema, kc, vc), make_cache(ema, kc, vc)
    o1 = ema.decode_step(qkv, None if flags & (1 | 8) else w, None if flags & (1 | 16) else w, 1e-6, 1e6, dev(off),
                         Hq, c1, cap, flags=flags)
    o2 = ema.decode_step(qkv, w, w, 1e-6, 1e6, dev(off), Hq, c2, cap, flags=flags)
    torch.cuda.synchronize()
    assert np.array_equal(host(o1), host(o2)) and np.array_equal(host(c1.k), host(c2.k))


def test_decode_step_fused_matches_unfused_pair(ema, ora):
    """Fused step == ema_pre_attention(T=1) + ema_decode_attention on the same inputs."""
    import torch

    B, Hq, Hkv, D, cap = 8, 32, 8, 128, 4096
    rng = np.random.default_rng(9)
    off = rng.integers(0, cap, size=B).astype(np.int32)
    qkv = ora.normal_bf16((B, (Hq + 2 * Hkv) * D), seed=630)
    qw = ora.normal_bf16(D, seed=631, mean=1.0, std=0.02)
    kw = ora.normal_bf16(D, seed=632, mean=1.0, std=0.02)
    kc = ora.normal_bf16((B, Hkv, cap, D), seed=633)
    vc = ora.normal_bf16((B, Hkv, cap, D), seed=634)
    c1, c2 = make_cache(ema, kc, vc), make_cache(ema, kc, vc)
    fused = ema.decode_step(dev(qkv), dev(qw), dev(kw), 1e-6, 1e6, dev(off), Hq, c1, cap)
    q = ema.pre_attention(dev(qkv.reshape(B, 1, -1)), dev(qw), dev(kw), 1e-6, 1e6, dev(off), Hq, c2)
    pair = ema.decode_attention(q, c2, dev(off + 1), cap)
    torch.cuda.synchronize()
    assert np.array_equal(host(c1.v), host(c2.v))
    assert_close(host(c1.k), host(c2.k), "k cache fused vs pair", max_abs=2e-2, mean_abs=1e-5)
    assert_close(host(fused), host(pair), "fused vs pair", max_abs=1e-2, mean_abs=1e-4)


def test_decode_step_fused_qwen3_8b_batched(ema, ora):
    """The benchmark step: batch 32, 32q/8kv, cap 8192, lengths U[512, 8192]."""
    L = np.random.default_rng(1234).integers(512, 8193, size=32)
    say("fused decode step B32 32q/8kv cap 8192")
    got, ref, kg, vg, kr, vr, _ = _fused_case(ema, ora, 32, 32, 8, 128, 8192, L - 1, seed=640)
    assert np.array_equal(vg, vr)
    assert_close(got, ref, "fused 8B batched step")
