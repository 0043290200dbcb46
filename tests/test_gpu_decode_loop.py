"""GPU parity of the batched decode loop: consecutive fused decode steps whose offsets
advance on the device (EMA_STEP_ADVANCE), the reference's static decode loop
(crates/serve/src/decode_compiled.rs:14-65: write the token's k/v at the offset, attend
offset + 1 positions, then `self.offset += 1` at :49; generate.rs:88-94 runs it once per
token).

The oracle runs the same loop step by step on the host: pre-attention into the cache at
each sequence's offset (where it fits), SDPA over clamp(offset + 1), then offset + 1 for
every sequence whose row was written. Tolerance as in the other parity tests (max-abs
2e-2, mean-abs 2e-3 against the f64 oracle); V rows bit-exact; offsets exact.
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


def oracle_loop(ora, qkvs, qw, kw, kc, vc, off, Hq, Hkv, D, cap):
    """Steps of the static decode loop on the host. Returns per-step outputs, the final
    caches and the final offsets."""
    kr, vr, off = kc.copy(), vc.copy(), np.asarray(off, np.int32).copy()
    B = kr.shape[0]
    outs = []
    for qkv in qkvs:
        q = np.zeros((B, Hq, 1, D), np.uint16)
        wrote = np.zeros(B, bool)
        for b in range(B):
            if 0 <= off[b] < cap:
                kb, vb = kr[b:b + 1].copy(), vr[b:b + 1].copy()
                q[b:b + 1] = ora.pre_attention(qkv[b:b + 1, None].copy(), qw, kw, 1e-6, 1e6, off[b:b + 1], Hq, Hkv,
                                               kb, vb)
                kr[b], vr[b] = kb[0], vb[0]
                wrote[b] = True
            else:  # nothing is written; q is still normalised and rotated at the offset
                x = ora.rms_norm(qkv[b, :Hq * D].reshape(Hq, D).copy(), qw, 1e-6)
                q[b] = ora.rope(x, np.full(Hq, off[b], np.int32), 1e6).reshape(Hq, 1, D)
        L = np.clip(off + 1, 0, cap).astype(np.int32)
        outs.append(ora.sdpa(q, kr, vr, L, scale_of(D), False))
        off = np.where(wrote, off + 1, off).astype(np.int32)
    return outs, kr, vr, off


def test_graph_of_eight_steps_b32_ragged(ema, ora):
    """Batch 32, 32q/8kv, ragged offsets (some reach the capacity mid-loop, one starts
    there): eight steps captured in one HIP graph and replayed once equal the oracle's
    loop step by step, and the offsets end where the oracle's do."""
    import torch

    B, Hq, Hkv, D, cap, n = 32, 32, 8, 128, 1024, 8
    rng = np.random.default_rng(77)
    off = rng.integers(0, cap - n, size=B).astype(np.int32)
    off[:6] = [0, 1, cap - 3, cap - 1, cap, 31]
    say(f"decode loop graph: B={B} {Hq}q/{Hkv}kv cap={cap} steps={n}")
    qkvs = [ora.normal_bf16((B, (Hq + 2 * Hkv) * D), seed=900 + i) for i in range(n)]
    qw = ora.normal_bf16(D, seed=950, mean=1.0, std=0.02)
    kw = ora.normal_bf16(D, seed=951, mean=1.0, std=0.02)
    kc = ora.normal_bf16((B, Hkv, cap, D), seed=952)
    vc = ora.normal_bf16((B, Hkv, cap, D), seed=953)
    refs, kr, vr, off_ref = oracle_loop(ora, qkvs, qw, kw, kc, vc, off, Hq, Hkv, D, cap)

    cache = ema.StaticCache(B, Hkv, cap, D, k=dev(kc), v=dev(vc))
    qkv_d = dev(np.stack(qkvs))
    qw_d, kw_d, off_d = dev(qw), dev(kw), dev(off)
    outs = torch.zeros((n, B, Hq * D), dtype=torch.bfloat16, device="cuda")
    ws = ema.decode_workspace(B, Hq, Hkv, D, cap)
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            for i in range(n):
                ema.decode_step(qkv_d[i], qw_d, kw_d, 1e-6, 1e6, off_d, Hq, cache, cap, out=outs[i], workspace=ws,
                                flags=ema.EMA_STEP_ADVANCE)
    torch.cuda.synchronize()
    # capture ran nothing: the cache and offsets are still the initial ones
    assert np.array_equal(host(off_d), off)
    g.replay()
    torch.cuda.synchronize()
    got = host(outs)
    for i in range(n):
        assert_close(got[i], refs[i], f"step {i}")
    assert np.array_equal(host(off_d), off_ref), "offsets after the loop"
    assert np.array_equal(host(cache.v), vr), "V rows: bit copies at each step's offset"
    assert_close(host(cache.k), kr, "k cache after the loop")


@pytest.mark.parametrize("noalloc", [False, True])
def test_batch1_loop_single_worker(ema, ora, noalloc):
    """Batch 1 with a short cache runs one decode workgroup (no split to merge): the
    offset still advances, up to the capacity and not past it."""
    import torch

    B, Hq, Hkv, D, cap, n = 1, 8, 2, 128, 64, 8
    off = np.array([59], np.int32)
    say(f"decode loop batch 1 cap={cap} from offset {off[0]} noalloc={noalloc}")
    qkvs = [ora.normal_bf16((B, (Hq + 2 * Hkv) * D), seed=960 + i) for i in range(n)]
    qw = ora.normal_bf16(D, seed=970, mean=1.0, std=0.02)
    kw = ora.normal_bf16(D, seed=971, mean=1.0, std=0.02)
    kc = ora.normal_bf16((B, Hkv, cap, D), seed=972)
    vc = ora.normal_bf16((B, Hkv, cap, D), seed=973)
    refs, kr, vr, off_ref = oracle_loop(ora, qkvs, qw, kw, kc, vc, off, Hq, Hkv, D, cap)
    assert off_ref[0] == cap
    cache = ema.StaticCache(B, Hkv, cap, D, k=dev(kc), v=dev(vc))
    off_d, qw_d, kw_d = dev(off), dev(qw), dev(kw)
    out = torch.empty((B, Hq * D), dtype=torch.bfloat16, device="cuda")
    for i in range(n):
        if noalloc:
            ema.decode_step_noalloc(dev(qkvs[i]), qw_d, kw_d, 1e-6, 1e6, off_d, Hq, cache, cap, out,
                                    flags=ema.EMA_STEP_ADVANCE)
        else:
            ema.decode_step(dev(qkvs[i]), qw_d, kw_d, 1e-6, 1e6, off_d, Hq, cache, cap, out=out,
                            flags=ema.EMA_STEP_ADVANCE)
        torch.cuda.synchronize()
        assert_close(host(out), refs[i], f"step {i}")
    assert np.array_equal(host(off_d), off_ref)
    assert np.array_equal(host(cache.v), vr)


def test_rotating_loop_wraps(ema, ora):
    """A rotating cache advances past its capacity: each step writes row offset % W and
    attends the last W positions, like the reference's RotatingCache fed one token per
    step (crates/kvcache/src/rotating.rs:56-122)."""
    import torch
    from test_gpu_rotating import ring_from

    B, Hq, Hkv, D, W, n = 3, 8, 2, 128, 64, 8
    off = np.array([60, 63, 200], np.int32)
    say(f"rotating decode loop W={W} offsets={off.tolist()} steps={n}")
    qkvs = [ora.normal_bf16((B, (Hq + 2 * Hkv) * D), seed=980 + i) for i in range(n)]
    qw = ora.normal_bf16(D, seed=990, mean=1.0, std=0.02)
    kw = ora.normal_bf16(D, seed=991, mean=1.0, std=0.02)
    total = int(off.max()) + n
    big_k = ora.normal_bf16((B, Hkv, total, D), seed=992)
    big_v = ora.normal_bf16((B, Hkv, total, D), seed=993)
    cache = ema.StaticCache(B, Hkv, W, D, k=dev(ring_from(ora, big_k, off, W)), v=dev(ring_from(ora, big_v, off, W)),
                            rotating=True)
    off_d, qw_d, kw_d = dev(off), dev(qw), dev(kw)
    cur = off.copy()
    for i in range(n):
        q = np.zeros((B, Hq, 1, D), np.uint16)
        for b in range(B):
            kb, vb = big_k[b:b + 1].copy(), big_v[b:b + 1].copy()
            q[b:b + 1] = ora.pre_attention(qkvs[i][b:b + 1, None].copy(), qw, kw, 1e-6, 1e6, cur[b:b + 1], Hq, Hkv,
                                           kb, vb)
            big_k[b], big_v[b] = kb[0], vb[0]
        L = cur + 1
        ref = ora.sdpa(q, big_k, big_v, L, scale_of(D), False, kv_begin=np.maximum(L - W, 0))
        out = ema.decode_step(dev(qkvs[i]), qw_d, kw_d, 1e-6, 1e6, off_d, Hq, cache, W, flags=ema.EMA_STEP_ADVANCE)
        torch.cuda.synchronize()
        assert_close(host(out), ref, f"rotating step {i}")
        cur = cur + 1
    assert np.array_equal(host(off_d), cur)
    assert np.array_equal(host(cache.v), ring_from(ora, big_v, cur, W))


def oracle_step_inplace(ora, qkv, qw, kw, kr, vr, off, Hq, Hkv, D, cap):
    """One step of the static decode loop on the host, writing into kr / vr in place
    (views of one sequence are contiguous, so nothing is copied). Returns the output and
    which sequences wrote their row."""
    B = kr.shape[0]
    q = np.zeros((B, Hq, 1, D), np.uint16)
    wrote = np.zeros(B, bool)
    for b in range(B):
        if 0 <= off[b] < cap:
            q[b:b + 1] = ora.pre_attention(qkv[b:b + 1, None].copy(), qw, kw, 1e-6, 1e6, off[b:b + 1], Hq, Hkv,
                                           kr[b:b + 1], vr[b:b + 1])
            wrote[b] = True
        else:
            x = ora.rms_norm(qkv[b, :Hq * D].reshape(Hq, D).copy(), qw, 1e-6)
            q[b] = ora.rope(x, np.full(Hq, off[b], np.int32), 1e6).reshape(Hq, 1, D)
    L = np.clip(off + 1, 0, cap).astype(np.int32)
    return ora.sdpa(q, kr, vr, L, scale_of(D), False), wrote


def test_graph_loop_qwen3_8b_batched_shape(ema, ora):
    """The batch-32 Qwen3-8B decode shape as a loop: 32q/8kv, capacity 8192, lengths
    uniform in [512, 8192] (seed 1234, the bench's), one sequence two rows below the
    capacity (it stops there mid-loop), one at it and one twelve rows below; eight steps captured in one HIP graph with EMA_STEP_ADVANCE
    and replayed once equal the oracle's loop step by step, the offsets stop at the
    capacity, and only the written rows change."""
    import torch

    B, Hq, Hkv, D, cap, n = 32, 32, 8, 128, 8192, 8
    off = (np.random.default_rng(1234).integers(512, cap + 1, size=B) - 1).astype(np.int32)
    off[[3, 17, 29]] = [cap - 12, cap - 2, cap]
    say(f"decode loop graph at the 8B batched shape: B={B} cap={cap} steps={n} sum(L)={int((off + 1).sum())}")
    qkvs = [ora.normal_bf16((B, (Hq + 2 * Hkv) * D), seed=1900 + i) for i in range(n)]
    qw = ora.normal_bf16(D, seed=1950, mean=1.0, std=0.02)
    kw = ora.normal_bf16(D, seed=1951, mean=1.0, std=0.02)
    kc = ora.normal_bf16((B, Hkv, cap, D), seed=1952)
    vc = ora.normal_bf16((B, Hkv, cap, D), seed=1953)

    cache = ema.StaticCache(B, Hkv, cap, D, k=dev(kc), v=dev(vc))
    qkv_d = dev(np.stack(qkvs))
    qw_d, kw_d, off_d = dev(qw), dev(kw), dev(off)
    outs = torch.zeros((n, B, Hq * D), dtype=torch.bfloat16, device="cuda")
    ws = ema.decode_workspace(B, Hq, Hkv, D, cap)
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            for i in range(n):
                ema.decode_step(qkv_d[i], qw_d, kw_d, 1e-6, 1e6, off_d, Hq, cache, cap, out=outs[i], workspace=ws,
                                flags=ema.EMA_STEP_ADVANCE)
    torch.cuda.synchronize()
    g.replay()
    torch.cuda.synchronize()
    got = host(outs)
    gk, gv = host(cache.k), host(cache.v)

    kr, vr, cur = kc.copy(), vc.copy(), off.copy()
    for i in range(n):
        ref, wrote = oracle_step_inplace(ora, qkvs[i], qw, kw, kr, vr, cur, Hq, Hkv, D, cap)
        assert_close(got[i], ref, f"step {i}")
        cur = np.where(wrote, cur + 1, cur).astype(np.int32)
    assert np.array_equal(host(off_d), cur), "offsets after the loop"
    assert cur[29] == cap and cur[17] == cap and cur[3] == cap - 12 + n
    assert np.array_equal(gv, vr), "V rows: bit copies at each step's offset, the rest untouched"
    rows = np.zeros((B, cap), bool)
    for b in range(B):
        rows[b, off[b]:cur[b]] = True
    assert np.array_equal(gk[~rows[:, None, :].repeat(Hkv, 1)], kc[~rows[:, None, :].repeat(Hkv, 1)]), \
        "K rows that no step wrote are untouched"
    wk = rows[:, None, :].repeat(Hkv, 1)
    assert_close(gk[wk][None], kr[wk][None], "written K rows")


def test_two_layers_share_one_offsets_array(ema, ora):
    """Two layers whose steps share one offsets array, the reference's one model-wide
    offset (crates/serve/src/decode_compiled.rs:49): EMA_STEP_ADVANCE on the second
    layer's step only. Six tokens captured in one graph (layer 0, layer 1 per token)
    equal the oracle's loop layer by layer: both layers write their row at the same
    offset and attend the same length, and the offset moves once per token."""
    import torch

    B, Hq, Hkv, D, cap, n = 4, 16, 8, 128, 512, 6
    off = np.array([0, 17, cap - 3, 300], np.int32)
    say(f"two layers, one offsets array: B={B} cap={cap} tokens={n}")
    layers = []
    for li in range(2):
        qkvs = [ora.normal_bf16((B, (Hq + 2 * Hkv) * D), seed=2000 + 100 * li + i) for i in range(n)]
        qw = ora.normal_bf16(D, seed=2050 + 100 * li, mean=1.0, std=0.02)
        kw = ora.normal_bf16(D, seed=2051 + 100 * li, mean=1.0, std=0.02)
        kc = ora.normal_bf16((B, Hkv, cap, D), seed=2052 + 100 * li)
        vc = ora.normal_bf16((B, Hkv, cap, D), seed=2053 + 100 * li)
        layers.append(dict(qkvs=qkvs, qw=qw, kw=kw, kc=kc, vc=vc,
                           cache=ema.StaticCache(B, Hkv, cap, D, k=dev(kc), v=dev(vc)),
                           qkv_d=dev(np.stack(qkvs)), qw_d=dev(qw), kw_d=dev(kw),
                           ws=ema.decode_workspace(B, Hq, Hkv, D, cap),
                           outs=torch.zeros((n, B, Hq * D), dtype=torch.bfloat16, device="cuda")))
    off_d = dev(off)
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            for i in range(n):
                for li, ly in enumerate(layers):
                    ema.decode_step(ly["qkv_d"][i], ly["qw_d"], ly["kw_d"], 1e-6, 1e6, off_d, Hq, ly["cache"], cap,
                                    out=ly["outs"][i], workspace=ly["ws"],
                                    flags=ema.EMA_STEP_ADVANCE if li == 1 else 0)
    torch.cuda.synchronize()
    g.replay()
    torch.cuda.synchronize()

    state = [(ly["kc"].copy(), ly["vc"].copy()) for ly in layers]
    cur = off.copy()
    for i in range(n):
        wrote_all = None
        for li, ly in enumerate(layers):
            kr, vr = state[li]
            ref, wrote = oracle_step_inplace(ora, ly["qkvs"][i], ly["qw"], ly["kw"], kr, vr, cur, Hq, Hkv, D, cap)
            assert_close(host(ly["outs"][i]), ref, f"token {i} layer {li}")
            wrote_all = wrote
        cur = np.where(wrote_all, cur + 1, cur).astype(np.int32)
    assert np.array_equal(host(off_d), cur), "the shared offsets moved once per token"
    for li, ly in enumerate(layers):
        assert np.array_equal(host(ly["cache"].v), state[li][1]), f"layer {li} V rows"
