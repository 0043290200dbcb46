"""ema_decode_step_noalloc (the decode step over the library's static per-device scratch)
against ema_decode_step with a caller workspace, through the C ABI: two calls in a row, the
second with a smaller shape, so the second call runs over scratch that still holds the
first call's split state. Same kernels, same split: outputs and cache writes are expected
bit-identical; the small call is also checked against the oracle."""
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


def _pair(ema, ora, B, Hq, Hkv, cap, off, seed):
    import torch

    D = 128
    qkv = dev(ora.normal_bf16((B, (Hq + 2 * Hkv) * D), seed=seed))
    qw = dev(ora.normal_bf16(D, seed=seed + 1, mean=1.0, std=0.02))
    kw = dev(ora.normal_bf16(D, seed=seed + 2, mean=1.0, std=0.02))
    kc = ora.normal_bf16((B, Hkv, cap, D), seed=seed + 3)
    vc = ora.normal_bf16((B, Hkv, cap, D), seed=seed + 4)
    offd = dev(np.asarray(off, np.int32))
    max_len = int(np.clip(np.asarray(off) + 1, 0, cap).max())
    c_ws = ema.StaticCache(B, Hkv, cap, D, k=dev(kc), v=dev(vc))
    c_na = ema.StaticCache(B, Hkv, cap, D, k=dev(kc), v=dev(vc))
    out_ws = ema.decode_step(qkv, qw, kw, 1e-6, 1e6, offd, Hq, c_ws, max_len)
    out_na = torch.empty((B, Hq * D), dtype=torch.bfloat16, device="cuda")
    ema.decode_step_noalloc(qkv, qw, kw, 1e-6, 1e6, offd, Hq, c_na, max_len, out_na)
    torch.cuda.synchronize()
    assert np.array_equal(host(out_na), host(out_ws)), "noalloc step differs from the workspace step"
    assert np.array_equal(host(c_na.k), host(c_ws.k)) and np.array_equal(host(c_na.v), host(c_ws.v))
    return host(out_na), kc, vc


def test_noalloc_step_matches_workspace_step_twice(ema, ora):
    # first call: the batch-32 Qwen3-8B decode shape (lengths U[512, 8192])
    L = np.random.default_rng(1234).integers(512, 8193, size=32)
    say("noalloc step: B32 32q/8kv cap 8192")
    _pair(ema, ora, 32, 32, 8, 8192, L - 1, seed=900)
    # second call, smaller: the scratch still holds the first call's partial states
    say("noalloc step: B3 16q/4kv cap 640 (after the larger call)")
    off = np.array([0, 300, 639], np.int32)
    got, kc, vc = _pair(ema, ora, 3, 16, 4, 640, off, seed=910)
    Hq, Hkv, D = 16, 4, 128
    qkv = ora.normal_bf16((3, (Hq + 2 * Hkv) * D), seed=910)
    qw = ora.normal_bf16(D, seed=911, mean=1.0, std=0.02)
    kw = ora.normal_bf16(D, seed=912, mean=1.0, std=0.02)
    kr, vr = kc.copy(), vc.copy()
    q_ref = ora.pre_attention(qkv[:, None].copy(), qw, kw, 1e-6, 1e6, off, Hq, Hkv, kr, vr)
    ref = ora.sdpa(q_ref, kr, vr, off + 1, scale_of(D), False)
    assert_close(got, ref, "noalloc step vs oracle")
