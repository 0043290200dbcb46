"""GPU parity of the affine quantized matmul (ema_quantized_matmul, MLX quantized_matmul
with transpose=true as called by crates/ops/src/quant.rs:57-76) against the oracle's f64
restatement (oracle.qmatmul), through the C ABI.

Bars. For up to 32 rows of x the kernels multiply exactly and accumulate in f32, so every
output is within one rounding of the exact sum: |y - ref| <= 2^-8 |ref| (bf16; 2^-10 for
f16) plus 4e-5 * sum_k |x_k w_k| for the f32 accumulation. For more rows (K a multiple of
64) the weights are dequantised into the activation type first, as MLX's qmm kernels do
(oracle.dequantize_act), and the same bar holds against x times those weights; against the
exact sum they add at most half an ulp of the type per weight (2^-8 sum |x w| for bf16;
2^-11 for f16, plus 2^-25 sum |x| below f16's normal range); at the Qwen3-8B decode shape also the
bf16 bar of the other parity tests (max-abs 2e-2, mean-abs 2e-3). Separate q, k and v
calls into one q|k|v row (ldy > N) and the fused call are each within one rounding of the
oracle, so within two of each other: the property the reference checks at 1e-3
(crates/serve/tests/forward_separate.rs:80-91); repeated calls are bit-identical.
"""
import numpy as np
import pytest

from gpu_util import MAX_ABS, MEAN_ABS, say

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ema():
    import torch

    if not torch.cuda.is_available():
        pytest.fail("GPU tests need a ROCm GPU")
    import ema_attn

    ema_attn.lib()
    return ema_attn


def make(ora, seed, M, N, K, gs, bits, dtype="bf16", wstd=0.02):
    """Host inputs: x [M, K] (activation values as f32), packed w, scales/biases as f32
    values of the activation type, and the matching device tensors."""
    import torch

    td = torch.bfloat16 if dtype == "bf16" else torch.float16
    rng = np.random.default_rng(seed)
    x = torch.from_numpy(rng.standard_normal((M, K)).astype(np.float32)).to(td)
    w = (rng.standard_normal((N, K)) * wstd).astype(np.float32)
    wq, sb, bb = ora.minmax_quantize(w, gs, bits)
    s = torch.from_numpy(ora.f32_from_bf16(sb)).to(td)  # bf16 values, exact in f16 at this range
    b = torch.from_numpy(ora.f32_from_bf16(bb)).to(td)
    hx, hs, hb = x.float().numpy(), s.float().numpy(), b.float().numpy()
    d = (x.cuda(), torch.from_numpy(wq.view(np.int32)).cuda(), s.cuda(), b.cuda())
    return d, (hx, wq, hs, hb)


def dq_path(M, K):
    """Whether ema_quantized_matmul takes the dequantising GEMM (more than 32 rows, K a
    multiple of its 64-wide chunks)."""
    return M > 32 and K % 64 == 0


def check(ora, y, h, gs, bits, what, dtype="bf16", bar=False):
    hx, wq, hs, hb = h
    W = ora.dequantize(wq, hs, hb, gs, bits)
    mag = np.abs(hx).astype(np.float64) @ np.abs(W).T
    if dq_path(*hx.shape):
        Wt = ora.dequantize_act(wq, hs, hb, gs, bits, dtype).astype(np.float64)
        ref = hx.astype(np.float64) @ Wt.T
        exact = ora.qmatmul(hx, wq, hs, hb, gs, bits)
        half_ulp, floor = (2.0**-8, 0.0) if dtype == "bf16" else (2.0**-11, 2.0**-25)
        xs = np.abs(hx).astype(np.float64).sum(axis=1, keepdims=True)
        assert np.all(np.abs(ref - exact) <= (half_ulp * mag + floor * xs) * (1 + 1e-6)), f"{what}: dequantised weights"
    else:
        ref = ora.qmatmul(hx, wq, hs, hb, gs, bits)
    got = y.float().cpu().numpy().astype(np.float64)
    assert got.shape == ref.shape and np.all(np.isfinite(got)), what
    rel = 2.0**-8 if dtype == "bf16" else 2.0**-10
    err = np.abs(got - ref)
    over = err - (rel * np.abs(ref) + 4e-5 * mag)
    say(f"  {what}: max_abs={err.max():.3e} mean_abs={err.mean():.3e} worst margin={over.max():.3e} "
        f"(|y| max {np.abs(ref).max():.2f})")
    assert np.all(over <= 0), f"{what}: {int((over > 0).sum())} outputs beyond one rounding"
    if bar:
        assert err.max() <= MAX_ABS and err.mean() <= MEAN_ABS, what


@pytest.mark.parametrize("dtype", ["bf16", "f16"])
@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("gs", [32, 64, 128])
def test_qmatmul_matches_oracle(ema, ora, dtype, bits, gs):
    for M, N, K in ((1, 96, 512), (5, 100, 1024), (16, 48, 256), (17, 64, 768), (32, 80, 2048)):
        say(f"qmatmul {dtype} bits={bits} gs={gs} M={M} N={N} K={K}")
        d, h = make(ora, M * 7 + N + K + gs + bits, M, N, K, gs, bits, dtype)
        y = ema.quantized_matmul(*d, group_size=gs, bits=bits)
        check(ora, y, h, gs, bits, f"M={M} N={N} K={K}", dtype)


@pytest.mark.parametrize("M,N,bits", [(1, 6144, 4), (8, 6144, 4), (32, 6144, 4), (32, 4096, 4), (1, 6144, 8),
                                      (16, 6144, 8), (32, 6144, 8), (32, 4096, 8)])
def test_qmatmul_qwen3_8b_qkv_decode_shape(ema, ora, M, N, bits):
    # x [M, 4096] -> q|k|v [M, 6144] or o_proj [M, 4096], group 64: the one-row kernel (M = 1)
    # and the staged kernel with one or two column tiles (chosen by the tile count; 8-bit
    # weights of 32 rows take most of the LDS)
    K, gs = 4096, 64
    say(f"qmatmul Qwen3-8B decode shape M={M} N={N} K={K} bits={bits}")
    d, h = make(ora, 1, M, N, K, gs, bits)
    y = ema.quantized_matmul(*d, group_size=gs, bits=bits)
    check(ora, y, h, gs, bits, "8B qkv", bar=True)


@pytest.mark.parametrize("M,N,bits", [(1, 7168, 4), (32, 7168, 4), (32, 5120, 4), (1, 5120, 8), (32, 7168, 8)])
def test_qmatmul_qwen3_14b_decode_shape(ema, ora, M, N, bits):
    # Qwen3-14B: hidden 5120, 40 query / 8 kv heads of 128, so x [M, 5120] -> q|k|v
    # [M, 7168] or o_proj [M, 5120], group 64 (K / 64 = 80 groups per row)
    K, gs = 5120, 64
    say(f"qmatmul Qwen3-14B decode shape M={M} N={N} K={K} bits={bits}")
    d, h = make(ora, 2, M, N, K, gs, bits)
    y = ema.quantized_matmul(*d, group_size=gs, bits=bits)
    check(ora, y, h, gs, bits, "14B qkv", bar=True)


@pytest.mark.parametrize("dtype", ["bf16", "f16"])
def test_qmatmul_one_row_8bit_group_128_many_rows(ema, ora, dtype):
    # one row of x over 6144 weight rows at 8 bits, group 128: enough rows that the one-row
    # kernel gives each lane its most rows (two for this format, whose 32-dword groups
    # would not fit four to a lane)
    M, N, K, gs, bits = 1, 6144, 2048, 128, 8
    say(f"qmatmul one-row {dtype} bits={bits} gs={gs} N={N} K={K}")
    d, h = make(ora, 11, M, N, K, gs, bits, dtype)
    y = ema.quantized_matmul(*d, group_size=gs, bits=bits)
    check(ora, y, h, gs, bits, "one row, 8-bit group 128", dtype)


@pytest.mark.parametrize("M,gs,dtype", [(20, 128, "bf16"), (12, 64, "f16")])
def test_qmatmul_8bit_wide_rows_x_in_registers(ema, ora, M, gs, dtype):
    # 8-bit weights of two 16-row column tiles fill most of the LDS, so x streams through
    # registers (qmvx_kernel); ragged rows of x
    N, K, bits = 6144, 4096, 8
    say(f"qmatmul 8-bit M={M} N={N} K={K} gs={gs} {dtype}")
    d, h = make(ora, 60 + M, M, N, K, gs, bits, dtype)
    y = ema.quantized_matmul(*d, group_size=gs, bits=bits)
    check(ora, y, h, gs, bits, f"M={M}", dtype)


@pytest.mark.parametrize("M,N,K,gs,bits,dtype", [
    (64, 256, 1024, 64, 4, "bf16"),     # tiled GEMM: one 128-row tile, several column tiles
    (300, 256, 1024, 64, 4, "bf16"),    # ragged last row tile
    (130, 100, 2048, 128, 4, "bf16"),   # group 128: 128-wide chunks; ragged columns
    (500, 70, 1024, 128, 8, "f16"),
    (96, 80, 512, 32, 8, "bf16"),
    (2048, 256, 2048, 64, 4, "bf16"),   # a prefill chunk's rows
    (40, 48, 320, 32, 4, "bf16"),       # K / gs = 10
    (70, 64, 320, 32, 8, "f16"),
    (40, 48, 288, 32, 4, "bf16"),       # K not a multiple of 64: the streaming kernel
    (70, 64, 288, 32, 8, "f16"),
    (257, 129, 512, 32, 4, "f16"),      # ragged tiles in both directions
])
def test_qmatmul_prefill_rows(ema, ora, M, N, K, gs, bits, dtype):
    say(f"qmatmul prefill rows M={M} N={N} K={K} gs={gs} bits={bits} {dtype}")
    d, h = make(ora, M + N, M, N, K, gs, bits, dtype)
    y = ema.quantized_matmul(*d, group_size=gs, bits=bits)
    check(ora, y, h, gs, bits, f"M={M}", dtype)


@pytest.mark.parametrize("M", [1, 32, 256])
def test_qmatmul_graph_replay(ema, ora, M):
    # captured in a HIP graph and replayed several times with eager work between the
    # replays: every replay equals the eager call (no memsets or host state in the call)
    import torch

    N, K, gs, bits = 192, 1024, 64, 4
    say(f"qmatmul graph replay M={M}")
    d, _ = make(ora, 5 + M, M, N, K, gs, bits)
    y_eager = ema.quantized_matmul(*d, group_size=gs, bits=bits)
    torch.cuda.synchronize()
    y = torch.empty_like(y_eager)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            ema.quantized_matmul(*d, group_size=gs, bits=bits, out=y, stream=s)
    torch.cuda.synchronize()
    for i in range(3):
        y.fill_(float(i + 3))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(y.view(torch.int16), y_eager.view(torch.int16)), f"replay {i}"


def test_qmatmul_separate_pieces_equal_fused(ema, ora):
    # run_qkv's separate branch (projection.rs:119-125) writing its three pieces straight
    # into one q|k|v row (ldy = 6144): columns of other pieces untouched, every piece and the
    # fused call within one rounding of the oracle, hence of each other (the reference checks
    # max-abs 1e-3, forward_separate.rs:80-91; the 4096-column piece and the fused call may be
    # tiled differently, which reorders the f32 sums)
    import torch

    M, K, gs, bits = 8, 4096, 64, 4
    sizes = (4096, 1024, 1024)
    say(f"qmatmul separate vs fused M={M} pieces={sizes}")
    made = [make(ora, 50 + i, M, n, K, gs, bits) for i, n in enumerate(sizes)]
    parts = [m[0] for m in made]
    x = parts[0][0]
    fused = ema.quantized_matmul(x, torch.cat([p[1] for p in parts]), torch.cat([p[2] for p in parts]),
                                 torch.cat([p[3] for p in parts]), group_size=gs, bits=bits)
    qkv = torch.full((M, sum(sizes)), 7.0, dtype=torch.bfloat16, device="cuda")
    col = 0
    for (_, w, s, b), n in zip(parts, sizes):
        if col == 0:
            assert torch.all(qkv[:, n:] == 7.0)
        ema.quantized_matmul(x, w, s, b, group_size=gs, bits=bits, out=qkv[:, col:col + n])
        if col + n < qkv.shape[1]:
            assert torch.all(qkv[:, col + n:] == 7.0), "wrote past its piece"
        col += n
    torch.cuda.synchronize()
    col = 0
    for (_, h), n in zip(made, sizes):
        h = (made[0][1][0],) + h[1:]  # every piece reads the same x
        check(ora, qkv[:, col:col + n], h, gs, bits, f"piece at column {col}")
        col += n
    hx = made[0][1][0]
    fused_h = (hx, np.concatenate([m[1][1] for m in made]), np.concatenate([m[1][2] for m in made]),
               np.concatenate([m[1][3] for m in made]))
    check(ora, fused, fused_h, gs, bits, "fused")
    # the two results are each within one rounding (plus the f32 accumulation allowance)
    # of the exact product, so within the sum of both allowances of each other
    a, b = qkv.float().cpu().numpy().astype(np.float64), fused.float().cpu().numpy().astype(np.float64)
    W = ora.dequantize(fused_h[1], fused_h[2], fused_h[3], gs, bits)
    mag = np.abs(hx).astype(np.float64) @ np.abs(W).T
    assert np.all(np.abs(a - b) <= 2.0**-7 * np.maximum(np.abs(a), np.abs(b)) + 8e-5 * mag)
    say(f"  separate vs fused: {int((a != b).sum())} of {a.size} outputs differ, max {np.abs(a - b).max():.3e}")


def test_qmatmul_strided_rows_and_determinism(ema, ora):
    import torch

    M, N, K, gs, bits = 9, 128, 1024, 64, 8
    say("qmatmul strided x rows, repeat determinism")
    d, h = make(ora, 3, M, N, K, gs, bits)
    x, w, s, b = d
    wide = torch.zeros((M, K + 64), dtype=x.dtype, device="cuda")
    wide[:, :K] = x
    y1 = ema.quantized_matmul(wide[:, :K], w, s, b, group_size=gs, bits=bits)
    y2 = ema.quantized_matmul(x, w, s, b, group_size=gs, bits=bits)
    torch.cuda.synchronize()
    assert torch.equal(y1.view(torch.int16), y2.view(torch.int16))
    check(ora, y1, h, gs, bits, "strided")


@pytest.mark.parametrize("M", [4, 64])
def test_qmatmul_extreme_fields_and_groups(ema, ora, M):
    # all-zero and all-max fields, zero and negative scales, large biases: the C + q
    # offset and the bias term cancel exactly (4 rows); dequantised into bf16 (64 rows)
    import torch

    N, K, gs = 32, 512, 64
    for bits in (4, 8):
        say(f"qmatmul extreme fields bits={bits} M={M}")
        rng = np.random.default_rng(bits)
        q = np.where(rng.random((N, K)) < 0.5, 0, (1 << bits) - 1).astype(np.uint32)
        wq = ora.pack_bits(q, bits)
        s = rng.choice([0.0, -0.015625, 0.03125, 1.0], (N, K // gs)).astype(np.float32)
        b = rng.choice([0.0, -3.0, 2.5, 100.0], (N, K // gs)).astype(np.float32)
        x = torch.from_numpy(rng.standard_normal((M, K)).astype(np.float32)).to(torch.bfloat16)
        args = (x.cuda(), torch.from_numpy(wq.view(np.int32)).cuda(), torch.from_numpy(s).to(torch.bfloat16).cuda(),
                torch.from_numpy(b).to(torch.bfloat16).cuda())
        y = ema.quantized_matmul(*args, group_size=gs, bits=bits)
        check(ora, y, (x.float().numpy(), wq, s, b), gs, bits, f"extreme bits={bits}")
