"""GPU parity of the Gated DeltaNet scan (ema_gdn_scan), through the C ABI, against the
oracle's restatement of gdn_step (crates/ops/src/gdn.rs:83-150) applied token by token
(crates/ops/src/gdn_forward.rs:173-192).

Inputs follow gdn_forward's scaling: q = rms_norm(q) / dk, k = rms_norm(k) / sqrt(dk) (so
|k| = 1), g = exp(-exp(A_log) softplus(a + dt_bias)), beta = sigmoid(b). The oracle reads
the same quantised activations (as f32) and the same f32 state, and computes in f64.

Bars: state (f32) within 2e-5 absolute + 1e-5 relative of the oracle; y within 1e-4 for
f32 activations, 2e-3 for f16, and the bf16 bar (max-abs 2e-2, mean-abs 2e-3) for bf16.
Scans of f16 / f32 activations, and bf16 scans under 32 tokens, run the token-by-token
kernel and are bit-identical to single-token calls; bf16 scans of 32 tokens or more run
the chunkwise kernel (32-token chunks on the matrix cores), held to the same bars against
the oracle and checked against the token-by-token kernel at the bench shape.
"""
import numpy as np
import pytest

from gpu_util import say

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ema():
    import torch

    if not torch.cuda.is_available():
        pytest.fail("GPU tests need a ROCm GPU")
    import ema_attn

    ema_attn.lib()
    return ema_attn


def _torch_dtype(name):
    import torch

    return {"bf16": torch.bfloat16, "f16": torch.float16, "f32": torch.float32}[name]


def make_inputs(seed, B, T, Hk, Hv, Dk, Dv, dtype):
    """Device tensors (q, k, v in dtype; g, beta, state f32) and their f32 host copies."""
    import torch

    rng = np.random.default_rng(seed)

    def rms(x):
        return x / np.sqrt((x * x).mean(axis=-1, keepdims=True) + 1e-6)

    q = rms(rng.standard_normal((B, T, Hk, Dk))) / Dk
    k = rms(rng.standard_normal((B, T, Hk, Dk))) / np.sqrt(Dk)
    v = rng.standard_normal((B, T, Hv, Dv))
    a = rng.standard_normal((B, T, Hv))
    a_log = rng.uniform(-2.0, 0.5, Hv)
    dt_bias = rng.uniform(-1.0, 1.0, Hv)
    g = np.exp(-np.exp(a_log) * np.log1p(np.exp(a + dt_bias)))
    beta = 1.0 / (1.0 + np.exp(-rng.standard_normal((B, T, Hv))))
    S0 = rng.standard_normal((B, Hv, Dv, Dk)) * 0.5
    td = _torch_dtype(dtype)
    dq, dk_, dv_ = (torch.from_numpy(x.astype(np.float32)).to(td).cuda() for x in (q, k, v))
    dg = torch.from_numpy(g.astype(np.float32)).cuda()
    db = torch.from_numpy(beta.astype(np.float32)).cuda()
    dS = torch.from_numpy(S0.astype(np.float32)).cuda()
    hq, hk, hv = (t.float().cpu().numpy() for t in (dq, dk_, dv_))
    return (dq, dk_, dv_, dg, db, dS), (hq, hk, hv, dg.cpu().numpy(), db.cpu().numpy(), dS.cpu().numpy())


def check_against_oracle(ora, y, S, host_in, dtype, what):
    hq, hk, hv, hg, hb, hS = host_in
    ry, rS = ora.gdn_scan(hq, hk, hv, hg, hb, hS.astype(np.float64))
    gS = S.cpu().numpy().astype(np.float64)
    gy = y.float().cpu().numpy().astype(np.float64)
    dS = np.abs(gS - rS)
    tolS = 2e-5 + 1e-5 * np.abs(rS)
    say(f"  {what}: state max_abs={dS.max():.3e}")
    assert np.all(np.isfinite(gS)) and np.all(dS <= tolS), f"{what}: state max_abs={dS.max()}"
    d = np.abs(gy - ry)
    say(f"  {what}: y max_abs={d.max():.3e} mean_abs={d.mean():.3e} (|y| max {np.abs(ry).max():.3f})")
    assert np.all(np.isfinite(gy))
    if dtype == "f32":
        assert d.max() <= 1e-4, what
    elif dtype == "f16":
        assert d.max() <= 2e-3, what
    else:
        assert d.max() <= 2e-2 and d.mean() <= 2e-3, what


@pytest.mark.parametrize("dtype", ["bf16", "f16", "f32"])
@pytest.mark.parametrize("Dk", [64, 128])
@pytest.mark.parametrize("T", [1, 7])
def test_gdn_scan_matches_oracle(ema, ora, dtype, Dk, T):
    B, Hk, Hv, Dv = 2, 2, 4, 32
    say(f"gdn scan dtype={dtype} B={B} T={T} Hk={Hk} Hv={Hv} Dk={Dk} Dv={Dv}")
    dev_in, host_in = make_inputs(100 + T + Dk, B, T, Hk, Hv, Dk, Dv, dtype)
    dq, dk_, dv_, dg, db, dS = dev_in
    y = ema.gdn_scan(dq, dk_, dv_, dg, db, dS)
    check_against_oracle(ora, y, dS, host_in, dtype, f"{dtype} Dk={Dk} T={T}")


@pytest.mark.parametrize("dtype", ["bf16", "f32"])
def test_gdn_scan_equals_single_token_calls(ema, dtype):
    import torch

    B, T, Hk, Hv, Dk, Dv = 2, 12, 2, 4, 128, 48
    say(f"gdn scan vs token steps dtype={dtype} T={T}")
    (dq, dk_, dv_, dg, db, dS), _ = make_inputs(7, B, T, Hk, Hv, Dk, Dv, dtype)
    S1 = dS.clone()
    y_scan = ema.gdn_scan(dq, dk_, dv_, dg, db, S1)
    S2 = dS.clone()
    ys = []
    for t in range(T):
        ys.append(ema.gdn_scan(dq[:, t:t + 1].contiguous(), dk_[:, t:t + 1].contiguous(), dv_[:, t:t + 1].contiguous(),
                               dg[:, t:t + 1].contiguous(), db[:, t:t + 1].contiguous(), S2))
    y_steps = torch.cat(ys, dim=1)
    torch.cuda.synchronize()
    assert torch.equal(S1, S2)
    assert torch.equal(y_scan.view(torch.int16) if dtype == "bf16" else y_scan,
                       y_steps.view(torch.int16) if dtype == "bf16" else y_steps)


def test_gdn_delta_rule_at_decode_shape(ema):
    # beta = 1, g = 1: after the step S k = kv + |k|^2 (v - kv), i.e. v for a unit key, for
    # every (batch, value head, row) of a batch-32 decode step with Qwen3-Next-style heads
    import torch

    B, T, Hk, Hv, Dk, Dv = 32, 1, 16, 32, 128, 128
    say(f"gdn delta rule B={B} Hk={Hk} Hv={Hv} Dk={Dk} Dv={Dv}")
    (dq, dk_, dv_, dg, db, dS), (hq, hk, hv, _, _, hS) = make_inputs(11, B, T, Hk, Hv, Dk, Dv, "f32")
    dg.fill_(1.0)
    db.fill_(1.0)
    ema.gdn_scan(dq, dk_, dv_, dg, db, dS)
    S = dS.cpu().numpy().astype(np.float64)
    kk = np.repeat(hk[:, 0].astype(np.float64), Hv // Hk, axis=1)  # [B, Hv, Dk]
    kv_old = np.einsum("bhrd,bhd->bhr", hS.astype(np.float64), kk)
    n2 = (kk * kk).sum(-1)[..., None]
    expect = kv_old + n2 * (hv[:, 0].astype(np.float64) - kv_old)
    got = np.einsum("bhrd,bhd->bhr", S, kk)
    err = np.abs(got - expect).max()
    say(f"  read-after-write max error {err:.3e}")
    assert err <= 1e-4


def test_gdn_decode_step_bench_shape_vs_oracle(ema, ora):
    B, T, Hk, Hv, Dk, Dv = 32, 1, 16, 32, 128, 128
    say(f"gdn decode step vs oracle B={B} Hk={Hk} Hv={Hv} Dk={Dk} Dv={Dv} bf16")
    dev_in, host_in = make_inputs(12, B, T, Hk, Hv, Dk, Dv, "bf16")
    dq, dk_, dv_, dg, db, dS = dev_in
    y = ema.gdn_scan(dq, dk_, dv_, dg, db, dS)
    check_against_oracle(ora, y, dS, host_in, "bf16", "decode step")


def test_gdn_long_scan_vs_oracle(ema, ora):
    # 256 tokens from a zero state (as a new sequence starts, gdn_forward.rs:166-170)
    B, T, Hk, Hv, Dk, Dv = 1, 256, 2, 4, 128, 64
    say(f"gdn long scan T={T}")
    dev_in, host_in = make_inputs(13, B, T, Hk, Hv, Dk, Dv, "f32")
    dq, dk_, dv_, dg, db, dS = dev_in
    dS.zero_()
    host_in = host_in[:5] + (np.zeros_like(host_in[5]),)
    y = ema.gdn_scan(dq, dk_, dv_, dg, db, dS)
    check_against_oracle(ora, y, dS, host_in, "f32", "long scan")


@pytest.mark.parametrize("T,Dk,Dv", [(32, 128, 64), (33, 128, 48), (64, 64, 32), (100, 128, 80), (257, 64, 128),
                                     (300, 128, 16)])
def test_gdn_chunked_scan_matches_oracle(ema, ora, T, Dk, Dv):
    # whole and partial last chunks; Dv not a multiple of the 64 rows of a workgroup
    B, Hk, Hv = 2, 2, 4
    say(f"gdn chunked scan B={B} T={T} Hk={Hk} Hv={Hv} Dk={Dk} Dv={Dv}")
    dev_in, host_in = make_inputs(200 + T + Dk + Dv, B, T, Hk, Hv, Dk, Dv, "bf16")
    dq, dk_, dv_, dg, db, dS = dev_in
    y = ema.gdn_scan(dq, dk_, dv_, dg, db, dS)
    check_against_oracle(ora, y, dS, host_in, "bf16", f"chunked T={T} Dk={Dk} Dv={Dv}")


def test_gdn_chunked_scan_gate_extremes(ema, ora):
    # g = 0 (the state is reset mid-chunk), g = 1 and beta = 0 / 1 runs, across chunk edges
    B, T, Hk, Hv, Dk, Dv = 1, 96, 1, 2, 128, 32
    say(f"gdn chunked scan gate extremes T={T}")
    dev_in, host_in = make_inputs(31, B, T, Hk, Hv, Dk, Dv, "bf16")
    dq, dk_, dv_, dg, db, dS = dev_in
    dg[:, 5] = 0.0
    dg[:, 40:70] = 1.0
    dg[:, 31, 0] = 0.0
    db[:, 10:20] = 0.0
    db[:, 60:80, 1] = 1.0
    host_in = host_in[:3] + (dg.cpu().numpy(), db.cpu().numpy(), host_in[5])
    y = ema.gdn_scan(dq, dk_, dv_, dg, db, dS)
    check_against_oracle(ora, y, dS, host_in, "bf16", "gate extremes")


def test_gdn_chunked_scan_bench_shape(ema, ora):
    # the prefill shape of a Qwen3-Next linear-attention layer: 2048 tokens, 16 key and
    # 32 value heads of 128; against the oracle, and against the token-by-token kernel
    # run over 31-token pieces
    import torch

    B, T, Hk, Hv, Dk, Dv = 1, 2048, 16, 32, 128, 128
    say(f"gdn chunked scan bench shape B={B} T={T} Hk={Hk} Hv={Hv} Dk={Dk} Dv={Dv}")
    dev_in, host_in = make_inputs(41, B, T, Hk, Hv, Dk, Dv, "bf16")
    dq, dk_, dv_, dg, db, dS = dev_in
    S_seq = dS.clone()
    y = ema.gdn_scan(dq, dk_, dv_, dg, db, dS)
    check_against_oracle(ora, y, dS, host_in, "bf16", "bench shape")
    ys = []
    for t0 in range(0, T, 31):
        sl = slice(t0, min(T, t0 + 31))
        ys.append(ema.gdn_scan(dq[:, sl].contiguous(), dk_[:, sl].contiguous(), dv_[:, sl].contiguous(),
                               dg[:, sl].contiguous(), db[:, sl].contiguous(), S_seq))
    y_seq = torch.cat(ys, dim=1)
    dS_ = (dS - S_seq).abs()
    tol = 4e-5 + 2e-5 * S_seq.abs()
    say(f"  chunked vs token-by-token: state max_abs={dS_.max().item():.3e}, "
        f"y max_abs={(y.float() - y_seq.float()).abs().max().item():.3e}")
    assert bool((dS_ <= tol).all())
    assert (y.float() - y_seq.float()).abs().max().item() <= 2e-2


# ---- WY form over a workspace (ema_gdn_scan_ws) ----

@pytest.mark.parametrize("T,Dk,Dv", [(32, 128, 64), (33, 128, 48), (64, 64, 32), (100, 128, 80), (257, 64, 128),
                                     (300, 128, 16), (200, 128, 512)])
def test_gdn_wy_scan_matches_oracle(ema, ora, T, Dk, Dv):
    B, Hk, Hv = 2, 2, 4
    say(f"gdn WY scan B={B} T={T} Hk={Hk} Hv={Hv} Dk={Dk} Dv={Dv}")
    dev_in, host_in = make_inputs(300 + T + Dk + Dv, B, T, Hk, Hv, Dk, Dv, "bf16")
    dq, dk_, dv_, dg, db, dS = dev_in
    ws = ema.gdn_workspace(B, T, Hk, Hv, Dk, Dv)
    y = ema.gdn_scan(dq, dk_, dv_, dg, db, dS, workspace=ws)
    check_against_oracle(ora, y, dS, host_in, "bf16", f"WY T={T} Dk={Dk} Dv={Dv}")


def test_gdn_wy_segments_are_bit_identical(ema):
    # a workspace of 1 or 3 chunks runs the sequence in segments, the state passing through
    # HBM between them: the same arithmetic as one segment, so the same bits
    import torch

    B, T, Hk, Hv, Dk, Dv = 1, 230, 2, 4, 128, 64
    say(f"gdn WY segments T={T}")
    (dq, dk_, dv_, dg, db, dS), _ = make_inputs(51, B, T, Hk, Hv, Dk, Dv, "bf16")
    full = ema.gdn_scan_workspace_size(B, T, Hk, Hv, Dk, Dv)
    per_chunk = full // ((T + 31) // 32)
    outs = []
    for n in (full, per_chunk, 3 * per_chunk + 100):
        S = dS.clone()
        ws = torch.empty(n, dtype=torch.uint8, device="cuda")
        y = ema.gdn_scan(dq, dk_, dv_, dg, db, S, workspace=ws)
        outs.append((y, S))
    torch.cuda.synchronize()
    for y, S in outs[1:]:
        assert torch.equal(S, outs[0][1])
        assert torch.equal(y.view(torch.int16), outs[0][0].view(torch.int16))


def test_gdn_wy_graph_replay(ema):
    # a WY scan in segments (a workspace of two chunks) and a whole one, each captured in a
    # graph and replayed with eager work between the replays: every replay gives the eager
    # call's bits
    import torch

    B, T, Hk, Hv, Dk, Dv = 1, 500, 2, 4, 128, 64
    say(f"gdn WY graph replay T={T}")
    (dq, dk_, dv_, dg, db, dS), _ = make_inputs(71, B, T, Hk, Hv, Dk, Dv, "bf16")
    full = ema.gdn_scan_workspace_size(B, T, Hk, Hv, Dk, Dv)
    per_chunk = full // ((T + 31) // 32)
    ws = ema.gdn_workspace(B, T, Hk, Hv, Dk, Dv)
    S0 = dS.clone()
    y0 = ema.gdn_scan(dq, dk_, dv_, dg, db, S0, workspace=ws)
    S1 = dS.clone()
    y1 = ema.gdn_scan(dq, dk_, dv_, dg, db, S1, workspace=torch.empty(2 * per_chunk, dtype=torch.uint8, device="cuda"))
    torch.cuda.synchronize()
    assert torch.equal(S1, S0) and torch.equal(y1.view(torch.int16), y0.view(torch.int16))
    for wsx in (ws, torch.empty(2 * per_chunk, dtype=torch.uint8, device="cuda")):
        Sg = dS.clone()
        yg = torch.empty_like(y0)
        st = torch.cuda.Stream()
        st.wait_stream(torch.cuda.current_stream())
        g = torch.cuda.CUDAGraph()
        with torch.cuda.stream(st):
            with torch.cuda.graph(g, stream=st):
                ema.gdn_scan(dq, dk_, dv_, dg, db, Sg, y=yg, workspace=wsx, stream=st)
        torch.cuda.synchronize()
        for i in range(3):
            Sg.copy_(dS)
            yg.fill_(float(i + 2))
            torch.cuda.synchronize()
            g.replay()
            torch.cuda.synchronize()
            assert torch.equal(Sg, S0), f"replay {i}: state"
            assert torch.equal(yg.view(torch.int16), y0.view(torch.int16)), f"replay {i}: y"


def test_gdn_wy_gate_extremes(ema, ora):
    B, T, Hk, Hv, Dk, Dv = 1, 96, 1, 2, 128, 32
    say(f"gdn WY gate extremes T={T}")
    dev_in, host_in = make_inputs(31, B, T, Hk, Hv, Dk, Dv, "bf16")
    dq, dk_, dv_, dg, db, dS = dev_in
    dg[:, 5] = 0.0
    dg[:, 40:70] = 1.0
    dg[:, 31, 0] = 0.0
    db[:, 10:20] = 0.0
    db[:, 60:80, 1] = 1.0
    host_in = host_in[:3] + (dg.cpu().numpy(), db.cpu().numpy(), host_in[5])
    y = ema.gdn_scan(dq, dk_, dv_, dg, db, dS, workspace=ema.gdn_workspace(B, T, Hk, Hv, Dk, Dv))
    check_against_oracle(ora, y, dS, host_in, "bf16", "WY gate extremes")


def test_gdn_wy_bench_shape(ema, ora):
    # 2048 tokens, 16 key and 32 value heads of 128: against the oracle and the one-kernel
    # chunkwise scan
    import torch

    B, T, Hk, Hv, Dk, Dv = 1, 2048, 16, 32, 128, 128
    say(f"gdn WY scan bench shape B={B} T={T} Hk={Hk} Hv={Hv} Dk={Dk} Dv={Dv}")
    dev_in, host_in = make_inputs(42, B, T, Hk, Hv, Dk, Dv, "bf16")
    dq, dk_, dv_, dg, db, dS = dev_in
    S1 = dS.clone()
    y = ema.gdn_scan(dq, dk_, dv_, dg, db, dS, workspace=ema.gdn_workspace(B, T, Hk, Hv, Dk, Dv))
    check_against_oracle(ora, y, dS, host_in, "bf16", "WY bench shape")
    y1 = ema.gdn_scan(dq, dk_, dv_, dg, db, S1)
    d = (dS - S1).abs()
    say(f"  WY vs one-kernel: state max_abs={d.max().item():.3e}, "
        f"y max_abs={(y.float() - y1.float()).abs().max().item():.3e}")
    assert bool((d <= 4e-5 + 2e-5 * S1.abs()).all())
    assert (y.float() - y1.float()).abs().max().item() <= 2e-2


@pytest.mark.parametrize("dtype,T", [("f32", 64), ("bf16", 31)])
def test_gdn_wy_other_calls_run_the_token_kernel(ema, dtype, T):
    # f32 activations and scans under 32 tokens leave the workspace unused: bit-identical
    # to ema_gdn_scan
    import torch

    B, Hk, Hv, Dk, Dv = 1, 2, 4, 64, 32
    (dq, dk_, dv_, dg, db, dS), _ = make_inputs(61, B, T, Hk, Hv, Dk, Dv, dtype)
    S1, S2 = dS.clone(), dS.clone()
    y1 = ema.gdn_scan(dq, dk_, dv_, dg, db, S1)
    y2 = ema.gdn_scan(dq, dk_, dv_, dg, db, S2, workspace=torch.empty(16, dtype=torch.uint8, device="cuda"))
    torch.cuda.synchronize()
    assert torch.equal(S1, S2)
    assert torch.equal(y1.view(torch.int16) if dtype == "bf16" else y1, y2.view(torch.int16) if dtype == "bf16" else y2)
