"""Helpers shared by the GPU parity tests (device upload/download, tolerance)."""
import math
import sys

import numpy as np

MAX_ABS = 2e-2   # bf16 outputs vs the f64 oracle: max-abs 2e-2 ...
MEAN_ABS = 2e-3  # ... and mean-abs 2e-3


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def dev(a: np.ndarray):
    import torch

    a = np.ascontiguousarray(a)
    if a.dtype == np.uint16:
        return torch.from_numpy(a.view(np.int16)).cuda().view(torch.bfloat16)
    return torch.from_numpy(a).cuda()


def host(t) -> np.ndarray:
    import torch

    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).cpu().numpy().view(np.uint16)
    return t.cpu().numpy()


def f32(h: np.ndarray) -> np.ndarray:
    return (np.asarray(h, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def assert_close(got: np.ndarray, ref: np.ndarray, what: str, max_abs=MAX_ABS, mean_abs=MEAN_ABS):
    g = f32(got).astype(np.float64)
    r = f32(ref).astype(np.float64)
    assert g.size == r.size, (g.shape, r.shape)
    r = r.reshape(g.shape)
    assert np.all(np.isfinite(g)), f"{what}: non-finite output"
    d = np.abs(g - r)
    mx, mn = float(d.max()), float(d.mean())
    say(f"  {what}: max_abs={mx:.3e} mean_abs={mn:.3e}")
    assert mx <= max_abs and mn <= mean_abs, f"{what}: max_abs={mx} mean_abs={mn}"


def scale_of(D: int) -> float:
    return 1.0 / math.sqrt(D)
