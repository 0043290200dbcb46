"""numpy front end of the CPU oracle (TEST INFRASTRUCTURE ONLY).

Only tests, ``__graft_entry__.smoke()`` and the CPU-baseline leg of
``bench.py`` import this module; it is the checker, never the product.
bf16 tensors are numpy ``uint16`` arrays holding IEEE bfloat16 bit patterns.
The C functions behind each wrapper cite the reference files they restate
(``oracle/ema_oracle.h``).
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None

FLAG_NO_NORM = 1
FLAG_NO_ROPE = 2
FLAG_NO_Q_NORM = 8
FLAG_NO_K_NORM = 16

_u16p = ctypes.POINTER(ctypes.c_uint16)
_i32p = ctypes.POINTER(ctypes.c_int32)
_f32p = ctypes.POINTER(ctypes.c_float)
_f64p = ctypes.POINTER(ctypes.c_double)
_u8p = ctypes.POINTER(ctypes.c_uint8)
_u32p = ctypes.POINTER(ctypes.c_uint32)
_i8p = ctypes.POINTER(ctypes.c_int8)


def build() -> None:
    """Compile liboracle.so with the recipe in oracle/Makefile."""
    import subprocess

    subprocess.run(["make", "-s", "-C", _HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            raise RuntimeError(f"oracle library not built: {_LIB_PATH} (run make -C oracle)")
        L = ctypes.CDLL(_LIB_PATH)
        L.ora_f32_to_bf16.restype = ctypes.c_uint16
        L.ora_f32_to_bf16.argtypes = [ctypes.c_float]
        L.ora_bf16_to_f32.restype = ctypes.c_float
        L.ora_bf16_to_f32.argtypes = [ctypes.c_uint16]
        L.ora_f32_to_bf16_array.argtypes = [_f32p, _u16p, ctypes.c_size_t]
        L.ora_bf16_to_f32_array.argtypes = [_u16p, _f32p, ctypes.c_size_t]
        L.ora_fill_normal_bf16.argtypes = [_u16p, ctypes.c_size_t, ctypes.c_uint64, ctypes.c_float, ctypes.c_float]
        L.ora_fill_normal_f32.argtypes = [_f32p, ctypes.c_size_t, ctypes.c_uint64, ctypes.c_float, ctypes.c_float]
        L.ora_rms_norm.argtypes = [_u16p, _u16p, ctypes.c_int64, ctypes.c_int, ctypes.c_float, _u16p]
        L.ora_rope.argtypes = [_u16p, _i32p, ctypes.c_int64, ctypes.c_int, ctypes.c_float, _u16p]
        L.ora_pre_attention.restype = ctypes.c_int
        L.ora_pre_attention.argtypes = [
            _u16p, _u16p, _u16p, ctypes.c_float, ctypes.c_float, _i32p,
            ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_uint32,
            _u16p, _u16p, _u16p, ctypes.c_int,
        ]
        L.ora_sdpa.argtypes = [
            _u16p, _u16p, _u16p, _i32p, _i32p,
            ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
            ctypes.c_float, ctypes.c_int, ctypes.c_int, _u16p,
        ]
        L.ora_sdpa_partial.argtypes = [_u16p, _u16p, _u16p, ctypes.c_int, ctypes.c_int, ctypes.c_float, _f64p, _f64p, _f64p]
        L.ora_lse_merge.argtypes = [_f64p, _f64p, _f64p, ctypes.c_int, ctypes.c_int, _f64p]
        L.ora_num_threads.restype = ctypes.c_int
        L.ora_e4m3_value.restype = ctypes.c_float
        L.ora_e4m3_value.argtypes = [ctypes.c_uint8]
        L.ora_e4m3fn_round.restype = ctypes.c_float
        L.ora_e4m3fn_round.argtypes = [ctypes.c_float, ctypes.POINTER(ctypes.c_uint8)]
        L.ora_fp8_block_exp.restype = ctypes.c_int
        L.ora_fp8_block_exp.argtypes = [_f32p, ctypes.c_int]
        L.ora_fp8_exp_of.restype = ctypes.c_int
        L.ora_fp8_exp_of.argtypes = [ctypes.c_float, ctypes.c_int]
        L.ora_fp8_exp_mismatches.restype = ctypes.c_int64
        L.ora_fp8_exp_mismatches.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int]
        L.ora_fp8_round_trip.argtypes = [_f32p, ctypes.c_int64, ctypes.c_int, ctypes.c_int]
        L.ora_fp8_quantize_rows.argtypes = [_f32p, ctypes.c_int64, ctypes.c_int, _u8p, _i8p]
        L.ora_fp8_dequantize_rows.argtypes = [_u8p, _i8p, ctypes.c_int64, ctypes.c_int, _f32p]
        L.ora_gdn_scan.argtypes = [_f32p, _f32p, _f32p, _f32p, _f32p, _f64p, _f64p] + [ctypes.c_int] * 6
        L.ora_qmatmul.argtypes = [_f32p, _u32p, _f32p, _f32p] + [ctypes.c_int] * 5 + [_f64p]
        L.ora_dequantize.argtypes = [_u32p, _f32p, _f32p] + [ctypes.c_int] * 4 + [_f64p]
        L.ora_int4_quantize_rows.argtypes = [_f32p, ctypes.c_int64, ctypes.c_int, _u32p, _u16p, _u16p]
        L.ora_int4_dequantize_rows.argtypes = [_u32p, _u16p, _u16p, ctypes.c_int64, ctypes.c_int, _f32p]
        _lib = L
    return _lib


def _p(a: np.ndarray, t):
    return a.ctypes.data_as(t)


def _c(a: np.ndarray, dtype) -> np.ndarray:
    a = np.ascontiguousarray(a)
    if a.dtype != dtype:
        raise TypeError(f"expected {dtype}, got {a.dtype}")
    return a


# ------------------------------------------------------------------ bf16
def bf16_from_f32(x) -> np.ndarray:
    x = np.ascontiguousarray(np.asarray(x, dtype=np.float32))
    out = np.empty(x.shape, dtype=np.uint16)
    lib().ora_f32_to_bf16_array(_p(x, _f32p), _p(out, _u16p), x.size)
    return out


def f32_from_bf16(h) -> np.ndarray:
    h = _c(np.asarray(h), np.uint16)
    out = np.empty(h.shape, dtype=np.float32)
    lib().ora_bf16_to_f32_array(_p(h, _u16p), _p(out, _f32p), h.size)
    return out


def normal_bf16(shape, seed: int, mean: float = 0.0, std: float = 1.0) -> np.ndarray:
    out = np.empty(shape, dtype=np.uint16)
    lib().ora_fill_normal_bf16(_p(out, _u16p), out.size, seed & 0xFFFFFFFFFFFFFFFF, mean, std)
    return out


def normal_f32(shape, seed: int, mean: float = 0.0, std: float = 1.0) -> np.ndarray:
    out = np.empty(shape, dtype=np.float32)
    lib().ora_fill_normal_f32(_p(out, _f32p), out.size, seed & 0xFFFFFFFFFFFFFFFF, mean, std)
    return out


# ------------------------------------------------------------------ ops
def rms_norm(x: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
    x = _c(x, np.uint16)
    w = _c(w, np.uint16)
    D = x.shape[-1]
    out = np.empty_like(x)
    lib().ora_rms_norm(_p(x, _u16p), _p(w, _u16p), x.size // D, D, eps, _p(out, _u16p))
    return out


def rope(x: np.ndarray, pos: np.ndarray, theta: float) -> np.ndarray:
    """x: [rows, D] bf16; pos: [rows] int32 absolute positions."""
    x = _c(x, np.uint16)
    D = x.shape[-1]
    rows = x.size // D
    pos = _c(np.asarray(pos, dtype=np.int32).reshape(rows), np.int32)
    out = np.empty_like(x)
    lib().ora_rope(_p(x, _u16p), _p(pos, _i32p), rows, D, theta, _p(out, _u16p))
    return out


def pre_attention(qkv, q_norm_w, k_norm_w, eps, theta, off, Hq, Hkv, kcache, vcache, flags=0):
    """qkv [B,T,(Hq+2Hkv)*D] bf16; caches [B,Hkv,cap,D] bf16 updated in place.

    Returns q_out [B,Hq,T,D]. Raises ValueError when off+T exceeds the capacity.
    """
    qkv = _c(qkv, np.uint16)
    B, T, F = qkv.shape
    D = F // (Hq + 2 * Hkv)
    cap = kcache.shape[2]
    off = _c(np.asarray(off, dtype=np.int32).reshape(B), np.int32)
    qw = _c(q_norm_w if q_norm_w is not None else np.zeros(D, np.uint16), np.uint16)
    kw = _c(k_norm_w if k_norm_w is not None else np.zeros(D, np.uint16), np.uint16)
    assert kcache.flags.c_contiguous and vcache.flags.c_contiguous
    q_out = np.empty((B, Hq, T, D), dtype=np.uint16)
    rc = lib().ora_pre_attention(
        _p(qkv, _u16p), _p(qw, _u16p), _p(kw, _u16p), eps, theta, _p(off, _i32p),
        B, T, Hq, Hkv, D, flags, _p(q_out, _u16p), _p(kcache, _u16p), _p(vcache, _u16p), cap,
    )
    if rc != 0:
        raise ValueError("static KV overflow")
    return q_out


def sdpa(q, kcache, vcache, kv_len, scale, causal, kv_begin=None, precision=0) -> np.ndarray:
    """q [B,Hq,Tq,D]; caches [B,Hkv,cap,D]; kv_len [B]. Returns out [B,Tq,Hq*D] bf16."""
    q = _c(q, np.uint16)
    kcache = _c(kcache, np.uint16)
    vcache = _c(vcache, np.uint16)
    B, Hq, Tq, D = q.shape
    Hkv, cap = kcache.shape[1], kcache.shape[2]
    kv_len = _c(np.asarray(kv_len, dtype=np.int32).reshape(B), np.int32)
    kb = None
    if kv_begin is not None:
        kb = _c(np.asarray(kv_begin, dtype=np.int32).reshape(B), np.int32)
    out = np.empty((B, Tq, Hq * D), dtype=np.uint16)
    lib().ora_sdpa(
        _p(q, _u16p), _p(kcache, _u16p), _p(vcache, _u16p), _p(kv_len, _i32p),
        _p(kb, _i32p) if kb is not None else None,
        B, Hq, Hkv, Tq, D, cap, scale, int(bool(causal)), precision, _p(out, _u16p),
    )
    return out


def sdpa_partial(q, k, v, scale):
    """One query q[D] against key/value rows k,v [n,D]: returns (m, l, acc[D]) in f64."""
    q = _c(q, np.uint16)
    k = _c(k, np.uint16)
    v = _c(v, np.uint16)
    n, D = k.shape
    m = ctypes.c_double()
    l = ctypes.c_double()
    acc = np.empty(D, dtype=np.float64)
    lib().ora_sdpa_partial(_p(q, _u16p), _p(k, _u16p), _p(v, _u16p), n, D, scale,
                           ctypes.byref(m), ctypes.byref(l), _p(acc, _f64p))
    return m.value, l.value, acc


def lse_merge(ms, ls, accs) -> np.ndarray:
    ms = np.ascontiguousarray(ms, dtype=np.float64)
    ls = np.ascontiguousarray(ls, dtype=np.float64)
    accs = np.ascontiguousarray(accs, dtype=np.float64)
    P, D = accs.shape
    out = np.empty(D, dtype=np.float64)
    lib().ora_lse_merge(_p(ms, _f64p), _p(ls, _f64p), _p(accs, _f64p), P, D, _p(out, _f64p))
    return out


def num_threads() -> int:
    return int(lib().ora_num_threads())


# ------------------------------------------------------------------ FP8 E4M3FN (crates/ops/src/fp8.rs)
def e4m3_value(code: int) -> float:
    return float(lib().ora_e4m3_value(code))


def e4m3fn_round(x: float):
    """e4m3fn_dequant (fp8.rs:36-64): returns (value, code)."""
    c = ctypes.c_uint8()
    v = lib().ora_e4m3fn_round(float(x), ctypes.byref(c))
    return float(v), int(c.value)


def e4m3fn_round_array(x) -> np.ndarray:
    x = np.asarray(x, dtype=np.float32).ravel()
    return np.array([lib().ora_e4m3fn_round(float(v), None) for v in x], dtype=np.float32)


def fp8_exp_of(r: float, ref: bool = True) -> int:
    return int(lib().ora_fp8_exp_of(float(r), 1 if ref else 0))


def fp8_exp_mismatches(kmin: int, kmax: int, nulps: int) -> int:
    return int(lib().ora_fp8_exp_mismatches(kmin, kmax, nulps))


def fp8_round_trip(x, D: int, n_rot: int = 0) -> np.ndarray:
    """fp8_round_trip_slice (fp8.rs:71-92) on rows of D f32 values; returns a new array."""
    x = np.array(x, dtype=np.float32, copy=True)
    lib().ora_fp8_round_trip(_p(x, _f32p), x.size // D, D, n_rot)
    return x


def fp8_quantize(x):
    """Rows of D (multiple of 64) f32 values -> (codes uint8 [..., D], exps int8 [..., D/64])."""
    x = _c(np.asarray(x, dtype=np.float32), np.float32)
    D = x.shape[-1]
    codes = np.empty(x.shape, dtype=np.uint8)
    exps = np.empty(x.shape[:-1] + (D // 64,), dtype=np.int8)
    lib().ora_fp8_quantize_rows(_p(x, _f32p), x.size // D, D, _p(codes, _u8p), _p(exps, _i8p))
    return codes, exps


def fp8_dequantize(codes, exps) -> np.ndarray:
    codes = _c(np.asarray(codes), np.uint8)
    exps = _c(np.asarray(exps), np.int8)
    D = codes.shape[-1]
    out = np.empty(codes.shape, dtype=np.float32)
    lib().ora_fp8_dequantize_rows(_p(codes, _u8p), _p(exps, _i8p), codes.size // D, D, _p(out, _f32p))
    return out


def int4_quantize(x):
    """Rows of D (multiple of 64) f32 values -> (words uint32 [..., D/8], scales and biases as
    bf16 bits [..., D/64]): MLX affine quantisation, group 64, 4 bits (quantize_kv_native,
    crates/mlx-ffi/src/ops/real/quant.rs:8-40; ora_int4_quantize_rows)."""
    x = _c(np.asarray(x, dtype=np.float32), np.float32)
    D = x.shape[-1]
    assert D % 64 == 0
    rows = x.size // D
    words = np.empty(x.shape[:-1] + (D // 8,), dtype=np.uint32)
    scales = np.empty(x.shape[:-1] + (D // 64,), dtype=np.uint16)
    biases = np.empty_like(scales)
    lib().ora_int4_quantize_rows(_p(x, _f32p), rows, D, _p(words, _u32p), _p(scales, _u16p), _p(biases, _u16p))
    return words, scales, biases


def int4_dequantize(words, scales, biases) -> np.ndarray:
    """MLX affine dequantize to bf16 (dequantize_kv_native, quant.rs:41-64): f32 values
    bf16(scale * code + bias), one rounding, shape [..., D]."""
    words = _c(np.asarray(words), np.uint32)
    scales = _c(np.asarray(scales), np.uint16)
    biases = _c(np.asarray(biases), np.uint16)
    D = words.shape[-1] * 8
    rows = words.size // (D // 8)
    out = np.empty(words.shape[:-1] + (D,), dtype=np.float32)
    lib().ora_int4_dequantize_rows(_p(words, _u32p), _p(scales, _u16p), _p(biases, _u16p), rows, D, _p(out, _f32p))
    return out


def int4_affine_values(words, scales, biases) -> np.ndarray:
    """The exact affine values scale * code + bias (float64) of int4 rows [..., D]."""
    D = np.asarray(words).shape[-1] * 8
    codes = unpack_bits(words, 4).astype(np.float64)
    s = np.repeat(f32_from_bf16(scales).astype(np.float64), 64, axis=-1)
    b = np.repeat(f32_from_bf16(biases).astype(np.float64), 64, axis=-1)
    assert codes.shape[-1] == D == s.shape[-1]
    return codes * s + b


def gdn_scan(q, k, v, g, beta, state):
    """Gated DeltaNet scan (gdn.rs:83-150 per token, gdn_forward.rs:173-192): q, k [B,T,Hk,Dk],
    v [B,T,Hv,Dv], g, beta [B,T,Hv] (f32 values), state [B,Hv,Dv,Dk]. Returns (y [B,T,Hv,Dv],
    new state), both float64; the input state is not modified."""
    q = _c(np.asarray(q, dtype=np.float32), np.float32)
    k = _c(np.asarray(k, dtype=np.float32), np.float32)
    v = _c(np.asarray(v, dtype=np.float32), np.float32)
    g = _c(np.asarray(g, dtype=np.float32), np.float32)
    beta = _c(np.asarray(beta, dtype=np.float32), np.float32)
    S = np.array(state, dtype=np.float64, copy=True)
    B, T, Hk, Dk = q.shape
    Hv, Dv = v.shape[2], v.shape[3]
    assert k.shape == q.shape and v.shape[:2] == (B, T) and g.shape == (B, T, Hv) == beta.shape
    assert S.shape == (B, Hv, Dv, Dk) and Hv % Hk == 0
    y = np.empty((B, T, Hv, Dv), dtype=np.float64)
    lib().ora_gdn_scan(_p(q, _f32p), _p(k, _f32p), _p(v, _f32p), _p(g, _f32p), _p(beta, _f32p), _p(S, _f64p),
                       _p(y, _f64p), B, T, Hk, Hv, Dk, Dv)
    return y, S



def pack_bits(q, bits: int) -> np.ndarray:
    """Packs integer fields q [..., K] (0 <= q < 2**bits) into uint32 words [..., K*bits/32],
    field k at bits (k % (32/bits))*bits of word k // (32/bits), lowest bits first (MLX's
    affine packing for widths that divide 32)."""
    q = np.asarray(q, dtype=np.uint32)
    per = 32 // bits
    assert 32 % bits == 0 and q.shape[-1] % per == 0 and int(q.max(initial=0)) < (1 << bits)
    f = q.reshape(q.shape[:-1] + (q.shape[-1] // per, per))
    shifts = (np.arange(per, dtype=np.uint32) * bits).astype(np.uint32)
    return np.bitwise_or.reduce(f << shifts, axis=-1).astype(np.uint32)


def unpack_bits(wq, bits: int) -> np.ndarray:
    """Inverse of pack_bits: uint32 words [..., W] -> fields [..., W*32/bits]."""
    wq = np.asarray(wq, dtype=np.uint32)
    per = 32 // bits
    shifts = (np.arange(per, dtype=np.uint32) * bits).astype(np.uint32)
    f = (wq[..., None] >> shifts) & np.uint32((1 << bits) - 1)
    return f.reshape(wq.shape[:-1] + (wq.shape[-1] * per,))


def minmax_quantize(w, gs: int, bits: int):
    """Test-data generator: min-max affine quantisation of w [N, K] in groups of gs along K
    (scale = (max - min) / (2**bits - 1), bias = min, q = round((w - bias) / scale)), with
    scale and bias rounded to bf16 first. Returns (wq uint32, scales bf16 bits, biases bf16
    bits). Not MLX's quantiser (which also moves the edge onto the grid); the kernels here
    consume stored (wq, scales, biases) and never quantise."""
    w = np.asarray(w, dtype=np.float32)
    N, K = w.shape
    g = w.reshape(N, K // gs, gs)
    lo, hi = g.min(-1), g.max(-1)
    s = bf16_from_f32(np.maximum((hi - lo) / ((1 << bits) - 1), 1e-7).astype(np.float32))
    b = bf16_from_f32(lo)
    sf, bf = f32_from_bf16(s), f32_from_bf16(b)
    q = np.clip(np.rint((g - bf[..., None]) / sf[..., None]), 0, (1 << bits) - 1).astype(np.uint32)
    return pack_bits(q.reshape(N, K), bits), s, b


def dequantize(wq, scales, biases, gs: int, bits: int) -> np.ndarray:
    """W [N, K] = scales * q + biases in float64 (MLX affine dequantize, transform.rs:45-58);
    scales and biases as f32 values [N, K/gs]."""
    wq = _c(np.asarray(wq), np.uint32)
    s = _c(np.asarray(scales, dtype=np.float32), np.float32)
    b = _c(np.asarray(biases, dtype=np.float32), np.float32)
    N = wq.shape[0]
    K = wq.shape[1] * 32 // bits
    assert s.shape == (N, K // gs) == b.shape
    out = np.empty((N, K), dtype=np.float64)
    lib().ora_dequantize(_p(wq, _u32p), _p(s, _f32p), _p(b, _f32p), N, K, gs, bits, _p(out, _f64p))
    return out


def dequantize_act(wq, scales, biases, gs: int, bits: int, dtype: str = "bf16") -> np.ndarray:
    """The weights as MLX's quantized matmul for many rows of x (its qmm kernels) multiplies
    them: dequantised into the activation type first. w = round_T(s * q + b) with s * q + b
    formed in f32 (s * q is exact there, so the sum is rounded once, as by an fma) and one
    round-to-nearest-even to T = bf16 / f16. Returns the f32 values [N, K]. Whether MLX
    rounds once or twice (s * q, then + b, in T) is parity unpinned; this one-rounding
    reading is the one the GPU's large-M path implements."""
    wq = _c(np.asarray(wq), np.uint32)
    N = wq.shape[0]
    K = wq.shape[1] * 32 // bits
    G = K // gs
    q = dequantize(wq, np.ones((N, G), np.float32), np.zeros((N, G), np.float32), gs, bits).astype(np.float32)
    s = np.repeat(np.asarray(scales, dtype=np.float32), gs, axis=1)
    b = np.repeat(np.asarray(biases, dtype=np.float32), gs, axis=1)
    w = (s * q).astype(np.float32) + b  # f32 ops: the product is exact, the sum rounds once
    if dtype == "bf16":
        return f32_from_bf16(bf16_from_f32(w))
    return w.astype(np.float16).astype(np.float32)


def qmatmul(x, wq, scales, biases, gs: int, bits: int) -> np.ndarray:
    """MLX quantized_matmul(x, w, scales, biases, transpose=true, gs, bits, "affine")
    (transform.rs:77-88; qmatmul, crates/ops/src/quant.rs:57-76) in float64: x [..., K]
    (activation values as f32), wq [N, K*bits/32], scales/biases [N, K/gs] (f32 values).
    Returns y [..., N]."""
    x = np.asarray(x, dtype=np.float32)
    lead = x.shape[:-1]
    K = x.shape[-1]
    x2 = _c(x.reshape(-1, K), np.float32)
    wq = _c(np.asarray(wq), np.uint32)
    s = _c(np.asarray(scales, dtype=np.float32), np.float32)
    b = _c(np.asarray(biases, dtype=np.float32), np.float32)
    N = wq.shape[0]
    assert wq.shape[1] * 32 // bits == K and K % gs == 0 and s.shape == (N, K // gs) == b.shape
    y = np.empty((x2.shape[0], N), dtype=np.float64)
    lib().ora_qmatmul(_p(x2, _f32p), _p(wq, _u32p), _p(s, _f32p), _p(b, _f32p), x2.shape[0], N, K, gs, bits,
                      _p(y, _f64p))
    return y.reshape(lead + (N,))


def rotating_append(kept, n_new, window):
    """One RotatingCache::append (crates/kvcache/src/rotating.rs:56-97) on the list of
    absolute positions the cache holds, in its order: the first call with n_new <= window
    stores the chunk as is (:60-67); otherwise the chunk is concatenated (:70-77) and, past
    the window, only the last `window` positions are kept (:81-92). Returns the new list."""
    total = kept[-1] + 1 if kept else 0
    new = list(range(total, total + n_new))
    if not kept and n_new <= window:
        return new
    full = list(kept) + new
    return full[-window:] if len(full) > window else full


def rotating_window(total, window):
    """Positions a rotating cache of `window` rows holds after `total` tokens: [lo, total)."""
    return max(0, total - window), total


def ring_rows(total, window):
    """Ring layout of the rotating cache here (EMA_KV_ROTATING): row r holds the position
    p in rotating_window(total, window) with p % window == r; returns {row: position}."""
    lo, hi = rotating_window(total, window)
    return {p % window: p for p in range(lo, hi)}
