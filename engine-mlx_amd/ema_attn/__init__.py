"""Python binding of the ema_attn C ABI (include/ema_attn.h).

Thin ctypes layer used by the tests and the benchmark: tensors are torch
device tensors (bf16 / int32), every call goes through ``libema_attn.so`` and
fails loudly when the library is missing or a call returns an error. There is
no fallback path.

The names mirror the reference's API for this path:
``KvCache``/``StaticCache`` (crates/kvcache/src/lib.rs:52-76) and
``gqa_attention`` (crates/attention/src/gqa.rs:62-107) minus the projections.
"""
from __future__ import annotations

import ctypes
import math
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libema_attn.so")

EMA_OK = 0
EMA_ERR_INVALID_ARG = -1
EMA_ERR_SHAPE = -2
EMA_ERR_CAPACITY = -3
EMA_ERR_WORKSPACE = -4
EMA_ERR_UNSUPPORTED = -5
EMA_ERR_HIP = -6

EMA_DTYPE_BF16 = 1
EMA_DTYPE_FP8_E4M3 = 2
EMA_DTYPE_F16 = 3
EMA_DTYPE_F32 = 4
EMA_DTYPE_INT4_AFFINE = 5
EMA_PRE_NO_NORM = 1
EMA_PRE_NO_ROPE = 2
EMA_PRE_NO_Q_NORM = 8
EMA_PRE_NO_K_NORM = 16
EMA_STEP_ADVANCE = 4
EMA_DECODE_COUNTER_BYTES = 131072
EMA_KV_ROTATING = 1
EMA_PREFILL_CAUSAL = 1
EMA_PREFILL_CHUNK_ONLY = 2
EMA_PREFILL_ROWS_DECODED = 4

EXPORTED = (
    "ema_last_error", "ema_version", "ema_kvcache_init", "ema_kvcache_alloc", "ema_kvcache_free",
    "ema_kvcache_init_fp8", "ema_kvcache_alloc_fp8", "ema_kvcache_init_int4", "ema_kvcache_alloc_int4",
    "ema_kvcache_quantize_int4", "ema_kvcache_convert", "ema_position_write",
    "ema_kvcache_memory_bytes", "ema_pre_attention", "ema_pre_attention_ws", "ema_decode_workspace_size",
    "ema_decode_attention", "ema_decode_step", "ema_decode_step_noalloc", "ema_prefill_attention", "ema_prefill_workspace_size",
    "ema_prefill_attention_ws", "ema_gdn_scan", "ema_gdn_scan_workspace_size", "ema_gdn_scan_ws",
    "ema_quantized_matmul",
)


class EmaError(RuntimeError):
    def __init__(self, code: int, op: str, msg: str):
        super().__init__(f"{op} failed with code {code}: {msg}")
        self.code = code
        self.op = op
        self.msg = msg


class KvCacheDesc(ctypes.Structure):
    _fields_ = [
        ("k", ctypes.c_void_p), ("v", ctypes.c_void_p),
        ("batch", ctypes.c_int32), ("n_kv_heads", ctypes.c_int32),
        ("capacity", ctypes.c_int32), ("head_dim", ctypes.c_int32),
        ("stride_batch", ctypes.c_int64), ("stride_head", ctypes.c_int64),
        ("stride_pos", ctypes.c_int64), ("dtype", ctypes.c_int32), ("flags", ctypes.c_int32),
        ("k_exp", ctypes.c_void_p), ("v_exp", ctypes.c_void_p),
        ("k_scales", ctypes.c_void_p), ("k_biases", ctypes.c_void_p),
        ("v_scales", ctypes.c_void_p), ("v_biases", ctypes.c_void_p),
        ("n_rot", ctypes.c_int32),
    ]


_lib = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"ema_attn HIP library not built: {LIB_PATH} (run __graft_entry__.build())")
        L = ctypes.CDLL(LIB_PATH)
        vp, i32, u32, f32, u64 = ctypes.c_void_p, ctypes.c_int32, ctypes.c_uint32, ctypes.c_float, ctypes.c_uint64
        i64 = ctypes.c_int64
        D = ctypes.POINTER(KvCacheDesc)
        sig = {
            "ema_last_error": (ctypes.c_char_p, []),
            "ema_version": (ctypes.c_char_p, []),
            "ema_kvcache_init": (i32, [D, vp, vp, i32, i32, i32, i32]),
            "ema_kvcache_alloc": (i32, [D, i32, i32, i32, i32]),
            "ema_kvcache_init_fp8": (i32, [D, vp, vp, vp, vp, i32, i32, i32, i32, i32]),
            "ema_kvcache_alloc_fp8": (i32, [D, i32, i32, i32, i32, i32]),
            "ema_kvcache_init_int4": (i32, [D, vp, vp, vp, vp, vp, vp, i32, i32, i32, i32]),
            "ema_kvcache_alloc_int4": (i32, [D, i32, i32, i32, i32]),
            "ema_kvcache_quantize_int4": (i32, [vp, D, i32, D, i32, i32]),
            "ema_kvcache_convert": (i32, [vp, D, i32, D, i32, i32]),
            "ema_position_write": (i32, [vp, vp, i32]),
            "ema_kvcache_free": (i32, [D]),
            "ema_kvcache_memory_bytes": (i32, [D, ctypes.POINTER(u64)]),
            "ema_pre_attention": (i32, [vp, vp, vp, vp, f32, f32, vp, i32, i32, i32, i32, i32, u32, vp, D]),
            "ema_pre_attention_ws": (i32, [vp, vp, vp, vp, f32, f32, vp, i32, i32, i32, i32, i32, u32, vp, D, i32, vp,
                                           u64]),
            "ema_decode_workspace_size": (i32, [i32, i32, i32, i32, i32, ctypes.POINTER(u64)]),
            "ema_decode_attention": (i32, [vp, vp, D, vp, i32, i32, f32, vp, vp, u64]),
            "ema_decode_step": (i32, [vp, vp, vp, vp, f32, f32, vp, i32, i32, u32, f32, D, vp, vp, u64]),
            "ema_decode_step_noalloc": (i32, [vp, vp, vp, vp, f32, f32, vp, i32, i32, u32, f32, D, vp]),
            "ema_prefill_attention": (i32, [vp, vp, D, vp, i32, i32, f32, u32, vp]),
            "ema_prefill_workspace_size": (i32, [D, i32, ctypes.POINTER(u64)]),
            "ema_prefill_attention_ws": (i32, [vp, vp, D, vp, i32, i32, f32, u32, vp, i32, vp, u64]),
            "ema_gdn_scan": (i32, [vp, vp, vp, vp, vp, vp, vp, vp, i32, i32, i32, i32, i32, i32, i32]),
            "ema_gdn_scan_workspace_size": (i32, [i32, i32, i32, i32, i32, i32, ctypes.POINTER(u64)]),
            "ema_gdn_scan_ws": (i32, [vp, vp, vp, vp, vp, vp, vp, vp, i32, i32, i32, i32, i32, i32, i32, vp, u64]),
            "ema_quantized_matmul": (i32, [vp, vp, i64, vp, vp, vp, vp, i64, i32, i32, i32, i32, i32, i32]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def last_error() -> str:
    return lib().ema_last_error().decode()


def version() -> str:
    return lib().ema_version().decode()


def _check(rc: int, op: str) -> None:
    if rc != EMA_OK:
        raise EmaError(rc, op, last_error())


def _ptr(t) -> int | None:
    return None if t is None else t.data_ptr()


def _stream(stream) -> int | None:
    import torch

    if stream is None:
        stream = torch.cuda.current_stream()
    return stream.cuda_stream


class StaticCache:
    """Static pre-allocated KV cache of one layer, [B, Hkv, cap, D], bf16 or FP8.

    Mirrors the reference's static KV state (crates/serve/src/engine.rs:31-42,
    alloc_kv_static at crates/serve/src/engine_ext.rs:266-306) behind the
    KvCache trait surface (crates/kvcache/src/lib.rs:52-76): ``len`` is the
    number of valid positions per sequence, ``reset`` only rewinds the offsets
    (stale rows stay and are excluded by length, engine_ext.rs:218-228).

    ``dtype="fp8"``: the stored form of the reference's Fp8Cache
    (crates/kvcache/src/fp8.rs): ``k``/``v`` are uint8 E4M3FN codes and
    ``k_exp``/``v_exp`` int8 [B, Hkv, cap, D/64] block exponents
    (value = code * 2^exp); head_dim 128. ``n_rot=64`` (Fp8Cache::new(128, 64)): the last
    64 dims of each row are kept as bf16, so a row of ``k``/``v`` is [B, Hkv, cap, 192]
    bytes, 64 codes then the 64 bf16 values (block 1's exponent is 0).

    ``dtype="int4"``: the reference's int4 KV buffers (alloc_kv_int4,
    crates/serve/src/engine_ext.rs:92-129): ``k``/``v`` are int32 words [B, Hkv, cap, D/8]
    (8 four-bit codes each, lowest bits first) and ``k_scales``/``k_biases``/``v_scales``/
    ``v_biases`` bf16 [B, Hkv, cap, D/64] (value = scale * code + bias); head_dim 128,
    capacity a multiple of 32, decode only (static or rotating).

    ``rotating=True``: the reference's RotatingCache (crates/kvcache/src/rotating.rs) as a
    ring of ``capacity`` rows (EMA_KV_ROTATING): position p lives in row p % capacity and
    attention covers the last ``capacity`` tokens; ``len`` is then min(tokens, capacity).
    """

    def __init__(self, batch: int, n_kv_heads: int, capacity: int, head_dim: int, device="cuda",
                 k=None, v=None, dtype="bf16", k_exp=None, v_exp=None, rotating=False, k_scales=None,
                 k_biases=None, v_scales=None, v_biases=None, n_rot=0):
        import torch

        shape = (batch, n_kv_heads, capacity, head_dim)
        self.desc = KvCacheDesc()
        self.dtype = dtype
        if dtype == "bf16":
            self.k = k if k is not None else torch.zeros(shape, dtype=torch.bfloat16, device=device)
            self.v = v if v is not None else torch.zeros(shape, dtype=torch.bfloat16, device=device)
            self.k_exp = self.v_exp = None
            _check(lib().ema_kvcache_init(ctypes.byref(self.desc), _ptr(self.k), _ptr(self.v), batch, n_kv_heads,
                                          capacity, head_dim), "ema_kvcache_init")
        elif dtype == "fp8":
            eshape = (batch, n_kv_heads, capacity, head_dim // 64)
            rshape = (batch, n_kv_heads, capacity, head_dim + n_rot)
            self.k = k if k is not None else torch.zeros(rshape, dtype=torch.uint8, device=device)
            self.v = v if v is not None else torch.zeros(rshape, dtype=torch.uint8, device=device)
            self.k_exp = k_exp if k_exp is not None else torch.zeros(eshape, dtype=torch.int8, device=device)
            self.v_exp = v_exp if v_exp is not None else torch.zeros(eshape, dtype=torch.int8, device=device)
            _check(lib().ema_kvcache_init_fp8(ctypes.byref(self.desc), _ptr(self.k), _ptr(self.v), _ptr(self.k_exp),
                                              _ptr(self.v_exp), batch, n_kv_heads, capacity, head_dim, n_rot),
                   "ema_kvcache_init_fp8")
        elif dtype == "int4":
            mshape = (batch, n_kv_heads, capacity, head_dim // 64)
            self.k = k if k is not None else torch.zeros(shape[:3] + (head_dim // 8,), dtype=torch.int32, device=device)
            self.v = v if v is not None else torch.zeros(shape[:3] + (head_dim // 8,), dtype=torch.int32, device=device)
            self.k_exp = self.v_exp = None
            self.k_scales, self.k_biases, self.v_scales, self.v_biases = (
                t if t is not None else torch.zeros(mshape, dtype=torch.bfloat16, device=device)
                for t in (k_scales, k_biases, v_scales, v_biases))
            _check(lib().ema_kvcache_init_int4(ctypes.byref(self.desc), _ptr(self.k), _ptr(self.v),
                                               _ptr(self.k_scales), _ptr(self.k_biases), _ptr(self.v_scales),
                                               _ptr(self.v_biases), batch, n_kv_heads, capacity, head_dim),
                   "ema_kvcache_init_int4")
        else:
            raise ValueError(f"unknown cache dtype {dtype!r} (bf16, fp8 or int4)")
        if n_rot and dtype != "fp8":
            raise ValueError("n_rot is an fp8 cache parameter")
        self.rotating = bool(rotating)
        if self.rotating:
            self.desc.flags = EMA_KV_ROTATING
        self.offsets = [0] * batch

    @property
    def capacity(self) -> int:
        return self.desc.capacity

    def len(self) -> int:
        n = max(self.offsets) if self.offsets else 0
        return min(n, self.capacity) if self.rotating else n

    def is_empty(self) -> bool:
        return self.len() == 0

    def reset(self) -> None:
        self.offsets = [0] * len(self.offsets)

    def memory_bytes(self) -> int:
        out = ctypes.c_uint64()
        _check(lib().ema_kvcache_memory_bytes(ctypes.byref(self.desc), ctypes.byref(out)), "ema_kvcache_memory_bytes")
        return out.value


def quantize_int4(src: StaticCache, dst: StaticCache, n_rows: int, src_row: int = 0, dst_row: int = 0,
                  stream=None) -> None:
    """Rows [src_row, src_row + n_rows) of the bf16 cache ``src`` quantised into rows
    [dst_row, ...) of the int4 cache ``dst`` (convert_kv_to_int4,
    crates/serve/src/engine_ext.rs:158-210)."""
    _check(lib().ema_kvcache_quantize_int4(_stream(stream), ctypes.byref(src.desc), src_row, ctypes.byref(dst.desc),
                                           dst_row, n_rows), "ema_kvcache_quantize_int4")


def kvcache_convert(src: StaticCache, dst: StaticCache, n_rows: int, src_row: int = 0, dst_row: int = 0,
                    stream=None) -> None:
    """Rows [src_row, src_row + n_rows) of ``src`` converted into rows [dst_row, ...) of
    ``dst``: bf16 -> FP8 (Fp8Cache::append's quantisation, crates/kvcache/src/fp8.rs:47-68),
    FP8 -> bf16 (the decoded values Fp8Cache::get returns) or bf16 -> int4."""
    _check(lib().ema_kvcache_convert(_stream(stream), ctypes.byref(src.desc), src_row, ctypes.byref(dst.desc),
                                     dst_row, n_rows), "ema_kvcache_convert")


def position_write(slot, value: int, stream=None) -> None:
    """Stream-ordered write of ``value`` into the device int32 tensor element ``slot``."""
    _check(lib().ema_position_write(_stream(stream), _ptr(slot), int(value)), "ema_position_write")


def pre_attention(qkv, q_norm_w, k_norm_w, eps, theta, offsets, n_heads, cache: StaticCache, flags=0,
                  q_out=None, stream=None, prefill_workspace=None, max_kv_len=None):
    """qkv [B,T,(Hq+2Hkv)*D] bf16; offsets int32 device [B]. Returns q_out [B,Hq,T,D].

    With prefill_workspace (an FP8 cache: the workspace of prefill_attention for max_kv_len,
    default the capacity), ema_pre_attention_ws also writes the stored rows, decoded, into
    its bf16 copy; pass rows_decoded=True to prefill_attention with the same workspace."""
    import torch

    B, T, F = qkv.shape
    D = cache.desc.head_dim
    Hkv = cache.desc.n_kv_heads
    if q_out is None:
        q_out = torch.empty((B, n_heads, T, D), dtype=torch.bfloat16, device=qkv.device)
    if prefill_workspace is not None:
        if max_kv_len is None:
            max_kv_len = cache.capacity
        _check(lib().ema_pre_attention_ws(_stream(stream), _ptr(qkv), _ptr(q_norm_w), _ptr(k_norm_w), eps, theta,
                                          _ptr(offsets), B, T, n_heads, Hkv, D, flags, _ptr(q_out),
                                          ctypes.byref(cache.desc), max_kv_len, _ptr(prefill_workspace),
                                          prefill_workspace.numel()), "ema_pre_attention_ws")
        return q_out
    _check(lib().ema_pre_attention(_stream(stream), _ptr(qkv), _ptr(q_norm_w), _ptr(k_norm_w), eps, theta,
                                   _ptr(offsets), B, T, n_heads, Hkv, D, flags, _ptr(q_out),
                                   ctypes.byref(cache.desc)), "ema_pre_attention")
    return q_out


def decode_workspace_size(batch, n_heads, n_kv_heads, head_dim, max_len) -> int:
    out = ctypes.c_uint64()
    _check(lib().ema_decode_workspace_size(batch, n_heads, n_kv_heads, head_dim, max_len, ctypes.byref(out)),
           "ema_decode_workspace_size")
    return out.value


def decode_workspace(batch, n_heads, n_kv_heads, head_dim, max_len, device="cuda", stream=None):
    """Allocate a decode workspace (reusable across calls on one stream, any shape): zero-
    filled, as the arrival counters at its start must be before the first call."""
    import torch

    n = decode_workspace_size(batch, n_heads, n_kv_heads, head_dim, max_len)
    return torch.zeros(n, dtype=torch.uint8, device=device)


def decode_attention(q, cache: StaticCache, lengths, max_len, scale=None, out=None, workspace=None, stream=None):
    """q [B,Hq,D] (or [B,Hq,1,D]) bf16; lengths int32 device [B]. Returns out [B, Hq*D]."""
    import torch

    B, Hq = q.shape[0], q.shape[1]
    D = cache.desc.head_dim
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    if out is None:
        out = torch.empty((B, Hq * D), dtype=torch.bfloat16, device=q.device)
    if workspace is None:
        workspace = decode_workspace(B, Hq, cache.desc.n_kv_heads, D, max_len, device=q.device, stream=stream)
    _check(lib().ema_decode_attention(_stream(stream), _ptr(q), ctypes.byref(cache.desc), _ptr(lengths), max_len, Hq,
                                      scale, _ptr(out), _ptr(workspace), workspace.numel()), "ema_decode_attention")
    return out


def decode_step(qkv, q_norm_w, k_norm_w, eps, theta, offsets, n_heads, cache: StaticCache, max_len, scale=None,
                flags=0, out=None, workspace=None, stream=None):
    """Fused pre-attention (one token per sequence) + decode attention.

    qkv [B,(Hq+2Hkv)*D] (or [B,1,...]) bf16; offsets int32 device [B]. Returns out [B, Hq*D]."""
    import torch

    B = qkv.shape[0]
    D = cache.desc.head_dim
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    if out is None:
        out = torch.empty((B, n_heads * D), dtype=torch.bfloat16, device=qkv.device)
    if workspace is None:
        workspace = decode_workspace(B, n_heads, cache.desc.n_kv_heads, D, max_len, device=qkv.device)
    _check(lib().ema_decode_step(_stream(stream), _ptr(qkv), _ptr(q_norm_w), _ptr(k_norm_w), eps, theta,
                                 _ptr(offsets), max_len, n_heads, flags, scale, ctypes.byref(cache.desc), _ptr(out),
                                 _ptr(workspace), workspace.numel()), "ema_decode_step")
    return out


def decode_step_noalloc(qkv, q_norm_w, k_norm_w, eps, theta, offsets, n_heads, cache: StaticCache, max_len, out,
                        scale=None, flags=0, stream=None):
    """ema_decode_step over the library's static per-device scratch: no workspace and no
    device allocation in the call (out is the caller's [B, Hq*D] bf16 buffer)."""
    D = cache.desc.head_dim
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    _check(lib().ema_decode_step_noalloc(_stream(stream), _ptr(qkv), _ptr(q_norm_w), _ptr(k_norm_w), eps, theta,
                                         _ptr(offsets), max_len, n_heads, flags, scale, ctypes.byref(cache.desc),
                                         _ptr(out)), "ema_decode_step_noalloc")
    return out


def prefill_workspace_size(cache: StaticCache, max_kv_len: int) -> int:
    out = ctypes.c_uint64()
    _check(lib().ema_prefill_workspace_size(ctypes.byref(cache.desc), max_kv_len, ctypes.byref(out)),
           "ema_prefill_workspace_size")
    return out.value


def prefill_attention(q, cache: StaticCache, q_offsets, scale=None, causal=True, chunk_only=False, out=None,
                      stream=None, max_kv_len=None, workspace=None, rows_decoded=False):
    """q [B,Hq,T,D] bf16; q_offsets int32 device [B]. Returns out [B,T,Hq*D].

    An FP8 cache goes through ema_prefill_attention_ws: its attended rows (at most
    max_kv_len per sequence, default the capacity) are decoded into a bf16 workspace.
    rows_decoded: the chunk's rows are in that workspace already (pre_attention with
    prefill_workspace, EMA_PREFILL_ROWS_DECODED)."""
    import torch

    B, Hq, T, D = q.shape
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    if out is None:
        out = torch.empty((B, T, Hq * D), dtype=torch.bfloat16, device=q.device)
    flags = (EMA_PREFILL_CAUSAL if causal else 0) | (EMA_PREFILL_CHUNK_ONLY if chunk_only else 0)
    flags |= EMA_PREFILL_ROWS_DECODED if rows_decoded else 0
    if cache.dtype == "bf16" and workspace is None:
        _check(lib().ema_prefill_attention(_stream(stream), _ptr(q), ctypes.byref(cache.desc), _ptr(q_offsets), T,
                                           Hq, scale, flags, _ptr(out)), "ema_prefill_attention")
        return out
    if max_kv_len is None:
        max_kv_len = cache.capacity
    if workspace is None:
        workspace = torch.empty(max(prefill_workspace_size(cache, max_kv_len), 16), dtype=torch.uint8,
                                device=q.device)
    _check(lib().ema_prefill_attention_ws(_stream(stream), _ptr(q), ctypes.byref(cache.desc), _ptr(q_offsets), T,
                                          Hq, scale, flags, _ptr(out), max_kv_len, _ptr(workspace),
                                          workspace.numel()), "ema_prefill_attention_ws")
    return out


def gdn_scan_workspace_size(B, T, Hk, Hv, Dk, Dv) -> int:
    """Bytes of the workspace with which gdn_scan runs T tokens in one segment
    (ema_gdn_scan_workspace_size)."""
    n = ctypes.c_uint64(0)
    _check(lib().ema_gdn_scan_workspace_size(B, T, Hk, Hv, Dk, Dv, ctypes.byref(n)), "ema_gdn_scan_workspace_size")
    return n.value


def gdn_workspace(B, T, Hk, Hv, Dk, Dv, device="cuda"):
    """A workspace tensor for gdn_scan (no initialisation needed)."""
    import torch

    return torch.empty(gdn_scan_workspace_size(B, T, Hk, Hv, Dk, Dv), dtype=torch.uint8, device=device)


def gdn_scan(q, k, v, g, beta, state, y=None, stream=None, workspace=None):
    """Gated DeltaNet recurrent scan (ema_gdn_scan): q, k [B,T,Hk,Dk], v [B,T,Hv,Dv] in bf16,
    f16 or f32; g, beta [B,T,Hv] f32; state [B,Hv,Dv,Dk] f32, updated in place. Returns
    y [B,T,Hv,Dv] in the activation dtype. With a workspace (a uint8 tensor, e.g. from
    gdn_workspace) bf16 scans of 32+ tokens run in WY form (ema_gdn_scan_ws)."""
    import torch

    dtypes = {torch.bfloat16: EMA_DTYPE_BF16, torch.float16: EMA_DTYPE_F16, torch.float32: EMA_DTYPE_F32}
    if q.dtype not in dtypes:
        raise EmaError(EMA_ERR_INVALID_ARG, "ema_gdn_scan", f"unsupported activation dtype {q.dtype}")
    B, T, Hk, Dk = q.shape
    Hv, Dv = v.shape[2], v.shape[3]
    if y is None:
        y = torch.empty((B, T, Hv, Dv), dtype=q.dtype, device=q.device)
    if workspace is None:
        _check(lib().ema_gdn_scan(_stream(stream), _ptr(q), _ptr(k), _ptr(v), _ptr(g), _ptr(beta), _ptr(state),
                                  _ptr(y), B, T, Hk, Hv, Dk, Dv, dtypes[q.dtype]), "ema_gdn_scan")
    else:
        _check(lib().ema_gdn_scan_ws(_stream(stream), _ptr(q), _ptr(k), _ptr(v), _ptr(g), _ptr(beta), _ptr(state),
                                     _ptr(y), B, T, Hk, Hv, Dk, Dv, dtypes[q.dtype], _ptr(workspace),
                                     workspace.numel() * workspace.element_size()), "ema_gdn_scan_ws")
    return y


def quantized_matmul(x, w, scales, biases, group_size=64, bits=4, out=None, stream=None):
    """MLX quantized_matmul(x, w, scales, biases, transpose=True, group_size, bits, "affine")
    (ema_quantized_matmul; the reference's qmatmul, crates/ops/src/quant.rs:57-76): x [..., K]
    bf16 or f16 with a contiguous last axis; w [N, K*bits/32] int32/uint32 words of MLX's
    packing; scales, biases [N, K/group_size] in x's dtype. Returns y [..., N] in x's dtype.
    `out` may be a 2-D view whose rows are wider than N (e.g. the q, k or v columns of a
    q|k|v buffer)."""
    import torch

    dtypes = {torch.bfloat16: EMA_DTYPE_BF16, torch.float16: EMA_DTYPE_F16}
    if x.dtype not in dtypes:
        raise EmaError(EMA_ERR_INVALID_ARG, "ema_quantized_matmul", f"unsupported activation dtype {x.dtype}")
    K = x.shape[-1]
    x2 = x.reshape(-1, K)
    M, N = x2.shape[0], w.shape[0]
    if w.shape[1] * 32 // bits != K:
        raise EmaError(EMA_ERR_SHAPE, "ema_quantized_matmul", f"w {tuple(w.shape)} does not pack K={K} at {bits} bits")
    if out is None:
        y2 = torch.empty((M, N), dtype=x.dtype, device=x.device)
    else:
        y2 = out
        if y2.dim() != 2 or y2.shape[0] != M or y2.shape[1] != N or y2.stride(1) != 1:
            raise EmaError(EMA_ERR_SHAPE, "ema_quantized_matmul", "out must be a [M, N] view with unit column stride")
    _check(lib().ema_quantized_matmul(_stream(stream), _ptr(x2), x2.stride(0), _ptr(w), _ptr(scales), _ptr(biases),
                                      _ptr(y2), y2.stride(0), M, N, K, group_size, bits, dtypes[x.dtype]),
           "ema_quantized_matmul")
    return y2.reshape(x.shape[:-1] + (N,)) if out is None else y2
