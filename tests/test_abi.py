"""C-ABI checks that need no GPU: the library loads, exports every symbol
include/ema_attn.h declares, and rejects bad arguments on the host with the
documented status codes and messages (no HIP call is reached)."""
import ctypes
import os
import re
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "ema_attn.h")


@pytest.fixture(scope="module")
def ema():
    import ema_attn

    if not os.path.exists(ema_attn.LIB_PATH):
        subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "engine-mlx_amd")], check=True)
    ema_attn.lib()
    return ema_attn


def declared_symbols():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"EMA_API\s+[\w\s\*]+?\b(ema_\w+)\s*\(", text)))


def test_header_declares_the_binding_set(ema):
    assert declared_symbols() == sorted(ema.EXPORTED)


def test_library_exports_every_declared_symbol(ema):
    out = subprocess.run(["nm", "-D", "--defined-only", ema.LIB_PATH], capture_output=True, text=True, check=True).stdout
    exported = set(re.findall(r"\sT\s(ema_\w+)$", out, re.M))
    missing = [s for s in declared_symbols() if s not in exported]
    assert not missing, missing
    # internal C++ helpers stay hidden
    assert not [s for s in exported if s not in ema.EXPORTED]


def test_version_and_empty_error(ema):
    assert "gfx950" in ema.version()


def _desc(ema, k=0x10000, v=0x20000, B=2, Hkv=8, cap=64, D=128):
    d = ema.KvCacheDesc()
    rc = ema.lib().ema_kvcache_init(ctypes.byref(d), k, v, B, Hkv, cap, D)
    return rc, d


def test_kvcache_init_and_memory_bytes(ema):
    rc, d = _desc(ema)
    assert rc == ema.EMA_OK
    assert (d.stride_pos, d.stride_head, d.stride_batch) == (128, 64 * 128, 8 * 64 * 128)
    n = ctypes.c_uint64()
    assert ema.lib().ema_kvcache_memory_bytes(ctypes.byref(d), ctypes.byref(n)) == 0
    assert n.value == 2 * 2 * 8 * 64 * 128 * 2


def test_empty_cache_is_rejected(ema):
    """Same contract text as ConcatCache::get (crates/kvcache/src/concat.rs:54)."""
    rc, d = _desc(ema, k=0, v=0)
    assert rc == ema.EMA_ERR_INVALID_ARG
    assert "KV cache is empty" in ema.last_error()


def test_bad_shapes_and_alignment(ema):
    rc, _ = _desc(ema, D=100)
    assert rc == ema.EMA_ERR_SHAPE
    rc, _ = _desc(ema, k=0x10008)
    assert rc == ema.EMA_ERR_INVALID_ARG and "aligned" in ema.last_error()
    rc, _ = _desc(ema, cap=0)
    assert rc == ema.EMA_ERR_SHAPE


def test_workspace_size_scales_with_shape(ema):
    a = ema.decode_workspace_size(32, 32, 8, 128, 8192)
    b = ema.decode_workspace_size(1, 16, 8, 128, 1024)
    assert a > b > 0
    with pytest.raises(ema.EmaError) as e:
        ema.decode_workspace_size(1, 12, 8, 128, 1024)
    assert e.value.code == ema.EMA_ERR_SHAPE and "multiple" in e.value.msg


def test_decode_argument_errors(ema):
    L = ema.lib()
    _, d = _desc(ema)
    good = 0x40000
    # GQA mapping needs n_heads % n_kv_heads == 0
    rc = L.ema_decode_attention(None, good, ctypes.byref(d), good, 64, 12, 0.088, good, good, 1 << 30)
    assert rc == ema.EMA_ERR_SHAPE
    # max_len beyond the static capacity (decode_compiled.rs:18-20 overflow guard)
    rc = L.ema_decode_attention(None, good, ctypes.byref(d), good, 65, 16, 0.088, good, good, 1 << 30)
    assert rc == ema.EMA_ERR_CAPACITY and "capacity" in ema.last_error()
    # workspace too small
    rc = L.ema_decode_attention(None, good, ctypes.byref(d), good, 64, 16, 0.088, good, good, 16)
    assert rc == ema.EMA_ERR_WORKSPACE and "workspace" in ema.last_error()
    # null q
    rc = L.ema_decode_attention(None, None, ctypes.byref(d), good, 64, 16, 0.088, good, good, 1 << 30)
    assert rc == ema.EMA_ERR_INVALID_ARG
    # null descriptor
    rc = L.ema_decode_attention(None, good, None, good, 64, 16, 0.088, good, good, 1 << 30)
    assert rc == ema.EMA_ERR_INVALID_ARG


def test_decode_size_limits(ema):
    """Shapes past the kernels' index ranges are refused before any launch: a tile count
    (batch * kv heads * ceil(capacity / 32)) of 2^31 - 1 or more, and a (sequence, kv head)
    plane of a bf16 cache over 4 GiB (addressed through a 32-bit buffer range)."""
    L = ema.lib()
    good = 0x40000
    # bf16, capacity 2^24 + 32: one plane is (2^24 + 32) * 256 bytes > 4 GiB
    rc, d = _desc(ema, B=1, Hkv=1, cap=(1 << 24) + 32)
    assert rc == ema.EMA_OK
    rc = L.ema_decode_attention(None, good, ctypes.byref(d), good, 64, 1, 0.088, good, good, 1 << 30)
    assert rc == ema.EMA_ERR_UNSUPPORTED and "2^32" in ema.last_error()
    # capacity 2^31 - 32 (2^26 - 1 tiles per plane) over 40 sequence x kv-head planes
    rc, d = _desc(ema, B=5, Hkv=8, cap=(1 << 31) - 32)
    assert rc == ema.EMA_OK
    rc = L.ema_decode_attention(None, good, ctypes.byref(d), good, 64, 8, 0.088, good, good, 1 << 30)
    assert rc == ema.EMA_ERR_UNSUPPORTED and "tiles" in ema.last_error()


def test_pre_attention_argument_errors(ema):
    L = ema.lib()
    _, d = _desc(ema)
    g = 0x40000
    # norm weights required unless NO_NORM
    rc = L.ema_pre_attention(None, g, None, None, 1e-6, 1e6, g, 2, 4, 16, 8, 128, 0, g, ctypes.byref(d))
    assert rc == ema.EMA_ERR_INVALID_ARG and "norm" in ema.last_error()
    # batch mismatch with the cache
    rc = L.ema_pre_attention(None, g, g, g, 1e-6, 1e6, g, 3, 4, 16, 8, 128, 0, g, ctypes.byref(d))
    assert rc == ema.EMA_ERR_SHAPE
    # more tokens than the static capacity
    rc = L.ema_pre_attention(None, g, g, g, 1e-6, 1e6, g, 2, 65, 16, 8, 128, 0, g, ctypes.byref(d))
    assert rc == ema.EMA_ERR_CAPACITY and "overflow" in ema.last_error()
    # unknown flag bits
    rc = L.ema_pre_attention(None, g, g, g, 1e-6, 1e6, g, 2, 4, 16, 8, 128, 32, g, ctypes.byref(d))
    assert rc == ema.EMA_ERR_INVALID_ARG and "flags" in ema.last_error()
    # one norm switched off: only that weight may be null
    # (batch 3 against the cache's 2: a call that passes the norm check stops at the shape
    # check, before any launch)
    no_q, no_k = ema.EMA_PRE_NO_Q_NORM, ema.EMA_PRE_NO_K_NORM
    rc = L.ema_pre_attention(None, g, None, g, 1e-6, 1e6, g, 3, 4, 16, 8, 128, no_q, g, ctypes.byref(d))
    assert rc == ema.EMA_ERR_SHAPE
    rc = L.ema_pre_attention(None, g, g, None, 1e-6, 1e6, g, 3, 4, 16, 8, 128, no_k, g, ctypes.byref(d))
    assert rc == ema.EMA_ERR_SHAPE
    rc = L.ema_pre_attention(None, g, g, None, 1e-6, 1e6, g, 3, 4, 16, 8, 128, no_q, g, ctypes.byref(d))
    assert rc == ema.EMA_ERR_INVALID_ARG and "norm" in ema.last_error()
    rc = L.ema_pre_attention(None, g, None, g, 1e-6, 1e6, g, 3, 4, 16, 8, 128, no_k, g, ctypes.byref(d))
    assert rc == ema.EMA_ERR_INVALID_ARG and "norm" in ema.last_error()


def test_decode_step_argument_errors(ema):
    L = ema.lib()
    _, d = _desc(ema)
    g = 0x40000
    rc = L.ema_decode_step(None, g, None, None, 1e-6, 1e6, g, 64, 16, 0, 0.088, ctypes.byref(d), g, g, 1 << 30)
    assert rc == ema.EMA_ERR_INVALID_ARG and "norm" in ema.last_error()
    rc = L.ema_decode_step(None, g, g, g, 1e-6, 1e6, g, 65, 16, 0, 0.088, ctypes.byref(d), g, g, 1 << 30)
    assert rc == ema.EMA_ERR_CAPACITY
    rc = L.ema_decode_step(None, g, g, g, 1e-6, 1e6, g, 64, 16, 0, 0.088, ctypes.byref(d), g, g, 8)
    assert rc == ema.EMA_ERR_WORKSPACE
    rc = L.ema_decode_step(None, g, g, g, 1e-6, 1e6, g, 64, 12, 0, 0.088, ctypes.byref(d), g, g, 1 << 30)
    assert rc == ema.EMA_ERR_SHAPE


def test_decode_step_noalloc_argument_errors(ema):
    """The allocation-free step validates like ema_decode_step, and a shape whose split
    workspace exceeds the static scratch is refused on the host (no HIP call)."""
    L = ema.lib()
    _, d = _desc(ema)
    g = 0x40000
    rc = L.ema_decode_step_noalloc(None, g, None, None, 1e-6, 1e6, g, 64, 16, 0, 0.088, ctypes.byref(d), g)
    assert rc == ema.EMA_ERR_INVALID_ARG and "norm" in ema.last_error()
    rc = L.ema_decode_step_noalloc(None, g, g, g, 1e-6, 1e6, g, 65, 16, 0, 0.088, ctypes.byref(d), g)
    assert rc == ema.EMA_ERR_CAPACITY
    rc = L.ema_decode_step_noalloc(None, g, g, g, 1e-6, 1e6, g, 64, 12, 0, 0.088, ctypes.byref(d), g)
    assert rc == ema.EMA_ERR_SHAPE
    # batch 1024 x 8 kv heads x 16 q heads each: the split state needs far more than 8 MiB
    _, big = _desc(ema, B=1024, Hkv=8, cap=4096)
    need = ctypes.c_uint64()
    assert L.ema_decode_workspace_size(1024, 128, 8, 128, 4096, ctypes.byref(need)) == 0
    assert need.value > (8 << 20)
    rc = L.ema_decode_step_noalloc(None, g, g, g, 1e-6, 1e6, g, 4096, 128, 0, 0.088, ctypes.byref(big), g)
    assert rc == ema.EMA_ERR_WORKSPACE and "static scratch" in ema.last_error()


def test_step_advance_flag_belongs_to_the_decode_step(ema):
    """EMA_STEP_ADVANCE passes the decode step's flag check (the call then fails later, on
    its missing workspace, without touching the GPU) and is an unknown flag elsewhere."""
    L = ema.lib()
    _, d = _desc(ema)
    g = 0x40000
    adv = ema.EMA_STEP_ADVANCE
    rc = L.ema_decode_step(None, g, g, g, 1e-6, 1e6, g, 64, 16, adv, 0.088, ctypes.byref(d), g, None, 0)
    assert rc == ema.EMA_ERR_WORKSPACE
    rc = L.ema_decode_step(None, g, g, g, 1e-6, 1e6, g, 64, 16, 32, 0.088, ctypes.byref(d), g, None, 0)
    assert rc == ema.EMA_ERR_INVALID_ARG and "flags" in ema.last_error()
    rc = L.ema_pre_attention(None, g, g, g, 1e-6, 1e6, g, 2, 1, 16, 4, 128, adv, g, ctypes.byref(d))
    assert rc == ema.EMA_ERR_INVALID_ARG and "flags" in ema.last_error()


def test_prefill_argument_errors(ema):
    L = ema.lib()
    _, d = _desc(ema)
    g = 0x40000
    rc = L.ema_prefill_attention(None, g, ctypes.byref(d), g, 0, 16, 0.088, 1, g)
    assert rc == ema.EMA_ERR_SHAPE
    rc = L.ema_prefill_attention(None, g, ctypes.byref(d), g, 65, 16, 0.088, 1, g)
    assert rc == ema.EMA_ERR_CAPACITY
    rc = L.ema_prefill_attention(None, g, ctypes.byref(d), g, 8, 16, 0.088, 4, g)
    assert rc == ema.EMA_ERR_INVALID_ARG
    rc = L.ema_prefill_attention(None, g, ctypes.byref(d), g, 8, 16, -1.0, 1, g)
    assert rc == ema.EMA_ERR_INVALID_ARG


def test_errors_are_thread_local(ema):
    import threading

    L = ema.lib()
    _, d = _desc(ema)
    L.ema_prefill_attention(None, 0x40000, ctypes.byref(d), 0x40000, 0, 16, 0.088, 1, 0x40000)
    main_msg = ema.last_error()
    seen = {}

    def worker():
        seen["msg"] = ema.last_error()

    t = threading.Thread(target=worker)
    t.start()
    t.join()
    assert main_msg and seen["msg"] == ""


def test_fp8_descriptor_and_memory_bytes(ema):
    L = ema.lib()
    d = ema.KvCacheDesc()
    rc = L.ema_kvcache_init_fp8(ctypes.byref(d), 0x10000, 0x20000, 0x30000, 0x40000, 2, 8, 64, 128, 0)
    assert rc == ema.EMA_OK
    assert d.dtype == ema.EMA_DTYPE_FP8_E4M3 and (d.stride_pos, d.stride_head) == (128, 64 * 128)
    n = ctypes.c_uint64()
    assert L.ema_kvcache_memory_bytes(ctypes.byref(d), ctypes.byref(n)) == 0
    assert n.value == 2 * 2 * 8 * 64 * (128 + 2)  # codes + one exponent byte per 64 values
    # exponents are required; head_dim 128 only
    rc = L.ema_kvcache_init_fp8(ctypes.byref(d), 0x10000, 0x20000, None, 0x40000, 2, 8, 64, 128, 0)
    assert rc == ema.EMA_ERR_INVALID_ARG and "exponent" in ema.last_error()
    rc = L.ema_kvcache_init_fp8(ctypes.byref(d), 0x10000, 0x20000, 0x30000, 0x40000, 2, 8, 64, 64, 0)
    assert rc == ema.EMA_ERR_UNSUPPORTED


def test_fp8_prefill_is_unsupported(ema):
    L = ema.lib()
    d = ema.KvCacheDesc()
    assert L.ema_kvcache_init_fp8(ctypes.byref(d), 0x10000, 0x20000, 0x30000, 0x40000, 2, 8, 64, 128, 0) == 0
    g = 0x40000
    rc = L.ema_prefill_attention(None, g, ctypes.byref(d), g, 8, 16, 0.088, 1, g)
    assert rc == ema.EMA_ERR_UNSUPPORTED and "fp8" in ema.last_error()


def test_pre_attention_ws_and_rows_decoded_flag(ema):
    """ema_pre_attention_ws takes FP8 caches only and the prefill workspace of its max_kv_len;
    EMA_PREFILL_ROWS_DECODED is an ema_prefill_attention_ws flag for FP8 caches."""
    L = ema.lib()
    g = 0x40000
    d8 = ema.KvCacheDesc()
    assert L.ema_kvcache_init_fp8(ctypes.byref(d8), 0x10000, 0x20000, 0x30000, 0x40000, 2, 8, 64, 128, 0) == 0
    n = ctypes.c_uint64()
    assert L.ema_prefill_workspace_size(ctypes.byref(d8), 64, ctypes.byref(n)) == 0
    args = (None, g, g, g, 1e-6, 1e6, g, 2, 8, 16, 8, 128, 0, g)
    # a bf16 cache has no prefill copy
    _, d16 = _desc(ema)
    rc = L.ema_pre_attention_ws(*args, ctypes.byref(d16), 64, g, 1 << 30)
    assert rc == ema.EMA_ERR_UNSUPPORTED and "FP8" in ema.last_error()
    # the workspace of the same max_kv_len, no smaller
    rc = L.ema_pre_attention_ws(*args, ctypes.byref(d8), 64, g, n.value - 16)
    assert rc == ema.EMA_ERR_WORKSPACE and "workspace" in ema.last_error()
    # max_kv_len below the chunk
    rc = L.ema_pre_attention_ws(*args, ctypes.byref(d8), 4, g, n.value)
    assert rc == ema.EMA_ERR_CAPACITY
    # the flag: FP8 caches through the workspace entry only
    rows = ema.EMA_PREFILL_ROWS_DECODED
    rc = L.ema_prefill_attention_ws(None, g, ctypes.byref(d16), g, 8, 16, 0.088, 1 | rows, g, 64, g, 1 << 30)
    assert rc == ema.EMA_ERR_INVALID_ARG and "ROWS_DECODED" in ema.last_error()
    rc = L.ema_prefill_attention(None, g, ctypes.byref(d16), g, 8, 16, 0.088, 1 | rows, g)
    assert rc == ema.EMA_ERR_INVALID_ARG and "flags" in ema.last_error()


def test_unknown_dtype_is_rejected(ema):
    rc, d = _desc(ema)
    d.dtype = 7
    n = ctypes.c_uint64()
    assert ema.lib().ema_kvcache_memory_bytes(ctypes.byref(d), ctypes.byref(n)) == ema.EMA_ERR_INVALID_ARG


def test_prefill_workspace_size_and_errors(ema):
    L = ema.lib()
    n = ctypes.c_uint64()
    _, d16 = _desc(ema)
    assert L.ema_prefill_workspace_size(ctypes.byref(d16), 64, ctypes.byref(n)) == 0 and n.value == 0
    d8 = ema.KvCacheDesc()
    assert L.ema_kvcache_init_fp8(ctypes.byref(d8), 0x10000, 0x20000, 0x30000, 0x40000, 2, 8, 64, 128, 0) == 0
    assert L.ema_prefill_workspace_size(ctypes.byref(d8), 48, ctypes.byref(n)) == 0
    assert n.value == 2 * 2 * 8 * 48 * 128 * 2  # bf16 K and V copies of 48 rows
    assert L.ema_prefill_workspace_size(ctypes.byref(d8), 65, ctypes.byref(n)) == ema.EMA_ERR_CAPACITY
    g = 0x40000
    # workspace too small, max_kv_len below n_tokens
    rc = L.ema_prefill_attention_ws(None, g, ctypes.byref(d8), g, 8, 16, 0.088, 1, g, 48, g, 16)
    assert rc == ema.EMA_ERR_WORKSPACE and "workspace" in ema.last_error()
    rc = L.ema_prefill_attention_ws(None, g, ctypes.byref(d8), g, 8, 16, 0.088, 1, g, 4, g, 1 << 30)
    assert rc == ema.EMA_ERR_CAPACITY


def test_gdn_scan_argument_errors(ema):
    L = ema.lib()
    p = 0x40000  # 16-byte aligned stand-in; every call below fails validation before any HIP call

    def call(q=p, k=p, v=p, g=p, beta=p, state=p, y=p, B=2, T=3, hk=2, hv=4, dk=128, dv=32, dtype=ema.EMA_DTYPE_BF16):
        return L.ema_gdn_scan(None, q, k, v, g, beta, state, y, B, T, hk, hv, dk, dv, dtype)

    assert call(state=None) == ema.EMA_ERR_INVALID_ARG and "null" in ema.last_error()
    assert call(dtype=ema.EMA_DTYPE_FP8_E4M3) == ema.EMA_ERR_INVALID_ARG
    assert call(T=0) == ema.EMA_ERR_SHAPE
    assert call(hv=6, hk=4) == ema.EMA_ERR_SHAPE and "multiple of hk" in ema.last_error()
    assert call(dk=96) == ema.EMA_ERR_UNSUPPORTED
    assert call(dv=24) == ema.EMA_ERR_SHAPE
    assert call(state=p + 4) == ema.EMA_ERR_INVALID_ARG and "misaligned" in ema.last_error()
    assert call(q=p + 8) == ema.EMA_ERR_INVALID_ARG
    assert call(v=p + 2, dtype=ema.EMA_DTYPE_F32) == ema.EMA_ERR_INVALID_ARG


def test_gdn_scan_workspace_size_and_errors(ema):
    L = ema.lib()
    n = ctypes.c_uint64()
    # per 32-token chunk: batch * (hv * (128 (dk + dv) + 5120) + hk * 128 dk)
    assert L.ema_gdn_scan_workspace_size(1, 2048, 16, 32, 128, 128, ctypes.byref(n)) == 0
    assert n.value == 64 * (32 * (128 * 256 + 5120) + 16 * 128 * 128)
    assert L.ema_gdn_scan_workspace_size(2, 33, 2, 4, 64, 48, ctypes.byref(n)) == 0
    assert n.value == 2 * 2 * (4 * (128 * 112 + 5120) + 2 * 128 * 64)
    assert L.ema_gdn_scan_workspace_size(1, 64, 2, 4, 96, 32, ctypes.byref(n)) == ema.EMA_ERR_UNSUPPORTED
    assert n.value == 0
    assert L.ema_gdn_scan_workspace_size(1, 64, 3, 4, 64, 32, ctypes.byref(n)) == ema.EMA_ERR_SHAPE
    assert L.ema_gdn_scan_workspace_size(1, 64, 2, 4, 64, 32, None) == ema.EMA_ERR_INVALID_ARG
    p = 0x40000  # 16-byte aligned stand-in; every call below fails before any HIP call
    L.ema_gdn_scan_workspace_size(1, 64, 2, 4, 128, 32, ctypes.byref(n))
    per_chunk = n.value // 2

    def call(ws=p, nbytes=n.value, T=64, dtype=ema.EMA_DTYPE_BF16, **kw):
        a = dict(q=p, k=p, v=p, g=p, beta=p, state=p, y=p)
        a.update(kw)
        return L.ema_gdn_scan_ws(None, a["q"], a["k"], a["v"], a["g"], a["beta"], a["state"], a["y"], 1, T, 2, 4,
                                 128, 32, dtype, ws, nbytes)

    assert call(state=None) == ema.EMA_ERR_INVALID_ARG  # the ema_gdn_scan checks come first
    assert call(ws=None) == ema.EMA_ERR_WORKSPACE
    assert call(ws=p + 8) == ema.EMA_ERR_WORKSPACE and "aligned" in ema.last_error()
    assert call(nbytes=per_chunk - 16) == ema.EMA_ERR_WORKSPACE and "one chunk" in ema.last_error()


def test_rotating_flag_is_validated(ema):
    L = ema.lib()
    rc, d = _desc(ema)
    d.flags = 2  # unknown flag
    n = ctypes.c_uint64()
    assert L.ema_kvcache_memory_bytes(ctypes.byref(d), ctypes.byref(n)) == ema.EMA_ERR_INVALID_ARG
    assert "flags" in ema.last_error()
    d.flags = ema.EMA_KV_ROTATING
    assert L.ema_kvcache_memory_bytes(ctypes.byref(d), ctypes.byref(n)) == 0
    d8 = ema.KvCacheDesc()
    assert L.ema_kvcache_init_fp8(ctypes.byref(d8), 0x10000, 0x20000, 0x30000, 0x40000, 2, 8, 64, 128, 0) == 0
    d8.flags = ema.EMA_KV_ROTATING
    g = 0x40000
    # a rotating fp8 cache is accepted by the prefill (stopped here by the too-small
    # workspace, before any launch)
    rc = L.ema_prefill_attention_ws(None, g, ctypes.byref(d8), g, 8, 16, 0.088, 1, g, 48, g, 16)
    assert rc == ema.EMA_ERR_WORKSPACE, ema.last_error()
    # the bf16 copy of a ring holds the whole ring whatever max_kv_len says (wrapped positions
    # sit at row p % capacity); a static fp8 cache's copy holds max_kv_len rows
    assert L.ema_prefill_workspace_size(ctypes.byref(d8), 48, ctypes.byref(n)) == 0
    assert n.value == 2 * 2 * 8 * 64 * 128 * 2
    need = n.value
    rc = L.ema_prefill_attention_ws(None, g, ctypes.byref(d8), g, 8, 16, 0.088, 1, g, 48, g, need - 16)
    assert rc == ema.EMA_ERR_WORKSPACE and str(need) in ema.last_error()
    d8.flags = 0
    assert L.ema_prefill_workspace_size(ctypes.byref(d8), 48, ctypes.byref(n)) == 0
    assert n.value == 2 * 2 * 8 * 48 * 128 * 2


def test_quantized_matmul_argument_errors(ema):
    L = ema.lib()
    p = 0x40000  # 16-byte aligned stand-in; every failing call below stops before any HIP call

    def call(x=p, ldx=4096, w=p, s=p, b=p, y=p, ldy=6144, M=4, N=6144, K=4096, gs=64, bits=4,
             dtype=ema.EMA_DTYPE_BF16):
        return L.ema_quantized_matmul(None, x, ldx, w, s, b, y, ldy, M, N, K, gs, bits, dtype)

    assert call(M=0, x=None, w=None) == ema.EMA_OK  # empty batch: no-op
    assert call(w=None) == ema.EMA_ERR_INVALID_ARG and "null" in ema.last_error()
    assert call(M=-1) == ema.EMA_ERR_SHAPE
    assert call(N=0) == ema.EMA_ERR_SHAPE
    assert call(dtype=ema.EMA_DTYPE_F32) == ema.EMA_ERR_INVALID_ARG
    assert call(bits=3) == ema.EMA_ERR_UNSUPPORTED and "bits" in ema.last_error()
    assert call(gs=16) == ema.EMA_ERR_UNSUPPORTED and "group_size" in ema.last_error()
    assert call(K=4000) == ema.EMA_ERR_SHAPE and "multiple" in ema.last_error()
    assert call(ldx=2048) == ema.EMA_ERR_SHAPE
    assert call(ldy=100) == ema.EMA_ERR_SHAPE
    assert call(x=p + 8) == ema.EMA_ERR_INVALID_ARG and "misaligned" in ema.last_error()
    assert call(ldx=4100) == ema.EMA_ERR_INVALID_ARG
    assert call(s=p + 1) == ema.EMA_ERR_INVALID_ARG
    assert call(K=1 << 21, ldx=1 << 21) == ema.EMA_ERR_SHAPE and "too large" in ema.last_error()


def test_int4_cache_descriptor_and_errors(ema):
    L = ema.lib()
    a = 0x40000  # 16-byte aligned stand-ins; no call below reaches HIP
    d = ema.KvCacheDesc()
    assert L.ema_kvcache_init_int4(ctypes.byref(d), a, a, a, a, a, a, 2, 8, 64, 128) == 0
    assert d.dtype == ema.EMA_DTYPE_INT4_AFFINE and d.stride_pos == 128 and d.stride_head == 64 * 128
    n = ctypes.c_uint64()
    assert L.ema_kvcache_memory_bytes(ctypes.byref(d), ctypes.byref(n)) == 0
    assert n.value == 2 * 2 * 8 * 64 * (64 + 2 * 2 * 2)  # K and V: 64 bytes of codes + 2 scales + 2 biases per row
    # capacity not a multiple of 32, head_dim 64, a missing bias buffer, a misaligned scale buffer
    assert L.ema_kvcache_init_int4(ctypes.byref(d), a, a, a, a, a, a, 2, 8, 48, 128) == ema.EMA_ERR_UNSUPPORTED
    assert "multiple of 32" in ema.last_error()
    assert L.ema_kvcache_init_int4(ctypes.byref(d), a, a, a, a, a, a, 2, 8, 64, 64) == ema.EMA_ERR_UNSUPPORTED
    assert L.ema_kvcache_init_int4(ctypes.byref(d), a, a, a, None, a, a, 2, 8, 64, 128) == ema.EMA_ERR_INVALID_ARG
    assert L.ema_kvcache_init_int4(ctypes.byref(d), a, a, a + 2, a, a, a, 2, 8, 64, 128) == ema.EMA_ERR_INVALID_ARG
    assert L.ema_kvcache_init_int4(ctypes.byref(d), a, a, a, a, a, a, 2, 8, 64, 128) == 0
    d.flags = ema.EMA_KV_ROTATING  # int4 rings are accepted
    assert L.ema_kvcache_memory_bytes(ctypes.byref(d), ctypes.byref(n)) == 0
    d.flags = 0
    # prefill over int4 is rejected by both entries
    assert L.ema_prefill_attention(None, a, ctypes.byref(d), a, 8, 16, 0.088, 1, a) == ema.EMA_ERR_UNSUPPORTED
    assert "int4" in ema.last_error()
    rc = L.ema_prefill_attention_ws(None, a, ctypes.byref(d), a, 8, 16, 0.088, 1, a, 48, a, 1 << 30)
    assert rc == ema.EMA_ERR_UNSUPPORTED and "int4" in ema.last_error()
    # the converter: bf16 source and int4 destination of one shape, rows inside both capacities
    s = ema.KvCacheDesc()
    assert L.ema_kvcache_init(ctypes.byref(s), a, a, 2, 8, 40, 128) == 0
    assert L.ema_kvcache_quantize_int4(None, ctypes.byref(s), 0, ctypes.byref(d), 0, 0) == 0  # nothing to do
    assert L.ema_kvcache_quantize_int4(None, ctypes.byref(s), 0, ctypes.byref(d), 30, 41) == ema.EMA_ERR_CAPACITY
    assert L.ema_kvcache_quantize_int4(None, ctypes.byref(s), 8, ctypes.byref(d), 60, 8) == ema.EMA_ERR_CAPACITY
    assert L.ema_kvcache_quantize_int4(None, ctypes.byref(d), 0, ctypes.byref(d), 0, 8) == ema.EMA_ERR_INVALID_ARG
    s2 = ema.KvCacheDesc()
    assert L.ema_kvcache_init(ctypes.byref(s2), a, a, 2, 4, 40, 128) == 0
    assert L.ema_kvcache_quantize_int4(None, ctypes.byref(s2), 0, ctypes.byref(d), 0, 8) == ema.EMA_ERR_SHAPE


def test_kvcache_convert_argument_errors(ema):
    L = ema.lib()
    a = 0x40000  # 16-byte aligned stand-ins; no call below reaches HIP
    bf = ema.KvCacheDesc()
    assert L.ema_kvcache_init(ctypes.byref(bf), a, a, 2, 8, 40, 128) == 0
    f8 = ema.KvCacheDesc()
    assert L.ema_kvcache_init_fp8(ctypes.byref(f8), a, a, a, a, 2, 8, 64, 128, 0) == 0
    i4 = ema.KvCacheDesc()
    assert L.ema_kvcache_init_int4(ctypes.byref(i4), a, a, a, a, a, a, 2, 8, 64, 128) == 0
    # zero rows of every supported pair is a no-op
    for s, d in ((bf, f8), (f8, bf), (bf, i4)):
        assert L.ema_kvcache_convert(None, ctypes.byref(s), 0, ctypes.byref(d), 0, 0) == 0
    # unsupported pairs: same dtype, fp8 <-> int4, int4 -> bf16
    for s, d in ((bf, bf), (f8, f8), (f8, i4), (i4, bf), (i4, f8)):
        assert L.ema_kvcache_convert(None, ctypes.byref(s), 0, ctypes.byref(d), 0, 4) == ema.EMA_ERR_UNSUPPORTED
    assert "converts" in ema.last_error()
    # rows outside either capacity, negative rows
    assert L.ema_kvcache_convert(None, ctypes.byref(bf), 0, ctypes.byref(f8), 30, 41) == ema.EMA_ERR_CAPACITY
    assert L.ema_kvcache_convert(None, ctypes.byref(bf), 8, ctypes.byref(f8), 0, 33) == ema.EMA_ERR_CAPACITY
    assert L.ema_kvcache_convert(None, ctypes.byref(f8), 60, ctypes.byref(bf), 0, 8) == ema.EMA_ERR_CAPACITY
    assert L.ema_kvcache_convert(None, ctypes.byref(bf), -1, ctypes.byref(f8), 0, 4) == ema.EMA_ERR_CAPACITY
    assert L.ema_kvcache_convert(None, ctypes.byref(bf), 0, ctypes.byref(f8), 0, -4) == ema.EMA_ERR_CAPACITY
    # shapes must agree; null or empty descriptors are rejected
    b4 = ema.KvCacheDesc()
    assert L.ema_kvcache_init(ctypes.byref(b4), a, a, 2, 4, 40, 128) == 0
    assert L.ema_kvcache_convert(None, ctypes.byref(b4), 0, ctypes.byref(f8), 0, 4) == ema.EMA_ERR_SHAPE
    assert "shapes differ" in ema.last_error()
    assert L.ema_kvcache_convert(None, None, 0, ctypes.byref(f8), 0, 4) == ema.EMA_ERR_INVALID_ARG
    empty = ema.KvCacheDesc()
    assert L.ema_kvcache_convert(None, ctypes.byref(bf), 0, ctypes.byref(empty), 0, 4) == ema.EMA_ERR_INVALID_ARG


def test_position_write_argument_errors(ema):
    L = ema.lib()
    assert L.ema_position_write(None, None, 5) == ema.EMA_ERR_INVALID_ARG
    assert "null" in ema.last_error()
    assert L.ema_position_write(None, 0x40002, 5) == ema.EMA_ERR_INVALID_ARG
    assert "aligned" in ema.last_error()


def test_fp8_rope_tail_descriptor(ema):
    """n_rot = 64 (the reference's Fp8Cache::new(128, 64)): rows of 64 codes + 64 bf16."""
    L = ema.lib()
    a = 0x40000
    d = ema.KvCacheDesc()
    assert L.ema_kvcache_init_fp8(ctypes.byref(d), a, a, a, a, 2, 8, 64, 128, 64) == 0
    assert d.n_rot == 64 and d.stride_pos == 192 and d.stride_head == 64 * 192 and d.stride_batch == 8 * 64 * 192
    n = ctypes.c_uint64()
    assert L.ema_kvcache_memory_bytes(ctypes.byref(d), ctypes.byref(n)) == 0
    assert n.value == 2 * 2 * 8 * 64 * (192 + 2)
    for bad in (32, 96, 128, -64):
        assert L.ema_kvcache_init_fp8(ctypes.byref(d), a, a, a, a, 2, 8, 64, 128, bad) == ema.EMA_ERR_UNSUPPORTED
        assert "n_rot" in ema.last_error()
        assert L.ema_kvcache_alloc_fp8(ctypes.byref(d), 2, 8, 64, 128, bad) == ema.EMA_ERR_UNSUPPORTED
    # rows too short for the tail; the field on another dtype
    assert L.ema_kvcache_init_fp8(ctypes.byref(d), a, a, a, a, 2, 8, 64, 128, 64) == 0
    d.stride_pos = 128
    n2 = ctypes.c_uint64()
    assert L.ema_kvcache_memory_bytes(ctypes.byref(d), ctypes.byref(n2)) == ema.EMA_ERR_SHAPE
    assert "stride_pos" in ema.last_error()
    b = ema.KvCacheDesc()
    assert L.ema_kvcache_init(ctypes.byref(b), a, a, 2, 8, 64, 128) == 0
    b.n_rot = 64
    assert L.ema_kvcache_memory_bytes(ctypes.byref(b), ctypes.byref(n2)) == ema.EMA_ERR_INVALID_ARG
