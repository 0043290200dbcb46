//! Rust binding of `libema_attn`, the MI355X (gfx950) attention path of engine-mlx.
//!
//! Three layers:
//! - [`sys`]: the C ABI of `include/ema_attn.h`, declared by hand (every export, every
//!   constant, the `ema_kvcache_desc` layout);
//! - [`hip`]: the few HIP runtime calls the safe layer needs (device memory and copies);
//! - the safe layer, in the shape of the reference's crates: the `KvCache` trait
//!   (`crates/kvcache/src/lib.rs:52-76`) and `HipKvCache`, the caches the kernels work on
//!   in place: a static pre-allocated cache (the serve crate's `kv_bufs` +
//!   `static_offsets`, `crates/serve/src/engine_ext.rs:266-306`), `RotatingCache`
//!   (`crates/kvcache/src/rotating.rs`, as a ring) and `Fp8Cache`
//!   (`crates/kvcache/src/fp8.rs`, stored as codes + block exponents);
//!   `QuantWeights` (`crates/ops/src/quant.rs:16-40`), `GqaConfig` / `GqaWeights` /
//!   `gqa_attention` (`crates/attention/src/gqa.rs:27-107`) and
//!   `sliding_window_attention` (`crates/attention/src/sliding_window.rs:40-50`), both
//!   generic over the cache as the reference's are.
//!
//! Arrays are device buffers ([`DeviceArray`]) instead of `mlx_array` handles, and the
//! context ([`HipCtx`]) carries the HIP stream and a caller-sized device arena instead of
//! MLX's stream and allocator: `gqa_attention` allocates nothing per call.
//! Errors keep the reference's shape: `ema op '<op>' failed with code <n>: <message>`
//! (`MlxCtx::check`, `crates/mlx-ffi/src/ops/real/mod.rs:35-40`), and the reference's
//! texts where it has them ("KV cache is empty", "static KV overflow offset=.. cap=..").

use std::ffi::{c_char, c_void, CStr};

use anyhow::{bail, Result};

/// The C ABI of `include/ema_attn.h`.
pub mod sys {
    use std::ffi::{c_char, c_void};

    /// `hipStream_t`; null is the default stream.
    pub type EmaStream = *mut c_void;

    pub const EMA_OK: i32 = 0;
    pub const EMA_ERR_INVALID_ARG: i32 = -1;
    pub const EMA_ERR_SHAPE: i32 = -2;
    pub const EMA_ERR_CAPACITY: i32 = -3;
    pub const EMA_ERR_WORKSPACE: i32 = -4;
    pub const EMA_ERR_UNSUPPORTED: i32 = -5;
    pub const EMA_ERR_HIP: i32 = -6;

    pub const EMA_DTYPE_BF16: i32 = 1;
    pub const EMA_DTYPE_FP8_E4M3: i32 = 2;
    pub const EMA_DTYPE_F16: i32 = 3;
    pub const EMA_DTYPE_F32: i32 = 4;
    pub const EMA_DTYPE_INT4_AFFINE: i32 = 5;

    /// `EmaKvCacheDesc::flags`: a ring of `capacity` rows (position p in row p % capacity).
    pub const EMA_KV_ROTATING: i32 = 1;

    /// `ema_pre_attention` / decode-step flags.
    pub const EMA_PRE_NO_NORM: u32 = 1;
    pub const EMA_PRE_NO_ROPE: u32 = 2;
    pub const EMA_STEP_ADVANCE: u32 = 4;
    pub const EMA_PRE_NO_Q_NORM: u32 = 8;
    pub const EMA_PRE_NO_K_NORM: u32 = 16;

    /// `ema_prefill_attention` flags.
    pub const EMA_PREFILL_CAUSAL: u32 = 1;
    pub const EMA_PREFILL_CHUNK_ONLY: u32 = 2;
    pub const EMA_PREFILL_ROWS_DECODED: u32 = 4;

    /// Arrival counters at the start of every decode workspace: zero before its first use;
    /// every call leaves them at zero.
    pub const EMA_DECODE_COUNTER_BYTES: u64 = 131072;

    /// Size of the static scratch behind `ema_decode_step_noalloc` (per device).
    pub const EMA_NOALLOC_SCRATCH_BYTES: u64 = 8 << 20;

    /// `ema_kvcache_desc`: one layer's K/V, logical shape [batch, n_kv_heads, capacity,
    /// head_dim], strides in elements.
    #[repr(C)]
    #[derive(Clone, Copy, Debug)]
    pub struct EmaKvCacheDesc {
        pub k: *mut c_void,
        pub v: *mut c_void,
        pub batch: i32,
        pub n_kv_heads: i32,
        pub capacity: i32,
        pub head_dim: i32,
        pub stride_batch: i64,
        pub stride_head: i64,
        pub stride_pos: i64,
        pub dtype: i32,
        pub flags: i32,
        pub k_exp: *mut c_void,
        pub v_exp: *mut c_void,
        pub k_scales: *mut c_void,
        pub k_biases: *mut c_void,
        pub v_scales: *mut c_void,
        pub v_biases: *mut c_void,
        pub n_rot: i32,
    }

    impl Default for EmaKvCacheDesc {
        fn default() -> Self {
            let null = std::ptr::null_mut();
            EmaKvCacheDesc {
                k: null,
                v: null,
                batch: 0,
                n_kv_heads: 0,
                capacity: 0,
                head_dim: 0,
                stride_batch: 0,
                stride_head: 0,
                stride_pos: 0,
                dtype: 0,
                flags: 0,
                k_exp: null,
                v_exp: null,
                k_scales: null,
                k_biases: null,
                v_scales: null,
                v_biases: null,
                n_rot: 0,
            }
        }
    }

    extern "C" {
        pub fn ema_last_error() -> *const c_char;
        pub fn ema_version() -> *const c_char;
        pub fn ema_kvcache_init(desc: *mut EmaKvCacheDesc, k: *mut c_void, v: *mut c_void, batch: i32,
                                n_kv_heads: i32, capacity: i32, head_dim: i32) -> i32;
        pub fn ema_kvcache_alloc(out: *mut EmaKvCacheDesc, batch: i32, n_kv_heads: i32, capacity: i32,
                                 head_dim: i32) -> i32;
        pub fn ema_kvcache_init_fp8(desc: *mut EmaKvCacheDesc, k: *mut c_void, v: *mut c_void,
                                    k_exp: *mut c_void, v_exp: *mut c_void, batch: i32, n_kv_heads: i32,
                                    capacity: i32, head_dim: i32, n_rot: i32) -> i32;
        pub fn ema_kvcache_alloc_fp8(out: *mut EmaKvCacheDesc, batch: i32, n_kv_heads: i32, capacity: i32,
                                     head_dim: i32, n_rot: i32) -> i32;
        pub fn ema_kvcache_init_int4(desc: *mut EmaKvCacheDesc, k: *mut c_void, v: *mut c_void,
                                     k_scales: *mut c_void, k_biases: *mut c_void, v_scales: *mut c_void,
                                     v_biases: *mut c_void, batch: i32, n_kv_heads: i32, capacity: i32,
                                     head_dim: i32) -> i32;
        pub fn ema_kvcache_alloc_int4(out: *mut EmaKvCacheDesc, batch: i32, n_kv_heads: i32, capacity: i32,
                                      head_dim: i32) -> i32;
        pub fn ema_kvcache_quantize_int4(stream: EmaStream, src: *const EmaKvCacheDesc, src_row: i32,
                                         dst: *const EmaKvCacheDesc, dst_row: i32, n_rows: i32) -> i32;
        pub fn ema_kvcache_convert(stream: EmaStream, src: *const EmaKvCacheDesc, src_row: i32,
                                   dst: *const EmaKvCacheDesc, dst_row: i32, n_rows: i32) -> i32;
        pub fn ema_position_write(stream: EmaStream, slot: *mut i32, value: i32) -> i32;
        pub fn ema_kvcache_free(desc: *mut EmaKvCacheDesc) -> i32;
        pub fn ema_kvcache_memory_bytes(desc: *const EmaKvCacheDesc, bytes: *mut u64) -> i32;
        pub fn ema_pre_attention(stream: EmaStream, qkv: *const c_void, q_norm_w: *const c_void,
                                 k_norm_w: *const c_void, eps: f32, theta: f32, offsets: *const i32, batch: i32,
                                 n_tokens: i32, n_heads: i32, n_kv_heads: i32, head_dim: i32, flags: u32,
                                 q_out: *mut c_void, cache: *const EmaKvCacheDesc) -> i32;
        pub fn ema_pre_attention_ws(stream: EmaStream, qkv: *const c_void, q_norm_w: *const c_void,
                                    k_norm_w: *const c_void, eps: f32, theta: f32, offsets: *const i32, batch: i32,
                                    n_tokens: i32, n_heads: i32, n_kv_heads: i32, head_dim: i32, flags: u32,
                                    q_out: *mut c_void, cache: *const EmaKvCacheDesc, max_kv_len: i32,
                                    workspace: *mut c_void, workspace_bytes: u64) -> i32;
        pub fn ema_decode_workspace_size(batch: i32, n_heads: i32, n_kv_heads: i32, head_dim: i32, max_len: i32,
                                         bytes: *mut u64) -> i32;
        pub fn ema_decode_attention(stream: EmaStream, q: *const c_void, cache: *const EmaKvCacheDesc,
                                    lengths: *const i32, max_len: i32, n_heads: i32, scale: f32, out: *mut c_void,
                                    workspace: *mut c_void, workspace_bytes: u64) -> i32;
        pub fn ema_decode_step(stream: EmaStream, qkv: *const c_void, q_norm_w: *const c_void,
                               k_norm_w: *const c_void, eps: f32, theta: f32, offsets: *mut i32, max_len: i32,
                               n_heads: i32, flags: u32, scale: f32, cache: *const EmaKvCacheDesc,
                               out: *mut c_void, workspace: *mut c_void, workspace_bytes: u64) -> i32;
        pub fn ema_decode_step_noalloc(stream: EmaStream, qkv: *const c_void, q_norm_w: *const c_void,
                                       k_norm_w: *const c_void, eps: f32, theta: f32, offsets: *mut i32,
                                       max_len: i32, n_heads: i32, flags: u32, scale: f32,
                                       cache: *const EmaKvCacheDesc, out: *mut c_void) -> i32;
        pub fn ema_prefill_attention(stream: EmaStream, q: *const c_void, cache: *const EmaKvCacheDesc,
                                     q_offsets: *const i32, n_tokens: i32, n_heads: i32, scale: f32, flags: u32,
                                     out: *mut c_void) -> i32;
        pub fn ema_prefill_workspace_size(cache: *const EmaKvCacheDesc, max_kv_len: i32, bytes: *mut u64) -> i32;
        pub fn ema_prefill_attention_ws(stream: EmaStream, q: *const c_void, cache: *const EmaKvCacheDesc,
                                        q_offsets: *const i32, n_tokens: i32, n_heads: i32, scale: f32,
                                        flags: u32, out: *mut c_void, max_kv_len: i32, workspace: *mut c_void,
                                        workspace_bytes: u64) -> i32;
        pub fn ema_gdn_scan(stream: EmaStream, q: *const c_void, k: *const c_void, v: *const c_void,
                            g: *const f32, beta: *const f32, state: *mut f32, y: *mut c_void, batch: i32,
                            n_tokens: i32, hk: i32, hv: i32, dk: i32, dv: i32, dtype: i32) -> i32;
        pub fn ema_gdn_scan_workspace_size(batch: i32, n_tokens: i32, hk: i32, hv: i32, dk: i32, dv: i32,
                                           bytes: *mut u64) -> i32;
        pub fn ema_gdn_scan_ws(stream: EmaStream, q: *const c_void, k: *const c_void, v: *const c_void,
                               g: *const f32, beta: *const f32, state: *mut f32, y: *mut c_void, batch: i32,
                               n_tokens: i32, hk: i32, hv: i32, dk: i32, dv: i32, dtype: i32,
                               workspace: *mut c_void, workspace_bytes: u64) -> i32;
        pub fn ema_quantized_matmul(stream: EmaStream, x: *const c_void, ldx: i64, w: *const u32,
                                    scales: *const c_void, biases: *const c_void, y: *mut c_void, ldy: i64,
                                    m: i32, n: i32, k: i32, group_size: i32, bits: i32, dtype: i32) -> i32;
    }
}

/// The HIP runtime calls the safe layer uses (libamdhip64).
pub mod hip {
    use std::ffi::{c_char, c_int, c_void};

    pub const HIP_SUCCESS: c_int = 0;
    pub const HIP_MEMCPY_HOST_TO_DEVICE: c_int = 1;
    pub const HIP_MEMCPY_DEVICE_TO_DEVICE: c_int = 3;

    extern "C" {
        pub fn hipMalloc(ptr: *mut *mut c_void, size: usize) -> c_int;
        pub fn hipFree(ptr: *mut c_void) -> c_int;
        pub fn hipMemcpy(dst: *mut c_void, src: *const c_void, size: usize, kind: c_int) -> c_int;
        pub fn hipMemset(dst: *mut c_void, value: c_int, size: usize) -> c_int;
        pub fn hipMemcpy2DAsync(dst: *mut c_void, dpitch: usize, src: *const c_void, spitch: usize, width: usize,
                                height: usize, kind: c_int, stream: *mut c_void) -> c_int;
        pub fn hipGetErrorString(err: c_int) -> *const c_char;
    }
}

fn last_error() -> String {
    unsafe { CStr::from_ptr(sys::ema_last_error()) }.to_string_lossy().into_owned()
}

/// 0 = OK, otherwise bail with the op name, the status code and the library's message
/// (the shape of `MlxCtx::check`, `crates/mlx-ffi/src/ops/real/mod.rs:35-40`).
pub fn check(rc: i32, op: &str) -> Result<()> {
    if rc != sys::EMA_OK {
        bail!("ema op '{}' failed with code {}: {}", op, rc, last_error());
    }
    Ok(())
}

fn check_hip(rc: i32, what: &str) -> Result<()> {
    if rc != hip::HIP_SUCCESS {
        let msg = unsafe { CStr::from_ptr(hip::hipGetErrorString(rc)) }.to_string_lossy().into_owned();
        bail!("{}: {}", what, msg);
    }
    Ok(())
}

/// Library version string.
pub fn version() -> String {
    unsafe { CStr::from_ptr(sys::ema_version() as *const c_char) }.to_string_lossy().into_owned()
}

/// A non-owning view of a device tensor (bf16 unless stated): the role of `mlx_array`.
/// `strides` are in elements; empty means contiguous.
#[derive(Clone, Debug)]
pub struct DeviceArray {
    pub data: *mut c_void,
    pub shape: Vec<i64>,
    pub strides: Vec<i64>,
}

impl DeviceArray {
    pub fn new(data: *mut c_void, shape: &[i64]) -> Self {
        DeviceArray { data, shape: shape.to_vec(), strides: Vec::new() }
    }
    pub fn numel(&self) -> i64 {
        self.shape.iter().product()
    }
}

/// The role of `MlxCtx` here: the HIP stream work is enqueued on, and the device arena
/// the layer calls take their temporaries from (sized once with
/// [`gqa_workspace_bytes`]; 256-byte aligned; zero-filled once, because its first
/// `EMA_DECODE_COUNTER_BYTES` hold the decode split's arrival counters, which every call
/// leaves at zero). An array a call returns from the arena is valid until the next call
/// that uses it.
pub struct HipCtx {
    pub stream: sys::EmaStream,
    pub workspace: *mut c_void,
    pub workspace_bytes: usize,
}

impl HipCtx {
    /// A context on `stream` with a zero-filled arena of `workspace_bytes` allocated once.
    pub fn with_workspace(stream: sys::EmaStream, workspace_bytes: usize) -> Result<Self> {
        let mut p: *mut c_void = std::ptr::null_mut();
        check_hip(unsafe { hip::hipMalloc(&mut p, workspace_bytes) }, "HipCtx: workspace")?;
        let ctx = HipCtx { stream, workspace: p, workspace_bytes };
        check_hip(unsafe { hip::hipMemset(p, 0, workspace_bytes) }, "HipCtx: workspace")?;
        Ok(ctx)
    }
}

impl Drop for HipCtx {
    fn drop(&mut self) {
        if !self.workspace.is_null() {
            unsafe { hip::hipFree(self.workspace) };
        }
    }
}

/// KV cache backend trait: the method set of the reference's `KvCache`
/// (`crates/kvcache/src/lib.rs:52-76`) over device arrays.
pub trait KvCache: Send {
    /// Append new K and V, shape [1, n_kv_heads, seq_len, head_dim] (attention order).
    fn append(&mut self, ctx: &HipCtx, k: &DeviceArray, v: &DeviceArray) -> Result<()>;
    /// The full accumulated K and V, [1, n_kv_heads, total_seq, head_dim].
    fn get(&self, ctx: &HipCtx) -> Result<(DeviceArray, DeviceArray)>;
    fn len(&self) -> usize;
    fn is_empty(&self) -> bool {
        self.len() == 0
    }
    fn reset(&mut self);
    fn memory_bytes(&self) -> usize;
}

/// A [`KvCache`] the kernels read and write in place: the generic parameter of the layer
/// functions, as the reference's `gqa_attention<C: KvCache>` (`crates/attention/src/gqa.rs:62-69`)
/// takes any cache (its documented uses pass an `Fp8Cache` or a `RotatingCache`,
/// `crates/attention/src/lib.rs:22-27`). The kernels write a call's new rows through the
/// descriptor and read the first new token's position from device memory.
pub trait HipKvCache: KvCache {
    /// The descriptor the kernels take: buffers, strides, dtype, `EMA_KV_ROTATING`.
    fn desc(&self) -> &sys::EmaKvCacheDesc;
    /// Device pointer to an int32 holding `p`, valid for work enqueued on `ctx.stream`
    /// after this call (a static cache: 0 <= p <= capacity).
    fn position(&self, ctx: &HipCtx, p: i64) -> Result<*const i32>;
    /// The cache now holds the tokens [0, n) (a ring: the last `capacity` of them).
    fn set_len(&mut self, n: i64) -> Result<()>;
    fn rotating(&self) -> bool {
        self.desc().flags & sys::EMA_KV_ROTATING != 0
    }
    fn capacity(&self) -> i32 {
        self.desc().capacity
    }
    fn n_kv_heads(&self) -> i32 {
        self.desc().n_kv_heads
    }
    fn head_dim(&self) -> i32 {
        self.desc().head_dim
    }
}

/// Device table of the int32 values 0, 1, ..., n: the analogue of the pre-built
/// `static_offsets` scalars (`crates/serve/src/engine_ext.rs:293-299`), so a step passes its
/// offset without a host-to-device copy.
struct PositionTable {
    table: *mut i32,
    n: i32,
}

impl PositionTable {
    fn new(n: i32) -> Result<Self> {
        if n < 0 {
            bail!("PositionTable: negative size {}", n);
        }
        let values: Vec<i32> = (0..=n).collect();
        let bytes = values.len() * std::mem::size_of::<i32>();
        let mut p: *mut c_void = std::ptr::null_mut();
        check_hip(unsafe { hip::hipMalloc(&mut p, bytes) }, "position table")?;
        let table = PositionTable { table: p as *mut i32, n }; // freed by Drop on the error path
        check_hip(
            unsafe { hip::hipMemcpy(p, values.as_ptr() as *const c_void, bytes, hip::HIP_MEMCPY_HOST_TO_DEVICE) },
            "position table upload",
        )?;
        Ok(table)
    }

    /// Device pointer to the value p, 0 <= p <= n (`cap` names the cache in the error).
    fn at(&self, p: i64, cap: i32) -> Result<*const i32> {
        if p < 0 || p > self.n as i64 {
            bail!("static KV overflow offset={} cap={}", p, cap);
        }
        Ok(unsafe { self.table.add(p as usize) } as *const i32)
    }
}

impl Drop for PositionTable {
    fn drop(&mut self) {
        if !self.table.is_null() {
            unsafe { hip::hipFree(self.table as *mut c_void) };
        }
    }
}

/// Checks k and v of an append: contiguous [1, n_kv_heads, seq, head_dim], equal lengths.
/// Returns seq.
fn append_len(desc: &sys::EmaKvCacheDesc, k: &DeviceArray, v: &DeviceArray, op: &str) -> Result<i64> {
    let hkv = desc.n_kv_heads as i64;
    let d = desc.head_dim as i64;
    for a in [k, v] {
        if a.data.is_null() {
            bail!("{}: null k/v", op);
        }
        if a.shape.len() != 4 || a.shape[0] != 1 || a.shape[1] != hkv || a.shape[3] != d || !a.strides.is_empty() {
            bail!("{}: expected contiguous [1, {}, seq, {}], got {:?}", op, hkv, d, a.shape);
        }
    }
    if k.shape[2] != v.shape[2] {
        bail!("{}: k/v lengths differ", op);
    }
    Ok(k.shape[2])
}

fn memory_bytes_of(desc: &sys::EmaKvCacheDesc) -> usize {
    let mut b: u64 = 0;
    unsafe { sys::ema_kvcache_memory_bytes(desc, &mut b) };
    b as usize
}

/// Static pre-allocated bf16 cache of one layer, [1, Hkv, capacity, head_dim], allocated
/// zeroed once and reused (`alloc_kv_static`, `crates/serve/src/engine_ext.rs:266-306`):
/// `reset` rewinds the length only. It also holds the device table 0..=capacity, the
/// analogue of the pre-built `static_offsets` scalars (`engine_ext.rs:293-299`), so a step
/// passes its offset without a host-to-device copy.
pub struct StaticCache {
    desc: sys::EmaKvCacheDesc,
    offset: i32,
    positions: PositionTable,
}

unsafe impl Send for StaticCache {}

impl StaticCache {
    pub fn new(n_kv_heads: i32, capacity: i32, head_dim: i32) -> Result<Self> {
        let positions = PositionTable::new(capacity.max(0))?;
        let mut desc = sys::EmaKvCacheDesc::default();
        check(unsafe { sys::ema_kvcache_alloc(&mut desc, 1, n_kv_heads, capacity, head_dim) }, "kvcache_alloc")?;
        Ok(StaticCache { desc, offset: 0, positions })
    }

    /// Device pointer to the int32 value p, 0 <= p <= capacity.
    pub fn device_position(&self, p: i32) -> Result<*const i32> {
        self.positions.at(p as i64, self.desc.capacity)
    }
}

impl Drop for StaticCache {
    fn drop(&mut self) {
        unsafe { sys::ema_kvcache_free(&mut self.desc) };
    }
}

impl KvCache for StaticCache {
    fn append(&mut self, ctx: &HipCtx, k: &DeviceArray, v: &DeviceArray) -> Result<()> {
        let t = append_len(&self.desc, k, v, "StaticCache::append")?;
        let hkv = self.desc.n_kv_heads as usize;
        let d = self.desc.head_dim as i64;
        if self.offset as i64 + t > self.desc.capacity as i64 {
            bail!("static KV overflow offset={} cap={}", self.offset as i64 + t, self.desc.capacity);
        }
        // one strided copy per tensor: Hkv rows of T*D elements into rows [offset, offset+T)
        let width = (t * d * 2) as usize;
        for (dst, src) in [(self.desc.k, k.data), (self.desc.v, v.data)] {
            let at = unsafe { (dst as *mut u8).add(self.offset as usize * self.desc.stride_pos as usize * 2) };
            check_hip(
                unsafe {
                    hip::hipMemcpy2DAsync(at as *mut c_void, self.desc.stride_head as usize * 2, src, width, width,
                                          hkv, hip::HIP_MEMCPY_DEVICE_TO_DEVICE, ctx.stream)
                },
                "StaticCache::append copy",
            )?;
        }
        self.offset += t as i32;
        Ok(())
    }

    fn get(&self, _ctx: &HipCtx) -> Result<(DeviceArray, DeviceArray)> {
        if self.offset == 0 {
            bail!("KV cache is empty");
        }
        let shape = vec![1, self.desc.n_kv_heads as i64, self.offset as i64, self.desc.head_dim as i64];
        let strides = vec![self.desc.stride_batch, self.desc.stride_head, self.desc.stride_pos, 1];
        Ok((
            DeviceArray { data: self.desc.k, shape: shape.clone(), strides: strides.clone() },
            DeviceArray { data: self.desc.v, shape, strides },
        ))
    }

    fn len(&self) -> usize {
        self.offset as usize
    }

    fn reset(&mut self) {
        self.offset = 0;
    }

    fn memory_bytes(&self) -> usize {
        memory_bytes_of(&self.desc)
    }
}

impl HipKvCache for StaticCache {
    fn desc(&self) -> &sys::EmaKvCacheDesc {
        &self.desc
    }
    fn position(&self, _ctx: &HipCtx, p: i64) -> Result<*const i32> {
        self.positions.at(p, self.desc.capacity)
    }
    fn set_len(&mut self, n: i64) -> Result<()> {
        if n < 0 || n > self.desc.capacity as i64 {
            bail!("static KV overflow offset={} cap={}", n, self.desc.capacity);
        }
        self.offset = n as i32;
        Ok(())
    }
}

/// Rotating (sliding-window) bf16 cache of one layer: the reference's `RotatingCache`
/// (`crates/kvcache/src/rotating.rs:22-122`), which keeps the last `window_size` tokens,
/// held as a ring [1, Hkv, window_size, head_dim] (`EMA_KV_ROTATING`): the token at
/// position p lives in row p % window_size, so an append writes rows in place instead of
/// concatenating and slicing. `len()` = min(tokens seen, window_size) (rotating.rs:108-110).
/// The layer calls write the ring rows themselves and attend the window.
pub struct RotatingCache {
    desc: sys::EmaKvCacheDesc,
    total: i64,
    slot: *mut i32,
}

unsafe impl Send for RotatingCache {}

impl RotatingCache {
    /// `RotatingCache::new(window_size, n_kv_heads, head_dim)` (rotating.rs:41-51); the
    /// ring is allocated zeroed here.
    pub fn new(window_size: usize, n_kv_heads: usize, head_dim: usize) -> Result<Self> {
        let w = i32::try_from(window_size)?;
        let hkv = i32::try_from(n_kv_heads)?;
        let hd = i32::try_from(head_dim)?;
        let mut slot: *mut c_void = std::ptr::null_mut();
        check_hip(unsafe { hip::hipMalloc(&mut slot, std::mem::size_of::<i32>()) }, "RotatingCache: position slot")?;
        let mut cache = RotatingCache { desc: sys::EmaKvCacheDesc::default(), total: 0, slot: slot as *mut i32 };
        check(unsafe { sys::ema_kvcache_alloc(&mut cache.desc, 1, hkv, w, hd) }, "kvcache_alloc")?;
        cache.desc.flags = sys::EMA_KV_ROTATING;
        Ok(cache)
    }

    pub fn window_size(&self) -> usize {
        self.desc.capacity as usize
    }

    /// Tokens seen since the last reset (may exceed the window).
    pub fn total_len(&self) -> i64 {
        self.total
    }
}

impl Drop for RotatingCache {
    fn drop(&mut self) {
        unsafe {
            sys::ema_kvcache_free(&mut self.desc);
            if !self.slot.is_null() {
                hip::hipFree(self.slot as *mut c_void);
            }
        }
    }
}

impl KvCache for RotatingCache {
    /// Appends at positions [total, total + T); with T > window_size only the last
    /// window_size tokens are kept (rotating.rs:81-92).
    fn append(&mut self, ctx: &HipCtx, k: &DeviceArray, v: &DeviceArray) -> Result<()> {
        let t_all = append_len(&self.desc, k, v, "RotatingCache::append")?;
        let hkv = self.desc.n_kv_heads as usize;
        let d = self.desc.head_dim as i64;
        let w = self.desc.capacity as i64;
        // tokens [skip, T) at positions total + t: one or two runs of consecutive ring rows
        let mut t = if t_all > w { t_all - w } else { 0 };
        while t < t_all {
            let row = (self.total + t) % w;
            let n = (t_all - t).min(w - row);
            let width = (n * d * 2) as usize;
            for (dst, src) in [(self.desc.k, k.data), (self.desc.v, v.data)] {
                let at = unsafe { (dst as *mut u8).add(row as usize * self.desc.stride_pos as usize * 2) };
                let from = unsafe { (src as *const u8).add((t * d * 2) as usize) };
                check_hip(
                    unsafe {
                        hip::hipMemcpy2DAsync(at as *mut c_void, self.desc.stride_head as usize * 2,
                                              from as *const c_void, (t_all * d * 2) as usize, width, hkv,
                                              hip::HIP_MEMCPY_DEVICE_TO_DEVICE, ctx.stream)
                    },
                    "RotatingCache::append copy",
                )?;
            }
            t += n;
        }
        self.total += t_all;
        Ok(())
    }

    /// The held tokens in order, [1, Hkv, len, head_dim]: the ring itself until it wraps,
    /// then a rotated copy in `ctx`'s arena (2 * Hkv * window * head_dim * 2 bytes; valid
    /// until the next call that uses the arena).
    fn get(&self, ctx: &HipCtx) -> Result<(DeviceArray, DeviceArray)> {
        if self.total == 0 {
            bail!("Rotating KV cache is empty");
        }
        let hkv = self.desc.n_kv_heads as i64;
        let d = self.desc.head_dim as i64;
        let w = self.desc.capacity as i64;
        let shape = vec![1, hkv, self.len() as i64, d];
        if self.total <= w {
            let strides = vec![self.desc.stride_batch, self.desc.stride_head, self.desc.stride_pos, 1];
            return Ok((
                DeviceArray { data: self.desc.k, shape: shape.clone(), strides: strides.clone() },
                DeviceArray { data: self.desc.v, shape, strides },
            ));
        }
        // wrapped: the oldest token is in row total % W; copy rows [start, W), then [0, start)
        let mut arena = Arena::new(ctx);
        let half = (hkv * w * d * 2) as usize;
        let buf = arena.take(2 * half) as *mut u8;
        arena.check("RotatingCache::get")?;
        let start = self.total % w;
        let pitch_src = self.desc.stride_head as usize * 2;
        let pitch_dst = (w * d * 2) as usize;
        for (i, src) in [self.desc.k, self.desc.v].into_iter().enumerate() {
            let dst = buf.wrapping_add(i * half);
            let src = src as *const u8;
            check_hip(
                unsafe {
                    hip::hipMemcpy2DAsync(dst as *mut c_void, pitch_dst,
                                          src.wrapping_add(start as usize * self.desc.stride_pos as usize * 2)
                                              as *const c_void,
                                          pitch_src, ((w - start) * d * 2) as usize, hkv as usize,
                                          hip::HIP_MEMCPY_DEVICE_TO_DEVICE, ctx.stream)
                },
                "RotatingCache::get copy",
            )?;
            if start > 0 {
                check_hip(
                    unsafe {
                        hip::hipMemcpy2DAsync(dst.wrapping_add(((w - start) * d * 2) as usize) as *mut c_void,
                                              pitch_dst, src as *const c_void, pitch_src, (start * d * 2) as usize,
                                              hkv as usize, hip::HIP_MEMCPY_DEVICE_TO_DEVICE, ctx.stream)
                    },
                    "RotatingCache::get copy",
                )?;
            }
        }
        Ok((
            DeviceArray::new(buf as *mut c_void, &shape),
            DeviceArray::new(buf.wrapping_add(half) as *mut c_void, &shape),
        ))
    }

    fn len(&self) -> usize {
        self.total.min(self.desc.capacity as i64) as usize
    }

    fn reset(&mut self) {
        self.total = 0;
    }

    fn memory_bytes(&self) -> usize {
        memory_bytes_of(&self.desc)
    }
}

impl HipKvCache for RotatingCache {
    fn desc(&self) -> &sys::EmaKvCacheDesc {
        &self.desc
    }
    /// The cache's one device slot, rewritten with `p` on `ctx.stream`
    /// (`ema_position_write`: stream-ordered, so a later call rewrites it only after the
    /// work that read it).
    fn position(&self, ctx: &HipCtx, p: i64) -> Result<*const i32> {
        if p < 0 || p > i32::MAX as i64 {
            bail!("rotating KV position {} out of range", p);
        }
        check(unsafe { sys::ema_position_write(ctx.stream, self.slot, p as i32) }, "position_write")?;
        Ok(self.slot as *const i32)
    }
    fn set_len(&mut self, n: i64) -> Result<()> {
        if n < 0 {
            bail!("rotating KV length {} out of range", n);
        }
        self.total = n;
        Ok(())
    }
}

/// FP8 E4M3FN cache of one layer: the reference's `Fp8Cache` (`crates/kvcache/src/fp8.rs:27-91`,
/// which keeps the E4M3FN round trip of every 64-value block of each K/V row), stored as one
/// code byte per value plus one exponent byte per block (`ema_kvcache_alloc_fp8`), allocated
/// zeroed once with a static capacity; `reset` rewinds the length only. The layer calls
/// quantise the rows they write and attend the decoded values. `n_rot` is the reference's
/// unquantised RoPE tail of each head (`Fp8Cache::new(head_dim, n_rot)`, fp8.rs:38-54): 0 or
/// 64, whose dims 64..127 are stored as bf16; head_dim 128.
pub struct Fp8Cache {
    desc: sys::EmaKvCacheDesc,
    offset: i32,
    positions: PositionTable,
}

unsafe impl Send for Fp8Cache {}

impl Fp8Cache {
    pub fn new(n_kv_heads: i32, capacity: i32, head_dim: i32, n_rot: i32) -> Result<Self> {
        let positions = PositionTable::new(capacity.max(0))?;
        let mut desc = sys::EmaKvCacheDesc::default();
        check(unsafe { sys::ema_kvcache_alloc_fp8(&mut desc, 1, n_kv_heads, capacity, head_dim, n_rot) },
              "kvcache_alloc_fp8")?;
        Ok(Fp8Cache { desc, offset: 0, positions })
    }

    /// Dims at the end of each head kept unquantised (bf16).
    pub fn n_rot(&self) -> i32 {
        self.desc.n_rot
    }
}

impl Drop for Fp8Cache {
    fn drop(&mut self) {
        unsafe { sys::ema_kvcache_free(&mut self.desc) };
    }
}

impl KvCache for Fp8Cache {
    /// Quantises K and V [1, Hkv, T, head_dim] bf16 into rows [len, len + T)
    /// (`fp8_round_trip` per 64-value block, `crates/kvcache/src/fp8.rs:47-68`).
    fn append(&mut self, ctx: &HipCtx, k: &DeviceArray, v: &DeviceArray) -> Result<()> {
        let t = append_len(&self.desc, k, v, "Fp8Cache::append")?;
        if self.offset as i64 + t > self.desc.capacity as i64 {
            bail!("static KV overflow offset={} cap={}", self.offset as i64 + t, self.desc.capacity);
        }
        if t == 0 {
            return Ok(());
        }
        // the new rows as a bf16 cache of T rows, quantised into rows [offset, offset + T)
        let mut src = sys::EmaKvCacheDesc::default();
        check(
            unsafe {
                sys::ema_kvcache_init(&mut src, k.data, v.data, 1, self.desc.n_kv_heads, t as i32, self.desc.head_dim)
            },
            "kvcache_init",
        )?;
        check(unsafe { sys::ema_kvcache_convert(ctx.stream, &src, 0, &self.desc, self.offset, t as i32) },
              "kvcache_convert")?;
        self.offset += t as i32;
        Ok(())
    }

    /// The held rows decoded to bf16 (exactly the values the reference keeps),
    /// [1, Hkv, len, head_dim] each, in `ctx`'s arena (valid until the next call that uses it).
    fn get(&self, ctx: &HipCtx) -> Result<(DeviceArray, DeviceArray)> {
        if self.offset == 0 {
            bail!("FP8 KV cache is empty");
        }
        let hkv = self.desc.n_kv_heads;
        let d = self.desc.head_dim;
        let n = self.offset;
        let bytes = hkv as usize * n as usize * d as usize * 2;
        let mut arena = Arena::new(ctx);
        let kb = arena.take(bytes);
        let vb = arena.take(bytes);
        arena.check("Fp8Cache::get")?;
        let mut dst = sys::EmaKvCacheDesc::default();
        check(unsafe { sys::ema_kvcache_init(&mut dst, kb, vb, 1, hkv, n, d) }, "kvcache_init")?;
        check(unsafe { sys::ema_kvcache_convert(ctx.stream, &self.desc, 0, &dst, 0, n) }, "kvcache_convert")?;
        let shape = [1, hkv as i64, n as i64, d as i64];
        Ok((DeviceArray::new(kb, &shape), DeviceArray::new(vb, &shape)))
    }

    fn len(&self) -> usize {
        self.offset as usize
    }

    fn reset(&mut self) {
        self.offset = 0;
    }

    fn memory_bytes(&self) -> usize {
        memory_bytes_of(&self.desc)
    }
}

impl HipKvCache for Fp8Cache {
    fn desc(&self) -> &sys::EmaKvCacheDesc {
        &self.desc
    }
    fn position(&self, _ctx: &HipCtx, p: i64) -> Result<*const i32> {
        self.positions.at(p, self.desc.capacity)
    }
    fn set_len(&mut self, n: i64) -> Result<()> {
        if n < 0 || n > self.desc.capacity as i64 {
            bail!("static KV overflow offset={} cap={}", n, self.desc.capacity);
        }
        self.offset = n as i32;
        Ok(())
    }
}

/// A quantised linear layer (`crates/ops/src/quant.rs:16-40`), MLX affine format:
/// weight [N, K * bits / 32] uint32, scales and biases [N, K / group_size] bf16; y = x W^T.
#[derive(Clone, Debug)]
pub struct QuantWeights {
    pub weight: DeviceArray,
    pub scales: DeviceArray,
    pub biases: DeviceArray,
    pub bits: i32,
    pub group_size: i32,
    pub mode: &'static str,
}

impl QuantWeights {
    /// 4-bit, group 64, affine (`QuantWeights::new` in the reference).
    pub fn new(weight: DeviceArray, scales: DeviceArray, biases: DeviceArray) -> Self {
        QuantWeights { weight, scales, biases, bits: 4, group_size: 64, mode: "affine" }
    }
    pub fn with_quant(weight: DeviceArray, scales: DeviceArray, biases: DeviceArray, bits: i32, group_size: i32) -> Self {
        QuantWeights { weight, scales, biases, bits, group_size, mode: "affine" }
    }
    pub fn is_quantized(&self) -> bool {
        self.group_size > 0
    }
}

/// `crates/attention/src/gqa.rs:27-42`.
#[derive(Debug, Clone)]
pub struct GqaConfig {
    pub n_heads: i32,
    pub n_kv_heads: i32,
    pub head_dim: i32,
    pub rope_theta: f32,
    pub norm_eps: f32,
    pub use_rope: bool,
}

/// `crates/attention/src/gqa.rs:45-53`: the four projections and the optional per-head
/// q/k RMSNorm weights ([head_dim] bf16), each norm optional on its own.
pub struct GqaWeights {
    pub q_proj: QuantWeights,
    pub k_proj: QuantWeights,
    pub v_proj: QuantWeights,
    pub o_proj: QuantWeights,
    pub q_norm: Option<DeviceArray>,
    pub k_norm: Option<DeviceArray>,
}

/// `crates/attention/src/sliding_window.rs:24-31`.
#[derive(Debug, Clone)]
pub struct SlidingWindowConfig {
    pub gqa: GqaConfig,
    pub window_size: usize,
}

const ALIGN: usize = 256;

fn aligned(n: usize) -> usize {
    (n + ALIGN - 1) & !(ALIGN - 1)
}

fn decode_ws_bytes(c: &GqaConfig, capacity: i32) -> Result<usize> {
    let mut need: u64 = 0;
    check(
        unsafe { sys::ema_decode_workspace_size(1, c.n_heads, c.n_kv_heads, c.head_dim, capacity, &mut need) },
        "decode_workspace_size",
    )?;
    Ok(need as usize)
}

/// Arena bytes `gqa_attention` needs for up to `max_seq_len` tokens of `hidden_size`
/// over a bf16 cache of `capacity` rows: q|k|v rows, o_proj output, q, attention output
/// and the decode split state. [`gqa_workspace_bytes_for`] covers any cache.
pub fn gqa_workspace_bytes(config: &GqaConfig, hidden_size: i64, max_seq_len: i32, capacity: i32) -> Result<usize> {
    let t = max_seq_len.max(1) as usize;
    let hd = (config.n_heads * config.head_dim) as usize;
    let f = ((config.n_heads + 2 * config.n_kv_heads) * config.head_dim) as usize;
    Ok(aligned(t * f * 2)
        + aligned(t * hidden_size as usize * 2)
        + aligned(hd * t * 2)
        + aligned(t * hd * 2)
        + aligned(decode_ws_bytes(config, capacity)?))
}

/// [`gqa_workspace_bytes`] for `cache`: an FP8 cache's prefill also needs the bf16 copy of
/// the rows it attends (`ema_prefill_workspace_size` over the whole capacity).
pub fn gqa_workspace_bytes_for<C: HipKvCache>(config: &GqaConfig, hidden_size: i64, max_seq_len: i32, cache: &C)
                                             -> Result<usize> {
    let desc = cache.desc();
    let mut bytes = gqa_workspace_bytes(config, hidden_size, max_seq_len, desc.capacity)?;
    if max_seq_len > 1 && desc.dtype != sys::EMA_DTYPE_BF16 {
        bytes += aligned(prefill_ws_bytes(desc, desc.capacity)?);
    }
    Ok(bytes)
}

/// Rows a prefill call attends: the ring for a rotating cache, else [0, offset + T).
fn prefill_rows(desc: &sys::EmaKvCacheDesc, offset: i64, t: i32) -> i32 {
    if desc.flags & sys::EMA_KV_ROTATING != 0 {
        return desc.capacity;
    }
    (offset + t as i64).min(desc.capacity as i64) as i32
}

fn prefill_ws_bytes(desc: &sys::EmaKvCacheDesc, rows: i32) -> Result<usize> {
    let mut need: u64 = 0;
    check(unsafe { sys::ema_prefill_workspace_size(desc, rows, &mut need) }, "prefill_workspace_size")?;
    Ok(need as usize)
}

/// Carves a call's temporaries out of the arena, in order. The decode counters stay at
/// its start in every layout: a decode workspace starts there, nothing else covers them.
struct Arena {
    base: *mut u8,
    have: usize,
    used: usize,
}

const COUNTERS: usize = sys::EMA_DECODE_COUNTER_BYTES as usize;

impl Arena {
    fn new(ctx: &HipCtx) -> Self {
        let have = if ctx.workspace.is_null() { 0 } else { ctx.workspace_bytes };
        Arena { base: ctx.workspace as *mut u8, have, used: COUNTERS }
    }
    /// The decode workspace of `bytes` (counters first); taken before anything else.
    fn take_decode_workspace(&mut self, bytes: usize) -> *mut c_void {
        self.used += aligned(bytes.saturating_sub(COUNTERS));
        self.base as *mut c_void
    }
    fn take(&mut self, bytes: usize) -> *mut c_void {
        let at = self.used;
        self.used += aligned(bytes);
        self.base.wrapping_add(at) as *mut c_void
    }
    fn check(&self, op: &str) -> Result<()> {
        if self.used > self.have || (self.base as usize) % ALIGN != 0 {
            bail!("{}: a 256-byte aligned ctx workspace of {} bytes is needed, {} given", op, self.used, self.have);
        }
        Ok(())
    }
}

fn check_proj(w: &QuantWeights, n: i32, k: i32, op: &str, which: &str) -> Result<()> {
    if !w.is_quantized() {
        bail!("{}: {} holds plain (dequantized) weights; only MLX affine-quantised ones are supported", op, which);
    }
    if w.mode != "affine" {
        bail!("{}: {}: quantisation mode '{}' (affine only)", op, which, w.mode);
    }
    if w.bits <= 0 || 32 % w.bits != 0 || k % w.group_size != 0 {
        bail!("{}: {}: bits {} / group_size {} do not fit K={}", op, which, w.bits, w.group_size, k);
    }
    let ws = vec![n as i64, k as i64 * w.bits as i64 / 32];
    let ss = vec![n as i64, (k / w.group_size) as i64];
    if w.weight.shape != ws || w.scales.shape != ss || w.biases.shape != ss {
        bail!("{}: {}: expected weight {:?} and scales/biases {:?}, got {:?} / {:?} / {:?}", op, which, ws, ss,
              w.weight.shape, w.scales.shape, w.biases.shape);
    }
    Ok(())
}

#[allow(clippy::too_many_arguments)]
fn project(ctx: &HipCtx, x: *const c_void, ldx: i64, w: &QuantWeights, m: i32, n: i32, k: i32, y: *mut c_void,
           ldy: i64) -> Result<()> {
    check(
        unsafe {
            sys::ema_quantized_matmul(ctx.stream, x, ldx, w.weight.data as *const u32, w.scales.data, w.biases.data,
                                      y, ldy, m, n, k, w.group_size, w.bits, sys::EMA_DTYPE_BF16)
        },
        "quantized_matmul",
    )
}

/// Full GQA attention layer (`crates/attention/src/gqa.rs:62-107`), generic over the cache
/// backend like the reference's (`StaticCache`, `RotatingCache`, `Fp8Cache`).
///
/// - `x`: hidden state [1, seq_len, hidden] bf16
/// - `offset`: position of the first new token
///
/// Returns [1, seq_len, hidden] bf16 in `ctx`'s arena. The q, k and v projections land in
/// one q|k|v row (`run_qkv`'s separate pieces without the concatenation); q/k norms,
/// RoPE and the cache write follow (`ema_pre_attention`: ring rows for a rotating cache,
/// quantised rows for an FP8 one), then causal attention over the cache for T > 1
/// (`is_prefill`, gqa.rs:78; a ring attends its window), or for T == 1 the fused decode
/// step over min(offset + 1, capacity) rows; then o_proj. The cache length becomes
/// offset + T.
pub fn gqa_attention<C: HipKvCache>(ctx: &HipCtx, x: &DeviceArray, weights: &GqaWeights, cache: &mut C,
                                    config: &GqaConfig, offset: i32) -> Result<DeviceArray> {
    gqa_layer(ctx, x, weights, cache, config, offset, "gqa_attention")
}

fn gqa_layer<C: HipKvCache>(ctx: &HipCtx, x: &DeviceArray, weights: &GqaWeights, cache: &mut C,
                            config: &GqaConfig, offset: i32, op: &str) -> Result<DeviceArray> {
    let (hq, hkv, d) = (config.n_heads, config.n_kv_heads, config.head_dim);
    if hq <= 0 || hkv <= 0 || d <= 0 || hq % hkv != 0 {
        bail!("{}: bad head config n_heads={} n_kv_heads={} head_dim={}", op, hq, hkv, d);
    }
    if hkv != cache.n_kv_heads() || d != cache.head_dim() {
        bail!("{}: config does not match the cache", op);
    }
    if x.data.is_null() || x.shape.len() != 3 || x.shape[0] != 1 || x.shape[1] <= 0 || x.shape[2] <= 0
        || !x.strides.is_empty() || x.shape[1] > i32::MAX as i64 || x.shape[2] > i32::MAX as i64
    {
        bail!("{}: x must be contiguous [1, seq, hidden], got {:?}", op, x.shape);
    }
    let t = x.shape[1] as i32;
    let hidden = x.shape[2] as i32;
    let cap = cache.capacity();
    if !cache.rotating() && (offset < 0 || offset as i64 + t as i64 > cap as i64) {
        bail!("static KV overflow offset={} cap={}", offset as i64 + t as i64 - 1, cap);
    }
    if cache.rotating() && (offset < 0 || t > cap) {
        bail!("{}: {} tokens exceed the window {}", op, t, cap);
    }
    check_proj(&weights.q_proj, hq * d, hidden, op, "q_proj")?;
    check_proj(&weights.k_proj, hkv * d, hidden, op, "k_proj")?;
    check_proj(&weights.v_proj, hkv * d, hidden, op, "v_proj")?;
    check_proj(&weights.o_proj, hidden, hq * d, op, "o_proj")?;

    let desc = *cache.desc();
    let f = ((hq + 2 * hkv) * d) as i64;
    let hd = (hq * d) as usize;
    let mut arena = Arena::new(ctx);
    let ws_bytes = if t == 1 { decode_ws_bytes(config, cap)? } else { 0 };
    let ws = if t == 1 { arena.take_decode_workspace(ws_bytes) } else { std::ptr::null_mut() };
    let qkv = arena.take(t as usize * f as usize * 2);
    let y = arena.take(t as usize * hidden as usize * 2);
    let q = if t > 1 { arena.take(hd * t as usize * 2) } else { std::ptr::null_mut() };
    let attn = arena.take(t as usize * hd * 2);
    // an FP8 cache's prefill attends a bf16 copy of its rows
    let quantised = desc.dtype != sys::EMA_DTYPE_BF16;
    let rows = prefill_rows(&desc, offset as i64, t);
    let pws_bytes = if t > 1 && quantised { prefill_ws_bytes(&desc, rows)? } else { 0 };
    let pws = if pws_bytes > 0 { arena.take(pws_bytes) } else { std::ptr::null_mut() };
    arena.check(op)?;

    // 1. q|k|v projections (project_qkv, crates/ops/src/attention.rs:31-51)
    let qkv_b = qkv as *mut u8;
    project(ctx, x.data, hidden as i64, &weights.q_proj, t, hq * d, hidden, qkv, f)?;
    project(ctx, x.data, hidden as i64, &weights.k_proj, t, hkv * d, hidden,
            qkv_b.wrapping_add((hq * d) as usize * 2) as *mut c_void, f)?;
    project(ctx, x.data, hidden as i64, &weights.v_proj, t, hkv * d, hidden,
            qkv_b.wrapping_add(((hq + hkv) * d) as usize * 2) as *mut c_void, f)?;

    // 2-6. norms (each optional on its own, attention.rs:57-76), RoPE, cache write, SDPA
    let mut flags = 0u32;
    if weights.q_norm.is_none() {
        flags |= sys::EMA_PRE_NO_Q_NORM;
    }
    if weights.k_norm.is_none() {
        flags |= sys::EMA_PRE_NO_K_NORM;
    }
    if !config.use_rope {
        flags |= sys::EMA_PRE_NO_ROPE;
    }
    let qw = weights.q_norm.as_ref().map_or(std::ptr::null(), |a| a.data as *const c_void);
    let kw = weights.k_norm.as_ref().map_or(std::ptr::null(), |a| a.data as *const c_void);
    let scale = 1.0f32 / (d as f32).sqrt();
    let pos = cache.position(ctx, offset as i64)?;
    if t > 1 {
        if quantised {
            // FP8: pre-attention also puts the chunk's decoded rows into the prefill's bf16
            // copy, so the prefill decodes only earlier rows (none for a static cache's first
            // chunk, whose keys are the chunk's own)
            check(
                unsafe {
                    sys::ema_pre_attention_ws(ctx.stream, qkv, qw, kw, config.norm_eps, config.rope_theta, pos, 1, t,
                                              hq, hkv, d, flags, q, &desc, rows, pws, pws_bytes as u64)
                },
                "pre_attention_ws",
            )?;
            let mut pf = sys::EMA_PREFILL_CAUSAL | sys::EMA_PREFILL_ROWS_DECODED;
            if offset == 0 && desc.flags & sys::EMA_KV_ROTATING == 0 {
                pf |= sys::EMA_PREFILL_CHUNK_ONLY;
            }
            check(
                unsafe {
                    sys::ema_prefill_attention_ws(ctx.stream, q, &desc, pos, t, hq, scale, pf, attn, rows, pws,
                                                  pws_bytes as u64)
                },
                "prefill_attention_ws",
            )?;
        } else {
            check(
                unsafe {
                    sys::ema_pre_attention(ctx.stream, qkv, qw, kw, config.norm_eps, config.rope_theta, pos, 1, t,
                                           hq, hkv, d, flags, q, &desc)
                },
                "pre_attention",
            )?;
            check(
                unsafe {
                    sys::ema_prefill_attention(ctx.stream, q, &desc, pos, t, hq, scale, sys::EMA_PREFILL_CAUSAL,
                                               attn)
                },
                "prefill_attention",
            )?;
        }
    } else {
        let max_len = (offset + 1).min(cap);
        check(
            unsafe {
                sys::ema_decode_step(ctx.stream, qkv, qw, kw, config.norm_eps, config.rope_theta, pos as *mut i32,
                                     max_len, hq, flags, scale, &desc, attn, ws, ws_bytes as u64)
            },
            "decode_step",
        )?;
    }
    cache.set_len(offset as i64 + t as i64)?;

    // 7-8. o_proj (attend_and_project, crates/ops/src/attention.rs:162-177)
    project(ctx, attn, hd as i64, &weights.o_proj, t, hidden, hq * d, y, hidden as i64)?;
    Ok(DeviceArray::new(y, &[1, t as i64, hidden as i64]))
}

/// `crates/attention/src/sliding_window.rs:40-50`: the reference delegates to
/// `gqa_attention` and leaves the window to the cache backend. A `RotatingCache` is that
/// window here (its ring of `window_size` rows), so a ring whose size differs from
/// `config.window_size` is an error; any other cache attends all its rows, as in the
/// reference.
pub fn sliding_window_attention<C: HipKvCache>(ctx: &HipCtx, x: &DeviceArray, weights: &GqaWeights, cache: &mut C,
                                               config: &SlidingWindowConfig, offset: i32) -> Result<DeviceArray> {
    if cache.rotating() && config.window_size != cache.capacity() as usize {
        bail!("sliding_window_attention: window_size {} differs from the cache's {}", config.window_size,
              cache.capacity());
    }
    gqa_layer(ctx, x, weights, cache, &config.gqa, offset, "sliding_window_attention")
}
