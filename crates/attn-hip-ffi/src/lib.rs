//! Rust binding of `libema_attn`, the MI355X (gfx950) attention path of engine-mlx.
//!
//! Three layers:
//! - [`sys`]: the C ABI of `include/ema_attn.h`, declared by hand (every export, every
//!   constant, the `ema_kvcache_desc` layout);
//! - [`hip`]: the few HIP runtime calls the safe layer needs (device memory and copies);
//! - the safe layer, in the shape of the reference's crates: the `KvCache` trait
//!   (`crates/kvcache/src/lib.rs:52-76`), a static pre-allocated cache (the serve crate's
//!   `kv_bufs` + `static_offsets`, `crates/serve/src/engine_ext.rs:266-306`),
//!   `QuantWeights` (`crates/ops/src/quant.rs:16-40`), `GqaConfig` / `GqaWeights` /
//!   `gqa_attention` (`crates/attention/src/gqa.rs:27-107`) and
//!   `sliding_window_attention` (`crates/attention/src/sliding_window.rs:40-50`).
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
                                    capacity: i32, head_dim: i32) -> i32;
        pub fn ema_kvcache_alloc_fp8(out: *mut EmaKvCacheDesc, batch: i32, n_kv_heads: i32, capacity: i32,
                                     head_dim: i32) -> i32;
        pub fn ema_kvcache_init_int4(desc: *mut EmaKvCacheDesc, k: *mut c_void, v: *mut c_void,
                                     k_scales: *mut c_void, k_biases: *mut c_void, v_scales: *mut c_void,
                                     v_biases: *mut c_void, batch: i32, n_kv_heads: i32, capacity: i32,
                                     head_dim: i32) -> i32;
        pub fn ema_kvcache_alloc_int4(out: *mut EmaKvCacheDesc, batch: i32, n_kv_heads: i32, capacity: i32,
                                      head_dim: i32) -> i32;
        pub fn ema_kvcache_quantize_int4(stream: EmaStream, src: *const EmaKvCacheDesc, src_row: i32,
                                         dst: *const EmaKvCacheDesc, dst_row: i32, n_rows: i32) -> i32;
        pub fn ema_kvcache_free(desc: *mut EmaKvCacheDesc) -> i32;
        pub fn ema_kvcache_memory_bytes(desc: *const EmaKvCacheDesc, bytes: *mut u64) -> i32;
        pub fn ema_pre_attention(stream: EmaStream, qkv: *const c_void, q_norm_w: *const c_void,
                                 k_norm_w: *const c_void, eps: f32, theta: f32, offsets: *const i32, batch: i32,
                                 n_tokens: i32, n_heads: i32, n_kv_heads: i32, head_dim: i32, flags: u32,
                                 q_out: *mut c_void, cache: *const EmaKvCacheDesc) -> i32;
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

/// Static pre-allocated bf16 cache of one layer, [1, Hkv, capacity, head_dim], allocated
/// zeroed once and reused (`alloc_kv_static`, `crates/serve/src/engine_ext.rs:266-306`):
/// `reset` rewinds the length only. It also holds the device table 0..=capacity, the
/// analogue of the pre-built `static_offsets` scalars (`engine_ext.rs:293-299`), so a step
/// passes its offset without a host-to-device copy.
pub struct StaticCache {
    desc: sys::EmaKvCacheDesc,
    offset: i32,
    positions: *mut i32,
}

unsafe impl Send for StaticCache {}

impl StaticCache {
    pub fn new(n_kv_heads: i32, capacity: i32, head_dim: i32) -> Result<Self> {
        let mut desc = sys::EmaKvCacheDesc::default();
        check(unsafe { sys::ema_kvcache_alloc(&mut desc, 1, n_kv_heads, capacity, head_dim) }, "kvcache_alloc")?;
        let table: Vec<i32> = (0..=capacity).collect();
        let bytes = table.len() * std::mem::size_of::<i32>();
        let mut p: *mut c_void = std::ptr::null_mut();
        let rc = unsafe { hip::hipMalloc(&mut p, bytes) };
        let rc = if rc == hip::HIP_SUCCESS {
            unsafe { hip::hipMemcpy(p, table.as_ptr() as *const c_void, bytes, hip::HIP_MEMCPY_HOST_TO_DEVICE) }
        } else {
            rc
        };
        if rc != hip::HIP_SUCCESS {
            unsafe {
                if !p.is_null() {
                    hip::hipFree(p);
                }
                sys::ema_kvcache_free(&mut desc);
            }
            check_hip(rc, "StaticCache: positions")?;
        }
        Ok(StaticCache { desc, offset: 0, positions: p as *mut i32 })
    }

    pub fn capacity(&self) -> i32 {
        self.desc.capacity
    }
    pub fn n_kv_heads(&self) -> i32 {
        self.desc.n_kv_heads
    }
    pub fn head_dim(&self) -> i32 {
        self.desc.head_dim
    }
    pub fn desc(&self) -> &sys::EmaKvCacheDesc {
        &self.desc
    }

    /// Device pointer to the int32 value p, 0 <= p <= capacity.
    pub fn device_position(&self, p: i32) -> Result<*const i32> {
        if p < 0 || p > self.desc.capacity {
            bail!("static KV overflow offset={} cap={}", p, self.desc.capacity);
        }
        Ok(unsafe { self.positions.add(p as usize) } as *const i32)
    }

    fn set_len(&mut self, n: i64) -> Result<()> {
        if n < 0 || n > self.desc.capacity as i64 {
            bail!("static KV overflow offset={} cap={}", n, self.desc.capacity);
        }
        self.offset = n as i32;
        Ok(())
    }
}

impl Drop for StaticCache {
    fn drop(&mut self) {
        unsafe {
            sys::ema_kvcache_free(&mut self.desc);
            if !self.positions.is_null() {
                hip::hipFree(self.positions as *mut c_void);
            }
        }
    }
}

impl KvCache for StaticCache {
    fn append(&mut self, ctx: &HipCtx, k: &DeviceArray, v: &DeviceArray) -> Result<()> {
        let hkv = self.desc.n_kv_heads as i64;
        let d = self.desc.head_dim as i64;
        for a in [k, v] {
            if a.data.is_null() {
                bail!("StaticCache::append: null k/v");
            }
            if a.shape.len() != 4 || a.shape[0] != 1 || a.shape[1] != hkv || a.shape[3] != d || !a.strides.is_empty() {
                bail!("StaticCache::append: expected contiguous [1, {}, seq, {}], got {:?}", hkv, d, a.shape);
            }
        }
        if k.shape[2] != v.shape[2] {
            bail!("StaticCache::append: k/v lengths differ");
        }
        let t = k.shape[2];
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
                                          hkv as usize, hip::HIP_MEMCPY_DEVICE_TO_DEVICE, ctx.stream)
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
        let mut b: u64 = 0;
        unsafe { sys::ema_kvcache_memory_bytes(&self.desc, &mut b) };
        b as usize
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
/// over a cache of `capacity` rows: q|k|v rows, o_proj output, q, attention output and
/// the decode split state.
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

/// Full GQA attention layer (`crates/attention/src/gqa.rs:62-107`) over a static cache.
///
/// - `x`: hidden state [1, seq_len, hidden] bf16
/// - `offset`: position of the first new token
///
/// Returns [1, seq_len, hidden] bf16 in `ctx`'s arena. The q, k and v projections land in
/// one q|k|v row (`run_qkv`'s separate pieces without the concatenation); q/k norms,
/// RoPE and the cache write follow (`ema_pre_attention`), then causal attention over
/// [0, offset + T) for T > 1 (`is_prefill`, gqa.rs:78), or for T == 1 the fused decode
/// step over offset + 1 rows; then o_proj. The cache length becomes offset + T.
pub fn gqa_attention(ctx: &HipCtx, x: &DeviceArray, weights: &GqaWeights, cache: &mut StaticCache,
                     config: &GqaConfig, offset: i32) -> Result<DeviceArray> {
    let op = "gqa_attention";
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
    if offset < 0 || offset as i64 + t as i64 > cap as i64 {
        bail!("static KV overflow offset={} cap={}", offset as i64 + t as i64 - 1, cap);
    }
    check_proj(&weights.q_proj, hq * d, hidden, op, "q_proj")?;
    check_proj(&weights.k_proj, hkv * d, hidden, op, "k_proj")?;
    check_proj(&weights.v_proj, hkv * d, hidden, op, "v_proj")?;
    check_proj(&weights.o_proj, hidden, hq * d, op, "o_proj")?;

    let f = ((hq + 2 * hkv) * d) as i64;
    let hd = (hq * d) as usize;
    let mut arena = Arena::new(ctx);
    let ws_bytes = if t == 1 { decode_ws_bytes(config, cap)? } else { 0 };
    let ws = if t == 1 { arena.take_decode_workspace(ws_bytes) } else { std::ptr::null_mut() };
    let qkv = arena.take(t as usize * f as usize * 2);
    let y = arena.take(t as usize * hidden as usize * 2);
    let q = if t > 1 { arena.take(hd * t as usize * 2) } else { std::ptr::null_mut() };
    let attn = arena.take(t as usize * hd * 2);
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
    let pos = cache.device_position(offset)?;
    if t > 1 {
        check(
            unsafe {
                sys::ema_pre_attention(ctx.stream, qkv, qw, kw, config.norm_eps, config.rope_theta, pos, 1, t, hq,
                                       hkv, d, flags, q, cache.desc())
            },
            "pre_attention",
        )?;
        check(
            unsafe {
                sys::ema_prefill_attention(ctx.stream, q, cache.desc(), pos, t, hq, scale, sys::EMA_PREFILL_CAUSAL,
                                           attn)
            },
            "prefill_attention",
        )?;
    } else {
        let max_len = (offset + 1).min(cap);
        check(
            unsafe {
                sys::ema_decode_step(ctx.stream, qkv, qw, kw, config.norm_eps, config.rope_theta, pos as *mut i32,
                                     max_len, hq, flags, scale, cache.desc(), attn, ws, ws_bytes as u64)
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
/// `gqa_attention` and leaves the window to the cache backend.
pub fn sliding_window_attention(ctx: &HipCtx, x: &DeviceArray, weights: &GqaWeights, cache: &mut StaticCache,
                                config: &SlidingWindowConfig, offset: i32) -> Result<DeviceArray> {
    gqa_attention(ctx, x, weights, cache, &config.gqa, offset)
}
