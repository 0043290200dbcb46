/*
 * ema_attn — MI355X (gfx950) attention hot path of engine-mlx, C ABI.
 *
 * Replaces, for the Qwen3 attention path, the MLX primitives the reference
 * reaches through mlx-c (dangranaz/engine-mlx 0.1.18):
 *
 *   reference call (file:line)                                  replaced by
 *   ----------------------------------------------------------  ----------------------
 *   MlxCtx::rms_norm   crates/mlx-ffi/src/ops/real/blas.rs:5-9  ema_pre_attention
 *   MlxCtx::rope_dynamic / rope            blas.rs:67-80        ema_pre_attention
 *   MlxCtx::scatter_single  crates/mlx-ffi/src/ops/real/slice.rs:106-113
 *                                                               ema_pre_attention (T=1)
 *   MlxCtx::slice_update    slice.rs:78-88                      ema_pre_attention (T>1)
 *   MlxCtx::sdpa_masked  crates/mlx-ffi/src/ops/real/transform.rs:8-29
 *                                                               ema_decode_attention
 *   MlxCtx::sdpa(causal=true)  blas.rs:82-101                   ema_prefill_attention
 *   static KV buffers  crates/serve/src/engine_ext.rs:266-306   ema_kvcache_*
 *   KvCache::memory_bytes  crates/kvcache/src/lib.rs:75         ema_kvcache_memory_bytes
 *   Fp8Cache (E4M3FN round trip per 64-value block)
 *              crates/kvcache/src/fp8.rs:47-68, crates/ops/src/fp8.rs:71-92
 *                                                               ema_kvcache_init_fp8 / _alloc_fp8
 *                                                               (stored, not simulated)
 *   int4 KV (quantize_kv_native / dequantize_kv_native, group 64, 4 bits)
 *              crates/serve/src/engine_ext.rs:92-157, crates/mlx-ffi/src/ops/real/quant.rs:8-64
 *                                                               ema_kvcache_init_int4 / _alloc_int4,
 *                                                               ema_decode_attention / _step read it
 *   convert_kv_to_int4 and the int4 prefill store
 *              crates/serve/src/engine_ext.rs:158-210, forward_qwen3.rs:69-120
 *                                                               ema_kvcache_quantize_int4
 *   gdn_step / gdn_step_metal and the per-token scan of gdn_forward
 *              crates/ops/src/gdn.rs:83-150, gdn_metal.rs:56-88, gdn_forward.rs:173-192
 *                                                               ema_gdn_scan, ema_gdn_scan_ws
 *   MlxCtx::quantized_matmul (affine, transpose=true)
 *              crates/mlx-ffi/src/ops/real/transform.rs:77-88, via qmatmul
 *              (crates/ops/src/quant.rs:57-76) and run_qkv / o_proj
 *              (crates/serve/src/forward/projection.rs:105-152)  ema_quantized_matmul
 *
 * Conventions
 *   - Every entry point returns int32_t: EMA_OK (0) or a negative EMA_ERR_*.
 *     On error, ema_last_error() returns a thread-local message (the analogue
 *     of the reference's "MLX op '<op>' failed with code <n>",
 *     crates/mlx-ffi/src/ops/real/mod.rs:35-40).
 *   - Eager and stream-ordered: work is enqueued on `stream` (a hipStream_t;
 *     NULL = the default stream). Nothing synchronises the host.
 *   - No allocation inside the hot calls (pre_attention, decode, prefill);
 *     buffers and workspace are owned by the caller. Re-entrant on distinct
 *     streams; the only global state is the thread-local error string.
 *   - bf16 = IEEE bfloat16 (RNE). Device pointers must be 16-byte aligned and
 *     head_dim-contiguous.
 *   - Masking is by valid length: the additive bf16 mask of
 *     crates/serve/src/engine_ext.rs:237-260 (0 for p <= offset, -1e9 beyond)
 *     is exactly a length offset+1, because exp(-1e9 - m) is 0 in f32.
 */
#ifndef EMA_ATTN_H
#define EMA_ATTN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define EMA_OK 0
#define EMA_ERR_INVALID_ARG (-1) /* null pointer, bad enum, misaligned      */
#define EMA_ERR_SHAPE (-2)       /* inconsistent or unsupported dimensions   */
#define EMA_ERR_CAPACITY (-3)    /* write/read beyond the static capacity    */
#define EMA_ERR_WORKSPACE (-4)   /* workspace missing or too small           */
#define EMA_ERR_UNSUPPORTED (-5) /* valid but not implemented (e.g. head_dim)*/
#define EMA_ERR_HIP (-6)         /* HIP runtime error (launch, malloc)       */

#define EMA_DTYPE_BF16 1
/* FP8 E4M3FN codes (one byte per element) plus one int8 exponent per 64-element block
 * of a row: element = e4m3(code) * 2^exp. Written with the quantisation of the
 * reference's FP8 cache (crates/ops/src/fp8.rs:71-92: exp = ceil(log2(amax / 448)),
 * amax = max(1e-4, max |x|) over the block, round to nearest even, saturate at 448).
 * Decoded exactly to bf16 by the readers. head_dim 128 only, static or rotating
 * (EMA_KV_ROTATING) caches. Values must be finite. With n_rot = 64 (the descriptor's
 * field; Fp8Cache::new(128, 64), crates/kvcache/src/fp8.rs:38-54) the last 64 dims of each
 * row are the RoPE tail that the reference leaves unquantised: they are stored as bf16. */
#define EMA_DTYPE_FP8_E4M3 2
/* 4-bit affine codes (MLX "affine" quantisation, group 64, the layout of the reference's
 * int4 KV buffers, crates/serve/src/engine_ext.rs:92-129): per row of head_dim values,
 * head_dim / 8 uint32 words (value i in bits 4(i % 8) of word i / 8) plus one bf16 scale and
 * one bf16 bias per 64 values; value = scale * code + bias. Rows are written with MLX's
 * affine quantiser (per group: scale = max((max - min) / 15, 1e-7), signed towards the
 * larger-magnitude end, which is moved onto the grid and becomes the bias; codes
 * round((x - bias) / scale), half away from zero, at most 15). Readers use the exact affine
 * value scale * code + bias; MLX's dequantize to bf16 rounds it once (at most half a bf16
 * step per element). head_dim 128, capacity a multiple of 32, static or
 * rotating (EMA_KV_ROTATING) caches; decode only (prefill attends bf16 keys, as the
 * reference's does). */
#define EMA_DTYPE_INT4_AFFINE 5
/* activation types of ema_gdn_scan (besides EMA_DTYPE_BF16) */
#define EMA_DTYPE_F16 3
#define EMA_DTYPE_F32 4

/* ema_kvcache_desc.flags */
/* Rotating (sliding-window) cache of the last `capacity` tokens, the reference's
 * RotatingCache (crates/kvcache/src/rotating.rs:56-122) as a ring: the token at absolute
 * position p lives in row p % capacity. Writes (ema_pre_attention, ema_decode_step) go to
 * that row, RoPE still uses p; a call writing n_tokens > capacity rows keeps the last
 * capacity of them. Decode attends min(length, capacity) rows (the window; attention does
 * not depend on the rows' order). Prefill attends, for query position p of a chunk that
 * ends at L = q_offset + n_tokens, the keys at positions [max(0, L - capacity), p]: the
 * window the reference's cache holds after the chunk's append (rotating.rs:86-97), with
 * MLX's end-aligned causal mask over it. */
#define EMA_KV_ROTATING 1

/* ema_pre_attention flags */
#define EMA_PRE_NO_NORM 1u /* q_norm/k_norm are None: crates/ops/src/attention.rs:57-76 */
#define EMA_PRE_NO_ROPE 2u /* NoPE layer (use_rope=false): crates/ops/src/rope.rs:38-40  */
/* One of the two norms absent: optional_qk_norm applies q_norm and k_norm independently
 * (crates/ops/src/attention.rs:57-76). The absent weight may be null. EMA_PRE_NO_NORM is
 * both together. Accepted by ema_pre_attention and the decode steps. */
#define EMA_PRE_NO_Q_NORM 8u
#define EMA_PRE_NO_K_NORM 16u
/* ema_decode_step / ema_decode_step_noalloc only: after the step, offsets[b] += 1 on the
 * device for every sequence whose new row was written (0 <= offset < capacity; any
 * offset >= 0 for a rotating cache). An offset that wrote nothing is left as it is, so a
 * sequence that reached the capacity stays there and the caller can see it. This is the
 * reference's per-token bookkeeping (crates/serve/src/decode_compiled.rs:49,
 * `self.offset += 1` after each step) kept on the device, so that one captured graph of
 * N steps decodes N tokens per sequence with no host work in between. The reference keeps
 * one offset for the whole model, shared by every layer of a token: when the layers of a
 * model share one offsets array, only the last layer's step of each token carries this
 * flag (an earlier layer's advance would move the later layers' write row and length);
 * otherwise each layer needs an offsets array of its own. */
#define EMA_STEP_ADVANCE 4u

/* ema_prefill_attention flags */
#define EMA_PREFILL_CAUSAL 1u     /* MLX "causal", query block end-aligned to the keys   */
#define EMA_PREFILL_CHUNK_ONLY 2u /* keys limited to the new chunk [q_off, q_off+T):
                                     crates/serve/src/forward_qwen3.rs:150 attends only
                                     the freshly projected k/v; without this flag the
                                     whole cache [0, q_off+T) is attended, as
                                     gqa_attention does (crates/attention/src/gqa.rs:100-106) */
#define EMA_PREFILL_ROWS_DECODED 4u /* FP8 cache, ema_prefill_attention_ws: the workspace's
                                     bf16 copy already holds the chunk's rows
                                     [q_off, q_off+T), written by ema_pre_attention_ws with
                                     the same max_kv_len; only the other attended rows are
                                     decoded (none with EMA_PREFILL_CHUNK_ONLY over a static
                                     cache, and then no decode pass runs) */

typedef void* ema_stream_t; /* hipStream_t */

#ifndef EMA_API
#define EMA_API __attribute__((visibility("default")))
#endif

/* Static KV cache of one layer: K and V of logical shape
 * [batch, n_kv_heads, capacity, head_dim], head_dim contiguous, bf16 or FP8 E4M3FN.
 * Owned by the caller (the reference allocates these once at MAX_CAP,
 * crates/serve/src/engine_ext.rs:266-306, and reuses them across requests).
 * FP8: k/v hold the codes (strides in elements = bytes, multiples of 16) and
 * k_exp/v_exp the block exponents, int8 [batch, n_kv_heads, capacity, head_dim / 64],
 * contiguous. With n_rot = 64 a row is 64 code bytes (dims 0..63, block 0) followed by
 * the 64 bf16 values of dims 64..127 (stride_pos >= 192 bytes); block 1's exponent is 0.
 * INT4: k/v hold the packed words (strides in 4-bit elements, multiples of 32, i.e. 16
 * bytes) and k_scales/k_biases/v_scales/v_biases the bf16 group parameters
 * [batch, n_kv_heads, capacity, head_dim / 64], contiguous. */
typedef struct ema_kvcache_desc {
  void* k;
  void* v;
  int32_t batch;
  int32_t n_kv_heads;
  int32_t capacity;
  int32_t head_dim;
  int64_t stride_batch; /* in elements */
  int64_t stride_head;  /* in elements */
  int64_t stride_pos;   /* in elements, >= head_dim */
  int32_t dtype;        /* EMA_DTYPE_BF16 or EMA_DTYPE_FP8_E4M3 */
  int32_t flags;        /* 0 or EMA_KV_ROTATING (set by the caller after init/alloc) */
  void* k_exp;          /* EMA_DTYPE_FP8_E4M3: block exponents of K and V (else NULL) */
  void* v_exp;
  void* k_scales;       /* EMA_DTYPE_INT4_AFFINE: group scales and biases (else NULL) */
  void* k_biases;
  void* v_scales;
  void* v_biases;
  int32_t n_rot;        /* EMA_DTYPE_FP8_E4M3: dims at the end of each row kept as bf16 (0 or 64; else 0) */
} ema_kvcache_desc;

/* Thread-local message of the last failed call on this thread ("" if none). */
EMA_API const char* ema_last_error(void);
/* Library version string. */
EMA_API const char* ema_version(void);

/* Fill a descriptor for caller-owned contiguous K/V buffers. */
EMA_API int32_t ema_kvcache_init(ema_kvcache_desc* desc, void* k, void* v, int32_t batch,
                         int32_t n_kv_heads, int32_t capacity, int32_t head_dim);
/* Allocate zeroed device K/V buffers (zeros_bf16 in alloc_kv_static,
 * crates/serve/src/engine_ext.rs:273-278). Not for the hot path. */
EMA_API int32_t ema_kvcache_alloc(ema_kvcache_desc* out, int32_t batch, int32_t n_kv_heads,
                          int32_t capacity, int32_t head_dim);
/* FP8 E4M3FN cache over caller-owned rows [batch, n_kv_heads, capacity, head_dim + n_rot]
 * (bytes: head_dim - n_rot codes, then n_rot bf16 values) and exponents
 * [batch, n_kv_heads, capacity, head_dim / 64] (int8), all contiguous. n_rot is the
 * reference's Fp8Cache::new(head_dim, n_rot) argument: 0 or 64 (EMA_ERR_UNSUPPORTED
 * otherwise). */
EMA_API int32_t ema_kvcache_init_fp8(ema_kvcache_desc* desc, void* k, void* v, void* k_exp, void* v_exp,
                                     int32_t batch, int32_t n_kv_heads, int32_t capacity, int32_t head_dim,
                                     int32_t n_rot);
/* Allocate a zeroed FP8 cache (rows and exponents). Not for the hot path. */
EMA_API int32_t ema_kvcache_alloc_fp8(ema_kvcache_desc* out, int32_t batch, int32_t n_kv_heads,
                                      int32_t capacity, int32_t head_dim, int32_t n_rot);
/* int4 affine cache over caller-owned words [batch, n_kv_heads, capacity, head_dim / 8]
 * (uint32) and scales/biases [batch, n_kv_heads, capacity, head_dim / 64] (bf16), all
 * contiguous: the six buffers of alloc_kv_int4 (crates/serve/src/engine_ext.rs:92-129). */
EMA_API int32_t ema_kvcache_init_int4(ema_kvcache_desc* desc, void* k, void* v, void* k_scales, void* k_biases,
                                      void* v_scales, void* v_biases, int32_t batch, int32_t n_kv_heads,
                                      int32_t capacity, int32_t head_dim);
/* Allocate a zeroed int4 cache (alloc_kv_int4, engine_ext.rs:98-129). Not for the hot path. */
EMA_API int32_t ema_kvcache_alloc_int4(ema_kvcache_desc* out, int32_t batch, int32_t n_kv_heads,
                                       int32_t capacity, int32_t head_dim);
/* Quantise rows [src_row, src_row + n_rows) of every (sequence, kv head) of the bf16 cache
 * `src` into rows [dst_row, dst_row + n_rows) of the int4 cache `dst` (same batch, heads and
 * head_dim): convert_kv_to_int4 (crates/serve/src/engine_ext.rs:158-210, src_row = dst_row
 * = 0, n_rows = the prompt length) and the per-position store of the int4 prefill
 * (crates/serve/src/forward_qwen3.rs:69-120: the chunk's k/v after norm and RoPE, e.g. from a
 * bf16 staging cache written by ema_pre_attention). Rows outside either capacity are an
 * error (EMA_ERR_CAPACITY). */
EMA_API int32_t ema_kvcache_quantize_int4(ema_stream_t stream, const ema_kvcache_desc* src, int32_t src_row,
                                          const ema_kvcache_desc* dst, int32_t dst_row, int32_t n_rows);
/* Convert rows [src_row, src_row + n_rows) of every (sequence, kv head) of `src` into rows
 * [dst_row, dst_row + n_rows) of `dst` (same batch, heads and head_dim; rows outside either
 * capacity are EMA_ERR_CAPACITY; ring rows are plain rows here):
 *   bf16 -> FP8   the quantisation of Fp8Cache::append (crates/kvcache/src/fp8.rs:47-68,
 *                 crates/ops/src/fp8.rs:71-92), as ema_pre_attention writes rows;
 *   FP8 -> bf16   the exact decoded values, what Fp8Cache::get hands SDPA (fp8.rs:60-68);
 *   bf16 -> int4  as ema_kvcache_quantize_int4.
 * Other pairs are EMA_ERR_UNSUPPORTED. */
EMA_API int32_t ema_kvcache_convert(ema_stream_t stream, const ema_kvcache_desc* src, int32_t src_row,
                                    const ema_kvcache_desc* dst, int32_t dst_row, int32_t n_rows);
/* Write `value` into the device int32 at `slot` on `stream` (a one-lane kernel, stream
 * ordered): the position a rotating cache's layer call passes as its offset, without a
 * host-to-device copy. No counterpart in the reference (MLX builds a scalar array). */
EMA_API int32_t ema_position_write(ema_stream_t stream, int32_t* slot, int32_t value);
/* Free buffers obtained from ema_kvcache_alloc, _alloc_fp8 or _alloc_int4 and clear the descriptor. */
EMA_API int32_t ema_kvcache_free(ema_kvcache_desc* desc);
/* Bytes held by K and V, exponents or scales and biases included (KvCache::memory_bytes,
 * crates/kvcache/src/lib.rs:75). */
EMA_API int32_t ema_kvcache_memory_bytes(const ema_kvcache_desc* desc, uint64_t* bytes);

/* Fused Qwen3 pre-attention for `batch` sequences of `n_tokens` new tokens.
 *   qkv      [batch, n_tokens, (n_heads + 2*n_kv_heads) * head_dim] bf16, order q|k|v
 *            (fused projection output, crates/serve/src/forward/projection.rs:105-128)
 *   q_norm_w, k_norm_w  [head_dim] bf16 (ignored with EMA_PRE_NO_NORM)
 *   offsets  device int32 [batch]: position of the first new token
 *   q_out    [batch, n_heads, n_tokens, head_dim] bf16
 * Per head vector: RMSNorm over head_dim (eps), split-half RoPE at offsets[b]+t
 * (base theta), then K and V are written into cache rows [offsets[b], offsets[b]+n_tokens).
 * Replaces forward_qwen3.rs:56-68,124-142 and compiled.rs:134-161.
 * Offsets are read on the device; offsets[b] + n_tokens > capacity writes nothing
 * for that sequence (callers guard on the host as decode_compiled.rs:18-20 does).
 * FP8 cache: each written K and V row is quantised per 64-element block (the bf16 k
 * after norm and RoPE, v as given), as Fp8Cache::append does (crates/kvcache/src/fp8.rs:47-68).
 * int4 cache: each written K and V row is quantised per 64-value group with MLX's affine
 * quantiser, as int4_update_and_dequant does (crates/serve/src/engine_ext.rs:131-157). */
EMA_API int32_t ema_pre_attention(ema_stream_t stream, const void* qkv, const void* q_norm_w,
                          const void* k_norm_w, float eps, float theta, const int32_t* offsets,
                          int32_t batch, int32_t n_tokens, int32_t n_heads, int32_t n_kv_heads,
                          int32_t head_dim, uint32_t flags, void* q_out,
                          const ema_kvcache_desc* cache);
/* ema_pre_attention over an FP8 cache that also writes each stored K and V row, decoded to
 * bf16 (code * 2^exp, exact), into the bf16 copy of the ema_prefill_attention_ws workspace
 * for the same max_kv_len (ema_prefill_workspace_size): row p of the copy for cache row p
 * (static caches: rows below max_kv_len). An ema_prefill_attention_ws call with
 * EMA_PREFILL_ROWS_DECODED then decodes only the other rows it attends, none with
 * EMA_PREFILL_CHUNK_ONLY over a static cache (a fresh prefill: the reference appends the
 * chunk and attends its round-tripped rows, crates/kvcache/src/fp8.rs:47-68). No
 * counterpart call in the reference; EMA_ERR_UNSUPPORTED for other caches. */
EMA_API int32_t ema_pre_attention_ws(ema_stream_t stream, const void* qkv, const void* q_norm_w,
                                     const void* k_norm_w, float eps, float theta, const int32_t* offsets,
                                     int32_t batch, int32_t n_tokens, int32_t n_heads, int32_t n_kv_heads,
                                     int32_t head_dim, uint32_t flags, void* q_out, const ema_kvcache_desc* cache,
                                     int32_t max_kv_len, void* workspace, uint64_t workspace_bytes);

/* Bytes at the start of every decode workspace that hold the split's arrival counters
 * (one per (sequence, kv head) segment, and one for the grid). They must be zero before a
 * workspace's first use (a zero-filled allocation, or one memset); every call returns them
 * to zero, so a workspace needs no clearing between calls, whatever their shapes. */
#define EMA_DECODE_COUNTER_BYTES 131072
/* Workspace (bytes) ema_decode_attention and ema_decode_step need for this shape: the
 * counters, then per-piece partial softmax states of the split (which need no
 * initialisation). Calls that share one workspace must not overlap. batch * n_kv_heads
 * is limited to EMA_DECODE_COUNTER_BYTES / 4 - 1 (EMA_ERR_UNSUPPORTED beyond). */
EMA_API int32_t ema_decode_workspace_size(int32_t batch, int32_t n_heads, int32_t n_kv_heads,
                                  int32_t head_dim, int32_t max_len, uint64_t* bytes);
/* Batched single-token decode attention over the static cache
 * (MlxCtx::sdpa_masked with the static mask, compiled.rs:163 / decode_eager.rs:140).
 *   q        [batch, n_heads, head_dim] bf16 (post norm/RoPE)
 *   lengths  device int32 [batch]: valid positions (offset + 1 after the write);
 *            clamped to [0, capacity]; a sequence with 0 valid positions yields zeros
 *   max_len  host upper bound of lengths (sizes the split; <= capacity). A bound below
 *            the true lengths still gives the exact result: the kernels take the split
 *            from the actual tile count, over the fewer workers the bound planned.
 *   out      [batch, n_heads * head_dim] bf16 (the o_proj input layout)
 * GQA: q head h reads kv head h / (n_heads / n_kv_heads).
 * FP8 cache: K/V rows are decoded exactly to bf16 (code value times 2^exp) and attended
 * as a bf16 cache holding those values would be.
 * int4 cache: attends the affine values scale * code + bias of every row (the reference
 * dequantizes the whole cache and runs the masked SDPA over it, decode_eager.rs:78-104).
 * Size limits (EMA_ERR_UNSUPPORTED beyond, also for ema_decode_step): batch * n_kv_heads *
 * ceil(capacity / 32) below 2^31 - 1, and for bf16 and int4 caches one (sequence, kv head)
 * plane, capacity * stride_pos bytes (int4: half that), within 4 GiB. */
EMA_API int32_t ema_decode_attention(ema_stream_t stream, const void* q, const ema_kvcache_desc* cache,
                             const int32_t* lengths, int32_t max_len, int32_t n_heads,
                             float scale, void* out, void* workspace, uint64_t workspace_bytes);

/* One fused decode step for `batch` sequences of one new token each: the
 * pre-attention of ema_pre_attention with n_tokens = 1 (q/k RMSNorm, RoPE, k and v
 * written into cache row offsets[b]) followed by ema_decode_attention over
 * offsets[b] + 1 positions, in one kernel pass plus the split merge. q stays in
 * registers (not written out). Replaces the per-layer attention slice of the
 * compiled decode step, crates/serve/src/compiled.rs:134-163.
 *   qkv      [batch, (n_heads + 2*n_kv_heads) * head_dim] bf16, order q|k|v
 *   offsets  device int32 [batch]; an offset outside [0, capacity) writes nothing; read
 *            only, unless flags hold EMA_STEP_ADVANCE (then advanced in place)
 *   max_len  host upper bound of offsets[b] + 1 (sizes the split; <= capacity)
 *   out      [batch, n_heads * head_dim] bf16
 * The workspace is the one ema_decode_workspace_size gives for max_len.
 * FP8 and int4 caches: the new k/v row is quantised as in ema_pre_attention and attended
 * in its decoded form, like every other row. */
EMA_API int32_t ema_decode_step(ema_stream_t stream, const void* qkv, const void* q_norm_w,
                                const void* k_norm_w, float eps, float theta,
                                int32_t* offsets, int32_t max_len, int32_t n_heads,
                                uint32_t flags, float scale, const ema_kvcache_desc* cache,
                                void* out, void* workspace, uint64_t workspace_bytes);

/* Size of the static scratch behind ema_decode_step_noalloc (8 MiB per device). */
#define EMA_NOALLOC_SCRATCH_BYTES (8ull << 20)
/* ema_decode_step without a workspace argument and without any device allocation: the
 * split's scratch lives in a static device array of EMA_NOALLOC_SCRATCH_BYTES per device,
 * located on the first call on each device. No counterpart in the reference (MLX
 * allocates inside its ops); it is for callers that cannot allocate device memory around
 * the step: code under HIP graph capture, tight serving loops, harnesses that forbid
 * allocation. Same arguments and results as ema_decode_step. A shape whose workspace
 * (ema_decode_workspace_size for max_len) exceeds the scratch returns EMA_ERR_WORKSPACE.
 * Every call on one device shares the array: calls that overlap on a device (concurrent
 * streams) race; stream-ordered calls do not. */
EMA_API int32_t ema_decode_step_noalloc(ema_stream_t stream, const void* qkv, const void* q_norm_w,
                                        const void* k_norm_w, float eps, float theta,
                                        int32_t* offsets, int32_t max_len, int32_t n_heads,
                                        uint32_t flags, float scale, const ema_kvcache_desc* cache,
                                        void* out);

/* Prefill / chunked-prefill attention over the static cache
 * (MlxCtx::sdpa(causal), blas.rs:82-101 via forward_qwen3.rs:150 and
 * attend_and_project, crates/ops/src/attention.rs:162-177).
 *   q          [batch, n_heads, n_tokens, head_dim] bf16
 *   q_offsets  device int32 [batch]: cache position of the first query; keys
 *              [0, q_offsets[b] + n_tokens) (or [q_offsets[b], ...) with CHUNK_ONLY)
 *   out        [batch, n_tokens, n_heads * head_dim] bf16
 * With EMA_PREFILL_CAUSAL, query i sees key j iff j <= q_offsets[b] + i.
 * bf16 caches only (EMA_ERR_UNSUPPORTED for FP8: use ema_prefill_attention_ws; for int4,
 * whose prefill the reference runs over the chunk's bf16 keys, use a bf16 cache and
 * ema_kvcache_quantize_int4). */
EMA_API int32_t ema_prefill_attention(ema_stream_t stream, const void* q, const ema_kvcache_desc* cache,
                              const int32_t* q_offsets, int32_t n_tokens, int32_t n_heads,
                              float scale, uint32_t flags, void* out);

/* Workspace (bytes) ema_prefill_attention_ws needs: 0 for a bf16 cache; for an FP8 cache
 * a bf16 copy of the attended rows, 2 * batch * n_kv_heads * rows * head_dim * 2, where rows
 * is max_kv_len for a static cache and the capacity for a rotating (EMA_KV_ROTATING) one:
 * a ring's positions sit at row p % capacity once they wrap, so its copy holds the whole
 * ring whatever max_kv_len says. */
EMA_API int32_t ema_prefill_workspace_size(const ema_kvcache_desc* cache, int32_t max_kv_len,
                                           uint64_t* bytes);
/* ema_prefill_attention for either cache format (the prefill over the reference's FP8
 * cache, whose SDPA sees the round-tripped values: crates/kvcache/src/fp8.rs:60-68). An
 * FP8 cache's attended rows are decoded exactly into bf16 in the workspace, and the bf16
 * prefill runs over that copy, so the result equals that of a bf16 cache holding the
 * decoded values. max_kv_len: host upper bound of q_offsets[b] + n_tokens (<= capacity;
 * rows at or past it are not attended); for a rotating cache it only has to lie in
 * [n_tokens, capacity], and every held row of the ring is decoded. The workspace needs no
 * initialisation; calls that share one must not overlap. */
EMA_API int32_t ema_prefill_attention_ws(ema_stream_t stream, const void* q, const ema_kvcache_desc* cache,
                                         const int32_t* q_offsets, int32_t n_tokens, int32_t n_heads,
                                         float scale, uint32_t flags, void* out, int32_t max_kv_len,
                                         void* workspace, uint64_t workspace_bytes);

/* Gated DeltaNet recurrent scan over n_tokens tokens (n_tokens = 1: the decode step of
 * gdn_step / gdn_step_metal, crates/ops/src/gdn.rs:83-150 and gdn_metal.rs:56-88; n_tokens
 * > 1: the token loop of gdn_forward, crates/ops/src/gdn_forward.rs:173-192). For each
 * token t and value head h, with key head h / (hv / hk):
 *   S = g S;  kv = S k;  delta = (v - kv) beta;  S = S + delta k^T;  y = S q
 * where S = state[b, h] is [dv, dk] f32.
 *   q, k:    [batch, n_tokens, hk, dk]  in `dtype`
 *   v:       [batch, n_tokens, hv, dv]  in `dtype`
 *   g, beta: [batch, n_tokens, hv] f32  the decay exp(-exp(A_log) softplus(a + dt_bias))
 *            and sigmoid(b), computed by the caller as in both reference paths
 *   state:   [batch, hv, dv, dk] f32, read and updated in place (zeros for a new sequence,
 *            as GdnState initialises it: gdn_forward.rs:166-170)
 *   y:       [batch, n_tokens, hv, dv] in `dtype` (gdn_step returns y cast to the
 *            activation type; pass EMA_DTYPE_F32 activations for the f32 y of
 *            gdn_step_metal)
 * dtype: EMA_DTYPE_BF16, EMA_DTYPE_F16 or EMA_DTYPE_F32. dk: 64 or 128; dv a multiple of
 * 16; hv a multiple of hk. q, k and state 16-byte aligned; v, y, g, beta element-aligned.
 * Calls that update the same state must not overlap. */
EMA_API int32_t ema_gdn_scan(ema_stream_t stream, const void* q, const void* k, const void* v,
                             const float* g, const float* beta, float* state, void* y,
                             int32_t batch, int32_t n_tokens, int32_t hk, int32_t hv, int32_t dk,
                             int32_t dv, int32_t dtype);

/* Workspace bytes for ema_gdn_scan_ws to run n_tokens tokens in one segment, into *bytes:
 * per 32-token chunk, batch * (hv * (128 * (dk + dv) + 5120) + hk * 128 * dk) bytes. Shapes
 * ema_gdn_scan rejects return its error. No counterpart in the reference, which allocates
 * its intermediates per call. */
EMA_API int32_t ema_gdn_scan_workspace_size(int32_t batch, int32_t n_tokens, int32_t hk, int32_t hv, int32_t dk,
                                            int32_t dv, uint64_t* bytes);

/* ema_gdn_scan with a workspace (the same arguments, semantics and tolerance). Scans of bf16
 * activations over at least 32 tokens with dv <= 512 and v 16-byte aligned run in WY form:
 * one parallel pass forms every 32-token chunk's matrices into the workspace, then one pass
 * carries the state through the chunks. A workspace smaller than
 * ema_gdn_scan_workspace_size's is used in segments of as many chunks as fit (at least one
 * chunk's bytes are required). Other calls run as ema_gdn_scan and leave the workspace
 * unused. The workspace needs no initialisation and must be 16-byte aligned; calls that
 * share one must not overlap. Replaces the same reference sites as ema_gdn_scan. */
EMA_API int32_t ema_gdn_scan_ws(ema_stream_t stream, const void* q, const void* k, const void* v,
                                const float* g, const float* beta, float* state, void* y,
                                int32_t batch, int32_t n_tokens, int32_t hk, int32_t hv, int32_t dk,
                                int32_t dv, int32_t dtype, void* workspace, uint64_t workspace_bytes);

/* y = x W^T over an affine-quantised W in MLX's packing: MLX quantized_matmul(x, w,
 * scales, biases, transpose=true, group_size, bits, "affine"), the call behind the
 * reference's qmatmul (crates/ops/src/quant.rs:57-76) for the q|k|v and o projections:
 *   y[m, n] = sum_k x[m, k] * (scales[n, k / group_size] * q[n, k] + biases[n, k / group_size])
 *   x:      [M, ldx] in `dtype` (row m's first K values are used)
 *   w:      [N, K * bits / 32] uint32; field k of row n is bits (k % (32 / bits)) * bits ..
 *           + bits - 1 of word k / (32 / bits) (lowest bits first)
 *   scales, biases: [N, K / group_size] in `dtype`
 *   y:      [M, ldy] in `dtype`; columns [0, N) of each row written, the rest untouched
 *           (ldy > N writes one piece of a wider row: the separate q, k and v projections
 *           of run_qkv land in one q|k|v row without a concatenation)
 * Up to 32 rows (and K not a multiple of 64): products are exact and accumulate in f32.
 * More than 32 rows with K a multiple of 64: as MLX's quantized matmul for many rows, the
 * weights are first dequantised into `dtype`, w = round(fma_f32(scale, q, bias)), and
 * x * w accumulates in f32. Either way y is rounded once (RNE) to `dtype`.
 * dtype: EMA_DTYPE_BF16 or EMA_DTYPE_F16. bits: 4 or 8; group_size: 32, 64 or 128; K a
 * multiple of group_size; ldx >= K, ldy >= N. x and w 16-byte aligned, ldx a multiple
 * of 8; scales, biases and y element-aligned. M = 0 is a no-op. */
EMA_API int32_t ema_quantized_matmul(ema_stream_t stream, const void* x, int64_t ldx, const uint32_t* w,
                                     const void* scales, const void* biases, void* y, int64_t ldy,
                                     int32_t M, int32_t N, int32_t K, int32_t group_size, int32_t bits,
                                     int32_t dtype);

#ifdef __cplusplus
}
#endif
#endif /* EMA_ATTN_H */
