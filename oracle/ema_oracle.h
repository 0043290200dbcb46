/*
 * CPU oracle for the Qwen3 attention hot path (TEST INFRASTRUCTURE ONLY).
 *
 * This library is the checker: only tests, the smoke entry and the bench's
 * CPU-baseline leg may load it. The product path (engine-mlx_amd/) never calls
 * it and never falls back to it.
 *
 * It restates, in plain C, the semantics of the MLX primitives the reference
 * calls on this path (reference: dangranaz/engine-mlx 0.1.18):
 *   - mlx_fast_rms_norm           crates/mlx-ffi/src/ops/real/blas.rs:5-9
 *   - mlx_fast_rope(_dynamic)     crates/mlx-ffi/src/ops/real/blas.rs:67-80
 *       (traditional=false, base=theta, scale=1.0, dims=head_dim)
 *   - static KV write             crates/serve/src/compiled.rs:157-161 (scatter_single)
 *                                 crates/serve/src/forward_qwen3.rs:124-142 (slice_update)
 *   - masked / causal SDPA        crates/mlx-ffi/src/ops/real/transform.rs:8-29 ("array" mask)
 *                                 crates/mlx-ffi/src/ops/real/blas.rs:82-101 ("causal")
 *   - op order norm -> transpose -> rope -> write -> sdpa
 *                                 crates/serve/src/forward_qwen3.rs:52-152
 *   - FP8 KV format               crates/ops/src/fp8.rs, crates/kvcache/src/fp8.rs
 *   - int4 affine KV format       crates/serve/src/engine_ext.rs:92-157 (MLX affine quantize)
 *   - Gated DeltaNet step/scan    crates/ops/src/gdn.rs:83-150, gdn_forward.rs:173-192
 *   - affine quantized_matmul     crates/mlx-ffi/src/ops/real/transform.rs:77-88 via
 *                                 crates/ops/src/quant.rs:57-76 (transpose = true)
 *
 * bf16 tensors are passed as uint16_t bit patterns (IEEE bfloat16, RNE).
 *
 * Layouts (all contiguous, row-major):
 *   qkv    [B, T, (Hq + 2*Hkv) * D]   fused projection output, order q | k | v
 *   q      [B, Hq, Tq, D]             attention-ordered queries
 *   cache  [B, Hkv, cap, D]           static K (and V) cache
 *   out    [B, Tq, Hq * D]            attention output, o_proj input layout
 *
 * Parity pins: see the header comment of each function (tests/test_oracle.py
 * holds the checks).
 */
#ifndef EMA_ORACLE_H
#define EMA_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ORA_FLAG_NO_NORM 1u /* q_norm/k_norm are None (optional_qk_norm no-op) */
#define ORA_FLAG_NO_ROPE 2u /* NoPE layer (apply_rope with use_rope=false)     */
#define ORA_FLAG_NO_Q_NORM 8u  /* q_norm None, k_norm given (each norm is optional on its own) */
#define ORA_FLAG_NO_K_NORM 16u /* k_norm None, q_norm given                                      */

/* bf16 <-> f32 (RNE, NaN kept quiet). */
uint16_t ora_f32_to_bf16(float f);
float ora_bf16_to_f32(uint16_t h);
void ora_f32_to_bf16_array(const float* in, uint16_t* out, size_t n);
void ora_bf16_to_f32_array(const uint16_t* in, float* out, size_t n);

/* Counter-based N(mean, std) generator (splitmix64 -> Box-Muller), rounded
 * to bf16. Element i depends only on (seed, i). */
void ora_fill_normal_bf16(uint16_t* out, size_t n, uint64_t seed, float mean, float std);
void ora_fill_normal_f32(float* out, size_t n, uint64_t seed, float mean, float std);

/* RMSNorm over the last axis, MLX fast::rms_norm semantics:
 *   y = bf16( w * bf16( x * rsqrt(mean(x^2) + eps) ) ), statistics in f64. */
void ora_rms_norm(const uint16_t* x, const uint16_t* w, int64_t rows, int D, float eps,
                  uint16_t* out);

/* Non-traditional (split-half) RoPE on rows of length D, MLX fast::rope
 * semantics with dims=D, scale=1: pair (x[i], x[i+D/2]) rotated by
 * angle = pos * theta^(-2i/D), inv-frequency and angle formed in f32.
 * x is [rows, D]; pos[r] is the absolute position of row r. */
void ora_rope(const uint16_t* x, const int32_t* pos, int64_t rows, int D, float theta,
              uint16_t* out);

/* Fused pre-attention step for B sequences of T new tokens:
 *   q,k <- rms_norm (unless NO_NORM), q,k <- rope at off[b]+t (unless NO_ROPE),
 *   q_out[b,h,t,:] = q ; kcache[b,h,off[b]+t,:] = k ; vcache[...] = v.
 * Rows of the caches outside [off[b], off[b]+T) are left untouched.
 * Returns 0, or -1 if some off[b] < 0 or off[b] + T > cap. */
int ora_pre_attention(const uint16_t* qkv, const uint16_t* q_norm_w, const uint16_t* k_norm_w,
                      float eps, float theta, const int32_t* off, int B, int T, int Hq, int Hkv,
                      int D, uint32_t flags, uint16_t* q_out, uint16_t* kcache, uint16_t* vcache,
                      int cap);

/* Scaled dot-product attention over the static cache, GQA mapping
 * q-head h -> kv-head h / (Hq/Hkv).
 * For batch b, keys live in [kv_begin[b], kv_len[b]) (kv_begin may be NULL = 0).
 * causal != 0: query row i may see key j only if j <= kv_len[b] - Tq + i
 *              (query block aligned to the end of the key range, MLX "causal").
 * causal == 0: every key in range is visible (the decode mask of
 *              crates/serve/src/engine_ext.rs:237-260 reduces to this with
 *              kv_len = offset + 1).
 * A query row with no visible key yields zeros.
 * precision 0: f64 scores/softmax/PV (the accurate oracle).
 * precision 1: f32 scores/softmax/PV (MLX CPU-stream arithmetic), OpenMP over
 *              (b, head, row); used as the timed CPU baseline. */
void ora_sdpa(const uint16_t* q, const uint16_t* kcache, const uint16_t* vcache,
              const int32_t* kv_len, const int32_t* kv_begin, int B, int Hq, int Hkv, int Tq,
              int D, int cap, float scale, int causal, int precision, uint16_t* out);

/* Split-K building blocks (flash-decoding). For one query vector q[D] and
 * keys rows [0, n) of K/V (row stride D): m = max_j s_j, l = sum_j exp(s_j - m),
 * acc = sum_j exp(s_j - m) v_j with s_j = scale * q.k_j, all in f64. */
void ora_sdpa_partial(const uint16_t* q, const uint16_t* k, const uint16_t* v, int n, int D,
                      float scale, double* m, double* l, double* acc);
/* Merge P partials by log-sum-exp; writes out[D] = (sum_p e^{m_p-M} acc_p) / (sum_p e^{m_p-M} l_p). */
void ora_lse_merge(const double* m, const double* l, const double* acc, int P, int D,
                   double* out);

/* Number of OpenMP threads ora_sdpa(precision=1) uses. */
int ora_num_threads(void);

/* ---- FP8 E4M3FN KV format: crates/ops/src/fp8.rs (used by crates/kvcache/src/fp8.rs) ----
 * E4M3FN (OCP): sign, 4 exponent bits (bias 7), 3 mantissa bits; exponent field 0 is
 * subnormal (mant * 2^-9); no infinities; codes 0x7F / 0xFF are NaN; largest finite 448. */

/* Value of an E4M3FN code (e4m3fn_value, fp8.rs:20-29, plus the sign bit). */
float ora_e4m3_value(uint8_t code);
/* e4m3fn_dequant (fp8.rs:36-64): the E4M3FN value nearest to x, ties to the even code,
 * |x| saturated at 448; NaN gives +448 (f32::min returns the non-NaN operand). The sign is
 * that of x < 0 as in the reference (so -0.0 gives +0). *code receives the byte. */
float ora_e4m3fn_round(float x, uint8_t* code);
/* The reference's block scale exponent, ceil(log2(amax / 448)) with
 * amax = max(1e-4, max_i |x_i|) (NaN ignored): fp8.rs:80-84 and :123-126, in f32 with the C
 * library's log2f and ceilf, as Rust's f32::log2 / f32::ceil do on Linux. */
int ora_fp8_block_exp(const float* x, int n);
/* Exponent of the reference formula for a given amax / 448 = r: ceilf(log2f(r)) (ref = 1) or
 * ceilf((float)log2((double)r)) (ref = 0, the device kernels' form). */
int ora_fp8_exp_of(float r, int ref);
/* Count of r = 2^k * (1 + n * 2^-23), k in [kmin, kmax], |n| < nulps, for which the two forms
 * of ora_fp8_exp_of differ. */
int64_t ora_fp8_exp_mismatches(int kmin, int kmax, int nulps);
/* fp8_round_trip_slice (fp8.rs:71-92), in place on rows of D values: values [0, D - n_rot) in
 * 64-value blocks are replaced by e4m3fn_dequant(clamp(v / s, -448, 448)) * s with
 * s = 2^ora_fp8_block_exp(block); the RoPE tail [D - n_rot, D) passes through. */
void ora_fp8_round_trip(float* x, int64_t rows, int D, int n_rot);
/* The stored form of the same quantisation (n_rot = 0, D a multiple of 64): codes[i] = the
 * E4M3FN byte of row value i, exps[r * D/64 + b] = exponent of block b of row r, so that
 * value = e4m3(code) * 2^exp. */
void ora_fp8_quantize_rows(const float* x, int64_t rows, int D, uint8_t* codes, int8_t* exps);
/* value = e4m3(code) * 2^exp, exact in f32. */
void ora_fp8_dequantize_rows(const uint8_t* codes, const int8_t* exps, int64_t rows, int D, float* out);

/* ---- 4-bit affine KV format: the reference's int4 KV buffers (crates/serve/src/engine_ext.rs:92-157)
 * filled by quantize_kv_native and read through dequantize_kv_native
 * (crates/mlx-ffi/src/ops/real/quant.rs:8-64): mlx_quantize / mlx_dequantize with mode "affine",
 * group 64, 4 bits. MLX itself (mlx-sys 0.2 over mlx-c, with the global_scale argument of MLX
 * 0.29 and later) is a third-party dependency absent here; these restate its published
 * affine kernels (affine_quantize / affine_dequantize), the same ones the reference's Metal
 * stream runs. Per group of 64 values, f32 arithmetic:
 *   scale = max((max - min) / 15, 1e-7); side = |min| > |max|; scale = side ? scale : -scale;
 *   edge = side ? min : max; q0 = round(edge / scale);
 *   q0 != 0: scale = edge / q0, bias = edge;  q0 == 0: bias = 0;
 *   code = min(round((x - bias) / scale), 15)   (round: half away from zero; codes >= 0)
 * scale and bias are stored rounded to bf16 (the input dtype); codes use the f32 values.
 * Words: value i of a row at bits 4(i % 8) of word i / 8 (lowest bits first).
 * Parity against MLX itself is unpinned (no MLX here and no int4 vectors in the reference's
 * tests); tests/test_oracle_int4.py pins the properties that the algorithm fixes. */
void ora_int4_quantize_rows(const float* x, int64_t rows, int D, uint32_t* words, uint16_t* scales,
                            uint16_t* biases);
/* MLX affine_dequantize into bf16: out = bf16(scale * code + bias), one rounding of the exact
 * affine value. MLX's kernel evaluates `scale * d + bias` as one expression, which its
 * clang-based Metal compiler contracts into a fused multiply-add (scale * code is exact in
 * f32 in any case); were the product rounded to bf16 first, values whose product and bias
 * cancel would differ by up to half a bf16 step of scale * code. Not pinned against MLX. */
void ora_int4_dequantize_rows(const uint32_t* words, const uint16_t* scales, const uint16_t* biases, int64_t rows,
                              int D, float* out);

/* ---- Gated DeltaNet recurrent scan ----
 * gdn_step (crates/ops/src/gdn.rs:83-150; the fused kernel body gdn_metal.rs:16-50 does the
 * same arithmetic) applied token by token as gdn_forward does (gdn_forward.rs:173-192), in
 * double. For each token t and value head h, with key head h / (hv / hk) (the tile-based
 * expansion of gdn.rs:100-110):
 *   S = g S (gdn.rs:97-99);  kv = S k (:112-115);  delta = (v - kv) beta (:117-121);
 *   S = S + delta k^T (:123-126);  y = S q (:138-141)
 * with S = state[b, h] of shape [dv, dk].
 *   q, k [B, T, hk, dk]; v [B, T, hv, dv]; g, beta [B, T, hv]  (f32 inputs)
 *   state [B, hv, dv, dk] double, updated in place; y [B, T, hv, dv] double. */
void ora_gdn_scan(const float* q, const float* k, const float* v, const float* g, const float* beta,
                  double* state, double* y, int B, int T, int hk, int hv, int dk, int dv);

/* MLX affine quantized_matmul(x, w, scales, biases, transpose=true, group_size, bits)
 * (transform.rs:77-88, called by qmatmul, quant.rs:57-76, and the fused / separate
 * projections, crates/serve/src/forward/projection.rs:105-152), in double:
 *   y[m, n] = sum_k x[m, k] * (scales[n, k / gs] * q[n, k] + biases[n, k / gs])
 * with q[n, k] the bits-wide field (k % (32 / bits)) * bits .. +bits of word
 * wq[n, k / (32 / bits)] (lowest bits first: MLX's affine packing for widths that divide
 * 32). Weight row n is output column n (transpose = true: y = x W^T, W [N, K]).
 *   x [M, K] f32 (the bf16/f16 activations as f32); wq [N, K * bits / 32] uint32;
 *   scales, biases [N, K / gs] f32; y [M, N] double. bits in {2, 4, 8}; K % gs == 0. */
void ora_qmatmul(const float* x, const uint32_t* wq, const float* scales, const float* biases,
                 int M, int N, int K, int gs, int bits, double* y);
/* The dequantised weight W [N, K] = scales * q + biases (MLX dequantize, affine mode,
 * transform.rs:45-58), in double. */
void ora_dequantize(const uint32_t* wq, const float* scales, const float* biases, int N, int K,
                    int gs, int bits, double* w);

#ifdef __cplusplus
}
#endif
#endif
