/*
 * ferrum_q8.h — Q8_0 weight GEMV/GEMM of libferrum_kv.so (gfx950, HIP).
 *
 * The decode layer's projections around the KV-cache path: Llama::forward_one_token
 * calls linear() (crates/model/src/weights.rs:15-26) for attn_q/attn_k/attn_v before
 * RoPE and the KV append and for attn_output after the attention loop
 * (crates/model/src/llama.rs:185-205,249-255), and linear() is Kernels::gemv. These
 * entry points replace Kernels::gemv and Kernels::gemm for DType::Q8_0 weights
 * (crates/kernels/src/lib.rs trait Kernels; scalar.rs:84-116; avx2.rs:103-144).
 *
 * Result, bit for bit: per token the f32 activation row is quantized to Q8_0 as
 * Q8Activation::quantize_into (crates/kernels/src/q8_dot.rs:35-61; the scale rounded
 * to binary16 with the reference's ties-away f32_to_f16_bits, q8_dot.rs:111-139), and
 * y = dot_q8_row_q8_act (q8_dot.rs:72-109): starting from +0, for each 32-value block
 * in order, acc += (float)sumi * (w_scale * x_scale), sumi the int32 dot of the two
 * int8 runs. The reference's scalar and AVX2 backends agree to the bit on this
 * (crates/kernels/src/tests.rs:770-830), and so does this one.
 *
 * Layout: w is `rows` rows of cols/32 blocks of 34 bytes ([f16 scale LE][32 x i8],
 * crates/core-types/src/dtype.rs:19-21; GGUF Q8_0 tensor bytes as stored), row-major.
 * x is f32 [n_tokens][cols], y is f32 [n_tokens][rows] (GemmArgs; par.rs:9-26).
 * Lengths are element counts, as the reference's slice lengths (w_len in bytes).
 *
 * All pointers are device pointers; the call is asynchronous on `stream` (a
 * hipStream_t, or NULL for the null stream) of the calling thread's current device,
 * allocates nothing and needs no workspace.
 *
 * Errors (FKV_ERR_* of ferrum_kv.h; message from fkv_last_error()), checked in the
 * reference's order (crates/kernels/src/validate.rs:110-150):
 *   cols == 0                      FKV_ERR_KERNEL "kernel: empty dot"
 *   cols % 32 != 0                 FKV_ERR_KERNEL "kernel: q8_0 k is not a multiple of 32"
 *   size overflow                  FKV_ERR_KERNEL "kernel: shape overflow"
 *   w_len != rows*(cols/32)*34     FKV_ERR_KERNEL "kernel: length mismatch"
 *   x_len, y_len                   FKV_ERR_KERNEL "kernel: length mismatch"
 * then, at this device boundary: null pointers, w not 2-byte aligned, x or y not
 * 4-byte aligned, or a matrix beyond one launch (cols > 65,536, rows or n_tokens
 * >= 2^31 - 2^16) -> FKV_ERR_INVALID. rows == 0 (with w_len == 0) succeeds and
 * launches nothing.
 */
#ifndef FERRUM_Q8_H
#define FERRUM_Q8_H

#include <stdint.h>

#include "ferrum_kv.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Kernels::gemv(DType::Q8_0, w, rows, cols, x, y) (crates/kernels/src/scalar.rs:84-96,
 * 191-204; validate.rs:110-124): y[r] for r < rows from one activation row x[cols]. */
int32_t fkv_gemv_q8_0(const void* w, uint64_t w_len, uint64_t rows, uint64_t cols,
                      const float* x, uint64_t x_len, float* y, uint64_t y_len, void* stream);

/* Kernels::gemm(GemmArgs { dtype: Q8_0, .. }) (crates/kernels/src/scalar.rs:98-116;
 * validate.rs:126-141): y[t][r] for t < n_tokens, each token exactly as
 * fkv_gemv_q8_0 on x[t]. n_tokens == 0 succeeds before any check (scalar.rs:99-101). */
int32_t fkv_gemm_q8_0(const void* w, uint64_t w_len, uint64_t rows, uint64_t cols,
                      const float* x, uint64_t x_len, uint64_t n_tokens, float* y,
                      uint64_t y_len, void* stream);

/* Kernels::gemm of up to 4 Q8_0 matrices that take the same activation rows (the
 * layer's attn_q/attn_k/attn_v of one normed row, crates/model/src/llama.rs:185-205, or
 * ffn_gate/ffn_up), in one launch: y[m] is bit for bit what fkv_gemm_q8_0(w[m], ...) gives.
 * No counterpart in the reference, which makes one gemv call per matrix; this saves the
 * small matrices' per-launch cost. w, w_len, rows, y, y_len are host arrays of n_mats
 * entries (the pointers in them are device pointers). Errors: n_mats outside 1..4 or a
 * null array -> FKV_ERR_INVALID; then n_tokens == 0 succeeds; then each matrix's checks
 * as fkv_gemm_q8_0's, in matrix order, the first failure returned and nothing launched. */
int32_t fkv_gemm_q8_0_multi(uint32_t n_mats, const void* const* w, const uint64_t* w_len,
                            const uint64_t* rows, uint64_t cols, const float* x,
                            uint64_t x_len, uint64_t n_tokens, float* const* y,
                            const uint64_t* y_len, void* stream);

/* fkv_gemm_q8_0_multi for batches of activation rows (a decode step's sequences, a
 * prefill chunk) on the matrix cores, with the same results bit for bit. No counterpart
 * in the reference, which loops over tokens (scalar.rs:98-116); the entry points above
 * read every weight once per 4 tokens. Here each activation row is quantized once into
 * `workspace`, and one v_mfma_i32_16x16x32_i8 gives a 32-value block's exact integer
 * dots for 16 weight rows x 16 tokens; each output then accumulates
 * f32(sumi) * (w_scale * x_scale) block by block in order, as dot_q8_row_q8_act does.
 * That path runs when n_tokens >= 8, cols is a multiple of 1024 and every w is 16-byte
 * aligned; other calls run the GEMV kernel (workspace unused). Same checks, strings
 * and order as fkv_gemm_q8_0_multi; then, for a call that takes the matrix-core path,
 * a workspace that is NULL, smaller than fkv_gemm_q8_0_batched_workspace_size() or not
 * 16-byte aligned is FKV_ERR_INVALID "gemm workspace too small" / "gemm workspace must
 * be 16-byte aligned". The workspace needs no initialisation; calls that share one
 * must not overlap. */
int32_t fkv_gemm_q8_0_batched_workspace_size(uint64_t cols, uint64_t n_tokens,
                                             uint64_t* bytes_out);
int32_t fkv_gemm_q8_0_batched(uint32_t n_mats, const void* const* w, const uint64_t* w_len,
                              const uint64_t* rows, uint64_t cols, const float* x,
                              uint64_t x_len, uint64_t n_tokens, float* const* y,
                              const uint64_t* y_len, void* workspace, uint64_t workspace_bytes,
                              void* stream);

#ifdef __cplusplus
}
#endif

#endif /* FERRUM_Q8_H */
