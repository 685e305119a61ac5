/*
 * ferrum_oracle.h — CPU restatement of Ferrum's KV-cache path (TEST INFRASTRUCTURE).
 *
 * This library is the checker, never the product: only tests/, the smoke() of
 * __graft_entry__.py and the cpu_baseline leg of bench.py load it. The shipped
 * path is libferrum_kv.so (HIP); it never calls into this file.
 *
 * Every function names the reference lines it restates. The paged functions
 * (fo_append, fo_gather_*, fo_copy_blocks, fo_attention) have no counterpart
 * in the reference, whose pool is dense (crates/kvcache/src/pool.rs:1-18):
 * they apply the reference's per-position semantics (pool.rs:122-204,
 * crates/model/src/llama.rs:220-247) through the paged layout documented in
 * include/ferrum_kv.h.
 *
 * Pinning (what checks each function against something other than itself):
 *   fo_f16_to_f32          exhaustive vs closed-form f64 formula + known values
 *                          (dtype.rs:160-199), and vs numpy float16
 *   fo_f32_to_f16 (RNE)    exhaustive 2^32 vs the x86 F16C instruction (fo_selftest)
 *                          and vs numpy astype(float16) on samples
 *   fo_f32_to_f16 (AWAY)   exhaustive 2^32 vs an f64 nearest-ties-away search
 *   fo_q8_quantize_*       reference KAT tests.rs:299-309, tie/rounding cases,
 *                          invariants (|q|<=127, amax lane = +-127, error <= d/2)
 *   fo_q8_dequant          every code x 65,536 scales (kernels_contract.rs:700-744)
 *   fo_q8_gemm             the reference KAT tests.rs:291-309; exact closed forms
 *                          (power-of-two scales: integer matmul; a 4-block row whose
 *                          left-to-right f32 sum differs from every other order; an
 *                          f16 tie of the activation scale, which rounds away);
 *                          sign and power-of-two scaling symmetries; f64 bound
 *   fo_dot, fo_softmax     KATs tests.rs:178-195, kernels_contract.rs:437-467
 *   fo_rope                KATs tests.rs:197-239 (pos 0 bit-identity, dims past rope_dim
 *                          untouched, NORMAL pairing); the rotation against an f64
 *                          evaluation of the same angle formula; pair norms kept
 *   fo_attention           numpy f64 brute force + closed forms (ctx=1, equal keys,
 *                          dominant key, non-finite max)
 *   fo_prefill_attention   equals fo_attention run once per query position (the
 *                          definition) and an f64 causal brute force
 *   fo_dense_*             the pool.rs:233-308 unit tests
 *   fo_avx2_*              bit-identity of dot to fo_dot (tests.rs:616-621);
 *                          attention within tolerance of fo_attention
 */
#ifndef FERRUM_ORACLE_H
#define FERRUM_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct fo_layout {
  uint32_t n_layers;
  uint32_t n_kv_heads;
  uint32_t head_dim;
  uint32_t block_size;
  uint64_t num_blocks;
  int32_t dtype;    /* 0 f32, 1 f16, 8 q8_0 */
  int32_t rounding; /* 0 nearest-even, 1 ties away */
} fo_layout;

uint64_t fo_tile_bytes(const fo_layout* l);
uint64_t fo_block_bytes(const fo_layout* l);

float fo_f16_to_f32(uint16_t bits);
uint16_t fo_f32_to_f16(float x, int32_t rounding);
void fo_f32_to_f16_array(const float* x, uint16_t* out, uint64_t n, int32_t rounding);
void fo_f16_to_f32_array(const uint16_t* x, float* out, uint64_t n);

void fo_q8_quantize_block(const float* x32, int32_t rounding, uint16_t* scale_out,
                          int8_t* q_out);
/* Ferrum 34-byte blocks ([f16 scale LE][32 x i8]) for n values (n % 32 == 0). */
void fo_q8_quantize_row(const float* x, uint64_t n, int32_t rounding, uint8_t* out);
void fo_q8_dequant(const uint8_t* blocks, uint64_t n, float* out);
/* Q8_0 weight GEMM/GEMV (ggml q8_0 . q8_0): y[t*rows + r], x [n_tokens][cols]. */
void fo_q8_gemm(const uint8_t* w, uint64_t rows, uint64_t cols, const float* x,
                uint64_t n_tokens, float* y, int32_t threads);

float fo_dot(const float* a, const float* b, uint64_t n);
void fo_softmax(float* x, uint64_t n);
void fo_rope(float* data, uint64_t n_rows, uint32_t head_dim, uint32_t rope_dim, uint32_t pos,
             float theta);

/* Returns the number of skipped out-of-range slots. */
uint64_t fo_append(const fo_layout* l, uint8_t* pool, uint32_t layer, const float* k,
                   const float* v, const int64_t* slots, uint64_t n_tokens);
void fo_gather_slots(const fo_layout* l, const uint8_t* pool, uint32_t layer,
                     const int64_t* slots, uint64_t n_tokens, int32_t format, void* out_k,
                     void* out_v);
void fo_gather_tables(const fo_layout* l, const uint8_t* pool, uint32_t layer,
                      const int32_t* block_tables, uint32_t max_blocks, const int32_t* ctx_lens,
                      const int64_t* out_offsets, uint32_t n_seqs, int32_t format,
                      void* out_k, void* out_v);
void fo_copy_blocks(const fo_layout* l, uint8_t* pool, const int64_t* pairs, uint64_t n_pairs);
void fo_attention(const fo_layout* l, const uint8_t* pool, uint32_t layer, uint32_t n_heads,
                  const float* q, float* out, const int32_t* block_tables, uint32_t max_blocks,
                  const int32_t* ctx_lens, uint32_t n_seqs, float scale);

/* Prefill: query i of sequence s at position ctx_lens[s] - q_lens[s] + i attends
 * to positions 0 ..= that position (crates/model/src/llama.rs:363-378). */
void fo_prefill_attention(const fo_layout* l, const uint8_t* pool, uint32_t layer,
                          uint32_t n_heads, const float* q, float* out,
                          const int32_t* block_tables, uint32_t max_blocks,
                          const int32_t* ctx_lens, const int32_t* q_lens,
                          const int64_t* q_offsets, uint32_t n_seqs, float scale);

/* AVX2 restatement used as the timed CPU baseline (crates/kernels/src/avx2.rs). */
int32_t fo_avx2_available(void);
float fo_avx2_dot(const float* a, const float* b, uint64_t n);
void fo_avx2_softmax(float* x, uint64_t n);
void fo_avx2_attention(const fo_layout* l, const uint8_t* pool, uint32_t layer,
                       uint32_t n_heads, const float* q, float* out,
                       const int32_t* block_tables, uint32_t max_blocks,
                       const int32_t* ctx_lens, uint32_t n_seqs, float scale,
                       int32_t n_threads);
int32_t fo_max_threads(void);

/* Dense revision-1 pool (crates/kvcache/src/pool.rs). Codes: 0 ok, 1 cache,
 * 2 unavailable. *msg receives the FerrumError Display string. */
typedef struct fo_dense fo_dense;
int32_t fo_dense_new(uint64_t n_layers, uint64_t n_kv_heads, uint64_t head_dim,
                     uint64_t max_seq_len, uint64_t max_slots, fo_dense** out,
                     const char** msg);
void fo_dense_destroy(fo_dense* p);
uint64_t fo_dense_storage_len(const fo_dense* p);
int32_t fo_dense_alloc(fo_dense* p, uint32_t* slot, const char** msg);
int32_t fo_dense_free(fo_dense* p, uint32_t slot, const char** msg);
int32_t fo_dense_seq_len(const fo_dense* p, uint32_t slot, uint64_t* out, const char** msg);
int32_t fo_dense_append_layer(fo_dense* p, uint32_t slot, uint64_t layer, const float* k,
                              uint64_t k_len, const float* v, uint64_t v_len,
                              const char** msg);
int32_t fo_dense_commit_token(fo_dense* p, uint32_t slot, const char** msg);
int32_t fo_dense_k(const fo_dense* p, uint32_t slot, uint64_t layer, uint64_t pos, float* out,
                   const char** msg);
int32_t fo_dense_v(const fo_dense* p, uint32_t slot, uint64_t layer, uint64_t pos, float* out,
                   const char** msg);
int32_t fo_dense_abandon_partial(fo_dense* p, uint32_t slot, const char** msg);
int32_t fo_dense_uncommit_token(fo_dense* p, uint32_t slot, const char** msg);

/* Exhaustive self-checks over all 2^32 f32 inputs. Returns the number of
 * mismatches; *first_bad receives the first failing input bits.
 * which = 0: RNE vs F16C hardware conversion (non-NaN), 1: ties-away vs an
 * f64 nearest search. stride > 1 samples every stride-th input. */
uint64_t fo_selftest_f16(int32_t which, uint32_t stride, uint32_t* first_bad);

#ifdef __cplusplus
}
#endif

#endif
