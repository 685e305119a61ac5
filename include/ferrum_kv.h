/*
 * ferrum_kv.h — C ABI of the MI355X (gfx950) paged KV-cache hot path.
 *
 * Two surfaces share one library (libferrum_kv.so):
 *
 *  1. The revision-1 compat surface (fkv_kvpool_*). It mirrors Ferrum's
 *     `trait KvPool` (/root/reference/crates/core-types/src/kv.rs:21-46) and the
 *     inherent methods of `PreallocatedKvPool`
 *     (/root/reference/crates/kvcache/src/pool.rs:20-231) one entry point per
 *     method, with the same checks in the same order and the same message
 *     strings. Storage is device memory; K/V cross the boundary as host f32
 *     arrays and reads copy out instead of borrowing.
 *
 *  2. The paged surface (fkv_paged_*, fkv_block_*, fkv_append, fkv_gather_*,
 *     fkv_copy_blocks, fkv_swap_*, fkv_decode_attention*). Ferrum revision 1
 *     has no paged pool (its pool is one dense slot per sequence, pool.rs:1-18),
 *     so this is a new interface placed beside the frozen one, not new methods
 *     on it (core-types/src/lib.rs:3-6, :44-45). Every device operation is
 *     asynchronous on the stream it is given and takes device pointers.
 *
 * Errors: every entry point returns an fkv_status. A non-zero status leaves a
 * thread-local message readable with fkv_last_error(), formatted exactly as
 * Ferrum's `FerrumError` Display (core-types/src/error.rs:21-46):
 *   FKV_ERR_CACHE       -> "cache: <msg>"      (FerrumError::Cache)
 *   FKV_ERR_UNAVAILABLE -> "<msg>"             (FerrumError::Unavailable, HTTP 503)
 *   FKV_ERR_KERNEL      -> "kernel: <msg>"     (FerrumError::Kernel)
 *   FKV_ERR_INVALID     -> "<msg>"             (FerrumError::InvalidRequest)
 *   FKV_ERR_INTERNAL    -> "<msg>"             (FerrumError::Internal; HIP failures)
 *
 * Threading: a pool handle is single-writer, like `&mut self` in Ferrum.
 * Concurrent calls on one handle must be serialised by the caller.
 *
 * HBM layout of a paged pool (one device allocation):
 *   pool[block][layer][kv (0=K,1=V)][kv_head][tile]
 *   tile (F32)   : [block_size tokens][head_dim] elements
 *   tile (F16 K) : [head_dim/8][block_size][8]: 16-byte runs of 8 dims, token-
 *                  contiguous per run (head_dim padded to a multiple of 8)
 *   tile (F16 V) : [head_dim][block_size]: dim-major
 *   tile (Q8_0)  : int8 quants in 16-token sub-tiles of 16*head_dim bytes, each in
 *                  the matrix-core operand order (t = token % 16):
 *                    K dim c*32+g*8+e at (c/2)*1024 + (g*16+t)*16 + (c%2)*8 + e
 *                    V dim m*16+j     at (m/4)*1024 + ((t/4)*16+j)*16 + (m%4)*4 + t%4
 *                  then f16 scales [block_size][head_dim/32] (one per 32-value run
 *                  of a token row, Ferrum's Q8_0 block). Needs head_dim % 64 == 0
 *                  and block_size % 16 == 0.
 * The F16 and Q8_0 orders are the operand orders of the MFMA attention kernels: one
 * load instruction reads 1 KiB of K or 512 B of V of consecutive bytes (F16). A block holds
 * every layer of block_size consecutive tokens, and the (block, layer, kv, head)
 * tile is contiguous (4 KiB for f16, D=128, B=16). Slot = block * block_size +
 * offset_in_block (the vLLM slot-mapping convention). The gather entry points
 * return token rows whatever the tile order.
 */
#ifndef FERRUM_KV_H
#define FERRUM_KV_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Revision of this ABI. 2: fkv_paged_take_fault_flags, fkv_paged_read and
 * fkv_paged_write take a stream; fkv_prefill_attention takes a workspace. A binding
 * checks fkv_abi_version() against the value it was written for before any other
 * call: C symbols carry no signature, so a library of another revision still links. */
#define FKV_ABI_VERSION 2

/* Status codes; one per FerrumError variant the path can return. */
#define FKV_OK 0
#define FKV_ERR_CACHE 1
#define FKV_ERR_UNAVAILABLE 2
#define FKV_ERR_KERNEL 3
#define FKV_ERR_INVALID 4
#define FKV_ERR_INTERNAL 5

/* KV storage dtypes. Values are the ggml type ids of core-types/src/dtype.rs:27-33. */
#define FKV_DTYPE_F32 0
#define FKV_DTYPE_F16 1
#define FKV_DTYPE_Q8_0 8

/* f32 -> binary16 rounding used for F16 storage and for Q8_0 block scales.
 * NEAREST_EVEN is IEEE 754 roundTiesToEven (the default).
 * HALF_AWAY reproduces Ferrum's only encoder, `f32_to_f16_bits`
 * (crates/kernels/src/q8_dot.rs:111-139), which rounds ties away from zero. */
#define FKV_ROUND_NEAREST_EVEN 0
#define FKV_ROUND_HALF_AWAY 1

/* Output formats of the gather entry points. */
#define FKV_GATHER_F32 0 /* decoded to f32, like KvPool::k/v (kv.rs:43-45) */
#define FKV_GATHER_RAW 1 /* storage bytes; Q8_0 as Ferrum's 34-byte blocks (dtype.rs:19-21) */

/* Bits reported by fkv_paged_take_fault_flags(): device-side input faults that
 * the kernels skipped instead of touching memory out of bounds. */
#define FKV_FAULT_SLOT_RANGE 1u   /* append/gather slot >= num_blocks*block_size */
#define FKV_FAULT_BLOCK_RANGE 2u  /* block table / copy pair id outside [0, num_blocks) */
#define FKV_FAULT_CTX_RANGE 4u    /* ctx_len < 0, > max_blocks_per_seq * block_size, or
                                     (decode attention) longer than the call's splits
                                     hold, which max_ctx_len sized: the context is
                                     clamped to that bound, and a fused decode step
                                     (every storage type) stores no token for that
                                     sequence and rotates it at the clamped position */
#define FKV_FAULT_VALUE_RANGE 8u  /* Q8_0 append stored a block scale past the binary16
                                     range (a 32-value run with |x| >= 65520 * 127): the
                                     scale is +-inf, as the reference's encoder stores it,
                                     and attention over it is non-finite */

/* Version of this ABI; equals FKV_ABI_VERSION of the header the library was built with. */
int32_t fkv_abi_version(void);

/* Thread-local message of the last failing call on this thread ("" if none). The destroy
 * and close entry points (fkv_paged_destroy, fkv_kvpool_destroy, fkv_seqs_destroy,
 * fkv_gguf_close) leave it as it is, so finalizers that run between a failing call and
 * this read cannot clear it. */
const char* fkv_last_error(void);

/* Overrides of the launch planners, for measurements and tests; no counterpart in the
 * reference (its CPU loops have nothing to plan). Process-wide: a launch planned while
 * another thread changes a knob sees the old or the new value. The environment variables
 * in brackets seed the values when the library first plans a launch.
 *   FKV_TUNE_ATTN_SPLIT_TOKENS     decode split length, a multiple of 16 up to 2^20;
 *                                  0: the planner's rule [FKV_ATTN_SPLIT_TOKENS]
 *   FKV_TUNE_ATTN_STREAM           1: F16 decode on the persistent kernel [FKV_ATTN_MODE=stream]
 *   FKV_TUNE_ATTN_ORDER            decode work order 0 grid, 1 full splits first, 2 longest
 *                                  first; -1: the planner's rule [FKV_ATTN_ORDER]
 *   FKV_TUNE_PREFILL_SPLIT_BLOCKS  prefill key-range piece length in blocks, 0 no pieces;
 *                                  -1: the planner's rule [FKV_PREFILL_SPLIT_BLOCKS]
 *   FKV_TUNE_ATTN_ENGINE           F16 decode arithmetic: 0 the matrix cores (default),
 *                                  1 the VALU partition kernel (group sizes 1, 2, 4, 8, 16;
 *                                  others stay on the matrix cores), kept to measure the
 *                                  choice [FKV_ATTN_ENGINE=valu]
 *   FKV_TUNE_ATTN_WGS_PER_CU       at most this many decode-attention workgroups on a CU
 *                                  (2 or 3; 0: no cap), by the LDS each one asks for: room
 *                                  for prefill work on another stream to run beside the
 *                                  decode call [FKV_ATTN_WGS_PER_CU]
 * Out-of-range values: FKV_ERR_INVALID, nothing changed. */
#define FKV_TUNE_ATTN_SPLIT_TOKENS 0
#define FKV_TUNE_ATTN_STREAM 1
#define FKV_TUNE_ATTN_ORDER 2
#define FKV_TUNE_PREFILL_SPLIT_BLOCKS 3
#define FKV_TUNE_ATTN_ENGINE 4
#define FKV_TUNE_ATTN_WGS_PER_CU 5
int32_t fkv_set_tuning(int32_t knob, int64_t value);

/* Number of visible HIP devices (0 when no GPU); never fails. */
int32_t fkv_device_count(void);

/* ------------------------------------------------------------------------- */
/* Revision-1 compat surface: Ferrum's KvPool over device storage.            */
/* ------------------------------------------------------------------------- */

/* Mirrors `KvPoolConfig` (core-types/src/kv.rs:12-19). */
typedef struct fkv_kvpool_config {
  uint64_t n_layers;
  uint64_t n_kv_heads;
  uint64_t head_dim;
  uint64_t max_seq_len;
  uint64_t max_slots;
} fkv_kvpool_config;

typedef struct fkv_kvpool fkv_kvpool;

/* PreallocatedKvPool::new (pool.rs:21-46): "kv pool dimension is zero",
 * "kv pool size overflow". Storage is max_slots*n_layers*max_seq_len*n_kv_heads*
 * head_dim*2 f32 on `device`, allocated once. */
int32_t fkv_kvpool_new(const fkv_kvpool_config* config, int32_t device, fkv_kvpool** out);
int32_t fkv_kvpool_destroy(fkv_kvpool* pool);
/* KvPool::config (kv.rs:22). */
int32_t fkv_kvpool_get_config(const fkv_kvpool* pool, fkv_kvpool_config* out);
/* f32 elements of device storage (pool.rs:293-307 checks this never grows). */
int32_t fkv_kvpool_storage_len(const fkv_kvpool* pool, uint64_t* out);
/* KvPool::alloc (pool.rs:83-101): first free slot, zero-filled; full pool is
 * FKV_ERR_UNAVAILABLE "no free kv slots". */
int32_t fkv_kvpool_alloc(fkv_kvpool* pool, uint32_t* slot_out);
/* KvPool::free (pool.rs:103-112): "free of unallocated slot". */
int32_t fkv_kvpool_free(fkv_kvpool* pool, uint32_t slot);
/* KvPool::seq_len (pool.rs:114-120): "unknown slot". */
int32_t fkv_kvpool_seq_len(const fkv_kvpool* pool, uint32_t slot, uint64_t* out);
/* KvPool::append_layer (pool.rs:122-153). k, v: host f32 [n_kv_heads*head_dim]. */
int32_t fkv_kvpool_append_layer(fkv_kvpool* pool, uint32_t slot, uint64_t layer,
                                const float* k, uint64_t k_len, const float* v,
                                uint64_t v_len);
/* KvPool::commit_token (pool.rs:155-172). */
int32_t fkv_kvpool_commit_token(fkv_kvpool* pool, uint32_t slot);
/* KvPool::k / KvPool::v (pool.rs:174-204); copies n_kv_heads*head_dim f32 to host out. */
int32_t fkv_kvpool_k(const fkv_kvpool* pool, uint32_t slot, uint64_t layer, uint64_t pos,
                     float* out, uint64_t out_len);
int32_t fkv_kvpool_v(const fkv_kvpool* pool, uint32_t slot, uint64_t layer, uint64_t pos,
                     float* out, uint64_t out_len);
/* PreallocatedKvPool::abandon_partial / uncommit_token (pool.rs:207-231). */
int32_t fkv_kvpool_abandon_partial(fkv_kvpool* pool, uint32_t slot);
int32_t fkv_kvpool_uncommit_token(fkv_kvpool* pool, uint32_t slot);

/* ------------------------------------------------------------------------- */
/* Paged surface.                                                              */
/* ------------------------------------------------------------------------- */

typedef struct fkv_paged_config {
  uint32_t n_layers;
  uint32_t n_kv_heads;
  uint32_t head_dim;        /* Q8_0 needs a multiple of 32 */
  uint32_t block_size;      /* tokens per block; decode attention needs 16 */
  uint64_t num_blocks;      /* device blocks */
  uint64_t num_host_blocks; /* pinned host blocks for swap (0 = none) */
  int32_t kv_dtype;         /* FKV_DTYPE_* */
  int32_t f16_rounding;     /* FKV_ROUND_* */
  int32_t device;           /* HIP device ordinal */
  int32_t reserved;
} fkv_paged_config;

typedef struct fkv_paged_info {
  uint64_t tile_bytes;   /* one (block, layer, kv, head) tile */
  uint64_t block_bytes;  /* one block: n_layers*2*n_kv_heads*tile_bytes */
  uint64_t pool_bytes;   /* num_blocks*block_bytes */
  uint64_t free_blocks;  /* blocks with refcount 0 */
  void* device_base;     /* start of device storage */
  void* host_base;       /* start of pinned host swap storage, or NULL (read-only for
                            callers: see the block marks below) */
} fkv_paged_info;

typedef struct fkv_pool fkv_pool;

/* Create a pool: one hipMalloc of num_blocks*block_bytes (plus hipHostMalloc for
 * swap). Zero dims: FKV_ERR_CACHE "kv pool dimension is zero" (pool.rs:28). */
int32_t fkv_paged_create(const fkv_paged_config* config, fkv_pool** out);
int32_t fkv_paged_destroy(fkv_pool* pool);
int32_t fkv_paged_get_info(const fkv_pool* pool, fkv_paged_info* out);
/* Reads and clears the FKV_FAULT_* bits the kernels raised, in stream order: the
 * bits of every call enqueued on `stream` before this one (and of any other work
 * already finished), then synchronises that stream only. The read and the clear
 * are one atomic exchange on the device, so a bit raised meanwhile by work on
 * another stream is reported by the next call. Calls on one pool from several
 * threads are serialised inside (each returns the bits its own exchange took). */
int32_t fkv_paged_take_fault_flags(fkv_pool* pool, void* stream, uint32_t* flags_out);
/* Block marks. A block is marked when a value the fast attention instances cannot take
 * is stored in it: a Q8_0 scale of 512 or more (or inf/NaN), or an Inf/NaN K or V of an
 * F16 pool. Attention reads the marks of the blocks each workgroup covers, and only
 * workgroups over marked blocks run the slower exact (Q8_0) or leak-safe (F16 prefill)
 * instance. A mark stays with the block's bytes: appends and the fused step set it,
 * fkv_copy_blocks copies it to the destination, fkv_swap_out keeps it with the host
 * block and fkv_swap_in brings it back, fkv_paged_fill sets every device block's mark
 * from the fill byte, fkv_paged_write sets it where the image holds such a value and
 * clears it where the image overwrites a whole block without one. Nothing else clears
 * it (a freed block keeps its mark until it is overwritten that way). Bytes written
 * into host blocks through fkv_paged_info.host_base are not scanned: write pool bytes
 * with fkv_paged_write, after fkv_swap_in where the block was swapped out.
 * fkv_paged_marked_blocks reports how many device blocks are marked, in stream order
 * (it synchronises `stream`). It has no counterpart in the reference, whose dense f32
 * pool holds every value exactly. */
int32_t fkv_paged_marked_blocks(fkv_pool* pool, void* stream, uint64_t* count_out);
/* Fill every byte of device storage with `byte` (async on stream). */
int32_t fkv_paged_fill(fkv_pool* pool, uint8_t byte, void* stream);
/* Raw copies between device storage and host memory (byte offsets into the pool),
 * ordered on `stream` after the work enqueued there, which is then synchronised (the
 * host buffer may be reused on return). Used to persist or inspect the pool image. */
int32_t fkv_paged_read(fkv_pool* pool, uint64_t offset, uint64_t bytes, void* host_dst,
                       void* stream);
int32_t fkv_paged_write(fkv_pool* pool, uint64_t offset, uint64_t bytes, const void* host_src,
                        void* stream);

/* Host-side block allocator (free list with refcounts). Replaces the slot scan
 * of pool.rs:83-101; exhaustion is FKV_ERR_UNAVAILABLE "no free kv blocks", the
 * analogue of "no free kv slots" that the scheduler stops admission on
 * (scheduler/src/batcher.rs:110-113). All-or-nothing. */
int32_t fkv_block_alloc(fkv_pool* pool, uint32_t n, int32_t* ids_out);
/* Drop one reference per id; a block returns to the free list at refcount 0.
 * Unallocated id: FKV_ERR_CACHE "free of unallocated block". */
int32_t fkv_block_free(fkv_pool* pool, uint32_t n, const int32_t* ids);
/* Add one reference per id (copy-on-write sharing after a fork). */
int32_t fkv_block_ref(fkv_pool* pool, uint32_t n, const int32_t* ids);
int32_t fkv_block_refcount(const fkv_pool* pool, int32_t id, uint32_t* out);

/* Append: the paged form of KvPool::append_layer (pool.rs:122-153).
 * k, v: device f32 [n_tokens][n_kv_heads][head_dim] (post-RoPE K, kv.rs:30-31).
 * slot_mapping: device int64 [n_tokens]; slot < 0 skips the token (padding). The
 * slots of one call are distinct (a slot named twice ends up holding one of its
 * tokens, which one unspecified). F16 storage rounds with the pool's f16_rounding; Q8_0 quantises each 32-value
 * run like Q8Activation::quantize_into (q8_dot.rs:35-61). */
int32_t fkv_append(fkv_pool* pool, uint32_t layer, const float* k, const float* v,
                   const int64_t* slot_mapping, uint32_t n_tokens, void* stream);

/* Gather by slot: the inverse of fkv_append, the paged form of KvPool::k/v
 * (pool.rs:174-204). out_k/out_v: device [n_tokens][n_kv_heads][head_dim] in
 * `format`; a slot < 0 leaves its output row untouched. */
int32_t fkv_gather_slots(fkv_pool* pool, uint32_t layer, const int64_t* slot_mapping,
                         uint32_t n_tokens, int32_t format, void* out_k, void* out_v,
                         void* stream);

/* Gather by block table: sequence s's positions 0..ctx_lens[s]-1 go to rows
 * out_offsets[s] .. out_offsets[s]+ctx_lens[s]-1 of out_k/out_v (device).
 * block_tables: device int32 [n_seqs][max_blocks_per_seq]. */
int32_t fkv_gather_tables(fkv_pool* pool, uint32_t layer, const int32_t* block_tables,
                          uint32_t max_blocks_per_seq, const int32_t* ctx_lens,
                          const int64_t* out_offsets, uint32_t n_seqs, uint32_t max_ctx_len,
                          int32_t format, void* out_k, void* out_v, void* stream);

/* Copy whole blocks (every layer, K and V): pairs is device int64 [n_pairs][2] of
 * (src, dst). Used for copy-on-write after a fork and for compaction. dst blocks
 * must be distinct and must not be sources in the same call. */
int32_t fkv_copy_blocks(fkv_pool* pool, const int64_t* pairs, uint32_t n_pairs, void* stream);

/* Swap whole blocks between HBM and the pool's pinned host storage.
 * pairs is HOST int64 [n_pairs][2]: swap_out (device_block, host_block),
 * swap_in (host_block, device_block). Asynchronous on stream. */
int32_t fkv_swap_out(fkv_pool* pool, const int64_t* pairs, uint32_t n_pairs, void* stream);
int32_t fkv_swap_in(fkv_pool* pool, const int64_t* pairs, uint32_t n_pairs, void* stream);

/* Paged decode attention: the attention loop of Llama::forward_one_token
 * (crates/model/src/llama.rs:220-247) over KV read through block tables.
 * For query head h of sequence s, with g = n_heads / n_kv_heads:
 *   score[p] = dot(q[s][h], K[p][h / g]) * scale, p < ctx_lens[s]
 *   out[s][h] = softmax(score) . V[.][h / g]
 * A non-finite maximum score gives zeros (kernels/src/scalar.rs:125-130).
 * q, out: device f32 [n_seqs][n_heads][head_dim]. block_tables: device int32
 * [n_seqs][max_blocks_per_seq]; ctx_lens: device int32 [n_seqs], each
 * <= max_ctx_len. Needs block_size 16, head_dim 64 or 128, and g <= 16 (F16 and
 * Q8_0, matrix cores) or g in {1,2,4,8,16} (F32). Q8_0 follows the reference's f32
 * dequantisation (kernels/src/scalar.rs:268-275) for every finite scale: over unmarked
 * blocks operands are scale x quant in binary16 (exact to one rounding); a workgroup
 * whose blocks include a marked one (a scale of 512 or more: see the block marks
 * above) runs a second kernel instance, which takes the quants as exact
 * operands and applies the scales in f32.
 * workspace: device scratch of fkv_decode_attention_workspace_size() bytes
 * holding the split partials (running max, sum and unnormalised output per
 * query head and context split) that the merge pass reads; it may be NULL when
 * that size is 0 (every sequence fits one split) and needs no initialisation.
 * Calls that share one workspace must not overlap (same stream, or ordered by
 * events). */
int32_t fkv_decode_attention_workspace_size(const fkv_pool* pool, uint32_t n_heads,
                                            uint32_t n_seqs, uint32_t max_ctx_len,
                                            uint64_t* bytes_out);
int32_t fkv_decode_attention(fkv_pool* pool, uint32_t layer, uint32_t n_heads,
                             const float* q, float* out, const int32_t* block_tables,
                             uint32_t max_blocks_per_seq, const int32_t* ctx_lens,
                             uint32_t n_seqs, uint32_t max_ctx_len, float scale,
                             void* workspace, uint64_t workspace_bytes, void* stream);

/* Decode step of one layer in one call: the append of Llama::forward_one_token
 * (crates/model/src/llama.rs:218, KvPool::append_layer of kv.rs:30-38) followed by
 * its attention loop (:220-247), which reads the token just appended. For each
 * sequence s with ctx_lens[s] > 0, k_new[s] and v_new[s] (device f32
 * [n_seqs][n_kv_heads][head_dim], post-RoPE K) are stored at position
 * ctx_lens[s] - 1 through block_tables (encoded like fkv_append), then decode
 * attention runs over ctx_lens[s] positions exactly as fkv_decode_attention.
 * The block holding that position must belong to sequence s alone (copy it with
 * fkv_copy_blocks first if it is shared). For F16 and Q8_0 storage this is one
 * kernel launch: the workgroup that reads the sequence's last context split
 * encodes the token (Q8_0: quantised as fkv_append does, FKV_FAULT_VALUE_RANGE
 * included), stores it and uses its encoded values in place of what it loaded; a
 * Q8_0 token with a scale of 512 or more marks its block, and the exact instance
 * that every Q8_0 call launches after the first recomputes the call's outputs.
 * F32 storage uses an append launch first.
 * workspace: fkv_append_decode_attention_workspace_size() bytes, same rules as
 * the decode-attention workspace. */
int32_t fkv_append_decode_attention_workspace_size(const fkv_pool* pool, uint32_t n_heads,
                                                   uint32_t n_seqs, uint32_t max_ctx_len,
                                                   uint64_t* bytes_out);
int32_t fkv_append_decode_attention(fkv_pool* pool, uint32_t layer, uint32_t n_heads,
                                    const float* k_new, const float* v_new, const float* q,
                                    float* out, const int32_t* block_tables,
                                    uint32_t max_blocks_per_seq, const int32_t* ctx_lens,
                                    uint32_t n_seqs, uint32_t max_ctx_len, float scale,
                                    void* workspace, uint64_t workspace_bytes, void* stream);

/* fkv_append_decode_attention without a workspace argument, and allocating nothing
 * (no hipMalloc, hipFree or allocating library call). It has no counterpart in the
 * reference: it is for callers that cannot allocate device memory (code under HIP
 * graph capture, tight serving loops, harnesses that forbid allocation). The split
 * partials go to a static device array of FKV_STATIC_SCRATCH_BYTES per GPU, held
 * until the process ends, whose address the library takes when a pool is created on
 * that GPU. A call whose fkv_append_decode_attention_workspace_size() exceeds that
 * is FKV_ERR_INVALID "decode step needs <n> bytes of scratch; the static scratch
 * holds <max>", with nothing launched. Every call on one GPU shares that GPU's array:
 * calls that overlap on one GPU (other streams, other threads, other pools) race and
 * must be ordered by the caller. Nothing in the array needs to start at zero.
 * Outputs and pool bytes are bit-identical to fkv_append_decode_attention's. */
#define FKV_STATIC_SCRATCH_BYTES (32ull << 20)
int32_t fkv_append_decode_attention_noalloc(fkv_pool* pool, uint32_t layer, uint32_t n_heads,
                                            const float* k_new, const float* v_new,
                                            const float* q, float* out,
                                            const int32_t* block_tables,
                                            uint32_t max_blocks_per_seq, const int32_t* ctx_lens,
                                            uint32_t n_seqs, uint32_t max_ctx_len, float scale,
                                            void* stream);

/* fkv_append_decode_attention with q and k_new before RoPE: the layer's
 * Kernels::rope call (crates/model/src/llama.rs:207-216; scalar.rs:77-82,167-189,
 * math.rs:27-34), then its append and attention loop. Every query head of q[s]
 * and every KV head of k_new[s] is rotated at position pos = ctx_lens[s] - 1:
 * dims (2i, 2i+1) with 2i < rope_dim (GGML_ROPE_TYPE_NORMAL) turn by
 * f = pos / theta^(2i / rope_dim), all in f32 as the reference computes it
 * (a' = a cos f - b sin f, b' = a sin f + b cos f); dims from rope_dim on are
 * unchanged; rope_dim = 0 rotates nothing. The rotated K is what the pool stores;
 * q is read only (the rotation is not written back). Checks, in the reference's
 * order (validate.rs:64-87), before any other: FKV_ERR_KERNEL "kernel: theta must
 * be positive" (theta <= 0 or NaN), "kernel: rope_dim must be even", "kernel:
 * rope_dim exceeds head_dim". F16 and Q8_0 storage rotate inside the one kernel
 * launch; F32 storage rotates q and k_new into the workspace first. sin and cos
 * come from a table the pool builds on the host on the first call for a (rope_dim,
 * theta) pair, and again when max_ctx_len outgrows it (doubling): the C library's
 * sinf and cosf of f for every position below max_ctx_len (rounded up to a power of
 * two, at least 4,096, at most 2^20), as the reference's f32::sin_cos gives them, so
 * the stored K is the reference's rotation bit for bit. That call blocks while the
 * table is built and uploaded (16 MiB at rope_dim 128 and 32,768 positions, 512 MiB at
 * 2^20; held until fkv_paged_destroy). Positions past 2^20 rotate with the device's
 * sincosf, which can differ from the C library's by an ulp (one f16 step in stored K).
 * workspace: fkv_rope_append_decode_attention_workspace_size() bytes. */
int32_t fkv_rope_append_decode_attention_workspace_size(const fkv_pool* pool, uint32_t n_heads,
                                                        uint32_t n_seqs, uint32_t max_ctx_len,
                                                        uint64_t* bytes_out);
int32_t fkv_rope_append_decode_attention(fkv_pool* pool, uint32_t layer, uint32_t n_heads,
                                         uint32_t rope_dim, float theta, const float* k_new,
                                         const float* v_new, const float* q, float* out,
                                         const int32_t* block_tables, uint32_t max_blocks_per_seq,
                                         const int32_t* ctx_lens, uint32_t n_seqs,
                                         uint32_t max_ctx_len, float scale, void* workspace,
                                         uint64_t workspace_bytes, void* stream);

/* Chunked-prefill attention over F16 or Q8_0 storage: the reference's token-by-token
 * prefill (crates/model/src/llama.rs:363-378, each token running the attention loop
 * of :220-247 over positions 0 ..= its own) for a chunk whose K/V are already
 * appended. Sequence s has q_lens[s] new tokens at the end of its ctx_lens[s]-token
 * context: query i sits at position ctx_lens[s] - q_lens[s] + i and attends to
 * positions 0 ..= that position. q, out: device f32 [rows][n_heads][head_dim];
 * sequence s's queries are rows q_offsets[s] .. q_offsets[s] + q_lens[s] - 1
 * (q_offsets: device int64). q_lens[s] = 1 is decode. Needs block_size 16, head_dim
 * 64 or 128, g <= 16, and a pool block (all layers' K and V) under 4 GiB
 * (FKV_ERR_KERNEL otherwise). The launch holds max_q_len queries a sequence: a q_lens[s]
 * above it (or above ctx_lens[s]) raises FKV_FAULT_CTX_RANGE, and only its first
 * max_q_len queries are computed, at the positions q_lens[s] gives them. A ctx_lens[s]
 * past max_ctx_len rounded up to whole blocks raises FKV_FAULT_CTX_RANGE and is
 * clamped to it (the sequence's queries then end at the clamped context). No query
 * reads a position past its own, Inf/NaN values included: workgroups over F16 blocks
 * marked as holding an Inf/NaN K or V (see the block marks above) run a slower
 * instance that keeps such V values from earlier queries of the same tile and gives an
 * infinite K's scores exactly. Q8_0 follows fkv_decode_attention's rule for blocks
 * marked with scales of 512 or more.
 * workspace: NULL, or device scratch of fkv_prefill_attention_workspace_size()
 * bytes (16-byte aligned; no initialisation) in which workgroups over long
 * contexts leave the partial results of pieces of their key range for a merge
 * pass, and (Q8_0 pools) the call's blocks are dequantised once to binary16 for
 * every workgroup that reads them: n_seqs x ceil(max_ctx_len / 16) blocks of K and V
 * tiles of every KV head, 2 x n_kv_heads x 16 x head_dim x 2 bytes each. With NULL
 * every workgroup reads its whole key range itself and Q8_0 workgroups dequantise
 * what they read (same results within the attention tolerance; slower). Calls that
 * share one workspace must not overlap. */
int32_t fkv_prefill_attention_workspace_size(const fkv_pool* pool, uint32_t n_heads,
                                             uint32_t n_seqs, uint32_t max_q_len,
                                             uint32_t max_ctx_len, uint64_t* bytes_out);
int32_t fkv_prefill_attention(fkv_pool* pool, uint32_t layer, uint32_t n_heads, const float* q,
                              float* out, const int32_t* block_tables,
                              uint32_t max_blocks_per_seq, const int32_t* ctx_lens,
                              const int32_t* q_lens, const int64_t* q_offsets, uint32_t n_seqs,
                              uint32_t max_q_len, uint32_t max_ctx_len, float scale,
                              void* workspace, uint64_t workspace_bytes, void* stream);

/* Device-to-device byte copy with the same 16-byte vector kernel style as the
 * pool kernels; used to calibrate HBM counters and to measure copy bandwidth. */
int32_t fkv_device_copy(void* dst, const void* src, uint64_t bytes, void* stream);

/* ------------------------------------------------------------------------- */
/* Sequence block manager: the scheduler's KV bookkeeping on the paged pool.   */
/* ------------------------------------------------------------------------- */

/* Per-sequence block lists over one paged pool. This is the paged replacement for
 * how crates/scheduler/src/batcher.rs uses KV slots: admission stops on
 * Unavailable (:108-129), rollback frees the slot and re-runs the prefix
 * (restore_kv, :291-308), finish frees the slot (:329-338). Here admission asks
 * for the blocks a sequence's tokens need; fkv_seqs_fork shares blocks by
 * reference (copy-on-write); rollback truncates the block list; preemption moves
 * a sequence's blocks to the pool's pinned host blocks and back. One manager per
 * pool (it owns the pool's host blocks); single writer, like the pool.
 * Errors: FKV_ERR_CACHE "cache: unknown sequence", "cache: sequence is swapped
 * out", ...; FKV_ERR_UNAVAILABLE "no free kv blocks" / "no free host blocks", with
 * nothing changed. */
typedef struct fkv_seqs fkv_seqs;
int32_t fkv_seqs_create(fkv_pool* pool, fkv_seqs** out);
/* Releases every sequence's blocks. */
int32_t fkv_seqs_destroy(fkv_seqs* m);
/* Admission: a new sequence (length 0) with blocks for n_tokens tokens. */
int32_t fkv_seqs_add(fkv_seqs* m, uint64_t n_tokens, uint32_t* seq_out);
/* Blocks for n more tokens after the committed length. If the block that holds
 * position len is shared with another sequence (after a fork) and already holds
 * some of this sequence's tokens, the sequence takes a private copy: copy_pair
 * (host int64[2]) receives (shared block, new block), which the caller copies
 * with fkv_copy_blocks before it appends; otherwise copy_pair is (-1, -1). */
int32_t fkv_seqs_reserve(fkv_seqs* m, uint32_t seq, uint64_t n, int64_t* copy_pair);
/* Slots of positions pos .. pos + n - 1 (within the reserved blocks) for fkv_append. */
int32_t fkv_seqs_slots(const fkv_seqs* m, uint32_t seq, uint64_t pos, uint64_t n,
                       int64_t* slots_out);
/* len += n: the tokens' K/V are in the pool (KvPool::commit_token, pool.rs:155-172). */
int32_t fkv_seqs_commit(fkv_seqs* m, uint32_t seq, uint64_t n);
/* Rollback: len = n_tokens (<= len); blocks past the new length are released. */
int32_t fkv_seqs_truncate(fkv_seqs* m, uint32_t seq, uint64_t n_tokens);
/* A new sequence of the parent's length sharing its committed blocks. */
int32_t fkv_seqs_fork(fkv_seqs* m, uint32_t parent, uint32_t* child_out);
/* Finish: releases the sequence's blocks (device or host). */
int32_t fkv_seqs_free(fkv_seqs* m, uint32_t seq);
/* Committed length; *swapped_out (may be NULL) is 1 while swapped out. */
int32_t fkv_seqs_len(const fkv_seqs* m, uint32_t seq, uint64_t* len_out, int32_t* swapped_out);
/* Preemption. swap_out copies the committed blocks to host blocks (fkv_swap_out)
 * and releases the device blocks; swap_in copies them into new device blocks
 * (fkv_swap_in). The copies are asynchronous on stream: released blocks may be
 * written again only by work ordered after them (the same stream). */
int32_t fkv_seqs_swap_out(fkv_seqs* m, uint32_t seq, void* stream);
int32_t fkv_seqs_swap_in(fkv_seqs* m, uint32_t seq, void* stream);
/* Host block-table rows (padded with block 0) and committed lengths of a batch,
 * for upload to the decode and gather entry points. */
int32_t fkv_seqs_tables(const fkv_seqs* m, const uint32_t* seqs, uint32_t n, uint32_t max_blocks,
                        int32_t* tables_out, int32_t* ctx_out);

#ifdef __cplusplus
}
#endif

#endif /* FERRUM_KV_H */
