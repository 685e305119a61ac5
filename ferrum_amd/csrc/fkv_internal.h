// Internal interface between the C ABI (fkv_api.cpp) and the HIP kernels
// (fkv_kernels.hip). Not installed; the public interface is include/ferrum_kv.h.
#pragma once

#include <hip/hip_runtime_api.h>
#include <stdint.h>

#include <atomic>
#include <string>

namespace fkv {

// The C ABI's error state (fkv_api.cpp): set the thread's Display string for an
// FKV_ERR_* code and return the code; clear it and return FKV_OK.
int32_t api_fail(int32_t code, const std::string& msg);
int32_t api_ok();
// Restores the thread's last-error message when it goes out of scope. The destroy and
// close entry points hold one: they run from finalizers (a garbage collector may call them
// between a failing call and the caller's read of fkv_last_error), so they must not
// change the message.
struct KeepLastError {
  KeepLastError();
  ~KeepLastError();
  std::string saved;
};

// Geometry of one paged pool, passed by value to every kernel.
// pool[block][layer][kv][head][tile]; tile = [B][D] elements (F32), [D/8][B][8]
// (F16 K: 16-byte runs of 8 dims, token-contiguous per run), [D][B] (F16 V), or
// int8 quants ([B][D] for K, [D][B] for V) then f16 scales [B][D/32] (Q8_0),
// padded to a multiple of 16 bytes. The F16 and Q8_0 orders are the QK and P.V
// operand orders of the MFMA decode kernel.
struct Geom {
  uint8_t* base;
  uint64_t tile_bytes;
  uint64_t block_bytes;
  uint64_t num_blocks;
  uint32_t n_layers;
  uint32_t n_kv_heads;
  uint32_t head_dim;
  uint32_t block_size;
  int32_t dtype;     // 0 f32, 1 f16, 8 q8_0
  int32_t rounding;  // 0 nearest-even, 1 ties away
  uint32_t* fault;   // device words: [0] FKV_FAULT_* bits; [1] number of marked
                     // blocks (bmark); [2] unused; [3] staging word of the fault read
  uint32_t* bmark;   // per device block: 1 when a value the fast attention instances
                     // cannot take was stored in it (Q8_0: a scale of 512 or more,
                     // q8_wide_scale; F16: an Inf/NaN K or V, f16_nonfinite), else 0
  uint32_t* hmark;   // per pinned host block: the mark its bytes carry
  uint32_t n_cus;    // compute units of the pool's device (read once, at creation)
};

// Overrides of the launch planners for measurements and tests (fkv_set_tuning), seeded
// from the environment once per process:
//   FKV_ATTN_SPLIT_TOKENS   decode split length (a multiple of 16)
//   FKV_ATTN_MODE=stream    F16 decode on the persistent kernel
//   FKV_ATTN_ORDER          decode work order (0 grid, 1 full splits first, 2 longest first)
//   FKV_PREFILL_SPLIT_BLOCKS  prefill key-range piece length in blocks (0: no pieces)
//   FKV_ATTN_ENGINE=valu    F16 decode on the VALU partition kernel
//   FKV_ATTN_WGS_PER_CU     decode workgroups a CU at most (2 or 3; 0: no cap)
// Read with relaxed loads per launch plan (no environment access per call).
struct Tuning {
  std::atomic<int32_t> split_tokens{0};    // 0: the planner's rule
  std::atomic<int32_t> stream_mode{0};
  std::atomic<int32_t> attn_order{-1};     // -1: the planner's rule
  std::atomic<int64_t> prefill_split{-1};  // -1: the planner's rule
  std::atomic<int32_t> attn_engine{0};     // 1: F16 decode on the VALU partition kernel
  std::atomic<int32_t> attn_wgs_per_cu{0}; // 2 or 3: decode workgroups a CU at most; 0: no cap
};
Tuning& tuning();

constexpr int kDtypeF32 = 0;
constexpr int kDtypeF16 = 1;
constexpr int kDtypeQ8 = 8;

// RoPE of the decode step's new token (GGML_ROPE_TYPE_NORMAL: dims (2i, 2i+1)
// rotate by pos / den[i], den[i] = theta^(2i / rope_dim) computed on the host
// exactly as the reference computes it in f32; crates/kernels/src/math.rs:27-34,
// scalar.rs:167-189). rope_dim = 0: no rotation.
struct RopeTable {
  int32_t rope_dim;  // even, <= head_dim <= 128
  float den[64];
  // (sin, cos) of pair p at position pos: sc[(pos * rope_dim / 2 + p) * 2 + {0, 1}], for
  // pos < sc_pos (the pool's table, built on the host with the C library's sinf and
  // cosf as the reference's f32::sin_cos); past it, or with sc null, the device sincosf
  const float* sc;
  uint32_t sc_pos;
};

constexpr uint32_t kFaultSlot = 1u;
constexpr uint32_t kFaultBlock = 2u;
constexpr uint32_t kFaultCtx = 4u;
constexpr uint32_t kFaultRange = 8u;

// Decode attention partitioning: 4 waves per workgroup, each wave owns 4 blocks
// of 16 tokens, so one workgroup covers a 256-token partition of one
// (sequence, kv head).
constexpr int kAttnBlock = 16;
constexpr int kAttnWaves = 4;
constexpr int kAttnBlocksPerWave = 4;
constexpr int kAttnPartTokens = kAttnBlock * kAttnWaves * kAttnBlocksPerWave;  // 256

inline uint64_t tile_bytes_for(int dtype, uint32_t block_size, uint32_t head_dim) {
  uint64_t e = (uint64_t)block_size * head_dim;
  // F16 K tiles store runs of 8 dims, so head_dim is padded to a multiple of 8.
  uint64_t raw = dtype == kDtypeF32 ? e * 4
                 : dtype == kDtypeF16 ? (uint64_t)block_size * ((head_dim + 7) / 8 * 8) * 2
                                      : e + (e / 32) * 2;
  return (raw + 15) / 16 * 16;
}

// Launchers (return the hipError_t of the launch).
hipError_t launch_append(const Geom& g, uint32_t layer, const float* k, const float* v,
                         const int64_t* slots, uint32_t n_tokens, hipStream_t s);
hipError_t launch_gather_slots(const Geom& g, uint32_t layer, const int64_t* slots,
                               uint32_t n_tokens, int format, void* out_k, void* out_v,
                               hipStream_t s);
hipError_t launch_gather_tables(const Geom& g, uint32_t layer, const int32_t* tables,
                                uint32_t max_blocks, const int32_t* ctx_lens,
                                const int64_t* out_offsets, uint32_t n_seqs,
                                uint32_t max_ctx_len, int format, void* out_k, void* out_v,
                                hipStream_t s);
hipError_t launch_copy_blocks(const Geom& g, const int64_t* pairs, uint32_t n_pairs,
                              hipStream_t s);
hipError_t launch_fill(void* dst, uint8_t byte, uint64_t bytes, hipStream_t s);
// Block marks (Geom::bmark). fill: every device block's mark = `mark`, the count with it.
hipError_t launch_marks_fill(const Geom& g, uint32_t mark, hipStream_t s);
// Up to kMarkPairs (device block, host block) pairs per launch: swap_out copies the device
// blocks' marks to the host blocks', swap_in the other way (keeping the count).
constexpr uint32_t kMarkPairs = 240;
struct MarkPairs {
  int32_t dev[kMarkPairs];
  int32_t host[kMarkPairs];
  uint32_t n;
};
hipError_t launch_marks_swap(const Geom& g, const MarkPairs& p, bool out, hipStream_t s);
// ops[i] for device block first + i: 0 keeps the mark, 1 sets it, 2 clears it.
hipError_t launch_marks_apply(const Geom& g, uint64_t first, uint64_t n, const uint8_t* ops,
                              hipStream_t s);
// fault[3] = fault[0], fault[0] = 0, atomically (fkv_paged_take_fault_flags).
hipError_t launch_take_fault(uint32_t* fault, hipStream_t s);
hipError_t launch_device_copy(void* dst, const void* src, uint64_t bytes, hipStream_t s);

// Returns hipErrorInvalidValue when no kernel is instantiated for the shape.
bool attention_supported(int dtype, uint32_t head_dim, uint32_t group);
// F16 decode attention on the matrix cores (fkv_attention_mfma.hip); head_dim 64
// or 128, any group size 1..16. With k_new/v_new (f32 [n_seqs][n_kv_heads][D])
// the kernel first appends each sequence's token at position ctx_lens[s] - 1.
hipError_t launch_attention_mfma(const Geom& g, uint32_t layer, uint32_t n_heads,
                                 const float* q, float* out, const int32_t* tables,
                                 uint32_t max_blocks, const int32_t* ctx_lens, uint32_t n_seqs,
                                 uint32_t max_splits, uint32_t split_tokens, float scale,
                                 float* ws_o, float* ws_ml, const float* k_new,
                                 const float* v_new, hipStream_t s,
                                 const RopeTable* rope = nullptr);
// F16 decode attention, persistent schedule (fkv_attention_mfma.hip): n_waves
// waves share the flattened (sequence, KV head, block) list equally; needs
// 1 <= n_seqs <= kStreamMaxSeqs (the LDS prefix table). ws_pre holds n_seqs + 1
// uint32; ws_o / ws_ml hold (n_waves + n_seqs * n_kv_heads) partial slots of G
// heads x (head_dim | 2) floats.
constexpr uint32_t kStreamMaxSeqs = 8192;
bool stream_attention_supported(uint32_t n_seqs);
// Waves of a full-occupancy stream launch on the current device (0: unavailable).
uint32_t stream_attention_waves(uint32_t head_dim, uint32_t n_seqs, uint32_t n_cus);
hipError_t launch_attention_stream(const Geom& g, uint32_t layer, uint32_t n_heads,
                                   const float* q, float* out, const int32_t* tables,
                                   uint32_t max_blocks, const int32_t* ctx_lens,
                                   uint32_t n_seqs, float scale, uint32_t n_waves,
                                   uint32_t* ws_pre, float* ws_o, float* ws_ml, hipStream_t s);
// Chunked-prefill attention (fkv_attention_mfma.hip), F16 or Q8_0 storage: query i
// of sequence s is at position ctx_lens[s] - q_lens[s] + i and attends causally;
// q/out rows of sequence s start at q_offsets[s]. Needs G <= 16.
// A workgroup (16 / G queries per wave, 4 waves) whose key range is longer than
// split_blocks blocks is cut into pieces of about equal length (at most max_splits),
// each its own workgroup, whose partials a combine kernel merges; the plan splits
// only grids smaller than the device's workgroup slots and sizes the workspace for
// the longest context the call allows. With split_blocks 0 or no workspace, every
// workgroup is one piece.
constexpr uint64_t kPrefillWgsPerCu = 4;         // resident prefill workgroups per CU
constexpr uint64_t kPrefillMinPieceBlocks = 64;  // shortest piece the plan makes
constexpr uint64_t kPrefillMaxSplits = 32;
struct PrefillPlan {
  uint32_t tile_groups;   // grid.y: groups of 4 query tiles
  uint32_t split_blocks;  // 0: no split
  uint32_t max_splits;
  uint64_t ws_o_floats;   // partial outputs, then (max, sum) pairs
  uint64_t ws_bytes;
  uint32_t prio_blocks;   // longest key range in blocks (issue-priority scale; 0: off)
  uint32_t cap_blocks;    // ceil(max_ctx_len / 16): longer contexts are clamped (fault)
  // Q8_0 pools: blocks a sequence stages (ceil(max_ctx_len / 16); 0: no staging), and
  // the workspace offsets of the binary16 tiles, the staging table and staging marks
  uint32_t stage_nblk;
  uint64_t stage_off, stage_tab_off, stage_mark_off;
};
PrefillPlan prefill_plan(const Geom& g, uint32_t n_heads, uint32_t n_seqs, uint32_t max_q_len,
                         uint32_t max_ctx_len);
hipError_t launch_prefill_attention(const Geom& g, uint32_t layer, uint32_t n_heads,
                                    const float* q, float* out, const int32_t* tables,
                                    uint32_t max_blocks, const int32_t* ctx_lens,
                                    const int32_t* q_lens, const int64_t* q_offsets,
                                    uint32_t n_seqs, uint32_t max_q_len, float scale,
                                    const PrefillPlan& plan, void* workspace, hipStream_t s);
// Merges split partials (m, l, o) per (sequence, query head) into out.
hipError_t launch_attention_combine(uint32_t head_dim, const int32_t* ctx_lens,
                                    uint32_t n_seqs, uint32_t n_heads, uint32_t max_blocks,
                                    uint32_t max_splits, uint32_t split_tokens,
                                    const float* ws_o, const float* ws_ml, float* out,
                                    hipStream_t s);
// k_new/v_new non-null: append each sequence's token at position ctx_lens[s] - 1
// (through its block table) before attending; one launch for F16 storage.
// rope non-null (with rope->rope_dim > 0): q and k_new are before RoPE; each
// sequence's are rotated at position ctx_lens[s] - 1 (in the kernel for F16
// storage; through the workspace's RoPE rows otherwise).
hipError_t launch_decode_attention(const Geom& g, uint32_t layer, uint32_t n_heads,
                                   const float* q, float* out, const int32_t* tables,
                                   uint32_t max_blocks, const int32_t* ctx_lens,
                                   uint32_t n_seqs, uint32_t max_ctx_len, float scale,
                                   void* workspace, const float* k_new, const float* v_new,
                                   hipStream_t s, const RopeTable* rope = nullptr);
// Workspace of a RoPE decode step: append_attention_workspace_bytes, plus room for
// the rotated q and k rows when the storage is not F16.
uint64_t rope_attention_workspace_bytes(const Geom& g, uint32_t n_heads, uint32_t n_seqs,
                                        uint32_t max_ctx_len);
// Slot of position ctx_lens[s] - 1 through the block table (-1 for an empty context,
// a context past min(ctx_cap, the table row) or an entry outside the pool, which
// raises kFaultBlock).
hipError_t launch_tail_slots(const Geom& g, const int32_t* tables, uint32_t max_blocks,
                             const int32_t* ctx_lens, uint32_t n_seqs, int64_t* slots,
                             hipStream_t s, uint64_t ctx_cap = ~0ull);
// Device scratch one call needs (0 when every sequence fits one split): the
// split partials, which need no initialisation.
uint64_t attention_workspace_bytes(const Geom& g, uint32_t n_heads, uint32_t n_seqs,
                                   uint32_t max_ctx_len);
// Workspace of the fused append + attention call: the above, plus the derived
// slots for the storage types whose append is a separate launch.
uint64_t append_attention_workspace_bytes(const Geom& g, uint32_t n_heads, uint32_t n_seqs,
                                          uint32_t max_ctx_len);

// Static scratch of the no-allocation decode step (fkv_attention.hip): one device
// array of kStaticScratchBytes per GPU, held until the process ends. setup takes
// its address on `device` (which must be current) once; static_scratch returns it
// (nullptr before setup). Calls that use it on one GPU share it.
constexpr uint64_t kStaticScratchBytes = 32ull << 20;
hipError_t static_scratch_setup(int device);
void* static_scratch(int device);

// Q8_0 weight GEMV/GEMM (fkv_gemv.hip): y[t][r] = dot_q8_row_q8_act(w row r, x[t]
// quantized) for t < n_tokens, r < rows; w rows of cols/32 34-byte blocks (w even,
// x 4-byte aligned, cols % 32 == 0, gemv_lds_bytes(1, cols) <= kGemvMaxLds: the
// LDS one workgroup may hold on gfx950).
constexpr size_t kGemvMaxLds = 163840;
size_t gemv_lds_bytes(uint32_t tokens, uint32_t cols);
uint32_t gemv_tokens_per_launch(uint32_t n_tokens, uint32_t cols);
// Up to kGemvMaxMats weight matrices that share the activation x (cols columns): one
// launch, workgroups [wg0, next wg0) on matrix m; each y[m] as its own launch would give.
constexpr int kGemvMaxMats = 4;
struct GemvMat {
  const uint8_t* w;
  float* y;
  uint32_t rows;
  uint32_t wg0;  // first workgroup of this matrix (filled by launch_gemv_q8)
};
struct GemvBatch {
  GemvMat m[kGemvMaxMats];
  uint32_t n;
};
hipError_t launch_gemv_q8(GemvBatch b, uint32_t cols, const float* x, uint32_t n_tokens,
                          hipStream_t s);
// Batched form on the matrix cores (same results bit for bit): the activation quantized
// once into a workspace of gemm_mfma_workspace_bytes, then one i8 MFMA per 32-value
// block of 16 rows x 16 tokens. Eligible for n_tokens >= kGemmMfmaMinTokens, cols a
// multiple of 1024 and 16-byte aligned weights.
constexpr uint32_t kGemmMfmaMinTokens = 8;
bool gemm_mfma_eligible(const GemvBatch& b, uint32_t cols, uint32_t n_tokens);
uint64_t gemm_mfma_workspace_bytes(uint32_t cols, uint32_t n_tokens);
hipError_t launch_gemm_q8_mfma(GemvBatch b, uint32_t cols, const float* x, uint32_t n_tokens,
                               void* workspace, hipStream_t s);

}  // namespace fkv
