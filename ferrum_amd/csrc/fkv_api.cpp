// C ABI of libferrum_kv.so (declared in include/ferrum_kv.h).
//
// Host-side state (block allocator, sequence bookkeeping of the compat pool,
// validation, error strings) is C++ here; all K/V bytes live in device memory
// and are touched only by the HIP kernels in fkv_kernels.hip.
#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/ferrum_kv.h"
#include "../../include/ferrum_q8.h"
#include "../../include/ferrum_gguf.h"
#include "fkv_internal.h"

static_assert(FKV_STATIC_SCRATCH_BYTES == fkv::kStaticScratchBytes,
              "the header states the static scratch size the library holds");

namespace {

thread_local std::string g_last_error;

// FerrumError Display forms (crates/core-types/src/error.rs:21-46).
int32_t fail(int32_t code, const std::string& msg) {
  switch (code) {
    case FKV_ERR_CACHE: g_last_error = "cache: " + msg; break;
    case FKV_ERR_KERNEL: g_last_error = "kernel: " + msg; break;
    case FKV_ERR_GGUF: g_last_error = "gguf: " + msg; break;
    default: g_last_error = msg; break;
  }
  return code;
}

int32_t ok() {
  g_last_error.clear();
  return FKV_OK;
}

int32_t hip_fail(hipError_t e, const char* what) {
  return fail(FKV_ERR_INTERNAL, std::string("hip: ") + what + ": " + hipGetErrorString(e));
}

#define FKV_HIP(call, what)                       \
  do {                                            \
    hipError_t e_ = (call);                       \
    if (e_ != hipSuccess) return hip_fail(e_, what); \
  } while (0)

// Makes `device` current for the lifetime of the guard (no runtime call beyond the
// query when it already is, the usual case of a one-GPU process).
struct DeviceGuard {
  int prev = -1;
  bool ok = false;
  explicit DeviceGuard(int device) {
    if (hipGetDevice(&prev) != hipSuccess) prev = -1;
    if (prev == device) {
      prev = -1;  // nothing to restore
      ok = true;
    } else {
      ok = hipSetDevice(device) == hipSuccess;
    }
  }
  ~DeviceGuard() {
    if (prev >= 0) (void)hipSetDevice(prev);
  }
};

bool mul_ovf(uint64_t a, uint64_t b, uint64_t* r) { return __builtin_mul_overflow(a, b, r); }

}  // namespace

namespace fkv {
int32_t api_fail(int32_t code, const std::string& msg) { return fail(code, msg); }
int32_t api_ok() { return ok(); }
KeepLastError::KeepLastError() : saved(g_last_error) {}
KeepLastError::~KeepLastError() { g_last_error = std::move(saved); }
}  // namespace fkv

struct fkv_pool {
  fkv_paged_config cfg{};
  fkv::Geom geom{};
  uint8_t* dev = nullptr;
  uint8_t* host = nullptr;
  uint32_t* fault = nullptr;
  uint32_t* marks = nullptr;       // device: num_blocks + num_host_blocks block marks
  uint32_t* fault_host = nullptr;  // pinned: the fault read's copy lands here
  std::mutex fault_mu;             // one fault read at a time owns fault[3] and fault_host
  std::vector<int32_t> free_list;  // stack; LIFO reuse, as a fragmented pool would see
  std::vector<uint32_t> refcount;
  std::vector<fkv_seqs*> managers;  // detached when the pool is destroyed
  // RoPE (sin, cos) table of the last (rope_dim, theta) used (RopeTable::sc): rope_pos
  // positions; a table outgrown or replaced stays allocated until the pool is destroyed
  // (calls in flight may still read it)
  std::mutex rope_mu;
  float* rope_sc = nullptr;
  uint32_t rope_pos = 0, rope_dim = 0;
  float rope_theta = 0.0f;
  std::vector<float*> rope_old;
};

static void detach_manager(fkv_seqs* m);

struct fkv_kvpool {
  fkv_kvpool_config cfg{};
  fkv_pool* paged = nullptr;  // block_size = max_seq_len, one block per slot
  std::vector<uint8_t> free_;
  std::vector<uint64_t> seq_len;
  std::vector<uint64_t> layers_appended;
  float* stage = nullptr;     // device: k row, v row
  int64_t* slot_dev = nullptr;
  hipStream_t stream = nullptr;
};

extern "C" {

int32_t fkv_abi_version(void) { return FKV_ABI_VERSION; }

const char* fkv_last_error(void) { return g_last_error.c_str(); }

int32_t fkv_set_tuning(int32_t knob, int64_t value) {
  fkv::Tuning& t = fkv::tuning();
  switch (knob) {
    case FKV_TUNE_ATTN_SPLIT_TOKENS:
      if (value != 0 && (value < 16 || value % 16 != 0 || value > (1 << 20)))
        return fail(FKV_ERR_INVALID, "split tokens must be 0 or a multiple of 16 up to 2^20");
      t.split_tokens.store((int32_t)value);
      return ok();
    case FKV_TUNE_ATTN_STREAM:
      if (value != 0 && value != 1) return fail(FKV_ERR_INVALID, "stream mode must be 0 or 1");
      t.stream_mode.store((int32_t)value);
      return ok();
    case FKV_TUNE_ATTN_ORDER:
      if (value < -1 || value > 2) return fail(FKV_ERR_INVALID, "order must be -1, 0, 1 or 2");
      t.attn_order.store((int32_t)value);
      return ok();
    case FKV_TUNE_PREFILL_SPLIT_BLOCKS:
      if (value < -1 || value > 0x7fffffffll)
        return fail(FKV_ERR_INVALID, "prefill split blocks must be -1 or a block count");
      t.prefill_split.store(value);
      return ok();
    case FKV_TUNE_ATTN_ENGINE:
      if (value != 0 && value != 1) return fail(FKV_ERR_INVALID, "engine must be 0 or 1");
      t.attn_engine.store((int32_t)value);
      return ok();
    case FKV_TUNE_ATTN_WGS_PER_CU:
      if (value != 0 && value != 2 && value != 3)
        return fail(FKV_ERR_INVALID, "decode workgroups per CU must be 0, 2 or 3");
      t.attn_wgs_per_cu.store((int32_t)value);
      return ok();
    default:
      return fail(FKV_ERR_INVALID, "unknown tuning knob");
  }
}

int32_t fkv_device_count(void) {
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess) return 0;
  return n;
}

// ---------------------------------------------------------------------------
// Paged pool
// ---------------------------------------------------------------------------

int32_t fkv_paged_create(const fkv_paged_config* config, fkv_pool** out) {
  if (!config || !out) return fail(FKV_ERR_INVALID, "null argument");
  *out = nullptr;
  const fkv_paged_config& c = *config;
  if (!c.n_layers || !c.n_kv_heads || !c.head_dim || !c.block_size || !c.num_blocks)
    return fail(FKV_ERR_CACHE, "kv pool dimension is zero");
  if (c.kv_dtype != FKV_DTYPE_F32 && c.kv_dtype != FKV_DTYPE_F16 && c.kv_dtype != FKV_DTYPE_Q8_0)
    return fail(FKV_ERR_KERNEL, "unsupported dtype");
  if (c.kv_dtype == FKV_DTYPE_Q8_0 && c.head_dim % 32 != 0)
    return fail(FKV_ERR_KERNEL, "q8_0 k is not a multiple of 32");
  // The Q8_0 tile order (16-token sub-tiles of 1 KiB operand runs) needs these.
  if (c.kv_dtype == FKV_DTYPE_Q8_0 && (c.head_dim % 64 != 0 || c.block_size % 16 != 0))
    return fail(FKV_ERR_KERNEL, "q8_0 kv needs head_dim % 64 == 0 and block_size % 16 == 0");
  if (c.f16_rounding != FKV_ROUND_NEAREST_EVEN && c.f16_rounding != FKV_ROUND_HALF_AWAY)
    return fail(FKV_ERR_INVALID, "unknown f16 rounding mode");
  if (c.num_blocks > 0x7fffffffull || c.num_host_blocks > 0x7fffffffull)
    return fail(FKV_ERR_CACHE, "kv pool size overflow");
  const uint64_t tile = fkv::tile_bytes_for(c.kv_dtype, c.block_size, c.head_dim);
  uint64_t block = 0, total = 0, host_total = 0;
  if (mul_ovf((uint64_t)c.n_layers * 2u, (uint64_t)c.n_kv_heads, &block) ||
      mul_ovf(block, tile, &block) || mul_ovf(block, c.num_blocks, &total) ||
      mul_ovf(block, c.num_host_blocks, &host_total))
    return fail(FKV_ERR_CACHE, "kv pool size overflow");
  if ((uint64_t)c.num_blocks * c.block_size > 0x7fffffffffffffffull)
    return fail(FKV_ERR_CACHE, "kv pool size overflow");

  DeviceGuard dg(c.device);
  if (!dg.ok) return fail(FKV_ERR_INTERNAL, "hip: cannot select device");
  // Set-up of the no-allocation decode step on this device: the address of the
  // device's static scratch, taken once per device with the device current.
  FKV_HIP(fkv::static_scratch_setup(c.device), "static scratch address");
  auto* p = new fkv_pool();
  p->cfg = c;
  hipError_t e = hipMalloc((void**)&p->dev, total);
  if (e != hipSuccess) {
    delete p;
    return fail(FKV_ERR_UNAVAILABLE, "no device memory for kv pool");
  }
  // Four device words: the FKV_FAULT_* bits; the number of marked device blocks; one
  // unused; the staging word of fkv_paged_take_fault_flags. Then one mark per device
  // block and per host block (a Q8_0 scale of 512 or more, or an Inf/NaN K or V of an
  // F16 pool, stored in the block: the attention kernels read them to pick the exact or
  // leak-safe instance for the workgroups that read such a block).
  e = hipMalloc((void**)&p->fault, 4 * sizeof(uint32_t));
  if (e == hipSuccess) e = hipMemset(p->fault, 0, 4 * sizeof(uint32_t));
  const uint64_t n_marks = c.num_blocks + c.num_host_blocks;
  if (e == hipSuccess) e = hipMalloc((void**)&p->marks, n_marks * sizeof(uint32_t));
  if (e == hipSuccess) e = hipMemset(p->marks, 0, n_marks * sizeof(uint32_t));
  if (e == hipSuccess)
    e = hipHostMalloc((void**)&p->fault_host, 64, hipHostMallocDefault);
  if (e == hipSuccess && host_total) e = hipHostMalloc((void**)&p->host, host_total, hipHostMallocDefault);
  if (e != hipSuccess) {
    (void)hipFree(p->dev);
    if (p->fault) (void)hipFree(p->fault);
    if (p->marks) (void)hipFree(p->marks);
    if (p->fault_host) (void)hipHostFree(p->fault_host);
    delete p;
    return hip_fail(e, "pool allocation");
  }
  p->geom.base = p->dev;
  p->geom.tile_bytes = tile;
  p->geom.block_bytes = block;
  p->geom.num_blocks = c.num_blocks;
  p->geom.n_layers = c.n_layers;
  p->geom.n_kv_heads = c.n_kv_heads;
  p->geom.head_dim = c.head_dim;
  p->geom.block_size = c.block_size;
  p->geom.dtype = c.kv_dtype;
  p->geom.rounding = c.f16_rounding;
  p->geom.fault = p->fault;
  p->geom.bmark = p->marks;
  p->geom.hmark = p->marks + c.num_blocks;
  int cus = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, c.device) != hipSuccess)
    cus = 0;
  p->geom.n_cus = cus > 0 ? (uint32_t)cus : 0u;
  p->free_list.resize(c.num_blocks);
  for (uint64_t i = 0; i < c.num_blocks; i++)
    p->free_list[i] = (int32_t)(c.num_blocks - 1 - i);  // pop order 0, 1, 2, ...
  p->refcount.assign(c.num_blocks, 0);
  *out = p;
  return ok();
}

int32_t fkv_paged_destroy(fkv_pool* pool) {
  fkv::KeepLastError keep;
  if (!pool) return ok();
  for (fkv_seqs* m : pool->managers) detach_manager(m);
  DeviceGuard dg(pool->cfg.device);
  (void)hipDeviceSynchronize();
  if (pool->dev) (void)hipFree(pool->dev);
  if (pool->fault) (void)hipFree(pool->fault);
  if (pool->marks) (void)hipFree(pool->marks);
  if (pool->fault_host) (void)hipHostFree(pool->fault_host);
  if (pool->host) (void)hipHostFree(pool->host);
  if (pool->rope_sc) (void)hipFree(pool->rope_sc);
  for (float* t : pool->rope_old) (void)hipFree(t);
  delete pool;
  return ok();
}

int32_t fkv_paged_get_info(const fkv_pool* pool, fkv_paged_info* out) {
  if (!pool || !out) return fail(FKV_ERR_INVALID, "null argument");
  out->tile_bytes = pool->geom.tile_bytes;
  out->block_bytes = pool->geom.block_bytes;
  out->pool_bytes = pool->geom.block_bytes * pool->geom.num_blocks;
  out->free_blocks = pool->free_list.size();
  out->device_base = pool->dev;
  out->host_base = pool->host;
  return ok();
}

int32_t fkv_paged_take_fault_flags(fkv_pool* pool, void* stream, uint32_t* flags_out) {
  if (!pool || !flags_out) return fail(FKV_ERR_INVALID, "null argument");
  // The exchange's staging word and the pinned copy are per pool: a second thread's
  // exchange between this one's and its copy would hand it the other's bits.
  std::lock_guard<std::mutex> lock(pool->fault_mu);
  DeviceGuard dg(pool->cfg.device);
  const hipStream_t s = (hipStream_t)stream;
  FKV_HIP(fkv::launch_take_fault(pool->fault, s), "take fault flags");
  FKV_HIP(hipMemcpyAsync(pool->fault_host, pool->fault + 3, sizeof(uint32_t),
                         hipMemcpyDeviceToHost, s),
          "read fault flags");
  FKV_HIP(hipStreamSynchronize(s), "synchronize");
  *flags_out = *(volatile uint32_t*)pool->fault_host;
  return ok();
}

int32_t fkv_paged_marked_blocks(fkv_pool* pool, void* stream, uint64_t* count_out) {
  if (!pool || !count_out) return fail(FKV_ERR_INVALID, "null argument");
  std::lock_guard<std::mutex> lock(pool->fault_mu);  // shares the pinned word
  DeviceGuard dg(pool->cfg.device);
  const hipStream_t s = (hipStream_t)stream;
  FKV_HIP(hipMemcpyAsync(pool->fault_host, pool->fault + 1, sizeof(uint32_t),
                         hipMemcpyDeviceToHost, s),
          "read block marks");
  FKV_HIP(hipStreamSynchronize(s), "synchronize");
  *count_out = *(volatile uint32_t*)pool->fault_host;
  return ok();
}

// Whether a value of the pool's dtype whose every byte is `byte` is one that marks its
// block: a Q8_0 scale (byte << 8 | byte) of 512 or more (exponent bits 14 and 13), an F16
// K or V value that is Inf or NaN (exponent bits 14 to 10).
static uint32_t fill_marks(const fkv_pool* pool, uint8_t byte) {
  if (pool->cfg.kv_dtype == FKV_DTYPE_Q8_0) return (byte & 0x60u) == 0x60u ? 1u : 0u;
  if (pool->cfg.kv_dtype == FKV_DTYPE_F16) return (byte & 0x7cu) == 0x7cu ? 1u : 0u;
  return 0u;
}

int32_t fkv_paged_fill(fkv_pool* pool, uint8_t byte, void* stream) {
  if (!pool) return fail(FKV_ERR_INVALID, "null argument");
  DeviceGuard dg(pool->cfg.device);
  FKV_HIP(fkv::launch_fill(pool->dev, byte, pool->geom.block_bytes * pool->geom.num_blocks,
                           (hipStream_t)stream),
          "fill");
  // Every device block now holds the same bytes, so every mark follows the fill byte,
  // whatever the block held before. Host blocks keep theirs (swap_in brings them back).
  FKV_HIP(fkv::launch_marks_fill(pool->geom, fill_marks(pool, byte), (hipStream_t)stream), "fill");
  return ok();
}

// Whether bytes [offset, offset + bytes) of an F16 pool image (src) write an Inf or NaN
// K or V value (every 16-bit word of a K or V tile is a value, little-endian, so its high
// byte decides; tiles start at even offsets, so the high bytes are the odd offsets).
static bool f16_image_has_nonfinite_kv(const fkv_pool* pool, uint64_t offset, uint64_t bytes,
                                       const uint8_t* src) {
  (void)pool;
  for (uint64_t x = offset + (offset % 2 == 0 ? 1 : 0); x < offset + bytes; x += 2)
    if ((src[x - offset] & 0x7cu) == 0x7cu) return true;
  return false;
}

// Whether bytes [offset, offset + bytes) of a Q8_0 pool image (src) write a scale of
// 512 or more. The f16 scales sit at the end of every tile ([B][D/32] little-endian
// after the B*D quants), and whether one is that large depends on its high byte only
// (exponent bits 14 and 13), so the high bytes the range covers decide.
static bool q8_image_has_wide_scale(const fkv_pool* pool, uint64_t offset, uint64_t bytes,
                                    const uint8_t* src) {
  const uint64_t tile = pool->geom.tile_bytes;
  const uint64_t q = (uint64_t)pool->cfg.block_size * pool->cfg.head_dim;
  const uint64_t sc_end = q + q / 32 * 2;
  const uint64_t end = offset + bytes;
  for (uint64_t t0 = offset / tile * tile; t0 < end; t0 += tile) {
    for (uint64_t x = t0 + q + 1; x < t0 + sc_end && x < end; x += 2)
      if (x >= offset && (src[x - offset] & 0x60u) == 0x60u) return true;
  }
  return false;
}

static int32_t check_range(const fkv_pool* pool, uint64_t offset, uint64_t bytes) {
  const uint64_t total = pool->geom.block_bytes * pool->geom.num_blocks;
  if (offset > total || bytes > total - offset) return fail(FKV_ERR_INVALID, "range outside the pool");
  return FKV_OK;
}

int32_t fkv_paged_read(fkv_pool* pool, uint64_t offset, uint64_t bytes, void* host_dst,
                       void* stream) {
  if (!pool || (bytes && !host_dst)) return fail(FKV_ERR_INVALID, "null argument");
  if (check_range(pool, offset, bytes)) return FKV_ERR_INVALID;
  DeviceGuard dg(pool->cfg.device);
  const hipStream_t s = (hipStream_t)stream;
  if (bytes)
    FKV_HIP(hipMemcpyAsync(host_dst, pool->dev + offset, bytes, hipMemcpyDeviceToHost, s),
            "pool read");
  FKV_HIP(hipStreamSynchronize(s), "synchronize");
  return ok();
}

int32_t fkv_paged_write(fkv_pool* pool, uint64_t offset, uint64_t bytes, const void* host_src,
                        void* stream) {
  if (!pool || (bytes && !host_src)) return fail(FKV_ERR_INVALID, "null argument");
  if (check_range(pool, offset, bytes)) return FKV_ERR_INVALID;
  DeviceGuard dg(pool->cfg.device);
  const hipStream_t s = (hipStream_t)stream;
  if (bytes)
    FKV_HIP(hipMemcpyAsync(pool->dev + offset, host_src, bytes, hipMemcpyHostToDevice, s),
            "pool write");
  // Marks of the blocks the range touches: set where the written bytes hold a marking
  // value, cleared where they overwrite a whole block without one, kept otherwise.
  const uint8_t* img = (const uint8_t*)host_src;
  uint8_t* ops_dev = nullptr;
  std::vector<uint8_t> ops;
  const uint64_t bb = pool->geom.block_bytes;
  const bool marking = pool->cfg.kv_dtype == FKV_DTYPE_Q8_0 || pool->cfg.kv_dtype == FKV_DTYPE_F16;
  if (bytes && marking) {
    const uint64_t b0 = offset / bb, b1 = (offset + bytes - 1) / bb + 1;
    ops.assign(b1 - b0, 0);
    for (uint64_t b = b0; b < b1; b++) {
      const uint64_t lo = std::max(offset, b * bb), hi = std::min(offset + bytes, (b + 1) * bb);
      const uint8_t* src = img + (lo - offset);
      const bool has = pool->cfg.kv_dtype == FKV_DTYPE_Q8_0
                           ? q8_image_has_wide_scale(pool, lo, hi - lo, src)
                           : f16_image_has_nonfinite_kv(pool, lo, hi - lo, src);
      ops[b - b0] = has ? 1 : (lo == b * bb && hi == (b + 1) * bb ? 2 : 0);
    }
    FKV_HIP(hipMalloc((void**)&ops_dev, ops.size()), "pool write");
    hipError_t e = hipMemcpyAsync(ops_dev, ops.data(), ops.size(), hipMemcpyHostToDevice, s);
    if (e == hipSuccess) e = fkv::launch_marks_apply(pool->geom, b0, ops.size(), ops_dev, s);
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    (void)hipFree(ops_dev);
    if (e != hipSuccess) return hip_fail(e, "pool write");
  }
  FKV_HIP(hipStreamSynchronize(s), "synchronize");
  return ok();
}

// ---------------------------------------------------------------------------
// Block allocator
// ---------------------------------------------------------------------------

int32_t fkv_block_alloc(fkv_pool* pool, uint32_t n, int32_t* ids_out) {
  if (!pool || (n && !ids_out)) return fail(FKV_ERR_INVALID, "null argument");
  if (pool->free_list.size() < n) return fail(FKV_ERR_UNAVAILABLE, "no free kv blocks");
  for (uint32_t i = 0; i < n; i++) {
    int32_t id = pool->free_list.back();
    pool->free_list.pop_back();
    pool->refcount[(size_t)id] = 1;
    ids_out[i] = id;
  }
  return ok();
}

int32_t fkv_block_free(fkv_pool* pool, uint32_t n, const int32_t* ids) {
  if (!pool || (n && !ids)) return fail(FKV_ERR_INVALID, "null argument");
  // Validate first (ids repeated in one call count once per occurrence) so a bad
  // id leaves the allocator unchanged.
  std::vector<int32_t> sorted(ids, ids + n);
  std::sort(sorted.begin(), sorted.end());
  for (size_t i = 0; i < sorted.size();) {
    size_t j = i;
    while (j < sorted.size() && sorted[j] == sorted[i]) j++;
    int32_t id = sorted[i];
    if (id < 0 || (uint64_t)id >= pool->cfg.num_blocks || pool->refcount[(size_t)id] < j - i)
      return fail(FKV_ERR_CACHE, "free of unallocated block");
    i = j;
  }
  for (uint32_t i = 0; i < n; i++) {
    uint32_t& rc = pool->refcount[(size_t)ids[i]];
    if (--rc == 0) pool->free_list.push_back(ids[i]);
  }
  return ok();
}

int32_t fkv_block_ref(fkv_pool* pool, uint32_t n, const int32_t* ids) {
  if (!pool || (n && !ids)) return fail(FKV_ERR_INVALID, "null argument");
  for (uint32_t i = 0; i < n; i++) {
    int32_t id = ids[i];
    if (id < 0 || (uint64_t)id >= pool->cfg.num_blocks || pool->refcount[(size_t)id] == 0)
      return fail(FKV_ERR_CACHE, "reference to unallocated block");
  }
  for (uint32_t i = 0; i < n; i++) pool->refcount[(size_t)ids[i]]++;
  return ok();
}

int32_t fkv_block_refcount(const fkv_pool* pool, int32_t id, uint32_t* out) {
  if (!pool || !out) return fail(FKV_ERR_INVALID, "null argument");
  if (id < 0 || (uint64_t)id >= pool->cfg.num_blocks) return fail(FKV_ERR_CACHE, "unknown block");
  *out = pool->refcount[(size_t)id];
  return ok();
}

// ---------------------------------------------------------------------------
// Device operations
// ---------------------------------------------------------------------------

int32_t fkv_append(fkv_pool* pool, uint32_t layer, const float* k, const float* v,
                   const int64_t* slot_mapping, uint32_t n_tokens, void* stream) {
  if (!pool) return fail(FKV_ERR_INVALID, "null argument");
  if (layer >= pool->cfg.n_layers) return fail(FKV_ERR_CACHE, "layer out of range");
  if (n_tokens == 0) return ok();
  if (!k || !v || !slot_mapping) return fail(FKV_ERR_INVALID, "null argument");
  DeviceGuard dg(pool->cfg.device);
  FKV_HIP(fkv::launch_append(pool->geom, layer, k, v, slot_mapping, n_tokens, (hipStream_t)stream),
          "append");
  return ok();
}

static int32_t check_format(int32_t format) {
  if (format != FKV_GATHER_F32 && format != FKV_GATHER_RAW)
    return fail(FKV_ERR_INVALID, "unknown gather format");
  return FKV_OK;
}

int32_t fkv_gather_slots(fkv_pool* pool, uint32_t layer, const int64_t* slot_mapping,
                         uint32_t n_tokens, int32_t format, void* out_k, void* out_v,
                         void* stream) {
  if (!pool) return fail(FKV_ERR_INVALID, "null argument");
  if (layer >= pool->cfg.n_layers) return fail(FKV_ERR_CACHE, "layer out of range");
  if (check_format(format)) return FKV_ERR_INVALID;
  if (n_tokens == 0) return ok();
  if (!slot_mapping || !out_k || !out_v) return fail(FKV_ERR_INVALID, "null argument");
  DeviceGuard dg(pool->cfg.device);
  FKV_HIP(fkv::launch_gather_slots(pool->geom, layer, slot_mapping, n_tokens, format, out_k, out_v,
                                   (hipStream_t)stream),
          "gather");
  return ok();
}

int32_t fkv_gather_tables(fkv_pool* pool, uint32_t layer, const int32_t* block_tables,
                          uint32_t max_blocks_per_seq, const int32_t* ctx_lens,
                          const int64_t* out_offsets, uint32_t n_seqs, uint32_t max_ctx_len,
                          int32_t format, void* out_k, void* out_v, void* stream) {
  if (!pool) return fail(FKV_ERR_INVALID, "null argument");
  if (layer >= pool->cfg.n_layers) return fail(FKV_ERR_CACHE, "layer out of range");
  if (check_format(format)) return FKV_ERR_INVALID;
  if (n_seqs == 0) return ok();
  if (n_seqs > 65535) return fail(FKV_ERR_INVALID, "too many sequences in one gather");
  if (!block_tables || !ctx_lens || !out_offsets || !out_k || !out_v)
    return fail(FKV_ERR_INVALID, "null argument");
  if ((uint64_t)max_ctx_len > (uint64_t)max_blocks_per_seq * pool->cfg.block_size)
    return fail(FKV_ERR_INVALID, "max_ctx_len exceeds the block table");
  if (pool->cfg.kv_dtype != FKV_DTYPE_Q8_0 && pool->cfg.head_dim % 8 != 0)
    return fail(FKV_ERR_KERNEL, "gather_tables needs head_dim % 8 == 0");
  DeviceGuard dg(pool->cfg.device);
  FKV_HIP(fkv::launch_gather_tables(pool->geom, layer, block_tables, max_blocks_per_seq, ctx_lens,
                                    out_offsets, n_seqs, max_ctx_len, format, out_k, out_v,
                                    (hipStream_t)stream),
          "gather_tables");
  return ok();
}

int32_t fkv_copy_blocks(fkv_pool* pool, const int64_t* pairs, uint32_t n_pairs, void* stream) {
  if (!pool) return fail(FKV_ERR_INVALID, "null argument");
  if (n_pairs == 0) return ok();
  if (!pairs) return fail(FKV_ERR_INVALID, "null argument");
  DeviceGuard dg(pool->cfg.device);
  FKV_HIP(fkv::launch_copy_blocks(pool->geom, pairs, n_pairs, (hipStream_t)stream), "copy_blocks");
  return ok();
}

static int32_t swap(fkv_pool* pool, const int64_t* pairs, uint32_t n_pairs, void* stream,
                    bool out) {
  if (!pool) return fail(FKV_ERR_INVALID, "null argument");
  if (n_pairs == 0) return ok();
  if (!pairs) return fail(FKV_ERR_INVALID, "null argument");
  if (!pool->host) return fail(FKV_ERR_CACHE, "pool has no host swap space");
  const uint64_t nb = pool->cfg.num_blocks, nh = pool->cfg.num_host_blocks;
  for (uint32_t i = 0; i < n_pairs; i++) {
    int64_t a = pairs[2 * i], b = pairs[2 * i + 1];
    int64_t dev = out ? a : b, host = out ? b : a;
    if (dev < 0 || (uint64_t)dev >= nb) return fail(FKV_ERR_CACHE, "unknown block");
    if (host < 0 || (uint64_t)host >= nh) return fail(FKV_ERR_CACHE, "unknown host block");
  }
  DeviceGuard dg(pool->cfg.device);
  const uint64_t bb = pool->geom.block_bytes;
  // The blocks' marks travel with their bytes: swap_out copies them to the host blocks'
  // before the bytes leave, swap_in back after the bytes arrive (stream order).
  auto move_marks = [&]() -> hipError_t {
    fkv::MarkPairs mp{};
    for (uint32_t i = 0; i < n_pairs; i++) {
      mp.dev[mp.n] = (int32_t)(out ? pairs[2 * i] : pairs[2 * i + 1]);
      mp.host[mp.n] = (int32_t)(out ? pairs[2 * i + 1] : pairs[2 * i]);
      if (++mp.n == fkv::kMarkPairs || i + 1 == n_pairs) {
        const hipError_t e = fkv::launch_marks_swap(pool->geom, mp, out, (hipStream_t)stream);
        if (e != hipSuccess) return e;
        mp.n = 0;
      }
    }
    return hipSuccess;
  };
  if (out) FKV_HIP(move_marks(), "swap_out");
  // Merge runs that are consecutive on both sides into one copy each.
  uint32_t i = 0;
  while (i < n_pairs) {
    uint32_t j = i + 1;
    while (j < n_pairs && pairs[2 * j] == pairs[2 * (j - 1)] + 1 &&
           pairs[2 * j + 1] == pairs[2 * (j - 1) + 1] + 1)
      j++;
    const uint64_t bytes = (uint64_t)(j - i) * bb;
    if (out) {
      FKV_HIP(hipMemcpyAsync(pool->host + (uint64_t)pairs[2 * i + 1] * bb,
                             pool->dev + (uint64_t)pairs[2 * i] * bb, bytes,
                             hipMemcpyDeviceToHost, (hipStream_t)stream),
              "swap_out");
    } else {
      FKV_HIP(hipMemcpyAsync(pool->dev + (uint64_t)pairs[2 * i + 1] * bb,
                             pool->host + (uint64_t)pairs[2 * i] * bb, bytes,
                             hipMemcpyHostToDevice, (hipStream_t)stream),
              "swap_in");
    }
    i = j;
  }
  if (!out) FKV_HIP(move_marks(), "swap_in");
  return ok();
}

int32_t fkv_swap_out(fkv_pool* pool, const int64_t* pairs, uint32_t n_pairs, void* stream) {
  return swap(pool, pairs, n_pairs, stream, true);
}

int32_t fkv_swap_in(fkv_pool* pool, const int64_t* pairs, uint32_t n_pairs, void* stream) {
  return swap(pool, pairs, n_pairs, stream, false);
}

static int32_t check_attention(const fkv_pool* pool, uint32_t n_heads, uint32_t max_ctx_len) {
  const fkv_paged_config& c = pool->cfg;
  if (n_heads == 0 || n_heads % c.n_kv_heads != 0) return fail(FKV_ERR_KERNEL, "length mismatch");
  if (c.block_size != (uint32_t)fkv::kAttnBlock ||
      !fkv::attention_supported(c.kv_dtype, c.head_dim, n_heads / c.n_kv_heads))
    return fail(FKV_ERR_KERNEL, "unsupported attention shape");
  uint64_t parts = ((uint64_t)max_ctx_len + fkv::kAttnPartTokens - 1) / fkv::kAttnPartTokens;
  if (parts > 65535 || max_ctx_len > (1u << 30)) return fail(FKV_ERR_KERNEL, "context too long");
  return FKV_OK;
}

int32_t fkv_decode_attention_workspace_size(const fkv_pool* pool, uint32_t n_heads,
                                            uint32_t n_seqs, uint32_t max_ctx_len,
                                            uint64_t* bytes_out) {
  if (!pool || !bytes_out) return fail(FKV_ERR_INVALID, "null argument");
  int32_t st = check_attention(pool, n_heads, max_ctx_len);
  if (st) return st;
  DeviceGuard dg(pool->cfg.device);  // the F16 plan depends on the device's CU count
  *bytes_out = fkv::attention_workspace_bytes(pool->geom, n_heads, n_seqs, max_ctx_len);
  return ok();
}

static int32_t decode_attention(fkv_pool* pool, uint32_t layer, uint32_t n_heads,
                                const float* k_new, const float* v_new, const float* q,
                                float* out, const int32_t* block_tables,
                                uint32_t max_blocks_per_seq, const int32_t* ctx_lens,
                                uint32_t n_seqs, uint32_t max_ctx_len, float scale,
                                void* workspace, uint64_t workspace_bytes, void* stream,
                                const fkv::RopeTable* rope = nullptr, bool use_static = false) {
  if (!pool) return fail(FKV_ERR_INVALID, "null argument");
  if (layer >= pool->cfg.n_layers) return fail(FKV_ERR_CACHE, "layer out of range");
  int32_t st = check_attention(pool, n_heads, max_ctx_len);
  if (st) return st;
  if (n_seqs == 0) return ok();
  if (!q || !out || !block_tables || !ctx_lens) return fail(FKV_ERR_INVALID, "null argument");
  if ((uintptr_t)q % 16 != 0) return fail(FKV_ERR_INVALID, "q must be 16-byte aligned");
  if ((uint64_t)n_seqs * pool->cfg.n_kv_heads > 0x7fffffffull)
    return fail(FKV_ERR_INVALID, "too many sequences");
  if ((uint64_t)max_ctx_len > (uint64_t)max_blocks_per_seq * pool->cfg.block_size)
    return fail(FKV_ERR_INVALID, "max_ctx_len exceeds the block table");
  DeviceGuard dg(pool->cfg.device);
  const uint64_t need =
      rope    ? fkv::rope_attention_workspace_bytes(pool->geom, n_heads, n_seqs, max_ctx_len)
      : k_new ? fkv::append_attention_workspace_bytes(pool->geom, n_heads, n_seqs, max_ctx_len)
              : fkv::attention_workspace_bytes(pool->geom, n_heads, n_seqs, max_ctx_len);
  if (use_static) {
    if (need > fkv::kStaticScratchBytes)
      return fail(FKV_ERR_INVALID,
                  "decode step needs " + std::to_string(need) +
                      " bytes of scratch; the static scratch holds " +
                      std::to_string(fkv::kStaticScratchBytes));
    workspace = fkv::static_scratch(pool->cfg.device);
    workspace_bytes = fkv::kStaticScratchBytes;
    if (!workspace) return fail(FKV_ERR_INTERNAL, "static scratch is not set up on the device");
  }
  if (workspace_bytes < need || (need && !workspace))
    return fail(FKV_ERR_INVALID, "attention workspace too small");
  FKV_HIP(fkv::launch_decode_attention(pool->geom, layer, n_heads, q, out, block_tables,
                                       max_blocks_per_seq, ctx_lens, n_seqs, max_ctx_len, scale,
                                       workspace, k_new, v_new, (hipStream_t)stream, rope),
          "decode_attention");
  return ok();
}

int32_t fkv_decode_attention(fkv_pool* pool, uint32_t layer, uint32_t n_heads, const float* q,
                             float* out, const int32_t* block_tables,
                             uint32_t max_blocks_per_seq, const int32_t* ctx_lens,
                             uint32_t n_seqs, uint32_t max_ctx_len, float scale,
                             void* workspace, uint64_t workspace_bytes, void* stream) {
  return decode_attention(pool, layer, n_heads, nullptr, nullptr, q, out, block_tables,
                          max_blocks_per_seq, ctx_lens, n_seqs, max_ctx_len, scale, workspace,
                          workspace_bytes, stream);
}

int32_t fkv_append_decode_attention_workspace_size(const fkv_pool* pool, uint32_t n_heads,
                                                   uint32_t n_seqs, uint32_t max_ctx_len,
                                                   uint64_t* bytes_out) {
  if (!pool || !bytes_out) return fail(FKV_ERR_INVALID, "null argument");
  int32_t st = check_attention(pool, n_heads, max_ctx_len);
  if (st) return st;
  DeviceGuard dg(pool->cfg.device);
  *bytes_out = fkv::append_attention_workspace_bytes(pool->geom, n_heads, n_seqs, max_ctx_len);
  return ok();
}

int32_t fkv_append_decode_attention(fkv_pool* pool, uint32_t layer, uint32_t n_heads,
                                    const float* k_new, const float* v_new, const float* q,
                                    float* out, const int32_t* block_tables,
                                    uint32_t max_blocks_per_seq, const int32_t* ctx_lens,
                                    uint32_t n_seqs, uint32_t max_ctx_len, float scale,
                                    void* workspace, uint64_t workspace_bytes, void* stream) {
  if (n_seqs && (!k_new || !v_new)) return fail(FKV_ERR_INVALID, "null argument");
  return decode_attention(pool, layer, n_heads, k_new, v_new, q, out, block_tables,
                          max_blocks_per_seq, ctx_lens, n_seqs, max_ctx_len, scale, workspace,
                          workspace_bytes, stream);
}

int32_t fkv_append_decode_attention_noalloc(fkv_pool* pool, uint32_t layer, uint32_t n_heads,
                                            const float* k_new, const float* v_new,
                                            const float* q, float* out,
                                            const int32_t* block_tables,
                                            uint32_t max_blocks_per_seq, const int32_t* ctx_lens,
                                            uint32_t n_seqs, uint32_t max_ctx_len, float scale,
                                            void* stream) {
  if (n_seqs && (!k_new || !v_new)) return fail(FKV_ERR_INVALID, "null argument");
  return decode_attention(pool, layer, n_heads, k_new, v_new, q, out, block_tables,
                          max_blocks_per_seq, ctx_lens, n_seqs, max_ctx_len, scale, nullptr, 0,
                          stream, nullptr, true);
}

// Kernels::rope's checks, in its order (crates/kernels/src/validate.rs:64-87: theta,
// then parity, then shape), and the per-pair denominators theta^(2i / rope_dim)
// computed in f32 as math.rs:31-34 does.
static int32_t rope_table(const fkv_pool* pool, uint32_t rope_dim, float theta,
                          fkv::RopeTable* t) {
  if (!(theta > 0.0f)) return fail(FKV_ERR_KERNEL, "theta must be positive");
  if (rope_dim % 2 != 0) return fail(FKV_ERR_KERNEL, "rope_dim must be even");
  if (rope_dim > pool->cfg.head_dim) return fail(FKV_ERR_KERNEL, "rope_dim exceeds head_dim");
  *t = fkv::RopeTable{};
  t->rope_dim = (int32_t)rope_dim;
  for (uint32_t i = 0; i < rope_dim / 2; i++)
    t->den[i] = powf(theta, (float)(2 * i) / (float)rope_dim);
  return FKV_OK;
}

// The pool's (sin, cos) table for rope_dim and theta covering positions [0, n_pos):
// sinf and cosf of f = pos / den[i] (the f32 division of math.rs:31-34) from the C
// library, as the reference's f32::sin_cos gives them, so the device rotates with the
// reference's values (the device sincosf can differ from them in the last bit, which
// moves a stored binary16 K across a rounding boundary now and then). Built on the host
// when the (rope_dim, theta) pair changes or n_pos outgrows it (doubling), uploaded with
// a blocking copy; 16 MiB at rope_dim 128 and 32,768 positions.
static int32_t rope_cache(fkv_pool* pool, fkv::RopeTable* t, float theta, uint32_t n_pos) {
  const uint32_t np = (uint32_t)t->rope_dim / 2u;
  if (np == 0 || n_pos == 0) return FKV_OK;
  // At most 2^20 positions (512 MiB at rope_dim 128, built once on the host); positions
  // past the table keep the device sincosf.
  constexpr uint64_t kMaxPos = 1ull << 20;
  std::lock_guard<std::mutex> lock(pool->rope_mu);
  const bool match = pool->rope_sc != nullptr && pool->rope_dim == (uint32_t)t->rope_dim &&
                     memcmp(&pool->rope_theta, &theta, sizeof(float)) == 0;
  if (!match || (pool->rope_pos < n_pos && pool->rope_pos < kMaxPos)) {
    uint64_t want = 4096;
    while (want < n_pos && want < kMaxPos) want *= 2;
    if (match && want < 2ull * pool->rope_pos) want = 2ull * pool->rope_pos;
    if (want > kMaxPos) want = kMaxPos;
    std::vector<float> h(want * np * 2u);
    for (uint64_t pos = 0; pos < want; pos++)
      for (uint32_t i = 0; i < np; i++) {
        const float f = (float)pos / t->den[i];  // math.rs:33, f32
        h[(pos * np + i) * 2u] = sinf(f);
        h[(pos * np + i) * 2u + 1u] = cosf(f);
      }
    float* d = nullptr;
    hipError_t e = hipMalloc((void**)&d, h.size() * sizeof(float));
    if (e != hipSuccess) return fail(FKV_ERR_INTERNAL, std::string("rope table: ") + hipGetErrorString(e));
    e = hipMemcpy(d, h.data(), h.size() * sizeof(float), hipMemcpyHostToDevice);
    if (e != hipSuccess) {
      (void)hipFree(d);
      return fail(FKV_ERR_INTERNAL, std::string("rope table: ") + hipGetErrorString(e));
    }
    if (pool->rope_sc) pool->rope_old.push_back(pool->rope_sc);
    pool->rope_sc = d;
    pool->rope_pos = (uint32_t)want;
    pool->rope_dim = (uint32_t)t->rope_dim;
    pool->rope_theta = theta;
  }
  t->sc = pool->rope_sc;
  t->sc_pos = pool->rope_pos;
  return FKV_OK;
}

int32_t fkv_rope_append_decode_attention_workspace_size(const fkv_pool* pool, uint32_t n_heads,
                                                        uint32_t n_seqs, uint32_t max_ctx_len,
                                                        uint64_t* bytes_out) {
  if (!pool || !bytes_out) return fail(FKV_ERR_INVALID, "null argument");
  int32_t st = check_attention(pool, n_heads, max_ctx_len);
  if (st) return st;
  DeviceGuard dg(pool->cfg.device);
  *bytes_out = fkv::rope_attention_workspace_bytes(pool->geom, n_heads, n_seqs, max_ctx_len);
  return ok();
}

int32_t fkv_rope_append_decode_attention(fkv_pool* pool, uint32_t layer, uint32_t n_heads,
                                         uint32_t rope_dim, float theta, const float* k_new,
                                         const float* v_new, const float* q, float* out,
                                         const int32_t* block_tables, uint32_t max_blocks_per_seq,
                                         const int32_t* ctx_lens, uint32_t n_seqs,
                                         uint32_t max_ctx_len, float scale, void* workspace,
                                         uint64_t workspace_bytes, void* stream) {
  if (!pool) return fail(FKV_ERR_INVALID, "null argument");
  fkv::RopeTable rope;
  int32_t st = rope_table(pool, rope_dim, theta, &rope);
  if (st) return st;
  if (n_seqs && (!k_new || !v_new)) return fail(FKV_ERR_INVALID, "null argument");
  if (n_seqs) {
    DeviceGuard dg(pool->cfg.device);
    st = rope_cache(pool, &rope, theta, max_ctx_len);
    if (st) return st;
  }
  return decode_attention(pool, layer, n_heads, k_new, v_new, q, out, block_tables,
                          max_blocks_per_seq, ctx_lens, n_seqs, max_ctx_len, scale, workspace,
                          workspace_bytes, stream, &rope);
}

// Argument checks shared by the prefill workspace query and the call.
static int32_t check_prefill(const fkv_pool* pool, uint32_t n_heads, uint32_t n_seqs,
                             uint32_t max_blocks_per_seq, uint32_t max_q_len,
                             uint32_t max_ctx_len) {
  int32_t st = check_attention(pool, n_heads, max_ctx_len);
  if (st) return st;
  if (pool->cfg.kv_dtype != FKV_DTYPE_F16 && pool->cfg.kv_dtype != FKV_DTYPE_Q8_0)
    return fail(FKV_ERR_KERNEL, "prefill attention needs f16 or q8_0 kv");
  // the kernel offsets blocks by a 32 x 32-bit product
  if (pool->geom.block_bytes > 0xffffffffull)
    return fail(FKV_ERR_KERNEL, "prefill attention needs kv blocks under 4 GiB");
  if ((uint64_t)n_seqs * pool->cfg.n_kv_heads > 0x7fffffffull)
    return fail(FKV_ERR_INVALID, "too many sequences");
  if (max_q_len > max_ctx_len) return fail(FKV_ERR_INVALID, "max_q_len exceeds max_ctx_len");
  const uint32_t tokens_per_tile = 16u / (n_heads / pool->cfg.n_kv_heads);
  if (((uint64_t)max_q_len + tokens_per_tile - 1) / tokens_per_tile > 65535ull * 4u)
    return fail(FKV_ERR_KERNEL, "prefill chunk too long");
  (void)max_blocks_per_seq;
  return FKV_OK;
}

int32_t fkv_prefill_attention_workspace_size(const fkv_pool* pool, uint32_t n_heads,
                                             uint32_t n_seqs, uint32_t max_q_len,
                                             uint32_t max_ctx_len, uint64_t* bytes_out) {
  if (!pool || !bytes_out) return fail(FKV_ERR_INVALID, "null argument");
  int32_t st = check_prefill(pool, n_heads, n_seqs, 0, max_q_len, max_ctx_len);
  if (st) return st;
  *bytes_out = (n_seqs == 0 || max_q_len == 0)
                   ? 0
                   : fkv::prefill_plan(pool->geom, n_heads, n_seqs, max_q_len, max_ctx_len).ws_bytes;
  return ok();
}

int32_t fkv_prefill_attention(fkv_pool* pool, uint32_t layer, uint32_t n_heads, const float* q,
                              float* out, const int32_t* block_tables,
                              uint32_t max_blocks_per_seq, const int32_t* ctx_lens,
                              const int32_t* q_lens, const int64_t* q_offsets, uint32_t n_seqs,
                              uint32_t max_q_len, uint32_t max_ctx_len, float scale,
                              void* workspace, uint64_t workspace_bytes, void* stream) {
  if (!pool) return fail(FKV_ERR_INVALID, "null argument");
  if (layer >= pool->cfg.n_layers) return fail(FKV_ERR_CACHE, "layer out of range");
  int32_t st = check_prefill(pool, n_heads, n_seqs, max_blocks_per_seq, max_q_len, max_ctx_len);
  if (st) return st;
  if (n_seqs == 0 || max_q_len == 0) return ok();
  if (!q || !out || !block_tables || !ctx_lens || !q_lens || !q_offsets)
    return fail(FKV_ERR_INVALID, "null argument");
  if ((uintptr_t)q % 16 != 0) return fail(FKV_ERR_INVALID, "q must be 16-byte aligned");
  if ((uint64_t)max_ctx_len > (uint64_t)max_blocks_per_seq * pool->cfg.block_size)
    return fail(FKV_ERR_INVALID, "max_ctx_len exceeds the block table");
  const fkv::PrefillPlan plan =
      fkv::prefill_plan(pool->geom, n_heads, n_seqs, max_q_len, max_ctx_len);
  if (workspace && workspace_bytes < plan.ws_bytes)
    return fail(FKV_ERR_INVALID, "prefill workspace too small");
  if ((uintptr_t)workspace % 16 != 0)
    return fail(FKV_ERR_INVALID, "workspace must be 16-byte aligned");
  DeviceGuard dg(pool->cfg.device);
  FKV_HIP(fkv::launch_prefill_attention(pool->geom, layer, n_heads, q, out, block_tables,
                                        max_blocks_per_seq, ctx_lens, q_lens, q_offsets, n_seqs,
                                        max_q_len, scale, plan,
                                        plan.ws_bytes ? workspace : nullptr, (hipStream_t)stream),
          "prefill_attention");
  return ok();
}

int32_t fkv_device_copy(void* dst, const void* src, uint64_t bytes, void* stream) {
  if (bytes && (!dst || !src)) return fail(FKV_ERR_INVALID, "null argument");
  if (((uintptr_t)dst | (uintptr_t)src) % 16 != 0)
    return fail(FKV_ERR_INVALID, "device_copy needs 16-byte aligned pointers");
  FKV_HIP(fkv::launch_device_copy(dst, src, bytes, (hipStream_t)stream), "device_copy");
  return ok();
}

// ---------------------------------------------------------------------------
// Revision-1 compat pool (crates/kvcache/src/pool.rs), device storage
// ---------------------------------------------------------------------------

int32_t fkv_kvpool_new(const fkv_kvpool_config* config, int32_t device, fkv_kvpool** out) {
  if (!config || !out) return fail(FKV_ERR_INVALID, "null argument");
  *out = nullptr;
  const fkv_kvpool_config& c = *config;
  // pool.rs:22-29
  if (!c.n_layers || !c.n_kv_heads || !c.head_dim || !c.max_seq_len || !c.max_slots)
    return fail(FKV_ERR_CACHE, "kv pool dimension is zero");
  // pool.rs:30-38 (plus the 32-bit fields of the paged geometry)
  uint64_t block = 0, per_slot = 0, total = 0;
  if (mul_ovf(c.n_kv_heads, c.head_dim, &block) || mul_ovf(block, 2, &block) ||
      mul_ovf(c.n_layers, c.max_seq_len, &per_slot) || mul_ovf(per_slot, block, &per_slot) ||
      mul_ovf(per_slot, c.max_slots, &total) || mul_ovf(total, 4, &total) ||
      c.n_layers > 0xffffffffull || c.n_kv_heads > 0xffffffffull ||
      c.head_dim > 0xffffffffull || c.max_seq_len > 0xffffffffull)
    return fail(FKV_ERR_CACHE, "kv pool size overflow");
  fkv_paged_config pc{};
  pc.n_layers = (uint32_t)c.n_layers;
  pc.n_kv_heads = (uint32_t)c.n_kv_heads;
  pc.head_dim = (uint32_t)c.head_dim;
  pc.block_size = (uint32_t)c.max_seq_len;
  pc.num_blocks = c.max_slots;
  pc.kv_dtype = FKV_DTYPE_F32;
  pc.f16_rounding = FKV_ROUND_NEAREST_EVEN;
  pc.device = device;
  fkv_pool* paged = nullptr;
  int32_t st = fkv_paged_create(&pc, &paged);
  if (st) return st;
  auto* p = new fkv_kvpool();
  p->cfg = c;
  p->paged = paged;
  p->free_.assign(c.max_slots, 1);
  p->seq_len.assign(c.max_slots, 0);
  p->layers_appended.assign(c.max_slots, 0);
  DeviceGuard dg(device);
  const uint64_t row = c.n_kv_heads * c.head_dim;
  hipError_t e = hipMalloc((void**)&p->stage, row * 2 * sizeof(float));
  if (e == hipSuccess) e = hipMalloc((void**)&p->slot_dev, sizeof(int64_t));
  if (e == hipSuccess) e = hipStreamCreateWithFlags(&p->stream, hipStreamNonBlocking);
  if (e != hipSuccess) {
    fkv_kvpool_destroy(p);
    return hip_fail(e, "kv pool allocation");
  }
  *out = p;
  return ok();
}

int32_t fkv_kvpool_destroy(fkv_kvpool* pool) {
  fkv::KeepLastError keep;
  if (!pool) return ok();
  {
    DeviceGuard dg(pool->paged ? pool->paged->cfg.device : 0);
    if (pool->stream) (void)hipStreamSynchronize(pool->stream);
    if (pool->stage) (void)hipFree(pool->stage);
    if (pool->slot_dev) (void)hipFree(pool->slot_dev);
    if (pool->stream) (void)hipStreamDestroy(pool->stream);
  }
  fkv_paged_destroy(pool->paged);
  delete pool;
  return ok();
}

int32_t fkv_kvpool_get_config(const fkv_kvpool* pool, fkv_kvpool_config* out) {
  if (!pool || !out) return fail(FKV_ERR_INVALID, "null argument");
  *out = pool->cfg;
  return ok();
}

int32_t fkv_kvpool_storage_len(const fkv_kvpool* pool, uint64_t* out) {
  if (!pool || !out) return fail(FKV_ERR_INVALID, "null argument");
  *out = pool->paged->geom.block_bytes * pool->paged->geom.num_blocks / sizeof(float);
  return ok();
}

// alloc, pool.rs:83-101: first free slot; the whole slot is zero-filled.
int32_t fkv_kvpool_alloc(fkv_kvpool* pool, uint32_t* slot_out) {
  if (!pool || !slot_out) return fail(FKV_ERR_INVALID, "null argument");
  for (uint64_t i = 0; i < pool->cfg.max_slots; i++) {
    if (!pool->free_[i]) continue;
    DeviceGuard dg(pool->paged->cfg.device);
    const uint64_t bb = pool->paged->geom.block_bytes;
    FKV_HIP(fkv::launch_fill(pool->paged->dev + i * bb, 0, bb, pool->stream), "alloc zero-fill");
    FKV_HIP(hipStreamSynchronize(pool->stream), "alloc zero-fill");
    pool->free_[i] = 0;
    pool->seq_len[i] = 0;
    pool->layers_appended[i] = 0;
    *slot_out = (uint32_t)i;
    return ok();
  }
  return fail(FKV_ERR_UNAVAILABLE, "no free kv slots");
}

// free, pool.rs:103-112.
int32_t fkv_kvpool_free(fkv_kvpool* pool, uint32_t slot) {
  if (!pool) return fail(FKV_ERR_INVALID, "null argument");
  if (slot >= pool->cfg.max_slots || pool->free_[slot])
    return fail(FKV_ERR_CACHE, "free of unallocated slot");
  pool->free_[slot] = 1;
  pool->seq_len[slot] = 0;
  pool->layers_appended[slot] = 0;
  return ok();
}

// seq_len, pool.rs:114-120.
int32_t fkv_kvpool_seq_len(const fkv_kvpool* pool, uint32_t slot, uint64_t* out) {
  if (!pool || !out) return fail(FKV_ERR_INVALID, "null argument");
  if (slot >= pool->cfg.max_slots) return fail(FKV_ERR_CACHE, "unknown slot");
  *out = pool->seq_len[slot];
  return ok();
}

// append_layer, pool.rs:122-153: same checks, same order. An out-of-range slot
// (a panic in the reference, which indexes `free[index]` unchecked) is
// "unknown slot" here.
int32_t fkv_kvpool_append_layer(fkv_kvpool* pool, uint32_t slot, uint64_t layer, const float* k,
                                uint64_t k_len, const float* v, uint64_t v_len) {
  if (!pool) return fail(FKV_ERR_INVALID, "null argument");
  const fkv_kvpool_config& c = pool->cfg;
  if (slot >= c.max_slots) return fail(FKV_ERR_CACHE, "unknown slot");
  if (pool->free_[slot]) return fail(FKV_ERR_CACHE, "append on free slot");
  if (layer >= c.n_layers) return fail(FKV_ERR_CACHE, "layer out of range");
  const uint64_t expected = c.n_kv_heads * c.head_dim;
  if (k_len != expected || v_len != expected) return fail(FKV_ERR_CACHE, "kv vector length mismatch");
  const uint64_t pos = pool->seq_len[slot];
  if (pos >= c.max_seq_len) return fail(FKV_ERR_CACHE, "sequence length exceeds max");
  if (pool->layers_appended[slot] != layer) return fail(FKV_ERR_CACHE, "layers must append in order");
  if (!k || !v) return fail(FKV_ERR_INVALID, "null argument");
  DeviceGuard dg(pool->paged->cfg.device);
  const int64_t s = (int64_t)((uint64_t)slot * c.max_seq_len + pos);
  FKV_HIP(hipMemcpyAsync(pool->stage, k, expected * 4, hipMemcpyHostToDevice, pool->stream), "append");
  FKV_HIP(hipMemcpyAsync(pool->stage + expected, v, expected * 4, hipMemcpyHostToDevice, pool->stream),
          "append");
  FKV_HIP(hipMemcpyAsync(pool->slot_dev, &s, sizeof s, hipMemcpyHostToDevice, pool->stream), "append");
  FKV_HIP(fkv::launch_append(pool->paged->geom, (uint32_t)layer, pool->stage, pool->stage + expected,
                             pool->slot_dev, 1, pool->stream),
          "append");
  FKV_HIP(hipStreamSynchronize(pool->stream), "append");
  pool->layers_appended[slot] += 1;
  return ok();
}

// commit_token, pool.rs:155-172.
int32_t fkv_kvpool_commit_token(fkv_kvpool* pool, uint32_t slot) {
  if (!pool) return fail(FKV_ERR_INVALID, "null argument");
  if (slot >= pool->cfg.max_slots) return fail(FKV_ERR_CACHE, "unknown slot");
  if (pool->free_[slot]) return fail(FKV_ERR_CACHE, "commit on free slot");
  if (pool->layers_appended[slot] != pool->cfg.n_layers)
    return fail(FKV_ERR_CACHE, "not every layer appended");
  const uint64_t next = pool->seq_len[slot] + 1;
  if (next > pool->cfg.max_seq_len) return fail(FKV_ERR_CACHE, "sequence length exceeds max");
  pool->seq_len[slot] = next;
  pool->layers_appended[slot] = 0;
  return ok();
}

// k / v, pool.rs:174-204.
static int32_t kvpool_read(const fkv_kvpool* pool, uint32_t slot, uint64_t layer, uint64_t pos,
                           float* out, uint64_t out_len, bool want_v) {
  if (!pool) return fail(FKV_ERR_INVALID, "null argument");
  const fkv_kvpool_config& c = pool->cfg;
  if (slot >= c.max_slots) return fail(FKV_ERR_CACHE, "unknown slot");
  if (pool->free_[slot]) return fail(FKV_ERR_CACHE, "read on free slot");
  if (pos >= pool->seq_len[slot]) return fail(FKV_ERR_CACHE, "position not yet committed");
  if (layer >= c.n_layers) return fail(FKV_ERR_CACHE, "layer out of range");
  const uint64_t n = c.n_kv_heads * c.head_dim;
  if (out_len != n) return fail(FKV_ERR_INVALID, "output length mismatch");
  if (!out) return fail(FKV_ERR_INVALID, "null argument");
  DeviceGuard dg(pool->paged->cfg.device);
  const int64_t s = (int64_t)((uint64_t)slot * c.max_seq_len + pos);
  FKV_HIP(hipMemcpyAsync(pool->slot_dev, &s, sizeof s, hipMemcpyHostToDevice, pool->stream), "read");
  FKV_HIP(fkv::launch_gather_slots(pool->paged->geom, (uint32_t)layer, pool->slot_dev, 1,
                                   FKV_GATHER_F32, pool->stage, pool->stage + n, pool->stream),
          "read");
  FKV_HIP(hipMemcpyAsync(out, pool->stage + (want_v ? n : 0), n * 4, hipMemcpyDeviceToHost,
                         pool->stream),
          "read");
  FKV_HIP(hipStreamSynchronize(pool->stream), "read");
  return ok();
}

int32_t fkv_kvpool_k(const fkv_kvpool* pool, uint32_t slot, uint64_t layer, uint64_t pos,
                     float* out, uint64_t out_len) {
  return kvpool_read(pool, slot, layer, pos, out, out_len, false);
}

int32_t fkv_kvpool_v(const fkv_kvpool* pool, uint32_t slot, uint64_t layer, uint64_t pos,
                     float* out, uint64_t out_len) {
  return kvpool_read(pool, slot, layer, pos, out, out_len, true);
}

// abandon_partial, pool.rs:207-216.
int32_t fkv_kvpool_abandon_partial(fkv_kvpool* pool, uint32_t slot) {
  if (!pool) return fail(FKV_ERR_INVALID, "null argument");
  if (slot >= pool->cfg.max_slots || pool->free_[slot])
    return fail(FKV_ERR_CACHE, "abandon on free slot");
  pool->layers_appended[slot] = 0;
  return ok();
}

// uncommit_token, pool.rs:218-231.
int32_t fkv_kvpool_uncommit_token(fkv_kvpool* pool, uint32_t slot) {
  if (!pool) return fail(FKV_ERR_INVALID, "null argument");
  if (slot >= pool->cfg.max_slots || pool->free_[slot])
    return fail(FKV_ERR_CACHE, "uncommit on free slot");
  if (pool->seq_len[slot] == 0) return fail(FKV_ERR_CACHE, "nothing to uncommit");
  pool->seq_len[slot] -= 1;
  pool->layers_appended[slot] = 0;
  return ok();
}

// ---------------------------------------------------------------------------
// Sequence block manager: the scheduler's KV bookkeeping on paged
// storage. crates/scheduler/src/batcher.rs admits while a dense slot is free
// (:108-129), rolls back by freeing the slot and re-running the prefix
// (restore_kv, :291-308) and frees the slot on finish (:329-338). Here a sequence
// is a list of blocks: admission asks for the blocks its tokens need, a fork
// shares blocks by reference and copies a shared block before its first write,
// a rollback truncates the list, and preemption moves the blocks to the pool's
// host storage and back.
// ---------------------------------------------------------------------------

}  // extern "C"

struct fkv_seqs {
  struct Seq {
    bool used = false;
    bool swapped = false;
    uint64_t len = 0;             // committed tokens
    std::vector<int32_t> blocks;  // device blocks; host blocks while swapped out
  };
  fkv_pool* pool = nullptr;
  std::vector<Seq> seqs;
  std::vector<uint32_t> free_ids;  // sequence ids to reuse
  std::vector<int32_t> host_free;  // the pool's free host blocks (LIFO)
};

// The pool is being destroyed: the manager keeps only its own memory.
static void detach_manager(fkv_seqs* m) { m->pool = nullptr; }

namespace {

fkv_seqs::Seq* seq_at(fkv_seqs* m, uint32_t id) {
  return m->pool && id < m->seqs.size() && m->seqs[id].used ? &m->seqs[id] : nullptr;
}
const fkv_seqs::Seq* seq_at(const fkv_seqs* m, uint32_t id) {
  return m->pool && id < m->seqs.size() && m->seqs[id].used ? &m->seqs[id] : nullptr;
}
uint64_t blocks_for(const fkv_pool* p, uint64_t tokens) {
  return (tokens + p->cfg.block_size - 1) / p->cfg.block_size;
}

}  // namespace

extern "C" {

int32_t fkv_seqs_create(fkv_pool* pool, fkv_seqs** out) {
  if (!pool || !out) return fail(FKV_ERR_INVALID, "null argument");
  auto* m = new fkv_seqs();
  m->pool = pool;
  pool->managers.push_back(m);
  for (uint64_t i = pool->cfg.num_host_blocks; i > 0; i--) m->host_free.push_back((int32_t)(i - 1));
  *out = m;
  return ok();
}

int32_t fkv_seqs_destroy(fkv_seqs* m) {
  fkv::KeepLastError keep;
  if (!m) return ok();
  if (m->pool) {  // a destroyed pool has detached its managers: nothing to release
    for (auto& s : m->seqs)
      if (s.used && !s.swapped && !s.blocks.empty())
        (void)fkv_block_free(m->pool, (uint32_t)s.blocks.size(), s.blocks.data());
    auto& ms = m->pool->managers;
    ms.erase(std::remove(ms.begin(), ms.end(), m), ms.end());
  }
  delete m;
  return ok();
}

int32_t fkv_seqs_add(fkv_seqs* m, uint64_t n_tokens, uint32_t* seq_out) {
  if (!m || !seq_out) return fail(FKV_ERR_INVALID, "null argument");
  if (!m->pool) return fail(FKV_ERR_INVALID, "pool destroyed");
  const uint64_t nb = blocks_for(m->pool, n_tokens);
  if (nb > m->pool->free_list.size()) return fail(FKV_ERR_UNAVAILABLE, "no free kv blocks");
  std::vector<int32_t> ids(nb);
  if (nb) {
    int32_t st = fkv_block_alloc(m->pool, (uint32_t)nb, ids.data());
    if (st) return st;
  }
  uint32_t id;
  if (!m->free_ids.empty()) {
    id = m->free_ids.back();
    m->free_ids.pop_back();
  } else {
    id = (uint32_t)m->seqs.size();
    m->seqs.emplace_back();
  }
  fkv_seqs::Seq& s = m->seqs[id];
  s = fkv_seqs::Seq();
  s.used = true;
  s.blocks = std::move(ids);
  *seq_out = id;
  return ok();
}

int32_t fkv_seqs_reserve(fkv_seqs* m, uint32_t seq, uint64_t n, int64_t* copy_pair) {
  if (!m || !copy_pair) return fail(FKV_ERR_INVALID, "null argument");
  fkv_seqs::Seq* s = seq_at(m, seq);
  if (!s) return fail(FKV_ERR_CACHE, "unknown sequence");
  if (s->swapped) return fail(FKV_ERR_CACHE, "sequence is swapped out");
  copy_pair[0] = copy_pair[1] = -1;
  fkv_pool* p = m->pool;
  const uint64_t B = p->cfg.block_size, have = s->blocks.size();
  const uint64_t need = blocks_for(p, s->len + n);
  // Only the block holding position len can be shared and partly written (a fork
  // shares the blocks of the committed tokens): it is copied before the write.
  const uint64_t first = s->len / B;
  const bool cow = n > 0 && s->len % B != 0 && first < have &&
                   p->refcount[(size_t)s->blocks[first]] > 1;
  const uint64_t extra = (need > have ? need - have : 0) + (cow ? 1 : 0);
  if (extra > p->free_list.size()) return fail(FKV_ERR_UNAVAILABLE, "no free kv blocks");
  std::vector<int32_t> ids(extra);
  if (extra) {
    int32_t st = fkv_block_alloc(p, (uint32_t)extra, ids.data());
    if (st) return st;
  }
  size_t k = 0;
  if (cow) {
    const int32_t src = s->blocks[first];
    s->blocks[first] = ids[k++];
    copy_pair[0] = src;
    copy_pair[1] = s->blocks[first];
    int32_t st = fkv_block_free(p, 1, &src);  // this sequence's reference to the shared block
    if (st) return st;
  }
  for (; k < ids.size(); k++) s->blocks.push_back(ids[k]);
  return ok();
}

int32_t fkv_seqs_commit(fkv_seqs* m, uint32_t seq, uint64_t n) {
  if (!m) return fail(FKV_ERR_INVALID, "null argument");
  fkv_seqs::Seq* s = seq_at(m, seq);
  if (!s) return fail(FKV_ERR_CACHE, "unknown sequence");
  if (s->swapped) return fail(FKV_ERR_CACHE, "sequence is swapped out");
  if (s->len + n > (uint64_t)s->blocks.size() * m->pool->cfg.block_size)
    return fail(FKV_ERR_CACHE, "commit past the reserved blocks");
  s->len += n;
  return ok();
}

int32_t fkv_seqs_slots(const fkv_seqs* m, uint32_t seq, uint64_t pos, uint64_t n,
                       int64_t* slots_out) {
  if (!m || (n && !slots_out)) return fail(FKV_ERR_INVALID, "null argument");
  const fkv_seqs::Seq* s = seq_at(m, seq);
  if (!s) return fail(FKV_ERR_CACHE, "unknown sequence");
  if (s->swapped) return fail(FKV_ERR_CACHE, "sequence is swapped out");
  const uint64_t B = m->pool->cfg.block_size;
  if (pos + n > (uint64_t)s->blocks.size() * B)
    return fail(FKV_ERR_CACHE, "position beyond the reserved blocks");
  for (uint64_t i = 0; i < n; i++) {
    const uint64_t q = pos + i;
    slots_out[i] = (int64_t)s->blocks[q / B] * (int64_t)B + (int64_t)(q % B);
  }
  return ok();
}

int32_t fkv_seqs_truncate(fkv_seqs* m, uint32_t seq, uint64_t n_tokens) {
  if (!m) return fail(FKV_ERR_INVALID, "null argument");
  fkv_seqs::Seq* s = seq_at(m, seq);
  if (!s) return fail(FKV_ERR_CACHE, "unknown sequence");
  if (s->swapped) return fail(FKV_ERR_CACHE, "sequence is swapped out");
  if (n_tokens > s->len) return fail(FKV_ERR_CACHE, "truncate past the sequence length");
  const uint64_t keep = blocks_for(m->pool, n_tokens);
  if (keep < s->blocks.size()) {
    int32_t st = fkv_block_free(m->pool, (uint32_t)(s->blocks.size() - keep), s->blocks.data() + keep);
    if (st) return st;
    s->blocks.resize(keep);
  }
  s->len = n_tokens;
  return ok();
}

int32_t fkv_seqs_fork(fkv_seqs* m, uint32_t parent, uint32_t* child_out) {
  if (!m || !child_out) return fail(FKV_ERR_INVALID, "null argument");
  fkv_seqs::Seq* s = seq_at(m, parent);
  if (!s) return fail(FKV_ERR_CACHE, "unknown sequence");
  if (s->swapped) return fail(FKV_ERR_CACHE, "sequence is swapped out");
  const uint64_t nb = blocks_for(m->pool, s->len);
  std::vector<int32_t> shared(s->blocks.begin(), s->blocks.begin() + (ptrdiff_t)nb);
  if (nb) {
    int32_t st = fkv_block_ref(m->pool, (uint32_t)nb, shared.data());
    if (st) return st;
  }
  const uint64_t len = s->len;  // s may move when seqs grows
  uint32_t id;
  if (!m->free_ids.empty()) {
    id = m->free_ids.back();
    m->free_ids.pop_back();
  } else {
    id = (uint32_t)m->seqs.size();
    m->seqs.emplace_back();
  }
  fkv_seqs::Seq& c = m->seqs[id];
  c = fkv_seqs::Seq();
  c.used = true;
  c.len = len;
  c.blocks = std::move(shared);
  *child_out = id;
  return ok();
}

int32_t fkv_seqs_free(fkv_seqs* m, uint32_t seq) {
  if (!m) return fail(FKV_ERR_INVALID, "null argument");
  fkv_seqs::Seq* s = seq_at(m, seq);
  if (!s) return fail(FKV_ERR_CACHE, "unknown sequence");
  if (s->swapped) {
    for (int32_t h : s->blocks) m->host_free.push_back(h);
  } else if (!s->blocks.empty()) {
    int32_t st = fkv_block_free(m->pool, (uint32_t)s->blocks.size(), s->blocks.data());
    if (st) return st;
  }
  *s = fkv_seqs::Seq();
  m->free_ids.push_back(seq);
  return ok();
}

int32_t fkv_seqs_len(const fkv_seqs* m, uint32_t seq, uint64_t* len_out, int32_t* swapped_out) {
  if (!m || !len_out) return fail(FKV_ERR_INVALID, "null argument");
  const fkv_seqs::Seq* s = seq_at(m, seq);
  if (!s) return fail(FKV_ERR_CACHE, "unknown sequence");
  *len_out = s->len;
  if (swapped_out) *swapped_out = s->swapped ? 1 : 0;
  return ok();
}

int32_t fkv_seqs_swap_out(fkv_seqs* m, uint32_t seq, void* stream) {
  if (!m) return fail(FKV_ERR_INVALID, "null argument");
  fkv_seqs::Seq* s = seq_at(m, seq);
  if (!s) return fail(FKV_ERR_CACHE, "unknown sequence");
  if (s->swapped) return fail(FKV_ERR_CACHE, "sequence is swapped out");
  const uint64_t nb = blocks_for(m->pool, s->len);
  if (nb > m->host_free.size()) return fail(FKV_ERR_UNAVAILABLE, "no free host blocks");
  std::vector<int64_t> pairs(2 * nb);
  std::vector<int32_t> host(nb);
  for (uint64_t i = 0; i < nb; i++) {
    host[i] = m->host_free[m->host_free.size() - 1 - i];
    pairs[2 * i] = s->blocks[i];
    pairs[2 * i + 1] = host[i];
  }
  if (nb) {
    int32_t st = fkv_swap_out(m->pool, pairs.data(), (uint32_t)nb, stream);
    if (st) return st;
  }
  m->host_free.resize(m->host_free.size() - nb);
  if (!s->blocks.empty()) {
    int32_t st = fkv_block_free(m->pool, (uint32_t)s->blocks.size(), s->blocks.data());
    if (st) return st;
  }
  s->blocks = std::move(host);
  s->swapped = true;
  return ok();
}

int32_t fkv_seqs_swap_in(fkv_seqs* m, uint32_t seq, void* stream) {
  if (!m) return fail(FKV_ERR_INVALID, "null argument");
  fkv_seqs::Seq* s = seq_at(m, seq);
  if (!s) return fail(FKV_ERR_CACHE, "unknown sequence");
  if (!s->swapped) return fail(FKV_ERR_CACHE, "sequence is not swapped out");
  const uint64_t nb = s->blocks.size();
  if (nb > m->pool->free_list.size()) return fail(FKV_ERR_UNAVAILABLE, "no free kv blocks");
  std::vector<int32_t> dev(nb);
  if (nb) {
    int32_t st = fkv_block_alloc(m->pool, (uint32_t)nb, dev.data());
    if (st) return st;
  }
  std::vector<int64_t> pairs(2 * nb);
  for (uint64_t i = 0; i < nb; i++) {
    pairs[2 * i] = s->blocks[i];
    pairs[2 * i + 1] = dev[i];
  }
  if (nb) {
    int32_t st = fkv_swap_in(m->pool, pairs.data(), (uint32_t)nb, stream);
    if (st) {
      (void)fkv_block_free(m->pool, (uint32_t)nb, dev.data());
      return st;
    }
  }
  for (int32_t h : s->blocks) m->host_free.push_back(h);
  s->blocks = std::move(dev);
  s->swapped = false;
  return ok();
}

int32_t fkv_seqs_tables(const fkv_seqs* m, const uint32_t* seqs, uint32_t n, uint32_t max_blocks,
                        int32_t* tables_out, int32_t* ctx_out) {
  if (!m || (n && (!seqs || !tables_out || !ctx_out))) return fail(FKV_ERR_INVALID, "null argument");
  for (uint32_t i = 0; i < n; i++) {
    const fkv_seqs::Seq* s = seq_at(m, seqs[i]);
    if (!s) return fail(FKV_ERR_CACHE, "unknown sequence");
    if (s->swapped) return fail(FKV_ERR_CACHE, "sequence is swapped out");
    if (s->blocks.size() > max_blocks) return fail(FKV_ERR_INVALID, "block table too narrow");
    if (s->len > 0x7fffffffull) return fail(FKV_ERR_INVALID, "sequence too long");
  }
  for (uint32_t i = 0; i < n; i++) {
    const fkv_seqs::Seq& s = m->seqs[seqs[i]];
    int32_t* row = tables_out + (uint64_t)i * max_blocks;
    std::copy(s.blocks.begin(), s.blocks.end(), row);
    std::fill(row + s.blocks.size(), row + max_blocks, 0);
    ctx_out[i] = (int32_t)s.len;
  }
  return ok();
}

// ---------------------------------------------------------------------------
// Q8_0 weight GEMV/GEMM (Kernels::gemv / Kernels::gemm for DType::Q8_0)
// ---------------------------------------------------------------------------

// check_matrix then the x/y lengths (crates/kernels/src/validate.rs:110-150), in
// that order and with those strings; then what the device boundary adds.
static int32_t check_gemm_q8(const void* w, uint64_t w_len, uint64_t rows, uint64_t cols,
                             const float* x, uint64_t x_len, uint64_t n_tokens, float* y,
                             uint64_t y_len) {
  if (cols == 0) return fail(FKV_ERR_KERNEL, "empty dot");
  if (cols % 32 != 0) return fail(FKV_ERR_KERNEL, "q8_0 k is not a multiple of 32");
  uint64_t row_bytes, w_bytes, xn, yn;
  if (mul_ovf(cols / 32, 34, &row_bytes) || mul_ovf(rows, row_bytes, &w_bytes))
    return fail(FKV_ERR_KERNEL, "shape overflow");
  if (w_len != w_bytes) return fail(FKV_ERR_KERNEL, "length mismatch");
  if (mul_ovf(n_tokens, cols, &xn) || mul_ovf(n_tokens, rows, &yn))
    return fail(FKV_ERR_KERNEL, "shape overflow");
  if (x_len != xn || y_len != yn) return fail(FKV_ERR_KERNEL, "length mismatch");
  if (rows == 0) return FKV_OK;
  if (!w || !x || !y) return fail(FKV_ERR_INVALID, "null argument");
  if ((uintptr_t)w % 2 != 0) return fail(FKV_ERR_INVALID, "w must be 2-byte aligned");
  if ((uintptr_t)x % 4 != 0 || (uintptr_t)y % 4 != 0)
    return fail(FKV_ERR_INVALID, "x and y must be 4-byte aligned");
  if (rows > 0x7fff0000ull || n_tokens > 0x7fff0000ull || cols > 0xffffffffull ||
      fkv::gemv_lds_bytes(1, (uint32_t)cols) > fkv::kGemvMaxLds)
    return fail(FKV_ERR_INVALID, "matrix too large for one launch");
  return FKV_OK;
}

static int32_t gemm_q8(const void* w, uint64_t w_len, uint64_t rows, uint64_t cols,
                       const float* x, uint64_t x_len, uint64_t n_tokens, float* y,
                       uint64_t y_len, void* stream) {
  int32_t st = check_gemm_q8(w, w_len, rows, cols, x, x_len, n_tokens, y, y_len);
  if (st) return st;
  if (rows == 0) return ok();
  fkv::GemvBatch b{};
  b.n = 1;
  b.m[0].w = (const uint8_t*)w;
  b.m[0].y = y;
  b.m[0].rows = (uint32_t)rows;
  FKV_HIP(fkv::launch_gemv_q8(b, (uint32_t)cols, x, (uint32_t)n_tokens, (hipStream_t)stream),
          "gemv launch");
  return ok();
}

int32_t fkv_gemv_q8_0(const void* w, uint64_t w_len, uint64_t rows, uint64_t cols,
                      const float* x, uint64_t x_len, float* y, uint64_t y_len, void* stream) {
  return gemm_q8(w, w_len, rows, cols, x, x_len, 1, y, y_len, stream);
}

int32_t fkv_gemm_q8_0(const void* w, uint64_t w_len, uint64_t rows, uint64_t cols,
                      const float* x, uint64_t x_len, uint64_t n_tokens, float* y,
                      uint64_t y_len, void* stream) {
  if (n_tokens == 0) return ok();
  return gemm_q8(w, w_len, rows, cols, x, x_len, n_tokens, y, y_len, stream);
}

// The multi-matrix checks (fkv_gemm_q8_0_multi) into b; FKV_OK with b.n == 0 when
// nothing is to be launched.
static int32_t gemm_q8_batch(uint32_t n_mats, const void* const* w, const uint64_t* w_len,
                             const uint64_t* rows, uint64_t cols, const float* x, uint64_t x_len,
                             uint64_t n_tokens, float* const* y, const uint64_t* y_len,
                             fkv::GemvBatch* b) {
  *b = fkv::GemvBatch{};
  if (n_mats == 0 || n_mats > (uint32_t)fkv::kGemvMaxMats)
    return fail(FKV_ERR_INVALID, "n_mats must be 1..4");
  if (!w || !w_len || !rows || !y || !y_len) return fail(FKV_ERR_INVALID, "null argument");
  if (n_tokens == 0) return FKV_OK;
  for (uint32_t m = 0; m < n_mats; ++m) {
    int32_t st = check_gemm_q8(w[m], w_len[m], rows[m], cols, x, x_len, n_tokens, y[m], y_len[m]);
    if (st) return st;
    if (rows[m] == 0) continue;
    b->m[b->n].w = (const uint8_t*)w[m];
    b->m[b->n].y = y[m];
    b->m[b->n].rows = (uint32_t)rows[m];
    b->n++;
  }
  return FKV_OK;
}

int32_t fkv_gemm_q8_0_multi(uint32_t n_mats, const void* const* w, const uint64_t* w_len,
                            const uint64_t* rows, uint64_t cols, const float* x,
                            uint64_t x_len, uint64_t n_tokens, float* const* y,
                            const uint64_t* y_len, void* stream) {
  fkv::GemvBatch b;
  int32_t st = gemm_q8_batch(n_mats, w, w_len, rows, cols, x, x_len, n_tokens, y, y_len, &b);
  if (st) return st;
  if (b.n == 0) return ok();
  FKV_HIP(fkv::launch_gemv_q8(b, (uint32_t)cols, x, (uint32_t)n_tokens, (hipStream_t)stream),
          "gemv launch");
  return ok();
}

int32_t fkv_gemm_q8_0_batched_workspace_size(uint64_t cols, uint64_t n_tokens,
                                             uint64_t* bytes_out) {
  if (!bytes_out) return fail(FKV_ERR_INVALID, "null argument");
  *bytes_out = 0;
  if (cols == 0 || cols % 1024 != 0 || cols > 0xffffffffull || n_tokens > 0x7fff0000ull ||
      n_tokens < fkv::kGemmMfmaMinTokens)
    return ok();  // such calls run the GEMV and need no workspace
  *bytes_out = fkv::gemm_mfma_workspace_bytes((uint32_t)cols, (uint32_t)n_tokens);
  return ok();
}

int32_t fkv_gemm_q8_0_batched(uint32_t n_mats, const void* const* w, const uint64_t* w_len,
                              const uint64_t* rows, uint64_t cols, const float* x,
                              uint64_t x_len, uint64_t n_tokens, float* const* y,
                              const uint64_t* y_len, void* workspace, uint64_t workspace_bytes,
                              void* stream) {
  fkv::GemvBatch b;
  int32_t st = gemm_q8_batch(n_mats, w, w_len, rows, cols, x, x_len, n_tokens, y, y_len, &b);
  if (st) return st;
  if (b.n == 0) return ok();
  if (!fkv::gemm_mfma_eligible(b, (uint32_t)cols, (uint32_t)n_tokens)) {
    FKV_HIP(fkv::launch_gemv_q8(b, (uint32_t)cols, x, (uint32_t)n_tokens, (hipStream_t)stream),
            "gemv launch");
    return ok();
  }
  const uint64_t need = fkv::gemm_mfma_workspace_bytes((uint32_t)cols, (uint32_t)n_tokens);
  if (!workspace || workspace_bytes < need) return fail(FKV_ERR_INVALID, "gemm workspace too small");
  if ((uintptr_t)workspace % 16 != 0)
    return fail(FKV_ERR_INVALID, "gemm workspace must be 16-byte aligned");
  FKV_HIP(fkv::launch_gemm_q8_mfma(b, (uint32_t)cols, x, (uint32_t)n_tokens, workspace,
                                   (hipStream_t)stream),
          "gemm launch");
  return ok();
}

}  // extern "C"
