// HIP kernels of the paged KV-cache hot path, written for gfx950 (CDNA4,
// wave64). Host-side validation lives in fkv_api.cpp; every launcher here
// assumes the shapes it is given were checked there.
//
// Reference semantics these kernels implement on the GPU:
//   append        KvPool::append_layer      crates/kvcache/src/pool.rs:122-153
//   gather        KvPool::k / KvPool::v     crates/kvcache/src/pool.rs:174-204
//   f16 decode    f16_to_f32                crates/core-types/src/dtype.rs:135-154
//   Q8_0 encode   Q8Activation::quantize_into crates/kernels/src/q8_dot.rs:46-59
//   attention     forward_one_token loop    crates/model/src/llama.rs:220-247
//   softmax       scalar softmax            crates/kernels/src/scalar.rs:125-141
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "fkv_internal.h"

namespace fkv {
namespace {

constexpr float kLog2e = 1.4426950408889634f;

__device__ __forceinline__ uint8_t* tile_ptr(const Geom& g, uint64_t block, uint32_t layer,
                                             uint32_t kv, uint32_t head) {
  return g.base + block * g.block_bytes +
         ((uint64_t)(layer * 2u + kv) * g.n_kv_heads + head) * g.tile_bytes;
}

__device__ __forceinline__ void raise_fault(uint32_t* f, uint32_t bit) {
  atomicOr(f, bit);
}

// ---------------------------------------------------------------------------
// binary16 <-> binary32
// ---------------------------------------------------------------------------

__device__ __forceinline__ float f16_bits_to_f32(uint32_t h) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)h);
}

// f32 -> binary16 bits. rounding 0: v_cvt_f16_f32 (IEEE roundTiesToEven).
// rounding 1: ties away from zero, as Ferrum's f32_to_f16_bits
// (crates/kernels/src/q8_dot.rs:111-139): the round-toward-zero neighbour from
// v_cvt_pkrtz_f16_f32 and the next binary16 up are compared by distance; both
// differences are exact near a tie (Sterbenz), which is where the choice matters.
// NaN keeps its top 10 payload bits and stays a NaN (q8_dot.rs:118-121).
__device__ __forceinline__ uint32_t encode_f16(float x, int rounding) {
  uint32_t u = __float_as_uint(x);
  uint32_t sign = (u >> 16) & 0x8000u;
  uint32_t ax = u & 0x7fffffffu;
  if (ax > 0x7f800000u) {
    uint32_t hf = (ax & 0x7fffffu) >> 13;
    return sign | 0x7c00u | hf | (hf == 0u ? 1u : 0u);
  }
  if (rounding == 0) {
    _Float16 h = (_Float16)x;
    return (uint32_t)__builtin_bit_cast(uint16_t, h);
  }
  if (ax == 0x7f800000u) return sign | 0x7c00u;
  float a = __uint_as_float(ax);
  auto pk = __builtin_amdgcn_cvt_pkrtz(a, 0.0f);
  uint32_t lo = __builtin_bit_cast(uint32_t, pk) & 0xffffu;
  float lo_v = f16_bits_to_f32(lo);
  float hi_v = (lo == 0x7bffu) ? 65536.0f : f16_bits_to_f32(lo + 1u);
  uint32_t r = (hi_v - a <= a - lo_v) ? lo + 1u : lo;
  return sign | r;
}

// ---------------------------------------------------------------------------
// Q8_0 block quantiser (q8_dot.rs:46-59)
// ---------------------------------------------------------------------------

__device__ __forceinline__ float round_half_away(float y) {
  float t = __builtin_truncf(y);
  return (__builtin_fabsf(y - t) >= 0.5f) ? t + __builtin_copysignf(1.0f, y) : t;
}

// x[32] -> 32 int8 packed in q[8] (little-endian bytes) and the f16 scale bits.
__device__ __forceinline__ uint32_t q8_quantize(const float (&x)[32], int rounding,
                                                uint32_t (&q)[8]) {
  float amax = 0.0f;
#pragma unroll
  for (int j = 0; j < 32; j++) amax = __builtin_fmaxf(amax, __builtin_fabsf(x[j]));
  float d = amax / 127.0f;
  float id = (d != 0.0f) ? 1.0f / d : 0.0f;
#pragma unroll
  for (int w = 0; w < 8; w++) {
    uint32_t packed = 0;
#pragma unroll
    for (int b = 0; b < 4; b++) {
      float r = round_half_away(x[w * 4 + b] * id);
      // Rust `as i32` saturates and maps NaN to 0; then clamp to [-128, 127].
      int qi = (r != r) ? 0 : (r >= 127.0f ? 127 : (r <= -128.0f ? -128 : (int)r));
      packed |= ((uint32_t)qi & 0xffu) << (8 * b);
    }
    q[w] = packed;
  }
  return encode_f16(d, rounding);
}

// ---------------------------------------------------------------------------
// Append (paged KvPool::append_layer)
// ---------------------------------------------------------------------------

// F32/F16 storage, head_dim % 8 == 0, 16-byte aligned k/v: one thread moves 8
// values of one (token, kv, head) row (32 B f32 in, 16 B f16 or 32 B f32 out).
template <int DT>
__global__ void __launch_bounds__(256) append_vec8_kernel(Geom g, uint32_t layer,
                                                          const float* __restrict__ k,
                                                          const float* __restrict__ v,
                                                          const int64_t* __restrict__ slots,
                                                          uint32_t n_tokens) {
  const uint32_t cpr = g.head_dim / 8;
  const uint32_t cph = g.n_kv_heads * cpr;
  const uint64_t total = (uint64_t)n_tokens * 2u * cph;
  const uint64_t cap = g.num_blocks * g.block_size;
  for (uint64_t u = (uint64_t)blockIdx.x * 256u + threadIdx.x; u < total;
       u += (uint64_t)gridDim.x * 256u) {
    uint32_t token = (uint32_t)(u / (2u * cph));
    uint32_t rem = (uint32_t)(u % (2u * cph));
    uint32_t kv = rem / cph, r2 = rem % cph, h = r2 / cpr, c = r2 % cpr;
    int64_t slot = slots[token];
    if (slot < 0) continue;
    if ((uint64_t)slot >= cap) {
      if (rem == 0) raise_fault(g.fault, kFaultSlot);
      continue;
    }
    const float* src = (kv ? v : k) + ((uint64_t)token * g.n_kv_heads + h) * g.head_dim + c * 8u;
    float4 a = *(const float4*)src;
    float4 b = *(const float4*)(src + 4);
    uint64_t blk = (uint64_t)slot / g.block_size;
    uint32_t off = (uint32_t)((uint64_t)slot % g.block_size);
    uint8_t* tile = tile_ptr(g, blk, layer, kv, h);
    if constexpr (DT == kDtypeF16) {
      uint4 o;
      o.x = encode_f16(a.x, g.rounding) | (encode_f16(a.y, g.rounding) << 16);
      o.y = encode_f16(a.z, g.rounding) | (encode_f16(a.w, g.rounding) << 16);
      o.z = encode_f16(b.x, g.rounding) | (encode_f16(b.y, g.rounding) << 16);
      o.w = encode_f16(b.z, g.rounding) | (encode_f16(b.w, g.rounding) << 16);
      *(uint4*)(tile + ((uint64_t)off * g.head_dim + c * 8u) * 2u) = o;
    } else {
      float4* dst = (float4*)(tile + ((uint64_t)off * g.head_dim + c * 8u) * 4u);
      dst[0] = a;
      dst[1] = b;
    }
  }
}

// Any head_dim, F32/F16 storage: one element per thread.
__global__ void __launch_bounds__(256) append_scalar_kernel(Geom g, uint32_t layer,
                                                            const float* __restrict__ k,
                                                            const float* __restrict__ v,
                                                            const int64_t* __restrict__ slots,
                                                            uint32_t n_tokens) {
  const uint32_t D = g.head_dim;
  const uint32_t per_kv = g.n_kv_heads * D;
  const uint64_t total = (uint64_t)n_tokens * 2u * per_kv;
  const uint64_t cap = g.num_blocks * g.block_size;
  for (uint64_t u = (uint64_t)blockIdx.x * 256u + threadIdx.x; u < total;
       u += (uint64_t)gridDim.x * 256u) {
    uint32_t token = (uint32_t)(u / (2u * per_kv));
    uint32_t rem = (uint32_t)(u % (2u * per_kv));
    uint32_t kv = rem / per_kv, e = rem % per_kv, h = e / D, d = e % D;
    int64_t slot = slots[token];
    if (slot < 0) continue;
    if ((uint64_t)slot >= cap) {
      if (rem == 0) raise_fault(g.fault, kFaultSlot);
      continue;
    }
    float x = (kv ? v : k)[(uint64_t)token * per_kv + e];
    uint8_t* tile = tile_ptr(g, (uint64_t)slot / g.block_size, layer, kv, h);
    uint64_t idx = ((uint64_t)slot % g.block_size) * D + d;
    if (g.dtype == kDtypeF16)
      ((uint16_t*)tile)[idx] = (uint16_t)encode_f16(x, g.rounding);
    else
      ((float*)tile)[idx] = x;
  }
}

// Q8_0 storage: one thread quantises one 32-value run of a (token, kv, head) row.
template <bool kAligned>
__global__ void __launch_bounds__(256) append_q8_kernel(Geom g, uint32_t layer,
                                                        const float* __restrict__ k,
                                                        const float* __restrict__ v,
                                                        const int64_t* __restrict__ slots,
                                                        uint32_t n_tokens) {
  const uint32_t D = g.head_dim, B = g.block_size;
  const uint32_t cpr = D / 32;
  const uint32_t cph = g.n_kv_heads * cpr;
  const uint64_t total = (uint64_t)n_tokens * 2u * cph;
  const uint64_t cap = g.num_blocks * B;
  for (uint64_t u = (uint64_t)blockIdx.x * 256u + threadIdx.x; u < total;
       u += (uint64_t)gridDim.x * 256u) {
    uint32_t token = (uint32_t)(u / (2u * cph));
    uint32_t rem = (uint32_t)(u % (2u * cph));
    uint32_t kv = rem / cph, r2 = rem % cph, h = r2 / cpr, c = r2 % cpr;
    int64_t slot = slots[token];
    if (slot < 0) continue;
    if ((uint64_t)slot >= cap) {
      if (rem == 0) raise_fault(g.fault, kFaultSlot);
      continue;
    }
    const float* src = (kv ? v : k) + ((uint64_t)token * g.n_kv_heads + h) * D + c * 32u;
    float x[32];
    if constexpr (kAligned) {
#pragma unroll
      for (int j = 0; j < 8; j++) {
        float4 t = ((const float4*)src)[j];
        x[4 * j] = t.x; x[4 * j + 1] = t.y; x[4 * j + 2] = t.z; x[4 * j + 3] = t.w;
      }
    } else {
#pragma unroll
      for (int j = 0; j < 32; j++) x[j] = src[j];
    }
    uint32_t q[8];
    uint32_t sc = q8_quantize(x, g.rounding, q);
    uint32_t off = (uint32_t)((uint64_t)slot % B);
    uint8_t* tile = tile_ptr(g, (uint64_t)slot / B, layer, kv, h);
    uint4* qdst = (uint4*)(tile + (uint64_t)off * D + c * 32u);
    qdst[0] = make_uint4(q[0], q[1], q[2], q[3]);
    qdst[1] = make_uint4(q[4], q[5], q[6], q[7]);
    ((uint16_t*)(tile + (uint64_t)B * D))[off * cpr + c] = (uint16_t)sc;
  }
}

// ---------------------------------------------------------------------------
// Gather (paged KvPool::k / v): one unit = one (row, kv, head, chunk)
// ---------------------------------------------------------------------------

// Copies/decodes chunk c of the (blk, off, kv, h) row into `dst_row` (the
// output row of head h). Chunk = 8 values (F32/F16) or 32 values (Q8_0).
__device__ __forceinline__ void gather_chunk(const Geom& g, uint32_t layer, uint64_t blk,
                                             uint32_t off, uint32_t kv, uint32_t h,
                                             uint32_t c, int format, uint8_t* dst_row,
                                             bool aligned) {
  const uint32_t D = g.head_dim;
  const uint8_t* tile = tile_ptr(g, blk, layer, kv, h);
  if (g.dtype == kDtypeQ8) {
    const uint8_t* qs = tile + (uint64_t)off * D + c * 32u;
    uint32_t sc = ((const uint16_t*)(tile + (uint64_t)g.block_size * D))[off * (D / 32u) + c];
    if (format == 0) {
      float s = f16_bits_to_f32(sc);
      float* o = (float*)dst_row + c * 32u;
      for (int j = 0; j < 32; j++) o[j] = s * (float)(int8_t)qs[j];
    } else {
      // Ferrum's 34-byte Q8_0 block: f16 scale (LE) then 32 x i8 (dtype.rs:19-21).
      uint16_t* o = (uint16_t*)(dst_row + (uint64_t)c * 34u);
      o[0] = (uint16_t)sc;
      for (int j = 0; j < 16; j++) o[1 + j] = (uint16_t)(qs[2 * j] | (qs[2 * j + 1] << 8));
    }
    return;
  }
  if (g.dtype == kDtypeF16) {
    const uint16_t* src = (const uint16_t*)tile + (uint64_t)off * D + c * 8u;
    if (format == 0) {
      float* o = (float*)dst_row + c * 8u;
      if (aligned) {
        uint4 w = *(const uint4*)src;
        ((float4*)o)[0] = make_float4(f16_bits_to_f32(w.x & 0xffffu), f16_bits_to_f32(w.x >> 16),
                                      f16_bits_to_f32(w.y & 0xffffu), f16_bits_to_f32(w.y >> 16));
        ((float4*)o)[1] = make_float4(f16_bits_to_f32(w.z & 0xffffu), f16_bits_to_f32(w.z >> 16),
                                      f16_bits_to_f32(w.w & 0xffffu), f16_bits_to_f32(w.w >> 16));
      } else {
        for (int j = 0; j < 8; j++) o[j] = f16_bits_to_f32(src[j]);
      }
    } else {
      uint16_t* o = (uint16_t*)dst_row + c * 8u;
      if (aligned) *(uint4*)o = *(const uint4*)src;
      else for (int j = 0; j < 8; j++) o[j] = src[j];
    }
    return;
  }
  const float* src = (const float*)tile + (uint64_t)off * D + c * 8u;
  float* o = (float*)dst_row + c * 8u;
  if (aligned) {
    ((float4*)o)[0] = ((const float4*)src)[0];
    ((float4*)o)[1] = ((const float4*)src)[1];
  } else {
    for (int j = 0; j < 8; j++) o[j] = src[j];
  }
}

// Output bytes per head row in `format`.
__device__ __forceinline__ uint64_t out_head_bytes(const Geom& g, int format) {
  if (format == 0) return (uint64_t)g.head_dim * 4u;
  if (g.dtype == kDtypeF32) return (uint64_t)g.head_dim * 4u;
  if (g.dtype == kDtypeF16) return (uint64_t)g.head_dim * 2u;
  return (uint64_t)g.head_dim / 32u * 34u;
}

__device__ __forceinline__ uint32_t chunk_values(const Geom& g) {
  return g.dtype == kDtypeQ8 ? 32u : 8u;
}

__global__ void __launch_bounds__(256) gather_slots_kernel(Geom g, uint32_t layer,
                                                           const int64_t* __restrict__ slots,
                                                           uint32_t n_tokens, int format,
                                                           uint8_t* out_k, uint8_t* out_v,
                                                           bool aligned) {
  const uint32_t cpr = g.head_dim / chunk_values(g);
  const uint32_t cph = g.n_kv_heads * cpr;
  const uint64_t total = (uint64_t)n_tokens * 2u * cph;
  const uint64_t cap = g.num_blocks * g.block_size;
  const uint64_t hb = out_head_bytes(g, format);
  for (uint64_t u = (uint64_t)blockIdx.x * 256u + threadIdx.x; u < total;
       u += (uint64_t)gridDim.x * 256u) {
    uint32_t token = (uint32_t)(u / (2u * cph));
    uint32_t rem = (uint32_t)(u % (2u * cph));
    uint32_t kv = rem / cph, r2 = rem % cph, h = r2 / cpr, c = r2 % cpr;
    int64_t slot = slots[token];
    if (slot < 0) continue;
    if ((uint64_t)slot >= cap) {
      if (rem == 0) raise_fault(g.fault, kFaultSlot);
      continue;
    }
    uint8_t* row = (kv ? out_v : out_k) + ((uint64_t)token * g.n_kv_heads + h) * hb;
    gather_chunk(g, layer, (uint64_t)slot / g.block_size,
                 (uint32_t)((uint64_t)slot % g.block_size), kv, h, c, format, row, aligned);
  }
}

// Gather whole sequences through their block tables; blockIdx.y = sequence.
__global__ void __launch_bounds__(256) gather_tables_kernel(
    Geom g, uint32_t layer, const int32_t* __restrict__ tables, uint32_t max_blocks,
    const int32_t* __restrict__ ctx_lens, const int64_t* __restrict__ out_offsets, int format,
    uint8_t* out_k, uint8_t* out_v, bool aligned) {
  const uint32_t seq = blockIdx.y;
  const uint32_t cpr = g.head_dim / chunk_values(g);
  const uint32_t cph = g.n_kv_heads * cpr;
  int32_t ctx = ctx_lens[seq];
  const int32_t cap = (int32_t)(max_blocks * g.block_size);
  if (ctx < 0 || ctx > cap) {
    if (blockIdx.x == 0 && threadIdx.x == 0) raise_fault(g.fault, kFaultCtx);
    ctx = ctx < 0 ? 0 : cap;
  }
  const uint64_t total = (uint64_t)ctx * 2u * cph;
  const uint64_t hb = out_head_bytes(g, format);
  const int64_t base_row = out_offsets[seq];
  for (uint64_t u = (uint64_t)blockIdx.x * 256u + threadIdx.x; u < total;
       u += (uint64_t)gridDim.x * 256u) {
    uint32_t pos = (uint32_t)(u / (2u * cph));
    uint32_t rem = (uint32_t)(u % (2u * cph));
    uint32_t kv = rem / cph, r2 = rem % cph, h = r2 / cpr, c = r2 % cpr;
    int32_t blk = tables[(uint64_t)seq * max_blocks + pos / g.block_size];
    if (blk < 0 || (uint64_t)blk >= g.num_blocks) {
      if (rem == 0) raise_fault(g.fault, kFaultBlock);
      continue;
    }
    uint8_t* row = (kv ? out_v : out_k) + ((uint64_t)(base_row + pos) * g.n_kv_heads + h) * hb;
    gather_chunk(g, layer, (uint64_t)blk, pos % g.block_size, kv, h, c, format, row, aligned);
  }
}

// ---------------------------------------------------------------------------
// copy_blocks / fill / device copy
// ---------------------------------------------------------------------------

// Native clang vector (the nontemporal builtins do not take HIP's uint4 struct).
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

constexpr uint32_t kCopyUnroll = 4;
constexpr uint64_t kCopyChunkVecs = 256u * kCopyUnroll;  // 16 KiB per workgroup step

__global__ void __launch_bounds__(256) copy_blocks_kernel(Geom g, const int64_t* __restrict__ pairs,
                                                          uint32_t n_pairs) {
  const uint64_t vecs = g.block_bytes / 16u;
  const uint64_t cpb = (vecs + kCopyChunkVecs - 1) / kCopyChunkVecs;
  const uint64_t total = (uint64_t)n_pairs * cpb;
  for (uint64_t w = blockIdx.x; w < total; w += gridDim.x) {
    uint64_t pr = w / cpb, ch = w % cpb;
    int64_t src = pairs[2 * pr], dst = pairs[2 * pr + 1];
    if (src < 0 || dst < 0 || (uint64_t)src >= g.num_blocks || (uint64_t)dst >= g.num_blocks) {
      if (ch == 0 && threadIdx.x == 0) raise_fault(g.fault, kFaultBlock);
      continue;
    }
    const u32x4* s = (const u32x4*)(g.base + (uint64_t)src * g.block_bytes);
    u32x4* d = (u32x4*)(g.base + (uint64_t)dst * g.block_bytes);
    uint64_t i0 = ch * kCopyChunkVecs + threadIdx.x;
    u32x4 r[kCopyUnroll];
#pragma unroll
    for (uint32_t j = 0; j < kCopyUnroll; j++) {
      uint64_t i = i0 + j * 256u;
      if (i < vecs) r[j] = __builtin_nontemporal_load(s + i);
    }
#pragma unroll
    for (uint32_t j = 0; j < kCopyUnroll; j++) {
      uint64_t i = i0 + j * 256u;
      if (i < vecs) __builtin_nontemporal_store(r[j], d + i);
    }
  }
}

__global__ void __launch_bounds__(256) fill_kernel(uint8_t* dst, uint32_t word, uint64_t bytes) {
  const uint64_t vecs = bytes / 16u;
  uint4 w = make_uint4(word, word, word, word);
  for (uint64_t i = (uint64_t)blockIdx.x * 256u + threadIdx.x; i < vecs;
       i += (uint64_t)gridDim.x * 256u)
    ((uint4*)dst)[i] = w;
  uint64_t tail = vecs * 16u + (uint64_t)blockIdx.x * 256u + threadIdx.x;
  if (tail < bytes && blockIdx.x == 0) dst[tail] = (uint8_t)word;
}

__global__ void __launch_bounds__(256) device_copy_kernel(u32x4* __restrict__ dst,
                                                          const u32x4* __restrict__ src,
                                                          uint64_t vecs) {
  for (uint64_t i0 = (uint64_t)blockIdx.x * kCopyChunkVecs + threadIdx.x; i0 < vecs;
       i0 += (uint64_t)gridDim.x * kCopyChunkVecs) {
    u32x4 r[kCopyUnroll];
#pragma unroll
    for (uint32_t j = 0; j < kCopyUnroll; j++) {
      uint64_t i = i0 + j * 256u;
      if (i < vecs) r[j] = __builtin_nontemporal_load(src + i);
    }
#pragma unroll
    for (uint32_t j = 0; j < kCopyUnroll; j++) {
      uint64_t i = i0 + j * 256u;
      if (i < vecs) __builtin_nontemporal_store(r[j], dst + i);
    }
  }
}

__global__ void copy_tail_kernel(uint8_t* dst, const uint8_t* src, uint64_t from, uint64_t bytes) {
  uint64_t i = from + threadIdx.x;
  if (i < bytes) dst[i] = src[i];
}

// ---------------------------------------------------------------------------
// Wave reductions (DPP inside 16-lane rows, readlane across rows)
// ---------------------------------------------------------------------------

template <int kCtrl>
__device__ __forceinline__ float dpp(float x) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), kCtrl, 0xf, 0xf, true));
}

// Sum over aligned groups of N lanes (N <= 16), result in every lane of the group.
template <int N>
__device__ __forceinline__ float group_sum(float x) {
  if constexpr (N >= 2) x += dpp<0xB1>(x);   // quad_perm [1,0,3,2]
  if constexpr (N >= 4) x += dpp<0x4E>(x);   // quad_perm [2,3,0,1]
  if constexpr (N >= 8) x += dpp<0x141>(x);  // row_half_mirror
  if constexpr (N >= 16) x += dpp<0x140>(x); // row_mirror
  if constexpr (N >= 32) x += __shfl_xor(x, 16);
  return x;
}

__device__ __forceinline__ float wave_max(float x) {
  x = __builtin_fmaxf(x, dpp<0xB1>(x));
  x = __builtin_fmaxf(x, dpp<0x4E>(x));
  x = __builtin_fmaxf(x, dpp<0x141>(x));
  x = __builtin_fmaxf(x, dpp<0x140>(x));
  float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), 0));
  float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), 16));
  float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), 32));
  float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), 48));
  return __builtin_fmaxf(__builtin_fmaxf(r0, r1), __builtin_fmaxf(r2, r3));
}

__device__ __forceinline__ float wave_sum(float x) {
  x = group_sum<16>(x);
  float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), 0));
  float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), 16));
  float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), 32));
  float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), 48));
  return (r0 + r1) + (r2 + r3);
}

// ---------------------------------------------------------------------------
// Paged decode attention
// ---------------------------------------------------------------------------
//
// One workgroup (4 waves) = one 256-token partition of one (sequence, kv head);
// all G = n_heads/n_kv_heads query heads of the group share every K/V tile.
// Each wave owns 4 consecutive 16-token blocks. A 16-token K or V tile is read
// as rows: LPR lanes cover one token row with 16-byte loads, RPP rows per load
// instruction, PASSES instructions per tile, so each load instruction reads
// 1 KiB of consecutive HBM.
//   phase 1  scores s[g][t] = (q_g . K_t) * scale  -> LDS
//   phase 2  per head: max m, e_t = exp(s_t - m), l = sum e_t   (exact per partition)
//   phase 3  acc[g][d] = sum_t e[g][t] * V_t[d]; rows and waves reduced via LDS
// With one partition the output is acc / l; otherwise (m, l, acc) go to the
// workspace and attn_combine_kernel merges partitions (log-sum-exp).

template <int DT>
struct KvTraits;
template <>
struct KvTraits<kDtypeF16> { static constexpr int kBytes = 2; };
template <>
struct KvTraits<kDtypeF32> { static constexpr int kBytes = 4; };
template <>
struct KvTraits<kDtypeQ8> { static constexpr int kBytes = 1; };

template <int DT, int D>
struct AttnShape {
  static constexpr int E = KvTraits<DT>::kBytes;
  static constexpr int EPL = 16 / E;            // values per lane per 16-byte load
  static constexpr int LPR = D / EPL;           // lanes per token row
  static constexpr int RPP = 64 / LPR;          // token rows per load instruction
  static constexpr int PASSES = kAttnBlock / RPP;
  static constexpr bool kPrefetchV = PASSES <= 4;
  static_assert(LPR >= 1 && LPR <= 32 && RPP * LPR == 64 && PASSES * RPP == kAttnBlock, "shape");
};

// Decode one 16-byte load (EPL values) to f32.
template <int DT, int EPL>
__device__ __forceinline__ void decode16(const uint4& w, float (&f)[EPL]) {
  if constexpr (DT == kDtypeF16) {
    const uint32_t a[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int i = 0; i < 4; i++) {
      f[2 * i] = f16_bits_to_f32(a[i] & 0xffffu);
      f[2 * i + 1] = f16_bits_to_f32(a[i] >> 16);
    }
  } else if constexpr (DT == kDtypeF32) {
    f[0] = __uint_as_float(w.x); f[1] = __uint_as_float(w.y);
    f[2] = __uint_as_float(w.z); f[3] = __uint_as_float(w.w);
  } else {
    const uint32_t a[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int i = 0; i < 4; i++) {
#pragma unroll
      for (int b = 0; b < 4; b++) f[4 * i + b] = (float)(int8_t)((a[i] >> (8 * b)) & 0xffu);
    }
  }
}

template <int DT, int D, int G>
__global__ void __launch_bounds__(256) attn_partition_kernel(
    Geom g, uint32_t layer, uint32_t n_heads, const float* __restrict__ q,
    float* __restrict__ out, const int32_t* __restrict__ tables, uint32_t max_blocks,
    const int32_t* __restrict__ ctx_lens, uint32_t max_parts, float scale,
    float* __restrict__ ws_o, float* __restrict__ ws_ml) {
  using S = AttnShape<DT, D>;
  constexpr int EPL = S::EPL, LPR = S::LPR, RPP = S::RPP, PASSES = S::PASSES;
  constexpr int NB = kAttnBlocksPerWave;

  // s_acc (phase 3 output) reuses the bytes of s_score, which is dead after phase 2.
  constexpr int kScoreFloats = G * kAttnPartTokens;
  constexpr int kAccFloats = kAttnWaves * G * D;
  __shared__ float s_union[kScoreFloats > kAccFloats ? kScoreFloats : kAccFloats];
  __shared__ float s_p[kAttnPartTokens][G];
  __shared__ float s_m[G];
  __shared__ float s_l[G];
  float (*s_score)[kAttnPartTokens] = reinterpret_cast<float (*)[kAttnPartTokens]>(s_union);
  float (*s_acc)[G][D] = reinterpret_cast<float (*)[G][D]>(s_union);

  const uint32_t sk = blockIdx.x;
  const uint32_t part = blockIdx.y;
  const uint32_t seq = sk / g.n_kv_heads, kvh = sk % g.n_kv_heads;
  const int32_t cap = (int32_t)(max_blocks * kAttnBlock);
  int32_t ctx = ctx_lens[seq];
  if (ctx < 0 || ctx > cap) {
    if (part == 0 && threadIdx.x == 0 && kvh == 0) raise_fault(g.fault, kFaultCtx);
    ctx = ctx < 0 ? 0 : cap;
  }
  const int32_t nparts = ctx > 0 ? (ctx + kAttnPartTokens - 1) / kAttnPartTokens : 1;
  if ((int32_t)part >= nparts) return;

  const int wave = threadIdx.x / 64, lane = threadIdx.x % 64;
  const int r = lane / LPR, c = lane % LPR;
  const int32_t part_start = (int32_t)part * kAttnPartTokens;
  const int32_t n_valid = ctx - part_start < kAttnPartTokens ? ctx - part_start : kAttnPartTokens;

  // Query slice of this lane for every head of the group.
  float qr[G][EPL];
  {
    const float* qb = q + ((uint64_t)seq * n_heads + (uint64_t)kvh * G) * D + c * EPL;
#pragma unroll
    for (int gg = 0; gg < G; gg++) {
#pragma unroll
      for (int i = 0; i < EPL; i += 4) {
        float4 t = *(const float4*)(qb + (uint64_t)gg * D + i);
        qr[gg][i] = t.x; qr[gg][i + 1] = t.y; qr[gg][i + 2] = t.z; qr[gg][i + 3] = t.w;
      }
    }
  }

  // Physical blocks of this wave (wave-uniform).
  const int32_t lblk0 = (int32_t)part * (kAttnWaves * NB) + wave * NB;
  const int32_t* table = tables + (uint64_t)seq * max_blocks;
  int32_t phys[NB];
  bool live[NB], valid_blk[NB];
#pragma unroll
  for (int j = 0; j < NB; j++) {
    int32_t lb = lblk0 + j;
    valid_blk[j] = lb * kAttnBlock < ctx;
    int32_t p = valid_blk[j] ? table[lb] : 0;
    p = __builtin_amdgcn_readfirstlane(p);
    bool ok = valid_blk[j] && p >= 0 && (uint64_t)p < g.num_blocks;
    if (valid_blk[j] && !ok && lane == 0) raise_fault(g.fault, kFaultBlock);
    live[j] = ok;
    phys[j] = p;
  }

  const uint64_t row_bytes = (uint64_t)D * S::E;
  const uint64_t scale_off = (uint64_t)kAttnBlock * D;  // Q8_0 scales follow the quants

  // Issue K loads for all blocks, then V loads (kept in flight through phase 1-2).
  uint4 kreg[NB][PASSES];
  uint32_t ksc[NB][PASSES];
#pragma unroll
  for (int j = 0; j < NB; j++) {
    if (live[j]) {
      const uint8_t* kt = tile_ptr(g, (uint64_t)phys[j], layer, 0, kvh);
#pragma unroll
      for (int ps = 0; ps < PASSES; ps++) {
        int row = ps * RPP + r;
        kreg[j][ps] = *(const uint4*)(kt + row * row_bytes + c * 16);
        if constexpr (DT == kDtypeQ8)
          ksc[j][ps] = ((const uint16_t*)(kt + scale_off))[row * (D / 32) + (c * EPL) / 32];
      }
    }
  }
  uint4 vreg[S::kPrefetchV ? NB : 1][PASSES];
  uint32_t vsc[S::kPrefetchV ? NB : 1][PASSES];
  if constexpr (S::kPrefetchV) {
#pragma unroll
    for (int j = 0; j < NB; j++) {
      if (live[j]) {
        const uint8_t* vt = tile_ptr(g, (uint64_t)phys[j], layer, 1, kvh);
#pragma unroll
        for (int ps = 0; ps < PASSES; ps++) {
          int row = ps * RPP + r;
          vreg[j][ps] = *(const uint4*)(vt + row * row_bytes + c * 16);
          if constexpr (DT == kDtypeQ8)
            vsc[j][ps] = ((const uint16_t*)(vt + scale_off))[row * (D / 32) + (c * EPL) / 32];
        }
      }
    }
  }

  // Phase 1: scores.
#pragma unroll
  for (int j = 0; j < NB; j++) {
#pragma unroll
    for (int ps = 0; ps < PASSES; ps++) {
      const int32_t tl = (wave * NB + j) * kAttnBlock + ps * RPP + r;  // token within partition
      float part_dot[G];
      if (live[j]) {
        float kf[EPL];
        decode16<DT, EPL>(kreg[j][ps], kf);
#pragma unroll
        for (int gg = 0; gg < G; gg++) {
          float a = 0.0f;
#pragma unroll
          for (int i = 0; i < EPL; i++) a = __builtin_fmaf(qr[gg][i], kf[i], a);
          if constexpr (DT == kDtypeQ8) a *= f16_bits_to_f32(ksc[j][ps]);
          part_dot[gg] = group_sum<LPR>(a);
        }
      }
      if (c == 0) {
#pragma unroll
        for (int gg = 0; gg < G; gg++)
          s_score[gg][tl] = (live[j] && tl < n_valid) ? part_dot[gg] * scale : -__builtin_inff();
      }
    }
  }
  __syncthreads();

  // Phase 2: exact softmax statistics of this partition, one wave per head.
  for (int gg = wave; gg < G; gg += kAttnWaves) {
    float m = -__builtin_inff();
    for (int t = lane; t < kAttnPartTokens; t += 64)
      if (t < n_valid) m = __builtin_fmaxf(m, s_score[gg][t]);  // NaN is skipped
    m = wave_max(m);
    float l = 0.0f;
    const bool m_neg_inf = (m == -__builtin_inff());
    for (int t = lane; t < kAttnPartTokens; t += 64) {
      float e = 0.0f;
      if (t < n_valid) {
        float s = s_score[gg][t];
        // All scores -inf/NaN: weights are 0, but a NaN score must stay NaN.
        e = m_neg_inf ? (s != s ? s : 0.0f) : __builtin_amdgcn_exp2f((s - m) * kLog2e);
      }
      s_p[t][gg] = e;
      l += e;
    }
    l = wave_sum(l);
    if (lane == 0) {
      s_m[gg] = m;
      s_l[gg] = l;
    }
  }
  __syncthreads();

  // Phase 3: weighted V.
  float acc[G][EPL];
#pragma unroll
  for (int gg = 0; gg < G; gg++)
#pragma unroll
    for (int i = 0; i < EPL; i++) acc[gg][i] = 0.0f;

#pragma unroll
  for (int j = 0; j < NB; j++) {
    if (!live[j]) continue;
    uint4 vl[PASSES];
    uint32_t vs[PASSES];
    if constexpr (S::kPrefetchV) {
#pragma unroll
      for (int ps = 0; ps < PASSES; ps++) {
        vl[ps] = vreg[j][ps];
        vs[ps] = vsc[j][ps];
      }
    } else {
      const uint8_t* vt = tile_ptr(g, (uint64_t)phys[j], layer, 1, kvh);
#pragma unroll
      for (int ps = 0; ps < PASSES; ps++) {
        int row = ps * RPP + r;
        vl[ps] = *(const uint4*)(vt + row * row_bytes + c * 16);
        if constexpr (DT == kDtypeQ8)
          vs[ps] = ((const uint16_t*)(vt + scale_off))[row * (D / 32) + (c * EPL) / 32];
      }
    }
#pragma unroll
    for (int ps = 0; ps < PASSES; ps++) {
      const int32_t tl = (wave * NB + j) * kAttnBlock + ps * RPP + r;
      if (tl < n_valid) {
        float vf[EPL];
        decode16<DT, EPL>(vl[ps], vf);
        float pw[G];
#pragma unroll
        for (int gg = 0; gg < G; gg++) pw[gg] = s_p[tl][gg];
        if constexpr (DT == kDtypeQ8) {
          float sv = f16_bits_to_f32(vs[ps]);
#pragma unroll
          for (int gg = 0; gg < G; gg++) pw[gg] *= sv;
        }
#pragma unroll
        for (int gg = 0; gg < G; gg++)
#pragma unroll
          for (int i = 0; i < EPL; i++) acc[gg][i] = __builtin_fmaf(pw[gg], vf[i], acc[gg][i]);
      }
    }
  }
  (void)vsc;

  // Reduce the RPP token rows of the wave (lanes with equal c).
#pragma unroll
  for (int gg = 0; gg < G; gg++)
#pragma unroll
    for (int i = 0; i < EPL; i++) {
      float x = acc[gg][i];
#pragma unroll
      for (int o = LPR; o < 64; o <<= 1) x += __shfl_xor(x, o);
      acc[gg][i] = x;
    }
  if (r == 0) {
#pragma unroll
    for (int gg = 0; gg < G; gg++)
#pragma unroll
      for (int i = 0; i < EPL; i++) s_acc[wave][gg][c * EPL + i] = acc[gg][i];
  }
  __syncthreads();

  for (int e = threadIdx.x; e < G * D; e += 256) {
    const int gg = e / D, d = e % D;
    float o = (s_acc[0][gg][d] + s_acc[1][gg][d]) + (s_acc[2][gg][d] + s_acc[3][gg][d]);
    const uint64_t head = (uint64_t)seq * n_heads + (uint64_t)kvh * G + gg;
    if (nparts == 1) {
      const float m = s_m[gg];
      out[head * D + d] = __builtin_isfinite(m) ? o * (1.0f / s_l[gg]) : 0.0f;
    } else {
      ws_o[(head * max_parts + part) * D + d] = o;
      if (d == 0) {
        ws_ml[(head * max_parts + part) * 2] = s_m[gg];
        ws_ml[(head * max_parts + part) * 2 + 1] = s_l[gg];
      }
    }
  }
}

// Merge the partitions of one (sequence, query head): M = max_p m_p (NaN
// skipped); a non-finite M gives zeros (scalar.rs:127-130); otherwise
// out = sum_p w_p o_p / sum_p w_p l_p with w_p = exp(m_p - M).
// 256 threads: thread t covers dims 4*(t % (D/4)).. and partitions p = t / (D/4) mod P.
template <int D>
__global__ void __launch_bounds__(256) attn_combine_kernel(
    const int32_t* __restrict__ ctx_lens, uint32_t n_heads, uint32_t max_blocks,
    uint32_t max_parts, const float* __restrict__ ws_o, const float* __restrict__ ws_ml,
    float* __restrict__ out) {
  constexpr int kLanesPerRow = D / 4;
  constexpr int kRows = 256 / kLanesPerRow;
  __shared__ float s_red[kRows][D];
  __shared__ float s_lred[kRows];
  __shared__ float s_max[4];

  const uint32_t head = blockIdx.x;  // seq * n_heads + h
  const uint32_t seq = head / n_heads;
  const int32_t cap = (int32_t)(max_blocks * kAttnBlock);
  int32_t ctx = ctx_lens[seq];
  ctx = ctx < 0 ? 0 : (ctx > cap ? cap : ctx);
  const int32_t nparts = ctx > 0 ? (ctx + kAttnPartTokens - 1) / kAttnPartTokens : 1;
  if (nparts == 1) return;

  const float* ml = ws_ml + (uint64_t)head * max_parts * 2;
  const float* po = ws_o + (uint64_t)head * max_parts * D;
  const int wave = threadIdx.x / 64, lane = threadIdx.x % 64;

  float m = -__builtin_inff();
  for (int p = threadIdx.x; p < nparts; p += 256) m = __builtin_fmaxf(m, ml[2 * p]);
  m = wave_max(m);
  if (lane == 0) s_max[wave] = m;
  __syncthreads();
  const float M = __builtin_fmaxf(__builtin_fmaxf(s_max[0], s_max[1]),
                                  __builtin_fmaxf(s_max[2], s_max[3]));
  float* o = out + (uint64_t)head * D;
  if (!__builtin_isfinite(M)) {
    for (int d = threadIdx.x; d < D; d += 256) o[d] = 0.0f;
    return;
  }
  const int col = threadIdx.x % kLanesPerRow, row = threadIdx.x / kLanesPerRow;
  float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
  float lsum = 0.0f;
  for (int p = row; p < nparts; p += kRows) {
    const float w = __builtin_amdgcn_exp2f((ml[2 * p] - M) * kLog2e);
    lsum = __builtin_fmaf(w, ml[2 * p + 1], lsum);
    const float4 v = *(const float4*)(po + (uint64_t)p * D + col * 4);
    acc.x = __builtin_fmaf(w, v.x, acc.x);
    acc.y = __builtin_fmaf(w, v.y, acc.y);
    acc.z = __builtin_fmaf(w, v.z, acc.z);
    acc.w = __builtin_fmaf(w, v.w, acc.w);
  }
  s_red[row][col * 4] = acc.x;
  s_red[row][col * 4 + 1] = acc.y;
  s_red[row][col * 4 + 2] = acc.z;
  s_red[row][col * 4 + 3] = acc.w;
  if (col == 0) s_lred[row] = lsum;
  __syncthreads();
  if (threadIdx.x < D) {
    float a = 0.0f, l = 0.0f;
#pragma unroll
    for (int rr = 0; rr < kRows; rr++) {
      a += s_red[rr][threadIdx.x];
      l += s_lred[rr];
    }
    o[threadIdx.x] = a * (1.0f / l);
  }
}

template <int DT, int D, int G>
hipError_t launch_attn_t(const Geom& g, uint32_t layer, uint32_t n_heads, const float* q,
                         float* out, const int32_t* tables, uint32_t max_blocks,
                         const int32_t* ctx_lens, uint32_t n_seqs, uint32_t max_parts,
                         float scale, float* ws_o, float* ws_ml, hipStream_t s) {
  dim3 grid(n_seqs * g.n_kv_heads, max_parts);
  attn_partition_kernel<DT, D, G><<<grid, 256, 0, s>>>(g, layer, n_heads, q, out, tables,
                                                       max_blocks, ctx_lens, max_parts, scale,
                                                       ws_o, ws_ml);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || max_parts <= 1) return e;
  attn_combine_kernel<D><<<n_seqs * n_heads, 256, 0, s>>>(ctx_lens, n_heads, max_blocks,
                                                          max_parts, ws_o, ws_ml, out);
  return hipGetLastError();
}

template <int DT, int D>
hipError_t dispatch_group(uint32_t G, const Geom& g, uint32_t layer, uint32_t n_heads,
                          const float* q, float* out, const int32_t* tables,
                          uint32_t max_blocks, const int32_t* ctx_lens, uint32_t n_seqs,
                          uint32_t max_parts, float scale, float* ws_o, float* ws_ml,
                          hipStream_t s) {
#define FKV_G(N)                                                                          \
  case N:                                                                                 \
    return launch_attn_t<DT, D, N>(g, layer, n_heads, q, out, tables, max_blocks, ctx_lens, \
                                   n_seqs, max_parts, scale, ws_o, ws_ml, s);
  switch (G) {
    FKV_G(1)
    FKV_G(2)
    FKV_G(4)
    FKV_G(8)
    default:
      break;
  }
  if constexpr (DT != kDtypeQ8) {
    if (G == 16)
      return launch_attn_t<DT, D, 16>(g, layer, n_heads, q, out, tables, max_blocks, ctx_lens,
                                      n_seqs, max_parts, scale, ws_o, ws_ml, s);
  }
#undef FKV_G
  return hipErrorInvalidValue;
}

inline uint32_t grid_for(uint64_t units, uint32_t max_wg = 8192) {
  uint64_t wg = (units + 255) / 256;
  if (wg < 1) wg = 1;
  return (uint32_t)(wg < max_wg ? wg : max_wg);
}

}  // namespace

// ---------------------------------------------------------------------------
// Launchers
// ---------------------------------------------------------------------------

hipError_t launch_append(const Geom& g, uint32_t layer, const float* k, const float* v,
                         const int64_t* slots, uint32_t n_tokens, hipStream_t s) {
  if (n_tokens == 0) return hipSuccess;
  const bool aligned = ((uintptr_t)k % 16 == 0) && ((uintptr_t)v % 16 == 0);
  if (g.dtype == kDtypeQ8) {
    uint64_t units = (uint64_t)n_tokens * 2u * g.n_kv_heads * (g.head_dim / 32u);
    if (aligned)
      append_q8_kernel<true><<<grid_for(units), 256, 0, s>>>(g, layer, k, v, slots, n_tokens);
    else
      append_q8_kernel<false><<<grid_for(units), 256, 0, s>>>(g, layer, k, v, slots, n_tokens);
  } else if (g.head_dim % 8 == 0 && aligned) {
    uint64_t units = (uint64_t)n_tokens * 2u * g.n_kv_heads * (g.head_dim / 8u);
    if (g.dtype == kDtypeF16)
      append_vec8_kernel<kDtypeF16><<<grid_for(units), 256, 0, s>>>(g, layer, k, v, slots, n_tokens);
    else
      append_vec8_kernel<kDtypeF32><<<grid_for(units), 256, 0, s>>>(g, layer, k, v, slots, n_tokens);
  } else {
    uint64_t units = (uint64_t)n_tokens * 2u * g.n_kv_heads * g.head_dim;
    append_scalar_kernel<<<grid_for(units), 256, 0, s>>>(g, layer, k, v, slots, n_tokens);
  }
  return hipGetLastError();
}

// The chunked gather path needs head_dim % 8 == 0 (F32/F16); callers with other
// head dims use it through the per-element fallback below.
__global__ void __launch_bounds__(256) gather_slots_scalar_kernel(Geom g, uint32_t layer,
                                                                  const int64_t* __restrict__ slots,
                                                                  uint32_t n_tokens, int format,
                                                                  uint8_t* out_k, uint8_t* out_v) {
  const uint32_t D = g.head_dim;
  const uint32_t per_kv = g.n_kv_heads * D;
  const uint64_t total = (uint64_t)n_tokens * 2u * per_kv;
  const uint64_t cap = g.num_blocks * g.block_size;
  for (uint64_t u = (uint64_t)blockIdx.x * 256u + threadIdx.x; u < total;
       u += (uint64_t)gridDim.x * 256u) {
    uint32_t token = (uint32_t)(u / (2u * per_kv));
    uint32_t rem = (uint32_t)(u % (2u * per_kv));
    uint32_t kv = rem / per_kv, e = rem % per_kv, h = e / D, d = e % D;
    int64_t slot = slots[token];
    if (slot < 0) continue;
    if ((uint64_t)slot >= cap) {
      if (rem == 0) raise_fault(g.fault, kFaultSlot);
      continue;
    }
    const uint8_t* tile = tile_ptr(g, (uint64_t)slot / g.block_size, layer, kv, h);
    uint64_t idx = ((uint64_t)slot % g.block_size) * D + d;
    uint8_t* o = kv ? out_v : out_k;
    uint64_t oi = (uint64_t)token * per_kv + e;
    if (g.dtype == kDtypeF16) {
      uint16_t bits = ((const uint16_t*)tile)[idx];
      if (format == 0) ((float*)o)[oi] = f16_bits_to_f32(bits);
      else ((uint16_t*)o)[oi] = bits;
    } else {
      ((float*)o)[oi] = ((const float*)tile)[idx];
    }
  }
}

hipError_t launch_gather_slots(const Geom& g, uint32_t layer, const int64_t* slots,
                               uint32_t n_tokens, int format, void* out_k, void* out_v,
                               hipStream_t s) {
  if (n_tokens == 0) return hipSuccess;
  if (g.dtype != kDtypeQ8 && g.head_dim % 8 != 0) {
    uint64_t units = (uint64_t)n_tokens * 2u * g.n_kv_heads * g.head_dim;
    gather_slots_scalar_kernel<<<grid_for(units), 256, 0, s>>>(
        g, layer, slots, n_tokens, format, (uint8_t*)out_k, (uint8_t*)out_v);
    return hipGetLastError();
  }
  const bool aligned = ((uintptr_t)out_k % 16 == 0) && ((uintptr_t)out_v % 16 == 0);
  uint32_t cv = g.dtype == kDtypeQ8 ? 32u : 8u;
  uint64_t units = (uint64_t)n_tokens * 2u * g.n_kv_heads * (g.head_dim / cv);
  gather_slots_kernel<<<grid_for(units), 256, 0, s>>>(g, layer, slots, n_tokens, format,
                                                      (uint8_t*)out_k, (uint8_t*)out_v, aligned);
  return hipGetLastError();
}

hipError_t launch_gather_tables(const Geom& g, uint32_t layer, const int32_t* tables,
                                uint32_t max_blocks, const int32_t* ctx_lens,
                                const int64_t* out_offsets, uint32_t n_seqs,
                                uint32_t max_ctx_len, int format, void* out_k, void* out_v,
                                hipStream_t s) {
  if (n_seqs == 0 || max_ctx_len == 0) return hipSuccess;
  const bool aligned = ((uintptr_t)out_k % 16 == 0) && ((uintptr_t)out_v % 16 == 0);
  uint32_t cv = g.dtype == kDtypeQ8 ? 32u : 8u;
  uint64_t units = (uint64_t)max_ctx_len * 2u * g.n_kv_heads * (g.head_dim / cv);
  dim3 grid(grid_for(units, 4096), n_seqs);
  gather_tables_kernel<<<grid, 256, 0, s>>>(g, layer, tables, max_blocks, ctx_lens, out_offsets,
                                            format, (uint8_t*)out_k, (uint8_t*)out_v, aligned);
  return hipGetLastError();
}

hipError_t launch_copy_blocks(const Geom& g, const int64_t* pairs, uint32_t n_pairs,
                              hipStream_t s) {
  if (n_pairs == 0) return hipSuccess;
  uint64_t vecs = g.block_bytes / 16u;
  uint64_t total = (uint64_t)n_pairs * ((vecs + kCopyChunkVecs - 1) / kCopyChunkVecs);
  uint32_t grid = (uint32_t)(total < 16384 ? total : 16384);
  copy_blocks_kernel<<<grid, 256, 0, s>>>(g, pairs, n_pairs);
  return hipGetLastError();
}

hipError_t launch_fill(void* dst, uint8_t byte, uint64_t bytes, hipStream_t s) {
  if (bytes == 0) return hipSuccess;
  uint32_t word = 0x01010101u * byte;
  fill_kernel<<<grid_for(bytes / 16 + 1, 16384), 256, 0, s>>>((uint8_t*)dst, word, bytes);
  return hipGetLastError();
}

hipError_t launch_device_copy(void* dst, const void* src, uint64_t bytes, hipStream_t s) {
  if (bytes == 0) return hipSuccess;
  uint64_t vecs = bytes / 16u;
  if (vecs) {
    uint64_t wg = (vecs + kCopyChunkVecs - 1) / kCopyChunkVecs;
    device_copy_kernel<<<(uint32_t)(wg < 16384 ? wg : 16384), 256, 0, s>>>(
        (u32x4*)dst, (const u32x4*)src, vecs);
  }
  if (bytes % 16)
    copy_tail_kernel<<<1, 64, 0, s>>>((uint8_t*)dst, (const uint8_t*)src, vecs * 16u, bytes);
  return hipGetLastError();
}

bool attention_supported(int dtype, uint32_t head_dim, uint32_t group) {
  if (head_dim != 64 && head_dim != 128) return false;
  if (dtype != kDtypeF16 && dtype != kDtypeF32 && dtype != kDtypeQ8) return false;
  if (group == 1 || group == 2 || group == 4 || group == 8) return true;
  return group == 16 && dtype != kDtypeQ8;
}

uint64_t attention_workspace_bytes(uint32_t n_heads, uint32_t head_dim, uint32_t n_seqs,
                                   uint32_t max_ctx_len) {
  uint64_t parts = max_ctx_len ? (max_ctx_len + kAttnPartTokens - 1) / kAttnPartTokens : 1;
  if (parts <= 1) return 0;
  return (uint64_t)n_seqs * n_heads * parts * ((uint64_t)head_dim + 2u) * 4u;
}

hipError_t launch_decode_attention(const Geom& g, uint32_t layer, uint32_t n_heads,
                                   const float* q, float* out, const int32_t* tables,
                                   uint32_t max_blocks, const int32_t* ctx_lens,
                                   uint32_t n_seqs, uint32_t max_ctx_len, float scale,
                                   void* workspace, hipStream_t s) {
  if (n_seqs == 0) return hipSuccess;
  const uint32_t G = n_heads / g.n_kv_heads;
  const uint32_t max_parts =
      max_ctx_len ? (max_ctx_len + kAttnPartTokens - 1) / kAttnPartTokens : 1;
  float* ws_o = (float*)workspace;
  float* ws_ml = ws_o ? ws_o + (uint64_t)n_seqs * n_heads * max_parts * g.head_dim : nullptr;
  if (g.head_dim == 128) {
    if (g.dtype == kDtypeF16)
      return dispatch_group<kDtypeF16, 128>(G, g, layer, n_heads, q, out, tables, max_blocks,
                                            ctx_lens, n_seqs, max_parts, scale, ws_o, ws_ml, s);
    if (g.dtype == kDtypeF32)
      return dispatch_group<kDtypeF32, 128>(G, g, layer, n_heads, q, out, tables, max_blocks,
                                            ctx_lens, n_seqs, max_parts, scale, ws_o, ws_ml, s);
    return dispatch_group<kDtypeQ8, 128>(G, g, layer, n_heads, q, out, tables, max_blocks,
                                         ctx_lens, n_seqs, max_parts, scale, ws_o, ws_ml, s);
  }
  if (g.dtype == kDtypeF16)
    return dispatch_group<kDtypeF16, 64>(G, g, layer, n_heads, q, out, tables, max_blocks,
                                         ctx_lens, n_seqs, max_parts, scale, ws_o, ws_ml, s);
  if (g.dtype == kDtypeF32)
    return dispatch_group<kDtypeF32, 64>(G, g, layer, n_heads, q, out, tables, max_blocks,
                                         ctx_lens, n_seqs, max_parts, scale, ws_o, ws_ml, s);
  return dispatch_group<kDtypeQ8, 64>(G, g, layer, n_heads, q, out, tables, max_blocks,
                                      ctx_lens, n_seqs, max_parts, scale, ws_o, ws_ml, s);
}

}  // namespace fkv
