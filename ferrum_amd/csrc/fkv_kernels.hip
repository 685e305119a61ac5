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

#include "fkv_device.h"
#include "fkv_internal.h"

namespace fkv {
namespace {

using namespace dev;

// ---------------------------------------------------------------------------
// Q8_0 block quantiser (q8_dot.rs:46-59)
// ---------------------------------------------------------------------------

// x[32] -> 32 int8 packed in q[8] (little-endian bytes) and the f16 scale bits.
__device__ __forceinline__ uint32_t q8_quantize(const float (&x)[32], int rounding,
                                                uint32_t (&q)[8]) {
  float amax = 0.0f;
#pragma unroll
  for (int j = 0; j < 32; j++) amax = __builtin_fmaxf(amax, __builtin_fabsf(x[j]));
  float id;
  const float d = q8_scale(amax, id);
#pragma unroll
  for (int w = 0; w < 8; w++) {
    uint32_t packed = 0;
#pragma unroll
    for (int b = 0; b < 4; b++) packed |= ((uint32_t)q8_quant(x[w * 4 + b], id) & 0xffu) << (8 * b);
    q[w] = packed;
  }
  return encode_f16(d, rounding);
}

// ---------------------------------------------------------------------------
// Append (paged KvPool::append_layer)
// ---------------------------------------------------------------------------

// F32 storage, head_dim % 8 == 0, 16-byte aligned k/v: one thread moves 8
// values of one (token, kv, head) row (32 B in, 32 B out).
__global__ void __launch_bounds__(256) append_f32_kernel(Geom g, uint32_t layer,
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
    uint8_t* tile = tile_ptr(g, (uint64_t)slot / g.block_size, layer, kv, h);
    float4* dst = (float4*)(tile + (((uint64_t)slot % g.block_size) * g.head_dim + c * 8u) * 4u);
    dst[0] = *(const float4*)src;
    dst[1] = *(const float4*)(src + 4);
  }
}

// F16 storage, head_dim % 16 == 0, 16-byte aligned k/v. Workgroups [0, k_groups)
// write K: one thread per 8 dims of a (token, head) row, one 16-byte store into
// run c of the [D/8][B][8] tile. The rest write V into the [D][B] tile: one wave
// per (16 input tokens, head, 16 dims), lane (t, g) holding dims 4g..4g+3 of
// token t, so each 2-byte store instruction fills whole 32-byte dim rows when
// the 16 tokens sit at consecutive offsets of one block (prefill), and is still
// exact for any other slot mapping.
__global__ void __launch_bounds__(256) append_f16_kernel(Geom g, uint32_t layer,
                                                         const float* __restrict__ k,
                                                         const float* __restrict__ v,
                                                         const int64_t* __restrict__ slots,
                                                         uint32_t n_tokens, uint32_t k_groups) {
  const uint32_t D = g.head_dim, Bs = g.block_size;
  const uint64_t cap = g.num_blocks * Bs;
  if (blockIdx.x < k_groups) {
    const uint32_t cpr = D / 8, cph = g.n_kv_heads * cpr;
    const uint64_t u = (uint64_t)blockIdx.x * 256u + threadIdx.x;
    if (u >= (uint64_t)n_tokens * cph) return;
    const uint32_t token = (uint32_t)(u / cph), r2 = (uint32_t)(u % cph);
    const uint32_t h = r2 / cpr, c = r2 % cpr;
    const int64_t slot = slots[token];
    if (slot < 0) return;
    if ((uint64_t)slot >= cap) {
      if (r2 == 0) raise_fault(g.fault, kFaultSlot);
      return;
    }
    const float* src = k + ((uint64_t)token * g.n_kv_heads + h) * D + c * 8u;
    const float4 a = *(const float4*)src, b = *(const float4*)(src + 4);
    uint8_t* tile = tile_ptr(g, (uint64_t)slot / Bs, layer, 0, h);
    const uint4 w = make_uint4(encode_f16(a.x, g.rounding) | (encode_f16(a.y, g.rounding) << 16),
                               encode_f16(a.z, g.rounding) | (encode_f16(a.w, g.rounding) << 16),
                               encode_f16(b.x, g.rounding) | (encode_f16(b.y, g.rounding) << 16),
                               encode_f16(b.z, g.rounding) | (encode_f16(b.w, g.rounding) << 16));
    *(uint4*)(tile + ((uint64_t)c * Bs + (uint64_t)slot % Bs) * 16u) = w;
    if (f16x2_nonfinite(w.x) || f16x2_nonfinite(w.y) || f16x2_nonfinite(w.z) ||
        f16x2_nonfinite(w.w))
      mark_block(g, (uint64_t)slot / Bs);  // chunked prefill's leak-safe instance reads it
    return;
  }
  const uint32_t dgs = D / 16;  // 16-dim groups per head
  const uint64_t wv = ((uint64_t)(blockIdx.x - k_groups) * 256u + threadIdx.x) / 64u;
  const uint32_t lane = threadIdx.x % 64u, t = lane % 16u, grp = lane / 16u;
  const uint64_t tb = wv / ((uint64_t)g.n_kv_heads * dgs);
  const uint32_t rem = (uint32_t)(wv % ((uint64_t)g.n_kv_heads * dgs));
  const uint32_t h = rem / dgs, dg = rem % dgs;
  const uint64_t token = tb * 16u + t;
  if (token >= n_tokens) return;
  const int64_t slot = slots[token];
  if (slot < 0) return;
  if ((uint64_t)slot >= cap) {
    if (rem == 0 && grp == 0) raise_fault(g.fault, kFaultSlot);
    return;
  }
  const uint32_t d0 = dg * 16u + grp * 4u;
  const float4 x = *(const float4*)(v + (token * g.n_kv_heads + h) * D + d0);
  uint16_t* vt = (uint16_t*)tile_ptr(g, (uint64_t)slot / Bs, layer, 1, h) + (uint64_t)d0 * Bs +
                 (uint64_t)slot % Bs;
  const uint32_t e0 = encode_f16(x.x, g.rounding), e1 = encode_f16(x.y, g.rounding);
  const uint32_t e2 = encode_f16(x.z, g.rounding), e3 = encode_f16(x.w, g.rounding);
  vt[0] = (uint16_t)e0;
  vt[Bs] = (uint16_t)e1;
  vt[2 * Bs] = (uint16_t)e2;
  vt[3 * Bs] = (uint16_t)e3;
  if (f16_nonfinite(e0) || f16_nonfinite(e1) || f16_nonfinite(e2) || f16_nonfinite(e3))
    mark_block(g, (uint64_t)slot / Bs);  // chunked prefill's leak-safe instance reads it
}

// F16 storage, block_size 16, head_dim 64 or 128, 16-byte aligned k/v: one workgroup
// per 16 consecutive input tokens (a window) x 256 / (2 D) KV heads; thread (c, o)
// of a head holds dims 8c .. 8c+7 of window token o, tokens fastest, so a wave's
// loads cover whole 128-byte lines of four token rows.
// - K: the thread's 16-byte run goes to run c of its token's [D/8][16][8] tile;
//   tokens at consecutive slots of one block make a wave's stores contiguous.
// - V: the window's rows are transposed through LDS ([dim][token]); thread (d, hh)
//   then stores tokens 8hh .. 8hh+7 of dim d: one 16-byte store when they sit at
//   offsets 0..7 or 8..15 of one block (the whole half of the tile's row d), else one
//   2-byte store per token (any slot mapping, slots < 0 skipped).
// Encoding and fault rules are append_f16_kernel's, bit for bit.
template <int D>
__global__ void __launch_bounds__(256) append_f16_tile_kernel(Geom g, uint32_t layer,
                                                              const float* __restrict__ k,
                                                              const float* __restrict__ v,
                                                              const int64_t* __restrict__ slots,
                                                              uint32_t n_tokens) {
  constexpr int kRuns = D / 8;           // 8-dim runs of a row
  constexpr int kTph = 16 * kRuns;       // threads per (window, head)
  constexpr int kHpw = 256 / kTph;       // heads per workgroup
  static_assert(kHpw * kTph == 256, "head_dim 64 or 128");
  __shared__ int64_t s_slot[16];
  __shared__ __align__(16) uint16_t s_v[kHpw][D][16];

  const uint32_t hgroups = (g.n_kv_heads + kHpw - 1) / kHpw;
  const uint32_t win = blockIdx.x / hgroups, hg = blockIdx.x % hgroups;
  const uint32_t hl = threadIdx.x / kTph, u = threadIdx.x % kTph;
  const uint32_t h = hg * kHpw + hl;
  const bool head_ok = h < g.n_kv_heads;
  const uint64_t cap = g.num_blocks * 16u;
  if (threadIdx.x < 16) {
    const uint64_t t = (uint64_t)win * 16u + threadIdx.x;
    int64_t sl = t < n_tokens ? slots[t] : -1;
    if (sl >= 0 && (uint64_t)sl >= cap) {
      raise_fault(g.fault, kFaultSlot);
      sl = -1;
    }
    s_slot[threadIdx.x] = sl;
  }
  __syncthreads();

  const uint32_t c = u / 16u, o = u % 16u;
  const int64_t slot = s_slot[o];
  uint32_t ve[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  if (slot >= 0 && head_ok) {
    const uint64_t row = ((uint64_t)win * 16u + o) * g.n_kv_heads + h;
    const float* ks = k + row * D + c * 8u;
    const float* vs = v + row * D + c * 8u;
    const float4 a = *(const float4*)ks, b = *(const float4*)(ks + 4);
    const float4 x = *(const float4*)vs, y = *(const float4*)(vs + 4);
    uint8_t* kt = tile_ptr(g, (uint64_t)slot / 16u, layer, 0, h);
    const uint4 kw = make_uint4(encode_f16(a.x, g.rounding) | (encode_f16(a.y, g.rounding) << 16),
                                encode_f16(a.z, g.rounding) | (encode_f16(a.w, g.rounding) << 16),
                                encode_f16(b.x, g.rounding) | (encode_f16(b.y, g.rounding) << 16),
                                encode_f16(b.z, g.rounding) | (encode_f16(b.w, g.rounding) << 16));
    *(uint4*)(kt + ((uint64_t)c * 16u + (uint64_t)slot % 16u) * 16u) = kw;
    ve[0] = encode_f16(x.x, g.rounding); ve[1] = encode_f16(x.y, g.rounding);
    ve[2] = encode_f16(x.z, g.rounding); ve[3] = encode_f16(x.w, g.rounding);
    ve[4] = encode_f16(y.x, g.rounding); ve[5] = encode_f16(y.y, g.rounding);
    ve[6] = encode_f16(y.z, g.rounding); ve[7] = encode_f16(y.w, g.rounding);
    bool nf = f16x2_nonfinite(kw.x) || f16x2_nonfinite(kw.y) || f16x2_nonfinite(kw.z) ||
              f16x2_nonfinite(kw.w);
#pragma unroll
    for (int e = 0; e < 8; e++) nf = nf || f16_nonfinite(ve[e]);
    if (nf) mark_block(g, (uint64_t)slot / 16u);  // chunked prefill's leak-safe instance reads it
  }
#pragma unroll
  for (int e = 0; e < 8; e++) s_v[hl][c * 8u + e][o] = (uint16_t)ve[e];
  __syncthreads();

  if (!head_ok) return;
  // V row d of each destination tile. The window's tokens split into segments: maximal
  // runs of consecutive slots inside one 8-aligned group of a block (a whole group when
  // the window is aligned with the blocks, else two or three per group where a sequence
  // begins mid-window). Thread (d, hh) stores the segments that start at its tokens
  // hh*8 .. hh*8+7 with the widest aligned stores the run allows.
  const uint32_t d = u / 2u, hh = u % 2u;
  const uint16_t* vrow = s_v[hl][d];
  for (uint32_t i = hh * 8u; i < hh * 8u + 8u; i++) {
    const int64_t s0 = s_slot[i];
    if (s0 < 0 || (i > 0 && s0 % 8 != 0 && s_slot[i - 1] == s0 - 1)) continue;
    uint32_t len = 1;
    while (i + len < 16u && (s0 + len) % 8 != 0 && s_slot[i + len] == s0 + (int64_t)len) len++;
    uint8_t* row = tile_ptr(g, (uint64_t)s0 / 16u, layer, 1, h) + (uint64_t)d * 32u;
    uint32_t p = (uint32_t)(s0 % 16), j = i;
    const uint32_t end = p + len;
    while (p < end) {
      const uint32_t n = end - p;
      if (p % 8 == 0 && n >= 8) {
        *(uint4*)(row + p * 2u) =
            make_uint4(vrow[j] | ((uint32_t)vrow[j + 1] << 16), vrow[j + 2] | ((uint32_t)vrow[j + 3] << 16),
                       vrow[j + 4] | ((uint32_t)vrow[j + 5] << 16), vrow[j + 6] | ((uint32_t)vrow[j + 7] << 16));
        p += 8; j += 8;
      } else if (p % 4 == 0 && n >= 4) {
        *(uint2*)(row + p * 2u) =
            make_uint2(vrow[j] | ((uint32_t)vrow[j + 1] << 16), vrow[j + 2] | ((uint32_t)vrow[j + 3] << 16));
        p += 4; j += 4;
      } else if (p % 2 == 0 && n >= 2) {
        *(uint32_t*)(row + p * 2u) = vrow[j] | ((uint32_t)vrow[j + 1] << 16);
        p += 2; j += 2;
      } else {
        *(uint16_t*)(row + p * 2u) = vrow[j];
        p += 1; j += 1;
      }
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
    const uint64_t off = (uint64_t)slot % g.block_size;
    if (g.dtype == kDtypeF16) {
      const uint32_t e = encode_f16(x, g.rounding);
      ((uint16_t*)tile)[kv ? (uint64_t)d * g.block_size + off
                           : ((uint64_t)(d / 8) * g.block_size + off) * 8 + d % 8] = (uint16_t)e;
      if (f16_nonfinite(e)) mark_block(g, (uint64_t)slot / g.block_size);
    } else
      ((float*)tile)[off * D + d] = x;
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
    if (kv == 0) {  // K: dims c*32 + g*8 .. +7 are one 8-byte run per g
#pragma unroll
      for (uint32_t gg = 0; gg < 4; gg++)
        *(uint2*)(tile + q8_quant_offset(0, off, c * 32u + gg * 8u, D)) =
            make_uint2(q[2 * gg], q[2 * gg + 1]);
    } else {  // V: one byte per dim
#pragma unroll
      for (uint32_t j = 0; j < 32; j++)
        tile[q8_quant_offset(1, off, c * 32u + j, D)] = (uint8_t)(q[j / 4] >> (8 * (j % 4)));
    }
    ((uint16_t*)(tile + (uint64_t)B * D))[off * cpr + c] = (uint16_t)sc;
    // A scale of 512 or more marks the block (attention over it takes the exact
    // instance); one past the binary16 range (|x| >= 65520 * 127) is stored as +-inf,
    // as the reference's encoder stores it, and flagged.
    if (q8_wide_scale(sc)) {
      mark_block(g, (uint64_t)slot / B);
      if ((sc & 0x7c00u) == 0x7c00u) raise_fault(g.fault, kFaultRange);
    }
  }
}

// Q8_0 storage, head_dim 64 or 128, 16-byte aligned k/v: one workgroup per 16
// consecutive tokens x 256 / (32 * D / 64) KV heads. Thread (token o, kv, pair i)
// quantises dims 64i .. 64i+63 of one row (two Q8_0 blocks, each as append_q8_kernel
// does). K: the two blocks' 8-dim runs g of one token share a 16-byte unit of the
// operand order, so K goes out as four 16-byte stores; the two scales as one 4-byte
// store. V: a 16-byte unit holds dims j, j+16, j+32, j+48 of 4 consecutive tokens, so
// the quants go through LDS and thread (head, pair i, dim j) stores, for each segment of
// the window (a maximal run of consecutive slots inside one 4-aligned token group), a
// whole unit when the segment is the whole group and single bytes otherwise.
template <int D>
__global__ void __launch_bounds__(256) append_q8_tile_kernel(Geom g, uint32_t layer,
                                                             const float* __restrict__ k,
                                                             const float* __restrict__ v,
                                                             const int64_t* __restrict__ slots,
                                                             uint32_t n_tokens) {
  constexpr int kPairs = D / 64;           // 64-dim pairs of Q8_0 blocks per row
  constexpr int kTph = 16 * 2 * kPairs;    // quantising threads per head
  constexpr int kHpw = 256 / kTph;         // heads per workgroup
  static_assert(kHpw * kTph == 256, "head_dim 64 or 128");
  constexpr uint32_t cpr = D / 32;
  __shared__ int64_t s_slot[16];
  __shared__ __align__(16) uint8_t s_vq[kHpw][kPairs][16][64];

  const uint32_t hgroups = (g.n_kv_heads + kHpw - 1) / kHpw;
  const uint32_t win = blockIdx.x / hgroups, hg = blockIdx.x % hgroups;
  const uint32_t hl = threadIdx.x / kTph, u = threadIdx.x % kTph;
  const uint32_t h = hg * kHpw + hl;
  const bool head_ok = h < g.n_kv_heads;
  const uint32_t B = g.block_size;
  const uint64_t cap = g.num_blocks * B;
  if (threadIdx.x < 16) {
    const uint64_t t = (uint64_t)win * 16u + threadIdx.x;
    int64_t sl = t < n_tokens ? slots[t] : -1;
    if (sl >= 0 && (uint64_t)sl >= cap) {
      raise_fault(g.fault, kFaultSlot);
      sl = -1;
    }
    s_slot[threadIdx.x] = sl;
  }
  __syncthreads();

  const uint32_t o = u % 16u, kv = (u / 16u) % 2u, i = u / 32u;
  const int64_t slot = s_slot[o];
  if (slot >= 0 && head_ok) {
    const float* src = (kv ? v : k) + (((uint64_t)win * 16u + o) * g.n_kv_heads + h) * D + i * 64u;
    uint32_t q[2][8], sc[2];
#pragma unroll
    for (int b = 0; b < 2; b++) {
      float x[32];
#pragma unroll
      for (int j = 0; j < 8; j++) {
        const float4 t = ((const float4*)(src + b * 32))[j];
        x[4 * j] = t.x; x[4 * j + 1] = t.y; x[4 * j + 2] = t.z; x[4 * j + 3] = t.w;
      }
      sc[b] = q8_quantize(x, g.rounding, q[b]);
      // A scale of 512 or more marks the block (attention over it takes the exact
      // instance); one past the binary16 range is stored as +-inf, as the reference's
      // encoder stores it, and flagged.
      if (q8_wide_scale(sc[b])) {
        mark_block(g, (uint64_t)slot / B);
        if ((sc[b] & 0x7c00u) == 0x7c00u) raise_fault(g.fault, kFaultRange);
      }
    }
    const uint32_t off = (uint32_t)((uint64_t)slot % B);
    uint8_t* tile = tile_ptr(g, (uint64_t)slot / B, layer, kv, h);
    *(uint32_t*)(tile + (uint64_t)B * D + ((uint64_t)off * cpr + 2u * i) * 2u) = sc[0] | (sc[1] << 16);
    if (kv == 0) {
#pragma unroll
      for (uint32_t gg = 0; gg < 4; gg++)
        *(uint4*)(tile + q8_quant_offset(0, off, i * 64u + gg * 8u, D)) =
            make_uint4(q[0][2 * gg], q[0][2 * gg + 1], q[1][2 * gg], q[1][2 * gg + 1]);
    } else {
      uint32_t* dst = (uint32_t*)s_vq[hl][i][o];
#pragma unroll
      for (int w = 0; w < 8; w++) {
        dst[w] = q[0][w];
        dst[8 + w] = q[1][w];
      }
    }
  }
  __syncthreads();

  if (threadIdx.x >= (uint32_t)(kHpw * kPairs * 16)) return;
  const uint32_t vh = threadIdx.x / (kPairs * 16u), vi = (threadIdx.x / 16u) % kPairs,
                 j = threadIdx.x % 16u;
  const uint32_t hv = hg * kHpw + vh;
  if (hv >= g.n_kv_heads) return;
  for (uint32_t e0 = 0; e0 < 16u; e0++) {
    const int64_t s0 = s_slot[e0];
    if (s0 < 0 || (e0 > 0 && s0 % 4 != 0 && s_slot[e0 - 1] == s0 - 1)) continue;
    uint32_t len = 1;
    while (e0 + len < 16u && (s0 + len) % 4 != 0 && s_slot[e0 + len] == s0 + (int64_t)len) len++;
    const uint32_t off = (uint32_t)((uint64_t)s0 % B);
    uint8_t* unit = tile_ptr(g, (uint64_t)s0 / B, layer, 1, hv) +
                    (q8_quant_offset(1, off, vi * 64u + j, D) & ~(uint64_t)15);
    if (len == 4) {  // the whole 4-token group: bytes mm*4 + e = token e0+e, dim j + 16mm
      uint32_t w[4];
#pragma unroll
      for (uint32_t mm = 0; mm < 4; mm++)
        w[mm] = (uint32_t)s_vq[vh][vi][e0][16 * mm + j] |
                ((uint32_t)s_vq[vh][vi][e0 + 1][16 * mm + j] << 8) |
                ((uint32_t)s_vq[vh][vi][e0 + 2][16 * mm + j] << 16) |
                ((uint32_t)s_vq[vh][vi][e0 + 3][16 * mm + j] << 24);
      *(uint4*)unit = make_uint4(w[0], w[1], w[2], w[3]);
    } else {
      for (uint32_t e = 0; e < len; e++)
#pragma unroll
        for (uint32_t mm = 0; mm < 4; mm++)
          unit[mm * 4u + (off + e) % 4u] = s_vq[vh][vi][e0 + e][16 * mm + j];
    }
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
    uint32_t sc = ((const uint16_t*)(tile + (uint64_t)g.block_size * D))[off * (D / 32u) + c];
    auto qv = [&](uint32_t j) { return tile[q8_quant_offset(kv, off, c * 32u + j, D)]; };
    if (format == 0) {
      float s = f16_bits_to_f32(sc);
      float* o = (float*)dst_row + c * 32u;
      for (uint32_t j = 0; j < 32; j++) o[j] = s * (float)(int8_t)qv(j);
    } else {
      // Ferrum's 34-byte Q8_0 block: f16 scale (LE) then 32 x i8 (dtype.rs:19-21).
      uint16_t* o = (uint16_t*)(dst_row + (uint64_t)c * 34u);
      o[0] = (uint16_t)sc;
      for (uint32_t j = 0; j < 16; j++) o[1 + j] = (uint16_t)(qv(2 * j) | (qv(2 * j + 1) << 8));
    }
    return;
  }
  if (g.dtype == kDtypeF16 && kv == 1) {  // V tile [D][B]: dims are rows
    const uint16_t* src = (const uint16_t*)tile + (uint64_t)c * 8u * g.block_size + off;
    const uint32_t B = g.block_size;
    if (format == 0) {
      float* o = (float*)dst_row + c * 8u;
      for (int j = 0; j < 8; j++) o[j] = f16_bits_to_f32(src[j * B]);
    } else {
      uint16_t* o = (uint16_t*)dst_row + c * 8u;
      for (int j = 0; j < 8; j++) o[j] = src[j * B];
    }
    return;
  }
  if (g.dtype == kDtypeF16) {  // K tile [D/8][B][8]: run c of token off
    const uint16_t* src = (const uint16_t*)tile + ((uint64_t)c * g.block_size + off) * 8u;
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
// Gather, tile path: one workgroup per 16 tokens of one 16-token block x kHpw KV heads
// (block size 16, head_dim 64 or 128, F16 or Q8_0 storage, 16-byte aligned outputs).
// The output rows of the 16 tokens are consecutive (row0 + o for token o), as both
// entry points lay them out: a sequence's positions (by block table) or a window of 16
// slots that are one whole block (by slot).
// ---------------------------------------------------------------------------

// Heads per workgroup: F16 one 16-byte unit of each tile a thread (1 at D = 128, 2 at
// 64); Q8_0 tiles are half the bytes and staged whole, so 4 (8) heads keep as many bytes
// in flight per workgroup (one head a workgroup ran at 43% of a device copy).
constexpr uint32_t gather_heads_per_wg(int dtype, uint32_t d) {
  return dtype == kDtypeF16 ? 256u / (2u * d) : 512u / d;
}

template <int DT, int D>
struct GatherShape {
  static constexpr int kTph = 2 * D;            // F16 threads per (block, head) tile
  static constexpr int kHpw = (int)gather_heads_per_wg(DT, D);
  static constexpr int kTile = DT == kDtypeF16 ? 16 * D * 2 : 16 * D + 16 * (D / 32) * 2;
  static constexpr int kUnits = kTile / 16;     // 16-byte units of a tile
  static constexpr int kVRow = D + 4;           // F16 V transpose row (halves): rows 8 apart
                                                // fall 16 banks apart
};

// Bytes of a Q8_0 workgroup's heads in one output row: kHpw heads of D / 32 34-byte
// blocks, 16 x 34 at head_dim 64 and 128 alike.
constexpr uint32_t kGatherQ8Span = 16u * 34u;

// LDS of the tile path: F16 the V tiles transposed to [token][dim]; Q8_0 both tiles as
// stored, and for the raw format the workgroup's output records [kv][token][span].
constexpr int kFmtF32 = 0;  // FKV_GATHER_F32
constexpr int kFmtRaw = 1;  // FKV_GATHER_RAW

// Q8_0 tiles in LDS: head hl's K tile, then its V tile. For the raw format 16 bytes of
// padding follow every 256 bytes of a tile and heads start 32 banks apart: the record
// pass's dword reads of one instruction (lanes of other token groups, blocks and heads,
// at multiples of 256 bytes in the stored tile) then fall on distinct banks (unpadded:
// 8 V lanes a bank).
template <int D, int FMT>
struct GatherQ8Lds {
  static constexpr uint32_t kTile = 16u * D + 16u * (D / 32u) * 2u;
  static constexpr bool kPad = FMT == kFmtRaw;
  static constexpr uint32_t kTileP = kPad ? kTile + (kTile + 255u) / 256u * 16u : kTile;
  static constexpr uint32_t kHead = kPad ? (2u * kTileP + 127u) / 256u * 256u + 128u : 2u * kTileP;
  // byte b of head hl's tile kv
  __device__ static uint32_t off(uint32_t hl, uint32_t kv, uint32_t b) {
    return hl * kHead + kv * kTileP + (kPad ? b + (b >> 8) * 16u : b);
  }
};

template <int DT, int D, int FMT>
struct __align__(16) GatherLds {  // 16-byte unit stores into q
  using S = GatherShape<DT, D>;
  using Q = GatherQ8Lds<D, FMT>;
  static constexpr bool kRec = DT == kDtypeQ8 && FMT == kFmtRaw;
  union {
    uint16_t v[S::kHpw][16][S::kVRow];
    uint8_t q[DT == kDtypeQ8 ? S::kHpw * Q::kHead : 16];
  };
  // records: token rows 560 bytes apart, V's 16 bytes past a whole number of K's (the
  // record pass's stores of one instruction then meet at most 2 to a bank, against 4)
  static constexpr uint32_t kRecRow = kGatherQ8Span + 16u;
  static constexpr uint32_t kRecKv = 16u * kRecRow + 16u;
  uint8_t rec[kRec ? 2u * kRecKv : 16u];
  __device__ uint8_t* rec_at(uint32_t kv, uint32_t o, uint32_t b) {
    return rec + kv * kRecKv + o * kRecRow + b;
  }
};

// Stores 8 binary16 values (one 16-byte unit) as FMT requires: RAW the 16 bytes, F32
// the 8 decoded floats (32 bytes).
template <int FMT>
__device__ __forceinline__ void store_f16_unit(uint8_t* dst, uint4 w) {
  if constexpr (FMT == kFmtRaw) {
    *(uint4*)dst = w;
  } else {
    ((float4*)dst)[0] = make_float4(f16_bits_to_f32(w.x & 0xffffu), f16_bits_to_f32(w.x >> 16),
                                    f16_bits_to_f32(w.y & 0xffffu), f16_bits_to_f32(w.y >> 16));
    ((float4*)dst)[1] = make_float4(f16_bits_to_f32(w.z & 0xffffu), f16_bits_to_f32(w.z >> 16),
                                    f16_bits_to_f32(w.w & 0xffffu), f16_bits_to_f32(w.w >> 16));
  }
}

// One tile group: head hl of the workgroup is KV head h (h_ok false past the last head);
// kt / vt the head's K and V tiles (null when the block's table entry is outside the
// pool: nothing is written); tokens o < n are written to rows row0 + o of out_k / out_v
// (row_bytes apart; head h at h * head_bytes within a row). All 256 threads call this.
template <int DT, int D, int FMT>
__device__ __forceinline__ void gather_tile(GatherLds<DT, D, FMT>& lds, const Geom& g, uint32_t layer,
                                            int64_t blk, uint32_t h0, int32_t n,
                                            uint8_t* out_k, uint8_t* out_v, uint64_t row0) {
  using S = GatherShape<DT, D>;
  constexpr uint64_t kHeadBytes = FMT == kFmtF32 ? (uint64_t)D * 4u
                                  : DT == kDtypeF16      ? (uint64_t)D * 2u
                                                         : (uint64_t)D / 32u * 34u;
  const uint64_t row_bytes = (uint64_t)g.n_kv_heads * kHeadBytes;
  const bool blk_ok = blk >= 0 && (uint64_t)blk < g.num_blocks;
  if constexpr (DT == kDtypeF16) {
    const uint32_t hl = threadIdx.x / S::kTph, u = threadIdx.x % S::kTph;
    const uint32_t h = h0 + hl;
    const bool live = blk_ok && h < g.n_kv_heads;
    uint4 kw = make_uint4(0, 0, 0, 0), vw = make_uint4(0, 0, 0, 0);
    if (live) {
      // unit u of each tile: K run c = u / 16 of token u % 16; V dim u / 2, tokens 8(u % 2) ..
      kw = *(const uint4*)(tile_ptr(g, (uint64_t)blk, layer, 0, h) + (uint64_t)u * 16u);
      vw = *(const uint4*)(tile_ptr(g, (uint64_t)blk, layer, 1, h) + (uint64_t)u * 16u);
    }
    const uint32_t d = u / 2u, t8 = (u % 2u) * 8u;
    const uint32_t vh[8] = {vw.x & 0xffffu, vw.x >> 16, vw.y & 0xffffu, vw.y >> 16,
                            vw.z & 0xffffu, vw.z >> 16, vw.w & 0xffffu, vw.w >> 16};
#pragma unroll
    for (int j = 0; j < 8; j++) lds.v[hl][t8 + j][d] = (uint16_t)vh[j];
    const uint32_t o = u % 16u, c = u / 16u;
    if (live && (int32_t)o < n) {
      const uint64_t off = (row0 + o) * row_bytes + (uint64_t)h * kHeadBytes;
      constexpr uint32_t kUnitOut = FMT == kFmtF32 ? 32u : 16u;
      store_f16_unit<FMT>(out_k + off + (uint64_t)c * kUnitOut, kw);
    }
    __syncthreads();
    if (live && (int32_t)o < n) {
      const uint16_t* r = &lds.v[hl][o][c * 8u];
      const uint4 w = make_uint4(r[0] | ((uint32_t)r[1] << 16), r[2] | ((uint32_t)r[3] << 16),
                                 r[4] | ((uint32_t)r[5] << 16), r[6] | ((uint32_t)r[7] << 16));
      const uint64_t off = (row0 + o) * row_bytes + (uint64_t)h * kHeadBytes;
      constexpr uint32_t kUnitOut = FMT == kFmtF32 ? 32u : 16u;
      store_f16_unit<FMT>(out_v + off + (uint64_t)c * kUnitOut, w);
    }
    __syncthreads();  // the LDS is reused by the caller's next tile group
  } else {
    // Q8_0: both tiles of every head to LDS as stored, then each output unit from there.
    for (uint32_t i = threadIdx.x; i < (uint32_t)(S::kHpw * 2 * S::kUnits); i += 256u) {
      const uint32_t hl = i / (2u * S::kUnits), r = i % (2u * S::kUnits);
      const uint32_t kv = r / S::kUnits, un = r % S::kUnits;
      const uint32_t h = h0 + hl;
      if (blk_ok && h < g.n_kv_heads)
        *(uint4*)&lds.q[GatherQ8Lds<D, FMT>::off(hl, kv, un * 16u)] =
            *(const uint4*)(tile_ptr(g, (uint64_t)blk, layer, kv, h) + (uint64_t)un * 16u);
    }
    __syncthreads();
    if (blk_ok) {
      if constexpr (FMT == kFmtRaw) {
        // Ferrum's 34-byte blocks (dtype.rs:19-21: f16 scale, then 32 x i8), in two
        // passes. First each output record is built in LDS: a step is one block b of 4
        // consecutive tokens 4q .. 4q + 3 of one tile, whose quants come from the staged
        // tile as whole dwords (K: 8 bytes of a token's run at a time; V: a dword holds
        // the 4 tokens' bytes of one dim, transposed by byte permutes), written as dwords
        // plus one 2-byte store (the scale or the last two quants, by b's parity: blocks
        // start 34 bytes apart, records 4-byte aligned). Then the records go out as
        // whole 16-byte units: a token's heads of the workgroup are one contiguous span
        // of its output row (written directly, the 4-byte stores of 64 lanes fell on as
        // many scattered blocks).
        // Wave 0 takes the V blocks (64 items: head, token quad, block; a quad's 4 tokens
        // share each dword read), waves 1-3 the K blocks (256 items: head, token, block),
        // so no wave runs both paths and all four work (kHpw x kNb = 16 at head_dim 64
        // and 128 alike).
        constexpr uint32_t kNb = D / 32u;
        static_assert(S::kHpw * kNb == 16, "64 V and 256 K items");
        using Q = GatherQ8Lds<D, FMT>;
        // byte b of a tile (the padding is inserted between 256-byte spans, and no read
        // below crosses one)
        auto tb = [](uint32_t b) { return Q::kPad ? b + (b >> 8) * 16u : b; };
        // one 34-byte block of token o from its quant dwords qw and its scale
        auto put = [&](uint32_t kv, uint32_t o, uint32_t hl, uint32_t b, const uint32_t (&qw)[8],
                       uint32_t sc) {
          uint8_t* dst = lds.rec_at(kv, o, hl * (uint32_t)kHeadBytes + b * 34u);
          if (b % 2u) {  // the block starts 2 mod 4: scale, then the quants on dword bounds
            *(uint16_t*)dst = (uint16_t)sc;
#pragma unroll
            for (uint32_t k = 0; k < 8; k++) *(uint32_t*)(dst + 2 + 4 * k) = qw[k];
          } else {  // on a dword bound: scale and two quants, then quants two bytes on
            *(uint32_t*)dst = sc | (qw[0] << 16);
#pragma unroll
            for (uint32_t k = 1; k < 8; k++)
              *(uint32_t*)(dst + 4 * k) = (qw[k - 1] >> 16) | (qw[k] << 16);
            *(uint16_t*)(dst + 32) = (uint16_t)(qw[7] >> 16);
          }
        };
        if (threadIdx.x < 64u) {
          const uint32_t hl = threadIdx.x / (4u * kNb), q = (threadIdx.x / kNb) % 4u,
                         b = threadIdx.x % kNb;
          if (h0 + hl < g.n_kv_heads && (int32_t)(4u * q) < n) {
            const uint8_t* t = lds.q + Q::off(hl, 1u, 0u);
            uint32_t qw[4][8];  // [token][quant dword]
#pragma unroll
            for (uint32_t k = 0; k < 8; k++) {  // dims b*32 + 4k .. 4k + 3: m = 2b + k/4
              const uint32_t m = 2u * b + k / 4u, j0 = (k % 4u) * 4u;
              uint32_t w[4];
#pragma unroll
              for (uint32_t jj = 0; jj < 4; jj++)
                w[jj] = *(const uint32_t*)&t[tb((m / 4u) * 1024u + (q * 16u + j0 + jj) * 16u + (m % 4u) * 4u)];
              // 4 x 4 byte transpose: token tt's bytes of dims 4k .. 4k + 3
              const uint32_t lo01 = __builtin_amdgcn_perm(w[1], w[0], 0x05010400u);
              const uint32_t hi01 = __builtin_amdgcn_perm(w[1], w[0], 0x07030602u);
              const uint32_t lo23 = __builtin_amdgcn_perm(w[3], w[2], 0x05010400u);
              const uint32_t hi23 = __builtin_amdgcn_perm(w[3], w[2], 0x07030602u);
              qw[0][k] = __builtin_amdgcn_perm(lo23, lo01, 0x05040100u);
              qw[1][k] = __builtin_amdgcn_perm(lo23, lo01, 0x07060302u);
              qw[2][k] = __builtin_amdgcn_perm(hi23, hi01, 0x05040100u);
              qw[3][k] = __builtin_amdgcn_perm(hi23, hi01, 0x07060302u);
            }
#pragma unroll
            for (uint32_t tt = 0; tt < 4; tt++) {
              const uint32_t o = 4u * q + tt;
              if ((int32_t)o >= n) break;
              put(1u, o, hl, b, qw[tt], *(const uint16_t*)&t[tb(16u * D + (o * kNb + b) * 2u)]);
            }
          }
        } else {
          for (uint32_t i = threadIdx.x - 64u; i < 16u * 16u; i += 192u) {
            const uint32_t hl = i / (16u * kNb), o = (i / kNb) % 16u, b = i % kNb;
            if (h0 + hl >= g.n_kv_heads || (int32_t)o >= n) continue;
            const uint8_t* t = lds.q + Q::off(hl, 0u, 0u);
            uint32_t qw[8];
#pragma unroll
            for (uint32_t gg = 0; gg < 4; gg++) {  // dims b*32 + gg*8 .. +7
              const uint2 w = *(const uint2*)&t[tb((b / 2u) * 1024u + (gg * 16u + o) * 16u + (b % 2u) * 8u)];
              qw[2 * gg] = w.x;
              qw[2 * gg + 1] = w.y;
            }
            put(0u, o, hl, b, qw, *(const uint16_t*)&t[tb(16u * D + (o * kNb + b) * 2u)]);
          }
        }
        __syncthreads();
        // The span of the group's heads that exist, at h0 * kHeadBytes = a multiple of 544
        // bytes into the row: whole 16-byte units where the rows keep that alignment,
        // dwords otherwise (records are dword multiples).
        const uint32_t nh = g.n_kv_heads - h0 < (uint32_t)S::kHpw ? g.n_kv_heads - h0 : (uint32_t)S::kHpw;
        const uint32_t span = nh * (uint32_t)kHeadBytes;
        const uint64_t col0 = (uint64_t)h0 * kHeadBytes;
        if (span % 16u == 0 && row_bytes % 16u == 0) {
          const uint32_t per = span / 16u;
          for (uint32_t i = threadIdx.x; i < 2u * (uint32_t)n * per; i += 256u) {
            const uint32_t kv = i / ((uint32_t)n * per), r = i % ((uint32_t)n * per);
            const uint32_t o = r / per, u = r % per;
            *(uint4*)((kv ? out_v : out_k) + (row0 + o) * row_bytes + col0 + u * 16u) =
                *(const uint4*)lds.rec_at(kv, o, u * 16u);
          }
        } else {
          const uint32_t per = span / 4u;
          for (uint32_t i = threadIdx.x; i < 2u * (uint32_t)n * per; i += 256u) {
            const uint32_t kv = i / ((uint32_t)n * per), r = i % ((uint32_t)n * per);
            const uint32_t o = r / per, u = r % per;
            *(uint32_t*)((kv ? out_v : out_k) + (row0 + o) * row_bytes + col0 + u * 4u) =
                *(const uint32_t*)lds.rec_at(kv, o, u * 4u);
          }
        }
      } else {
        // f16_to_f32(scale) * (i8 as f32), scalar.rs:268-275: 8 dims a step
        constexpr uint32_t kPer = 2u * 16u * (D / 8u);
        for (uint32_t i = threadIdx.x; i < (uint32_t)S::kHpw * kPer; i += 256u) {
          const uint32_t hl = i / kPer, r = i % kPer;
          const uint32_t kv = r / (16u * (D / 8u)), o = (r / (D / 8u)) % 16u, c8 = r % (D / 8u);
          const uint32_t h = h0 + hl;
          if (h >= g.n_kv_heads || (int32_t)o >= n) continue;
          const uint8_t* t = lds.q + GatherQ8Lds<D, FMT>::off(hl, kv, 0u);  // unpadded
          const float sc =
              f16_bits_to_f32(*(const uint16_t*)&t[16u * D + (o * (D / 32u) + c8 / 4u) * 2u]);
          float x[8];
#pragma unroll
          for (uint32_t e = 0; e < 8; e++)
            x[e] = sc * (float)(int8_t)t[q8_quant_offset(kv, o, c8 * 8u + e, D)];
          float4* dst = (float4*)((kv ? out_v : out_k) + (row0 + o) * row_bytes +
                                  (uint64_t)h * kHeadBytes + c8 * 32u);
          dst[0] = make_float4(x[0], x[1], x[2], x[3]);
          dst[1] = make_float4(x[4], x[5], x[6], x[7]);
        }
      }
    }
    __syncthreads();
  }
}

// By block table: workgroup (x, y) takes sequence y, block x / head_groups of its table
// (positions 16j .. 16j + 15, clamped to the context), head group x % head_groups.
template <int DT, int D, int FMT>
__global__ void __launch_bounds__(256) gather_tables_tile_kernel(
    Geom g, uint32_t layer, const int32_t* __restrict__ tables, uint32_t max_blocks,
    const int32_t* __restrict__ ctx_lens, const int64_t* __restrict__ out_offsets,
    uint8_t* out_k, uint8_t* out_v) {
  using S = GatherShape<DT, D>;
  __shared__ GatherLds<DT, D, FMT> lds;
  const uint32_t hgroups = (g.n_kv_heads + S::kHpw - 1) / S::kHpw;
  const uint32_t seq = blockIdx.y, j = blockIdx.x / hgroups, hg = blockIdx.x % hgroups;
  int32_t ctx = ctx_lens[seq];
  const int32_t cap = (int32_t)(max_blocks * 16u);
  if (ctx < 0 || ctx > cap) {
    if (blockIdx.x == 0 && threadIdx.x == 0) raise_fault(g.fault, kFaultCtx);
    ctx = ctx < 0 ? 0 : cap;
  }
  const int32_t n = ctx - (int32_t)j * 16 < 16 ? ctx - (int32_t)j * 16 : 16;
  if (n <= 0) return;  // uniform over the workgroup
  const int32_t blk = tables[(uint64_t)seq * max_blocks + j];
  if ((blk < 0 || (uint64_t)blk >= g.num_blocks) && hg == 0 && threadIdx.x == 0)
    raise_fault(g.fault, kFaultBlock);
  gather_tile<DT, D, FMT>(lds, g, layer, blk, hg * S::kHpw, n, out_k, out_v,
                          (uint64_t)(out_offsets[seq] + (int64_t)j * 16));
}

// By slot: workgroup x takes input tokens 16w .. 16w + 15 (w = x / head_groups). When
// they are the 16 slots of one block in order (a sequence read block by block) they go
// through the tile path; any other window (a partial or scattered one) takes the
// per-chunk path of gather_slots_kernel for its tokens.
template <int DT, int D, int FMT>
__global__ void __launch_bounds__(256) gather_slots_tile_kernel(
    Geom g, uint32_t layer, const int64_t* __restrict__ slots, uint32_t n_tokens,
    uint8_t* out_k, uint8_t* out_v) {
  using S = GatherShape<DT, D>;
  __shared__ GatherLds<DT, D, FMT> lds;
  __shared__ int32_t s_whole;
  const uint32_t hgroups = (g.n_kv_heads + S::kHpw - 1) / S::kHpw;
  const uint32_t win = blockIdx.x / hgroups, hg = blockIdx.x % hgroups;
  const uint64_t t0 = (uint64_t)win * 16u;
  const uint64_t cap = g.num_blocks * 16u;
  if (threadIdx.x == 0) s_whole = 1;
  __syncthreads();
  if (threadIdx.x < 16) {
    const uint64_t t = t0 + threadIdx.x;
    const int64_t sl = t < n_tokens ? slots[t] : -1;
    const int64_t s0 = t0 < n_tokens ? slots[t0] : -1;
    if (sl < 0 || (uint64_t)sl >= cap || s0 < 0 || s0 % 16 != 0 || sl != s0 + (int64_t)threadIdx.x)
      s_whole = 0;
  }
  __syncthreads();
  if (s_whole) {
    gather_tile<DT, D, FMT>(lds, g, layer, slots[t0] / 16, hg * S::kHpw, 16, out_k, out_v, t0);
    return;
  }
  constexpr uint32_t kCv = DT == kDtypeQ8 ? 32u : 8u;  // values per chunk
  constexpr uint32_t kCpr = D / kCv;
  constexpr uint64_t kHeadBytes = FMT == kFmtF32 ? (uint64_t)D * 4u
                                  : DT == kDtypeF16      ? (uint64_t)D * 2u
                                                         : (uint64_t)D / 32u * 34u;
  const uint32_t units = 16u * 2u * S::kHpw * kCpr;
  for (uint32_t i = threadIdx.x; i < units; i += 256u) {
    const uint32_t o = i / (2u * S::kHpw * kCpr), r = i % (2u * S::kHpw * kCpr);
    const uint32_t kv = r / (S::kHpw * kCpr), hl = (r / kCpr) % S::kHpw, c = r % kCpr;
    const uint32_t h = hg * S::kHpw + hl;
    const uint64_t t = t0 + o;
    if (t >= n_tokens || h >= g.n_kv_heads) continue;
    const int64_t slot = slots[t];
    if (slot < 0) continue;
    if ((uint64_t)slot >= cap) {
      if (hg == 0 && r == 0) raise_fault(g.fault, kFaultSlot);
      continue;
    }
    uint8_t* row = (kv ? out_v : out_k) + (t * g.n_kv_heads + h) * kHeadBytes;
    gather_chunk(g, layer, (uint64_t)slot / 16u, (uint32_t)((uint64_t)slot % 16u), kv, h, c, FMT,
                 row, true);
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
    if (ch == 0 && threadIdx.x == 0) {  // the block's mark goes with its bytes
      const uint32_t m = g.bmark[src] ? 1u : 0u;
      const uint32_t old = atomicExch(g.bmark + dst, m);
      if (m != (old ? 1u : 0u)) atomicAdd(g.fault + 1, m ? 1u : 0xffffffffu);
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

// Every device block's mark = m, and the count of marked blocks with it.
__global__ void __launch_bounds__(256) marks_fill_kernel(Geom g, uint32_t m) {
  for (uint64_t b = (uint64_t)blockIdx.x * 256u + threadIdx.x; b < g.num_blocks;
       b += (uint64_t)gridDim.x * 256u)
    g.bmark[b] = m;
  if (blockIdx.x == 0 && threadIdx.x == 0) g.fault[1] = m ? (uint32_t)g.num_blocks : 0u;
}

// swap_out (out): host block p.host[i] takes device block p.dev[i]'s mark; swap_in: the
// reverse, keeping the count of marked device blocks.
__global__ void __launch_bounds__(256) marks_swap_kernel(Geom g, MarkPairs p, bool out) {
  const uint32_t i = threadIdx.x;
  if (i >= p.n) return;
  if (out) {
    g.hmark[p.host[i]] = g.bmark[p.dev[i]] ? 1u : 0u;
  } else {
    const uint32_t m = g.hmark[p.host[i]] ? 1u : 0u;
    const uint32_t old = atomicExch(g.bmark + p.dev[i], m);
    if (m != (old ? 1u : 0u)) atomicAdd(g.fault + 1, m ? 1u : 0xffffffffu);
  }
}

__global__ void __launch_bounds__(256) marks_apply_kernel(Geom g, uint64_t first, uint64_t n,
                                                          const uint8_t* __restrict__ ops) {
  for (uint64_t i = (uint64_t)blockIdx.x * 256u + threadIdx.x; i < n;
       i += (uint64_t)gridDim.x * 256u) {
    if (ops[i] == 0) continue;
    const uint32_t m = ops[i] == 1 ? 1u : 0u;
    const uint32_t old = atomicExch(g.bmark + first + i, m);
    if (m != (old ? 1u : 0u)) atomicAdd(g.fault + 1, m ? 1u : 0xffffffffu);
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
  if (g.dtype == kDtypeQ8 && (g.head_dim == 64 || g.head_dim == 128) && aligned) {
    const uint32_t hpw = g.head_dim == 128 ? 4u : 8u;
    const uint64_t wgs = ((uint64_t)n_tokens + 15u) / 16u * ((g.n_kv_heads + hpw - 1) / hpw);
    if (wgs > 0x7fffffffull) return hipErrorInvalidValue;
    if (g.head_dim == 128)
      append_q8_tile_kernel<128><<<(uint32_t)wgs, 256, 0, s>>>(g, layer, k, v, slots, n_tokens);
    else
      append_q8_tile_kernel<64><<<(uint32_t)wgs, 256, 0, s>>>(g, layer, k, v, slots, n_tokens);
  } else if (g.dtype == kDtypeQ8) {
    uint64_t units = (uint64_t)n_tokens * 2u * g.n_kv_heads * (g.head_dim / 32u);
    if (aligned)
      append_q8_kernel<true><<<grid_for(units), 256, 0, s>>>(g, layer, k, v, slots, n_tokens);
    else
      append_q8_kernel<false><<<grid_for(units), 256, 0, s>>>(g, layer, k, v, slots, n_tokens);
  } else if (g.dtype == kDtypeF16 && g.block_size == 16 && (g.head_dim == 64 || g.head_dim == 128) &&
             aligned) {
    const uint32_t hpw = gather_heads_per_wg(g.dtype, g.head_dim);
    const uint64_t wgs = ((uint64_t)n_tokens + 15u) / 16u * ((g.n_kv_heads + hpw - 1) / hpw);
    if (wgs > 0x7fffffffull) return hipErrorInvalidValue;
    if (g.head_dim == 128)
      append_f16_tile_kernel<128><<<(uint32_t)wgs, 256, 0, s>>>(g, layer, k, v, slots, n_tokens);
    else
      append_f16_tile_kernel<64><<<(uint32_t)wgs, 256, 0, s>>>(g, layer, k, v, slots, n_tokens);
  } else if (g.dtype == kDtypeF16 && g.head_dim % 16 == 0 && aligned) {
    const uint64_t k_threads = (uint64_t)n_tokens * g.n_kv_heads * (g.head_dim / 8u);
    const uint64_t v_waves =
        ((uint64_t)n_tokens + 15u) / 16u * g.n_kv_heads * (g.head_dim / 16u);
    const uint64_t k_groups = (k_threads + 255u) / 256u, v_groups = (v_waves + 3u) / 4u;
    if (k_groups + v_groups > 0x7fffffffull) return hipErrorInvalidValue;
    append_f16_kernel<<<(uint32_t)(k_groups + v_groups), 256, 0, s>>>(g, layer, k, v, slots,
                                                                      n_tokens, (uint32_t)k_groups);
  } else if (g.dtype == kDtypeF32 && g.head_dim % 8 == 0 && aligned) {
    uint64_t units = (uint64_t)n_tokens * 2u * g.n_kv_heads * (g.head_dim / 8u);
    append_f32_kernel<<<grid_for(units), 256, 0, s>>>(g, layer, k, v, slots, n_tokens);
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
    const uint64_t off = (uint64_t)slot % g.block_size;
    uint64_t idx = off * D + d;
    uint8_t* o = kv ? out_v : out_k;
    uint64_t oi = (uint64_t)token * per_kv + e;
    if (g.dtype == kDtypeF16) {
      uint16_t bits = ((const uint16_t*)tile)[kv ? (uint64_t)d * g.block_size + off
                                                 : ((uint64_t)(d / 8) * g.block_size + off) * 8 + d % 8];
      if (format == 0) ((float*)o)[oi] = f16_bits_to_f32(bits);
      else ((uint16_t*)o)[oi] = bits;
    } else {
      ((float*)o)[oi] = ((const float*)tile)[idx];
    }
  }
}

// The tile path's shapes: F16 or Q8_0, block size 16, head_dim 64 or 128, 16-byte
// aligned outputs.
static bool gather_tile_ok(const Geom& g, const void* out_k, const void* out_v) {
  return (g.dtype == kDtypeF16 || g.dtype == kDtypeQ8) && g.block_size == 16 &&
         (g.head_dim == 64 || g.head_dim == 128) && (uintptr_t)out_k % 16 == 0 &&
         (uintptr_t)out_v % 16 == 0;
}

#define FKV_GATHER_TILE_DISPATCH(KERNEL, GRID, ...)                                    \
  do {                                                                                  \
    const bool raw = format == kFmtRaw;                                                 \
    if (g.dtype == kDtypeF16 && g.head_dim == 128) {                                    \
      if (raw) KERNEL<kDtypeF16, 128, kFmtRaw><<<GRID, 256, 0, s>>>(__VA_ARGS__);       \
      else KERNEL<kDtypeF16, 128, kFmtF32><<<GRID, 256, 0, s>>>(__VA_ARGS__);           \
    } else if (g.dtype == kDtypeF16) {                                                  \
      if (raw) KERNEL<kDtypeF16, 64, kFmtRaw><<<GRID, 256, 0, s>>>(__VA_ARGS__);        \
      else KERNEL<kDtypeF16, 64, kFmtF32><<<GRID, 256, 0, s>>>(__VA_ARGS__);            \
    } else if (g.head_dim == 128) {                                                     \
      if (raw) KERNEL<kDtypeQ8, 128, kFmtRaw><<<GRID, 256, 0, s>>>(__VA_ARGS__);        \
      else KERNEL<kDtypeQ8, 128, kFmtF32><<<GRID, 256, 0, s>>>(__VA_ARGS__);            \
    } else {                                                                            \
      if (raw) KERNEL<kDtypeQ8, 64, kFmtRaw><<<GRID, 256, 0, s>>>(__VA_ARGS__);         \
      else KERNEL<kDtypeQ8, 64, kFmtF32><<<GRID, 256, 0, s>>>(__VA_ARGS__);             \
    }                                                                                   \
  } while (0)

hipError_t launch_gather_slots(const Geom& g, uint32_t layer, const int64_t* slots,
                               uint32_t n_tokens, int format, void* out_k, void* out_v,
                               hipStream_t s) {
  if (n_tokens == 0) return hipSuccess;
  if (gather_tile_ok(g, out_k, out_v)) {
    const uint32_t hpw = gather_heads_per_wg(g.dtype, g.head_dim);
    const uint64_t wgs = ((uint64_t)n_tokens + 15u) / 16u * ((g.n_kv_heads + hpw - 1) / hpw);
    if (wgs > 0x7fffffffull) return hipErrorInvalidValue;
    const dim3 grid((uint32_t)wgs);
    FKV_GATHER_TILE_DISPATCH(gather_slots_tile_kernel, grid, g, layer, slots, n_tokens,
                             (uint8_t*)out_k, (uint8_t*)out_v);
    return hipGetLastError();
  }
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
  if (gather_tile_ok(g, out_k, out_v)) {
    const uint32_t hpw = gather_heads_per_wg(g.dtype, g.head_dim);
    const uint64_t wgs = ((uint64_t)max_ctx_len + 15u) / 16u * ((g.n_kv_heads + hpw - 1) / hpw);
    if (wgs > 0x7fffffffull) return hipErrorInvalidValue;
    const dim3 grid((uint32_t)wgs, n_seqs);
    FKV_GATHER_TILE_DISPATCH(gather_tables_tile_kernel, grid, g, layer, tables, max_blocks,
                             ctx_lens, out_offsets, (uint8_t*)out_k, (uint8_t*)out_v);
    return hipGetLastError();
  }
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

// Moves the FKV_FAULT_* word into the staging word fault[3] and clears it in one
// atomic exchange, so a bit that a kernel on another stream raises meanwhile is kept
// for the next read.
__global__ void take_fault_kernel(uint32_t* fault) {
  if (threadIdx.x == 0) fault[3] = atomicExch(fault, 0u);
}

hipError_t launch_take_fault(uint32_t* fault, hipStream_t s) {
  take_fault_kernel<<<1, 64, 0, s>>>(fault);
  return hipGetLastError();
}

hipError_t launch_fill(void* dst, uint8_t byte, uint64_t bytes, hipStream_t s) {
  if (bytes == 0) return hipSuccess;
  uint32_t word = 0x01010101u * byte;
  fill_kernel<<<grid_for(bytes / 16 + 1, 16384), 256, 0, s>>>((uint8_t*)dst, word, bytes);
  return hipGetLastError();
}

hipError_t launch_marks_fill(const Geom& g, uint32_t mark, hipStream_t s) {
  marks_fill_kernel<<<grid_for(g.num_blocks, 1024), 256, 0, s>>>(g, mark ? 1u : 0u);
  return hipGetLastError();
}

hipError_t launch_marks_swap(const Geom& g, const MarkPairs& p, bool out, hipStream_t s) {
  if (p.n == 0) return hipSuccess;
  if (p.n > kMarkPairs) return hipErrorInvalidValue;
  marks_swap_kernel<<<1, 256, 0, s>>>(g, p, out);
  return hipGetLastError();
}

hipError_t launch_marks_apply(const Geom& g, uint64_t first, uint64_t n, const uint8_t* ops,
                              hipStream_t s) {
  if (n == 0) return hipSuccess;
  marks_apply_kernel<<<grid_for(n, 1024), 256, 0, s>>>(g, first, n, ops);
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

}  // namespace fkv
