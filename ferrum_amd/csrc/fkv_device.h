// Device-side helpers shared by the HIP kernels of libferrum_kv.so (gfx950).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "fkv_internal.h"

namespace fkv {
namespace dev {

constexpr float kLog2e = 1.4426950408889634f;

__device__ __forceinline__ uint8_t* tile_ptr(const Geom& g, uint64_t block, uint32_t layer,
                                             uint32_t kv, uint32_t head) {
  return g.base + block * g.block_bytes +
         ((uint64_t)(layer * 2u + kv) * g.n_kv_heads + head) * g.tile_bytes;
}

// The largest context a split-attention launch can hold: the block table's capacity and
// the max_parts partitions of part_tokens its grid and workspace were sized for (from the
// caller's max_ctx_len). A longer context is an input fault: every kernel of the launch
// clamps to the same bound, so none reads another head's partitions or past the workspace.
__device__ __forceinline__ int32_t split_ctx_cap(uint32_t max_blocks, uint32_t block,
                                                 uint32_t max_parts, uint32_t part_tokens) {
  const uint64_t a = (uint64_t)max_blocks * block, b = (uint64_t)max_parts * part_tokens;
  const uint64_t c = a < b ? a : b;
  return (int32_t)(c < 0x7fffffffull ? c : 0x7fffffffull);
}

__device__ __forceinline__ void raise_fault(uint32_t* f, uint32_t bit) {
  atomicOr(f, bit);
}

// Q8_0 scales of 512 or more (binary16 exponent bits 14 and 13 set: 512 <= |s|,
// inf, NaN): scale x quant of such a block can pass 65504, the binary16 range of the
// fast attention operands.
__device__ __forceinline__ bool q8_wide_scale(uint32_t bits) { return (bits & 0x6000u) == 0x6000u; }
// F16 values the fast chunked-prefill instance cannot take: it lets 0 x NaN reach
// queries whose causal end lies before such a V, and scores an infinite K against q's
// lo part (inf x 0).
__device__ __forceinline__ bool f16_nonfinite(uint32_t bits) { return (bits & 0x7c00u) == 0x7c00u; }
// either binary16 of a packed pair
__device__ __forceinline__ bool f16x2_nonfinite(uint32_t w) {
  return f16_nonfinite(w & 0xffffu) || f16_nonfinite(w >> 16);
}

// Block marks. A store of such a value (Q8_0: a wide scale; F16: an Inf/NaN K or V)
// marks its block; the pool's second fault word counts the marked blocks. A mark
// stays with the block's bytes: copy_blocks copies it, swap carries it through the
// host block's mark, fill and whole-block writes replace it; nothing else clears it.
// Attention launches a fast instance and the exact (Q8_0) or leak-safe (F16) one
// after it. While no block is marked (the count is 0) the fast instance computes
// everything and the other leaves at once; otherwise every workgroup of both ORs the
// marks of the blocks it reads, and the instance that can take them computes.
__device__ __forceinline__ void mark_block(const Geom& g, uint64_t block) {
  uint32_t* m = g.bmark + block;
  if (__atomic_load_n(m, __ATOMIC_RELAXED) == 0u && atomicExch(m, 1u) == 0u)
    atomicAdd(g.fault + 1, 1u);
}
// Marks the block of table entry j (the caller has checked j against the table row;
// an entry outside the pool marks nothing: the kernels fault it).
__device__ __forceinline__ void mark_table_block(const Geom& g, const int32_t* table, int32_t j) {
  const int32_t p = table[j];
  if (p >= 0 && (uint64_t)p < g.num_blocks) mark_block(g, (uint64_t)p);
}
__device__ __forceinline__ bool pool_has_marks(const Geom& g) {
  return __builtin_amdgcn_readfirstlane(__atomic_load_n(g.fault + 1, __ATOMIC_RELAXED)) != 0;
}
// Whether any block of table entries [j0, j1) is marked (entries outside the pool are
// skipped: the kernels fault them). Every thread of the workgroup calls it and gets
// the same answer.
__device__ __forceinline__ bool blocks_marked(const Geom& g, const int32_t* __restrict__ table,
                                              int32_t j0, int32_t j1) {
  uint32_t m = 0;
  for (int32_t j = j0 + (int32_t)threadIdx.x; j < j1; j += (int32_t)blockDim.x) {
    const int32_t p = table[j];
    if (p >= 0 && (uint64_t)p < g.num_blocks) m |= g.bmark[p];
  }
  return __syncthreads_or(m != 0u) != 0;
}

// 16-byte load of K/V bytes that are read once per launch: the nontemporal hint
// keeps the stream from evicting reusable lines (block tables, q) and measured
// 7.1 TB/s against 6.3 TB/s for plain loads in a read-only sweep on MI355X.
typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint4 load_stream16(const uint8_t* p) {
  const u32x4_t v = __builtin_nontemporal_load((const u32x4_t*)p);
  return make_uint4(v.x, v.y, v.z, v.w);
}

// Byte offset of the int8 quant of (token off, dim d) in a Q8_0 tile of kind kv.
// Quants come in 16-token sub-tiles of 16*D bytes, in the operand order of the
// matrix-core attention (each lane's 32 bytes of a block contiguous, 1 KiB per
// load instruction); with t = off % 16:
//   K: d = c*32 + g*8 + e -> (c/2)*1024 + (g*16 + t)*16 + (c%2)*8 + e
//   V: d = m*16 + j, t = q*4 + r -> (m/4)*1024 + (q*16 + j)*16 + (m%4)*4 + r
// (pools need D % 64 == 0 and B % 16 == 0). The f16 scales [B][D/32] follow.
__device__ __forceinline__ uint64_t q8_quant_offset(uint32_t kv, uint32_t off, uint32_t d,
                                                    uint32_t D) {
  const uint64_t sub = (uint64_t)(off / 16u) * 16u * D;
  const uint32_t t = off % 16u;
  if (kv) {
    const uint32_t m = d / 16u, j = d % 16u;
    return sub + (uint64_t)(m / 4u) * 1024u + (uint64_t)((t / 4u) * 16u + j) * 16u +
           (m % 4u) * 4u + t % 4u;
  }
  const uint32_t c = d / 32u, g = (d % 32u) / 8u;
  return sub + (uint64_t)(c / 2u) * 1024u + (uint64_t)(g * 16u + t) * 16u + (c % 2u) * 8u +
         d % 8u;
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
// Q8_0 quantiser steps (crates/kernels/src/q8_dot.rs:46-59)
// ---------------------------------------------------------------------------

// Rust's f32::round: half away from zero.
__device__ __forceinline__ float round_half_away(float y) {
  float t = __builtin_truncf(y);
  return (__builtin_fabsf(y - t) >= 0.5f) ? t + __builtin_copysignf(1.0f, y) : t;
}

// d = amax / 127 and id = 1 / d (0 when d is 0), both in f32.
__device__ __forceinline__ float q8_scale(float amax, float& id) {
  const float d = amax / 127.0f;
  id = (d != 0.0f) ? 1.0f / d : 0.0f;
  return d;
}

// round(x * id) as Rust's `as i32` takes it (saturating, NaN -> 0), clamped to
// [-128, 127].
__device__ __forceinline__ int q8_quant(float x, float id) {
  const float r = round_half_away(x * id);
  return (r != r) ? 0 : (r >= 127.0f ? 127 : (r <= -128.0f ? -128 : (int)r));
}

}  // namespace dev
}  // namespace fkv
