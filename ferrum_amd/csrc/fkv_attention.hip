// Paged decode attention for gfx950: the attention loop of
// Llama::forward_one_token (crates/model/src/llama.rs:220-247) over K/V read
// through block tables, with the softmax of crates/kernels/src/scalar.rs:125-141
// (a non-finite maximum gives zeros).
//
// This file holds the VALU kernels and the dispatch:
//   Q8_0 storage   attn_split_kernel (G <= 8), dequantising inside the dot products
//   F32 storage    attn_partition_kernel (G in {1, 2, 4, 8, 16})
//   F16 storage    the MFMA kernels of fkv_attention_mfma.hip
// and attn_combine_kernel, which merges split partials for all of them.
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include <type_traits>

// Blocks per range of the split kernel: 2 (16 KiB of K+V in flight per wave)
// leaves room for two or three waves per SIMD; measured faster than 4.
#ifndef FKV_SPLIT_RANGE_BLOCKS
#define FKV_SPLIT_RANGE_BLOCKS 2
#endif

#include "fkv_device.h"
#include "fkv_internal.h"

namespace fkv {
namespace {

using namespace dev;

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
  if constexpr (DT == kDtypeF32) {
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
        kreg[j][ps] = load_stream16(kt + row * row_bytes + c * 16);
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
          vreg[j][ps] = load_stream16(vt + row * row_bytes + c * 16);
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
        vl[ps] = load_stream16(vt + row * row_bytes + c * 16);
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
// One wave per (sequence, query head), four per workgroup, no LDS: lane p holds
// partition p's (m, l) (64 partitions per pass), every lane holds D/64 dims, and
// the partial-output loads of a pass are issued before its maximum is known.
// Heads with many partitions (few sequences, long contexts) use
// attn_combine_wide_kernel instead.
template <int D>
__global__ void __launch_bounds__(256) attn_combine_kernel(
    const int32_t* __restrict__ ctx_lens, uint32_t n_seq_heads, uint32_t n_heads,
    uint32_t max_blocks, uint32_t max_parts, int32_t part_tokens,
    const float* __restrict__ ws_o, const float* __restrict__ ws_ml, float* __restrict__ out) {
  constexpr int DPL = D / 64;  // dims per lane
  constexpr int kChunk = 16;   // partial outputs held in registers per step
  const uint32_t head = blockIdx.x * 4 + (threadIdx.x >> 6);  // seq * n_heads + h
  if (head >= n_seq_heads) return;
  const int lane = threadIdx.x & 63;
  const uint32_t seq = head / n_heads;
  const float* ml = ws_ml + (uint64_t)head * max_parts * 2;
  const float* po = ws_o + (uint64_t)head * max_parts * D + lane * DPL;
  // The context length, the first 64 partitions' (m, l) and the first kChunk
  // partial outputs are loaded together: slots past the head's partition count
  // hold stale bytes and are masked once the count is known (the workspace has
  // max_parts slots per head, so every load is in bounds).
  const int32_t raw_ctx = ctx_lens[seq];
  const int32_t n0 = (int32_t)max_parts < 64 ? (int32_t)max_parts : 64;
  float mp = lane < n0 ? ml[2 * lane] : -__builtin_inff();
  float lp = lane < n0 ? ml[2 * lane + 1] : 0.0f;
  float v0[kChunk][DPL];
#pragma unroll
  for (int j = 0; j < kChunk; j++)
#pragma unroll
    for (int i = 0; i < DPL; i++) v0[j][i] = j < (int)max_parts ? po[(uint64_t)j * D + i] : 0.0f;

  const int32_t cap = (int32_t)(max_blocks * kAttnBlock);
  const int32_t ctx = raw_ctx < 0 ? 0 : (raw_ctx > cap ? cap : raw_ctx);
  const int32_t nparts = ctx > 0 ? (ctx + part_tokens - 1) / part_tokens : 1;
  if (nparts == 1) return;
  if (lane >= nparts) {
    mp = -__builtin_inff();
    lp = 0.0f;
  }

  // The global maximum (partitions past the first 64 need more loads).
  float M = mp;
  for (int32_t p0 = 64; p0 < nparts; p0 += 64)
    if (p0 + lane < nparts) M = __builtin_fmaxf(M, ml[2 * (p0 + lane)]);
  M = wave_max(M);
  float* o = out + (uint64_t)head * D + lane * DPL;
  if (!__builtin_isfinite(M)) {
#pragma unroll
    for (int i = 0; i < DPL; i++) o[i] = 0.0f;
    return;
  }
  float acc[DPL];
#pragma unroll
  for (int i = 0; i < DPL; i++) acc[i] = 0.0f;
  float lsum = 0.0f;
  for (int32_t p0 = 0; p0 < nparts; p0 += 64) {
    if (p0 > 0) {
      const bool mine = p0 + lane < nparts;
      mp = mine ? ml[2 * (p0 + lane)] : -__builtin_inff();
      lp = mine ? ml[2 * (p0 + lane) + 1] : 0.0f;
    }
    const float wp = __builtin_amdgcn_exp2f((mp - M) * kLog2e);
    const int32_t n = nparts - p0 < 64 ? nparts - p0 : 64;
    for (int32_t c0 = 0; c0 < n; c0 += kChunk) {
      float v[kChunk][DPL];
      if (p0 == 0 && c0 == 0) {
#pragma unroll
        for (int j = 0; j < kChunk; j++)
#pragma unroll
          for (int i = 0; i < DPL; i++) v[j][i] = v0[j][i];
      } else {
#pragma unroll
        for (int j = 0; j < kChunk; j++)
#pragma unroll
          for (int i = 0; i < DPL; i++)
            v[j][i] = c0 + j < n ? po[(uint64_t)(p0 + c0 + j) * D + i] : 0.0f;
      }
#pragma unroll
      for (int j = 0; j < kChunk; j++) {
        if (c0 + j < n) {
          const float w = __shfl(wp, c0 + j);
          lsum = __builtin_fmaf(w, __shfl(lp, c0 + j), lsum);
#pragma unroll
          for (int i = 0; i < DPL; i++) acc[i] = __builtin_fmaf(w, v[j][i], acc[i]);
        }
      }
    }
  }
  const float inv = 1.0f / lsum;
#pragma unroll
  for (int i = 0; i < DPL; i++) o[i] = acc[i] * inv;
}

// The same merge with one 16-wave workgroup per (sequence, query head): wave w
// takes partitions w, w + 16, ..., each lane D/64 dims, and the waves' (l, o) are
// summed through LDS. For heads with more than kWideParts partitions (few
// sequences with long contexts), where one wave per head would walk hundreds of
// partitions one latency after another.
constexpr uint32_t kWideParts = 32;
constexpr int kWideWaves = 16;
template <int D>
__global__ void __launch_bounds__(64 * kWideWaves) attn_combine_wide_kernel(
    const int32_t* __restrict__ ctx_lens, uint32_t n_heads, uint32_t max_blocks,
    uint32_t max_parts, int32_t part_tokens, const float* __restrict__ ws_o,
    const float* __restrict__ ws_ml, float* __restrict__ out) {
  constexpr int DPL = D / 64;
  constexpr int kUnroll = 8;
  constexpr int W = kWideWaves;
  __shared__ float s_l[W];
  __shared__ float s_acc[W][D];
  const uint32_t head = blockIdx.x;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const uint32_t seq = head / n_heads;
  const int32_t cap = (int32_t)(max_blocks * kAttnBlock);
  int32_t ctx = ctx_lens[seq];
  ctx = ctx < 0 ? 0 : (ctx > cap ? cap : ctx);
  const int32_t nparts = ctx > 0 ? (ctx + part_tokens - 1) / part_tokens : 1;
  if (nparts == 1) return;
  const float* ml = ws_ml + (uint64_t)head * max_parts * 2;
  const float* po = ws_o + (uint64_t)head * max_parts * D + lane * DPL;
  float* o = out + (uint64_t)head * D;

  // maximum over all partitions (every wave computes it; the loads hit in cache)
  float M = -__builtin_inff();
  for (int32_t p = lane; p < nparts; p += 64) M = __builtin_fmaxf(M, ml[2 * p]);
  M = wave_max(M);
  if (!__builtin_isfinite(M)) {
    if (wave == 0)
#pragma unroll
      for (int i = 0; i < DPL; i++) o[lane * DPL + i] = 0.0f;
    return;
  }
  float acc[DPL];
#pragma unroll
  for (int i = 0; i < DPL; i++) acc[i] = 0.0f;
  float lsum = 0.0f;
  for (int32_t p0 = wave; p0 < nparts; p0 += W * kUnroll) {
    float v[kUnroll][DPL], w[kUnroll], l[kUnroll];
#pragma unroll
    for (int j = 0; j < kUnroll; j++) {
      const int32_t p = p0 + W * j;
      const bool ok = p < nparts;
      w[j] = ok ? ml[2 * p] : -__builtin_inff();
      l[j] = ok ? ml[2 * p + 1] : 0.0f;
#pragma unroll
      for (int i = 0; i < DPL; i++) v[j][i] = ok ? po[(uint64_t)p * D + i] : 0.0f;
    }
#pragma unroll
    for (int j = 0; j < kUnroll; j++) {
      if (p0 + W * j < nparts) {
        const float wt = __builtin_amdgcn_exp2f((w[j] - M) * kLog2e);
        lsum = __builtin_fmaf(wt, l[j], lsum);
#pragma unroll
        for (int i = 0; i < DPL; i++) acc[i] = __builtin_fmaf(wt, v[j][i], acc[i]);
      }
    }
  }
#pragma unroll
  for (int i = 0; i < DPL; i++) s_acc[wave][lane * DPL + i] = acc[i];
  if (lane == 0) s_l[wave] = lsum;
  __syncthreads();
  if (threadIdx.x < D) {
    float a = 0.0f, L = 0.0f;
#pragma unroll
    for (int k = 0; k < W; k++) {
      a += s_acc[k][threadIdx.x];
      L += s_l[k];
    }
    o[threadIdx.x] = a * (1.0f / L);
  }
}

// ---------------------------------------------------------------------------
// Split-context streaming kernel (Q8_0 storage, G <= 8)
// ---------------------------------------------------------------------------
//
// Workgroup = 4 waves = one split (split_tokens tokens) of one (sequence, kv
// head); all G query heads of the group share every K/V tile. The split is cut
// into ranges of RB blocks; wave w takes ranges w, w+4, ... and keeps the next
// range's K and V loads in flight while it computes on the current one. Every
// K/V load is unconditional (blocks past the split re-read the range's first
// block), so the compiler's waits cover exactly the loads they need. No barrier
// runs until the final merge.
//
// Per range:
//   QK       lane (r, c) holds EPL dims of token rows r, r+RPP, ... and forms G
//            partial dots per row (v_fma_mix: f16 operands, f32 accumulate);
//            partials go to LDS as T[token][head][c], and the lane that owns
//            (token tq, head h) sums one contiguous row of it.
//   softmax  lazy online softmax in the log2 domain: each quad lane owns heads
//            cq, cq+4, ... and keeps a private partial sum; scores are taken
//            relative to a per-head reference max m_ref, and only when a score
//            exceeds m_ref by 2^8 (any lane, by ballot) does the wave compute
//            the exact running max and rescale l and acc. NaN is skipped by the
//            max and propagates through the weights; a head whose scores are all
//            -inf/NaN keeps m_ref = -inf.
//   PV       row layout, token weights read from LDS.
// At the end the 4 waves merge (m, l, acc) in LDS. A sequence with one split
// writes the output; otherwise each split writes (m, l, o) to the workspace and
// attn_combine_kernel merges the splits. (Merging in the last split to finish
// would need agent-scope release/acquire fences, which on this multi-XCD part
// write back and invalidate L2 once per workgroup; a second launch is cheaper.)

template <int kCtrl>
__device__ __forceinline__ float dppf(float x) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), kCtrl, 0xf, 0xf, true));
}

// Row stride (floats) of the QK transpose buffer T[token][G][LPR]: G*LPR padded
// so that it is congruent to LPR mod 64, which spreads the RPP token rows of one
// ds_write over distinct banks.
template <int G, int LPR>
constexpr int transpose_stride() {
  return G * LPR + (((LPR - G * LPR) % 64) + 64) % 64;
}

constexpr float kRescaleLog2 = 8.0f;  // rescale when a score exceeds m_ref by 2^8

template <int DT, int D, int G, int RB>
__global__ void __launch_bounds__(256) attn_split_kernel(
    Geom g, uint32_t layer, uint32_t n_heads, const float* __restrict__ q,
    float* __restrict__ out, const int32_t* __restrict__ tables, uint32_t max_blocks,
    const int32_t* __restrict__ ctx_lens, uint32_t max_splits, int32_t split_tokens,
    float scale, float* __restrict__ ws_o, float* __restrict__ ws_ml) {
  using S = AttnShape<DT, D>;
  constexpr int EPL = S::EPL, LPR = S::LPR, RPP = S::RPP, PASSES = S::PASSES;
  constexpr int RT = RB * kAttnBlock;               // tokens per range
  constexpr int HPL = G >= 4 ? G / 4 : 1;           // heads owned per quad lane
  constexpr int TST = transpose_stride<G, LPR>();   // transpose row stride
  constexpr int TS = kAttnBlock * TST;              // transpose floats per wave
  static_assert(LPR >= 4 && LPR <= 16, "4..16 lanes per token row");
  static_assert(G * D <= TS, "merge buffer aliases the transpose buffer");

  __shared__ float s_t[kAttnWaves * TS];
  __shared__ float s_p[kAttnWaves][RT * G];
  __shared__ float s_m[kAttnWaves][G];
  __shared__ float s_l[kAttnWaves][G];

  const uint32_t sk = blockIdx.x, split = blockIdx.y;
  const uint32_t seq = sk / g.n_kv_heads, kvh = sk % g.n_kv_heads;
  const int32_t cap = (int32_t)(max_blocks * kAttnBlock);
  int32_t ctx = ctx_lens[seq];
  if (ctx < 0 || ctx > cap) {
    if (split == 0 && threadIdx.x == 0 && kvh == 0) raise_fault(g.fault, kFaultCtx);
    ctx = ctx < 0 ? 0 : cap;
  }
  const int32_t nsplits = ctx > 0 ? (ctx + split_tokens - 1) / split_tokens : 1;
  if ((int32_t)split >= nsplits) return;
  const int32_t s0 = (int32_t)split * split_tokens;
  const int32_t s1 = ctx - s0 < split_tokens ? ctx : s0 + split_tokens;
  const int32_t nranges = s1 > s0 ? (s1 - s0 + RT - 1) / RT : 0;

  // readfirstlane: `wave` and every block index derived from it are known to be
  // wave-uniform, so block-table reads are scalar loads.
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int r = lane / LPR, c = lane % LPR;  // row layout (loads, QK partials, PV)
  const int tq = lane >> 2, cq = lane & 3;   // owner layout (token in block, quad lane)
  float* tw = s_t + wave * TS;
  float* pl = s_p[wave];

  // Scores are kept in the log2 domain: dot * scale * log2(e).
  const float qscale = scale * kLog2e;
  float qr[G][EPL];
  {
    const float* qb = q + ((uint64_t)seq * n_heads + (uint64_t)kvh * G) * D + c * EPL;
#pragma unroll
    for (int gg = 0; gg < G; gg++)
#pragma unroll
      for (int i = 0; i < EPL; i += 4) {
        float4 t = *(const float4*)(qb + (uint64_t)gg * D + i);
        qr[gg][i] = t.x; qr[gg][i + 1] = t.y; qr[gg][i + 2] = t.z; qr[gg][i + 3] = t.w;
      }
  }

  const int32_t* table = tables + (uint64_t)seq * max_blocks;
  const uint64_t row_bytes = (uint64_t)D * S::E;
  const uint64_t scale_off = (uint64_t)kAttnBlock * D;

  float m_ref[HPL], l_part[HPL], acc[G][EPL];
#pragma unroll
  for (int k = 0; k < HPL; k++) {
    m_ref[k] = -__builtin_inff();
    l_part[k] = 0.0f;
  }
#pragma unroll
  for (int gg = 0; gg < G; gg++)
#pragma unroll
    for (int i = 0; i < EPL; i++) acc[gg][i] = 0.0f;
  // Heads this lane owns in the softmax: cq + 4k (G >= 4) or cq (G < 4, lanes
  // cq >= G duplicate head cq % G and contribute nothing).
  const bool owner = (G >= 4) || cq < G;
  auto head_of = [&](int k) { return G >= 4 ? cq + 4 * k : (cq % G); };

  uint4 kr[RB][PASSES], vr[RB][PASSES];
  uint32_t ksc[RB][PASSES], vsc[RB][PASSES];

  auto fetch_ids = [&](int rg, int32_t (&ids)[RB], bool (&live)[RB]) {
    const int32_t b0 = (s0 + rg * RT) / kAttnBlock;
    const int32_t p0 = table[b0];
#pragma unroll
    for (int j = 0; j < RB; j++) {
      const bool v = (b0 + j) * kAttnBlock < s1;
      int32_t p = v ? (j == 0 ? p0 : table[b0 + j]) : p0;
      const bool okb = p >= 0 && (uint64_t)p < g.num_blocks;
      if (v && !okb && lane == 0) raise_fault(g.fault, kFaultBlock);
      live[j] = v && okb;
      ids[j] = okb ? p : 0;
    }
  };
  auto load_kv = [&](int kv, const int32_t (&ids)[RB], uint4 (&reg)[RB][PASSES],
                     uint32_t (&sc)[RB][PASSES]) {
#pragma unroll
    for (int j = 0; j < RB; j++) {
      const uint8_t* t = tile_ptr(g, (uint64_t)ids[j], layer, kv, kvh);
#pragma unroll
      for (int ps = 0; ps < PASSES; ps++) {
        const int row = ps * RPP + r;
        reg[j][ps] = load_stream16(t + row * row_bytes + c * 16);
        if constexpr (DT == kDtypeQ8)
          sc[j][ps] = ((const uint16_t*)(t + scale_off))[row * (D / 32) + (c * EPL) / 32];
      }
    }
  };

  int rg = wave;
  int32_t ids[RB], nids[RB];
  bool live[RB], nlive[RB];

  auto range_body = [&](auto prefetch_tag) {
    constexpr bool kPrefetch = decltype(prefetch_tag)::value;
    if constexpr (kPrefetch) fetch_ids(rg + kAttnWaves, nids, nlive);
    const int32_t rbase = s0 + rg * RT;

    // ---- QK: partial dots -> T[token][head][c] -> owner sums one row.
    float sc[RB][HPL];
#pragma unroll
    for (int j = 0; j < RB; j++) {
#pragma unroll
      for (int ps = 0; ps < PASSES; ps++) {
        float kf[EPL];
        decode16<DT, EPL>(kr[j][ps], kf);
        float* dst = tw + (ps * RPP + r) * TST + c;
#pragma unroll
        for (int gg = 0; gg < G; gg++) {
          float a = 0.0f;
#pragma unroll
          for (int i = 0; i < EPL; i++) a = __builtin_fmaf(qr[gg][i], kf[i], a);
          if constexpr (DT == kDtypeQ8) a *= f16_bits_to_f32(ksc[j][ps]);
          dst[gg * LPR] = a;
        }
      }
      const bool tok_ok = live[j] && rbase + j * kAttnBlock + tq < s1;
#pragma unroll
      for (int k = 0; k < HPL; k++) {
        const float4* src = (const float4*)(tw + tq * TST + head_of(k) * LPR);
        float x = 0.0f;
#pragma unroll
        for (int c4 = 0; c4 < LPR / 4; c4++) {
          const float4 v4 = src[c4];
          x += (v4.x + v4.y) + (v4.z + v4.w);
        }
        sc[j][k] = tok_ok ? x * qscale : -__builtin_inff();  // scale after the dot (llama.rs:231)
      }
    }
    if constexpr (kPrefetch) load_kv(0, nids, kr, ksc);

    // ---- lazy online softmax (log2 domain).
    float lmax[HPL];
    bool bad = false;
#pragma unroll
    for (int k = 0; k < HPL; k++) {
      float x = sc[0][k];
#pragma unroll
      for (int j = 1; j < RB; j++) x = __builtin_fmaxf(x, sc[j][k]);
      lmax[k] = x;
      bad |= !(x <= m_ref[k] + kRescaleLog2) || !__builtin_isfinite(m_ref[k]);
    }
    if (__builtin_amdgcn_ballot_w64(bad) != 0) {
      // Exact running max of every head over this range, then rescale.
#pragma unroll
      for (int k = 0; k < HPL; k++) {
        float x = lmax[k];
        x = __builtin_fmaxf(x, dppf<0x124>(x));  // row_ror:4 (next token, same quad lane)
        x = __builtin_fmaxf(x, dppf<0x128>(x));  // row_ror:8
        x = __builtin_fmaxf(x, __shfl_xor(x, 16));
        x = __builtin_fmaxf(x, __shfl_xor(x, 32));
        const float mn = __builtin_fmaxf(m_ref[k], x);
        const float alpha =
            (mn == -__builtin_inff()) ? 1.0f : __builtin_amdgcn_exp2f(m_ref[k] - mn);
        l_part[k] *= alpha;
        m_ref[k] = mn;
        lmax[k] = alpha;  // reuse: per-lane alpha of head head_of(k)
      }
#pragma unroll
      for (int gg = 0; gg < G; gg++) {
        // alpha of head gg lives in quad lane gg % 4 (slot gg / 4), e.g. lane gg % 4.
        const int src_lane = G >= 4 ? (gg & 3) : gg;
        const float a = __int_as_float(__builtin_amdgcn_readlane(
            __float_as_int(lmax[G >= 4 ? gg / 4 : 0]), src_lane));
#pragma unroll
        for (int i = 0; i < EPL; i++) acc[gg][i] *= a;
      }
    }
#pragma unroll
    for (int k = 0; k < HPL; k++) {
      const float mr = m_ref[k];
      const bool dead = (mr == -__builtin_inff());
#pragma unroll
      for (int j = 0; j < RB; j++) {
        const float sv = sc[j][k];
        const float e = dead ? (sv != sv ? sv : 0.0f) : __builtin_amdgcn_exp2f(sv - mr);
        sc[j][k] = e;
        l_part[k] += e;
      }
    }
    if (owner) {
#pragma unroll
      for (int j = 0; j < RB; j++)
#pragma unroll
        for (int k = 0; k < HPL; k++) pl[(j * kAttnBlock + tq) * G + head_of(k)] = sc[j][k];
    }

    // ---- PV. Rows past the split are skipped: their V bytes may be anything.
#pragma unroll
    for (int j = 0; j < RB; j++) {
      if (!live[j]) continue;
      const bool full = rbase + (j + 1) * kAttnBlock <= s1;
#pragma unroll
      for (int ps = 0; ps < PASSES; ps++) {
        const int t = ps * RPP + r;
        if (full || rbase + j * kAttnBlock + t < s1) {
          float vf[EPL];
          decode16<DT, EPL>(vr[j][ps], vf);
          float pwt[G];
#pragma unroll
          for (int gg = 0; gg < G; gg++) pwt[gg] = pl[(j * kAttnBlock + t) * G + gg];
          if constexpr (DT == kDtypeQ8) {
            const float sv = f16_bits_to_f32(vsc[j][ps]);
#pragma unroll
            for (int gg = 0; gg < G; gg++) pwt[gg] *= sv;
          }
#pragma unroll
          for (int gg = 0; gg < G; gg++)
#pragma unroll
            for (int i = 0; i < EPL; i++) acc[gg][i] = __builtin_fmaf(pwt[gg], vf[i], acc[gg][i]);
        }
      }
    }
    if constexpr (kPrefetch) {
      load_kv(1, nids, vr, vsc);
#pragma unroll
      for (int j = 0; j < RB; j++) {
        ids[j] = nids[j];
        live[j] = nlive[j];
      }
    }
  };

  if (rg < nranges) {
    fetch_ids(rg, ids, live);
    load_kv(0, ids, kr, ksc);
    load_kv(1, ids, vr, vsc);
    for (; rg + kAttnWaves < nranges; rg += kAttnWaves) range_body(std::true_type{});
    range_body(std::false_type{});
  }

  // ---- per wave: l over the 16 owner lanes of each head, acc over token rows.
#pragma unroll
  for (int k = 0; k < HPL; k++) {
    float x = owner ? l_part[k] : 0.0f;
    x += dppf<0x124>(x);
    x += dppf<0x128>(x);
    x += __shfl_xor(x, 16);
    x += __shfl_xor(x, 32);
    l_part[k] = x;
  }
#pragma unroll
  for (int gg = 0; gg < G; gg++)
#pragma unroll
    for (int i = 0; i < EPL; i++) {
      float x = acc[gg][i];
#pragma unroll
      for (int o = LPR; o < 64; o <<= 1) x += __shfl_xor(x, o);
      acc[gg][i] = x;
    }
  __syncthreads();  // every wave is done with its transpose buffer
  float* s_o = s_t;
  if (r == 0) {
#pragma unroll
    for (int gg = 0; gg < G; gg++)
#pragma unroll
      for (int i = 0; i < EPL; i++) s_o[(wave * G + gg) * D + c * EPL + i] = acc[gg][i];
  }
  if (lane < 4 && owner) {
#pragma unroll
    for (int k = 0; k < HPL; k++) {
      s_m[wave][head_of(k)] = m_ref[k];
      s_l[wave][head_of(k)] = l_part[k];
    }
  }
  __syncthreads();

  // ---- merge the 4 waves (m in the log2 domain).
  const uint64_t head0 = (uint64_t)seq * n_heads + (uint64_t)kvh * G;
  for (int e = threadIdx.x; e < G * D; e += 256) {
    const int gg = e / D, d = e % D;
    float M = -__builtin_inff();
#pragma unroll
    for (int w = 0; w < kAttnWaves; w++) M = __builtin_fmaxf(M, s_m[w][gg]);
    float o = 0.0f, L = 0.0f;
#pragma unroll
    for (int w = 0; w < kAttnWaves; w++) {
      const float mw = s_m[w][gg];
      const float wt = (mw == -__builtin_inff()) ? 0.0f : __builtin_amdgcn_exp2f(mw - M);
      o = __builtin_fmaf(wt, s_o[(w * G + gg) * D + d], o);
      L = __builtin_fmaf(wt, s_l[w][gg], L);
    }
    const uint64_t head = head0 + gg;
    if (nsplits == 1) {
      out[head * D + d] = __builtin_isfinite(M) ? o * (1.0f / L) : 0.0f;
    } else {
      ws_o[(head * max_splits + split) * D + d] = o;
      if (d == 0) {
        // natural-log max, as attn_partition_kernel writes it
        ws_ml[(head * max_splits + split) * 2] = M * 0.6931471805599453f;
        ws_ml[(head * max_splits + split) * 2 + 1] = L;
      }
    }
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
  return launch_attention_combine(D, ctx_lens, n_seqs, n_heads, max_blocks, max_parts,
                                  kAttnPartTokens, ws_o, ws_ml, out, s);
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

}  // namespace

bool attention_supported(int dtype, uint32_t head_dim, uint32_t group) {
  if (head_dim != 64 && head_dim != 128) return false;
  if (dtype == kDtypeF16) return group >= 1 && group <= 16;
  if (dtype != kDtypeF32 && dtype != kDtypeQ8) return false;
  if (group == 1 || group == 2 || group == 4 || group == 8) return true;
  return group == 16 && dtype != kDtypeQ8;
}

hipError_t launch_attention_combine(uint32_t head_dim, const int32_t* ctx_lens,
                                    uint32_t n_seqs, uint32_t n_heads, uint32_t max_blocks,
                                    uint32_t max_splits, uint32_t split_tokens,
                                    const float* ws_o, const float* ws_ml, float* out,
                                    hipStream_t s) {
  const uint32_t nh = n_seqs * n_heads, grid = (nh + 3) / 4;
  if (max_splits > kWideParts && nh < 2048) {  // few heads with many splits each
    if (head_dim == 128)
      attn_combine_wide_kernel<128><<<nh, 64 * kWideWaves, 0, s>>>(
          ctx_lens, n_heads, max_blocks, max_splits, (int32_t)split_tokens, ws_o, ws_ml, out);
    else
      attn_combine_wide_kernel<64><<<nh, 64 * kWideWaves, 0, s>>>(
          ctx_lens, n_heads, max_blocks, max_splits, (int32_t)split_tokens, ws_o, ws_ml, out);
    return hipGetLastError();
  }
  if (head_dim == 128)
    attn_combine_kernel<128><<<grid, 256, 0, s>>>(
        ctx_lens, nh, n_heads, max_blocks, max_splits, (int32_t)split_tokens, ws_o, ws_ml, out);
  else
    attn_combine_kernel<64><<<grid, 256, 0, s>>>(
        ctx_lens, nh, n_heads, max_blocks, max_splits, (int32_t)split_tokens, ws_o, ws_ml, out);
  return hipGetLastError();
}

namespace {

// How one decode-attention call is cut up, and where its workspace regions live.
struct AttnPlan {
  bool stream_path = false; // attn_mfma_stream_kernel (F16) + stream combine
  uint32_t stream_waves = 0;
  uint64_t pre_off = 0;
  bool mfma_path = false;   // attn_mfma_kernel (F16) + combine
  bool split_path = false;  // attn_split_kernel (Q8_0) + combine; else attn_partition + combine
  uint32_t split_tokens = kAttnPartTokens;
  uint32_t max_splits = 1;
  uint64_t o_off = 0, ml_off = 0, total = 0;
};

inline uint64_t align256(uint64_t x) { return (x + 255) / 256 * 256; }

// Split length: long enough that the final cross-split merge stays small
// (<= 64 splits per sequence when there are many sequences), short enough that
// the launch has thousands of workgroups: a batch of few sequences may split
// further, up to ~4096 (sequence, KV head, split) workgroups, never below 512
// tokens. FKV_ATTN_SPLIT_TOKENS (a multiple of 16) overrides.
uint32_t choose_split_tokens(uint32_t max_ctx_len, uint32_t n_seqs, uint32_t n_kv_heads) {
  if (const char* e = getenv("FKV_ATTN_SPLIT_TOKENS")) {
    long v = strtol(e, nullptr, 10);
    if (v >= 16 && v % 16 == 0 && v <= (1 << 20)) return (uint32_t)v;
  }
  const uint64_t segs = (uint64_t)n_seqs * (n_kv_heads ? n_kv_heads : 1);
  uint64_t max_splits = segs ? 4096 / segs : 64;
  if (max_splits < 64) max_splits = 64;
  uint64_t st = (((uint64_t)max_ctx_len + max_splits - 1) / max_splits + 255) / 256 * 256;
  if (st < 512) st = 512;
  if (st > 8192) st = 8192;
  return (uint32_t)st;
}

AttnPlan plan_attention(const Geom& g, uint32_t n_heads, uint32_t n_seqs, uint32_t max_ctx_len) {
  AttnPlan p;
  const uint32_t G = g.n_kv_heads ? n_heads / g.n_kv_heads : 0;
  const char* mode = getenv("FKV_ATTN_MODE");
  // F16: the split kernel by default; FKV_ATTN_MODE=stream selects the persistent one.
  if (g.dtype == kDtypeF16 && G >= 1 && G <= 16 && stream_attention_supported(n_seqs) && mode &&
      strcmp(mode, "stream") == 0) {
    p.stream_waves = stream_attention_waves(g.head_dim, n_seqs);
    if (p.stream_waves > 0) {
      p.stream_path = true;
      const uint64_t slots = (uint64_t)p.stream_waves + (uint64_t)n_seqs * g.n_kv_heads;
      p.pre_off = 0;
      p.o_off = align256(((uint64_t)n_seqs + 1) * 4u);
      p.ml_off = p.o_off + align256(slots * G * g.head_dim * 4u);
      p.total = p.ml_off + align256(slots * G * 2u * 4u);
      return p;
    }
  }
  p.mfma_path = g.dtype == kDtypeF16 && G >= 1 && G <= 16;
  p.split_path = g.dtype == kDtypeQ8 && G >= 1 && G <= 8;
  p.split_tokens = (p.mfma_path || p.split_path) ? choose_split_tokens(max_ctx_len, n_seqs, g.n_kv_heads)
                                                    : kAttnPartTokens;
  p.max_splits = max_ctx_len ? (max_ctx_len + p.split_tokens - 1) / p.split_tokens : 1;
  if (p.max_splits <= 1) return p;  // single split: no workspace
  const uint64_t items = (uint64_t)n_seqs * n_heads * p.max_splits;
  p.o_off = 0;
  p.ml_off = p.o_off + align256(items * g.head_dim * 4u);
  p.total = p.ml_off + align256(items * 2u * 4u);
  return p;
}

template <int DT, int D, int G, int RB = FKV_SPLIT_RANGE_BLOCKS>
hipError_t launch_split_t(const Geom& g, uint32_t layer, uint32_t n_heads, const float* q,
                          float* out, const int32_t* tables, uint32_t max_blocks,
                          const int32_t* ctx_lens, uint32_t n_seqs, const AttnPlan& p,
                          float scale, uint8_t* ws, hipStream_t s) {
  dim3 grid(n_seqs * g.n_kv_heads, p.max_splits);
  float* ws_o = ws ? (float*)(ws + p.o_off) : nullptr;
  float* ws_ml = ws ? (float*)(ws + p.ml_off) : nullptr;
  attn_split_kernel<DT, D, G, RB><<<grid, 256, 0, s>>>(
      g, layer, n_heads, q, out, tables, max_blocks, ctx_lens, p.max_splits,
      (int32_t)p.split_tokens, scale, ws_o, ws_ml);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || p.max_splits <= 1) return e;
  return launch_attention_combine(D, ctx_lens, n_seqs, n_heads, max_blocks, p.max_splits,
                                  p.split_tokens, ws_o, ws_ml, out, s);
}

template <int DT, int D>
hipError_t dispatch_split(uint32_t G, const Geom& g, uint32_t layer, uint32_t n_heads,
                          const float* q, float* out, const int32_t* tables, uint32_t max_blocks,
                          const int32_t* ctx_lens, uint32_t n_seqs, const AttnPlan& p,
                          float scale, uint8_t* ws, hipStream_t s) {
  switch (G) {
    case 1: return launch_split_t<DT, D, 1>(g, layer, n_heads, q, out, tables, max_blocks, ctx_lens, n_seqs, p, scale, ws, s);
    case 2: return launch_split_t<DT, D, 2>(g, layer, n_heads, q, out, tables, max_blocks, ctx_lens, n_seqs, p, scale, ws, s);
    case 4: return launch_split_t<DT, D, 4>(g, layer, n_heads, q, out, tables, max_blocks, ctx_lens, n_seqs, p, scale, ws, s);
    case 8: return launch_split_t<DT, D, 8>(g, layer, n_heads, q, out, tables, max_blocks, ctx_lens, n_seqs, p, scale, ws, s);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace

uint64_t attention_workspace_bytes(const Geom& g, uint32_t n_heads, uint32_t n_seqs,
                                   uint32_t max_ctx_len) {
  return plan_attention(g, n_heads, n_seqs, max_ctx_len).total;
}

uint64_t append_attention_workspace_bytes(const Geom& g, uint32_t n_heads, uint32_t n_seqs,
                                          uint32_t max_ctx_len) {
  const AttnPlan p = plan_attention(g, n_heads, n_seqs, max_ctx_len);
  if (p.mfma_path) return p.total;  // appended inside the attention kernel
  return p.total + align256((uint64_t)n_seqs * sizeof(int64_t));
}

namespace {

__global__ void __launch_bounds__(256) tail_slots_kernel(Geom g, const int32_t* __restrict__ tables,
                                                         uint32_t max_blocks,
                                                         const int32_t* __restrict__ ctx_lens,
                                                         uint32_t n_seqs, int64_t* __restrict__ slots) {
  const uint32_t s = blockIdx.x * 256u + threadIdx.x;
  if (s >= n_seqs) return;
  const int32_t ctx = ctx_lens[s];
  const int64_t cap = (int64_t)max_blocks * g.block_size;
  int64_t slot = -1;
  if (ctx > 0 && ctx <= cap) {
    const int32_t pos = ctx - 1;
    const int32_t pb = tables[(uint64_t)s * max_blocks + (uint32_t)pos / g.block_size];
    if (pb >= 0 && (uint64_t)pb < g.num_blocks)
      slot = (int64_t)pb * g.block_size + pos % (int32_t)g.block_size;
    else
      raise_fault(g.fault, kFaultBlock);
  }
  slots[s] = slot;
}

}  // namespace

hipError_t launch_tail_slots(const Geom& g, const int32_t* tables, uint32_t max_blocks,
                             const int32_t* ctx_lens, uint32_t n_seqs, int64_t* slots,
                             hipStream_t s) {
  tail_slots_kernel<<<(n_seqs + 255) / 256, 256, 0, s>>>(g, tables, max_blocks, ctx_lens, n_seqs,
                                                          slots);
  return hipGetLastError();
}

hipError_t launch_decode_attention(const Geom& g, uint32_t layer, uint32_t n_heads,
                                   const float* q, float* out, const int32_t* tables,
                                   uint32_t max_blocks, const int32_t* ctx_lens,
                                   uint32_t n_seqs, uint32_t max_ctx_len, float scale,
                                   void* workspace, const float* k_new, const float* v_new,
                                   hipStream_t s) {
  if (n_seqs == 0) return hipSuccess;
  const uint32_t G = n_heads / g.n_kv_heads;
  const AttnPlan p = plan_attention(g, n_heads, n_seqs, max_ctx_len);
  uint8_t* ws = (uint8_t*)workspace;
  if (k_new != nullptr && !p.mfma_path) {
    // Separate append launch: slots derived from the block tables first.
    int64_t* slots = (int64_t*)(ws + p.total);
    hipError_t e = launch_tail_slots(g, tables, max_blocks, ctx_lens, n_seqs, slots, s);
    if (e == hipSuccess) e = launch_append(g, layer, k_new, v_new, slots, n_seqs, s);
    if (e != hipSuccess) return e;
    k_new = v_new = nullptr;
  }
  if (p.stream_path)
    return launch_attention_stream(g, layer, n_heads, q, out, tables, max_blocks, ctx_lens,
                                   n_seqs, scale, p.stream_waves, (uint32_t*)(ws + p.pre_off),
                                   (float*)(ws + p.o_off), (float*)(ws + p.ml_off), s);
  if (p.mfma_path) {
    float* ws_o = ws ? (float*)(ws + p.o_off) : nullptr;
    float* ws_ml = ws ? (float*)(ws + p.ml_off) : nullptr;
    hipError_t e = launch_attention_mfma(g, layer, n_heads, q, out, tables, max_blocks, ctx_lens,
                                         n_seqs, p.max_splits, p.split_tokens, scale, ws_o,
                                         ws_ml, k_new, v_new, s);
    if (e != hipSuccess || p.max_splits <= 1) return e;
    return launch_attention_combine(g.head_dim, ctx_lens, n_seqs, n_heads, max_blocks,
                                    p.max_splits, p.split_tokens, ws_o, ws_ml, out, s);
  }
  if (p.split_path) {
    return g.head_dim == 128
               ? dispatch_split<kDtypeQ8, 128>(G, g, layer, n_heads, q, out, tables, max_blocks, ctx_lens, n_seqs, p, scale, ws, s)
               : dispatch_split<kDtypeQ8, 64>(G, g, layer, n_heads, q, out, tables, max_blocks, ctx_lens, n_seqs, p, scale, ws, s);
  }
  const uint32_t max_parts = p.max_splits;
  float* ws_o = ws ? (float*)(ws + p.o_off) : nullptr;
  float* ws_ml = ws ? (float*)(ws + p.ml_off) : nullptr;
  // F16 never gets here (mfma_path covers every supported group size).
  if (g.head_dim == 128) {
    if (g.dtype == kDtypeF32)
      return dispatch_group<kDtypeF32, 128>(G, g, layer, n_heads, q, out, tables, max_blocks,
                                            ctx_lens, n_seqs, max_parts, scale, ws_o, ws_ml, s);
    return dispatch_group<kDtypeQ8, 128>(G, g, layer, n_heads, q, out, tables, max_blocks,
                                         ctx_lens, n_seqs, max_parts, scale, ws_o, ws_ml, s);
  }
  if (g.dtype == kDtypeF32)
    return dispatch_group<kDtypeF32, 64>(G, g, layer, n_heads, q, out, tables, max_blocks,
                                         ctx_lens, n_seqs, max_parts, scale, ws_o, ws_ml, s);
  return dispatch_group<kDtypeQ8, 64>(G, g, layer, n_heads, q, out, tables, max_blocks,
                                      ctx_lens, n_seqs, max_parts, scale, ws_o, ws_ml, s);
}

}  // namespace fkv
