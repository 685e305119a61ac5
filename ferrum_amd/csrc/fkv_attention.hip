// Paged decode attention for gfx950: the attention loop of
// Llama::forward_one_token (crates/model/src/llama.rs:220-247) over K/V read
// through block tables, with the softmax of crates/kernels/src/scalar.rs:125-141
// (a non-finite maximum gives zeros).
//
// This file holds the VALU kernel, the merge kernels and the dispatch:
//   F32 storage          attn_partition_kernel (G in {1, 2, 4, 8, 16})
//   F16, Q8_0 storage    the MFMA kernels of fkv_attention_mfma.hip (G <= 16)
// and attn_combine_kernel, which merges split partials for all of them.
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <atomic>
#include <mutex>
#include <type_traits>

#include "fkv_device.h"
#include "fkv_internal.h"

// Scratch of fkv_append_decode_attention_noalloc: the split partials (and, for F32
// storage, the derived slots) that the workspace argument holds for the other entry
// points. Every GPU the library runs on holds its own copy until the process ends.
// In host code `scratch` is only a stand-in for the symbol: host code passes the
// per-device address from static_scratch_setup to kernels, never the name itself.
// Nothing in it has to start at zero (every partial is written before it is read).
static __device__ __align__(256) uint8_t scratch[fkv::kStaticScratchBytes];

namespace fkv {

namespace {
constexpr int kMaxScratchDevices = 64;
std::mutex g_scratch_mu;  // serialises set-up; readers take the published address
std::atomic<void*> g_scratch_addr[kMaxScratchDevices];
}  // namespace

hipError_t static_scratch_setup(int device) {
  if (device < 0 || device >= kMaxScratchDevices) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_addr[device].load(std::memory_order_acquire) != nullptr) return hipSuccess;
  void* p = nullptr;
  const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
  if (e != hipSuccess) return e;
  if (p == nullptr) return hipErrorInvalidSymbol;
  g_scratch_addr[device].store(p, std::memory_order_release);
  return hipSuccess;
}

void* static_scratch(int device) {
  if (device < 0 || device >= kMaxScratchDevices) return nullptr;
  return g_scratch_addr[device].load(std::memory_order_acquire);
}

Tuning& tuning() {
  static Tuning t;
  static std::once_flag seeded;
  std::call_once(seeded, [] {
    if (const char* e = getenv("FKV_ATTN_SPLIT_TOKENS")) {
      const long v = strtol(e, nullptr, 10);
      if (v >= 16 && v % 16 == 0 && v <= (1 << 20)) t.split_tokens = (int32_t)v;
    }
    if (const char* e = getenv("FKV_ATTN_MODE")) t.stream_mode = strcmp(e, "stream") == 0;
    if (const char* e = getenv("FKV_ATTN_ORDER")) {
      const long v = strtol(e, nullptr, 10);
      if (v >= 0 && v <= 2) t.attn_order = (int32_t)v;
    }
    if (const char* e = getenv("FKV_PREFILL_SPLIT_BLOCKS")) {
      const long long v = strtoll(e, nullptr, 10);
      if (v >= 0) t.prefill_split = v;
    }
    if (const char* e = getenv("FKV_ATTN_ENGINE")) t.attn_engine = strcmp(e, "valu") == 0;
    if (const char* e = getenv("FKV_ATTN_WGS_PER_CU")) {
      const int v = atoi(e);
      if (v == 2 || v == 3) t.attn_wgs_per_cu = v;
    }
  });
  return t;
}

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
// F32 storage: K and V tiles [token][D]. F16 storage (the matrix-core operand order the
// pool keeps, read here only when FKV_TUNE_ATTN_ENGINE selects this kernel, to measure
// the choice): K [D/8][16][8], a 16-byte unit = 8 dims of one token, so a lane's unit
// of token row r is run c; V [D][16], a unit = 8 tokens of one dim, so phase 3 runs
// per (dim, 8 tokens) unit instead of per token row (pv_f16 below).

template <int DT, int D>
struct AttnShape {
  static_assert(DT == kDtypeF32 || DT == kDtypeF16, "the VALU partition kernel reads F32 or F16");
  static constexpr int E = DT == kDtypeF32 ? 4 : 2;
  static constexpr int EPL = 16 / E;            // values per lane per 16-byte load
  static constexpr int LPR = D / EPL;           // lanes per token row
  static constexpr int RPP = 64 / LPR;          // token rows per load instruction
  static constexpr int PASSES = kAttnBlock / RPP;
  static constexpr bool kPrefetchV = PASSES <= 4;
  static_assert(LPR >= 1 && LPR <= 32 && RPP * LPR == 64 && PASSES * RPP == kAttnBlock, "shape");
};

// One 16-byte load of storage as floats: F32 4, F16 8 (binary16 -> binary32 is exact).
template <int DT, int EPL>
__device__ __forceinline__ void decode16(const uint4& w, float (&f)[EPL]) {
  if constexpr (DT == kDtypeF32) {
    f[0] = __uint_as_float(w.x); f[1] = __uint_as_float(w.y);
    f[2] = __uint_as_float(w.z); f[3] = __uint_as_float(w.w);
  } else {
    const uint32_t u[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int i = 0; i < 4; i++) {
      f[2 * i] = f16_bits_to_f32(u[i] & 0xffffu);
      f[2 * i + 1] = f16_bits_to_f32(u[i] >> 16);
    }
  }
}
// Byte offset of lane (row r, column c)'s 16-byte unit of a K tile.
template <int DT>
__device__ __forceinline__ uint64_t k_unit_off(int row, int c, uint64_t row_bytes) {
  return DT == kDtypeF32 ? (uint64_t)row * row_bytes + (uint64_t)c * 16u
                         : ((uint64_t)c * kAttnBlock + (uint64_t)row) * 16u;
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
  const int32_t cap = dev::split_ctx_cap(max_blocks, kAttnBlock, max_parts, kAttnPartTokens);
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

  // Issue K loads for all blocks, then V loads (kept in flight through phase 1-2).
  uint4 kreg[NB][PASSES];
#pragma unroll
  for (int j = 0; j < NB; j++) {
    if (live[j]) {
      const uint8_t* kt = tile_ptr(g, (uint64_t)phys[j], layer, 0, kvh);
#pragma unroll
      for (int ps = 0; ps < PASSES; ps++) {
        int row = ps * RPP + r;
        kreg[j][ps] = load_stream16(kt + k_unit_off<DT>(row, c, row_bytes));
      }
    }
  }
  // F16 V: D / 32 units of 16 bytes a lane (unit ps * 64 + lane: dim (ps * 64 + lane) / 2,
  // tokens 8 (lane % 2) .. + 7), 1 KiB of consecutive bytes an instruction.
  constexpr int PV = DT == kDtypeF16 ? D / 32 : PASSES;
  uint4 vreg[S::kPrefetchV ? NB : 1][PV];
  if constexpr (S::kPrefetchV) {
#pragma unroll
    for (int j = 0; j < NB; j++) {
      if (live[j]) {
        const uint8_t* vt = tile_ptr(g, (uint64_t)phys[j], layer, 1, kvh);
#pragma unroll
        for (int ps = 0; ps < PV; ps++) {
          if constexpr (DT == kDtypeF16) {
            vreg[j][ps] = load_stream16(vt + (uint64_t)(ps * 64 + lane) * 16u);
          } else {
            int row = ps * RPP + r;
            vreg[j][ps] = load_stream16(vt + row * row_bytes + c * 16);
          }
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
  if constexpr (DT == kDtypeF16) {
    // per unit: dim n = (ps * 64 + lane) / 2, its 8 tokens of half lane % 2; the two
    // halves of a dim (lanes l, l ^ 1) are summed at the end
    float acc3[PV][G];
#pragma unroll
    for (int ps = 0; ps < PV; ps++)
#pragma unroll
      for (int gg = 0; gg < G; gg++) acc3[ps][gg] = 0.0f;
#pragma unroll
    for (int j = 0; j < NB; j++) {
      if (!live[j]) continue;
      float vf[PV][8];
#pragma unroll
      for (int ps = 0; ps < PV; ps++) {
        const uint4 w = S::kPrefetchV ? vreg[j][ps]
                                      : load_stream16(tile_ptr(g, (uint64_t)phys[j], layer, 1, kvh) +
                                                      (uint64_t)(ps * 64 + lane) * 16u);
        decode16<DT, 8>(w, vf[ps]);
      }
      const int32_t tb = (wave * NB + j) * kAttnBlock + (lane & 1) * 8;
#pragma unroll
      for (int i = 0; i < 8; i++) {
        if (tb + i < n_valid) {  // tokens past the context: no term (V there may be NaN)
          float pw[G];
#pragma unroll
          for (int gg = 0; gg < G; gg++) pw[gg] = s_p[tb + i][gg];
#pragma unroll
          for (int ps = 0; ps < PV; ps++)
#pragma unroll
            for (int gg = 0; gg < G; gg++) acc3[ps][gg] = __builtin_fmaf(pw[gg], vf[ps][i], acc3[ps][gg]);
        }
      }
    }
#pragma unroll
    for (int ps = 0; ps < PV; ps++)
#pragma unroll
      for (int gg = 0; gg < G; gg++) acc3[ps][gg] += __shfl_xor(acc3[ps][gg], 1);
    if ((lane & 1) == 0) {
#pragma unroll
      for (int ps = 0; ps < PV; ps++)
#pragma unroll
        for (int gg = 0; gg < G; gg++) s_acc[wave][gg][(ps * 64 + lane) / 2] = acc3[ps][gg];
    }
  } else {
  float acc[G][EPL];
#pragma unroll
  for (int gg = 0; gg < G; gg++)
#pragma unroll
    for (int i = 0; i < EPL; i++) acc[gg][i] = 0.0f;

#pragma unroll
  for (int j = 0; j < NB; j++) {
    if (!live[j]) continue;
    uint4 vl[PASSES];
    if constexpr (S::kPrefetchV) {
#pragma unroll
      for (int ps = 0; ps < PASSES; ps++) vl[ps] = vreg[j][ps];
    } else {
      const uint8_t* vt = tile_ptr(g, (uint64_t)phys[j], layer, 1, kvh);
#pragma unroll
      for (int ps = 0; ps < PASSES; ps++) {
        int row = ps * RPP + r;
        vl[ps] = load_stream16(vt + row * row_bytes + c * 16);
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
#pragma unroll
        for (int gg = 0; gg < G; gg++)
#pragma unroll
          for (int i = 0; i < EPL; i++) acc[gg][i] = __builtin_fmaf(pw[gg], vf[i], acc[gg][i]);
      }
    }
  }

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
  }  // F32
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
// partition p's (m, l) (64 partitions per pass) and every lane holds D/64 dims.
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
  // The context length and the first 64 partitions' (m, l) are loaded together:
  // slots past the head's partition count hold stale bytes and are masked once
  // the count is known (the workspace has max_parts slots per head, so every load
  // is in bounds). Partial outputs are read only for the head's own partitions.
  const int32_t raw_ctx = ctx_lens[seq];
  const int32_t n0 = (int32_t)max_parts < 64 ? (int32_t)max_parts : 64;
  float mp = lane < n0 ? ml[2 * lane] : -__builtin_inff();
  float lp = lane < n0 ? ml[2 * lane + 1] : 0.0f;

  const int32_t cap = dev::split_ctx_cap(max_blocks, kAttnBlock, max_parts, (uint32_t)part_tokens);
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
#pragma unroll
      for (int j = 0; j < kChunk; j++)
#pragma unroll
        for (int i = 0; i < DPL; i++)
          v[j][i] = c0 + j < n ? po[(uint64_t)(p0 + c0 + j) * D + i] : 0.0f;
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
  const int32_t cap = dev::split_ctx_cap(max_blocks, kAttnBlock, max_parts, (uint32_t)part_tokens);
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
#define FKV_G(N)                                                                             \
  case N:                                                                                    \
    return launch_attn_t<DT, D, N>(g, layer, n_heads, q, out, tables, max_blocks,            \
                                          ctx_lens, n_seqs, max_parts, scale, ws_o, ws_ml, s);
  switch (G) {
    FKV_G(1)
    FKV_G(2)
    FKV_G(4)
    FKV_G(8)
    FKV_G(16)
    default:
      break;
  }
#undef FKV_G
  return hipErrorInvalidValue;
}

}  // namespace

bool attention_supported(int dtype, uint32_t head_dim, uint32_t group) {
  if (head_dim != 64 && head_dim != 128) return false;
  if (dtype == kDtypeF16 || dtype == kDtypeQ8) return group >= 1 && group <= 16;
  if (dtype != kDtypeF32) return false;
  return group == 1 || group == 2 || group == 4 || group == 8 || group == 16;
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
  bool mfma_path = false;   // attn_mfma_kernel (F16, Q8_0) + combine
  uint32_t split_tokens = kAttnPartTokens;
  uint32_t max_splits = 1;
  uint64_t o_off = 0, ml_off = 0, total = 0;
};

inline uint64_t align256(uint64_t x) { return (x + 255) / 256 * 256; }

// Split length. A workgroup pays a fixed cost (its start, the latency of its first
// block-table and K/V loads, the merge of its 4 waves, the partial it writes, and
// the combine's read of it) that a longer split spreads over more bytes, while
// the last workgroups' lengths set how ragged the kernel's end is. Measured on
// MI355X with the longest-first order, the best lengths made about 2,048 (sequence,
// KV head, split) workgroups at the longest context in the batch (64 x U[128, 4096]
// tokens: 1,024; 128 x 8,192: 4,096; 256 log-normal contexts up to 32k: 8,192),
// with at most about 64 splits per head (1 x 131,072 tokens: 2,048; longer splits
// leave CUs idle there). So: the larger of max_ctx * segments / 2048 and
// max_ctx / 64, to the nearest multiple of 256, up to 8192. A batch too small for
// 512-token splits to fill the GPU is latency-bound instead: it gets about 512
// workgroups, splits of 64 tokens or more (a multiple of 64), still at most about
// 64 per head (1 x 576 tokens, 4 KV heads: 64 tokens, 9.7 us per call against
// 13.8 us at 512). FKV_ATTN_SPLIT_TOKENS (a multiple of 16) overrides.
uint32_t choose_split_tokens(uint32_t max_ctx_len, uint32_t n_seqs, uint32_t n_kv_heads) {
  if (const int32_t v = tuning().split_tokens.load(std::memory_order_relaxed)) return (uint32_t)v;
  const uint64_t segs = (uint64_t)n_seqs * (n_kv_heads ? n_kv_heads : 1);
  const uint64_t by_items = (uint64_t)max_ctx_len * segs / 2048;
  const uint64_t by_head = ((uint64_t)max_ctx_len + 63) / 64;
  uint64_t st = ((by_items > by_head ? by_items : by_head) + 128) / 256 * 256;
  if (st > 8192) st = 8192;
  if (st >= 512) return (uint32_t)st;
  const uint64_t small = (uint64_t)max_ctx_len * segs / 512;
  st = ((small > by_head ? small : by_head) + 63) / 64 * 64;
  if (st < 64) st = 64;
  if (st > 512) st = 512;
  return (uint32_t)st;
}

AttnPlan plan_attention(const Geom& g, uint32_t n_heads, uint32_t n_seqs, uint32_t max_ctx_len) {
  AttnPlan p;
  const uint32_t G = g.n_kv_heads ? n_heads / g.n_kv_heads : 0;
  // F16: the split kernel by default; FKV_ATTN_MODE=stream selects the persistent one.
  if (g.dtype == kDtypeF16 && G >= 1 && G <= 16 && stream_attention_supported(n_seqs) &&
      tuning().stream_mode.load(std::memory_order_relaxed)) {
    p.stream_waves = stream_attention_waves(g.head_dim, n_seqs, g.n_cus);
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
  p.mfma_path = (g.dtype == kDtypeF16 || g.dtype == kDtypeQ8) && G >= 1 && G <= 16;
  // FKV_TUNE_ATTN_ENGINE = 1: F16 on the VALU partition kernel where it has an instance
  if (p.mfma_path && g.dtype == kDtypeF16 && tuning().attn_engine.load(std::memory_order_relaxed) &&
      (G == 1 || G == 2 || G == 4 || G == 8 || G == 16))
    p.mfma_path = false;
  p.split_tokens = p.mfma_path ? choose_split_tokens(max_ctx_len, n_seqs, g.n_kv_heads)
                                                    : kAttnPartTokens;
  p.max_splits = max_ctx_len ? (max_ctx_len + p.split_tokens - 1) / p.split_tokens : 1;
  if (p.max_splits <= 1) return p;  // single split: no workspace
  const uint64_t items = (uint64_t)n_seqs * n_heads * p.max_splits;
  p.o_off = 0;
  p.ml_off = p.o_off + align256(items * g.head_dim * 4u);
  p.total = p.ml_off + align256(items * 2u * 4u);
  return p;
}

}  // namespace

uint64_t attention_workspace_bytes(const Geom& g, uint32_t n_heads, uint32_t n_seqs,
                                   uint32_t max_ctx_len) {
  return plan_attention(g, n_heads, n_seqs, max_ctx_len).total;
}

uint64_t append_attention_workspace_bytes(const Geom& g, uint32_t n_heads, uint32_t n_seqs,
                                          uint32_t max_ctx_len) {
  const AttnPlan p = plan_attention(g, n_heads, n_seqs, max_ctx_len);
  if (p.mfma_path) return p.total;  // appended inside the kernel
  return p.total + align256((uint64_t)n_seqs * sizeof(int64_t));
}

uint64_t rope_attention_workspace_bytes(const Geom& g, uint32_t n_heads, uint32_t n_seqs,
                                        uint32_t max_ctx_len) {
  const uint64_t base = append_attention_workspace_bytes(g, n_heads, n_seqs, max_ctx_len);
  const AttnPlan p = plan_attention(g, n_heads, n_seqs, max_ctx_len);
  if (p.mfma_path) return base;  // rotated inside the kernel
  return base +
         align256((uint64_t)n_seqs * (n_heads + g.n_kv_heads) * g.head_dim * sizeof(float));
}

namespace {

// RoPE rows for storage the decode kernels do not rotate in place: pair p of row
// (s, h) of q [n_seqs][n_heads][D] and of k [n_seqs][n_kv][D], rotated at position
// ctx_lens[s] - 1 as the reference does (crates/kernels/src/scalar.rs:167-189).
__global__ void __launch_bounds__(256) rope_rows_kernel(RopeTable rope, const int32_t* __restrict__ ctx_lens,
                                                        int32_t cap, uint32_t n_seqs, uint32_t n_heads,
                                                        uint32_t n_kv, uint32_t D,
                                                        const float* __restrict__ q,
                                                        const float* __restrict__ k,
                                                        float* __restrict__ q_out,
                                                        float* __restrict__ k_out) {
  const uint32_t half = D / 2, rows = n_heads + n_kv;
  const uint64_t i = (uint64_t)blockIdx.x * 256u + threadIdx.x;
  if (i >= (uint64_t)n_seqs * rows * half) return;
  const uint32_t pr = (uint32_t)(i % half);
  const uint64_t row = i / half;
  const uint32_t s = (uint32_t)(row / rows), h = (uint32_t)(row % rows);
  const uint64_t off = h < n_heads ? ((uint64_t)s * n_heads + h) * D + 2 * pr
                                   : ((uint64_t)s * n_kv + (h - n_heads)) * D + 2 * pr;
  const float* src = h < n_heads ? q : k;
  float* dst = h < n_heads ? q_out : k_out;
  float a = src[off], b = src[off + 1];
  if ((int32_t)(2 * pr) < rope.rope_dim) {
    int32_t c = ctx_lens[s];
    c = c < 0 ? 0 : (c > cap ? cap : c);
    const uint32_t pos = (uint32_t)(c > 0 ? c - 1 : 0);
    float sn, cs;
    if (rope.sc != nullptr && pos < rope.sc_pos) {
      sn = rope.sc[((uint64_t)pos * (uint32_t)(rope.rope_dim / 2) + pr) * 2u];
      cs = rope.sc[((uint64_t)pos * (uint32_t)(rope.rope_dim / 2) + pr) * 2u + 1u];
    } else {
      sincosf((float)pos / rope.den[pr], &sn, &cs);
    }
    const float a2 = a * cs - b * sn, b2 = a * sn + b * cs;
    a = a2;
    b = b2;
  }
  dst[off] = a;
  dst[off + 1] = b;
}

__global__ void __launch_bounds__(256) tail_slots_kernel(Geom g, const int32_t* __restrict__ tables,
                                                         uint32_t max_blocks,
                                                         const int32_t* __restrict__ ctx_lens,
                                                         uint32_t n_seqs, int64_t cap,
                                                         int64_t* __restrict__ slots) {
  const uint32_t s = blockIdx.x * 256u + threadIdx.x;
  if (s >= n_seqs) return;
  const int32_t ctx = ctx_lens[s];
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
                             hipStream_t s, uint64_t ctx_cap) {
  const uint64_t rows = (uint64_t)max_blocks * g.block_size;
  const uint64_t cap = ctx_cap < rows ? ctx_cap : rows;
  tail_slots_kernel<<<(n_seqs + 255) / 256, 256, 0, s>>>(g, tables, max_blocks, ctx_lens, n_seqs,
                                                          (int64_t)cap, slots);
  return hipGetLastError();
}

hipError_t launch_decode_attention(const Geom& g, uint32_t layer, uint32_t n_heads,
                                   const float* q, float* out, const int32_t* tables,
                                   uint32_t max_blocks, const int32_t* ctx_lens,
                                   uint32_t n_seqs, uint32_t max_ctx_len, float scale,
                                   void* workspace, const float* k_new, const float* v_new,
                                   hipStream_t s, const RopeTable* rope) {
  if (n_seqs == 0) return hipSuccess;
  const uint32_t G = n_heads / g.n_kv_heads;
  const AttnPlan p = plan_attention(g, n_heads, n_seqs, max_ctx_len);
  uint8_t* ws = (uint8_t*)workspace;
  // The context a launch holds: the table row, and what its splits cover. A longer one
  // is clamped to it by every kernel (FKV_FAULT_CTX_RANGE), which then stores no token
  // for the sequence and rotates at the clamped position.
  const uint64_t split_cap = (uint64_t)p.max_splits * p.split_tokens;
  const uint64_t row_cap = (uint64_t)max_blocks * g.block_size;
  const int32_t ctx_cap = (int32_t)std::min<uint64_t>(std::min(split_cap, row_cap), 0x7fffffffull);
  if (rope != nullptr && rope->rope_dim > 0 && !p.mfma_path) {
    // Rotate q and the new K rows into the workspace, then run the unrotated step.
    float* q_rot = (float*)(ws + append_attention_workspace_bytes(g, n_heads, n_seqs, max_ctx_len));
    float* k_rot = q_rot + (uint64_t)n_seqs * n_heads * g.head_dim;
    const uint64_t pairs = (uint64_t)n_seqs * (n_heads + g.n_kv_heads) * (g.head_dim / 2);
    rope_rows_kernel<<<(uint32_t)((pairs + 255) / 256), 256, 0, s>>>(
        *rope, ctx_lens, ctx_cap, n_seqs, n_heads, g.n_kv_heads,
        g.head_dim, q, k_new, q_rot, k_rot);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    q = q_rot;
    k_new = k_rot;
    rope = nullptr;
  }
  if (k_new != nullptr && !p.mfma_path) {
    // Separate append launch: slots derived from the block tables first.
    int64_t* slots = (int64_t*)(ws + p.total);
    hipError_t e = launch_tail_slots(g, tables, max_blocks, ctx_lens, n_seqs, slots, s,
                                     (uint64_t)ctx_cap);
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
                                         ws_ml, k_new, v_new, s, rope);
    if (e != hipSuccess || p.max_splits <= 1) return e;
    return launch_attention_combine(g.head_dim, ctx_lens, n_seqs, n_heads, max_blocks,
                                    p.max_splits, p.split_tokens, ws_o, ws_ml, out, s);
  }
  const uint32_t max_parts = p.max_splits;
  float* ws_o = ws ? (float*)(ws + p.o_off) : nullptr;
  float* ws_ml = ws ? (float*)(ws + p.ml_off) : nullptr;
  // Q8_0 never gets here, F16 only when FKV_TUNE_ATTN_ENGINE selects the VALU kernel.
  if (g.dtype == kDtypeF16) {
    if (g.head_dim == 128)
      return dispatch_group<kDtypeF16, 128>(G, g, layer, n_heads, q, out, tables, max_blocks,
                                            ctx_lens, n_seqs, max_parts, scale, ws_o, ws_ml, s);
    return dispatch_group<kDtypeF16, 64>(G, g, layer, n_heads, q, out, tables, max_blocks,
                                         ctx_lens, n_seqs, max_parts, scale, ws_o, ws_ml, s);
  }
  if (g.head_dim == 128)
    return dispatch_group<kDtypeF32, 128>(G, g, layer, n_heads, q, out, tables, max_blocks, ctx_lens,
                               n_seqs, max_parts, scale, ws_o, ws_ml, s);
  return dispatch_group<kDtypeF32, 64>(G, g, layer, n_heads, q, out, tables, max_blocks, ctx_lens, n_seqs,
                            max_parts, scale, ws_o, ws_ml, s);
}

}  // namespace fkv
