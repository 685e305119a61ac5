// Paged decode attention on the matrix cores of gfx950, for F16 KV storage.
// Same contract as the attention loop of Llama::forward_one_token
// (crates/model/src/llama.rs:220-247): for each query head h of a sequence,
// score[p] = dot(q_h, K[p][h / g]) * scale, softmax over the context
// (crates/kernels/src/scalar.rs:125-141, a non-finite maximum gives zeros), then
// out_h = sum_p w_p V[p][h / g], with f32 accumulation.
//
// Decode attention is a GEMV over HBM, but with a GQA group of G query heads it
// is G GEMVs over the same K/V bytes. On the VALU that work grows with G: the
// F32-storage VALU kernel (fkv_attention.hip) issues 677 VALU instructions per
// 16-token block and KV head at G = 4 and 1,214 at G = 8, where it streams at
// 3.7 TB/s (46% of HBM peak), and F16 storage would bring half the bytes for the
// same FMAs. Here the G heads are MFMA columns: ~200 VALU instructions and 16
// MFMAs per block at any G (the matrix cores busy ~7% of the time), 5.7-5.9 TB/s
// at G = 4 and 8 (C2, measured with rocprof counters).
//
// One wave processes one 16-token block at a time:
//
//   QK   S[token][head] = K[16 x D] . Q^T[D x 16] with v_mfma_f32_16x16x32_f16:
//        A = the K tile (lane l: token l%16, dims c*32 + (l/16)*8 .. +7, one
//        16-byte load per chunk c from the [D/8][B][8] tile, so each load
//        instruction reads 1 KiB of consecutive bytes); B = q split into f16 hi +
//        lo parts (two MFMAs per chunk, ~22 significant bits) after a per-head
//        power-of-two scaling that keeps q inside the f16 range. Output lane l
//        holds tokens (l/16)*4 + r of head l%16.
//   soft lazy online softmax in the log2 domain: each lane keeps a partial sum
//        for its head; only when a score exceeds the head's reference max by
//        2^8 (any lane, by ballot) does the wave take the exact running max and
//        rescale the partial sums and accumulators.
//   PV   O[head][dim] += P[16 x 16 tokens] . V[16 tokens x 16 dims] with
//        v_mfma_f32_16x16x16_f16 for each 16-dim column tile: A = P in f16 (lane
//        l: head l%16, tokens (l/16)*4 .. +3 -- exactly the QK output layout, so
//        no lane exchange), B = V from the dim-major V tile (lane l: dim
//        16m + l%16, tokens (l/16)*4 .. +3, one 8-byte load; 512 consecutive
//        bytes per load instruction).
//
// Heads >= G in the 16-wide MFMA are padding: their q is zero and their scores
// are forced to -inf, so they never trigger a rescale and are never written.
//
// Two schedules share that block step:
//   attn_mfma_kernel  (default) one workgroup per (sequence, KV head, 512-token
//        split); its 4 waves take every fourth block and merge in LDS; splits
//        of one sequence are merged by attn_combine_kernel (log-sum-exp).
//   attn_mfma_stream_kernel  (FKV_ATTN_MODE=stream) persistent: the grid is the
//        number of workgroups the GPU holds at once; every wave takes an equal
//        contiguous range of the flattened (sequence, KV head, block) list and
//        streams it without a break. A (sequence, KV head) inside one wave's
//        range is written to `out` directly; one cut by a range boundary leaves
//        partials that attn_stream_combine_kernel merges. Measured on MI355X it
//        is no faster than the split kernel: equal ranges finish 55-98 us apart
//        because XCDs stream at different rates.
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdlib.h>

#include <algorithm>

#include "fkv_device.h"
#include "fkv_internal.h"

// Blocks in flight per wave (the load ring depth) of attn_mfma_kernel.
#ifndef FKV_MFMA_RING
#define FKV_MFMA_RING 1
#endif

namespace fkv {
namespace {

using namespace dev;

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef short s16x4 __attribute__((ext_vector_type(4)));  // bf16 MFMA operands

constexpr int kHeads = 16;            // MFMA column count: query heads of one group
constexpr float kRescaleLog2 = 8.0f;  // rescale when a score passes the reference max by 2^8
constexpr int B = kAttnBlock;

__device__ __forceinline__ u32x2_t load_stream8(const uint8_t* p) {
  return __builtin_nontemporal_load((const u32x2_t*)p);
}

// Per-lane view of one wave's 16 x 16 MFMA tiles.
struct Lane {
  int lane;   // 0..63
  int col;    // K token row / q head / score head / V dim within a 16-column tile
  int grp;    // MFMA k group (0..3)
  bool real;  // col < G: this lane's score column is a real query head
};

// q rows -> QK B operand. Lane (col, grp) reads dims c*32 + grp*8 .. +7 of the
// query row of column col (qrow: any readable row for padding columns). Each row
// gets a power-of-two scaling (its largest |q * scale * log2 e| lands in
// [2^14, 2^15), far from f16 overflow), then an f16 hi + lo split; hscale undoes
// the scaling.
//
// ROPE: q is before RoPE. The lane's eight dims of chunk c are the four whole pairs
// c*16 + grp*4 + e' (e' < 4), rotated as the reference does (a' = a cos - b sin,
// b' = a sin + b cos, each product rounded) before the scaling. rsin / rcos hold
// the (sin, cos) of pair rope_pair(lane): lane c*4 + e' of each 16-lane row has the
// pair its row needs, broadcast to the row with DPP.
// Lane L of each 16-lane row, broadcast to the row (DPP row_newbcast). L must
// fold to a constant (an unrolled loop index): the switch then leaves one move.
template <int L>
__device__ __forceinline__ float row_bcast_c(float v) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x150 + L, 0xF, 0xF, false));
}
__device__ __forceinline__ float row_bcast(float v, int l) {
  switch (l) {
#define FKV_ROW_BCAST(L_) \
  case L_:                \
    return row_bcast_c<L_>(v);
    FKV_ROW_BCAST(0) FKV_ROW_BCAST(1) FKV_ROW_BCAST(2) FKV_ROW_BCAST(3)
    FKV_ROW_BCAST(4) FKV_ROW_BCAST(5) FKV_ROW_BCAST(6) FKV_ROW_BCAST(7)
    FKV_ROW_BCAST(8) FKV_ROW_BCAST(9) FKV_ROW_BCAST(10) FKV_ROW_BCAST(11)
    FKV_ROW_BCAST(12) FKV_ROW_BCAST(13) FKV_ROW_BCAST(14) FKV_ROW_BCAST(15)
#undef FKV_ROW_BCAST
    default: return v;
  }
}

// The RoPE pair whose (sin, cos) a lane holds: c*16 + grp*4 + e' for lane
// (col = c*4 + e', grp), so that every 16-lane row holds the 16 pairs prep_q needs
// for its 8 dims of each 32-dim chunk.
__device__ __forceinline__ int rope_pair(int lane) {
  const int col = lane & 15, grp = lane >> 4;
  return (col >> 2) * 16 + grp * 4 + (col & 3);
}

template <int D, bool ROPE = false>
__device__ __forceinline__ void prep_q(const float* qrow, const Lane& ln, float qscale,
                                       f16x8 (&qh)[D / 32], f16x8 (&ql)[D / 32],
                                       float& hscale, float rsin = 0.0f, float rcos = 1.0f,
                                       int rope_dim = 0) {
  constexpr int NC = D / 32;
  const float* qb = qrow + ln.grp * 8;
  float x[NC][8];
  float amax = 0.0f;
#pragma unroll
  for (int c = 0; c < NC; c++) {
    const float4 a = *(const float4*)(qb + c * 32);
    const float4 b = *(const float4*)(qb + c * 32 + 4);
    float v8[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
    if constexpr (ROPE) {
#pragma unroll
      for (int e = 0; e < 8; e += 2) {
        const int dim = c * 32 + ln.grp * 8 + e;
        const float sn = row_bcast(rsin, c * 4 + e / 2), cs = row_bcast(rcos, c * 4 + e / 2);
        if (dim < rope_dim) {
          const float u = v8[e], w = v8[e + 1];
          v8[e] = u * cs - w * sn;
          v8[e + 1] = u * sn + w * cs;
        }
      }
    }
#pragma unroll
    for (int e = 0; e < 8; e++) {
      x[c][e] = ln.real ? v8[e] * qscale : 0.0f;
      amax = __builtin_fmaxf(amax, __builtin_fabsf(x[c][e]));
    }
  }
  amax = __builtin_fmaxf(amax, __shfl_xor(amax, 16));
  amax = __builtin_fmaxf(amax, __shfl_xor(amax, 32));
  int k = 0;
  if (amax > 0.0f && __builtin_isfinite(amax)) {
    int ex;
    (void)__builtin_frexpf(amax, &ex);
    k = 15 - ex;
  }
  const float up = __builtin_ldexpf(1.0f, k);
  hscale = __builtin_ldexpf(1.0f, -k);
#pragma unroll
  for (int c = 0; c < NC; c++)
#pragma unroll
    for (int e = 0; e < 8; e++) {
      const float y = x[c][e] * up;
      const _Float16 hi = (_Float16)y;
      qh[c][e] = hi;
      ql[c][e] = (_Float16)(y - (float)hi);
    }
}

// Running softmax state of the lane's head plus the wave's O accumulators
// (row r of acc[m] is head grp*4 + r, dim 16m + col).
template <int D>
struct Accum {
  float m_ref, l_part;
  f32x4 acc[D / 16];
  __device__ __forceinline__ void reset() {
    m_ref = -__builtin_inff();
    l_part = 0.0f;
#pragma unroll
    for (int m = 0; m < D / 16; m++) acc[m] = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};
  }
};

// Scores of one block (log2 domain) for this lane's head and tokens
// t0 + grp*4 + r; tokens at or past `end`, dead blocks and padding heads get -inf.
template <int D>
__device__ __forceinline__ void qk_block(const uint4 (&kr)[D / 32], const f16x8 (&qh)[D / 32],
                                         const f16x8 (&ql)[D / 32], float hscale,
                                         const Lane& ln, bool live, int32_t t0, int32_t end,
                                         float (&s)[4]) {
  // hi and lo parts in separate chains. An infinite K value meets q's hi part with
  // the sign of q (its hi part is q rounded), so the hi chain holds every infinity of
  // the reference's f32 dot with the right sign; the lo part can be zero (inf * 0 =
  // NaN) or of the other sign (+inf + -inf = NaN in the sum). So a NaN sum whose hi
  // chain is not NaN takes the hi chain alone.
  f32x4 ah = {0.0f, 0.0f, 0.0f, 0.0f}, al = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int c = 0; c < D / 32; c++) {
    const f16x8 kv = __builtin_bit_cast(f16x8, kr[c]);
    ah = __builtin_amdgcn_mfma_f32_16x16x32_f16(kv, qh[c], ah, 0, 0, 0);
    al = __builtin_amdgcn_mfma_f32_16x16x32_f16(kv, ql[c], al, 0, 0, 0);
  }
#pragma unroll
  for (int r = 0; r < 4; r++) {
    const bool ok = ln.real && live && t0 + ln.grp * 4 + r < end;
    const float sum = ah[r] + al[r];
    const float x = (sum != sum && ah[r] == ah[r]) ? ah[r] : sum;
    s[r] = ok ? x * hscale : -__builtin_inff();
  }
}

// Lazy online softmax update and P (f16, the PV A operand) of one block.
template <int D>
__device__ __forceinline__ f16x4 softmax_block(const float (&s)[4], const Lane& ln,
                                               Accum<D>& st, float (&ef)[4]) {
  const float lmax = __builtin_fmaxf(__builtin_fmaxf(s[0], s[1]), __builtin_fmaxf(s[2], s[3]));
  const bool bad =
      ln.real && (!(lmax <= st.m_ref + kRescaleLog2) || !__builtin_isfinite(st.m_ref));
  // Accumulator row r of this lane is head grp*4 + r, whose alpha lives in lane
  // grp*4 + r. The factors are found only on the rare rescale path, but applied
  // unconditionally: a multiply inside the branch makes the compiler keep a second
  // copy of every accumulator register across the loop.
  float ar[4] = {1.0f, 1.0f, 1.0f, 1.0f};
  if (__builtin_amdgcn_ballot_w64(bad) != 0) {
    float x = lmax;
    x = __builtin_fmaxf(x, __shfl_xor(x, 16));
    x = __builtin_fmaxf(x, __shfl_xor(x, 32));
    const float mn = __builtin_fmaxf(st.m_ref, x);
    const float alpha = (mn == -__builtin_inff()) ? 1.0f : __builtin_amdgcn_exp2f(st.m_ref - mn);
    st.l_part *= alpha;
    st.m_ref = mn;
#pragma unroll
    for (int r = 0; r < 4; r++) ar[r] = __shfl(alpha, ln.grp * 4 + r);
  }
#pragma unroll
  for (int m = 0; m < D / 16; m++)
#pragma unroll
    for (int r = 0; r < 4; r++) st.acc[m][r] *= ar[r];
  const bool dead = (st.m_ref == -__builtin_inff());
  f16x4 pw;
#pragma unroll
  for (int r = 0; r < 4; r++) {
    const float sv = s[r];
    // all scores so far -inf/NaN: weight 0, but a NaN score stays NaN
    const float e = dead ? (sv != sv ? sv : 0.0f) : __builtin_amdgcn_exp2f(sv - st.m_ref);
    st.l_part += e;
    ef[r] = e;
    pw[r] = (_Float16)e;
  }
  return pw;
}
template <int D>
__device__ __forceinline__ f16x4 softmax_block(const float (&s)[4], const Lane& ln,
                                               Accum<D>& st) {
  float ef[4];
  return softmax_block<D>(s, ln, st, ef);
}

// O += P . V for one block. Tokens at or past `end` carry weight 0 but their V
// bytes may be anything (0 * NaN = NaN), so a partial block zeroes them first.
template <int D>
__device__ __forceinline__ void mask_v_tail(u32x2_t (&vr)[D / 16], const Lane& ln, int32_t t0,
                                            int32_t end) {
  if (t0 + B > end) {
    const int nv = end - (t0 + ln.grp * 4);  // valid tokens among this lane's 4
    const uint32_t m0 = nv >= 2 ? 0xffffffffu : (nv == 1 ? 0x0000ffffu : 0u);
    const uint32_t m1 = nv >= 4 ? 0xffffffffu : (nv == 3 ? 0x0000ffffu : 0u);
#pragma unroll
    for (int m = 0; m < D / 16; m++) {
      vr[m].x &= m0;
      vr[m].y &= m1;
    }
  }
}

template <int D>
__device__ __forceinline__ void pv_block(u32x2_t (&vr)[D / 16], f16x4 pw, const Lane& ln,
                                         int32_t t0, int32_t end, Accum<D>& st) {
  mask_v_tail<D>(vr, ln, t0, end);
#pragma unroll
  for (int m = 0; m < D / 16; m++)
    st.acc[m] = __builtin_amdgcn_mfma_f32_16x16x16f16(pw, __builtin_bit_cast(f16x4, vr[m]),
                                                      st.acc[m], 0, 0, 0);
}

// K tile [D/8][B][8]: lane (col, grp) reads run (c*4 + grp) of token col; one
// load instruction covers runs c*4 .. c*4+3 of all 16 tokens (1 KiB).
template <int D>
__device__ __forceinline__ void load_k(const uint8_t* ktile, const Lane& ln,
                                       uint4 (&kr)[D / 32]) {
  const uint8_t* t = ktile + ((uint64_t)ln.grp * B + ln.col) * 16;
#pragma unroll
  for (int c = 0; c < D / 32; c++) kr[c] = load_stream16(t + c * 4 * B * 16);
}

// V tile [D][B]: lane (col, grp) reads tokens grp*4 .. +3 of dim 16m + col.
template <int D>
__device__ __forceinline__ void load_v(const uint8_t* vtile, const Lane& ln,
                                       u32x2_t (&vr)[D / 16]) {
  const uint8_t* t = vtile + ((uint64_t)ln.col * B + ln.grp * 4) * 2;
#pragma unroll
  for (int m = 0; m < D / 16; m++) vr[m] = load_stream8(t + m * 16 * B * 2);
}

// Registers of one block's K and V tiles as loaded, and their f16 MFMA operands
// (the operand orders of load_k / load_v above).
template <int DT, int D>
struct BlockRegs;

template <int D>
struct BlockRegs<kDtypeF16, D> {
  uint4 k[D / 32];
  u32x2_t v[D / 16];
  __device__ __forceinline__ void load_k_tile(const uint8_t* kt, const Lane& ln) {
    load_k<D>(kt, ln, k);
  }
  __device__ __forceinline__ void load_v_tile(const uint8_t* vt, const Lane& ln) {
    load_v<D>(vt, ln, v);
  }
  __device__ __forceinline__ void k_operand(uint4 (&kr)[D / 32]) const {
#pragma unroll
    for (int c = 0; c < D / 32; c++) kr[c] = k[c];
  }
  __device__ __forceinline__ void v_operand(u32x2_t (&vr)[D / 16]) const {
#pragma unroll
    for (int m = 0; m < D / 16; m++) vr[m] = v[m];
  }
};

// int8 pair -> exact binary16 pair. u holds four int8 with the sign bit flipped
// (x + 128 as unsigned); sel picks bytes (0, 1) or (2, 3). Each picked byte
// becomes the low mantissa byte of binary16 0x64XX = 1024 + (x + 128), and
// subtracting 1152 leaves x exactly.
__device__ __forceinline__ f16x2 i8_pair_to_f16(uint32_t u, uint32_t sel) {
  const uint32_t b = __builtin_amdgcn_perm(0x64646464u, u, sel);
  return __builtin_bit_cast(f16x2, b) - (f16x2){(_Float16)1152.0f, (_Float16)1152.0f};
}
constexpr uint32_t kSelLo = 0x04010400u;  // bytes 0, 1 under 0x64
constexpr uint32_t kSelHi = 0x04030402u;  // bytes 2, 3 under 0x64

// Q8_0 tiles: int8 quants in the operand order (q8_quant_offset: lane l = grp*16 +
// col holds 32 contiguous bytes of the block, 1 KiB per load instruction), then
// the f16 scales [B][D/32] (one per 32-dim group of a token). The operands are
// the dequantised values as binary16: the int8 -> binary16 step is exact and the
// product with the scale is rounded once (v_pk_mul_f16), which is the value an
// f16 pool would hold for the reference's f32 dequant
// (f16_to_f32(scale) * (i8 as f32), crates/kernels/src/scalar.rs:268-275).
template <int D>
struct BlockRegs<kDtypeQ8, D> {
  static constexpr int NG = D / 32;  // scale groups per token (= QK chunks)
  static_assert(D % 64 == 0, "Q8_0 tiles pair the 32-dim chunks");
  u32x2_t kq[NG];       // chunk c: dims c*32 + grp*8 .. +7 of token col
  uint32_t ks[NG / 2];  // the NG scales of token col
  uint32_t vq[D / 16];  // tile m: tokens grp*4 .. +3 of dim 16m + col
  uint32_t vs[2 * NG];  // the scales of tokens grp*4 .. +3: [4][NG]
  // LDS: the tile is a byte copy staged in shared memory (chunked prefill), read with
  // ordinary loads; otherwise it is in the pool, read with the streaming hint.
  template <bool LDS = false>
  __device__ __forceinline__ void load_k_tile(const uint8_t* kt, const Lane& ln) {
    const uint8_t* lp = kt + (uint64_t)ln.lane * 16;
#pragma unroll
    for (int p = 0; p < NG / 2; p++) {  // chunks 2p, 2p + 1
      const uint4 w = LDS ? *(const uint4*)(lp + p * 1024) : load_stream16(lp + p * 1024);
      kq[2 * p] = (u32x2_t){w.x, w.y};
      kq[2 * p + 1] = (u32x2_t){w.z, w.w};
    }
    const uint8_t* sc = kt + (uint64_t)B * D + (uint64_t)ln.col * NG * 2;
    if constexpr (NG == 4) {
      const u32x2_t w = LDS ? *(const u32x2_t*)sc : load_stream8(sc);
      ks[0] = w.x;
      ks[1] = w.y;
    } else {
      ks[0] = LDS ? *(const uint32_t*)sc : __builtin_nontemporal_load((const uint32_t*)sc);
    }
  }
  template <bool LDS = false>
  __device__ __forceinline__ void load_v_tile(const uint8_t* vt, const Lane& ln) {
    const uint8_t* lp = vt + (uint64_t)ln.lane * 16;
#pragma unroll
    for (int p = 0; p < D / 64; p++) {  // dim tiles 4p .. 4p + 3
      const uint4 w = LDS ? *(const uint4*)(lp + p * 1024) : load_stream16(lp + p * 1024);
      vq[4 * p] = w.x;
      vq[4 * p + 1] = w.y;
      vq[4 * p + 2] = w.z;
      vq[4 * p + 3] = w.w;
    }
    const uint8_t* sc = vt + (uint64_t)B * D + (uint64_t)ln.grp * 4 * NG * 2;
#pragma unroll
    for (int i = 0; i < NG / 2; i++) {
      const uint4 w = LDS ? *(const uint4*)(sc + i * 16) : load_stream16(sc + i * 16);
      vs[4 * i] = w.x;
      vs[4 * i + 1] = w.y;
      vs[4 * i + 2] = w.z;
      vs[4 * i + 3] = w.w;
    }
  }
  __device__ __forceinline__ void k_operand(uint4 (&kr)[D / 32]) const {
#pragma unroll
    for (int c = 0; c < NG; c++) {
      const uint32_t sw = ks[c / 2];
      const f16x2 s2 = __builtin_bit_cast(
          f16x2, __builtin_amdgcn_perm(sw, sw, (c & 1) ? 0x03020302u : 0x01000100u));
      const uint32_t w0 = kq[c].x ^ 0x80808080u, w1 = kq[c].y ^ 0x80808080u;
      kr[c] = make_uint4(__builtin_bit_cast(uint32_t, i8_pair_to_f16(w0, kSelLo) * s2),
                         __builtin_bit_cast(uint32_t, i8_pair_to_f16(w0, kSelHi) * s2),
                         __builtin_bit_cast(uint32_t, i8_pair_to_f16(w1, kSelLo) * s2),
                         __builtin_bit_cast(uint32_t, i8_pair_to_f16(w1, kSelHi) * s2));
    }
  }
  __device__ __forceinline__ void v_operand(u32x2_t (&vr)[D / 16]) const {
#pragma unroll
    for (int m = 0; m < D / 16; m++) {
      const int gg = m / 2;  // dims 16m .. 16m + 15 lie in group m / 2
      // scale of (token r, group gg) is half (gg & 1) of dword r * NG / 2 + gg / 2
      const uint32_t sel = (gg & 1) ? 0x07060302u : 0x05040100u;
      const f16x2 s01 = __builtin_bit_cast(
          f16x2, __builtin_amdgcn_perm(vs[NG / 2 + gg / 2], vs[gg / 2], sel));
      const f16x2 s23 = __builtin_bit_cast(
          f16x2, __builtin_amdgcn_perm(vs[3 * NG / 2 + gg / 2], vs[NG + gg / 2], sel));
      const uint32_t w = vq[m] ^ 0x80808080u;
      vr[m].x = __builtin_bit_cast(uint32_t, i8_pair_to_f16(w, kSelLo) * s01);
      vr[m].y = __builtin_bit_cast(uint32_t, i8_pair_to_f16(w, kSelHi) * s23);
    }
  }

  // ---- exact path (qk_block_q8x / pv_block_q8x), for pools holding a scale >= 512 ----

  // K operand of chunk c without its scale: the quants as binary16, exactly.
  __device__ __forceinline__ uint4 k_quants_chunk(int c) const {
    const uint32_t w0 = kq[c].x ^ 0x80808080u, w1 = kq[c].y ^ 0x80808080u;
    return make_uint4(__builtin_bit_cast(uint32_t, i8_pair_to_f16(w0, kSelLo)),
                      __builtin_bit_cast(uint32_t, i8_pair_to_f16(w0, kSelHi)),
                      __builtin_bit_cast(uint32_t, i8_pair_to_f16(w1, kSelLo)),
                      __builtin_bit_cast(uint32_t, i8_pair_to_f16(w1, kSelHi)));
  }
  // Scale dwords of the QK output's tokens grp*4 + r: token t's are ks of lane t.
  __device__ __forceinline__ void k_scales_out(const Lane& ln, uint32_t (&o)[4][NG / 2]) const {
#pragma unroll
    for (int r = 0; r < 4; r++)
#pragma unroll
      for (int i = 0; i < NG / 2; i++) o[r][i] = (uint32_t)__shfl((int)ks[i], ln.grp * 4 + r);
  }
  // V quants of tile m (tokens grp*4 .. +3 of dim 16m + col) as bf16, exactly.
  __device__ __forceinline__ s16x4 v_quants_bf16(int m) const {
    const uint32_t w = vq[m];
    const uint32_t f0 = __builtin_bit_cast(uint32_t, (float)(int8_t)(w & 0xffu));
    const uint32_t f1 = __builtin_bit_cast(uint32_t, (float)(int8_t)((w >> 8) & 0xffu));
    const uint32_t f2 = __builtin_bit_cast(uint32_t, (float)(int8_t)((w >> 16) & 0xffu));
    const uint32_t f3 = __builtin_bit_cast(uint32_t, (float)(int8_t)(w >> 24));
    const u32x2_t p = {__builtin_amdgcn_perm(f1, f0, 0x07060302u),
                       __builtin_amdgcn_perm(f3, f2, 0x07060302u)};
    return __builtin_bit_cast(s16x4, p);
  }
  // Scale (f16 bits) of V token grp*4 + r, group gg.
  __device__ __forceinline__ uint32_t v_scale_bits(int r, int gg) const {
    return (vs[r * NG / 2 + gg / 2] >> (16 * (gg & 1))) & 0xffffu;
  }

  // The fused append's token (quants q[kv][d], scales sc[kv][group]) in place of what
  // was loaded for token off: lanes read it and keep it only if they hold token off.
  __device__ __forceinline__ void patch_token(const Lane& ln, int off, const uint8_t (*q)[D],
                                              const uint16_t (*sc)[D / 32]) {
    const bool kme = ln.col == off, vme = ln.grp == off / 4;
    const int r = off & 3, sh = 8 * r;
#pragma unroll
    for (int c = 0; c < NG; c++) {
      const u32x2_t t = *(const u32x2_t*)&q[0][c * 32 + ln.grp * 8];
      kq[c].x = kme ? t.x : kq[c].x;
      kq[c].y = kme ? t.y : kq[c].y;
    }
#pragma unroll
    for (int i = 0; i < NG / 2; i++) {
      const uint32_t tk = *(const uint32_t*)&sc[0][2 * i], tv = *(const uint32_t*)&sc[1][2 * i];
      ks[i] = kme ? tk : ks[i];
#pragma unroll
      for (int rr = 0; rr < 4; rr++)
        vs[rr * NG / 2 + i] = (vme && rr == r) ? tv : vs[rr * NG / 2 + i];
    }
#pragma unroll
    for (int m = 0; m < D / 16; m++) {
      const uint32_t t = (vq[m] & ~(0xffu << sh)) | ((uint32_t)q[1][m * 16 + ln.col] << sh);
      vq[m] = vme ? t : vq[m];
    }
  }
};

// Exact Q8_0 scores of one block: the reference's dot over scale x quant in f32
// (crates/kernels/src/scalar.rs:268-275), as sum over 32-dim chunks c of
// scale[token][c] * (q . quants of chunk c). The quants are exact binary16 operands,
// q is the hi + lo split of prep_q, and the scales multiply the chunk's f32 result, so
// no value passes through the binary16 range whatever the scale.
template <int D>
__device__ __forceinline__ void qk_block_q8x(const BlockRegs<kDtypeQ8, D>& rg,
                                             const f16x8 (&qh)[D / 32], const f16x8 (&ql)[D / 32],
                                             float hscale, const Lane& ln, bool live, int32_t t0,
                                             int32_t end, float (&s)[4]) {
  constexpr int NG = D / 32;
  uint32_t sc[4][NG / 2];
  rg.k_scales_out(ln, sc);
  float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  // One chunk at a time (sched_barrier): the exact loop runs beside the fast loop's
  // register allocation and must not hold every chunk's products at once.
#pragma unroll
  for (int c = 0; c < NG; c++) {
    __builtin_amdgcn_sched_barrier(0);
    const f16x8 kv = __builtin_bit_cast(f16x8, rg.k_quants_chunk(c));
    const f32x4 zero = {0.0f, 0.0f, 0.0f, 0.0f};
    const f32x4 th = __builtin_amdgcn_mfma_f32_16x16x32_f16(kv, qh[c], zero, 0, 0, 0);
    const f32x4 tl = __builtin_amdgcn_mfma_f32_16x16x32_f16(kv, ql[c], zero, 0, 0, 0);
#pragma unroll
    for (int r = 0; r < 4; r++) {
      const float sum = th[r] + tl[r];  // see qk_block: a NaN sum, hi chain not NaN
      const float x = (sum != sum && th[r] == th[r]) ? th[r] : sum;
      const float d = f16_bits_to_f32((sc[r][c / 2] >> (16 * (c & 1))) & 0xffffu);
      acc[r] = __builtin_fmaf(d, x, acc[r]);
    }
  }
#pragma unroll
  for (int r = 0; r < 4; r++) {
    const bool ok = ln.real && live && t0 + ln.grp * 4 + r < end;
    s[r] = ok ? acc[r] * hscale : -__builtin_inff();
  }
}

// Exact Q8_0 O += P . V of one block: per 32-dim group, the f32 softmax weight times
// the token's V scale in f32, split into three bf16 parts (24 significant bits: the
// f32 product to within its last bit, in bf16's range), against the quants as bf16
// (exact). Tokens at or past `end` get weight 0 and their scales are not read.
template <int D>
__device__ __forceinline__ void pv_block_q8x(const BlockRegs<kDtypeQ8, D>& rg,
                                             const float (&w)[4], const Lane& ln, int32_t t0,
                                             int32_t end, Accum<D>& st) {
  constexpr int NG = D / 32;
  const int nvt = end - (t0 + ln.grp * 4);  // valid tokens among this lane's 4
#pragma unroll
  for (int gg = 0; gg < NG; gg++) {
    __builtin_amdgcn_sched_barrier(0);
    uint32_t part[3][4];
#pragma unroll
    for (int r = 0; r < 4; r++) {
      float y = r < nvt ? w[r] * f16_bits_to_f32(rg.v_scale_bits(r, gg)) : 0.0f;
#pragma unroll
      for (int k = 0; k < 3; k++) {  // truncate to bf16, keep the exact remainder
        const uint32_t yb = __builtin_bit_cast(uint32_t, y);
        part[k][r] = yb >> 16;
        y -= __builtin_bit_cast(float, yb & 0xffff0000u);
      }
    }
    s16x4 p[3];
#pragma unroll
    for (int k = 0; k < 3; k++)
      p[k] = __builtin_bit_cast(
          s16x4, (u32x2_t){part[k][0] | (part[k][1] << 16), part[k][2] | (part[k][3] << 16)});
#pragma unroll
    for (int m = 2 * gg; m < 2 * gg + 2; m++) {
      const s16x4 vb = rg.v_quants_bf16(m);
#pragma unroll
      for (int k = 0; k < 3; k++)
        st.acc[m] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(p[k], vb, st.acc[m], 0, 0, 0);
    }
  }
}

// ---------------------------------------------------------------------------
// Persistent streaming kernel
// ---------------------------------------------------------------------------

// Block-count prefix of the sequences (clamped contexts) into s_pre[0..n_seqs]
// by one 256-thread workgroup.
__device__ void block_prefix(const int32_t* __restrict__ ctx_lens, uint32_t n_seqs, int32_t cap,
                             uint32_t* s_pre, uint32_t* s_tmp, uint32_t* fault, bool report) {
  const uint32_t tid = threadIdx.x;
  const uint32_t per = (n_seqs + 255u) / 256u;
  const uint32_t lo = tid * per < n_seqs ? tid * per : n_seqs;
  const uint32_t hi = lo + per < n_seqs ? lo + per : n_seqs;
  uint32_t sum = 0;
  for (uint32_t i = lo; i < hi; i++) {
    int32_t c = ctx_lens[i];
    if (c < 0 || c > cap) {
      if (report) raise_fault(fault, kFaultCtx);
      c = c < 0 ? 0 : cap;
    }
    const uint32_t nb = (uint32_t)(c + B - 1) / B;
    s_pre[i] = nb;
    sum += nb;
  }
  s_tmp[tid] = sum;
  __syncthreads();
  if (tid < 64) {  // exclusive scan of the 256 chunk sums by wave 0
    uint32_t v[4], t = 0;
#pragma unroll
    for (int k = 0; k < 4; k++) {
      v[k] = t;
      t += s_tmp[tid * 4 + k];
    }
    uint32_t incl = t;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const uint32_t y = __shfl_up(incl, o);
      if ((int)tid >= o) incl += y;
    }
    const uint32_t excl = incl - t;
#pragma unroll
    for (int k = 0; k < 4; k++) s_tmp[tid * 4 + k] = excl + v[k];
  }
  __syncthreads();
  uint32_t run = s_tmp[tid];
  for (uint32_t i = lo; i < hi; i++) {
    const uint32_t nb = s_pre[i];
    s_pre[i] = run;
    run += nb;
  }
  if (tid == 255) s_pre[n_seqs] = run;
  __syncthreads();
}

// Waves that share T flattened items: all of the grid's, but never more than T.
__device__ __forceinline__ uint64_t stream_waves(uint64_t grid_waves, uint64_t T) {
  return grid_waves < T ? grid_waves : T;
}

// Wave owning flattened item x: the largest w with floor(w * T / NW) <= x.
__device__ __forceinline__ uint64_t wave_of(uint64_t x, uint64_t T, uint64_t NW) {
  return ((x + 1) * NW - 1) / T;
}

// Three waves per SIMD: 170 VGPRs at most (unconstrained the compiler takes 186
// at D = 128 and the CU holds only two of these workgroups).
#ifndef FKV_STREAM_WAVES_PER_EU
#define FKV_STREAM_WAVES_PER_EU 3
#endif

template <int D>
__global__ void __launch_bounds__(256)
__attribute__((amdgpu_waves_per_eu(FKV_STREAM_WAVES_PER_EU, 8))) attn_mfma_stream_kernel(
    Geom g, uint32_t layer, uint32_t n_heads, uint32_t G, const float* __restrict__ q,
    float* __restrict__ out, const int32_t* __restrict__ tables, uint32_t max_blocks,
    const int32_t* __restrict__ ctx_lens, uint32_t n_seqs, float scale,
    uint32_t* __restrict__ ws_pre, float* __restrict__ ws_o, float* __restrict__ ws_ml) {
  constexpr int NC = D / 32, NM = D / 16;
  extern __shared__ uint32_t s_pre[];  // n_seqs + 1 block prefix sums
  __shared__ uint32_t s_tmp[256];

  const int32_t cap = (int32_t)(max_blocks * B);
  block_prefix(ctx_lens, n_seqs, cap, s_pre, s_tmp, g.fault, blockIdx.x == 0);
  if (blockIdx.x == 0)
    for (uint32_t i = threadIdx.x; i <= n_seqs; i += 256) ws_pre[i] = s_pre[i];

  // Every value read from the prefix table is the same in all lanes; readfirstlane
  // keeps the cursor arithmetic in scalar registers.
  auto pre = [&](uint32_t i) { return (uint32_t)__builtin_amdgcn_readfirstlane(s_pre[i]); };
  const uint64_t hkv = g.n_kv_heads;
  const uint64_t T = hkv * pre(n_seqs);
  // At most one wave per item, so every wave that takes part owns at least one.
  const uint64_t NW = stream_waves((uint64_t)gridDim.x * kAttnWaves, T);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const uint64_t w = (uint64_t)blockIdx.x * kAttnWaves + wave;
  if (w >= NW) return;
  const uint64_t a = w * T / NW, b_end = (w + 1) * T / NW;

  Lane ln;
  ln.lane = threadIdx.x & 63;
  ln.col = ln.lane & 15;
  ln.grp = ln.lane >> 4;
  ln.real = ln.col < (int)G;
  const float qscale = scale * kLog2e;

  // Cursor over (sequence, KV head, block), starting at item a.
  struct Cursor {
    uint32_t s, kvh, bi, nb;
    uint64_t seg0;  // flattened index of the segment's first item
  };
  Cursor cur;
  {
    uint32_t lo = 0, hi = n_seqs;  // largest s with hkv * s_pre[s] <= a: it has blocks
    while (hi - lo > 1) {
      const uint32_t mid = (lo + hi) / 2;
      if (hkv * pre(mid) <= a) lo = mid;
      else hi = mid;
    }
    cur.s = lo;
    cur.nb = pre(lo + 1) - pre(lo);
    const uint64_t rel = a - hkv * pre(lo);
    cur.kvh = (uint32_t)(rel / cur.nb);
    cur.bi = (uint32_t)(rel % cur.nb);
    cur.seg0 = hkv * pre(lo) + (uint64_t)cur.kvh * cur.nb;
  }
  auto advance = [&](Cursor c) {
    if (++c.bi == c.nb) {
      c.bi = 0;
      c.seg0 += c.nb;
      if (++c.kvh == hkv) {
        c.kvh = 0;
        do {
          c.s++;
        } while (pre(c.s + 1) == pre(c.s));  // skip sequences without blocks
        c.nb = pre(c.s + 1) - pre(c.s);
      }
    }
    return c;
  };
  // Physical block of an item; an entry outside the pool raises the fault flag,
  // reads block 0 instead and is skipped.
  auto phys = [&](const Cursor& c, bool& ok) {
    const int32_t p = __builtin_amdgcn_readfirstlane(tables[(uint64_t)c.s * max_blocks + c.bi]);
    ok = p >= 0 && (uint64_t)p < g.num_blocks;
    if (!ok && ln.lane == 0) raise_fault(g.fault, kFaultBlock);
    return ok ? (uint64_t)p : 0;
  };

  uint4 kr[NC];
  u32x2_t vr[NM];
  bool live;
  {
    const uint64_t p = phys(cur, live);
    load_k<D>(tile_ptr(g, p, layer, 0, cur.kvh), ln, kr);
    load_v<D>(tile_ptr(g, p, layer, 1, cur.kvh), ln, vr);
  }
  f16x8 qh[NC], ql[NC];
  float hscale;
  Accum<D> st;

  uint64_t i = a;
  for (;;) {  // one (sequence, KV head) segment per pass; cur is its first item here
    const uint32_t seq = cur.s, kvh = cur.kvh, nb = cur.nb;
    const uint64_t seg0 = cur.seg0;
    const uint64_t stop = seg0 + nb < b_end ? seg0 + nb : b_end;
    int32_t end = __builtin_amdgcn_readfirstlane(ctx_lens[seq]);
    end = end < 0 ? 0 : (end > cap ? cap : end);
    prep_q<D>(q + ((uint64_t)seq * n_heads + (uint64_t)kvh * G + (ln.real ? ln.col : 0)) * D, ln,
            qscale, qh, ql, hscale);
    st.reset();

    for (; i < stop; i++) {
      const bool more = i + 1 < b_end;
      const int32_t t0 = (int32_t)cur.bi * B;
      float s[4];
      qk_block<D>(kr, qh, ql, hscale, ln, live, t0, end, s);
      const bool cur_live = live;
      uint64_t np = 0;
      if (more) {  // next item, possibly the next segment's first
        cur = advance(cur);
        np = phys(cur, live);
        load_k<D>(tile_ptr(g, np, layer, 0, cur.kvh), ln, kr);
      }
      const f16x4 pw = softmax_block<D>(s, ln, st);
      if (cur_live) pv_block<D>(vr, pw, ln, t0, end, st);
      if (more) load_v<D>(tile_ptr(g, np, layer, 1, cur.kvh), ln, vr);
    }

    // The wave's last item of this segment.
    float lsum = st.l_part;
    lsum += __shfl_xor(lsum, 16);
    lsum += __shfl_xor(lsum, 32);
    const uint64_t head0 = (uint64_t)seq * n_heads + (uint64_t)kvh * G;
    if (seg0 >= a && seg0 + nb <= b_end) {  // whole segment in this wave: final output
      // M and L of head grp*4 + r live in lane grp*4 + r
#pragma unroll
      for (int r = 0; r < 4; r++) {
        const int h = ln.grp * 4 + r;
        const float M = __shfl(st.m_ref, h);
        const float L = __shfl(lsum, h);
        const float inv = 1.0f / L;
        if (h < (int)G) {
#pragma unroll
          for (int m = 0; m < NM; m++)
            out[(head0 + h) * D + m * 16 + ln.col] =
                __builtin_isfinite(M) ? st.acc[m][r] * inv : 0.0f;
        }
      }
    } else {
      const uint64_t slot = w + (uint64_t)seq * hkv + kvh;
#pragma unroll
      for (int r = 0; r < 4; r++) {
        const int h = ln.grp * 4 + r;
        if (h < (int)G) {
#pragma unroll
          for (int m = 0; m < NM; m++)
            ws_o[(slot * G + h) * D + m * 16 + ln.col] = st.acc[m][r];
        }
      }
      if (ln.lane < (int)G) {
        ws_ml[(slot * G + ln.lane) * 2] = st.m_ref;  // log2 domain
        ws_ml[(slot * G + ln.lane) * 2 + 1] = lsum;
      }
    }
    if (i >= b_end) break;
  }
}

// Merges the partials of every (sequence, KV head) segment that the stream
// kernel cut between waves; one workgroup per (segment, query head of the group).
// Segments held whole by one wave were written by the stream kernel; empty ones
// (context 0) get zeros. 256 threads: dims 4*(t % (D/4)) .., partial rows t / (D/4).
template <int D>
__global__ void __launch_bounds__(256) attn_stream_combine_kernel(
    uint32_t n_seqs, uint32_t hkv, uint32_t G, uint64_t grid_waves, const uint32_t* __restrict__ ws_pre,
    const float* __restrict__ ws_o, const float* __restrict__ ws_ml, float* __restrict__ out) {
  constexpr int kLanesPerRow = D / 4;
  constexpr int kRows = 256 / kLanesPerRow;
  __shared__ float s_red[kRows][D];
  __shared__ float s_lred[kRows];
  __shared__ float s_max[4];

  const uint32_t seg = blockIdx.x / G, h = blockIdx.x % G;
  const uint32_t s = seg / hkv, kvh = seg % hkv;
  const uint32_t nb = ws_pre[s + 1] - ws_pre[s];
  float* o = out + ((uint64_t)s * hkv * G + (uint64_t)kvh * G + h) * D;
  if (nb == 0) {
    for (int d = threadIdx.x; d < D; d += 256) o[d] = 0.0f;
    return;
  }
  const uint64_t T = (uint64_t)hkv * ws_pre[n_seqs];
  const uint64_t NW = stream_waves(grid_waves, T);
  const uint64_t seg0 = (uint64_t)hkv * ws_pre[s] + (uint64_t)kvh * nb;
  const uint64_t wf = wave_of(seg0, T, NW), wl = wave_of(seg0 + nb - 1, T, NW);
  if (wf == wl) return;
  const uint32_t np = (uint32_t)(wl - wf + 1);
  const uint64_t slot0 = wf + seg;  // slot of partial p: wf + p + seg
  const int wave = threadIdx.x / 64, lane = threadIdx.x % 64;

  float m = -__builtin_inff();
  for (uint32_t p = threadIdx.x; p < np; p += 256)
    m = __builtin_fmaxf(m, ws_ml[((slot0 + p) * G + h) * 2]);
  m = wave_max(m);
  if (lane == 0) s_max[wave] = m;
  __syncthreads();
  const float M = __builtin_fmaxf(__builtin_fmaxf(s_max[0], s_max[1]),
                                  __builtin_fmaxf(s_max[2], s_max[3]));
  if (!__builtin_isfinite(M)) {
    for (int d = threadIdx.x; d < D; d += 256) o[d] = 0.0f;
    return;
  }
  const int col = threadIdx.x % kLanesPerRow, row = threadIdx.x / kLanesPerRow;
  float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
  float lsum = 0.0f;
  for (uint32_t p = row; p < np; p += kRows) {
    const uint64_t sl = (slot0 + p) * G + h;
    const float mp = ws_ml[sl * 2];
    const float wgt = (mp == -__builtin_inff()) ? 0.0f : __builtin_amdgcn_exp2f(mp - M);
    lsum = __builtin_fmaf(wgt, ws_ml[sl * 2 + 1], lsum);
    const float4 v = *(const float4*)(ws_o + sl * D + col * 4);
    acc.x = __builtin_fmaf(wgt, v.x, acc.x);
    acc.y = __builtin_fmaf(wgt, v.y, acc.y);
    acc.z = __builtin_fmaf(wgt, v.z, acc.z);
    acc.w = __builtin_fmaf(wgt, v.w, acc.w);
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

// ---------------------------------------------------------------------------
// Split kernel (one workgroup per (sequence, KV head, split))
// ---------------------------------------------------------------------------

// Work order of the split grid.
//
// Within each XCD, the hardware hands a launch's workgroups to the shader engines
// in a fixed rotation, whatever their load; each engine then runs its share on
// its own CUs. With one workgroup per (sequence, KV head, split) in grid order,
// every split of a sequence falls to the same engine. The engines' loads then
// differ as much as sums of random context lengths do, and the most loaded engine
// sets the kernel's end.
//
// In the longest-first order, workgroup r of the launch takes unit r / n_kv_heads
// (KV head r % n_kv_heads) of this list:
// - every full split (split_tokens positions) of every sequence, sequence-major;
// - then each sequence's last, partial split, including the zero-length one of an
//   empty context. These are taken by block count, largest first, ties by
//   sequence (n_seqs <= 256); for larger batches, in sequence order.
// Ranks past the list exit at once. A rotation dealing from a list sorted this
// way gives every engine the same work to within about one item.
enum : uint32_t { kOrderGrid = 0, kOrderFullFirst = 1, kOrderLongestFirst = 2 };
constexpr uint32_t kOrderMaxSeqs = 1024;    // contiguous runs of <= 4 sequences per thread
constexpr uint32_t kOrderSortSeqs = 256;    // one sequence per thread for the block-count ranks

struct OrderedItem {
  int32_t seq;    // < 0: past the list
  int32_t split;
  int32_t ctx;    // ctx_lens[seq] as read (unclamped)
  int32_t marks;  // *marks_word as thread 0 read it (0 without one)
};

// Unit u of the longest-first list. Every thread of the workgroup calls this with
// the same u and receives the same item.
__device__ OrderedItem ordered_item(uint32_t u, const int32_t* __restrict__ ctx_lens,
                                    uint32_t n_seqs, int32_t cap, int32_t split_tokens,
                                    uint32_t order, int32_t* s_scan, int32_t* s_key,
                                    int32_t* s_res, const uint32_t* marks_word) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int K = (int)((n_seqs + 255u) / 256u);  // <= 4
  int32_t raw[4], full[4], part[4];
  int32_t fsum = 0, psum = 0;
#pragma unroll
  for (int k = 0; k < 4; k++) {
    const int s = tid * K + k;
    raw[k] = 0;
    full[k] = part[k] = 0;
    if (k < K && s < (int)n_seqs) {
      raw[k] = ctx_lens[s];
      const int32_t c = raw[k] < 0 ? 0 : (raw[k] > cap ? cap : raw[k]);
      full[k] = c / split_tokens;
      part[k] = (c == 0 || c % split_tokens != 0) ? 1 : 0;
    }
    fsum += full[k];
    psum += part[k];
  }
  if (order == kOrderLongestFirst) {  // K == 1: sort key of the thread's partial split
    const int32_t c = raw[0] < 0 ? 0 : (raw[0] > cap ? cap : raw[0]);
    const int32_t nb = (c - full[0] * split_tokens + B - 1) / B;  // <= 65536 blocks
    s_key[tid] = part[0] ? (((65536 - nb) << 10) | tid) : 0x7fffffff;
  }
  // Exclusive scans of the full and partial counts over the threads.
  int32_t fin = fsum, pin = psum;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int32_t a = __shfl_up(fin, o), b = __shfl_up(pin, o);
    if (lane >= o) {
      fin += a;
      pin += b;
    }
  }
  if (lane == 63) {
    s_scan[wave] = fin;
    s_scan[kAttnWaves + wave] = pin;
  }
  if (tid == 0) {
    s_res[0] = -1;
    s_res[3] = marks_word ? (int32_t)__atomic_load_n(marks_word, __ATOMIC_RELAXED) : 0;
  }
  __syncthreads();
  int32_t fpre = fin - fsum, ppre = pin - psum, F = 0, P = 0;
#pragma unroll
  for (int w = 0; w < kAttnWaves; w++) {
    if (w < wave) {
      fpre += s_scan[w];
      ppre += s_scan[kAttnWaves + w];
    }
    F += s_scan[w];
    P += s_scan[kAttnWaves + w];
  }
  if ((int64_t)u < F) {  // a full split: the thread whose run holds unit u
    if ((int32_t)u >= fpre && (int32_t)u < fpre + fsum) {
      int32_t base = fpre;
#pragma unroll
      for (int k = 0; k < 4; k++) {
        if ((int32_t)u >= base && (int32_t)u < base + full[k]) {
          s_res[0] = tid * K + k;
          s_res[1] = (int32_t)u - base;
          s_res[2] = raw[k];
        }
        base += full[k];
      }
    }
  } else if ((int64_t)u < (int64_t)F + P) {  // a sequence's last, partial split
    const int32_t p = (int32_t)u - F;
    if (order == kOrderLongestFirst) {
      if (part[0]) {
        const int32_t key = s_key[tid];
        int32_t rank = 0;
        for (int j = 0; j < (int)n_seqs; j++) rank += s_key[j] < key ? 1 : 0;
        if (rank == p) {
          s_res[0] = tid;
          s_res[1] = full[0];
          s_res[2] = raw[0];
        }
      }
    } else if (p >= ppre && p < ppre + psum) {
      int32_t base = ppre;
#pragma unroll
      for (int k = 0; k < 4; k++) {
        if (part[k] && p == base) {
          s_res[0] = tid * K + k;
          s_res[1] = full[k];
          s_res[2] = raw[k];
        }
        base += part[k];
      }
    }
  }
  __syncthreads();
  return OrderedItem{s_res[0], s_res[1], s_res[2], s_res[3]};
}

// Waves per SIMD the split kernel is compiled for (the VGPR budget: 4 -> 128).
#ifndef FKV_MFMA_WAVES_PER_EU
#define FKV_MFMA_WAVES_PER_EU 3
#endif

// EXACT (Q8_0 only): the instance for blocks holding scales of 512 or more. Every Q8_0
// call launches the fast instance and then this one over the same grid. Each workgroup
// of both reads the pool's count of marked blocks once; while it is 0 the fast one
// computes and the exact one leaves at once. Otherwise each ORs the marks of the blocks
// its split reads: the fast instance computes an unmarked split, the exact one a marked
// split, without binary16 dequantised operands (qk_block_q8x, pv_block_q8x). A fast
// workgroup whose appended token has such a scale marks that token's block, and the
// exact instance's workgroup for the same split then recomputes its outputs. Its own
// register allocation keeps the fast instance's at three waves per SIMD.
template <int DT, int D, int NBUF, bool ROPE, bool EXACT>
__global__ void __launch_bounds__(256)
__attribute__((amdgpu_waves_per_eu(EXACT ? 2 : FKV_MFMA_WAVES_PER_EU, 8))) attn_mfma_kernel(
    Geom g, uint32_t layer, uint32_t n_heads, uint32_t G, const float* __restrict__ q,
    float* __restrict__ out, const int32_t* __restrict__ tables, uint32_t max_blocks,
    const int32_t* __restrict__ ctx_lens, uint32_t n_seqs, uint32_t max_splits,
    int32_t split_tokens, uint32_t order, float scale, float* __restrict__ ws_o,
    float* __restrict__ ws_ml, const float* __restrict__ k_new, const float* __restrict__ v_new,
    const RopeTable rope) {
  constexpr int NC = D / 32, NM = D / 16;

  __shared__ float s_o[kAttnWaves][kHeads * D];
  __shared__ float s_m[kAttnWaves][kHeads];
  __shared__ float s_l[kAttnWaves][kHeads];
  __shared__ __align__(16) uint16_t s_app[2][D];  // fused append: K, V operand values
  __shared__ uint8_t s_appq[2][D];                 // fused Q8_0 append: quants
  __shared__ uint16_t s_apps[2][D / 32];           // and scales
  __shared__ int32_t s_ord[2 * kAttnWaves + 4 + kOrderSortSeqs];  // work order: scans, item, keys
  __shared__ uint32_t s_marks;  // the pool's count of marked blocks as this workgroup read it

  // the work list and the split clamp share this bound, so the list never holds more
  // items than the grid has workgroups
  const int32_t cap = dev::split_ctx_cap(max_blocks, B, max_splits, (uint32_t)split_tokens);
  // The exact instance has work only where a block is marked; the count cannot change
  // during its launch (only fast instances mark blocks), so each wave reads it alone.
  if constexpr (EXACT) {
    if (!pool_has_marks(g)) return;
  }
  const uint32_t kvh = blockIdx.x % g.n_kv_heads;
  uint32_t seq;
  int32_t split, ctx = 0;
  // Q8_0: whether any block of the pool is marked, read once per workgroup (a fast
  // workgroup appending a wide token marks a block during the launch, and the waves of
  // one workgroup must agree before the barrier of blocks_marked).
  bool any_marks = EXACT;
  if (order != kOrderGrid) {
    const OrderedItem it = ordered_item(
        blockIdx.x / g.n_kv_heads, ctx_lens, n_seqs, cap, split_tokens, order, s_ord,
        s_ord + 2 * kAttnWaves + 4, s_ord + 2 * kAttnWaves,
        DT == kDtypeQ8 && !EXACT ? g.fault + 1 : nullptr);
    if (it.seq < 0) return;
    seq = (uint32_t)it.seq;
    split = it.split;
    ctx = it.ctx;
    if constexpr (!EXACT) any_marks = it.marks != 0;
  } else {
    const uint32_t segs = n_seqs * g.n_kv_heads;
    seq = (blockIdx.x % segs) / g.n_kv_heads;
    split = (int32_t)(blockIdx.x / segs);
  }
  const int32_t s0 = split * split_tokens;
  const int32_t blk0 = s0 / B;  // < max_blocks for every grid row
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  Lane ln;
  ln.lane = threadIdx.x & 63;
  ln.col = ln.lane & 15;
  ln.grp = ln.lane >> 4;
  ln.real = ln.col < (int)G;

  // The wave's block-table entries, 64 at a time: lane j holds the entry of the
  // wave's block (t & ~63) + j. A block's physical id then comes from a register
  // (readlane) instead of a load that its K/V loads would have to wait for. In
  // grid order the first 64 are loaded before the context length is known
  // (indices clamped to the table row; entries past the split are never used),
  // so the two loads' latencies overlap.
  const int32_t* table = tables + (uint64_t)seq * max_blocks;
  int32_t tabv = 0;
  auto load_tab = [&](int tb) {
    int64_t j = (int64_t)blk0 + wave + (int64_t)kAttnWaves * (tb + ln.lane);
    if (j > (int64_t)max_blocks - 1) j = (int64_t)max_blocks - 1;
    tabv = j >= 0 ? table[j] : 0;
  };
  load_tab(0);
  if constexpr (DT == kDtypeQ8 && !EXACT) {
    if (order == kOrderGrid) {  // no ordering pass to carry the word: one barrier
      if (threadIdx.x == 0) s_marks = __atomic_load_n(g.fault + 1, __ATOMIC_RELAXED);
      __syncthreads();
      any_marks = s_marks != 0;
    }
  }

  if (order == kOrderGrid) ctx = ctx_lens[seq];
  const bool ctx_ok = ctx >= 0 && ctx <= cap;
  if (!ctx_ok) {
    if (split == 0 && threadIdx.x == 0 && kvh == 0) raise_fault(g.fault, kFaultCtx);
    ctx = ctx < 0 ? 0 : cap;
  }
  const int32_t nsplits = ctx > 0 ? (ctx + split_tokens - 1) / split_tokens : 1;
  if (split >= nsplits) return;
  const int32_t s1 = ctx - s0 < split_tokens ? ctx : s0 + split_tokens;
  const int32_t nblk = s1 > s0 ? (s1 - s0 + B - 1) / B : 0;
  // Q8_0 with marked blocks in the pool: the split's own marks pick the instance (the
  // fast one then only stores the appended token of a marked split).
  bool split_marked = false;
  if constexpr (DT == kDtypeQ8) {
    if (any_marks) split_marked = blocks_marked(g, table, blk0, blk0 + nblk);
    if constexpr (EXACT) {
      if (!split_marked) return;
    }
  }

  // RoPE at the new token's position ctx - 1: the lane holds (sin, cos) of pair
  // rope_pair(lane), pos / den[p] as the reference computes it (f32 division, then
  // sin and cos). Computed after the first K/V loads are issued, so the range
  // reduction of large angles overlaps their latency.
  float rsin = 0.0f, rcos = 1.0f;
  auto rope_angles = [&]() {
    const int pr = rope_pair(ln.lane);
    if (2 * pr < rope.rope_dim) {
      const uint32_t pos = (uint32_t)(ctx > 0 ? ctx - 1 : 0);
      if (rope.sc != nullptr && pos < rope.sc_pos) {
        const float2 v = *(const float2*)(rope.sc + ((uint64_t)pos * (uint32_t)(rope.rope_dim / 2) + pr) * 2u);
        rsin = v.x;
        rcos = v.y;
      } else {
        sincosf((float)pos / rope.den[pr], &rsin, &rcos);
      }
    }
  };

  // Fused append (k_new != nullptr): the token at position ctx - 1 of this KV
  // head is stored by the wave of the last split that reads its block. That wave
  // encodes the token up front (F16: f32 -> binary16 with the pool's rounding;
  // Q8_0: each 32-dim group quantised as append_q8_kernel does) and, when it
  // reaches the block, puts the operand values of the token (F16: the binary16
  // values; Q8_0: scale x quant rounded once to binary16, what the block's operand
  // conversion gives for the stored bytes) into its K and V operands in place of
  // what it loaded, and stores the encoded token to the pool. No other workgroup
  // reads the position, and this one never reads back what it stores, so the
  // stores need no ordering.
  const bool app = (DT == kDtypeF16 || DT == kDtypeQ8) && !EXACT && k_new != nullptr &&
                   split == nsplits - 1 && ctx > 0 && ctx_ok;
  const int32_t app_pos = ctx - 1;
  const int32_t app_lb = app ? app_pos / B - blk0 : -1;  // block of the split
  const bool app_wave = app && app_lb % kAttnWaves == wave;
  const int32_t app_t = app_lb / kAttnWaves;             // the wave's block index
  const int32_t app_off = app_pos % B;                   // token within the block
  // Encoded K and V rows of the token to s_app (the appending wave's own LDS use).
  // With RoPE the K row is rotated first; dims (dd & ~1, dd | 1) are a pair on
  // adjacent lanes.
  auto encode_app = [&]() {
    const float* ksrc = k_new + ((uint64_t)seq * g.n_kv_heads + kvh) * D;
    const float* vsrc = v_new + ((uint64_t)seq * g.n_kv_heads + kvh) * D;
#pragma unroll
    for (int i = 0; i < D / 64; i++) {
      const int dd = i * 64 + ln.lane;
      float kv = ksrc[dd];
      if constexpr (ROPE) {
        const int pr = dd >> 1;  // held by lane (pr%16/4)*16 + (pr/16)*4 + pr%4
        const int src = ((pr & 15) >> 2) * 16 + (pr >> 4) * 4 + (pr & 3);
        const float other = __shfl_xor(kv, 1);
        const float sn = __shfl(rsin, src), cs = __shfl(rcos, src);
        if (dd < rope.rope_dim) kv = (dd & 1) ? other * sn + kv * cs : kv * cs - other * sn;
      }
      const float vv = vsrc[dd];
      if constexpr (DT == kDtypeQ8) {
        // Group dd / 32 is this half of the wave: amax over its 32 lanes.
        float ka = __builtin_fabsf(kv), va = __builtin_fabsf(vv);
#pragma unroll
        for (int o = 1; o < 32; o <<= 1) {
          ka = __builtin_fmaxf(ka, __shfl_xor(ka, o));
          va = __builtin_fmaxf(va, __shfl_xor(va, o));
        }
        float kid, vid;
        const uint32_t ksc = encode_f16(q8_scale(ka, kid), g.rounding);
        const uint32_t vsc = encode_f16(q8_scale(va, vid), g.rounding);
        const int kq = q8_quant(kv, kid), vq = q8_quant(vv, vid);
        s_appq[0][dd] = (uint8_t)kq;
        s_appq[1][dd] = (uint8_t)vq;
        s_app[0][dd] = __builtin_bit_cast(uint16_t, (_Float16)(f16_bits_to_f32(ksc) * (float)kq));
        s_app[1][dd] = __builtin_bit_cast(uint16_t, (_Float16)(f16_bits_to_f32(vsc) * (float)vq));
        if ((ln.lane & 31) == 0) {
          s_apps[0][dd / 32] = (uint16_t)ksc;
          s_apps[1][dd / 32] = (uint16_t)vsc;
          // a scale past the binary16 range (append_q8_kernel's rule)
          if ((ksc & 0x7c00u) == 0x7c00u || (vsc & 0x7c00u) == 0x7c00u)
            raise_fault(g.fault, kFaultRange);
        }
        // A scale of 512 or more marks the token's block (q8_wide_scale): the exact
        // instance, launched after this one, then recomputes this split's outputs.
        if (__builtin_amdgcn_ballot_w64(q8_wide_scale(ksc) || q8_wide_scale(vsc)) != 0 &&
            ln.lane == 0)
          mark_table_block(g, table, app_pos / B);
      } else {
        const uint32_t ke = encode_f16(kv, g.rounding);
        s_app[0][dd] = (uint16_t)ke;
        const uint32_t ve = encode_f16(vv, g.rounding);
        s_app[1][dd] = (uint16_t)ve;
        // an Inf/NaN K or V marks the token's block (chunked prefill's leak-safe instance)
        if (__builtin_amdgcn_ballot_w64(f16_nonfinite(ke) || f16_nonfinite(ve)) != 0 &&
            ln.lane == 0)
          mark_table_block(g, table, app_pos / B);
      }
    }
  };
  if constexpr (!ROPE) {
    if (app_wave) encode_app();
  }
  // Q8_0 fast instance over a marked split: the exact instance computes this
  // workgroup's outputs; only the appended token is stored here.
  bool store_only = false;
  if constexpr (DT == kDtypeQ8 && !EXACT) store_only = split_marked;

  Accum<D> st;
  st.reset();

  // Ring of NBUF block buffers: wave w owns blocks w, w + 4, w + 8, ... of the
  // split; block t of the wave lives in buffer t % NBUF. Block t + NBUF's K load
  // is issued as soon as block t's QK has consumed the buffer, and its V load
  // once block t's P.V has.
  BlockRegs<DT, D> ring[NBUF];
  int32_t bid[NBUF];
  bool blive[NBUF];
  f16x8 qh[NC], ql[NC];
  float hscale;
  const int32_t nt = wave < nblk ? (nblk - wave + kAttnWaves - 1) / kAttnWaves : 0;

  // Physical block of the wave's block t (wave-uniform). A block-table entry
  // outside the pool raises the fault flag, loads block 0 instead and is skipped.
  auto fetch = [&](int t, int b) {
    if (t > 0 && (t & 63) == 0) load_tab(t);
    const int32_t p = __builtin_amdgcn_readlane(tabv, t & 63);
    const bool okb = p >= 0 && (uint64_t)p < g.num_blocks;
    if (!okb && ln.lane == 0) raise_fault(g.fault, kFaultBlock);
    blive[b] = okb;
    bid[b] = okb ? p : 0;
  };
  // The Q8_0 token's quants and scales to the pool (the whole appending wave).
  auto store_q8_token = [&](int b) {
    uint8_t* kt = tile_ptr(g, (uint64_t)bid[b], layer, 0, kvh);
    uint8_t* vt = tile_ptr(g, (uint64_t)bid[b], layer, 1, kvh);
#pragma unroll
    for (int i = 0; i < D / 64; i++) {
      const int dd = i * 64 + ln.lane;
      kt[q8_quant_offset(0, app_off, dd, D)] = s_appq[0][dd];
      vt[q8_quant_offset(1, app_off, dd, D)] = s_appq[1][dd];
    }
    if (ln.lane < D / 32) {
      ((uint16_t*)(kt + B * D))[app_off * (D / 32) + ln.lane] = s_apps[0][ln.lane];
      ((uint16_t*)(vt + B * D))[app_off * (D / 32) + ln.lane] = s_apps[1][ln.lane];
    }
  };
  auto process = [&](int t, int b) {
    const bool live = blive[b];
    const bool refill = t + NBUF < nt;
    const int32_t t0 = s0 + (wave + kAttnWaves * t) * B;  // first token of the block
    const bool patch = app_wave && t == app_t && live;
    if constexpr (DT == kDtypeQ8) {
      if (patch) store_q8_token(b);
    }
    // F16 operands are the ring registers themselves; Q8_0 ones are dequantised.
    uint4 kdq[DT == kDtypeF16 ? 1 : NC];
    uint4(&kr)[NC] = *[&]() -> uint4(*)[NC] {
      if constexpr (DT == kDtypeF16) {
        return &ring[b].k;
      } else {
        ring[b].k_operand(kdq);
        return &kdq;
      }
    }();
    if (patch && ln.col == app_off) {  // K operand: run c*4 + grp of the token
#pragma unroll
      for (int c = 0; c < NC; c++) {
        kr[c] = *(const uint4*)&s_app[0][c * 32 + ln.grp * 8];
        if constexpr (DT == kDtypeF16) {  // F16 K tile [D/8][B][8]
          uint8_t* kt = tile_ptr(g, (uint64_t)bid[b], layer, 0, kvh);
          *(uint4*)(kt + ((uint64_t)(c * 4 + ln.grp) * B + app_off) * 16) = kr[c];
        }
      }
    }
    float s[4];
    qk_block<D>(kr, qh, ql, hscale, ln, live, t0, s1, s);
    if (refill) {
      fetch(t + NBUF, b);
      ring[b].load_k_tile(tile_ptr(g, (uint64_t)bid[b], layer, 0, kvh), ln);
    }
    const f16x4 pw = softmax_block<D>(s, ln, st);
    u32x2_t vdq[DT == kDtypeF16 ? 1 : NM];
    u32x2_t(&vr)[NM] = *[&]() -> u32x2_t(*)[NM] {
      if constexpr (DT == kDtypeF16) {
        return &ring[b].v;
      } else {
        ring[b].v_operand(vdq);
        return &vdq;
      }
    }();
    if (patch && ln.grp == app_off / 4) {  // V operand: dim 16m + col, token app_off
      const int sh = (app_off & 1) * 16;
      const uint32_t keep = ~(0xffffu << sh);
#pragma unroll
      for (int m = 0; m < NM; m++) {
        const uint32_t h = s_app[1][m * 16 + ln.col];
        if (app_off & 2) vr[m].y = (vr[m].y & keep) | (h << sh);
        else vr[m].x = (vr[m].x & keep) | (h << sh);
        if constexpr (DT == kDtypeF16) {  // F16 V tile [D][B]
          uint16_t* vt = (uint16_t*)tile_ptr(g, (uint64_t)bid[b], layer, 1, kvh);
          vt[(uint64_t)(m * 16 + ln.col) * B + app_off] = (uint16_t)h;
        }
      }
    }
    if (live) pv_block<D>(vr, pw, ln, t0, s1, st);
    if (refill) ring[b].load_v_tile(tile_ptr(g, (uint64_t)bid[b], layer, 1, kvh), ln);
  };

#pragma unroll
  for (int b = 0; b < NBUF; b++) {
    if (b < nt) {
      fetch(b, b);
      ring[b].load_k_tile(tile_ptr(g, (uint64_t)bid[b], layer, 0, kvh), ln);
      ring[b].load_v_tile(tile_ptr(g, (uint64_t)bid[b], layer, 1, kvh), ln);
    }
  }
  if constexpr (ROPE) {
    rope_angles();
    if (app_wave) encode_app();
  }
  // q is read after the first K/V loads are issued, so its latency overlaps theirs.
  prep_q<D, ROPE>(q + ((uint64_t)seq * n_heads + (uint64_t)kvh * G + (ln.real ? ln.col : 0)) * D,
                  ln, scale * kLog2e, qh, ql, hscale, rsin, rcos, rope.rope_dim);
  if constexpr (DT == kDtypeQ8 && EXACT) {
    // One block at a time: the ring's single buffer, refilled after each block.
    for (int t = 0; t < nt; t++) {
      if (t > 0) {
        fetch(t, 0);
        ring[0].load_k_tile(tile_ptr(g, (uint64_t)bid[0], layer, 0, kvh), ln);
        ring[0].load_v_tile(tile_ptr(g, (uint64_t)bid[0], layer, 1, kvh), ln);
      }
      const int32_t t0 = s0 + (wave + kAttnWaves * t) * B;
      float sc[4], w[4];
      qk_block_q8x<D>(ring[0], qh, ql, hscale, ln, blive[0], t0, s1, sc);
      (void)softmax_block<D>(sc, ln, st, w);
      if (blive[0]) pv_block_q8x<D>(ring[0], w, ln, t0, s1, st);
    }
  } else if (store_only) {
    if (app_wave && app_t < nt) {  // the block holding the token: the wave's block app_t
      if (app_t >= 64) load_tab(app_t & ~63);
      const int32_t p = __builtin_amdgcn_readlane(tabv, app_t & 63);
      bid[0] = p;
      if (p >= 0 && (uint64_t)p < g.num_blocks) store_q8_token(0);
      else if (ln.lane == 0) raise_fault(g.fault, kFaultBlock);
    }
    return;  // the whole workgroup (split_marked is the same in all its waves)
  } else {
    for (int t = 0; t < nt; t += NBUF) {
#pragma unroll
      for (int b = 0; b < NBUF; b++)
        if (t + b < nt) process(t + b, b);
    }
  }

  // ---- per wave: l over the 4 lanes of each head; O rows to LDS.
  float lsum = st.l_part;
  lsum += __shfl_xor(lsum, 16);
  lsum += __shfl_xor(lsum, 32);
#pragma unroll
  for (int r = 0; r < 4; r++) {
    const int h = ln.grp * 4 + r;
    if (h < (int)G) {
#pragma unroll
      for (int m = 0; m < NM; m++) s_o[wave][h * D + m * 16 + ln.col] = st.acc[m][r];
    }
  }
  if (ln.lane < (int)G) {
    s_m[wave][ln.lane] = st.m_ref;
    s_l[wave][ln.lane] = lsum;
  }
  __syncthreads();

  // ---- merge the 4 waves (m in the log2 domain).
  const uint64_t head0 = (uint64_t)seq * n_heads + (uint64_t)kvh * G;
  for (int e = threadIdx.x; e < (int)G * D; e += 256) {
    const int gg = e / D, d = e % D;
    float M = -__builtin_inff();
#pragma unroll
    for (int w = 0; w < kAttnWaves; w++) M = __builtin_fmaxf(M, s_m[w][gg]);
    float o = 0.0f, L = 0.0f;
#pragma unroll
    for (int w = 0; w < kAttnWaves; w++) {
      const float mw = s_m[w][gg];
      const float wt = (mw == -__builtin_inff()) ? 0.0f : __builtin_amdgcn_exp2f(mw - M);
      o = __builtin_fmaf(wt, s_o[w][gg * D + d], o);
      L = __builtin_fmaf(wt, s_l[w][gg], L);
    }
    const uint64_t head = head0 + gg;
    if (nsplits == 1) {
      out[head * D + d] = __builtin_isfinite(M) ? o * (1.0f / L) : 0.0f;
    } else {
      ws_o[(head * max_splits + split) * D + d] = o;
      if (d == 0) {
        ws_ml[(head * max_splits + split) * 2] = M * 0.6931471805599453f;  // natural log
        ws_ml[(head * max_splits + split) * 2 + 1] = L;
      }
    }
  }
}

// Prefill versions of qk_block and softmax_block; qk_block_pf leaves the scores
// without q's power-of-two scale (hscale), which softmax_step_pf applies inside its
// exponent's fma (x * hscale is exact, so the sum is the one a separate product
// would give). The prefill kernel is bound by
// the VALU work around its MFMAs, so the work that is rare per block sits behind
// wave-uniform branches: the lo-chain NaN repair (only when a score is NaN), the
// causal mask (only on a block that crosses some column's causal end) and the
// empty-column rule (only while a real column has seen no finite score). The
// accumulator rescale stays unconditional (x 1.0 when no column's max moved): in
// the branch it costs 32 VGPRs, 4 -> 3 waves per SIMD, and 180 -> 222 us on a C3
// layer. Padding columns (ln.real false) are not masked: their q is zero, their
// accumulator rows are their own (an MFMA output row depends on its A row only)
// and never written.
template <int D>
__device__ __forceinline__ void qk_mfma_pf(const uint4 (&kr)[D / 32], const f16x8 (&qh)[D / 32],
                                           const f16x8 (&ql)[D / 32], f32x4& ah, f32x4& al) {
  ah = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};
  al = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int c = 0; c < D / 32; c++) {
    const f16x8 kv = __builtin_bit_cast(f16x8, kr[c]);
    ah = __builtin_amdgcn_mfma_f32_16x16x32_f16(kv, qh[c], ah, 0, 0, 0);
    al = __builtin_amdgcn_mfma_f32_16x16x32_f16(kv, ql[c], al, 0, 0, 0);
  }
}

// The same dot in one chain (hi then lo part of each 32-dim run into one accumulator):
// for pools without an infinite K, where no score needs the hi chain alone.
template <int D>
__device__ __forceinline__ f32x4 qk_mfma_pf1(const uint4 (&kr)[D / 32], const f16x8 (&qh)[D / 32],
                                             const f16x8 (&ql)[D / 32]) {
  f32x4 a = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int c = 0; c < D / 32; c++) {
    const f16x8 kv = __builtin_bit_cast(f16x8, kr[c]);
    a = __builtin_amdgcn_mfma_f32_16x16x32_f16(kv, qh[c], a, 0, 0, 0);
    a = __builtin_amdgcn_mfma_f32_16x16x32_f16(kv, ql[c], a, 0, 0, 0);
  }
  return a;
}

template <int D, bool REPAIR = true>
__device__ __forceinline__ void qk_block_pf(const uint4 (&kr)[D / 32], const f16x8 (&qh)[D / 32],
                                            const f16x8 (&ql)[D / 32],
                                            const Lane& ln, bool live, bool full, int32_t t0,
                                            int32_t end, float (&s)[4]) {
  f32x4 ah, al;
  qk_mfma_pf<D>(kr, qh, ql, ah, al);
  float x[4];
#pragma unroll
  for (int r = 0; r < 4; r++) x[r] = ah[r] + al[r];
  // One test for the four: a NaN score makes the sum NaN. Only an infinite K makes the
  // sum NaN with a hi chain that is not (see qk_block); the fast F16 instance runs over
  // pools that never stored one (the non-finite mark) and skips the test.
  if constexpr (REPAIR) {
    const float xs = (x[0] + x[1]) + (x[2] + x[3]);
    if (__builtin_amdgcn_ballot_w64(xs != xs) != 0) {  // see qk_block
#pragma unroll
      for (int r = 0; r < 4; r++) x[r] = ((x[r] != x[r]) & (ah[r] == ah[r])) ? ah[r] : x[r];
    }
  }
  if (live && full) {
#pragma unroll
    for (int r = 0; r < 4; r++) s[r] = x[r];
  } else {
#pragma unroll
    for (int r = 0; r < 4; r++) {
      const bool ok = ln.real && live && t0 + ln.grp * 4 + r < end;
      s[r] = ok ? x[r] : -__builtin_inff();
    }
  }
}

// Lazy online softmax of NB blocks at once (prefill): one max test, one rescale of the
// accumulators and one rare-path ballot per NB blocks instead of per block. ef gets the
// f32 weights (the exact Q8_0 P.V forms scale x weight from them), pw their binary16.
template <int D, int NB>
__device__ __forceinline__ void softmax_step_pf(const float (&s)[NB][4], float hscale,
                                                const Lane& ln, Accum<D>& st, f16x4 (&pw)[NB],
                                                float (&ef)[NB][4]) {
  float lmax = s[0][0];
#pragma unroll
  for (int b = 0; b < NB; b++)
#pragma unroll
    for (int r = 0; r < 4; r++) lmax = __builtin_fmaxf(lmax, s[b][r]);
  lmax *= hscale;
  const bool bad =
      ln.real & (!(lmax <= st.m_ref + kRescaleLog2) | !__builtin_isfinite(st.m_ref));
  if (__builtin_amdgcn_ballot_w64(bad) != 0) {  // some column's max moved: rescale
    float x = lmax;
    x = __builtin_fmaxf(x, __shfl_xor(x, 16));
    x = __builtin_fmaxf(x, __shfl_xor(x, 32));
    const float mn = __builtin_fmaxf(st.m_ref, x);
    const float alpha = (mn == -__builtin_inff()) ? 1.0f : __builtin_amdgcn_exp2f(st.m_ref - mn);
    st.l_part *= alpha;
    st.m_ref = mn;
    float ar[4];
#pragma unroll
    for (int r = 0; r < 4; r++) ar[r] = __shfl(alpha, ln.grp * 4 + r);
#pragma unroll
    for (int m = 0; m < D / 16; m++)
#pragma unroll
      for (int r = 0; r < 4; r++) st.acc[m][r] *= ar[r];
  }
  if (__builtin_amdgcn_ballot_w64(ln.real & (st.m_ref == -__builtin_inff())) == 0) {
#pragma unroll
    for (int b = 0; b < NB; b++)
#pragma unroll
      for (int r = 0; r < 4; r++) {
        const float e = __builtin_amdgcn_exp2f(__builtin_fmaf(s[b][r], hscale, -st.m_ref));
        st.l_part += e;
        ef[b][r] = e;
        pw[b][r] = (_Float16)e;
      }
  } else {
    const bool dead = (st.m_ref == -__builtin_inff());
#pragma unroll
    for (int b = 0; b < NB; b++)
#pragma unroll
      for (int r = 0; r < 4; r++) {
        const float sv = s[b][r];
        const float e = dead ? (sv != sv ? sv : 0.0f)
                             : __builtin_amdgcn_exp2f(__builtin_fmaf(sv, hscale, -st.m_ref));
        st.l_part += e;
        ef[b][r] = e;
        pw[b][r] = (_Float16)e;
      }
  }
}

// Whether an F16 V operand (tokens t0 + grp*4 + r of dims 16m + col) holds an Inf or
// NaN at a token in [lo, hi).
template <int D>
__device__ __forceinline__ bool v_nonfinite_in(const u32x2_t (&vr)[D / 16], const Lane& ln,
                                               int32_t t0, int32_t lo, int32_t hi) {
  uint32_t ex = 0;  // bit r: token r's values with all-ones exponents
#pragma unroll
  for (int m = 0; m < D / 16; m++) {
    const uint32_t a = ~vr[m].x & 0x7c007c00u, b = ~vr[m].y & 0x7c007c00u;
    ex |= ((a & 0xffffu) == 0 ? 1u : 0u) | ((a >> 16) == 0 ? 2u : 0u) |
          ((b & 0xffffu) == 0 ? 4u : 0u) | ((b >> 16) == 0 ? 8u : 0u);
  }
  uint32_t in = 0;
#pragma unroll
  for (int r = 0; r < 4; r++) {
    const int32_t t = t0 + ln.grp * 4 + r;
    in |= (t >= lo && t < hi) ? (1u << r) : 0u;
  }
  return (ex & in) != 0;
}

// ---------------------------------------------------------------------------
// Chunked-prefill attention
// ---------------------------------------------------------------------------
//
// The reference prefills token by token (crates/model/src/llama.rs:363-378), each
// token running the attention loop of :220-247 over positions 0 ..= its own.
// Here the chunk's K/V are already in the pool, and the 16 MFMA columns carry
// query rows instead of heads: column c of a wave's tile is (token c / G, head
// c % G) for 16 / G consecutive query tokens, each with its own causal end. QK,
// the softmax reductions (over the 4 lanes of a column) and PV are the decode
// block step.
//
// A workgroup holds 4 consecutive tiles (4 waves) of one (sequence, KV head) and
// streams the blocks up to its furthest causal end once, two blocks per step: the
// 256 threads stage the next step's blocks into the other half of an LDS double
// buffer (one block in registers at a time, stored at the middle and at the end of
// the step) while the waves compute the current step. Per step a wave does both
// blocks' QK, one softmax update over their 32 keys, then both P.V products.
//
// Storage: F16 tiles are staged as loaded except V, whose 16-byte units are
// XOR-swizzled by row so the P.V operand reads hit distinct banks. Q8_0 tiles are
// staged as loaded (their operand order reads conflict-free) and converted by the
// decode kernel's BlockRegs; for a workgroup whose blocks include one marked as
// holding a scale of 512 or more (mark_block), the fast instance exits and the EXACT
// instance, launched after it, computes with qk_block_q8x / pv_block_q8x.
//
// Tokens past a column's causal end carry weight 0 in the P.V product, but an
// Inf/NaN V there would still reach the column through 0 * NaN. F16 blocks that hold a
// non-finite K or V are marked (mark_block), and workgroups that read one run the
// leak-safe instance: on a block that crosses the tile's nearest causal end, a
// wave-uniform check for non-finite V values past that end sends the block down a
// masked path, one P.V per query token of the tile with P restricted to that token's
// columns and V zeroed from its end, so no column reads a position past its own (as
// the reference's token loop never does). Q8_0 V values are finite unless a scale
// is, and a block holding an inf or NaN scale is marked like a wide one, so the fast
// Q8_0 instance needs no check; the exact one masks P x scale per lane at the lane's
// own column end.
template <int DT, int D>
constexpr int prefill_tile_bytes() {
  return DT == kDtypeF16 ? B * D * 2 : B * D + B * D / 32 * 2;
}

enum : int { kPfFast = 0, kPfExact = 1, kPfLeakSafe = 2 };
// F16 tiles of a prefill step in LDS, both loaded 16 bytes a lane (a block is 4 K and
// 4 V load instructions at head_dim 128):
// - K: the stored [D/8][B][8] layout with the 16 token rows of each 8-dim run permuted,
//   token t at row pf_k_row(t, b) for the step's block b (bits 2 and 3 of t swapped, then
//   bit 3 flipped for the second block). Rows 0-7 of a run then hold tokens 0-3 and
//   8-11 of the first block, and the score MFMAs read their K operands as runs of 8
//   consecutive rows (below).
// - V: the stored [D][B] layout of 16-byte halves (dim n, tokens 8h .. 8h + 7), half (n, h)
//   at unit pf_v_unit<SW>(n, h) = 2n + (h ^ (SW ? bit 3 of n : 0)). The fast instances'
//   P.V operand of lane (col, grp) is one half (dim 16m + col, h = grp % 2) of block
//   grp / 2; the leak-safe instance reads 8 bytes, tokens grp*4 .. +3 (half grp / 2). An
//   LDS probe of the two patterns (SQ_LDS_BANK_CONFLICT) found the 16-byte reads free of
//   bank conflicts as stored and 2-way conflicted with the swap, the 8-byte reads the
//   other way round: the leak-safe instance stages V with the swap (SW), the fast ones
//   without.
__device__ __forceinline__ uint32_t pf_swap23(uint32_t t) {
  return (t & 3u) | ((t & 4u) << 1) | ((t & 8u) >> 1);
}
__device__ __forceinline__ uint32_t pf_k_row(uint32_t t, uint32_t b) { return pf_swap23(t) ^ (b * 8u); }
__device__ __forceinline__ uint32_t pf_k_token(uint32_t r, uint32_t b) { return pf_swap23(r ^ (b * 8u)); }
template <bool SW>
__device__ __forceinline__ uint32_t pf_v_unit(uint32_t n, uint32_t h) {
  return 2u * n + (h ^ (SW ? (n >> 3) & 1u : 0u));
}

// Fast Q8_0 prefill: a step's two staged Q8_0 blocks (raw: block b's K tile at
// raw + 2b * kTileQ, its V tile after it, both as stored: q8_quant_offset's order, then
// the f16 scales [B][D/32]) dequantised into binary16 tiles in the F16 staging layout
// above (block b's K tile at f16 + 2b * kTileF, its V tile after it), once per
// workgroup. The work is wave tasks of 64 lanes (dealt to the waves in pf_q8_to_f16):
// - K task (b, p): lane (g = l / 16, s = l % 16) reads the 16-byte unit holding runs
//   4(2p) + g and 4(2p + 1) + g of token t = pf_k_token(s, b) (the two 32-dim chunks
//   2p, 2p + 1 share a unit) and writes K rows s of both runs;
// - V task (b, P, hh): lane l writes V unit 128P + 64hh + l, i.e. half h = l % 2 (tokens
//   8h .. 8h + 7) of dim n = 64P + 32hh + l / 2, from two dwords of the stored tile
//   (tokens 8h .. 8h + 3 and 8h + 4 .. 8h + 7, 256 bytes apart); all its dims share the
//   scale group 2P + hh.
// The K task's reads and both tasks' writes cover contiguous 1 KiB spans (strided 16-byte
// writes measured 2-way bank conflicts in an LDS probe; contiguous ones none); the V
// dword reads of the two halves meet on the same banks, at one extra clock an
// instruction. A value is int8 -> binary16 exactly, times the scale with
// one rounding (v_pk_mul_f16): the operand the decode kernel's BlockRegs<Q8_0> forms in
// registers. No value overflows: blocks holding a scale of 512 or more are computed by
// the exact instance.
// The lane's offsets (three registers at 128 VGPRs): kq0 the K unit of block 0 (block 1's
// token is t ^ 4: kq0 ^ 64), l16 = 16 × lane (the K row offset (g·16 + s)·16 and the V
// unit offset within a task), and vq the V dword of dim l / 2's unit group, half l % 2
// (its scale row offset is bit 9 of vq, times 16·NG).
struct PfQ8Lane {
  uint32_t kq0, l16, vq;
};
template <int D>
__device__ __forceinline__ PfQ8Lane pf_q8_lane(uint32_t lane) {
  const uint32_t g = lane >> 4, s = lane & 15u;
  PfQ8Lane l;
  l.kq0 = (g * 16u + pf_k_token(s, 0u)) * 16u;
  l.l16 = lane * 16u;
  // dim 32hh + lane / 2 of unit group P: j = (lane / 2) % 16, m % 4 = 2hh + lane / 32
  l.vq = (lane & 1u) * 512u + ((lane >> 1) & 15u) * 16u + (lane >> 5) * 4u;
  // opaque from here: the per-step code adds only constants (task and buffer offsets)
  asm volatile("" : "+v"(l.kq0), "+v"(l.l16), "+v"(l.vq));
  return l;
}
// One K task (block b, chunk pair p) and one V task (block b, unit group P, half h).
template <int D>
__device__ __forceinline__ void pf_q8_k_task(const uint8_t* raw, uint8_t* f16, const PfQ8Lane& l,
                                             uint32_t b, uint32_t p) {
  constexpr uint32_t NG = D / 32, kTileQ = B * D + B * NG * 2, kTileF = B * D * 2;
  const uint8_t* rt = raw + 2u * b * kTileQ;
  const uint32_t kq = l.kq0 ^ (b * 64u);  // token t ^ 4 for block 1 (pf_k_token)
  const uint4 q = *(const uint4*)(rt + p * 1024u + kq);
  const uint32_t t = (kq / 16u) & 15u;
  // scales of chunks 2p, 2p + 1 of token t: one dword
  const uint32_t sw = *(const uint32_t*)(rt + B * D + (t * NG + 2u * p) * 2u);
  uint8_t* kf = f16 + 2u * b * kTileF + l.l16;  // run g of chunk 0, row s
#pragma unroll
  for (uint32_t h = 0; h < 2; h++) {
    const f16x2 s2 = __builtin_bit_cast(
        f16x2, __builtin_amdgcn_perm(sw, sw, h ? 0x03020302u : 0x01000100u));
    const uint32_t w0 = (h ? q.z : q.x) ^ 0x80808080u, w1 = (h ? q.w : q.y) ^ 0x80808080u;
    *(uint4*)(kf + (2u * p + h) * 1024u) =  // run 4(2p + h) + g
        make_uint4(__builtin_bit_cast(uint32_t, i8_pair_to_f16(w0, kSelLo) * s2),
                   __builtin_bit_cast(uint32_t, i8_pair_to_f16(w0, kSelHi) * s2),
                   __builtin_bit_cast(uint32_t, i8_pair_to_f16(w1, kSelLo) * s2),
                   __builtin_bit_cast(uint32_t, i8_pair_to_f16(w1, kSelHi) * s2));
  }
}
template <int D>
__device__ __forceinline__ void pf_q8_v_task(const uint8_t* raw, uint8_t* f16, const PfQ8Lane& l,
                                             uint32_t b, uint32_t P, uint32_t hh) {
  constexpr uint32_t NG = D / 32, kTileQ = B * D + B * NG * 2, kTileF = B * D * 2;
  const uint8_t* rt = raw + (2u * b + 1u) * kTileQ;
  const uint8_t* qp = rt + P * 1024u + hh * 8u + l.vq;
  const uint32_t qa = *(const uint32_t*)qp ^ 0x80808080u;          // tokens 8h .. +3
  const uint32_t qb = *(const uint32_t*)(qp + 256) ^ 0x80808080u;  // tokens 8h + 4 .. +7
  // tokens 8h .. 8h + 7 (h = lane % 2, bit 9 of vq), groups 2P and 2P + 1: a dword a token
  const uint8_t* sp = rt + B * D + 4u * P + ((l.vq >> 9) & 1u) * 16u * NG;
  const uint32_t sel = hh ? 0x07060302u : 0x05040100u;  // group 2P + hh: wave-uniform
  f16x2 sc[4];
#pragma unroll
  for (int pr = 0; pr < 4; pr++)
    sc[pr] = __builtin_bit_cast(
        f16x2, __builtin_amdgcn_perm(*(const uint32_t*)(sp + (2 * pr + 1) * NG * 2),
                                     *(const uint32_t*)(sp + 2 * pr * NG * 2), sel));
  // unit pf_v_unit(64P + 32hh + l / 2, l % 2) = 128P + 64hh + l
  *(uint4*)(f16 + (2u * b + 1u) * kTileF + (128u * P + 64u * hh) * 16u + l.l16) =
      make_uint4(__builtin_bit_cast(uint32_t, i8_pair_to_f16(qa, kSelLo) * sc[0]),
                 __builtin_bit_cast(uint32_t, i8_pair_to_f16(qa, kSelHi) * sc[1]),
                 __builtin_bit_cast(uint32_t, i8_pair_to_f16(qb, kSelLo) * sc[2]),
                 __builtin_bit_cast(uint32_t, i8_pair_to_f16(qb, kSelHi) * sc[3]));
}
// A step's 2 (K tasks a block + V tasks a block) tasks over the 4 waves. head_dim 128:
// wave w the K task (w / 2, w % 2) and the V tasks (0 and 1, P = w / 2, hh = w % 2), 3
// each; head_dim 64: tasks K(0), K(1), V(0, 0, 0), V(0, 0, 1), V(1, 0, 0), V(1, 0, 1)
// dealt w, w + 4.
template <int D>
__device__ __forceinline__ void pf_q8_to_f16(const uint8_t* raw, uint8_t* f16, const PfQ8Lane& l,
                                             uint32_t wave) {
  static_assert(D == 128 || D == 64, "head_dim 64 or 128");
  if constexpr (D == 128) {
    pf_q8_k_task<D>(raw, f16, l, wave >> 1, wave & 1u);
    __builtin_amdgcn_sched_barrier(0);  // one task's registers live at a time
    pf_q8_v_task<D>(raw, f16, l, 0u, wave >> 1, wave & 1u);
    __builtin_amdgcn_sched_barrier(0);
    pf_q8_v_task<D>(raw, f16, l, 1u, wave >> 1, wave & 1u);
  } else {
    if (wave < 2u) {
      pf_q8_k_task<D>(raw, f16, l, wave, 0u);
      __builtin_amdgcn_sched_barrier(0);
      pf_q8_v_task<D>(raw, f16, l, 1u, 0u, wave);
    } else {
      pf_q8_v_task<D>(raw, f16, l, 0u, 0u, wave - 2u);
    }
  }
}
template <int N>
struct PfBuf {  // a staging buffer index as a type
  static constexpr int value = N;
};

// One sequence of a prefill launch: the context clamped to the block table, the
// number of queries computed (q_lens[s] clamped to the context and to max_q_len) and
// the position of query 0 (from the stated q_len). The kernel and its combine agree
// on these through this function.
struct PfSeq {
  int32_t ctx, ql, p0;
  bool clamped;  // ctx or q_len was out of range: FKV_FAULT_CTX_RANGE
};
__device__ __forceinline__ PfSeq pf_seq(const int32_t* ctx_lens, const int32_t* q_lens,
                                        uint32_t seq, int32_t cap, uint32_t max_q_len) {
  const int32_t ctx = ctx_lens[seq], ql = q_lens[seq];
  const int32_t c = ctx < 0 ? 0 : (ctx > cap ? cap : ctx);
  const int32_t qc = ql < 0 ? 0 : (ql > c ? c : ql);
  const int32_t nq = qc < (int32_t)max_q_len ? qc : (int32_t)max_q_len;
  return PfSeq{c, nq, c - qc, ctx != c || ql != nq};
}

// Blocks the workgroup of tiles tile0 .. tile0 + 3 streams (up to its furthest causal
// end), and the number of key-range pieces it is cut into: pieces of about
// split_blocks blocks (split_blocks 0: one piece), at most max_splits.
__device__ __forceinline__ int32_t pf_wg_blocks(const PfSeq& sq, int32_t tile0, int32_t T) {
  const int32_t last = (tile0 + kAttnWaves) * T - 1 < sq.ql - 1 ? (tile0 + kAttnWaves) * T - 1 : sq.ql - 1;
  return (sq.p0 + last + 1 + B - 1) / B;
}
__device__ __forceinline__ int32_t pf_pieces(int32_t nblk, uint32_t split_blocks,
                                             uint32_t max_splits) {
  if (split_blocks == 0) return 1;
  const int32_t n = (nblk + (int32_t)split_blocks - 1) / (int32_t)split_blocks;
  return n < 1 ? 1 : (n > (int32_t)max_splits ? (int32_t)max_splits : n);
}

template <int DT, int D, int MODE>
// The fast instances hold 4 waves per SIMD (at most 128 VGPRs): the kernel is bound by
// instruction issue, and the fourth wave fills the others' dependency stalls.
__global__ void __launch_bounds__(256)
__attribute__((amdgpu_waves_per_eu(MODE == kPfFast ? 4 : 2, 8))) attn_prefill_kernel(
    Geom g, uint32_t layer, uint32_t n_heads, uint32_t G, const float* __restrict__ q,
    float* __restrict__ out, const int32_t* __restrict__ tables, uint32_t max_blocks,
    uint32_t cap_blocks, const int32_t* __restrict__ ctx_lens,
    const int32_t* __restrict__ q_lens, const int64_t* __restrict__ q_offsets,
    uint32_t max_q_len, float scale, uint32_t split_blocks, uint32_t max_splits,
    float* __restrict__ ws_o, float* __restrict__ ws_ml, uint32_t prio_blocks) {
  constexpr int NC = D / 32, NM = D / 16;
  constexpr int kStep = 2;  // blocks per softmax step
  constexpr int kTile = prefill_tile_bytes<DT, D>();
  static_assert(kTile % 16 == 0, "tiles are whole 16-byte chunks");
  constexpr int kBlk = 2 * kTile;               // K tile | V tile
  // Two staging buffers (steps alternate), as two arrays: the loop runs two steps an
  // iteration, each with its buffer known at compile time, so the compiler sees that a
  // step's LDS reads do not touch the loads landing in the other buffer and does not
  // wait for them.
  __shared__ __align__(16) uint8_t s_kv0[kStep][kBlk];
  __shared__ __align__(16) uint8_t s_kv1[kStep][kBlk];
  constexpr bool EXACT = MODE == kPfExact;
  // The fast instances compute from binary16 tiles in the F16 staging layout: F16 from
  // the staged blocks themselves, Q8_0 from s_f16, into which each step's staged blocks
  // are dequantised once per workgroup (pf_q8_to_f16).
  constexpr bool kQ8F = DT == kDtypeQ8 && MODE == kPfFast;
  constexpr int kTileF = B * D * 2, kBlkF = 2 * kTileF;
  __shared__ __align__(16) uint8_t s_f16[kQ8F ? kStep : 1][kQ8F ? kBlkF : 16];

  // The pool's count of marked blocks cannot change during a prefill launch (only
  // appends mark blocks), so every wave reads the same value. While it is 0 the fast
  // instance computes everything; otherwise each workgroup's own blocks decide below.
  const bool any_marks = pool_has_marks(g);
  if (MODE != kPfFast && !any_marks) return;
  // Which sequence this workgroup takes: its grid column's, moved on by a quarter of
  // the batch per step of q(y) = (y + y / 8) % 4. The hardware deals workgroups
  // w = x + gridDim.x * y to the 8 XCDs and their 4 shader engines in rotation, so
  // with gridDim.x dividing 256 the four that share a CU (w 32 apart, or 256 apart,
  // depending on how the engine fills its CUs) all had the same x, hence the same
  // sequence: the CUs holding the longest history carried 3x the others' blocks and
  // the kernel ended on them. q differs between the four under either fill, so a CU
  // now gets one workgroup from each quarter of the batch (C3: 194.8 -> 173.2 us).
  const uint32_t ns = gridDim.x / g.n_kv_heads;
  const uint32_t q4 = (blockIdx.y + blockIdx.y / 8u) % 4u;
  const uint32_t sk = ((blockIdx.x / g.n_kv_heads + q4 * ns / 4u) % ns) * g.n_kv_heads +
                      blockIdx.x % g.n_kv_heads;
  const uint32_t seq = sk / g.n_kv_heads, kvh = sk % g.n_kv_heads;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int32_t T = 16 / (int32_t)G;  // query tokens per wave tile
  // contexts are clamped to cap_blocks (the table row, or the staged blocks of a Q8_0
  // call through pf_stage_q8_kernel, whose instances must agree on every piece)
  const PfSeq sq = pf_seq(ctx_lens, q_lens, seq, (int32_t)(cap_blocks * B), max_q_len);
  // The grid holds max_q_len queries a sequence: past that the first max_q_len are
  // computed, at the positions the caller gave them, and the fault is raised.
  if (sq.clamped && blockIdx.y == 0 && blockIdx.z == 0 && threadIdx.x == 0 && kvh == 0)
    raise_fault(g.fault, kFaultCtx);
  const int32_t ql = sq.ql, p0 = sq.p0;  // queries computed; position of query 0
  const int32_t tile0 = (int32_t)blockIdx.y * kAttnWaves;  // first tile of the workgroup
  if (tile0 * T >= ql) return;                              // uniform over the workgroup
  // Key blocks [jbeg, jend): piece blockIdx.z of the workgroup's range, whose length
  // follows its furthest causal end (pieces of a range differ by at most one block).
  const int32_t nblk = pf_wg_blocks(sq, tile0, T);
  const int32_t npiece = pf_pieces(nblk, split_blocks, max_splits);
  if ((int32_t)blockIdx.z >= npiece) return;
  const int32_t jbeg = (int32_t)blockIdx.z * nblk / npiece;
  const int32_t jend = ((int32_t)blockIdx.z + 1) * nblk / npiece;
  const int32_t tile = tile0 + wave;
  const bool wave_on = tile * T < ql;

  Lane ln;
  ln.lane = threadIdx.x & 63;
  ln.col = ln.lane & 15;
  ln.grp = ln.lane >> 4;
  const int32_t jcol = tile * T + ln.col / (int32_t)G;  // query token of this column
  ln.real = wave_on && ln.col < T * (int32_t)G && jcol < ql;
  const int32_t end_col = p0 + jcol + 1;                // causal end of the column
  const int32_t jlast = tile * T + T - 1 < ql - 1 ? tile * T + T - 1 : ql - 1;
  const int32_t end_max = wave_on ? p0 + jlast + 1 : 0;  // furthest end of the wave's tile
  const int32_t end_min = p0 + tile * T + 1;             // nearest end: blocks before it
                                                         // need no causal mask
  const int32_t nblk_w = (end_max + B - 1) / B;
  const int64_t qrow0 = q_offsets[seq];
  auto row_of = [&](int32_t colv) {  // q/out row of column colv (clamped for padding)
    const int32_t j = tile * T + colv / (int32_t)G;
    const int32_t jj = j < ql ? j : ql - 1;
    return ((uint64_t)(qrow0 + jj) * n_heads + (uint64_t)kvh * G + (uint64_t)(colv % (int32_t)G)) * D;
  };

  const int32_t* table = tables + (uint64_t)seq * max_blocks;
  // With marked blocks in the pool, the marks of the piece's blocks pick the instance:
  // the exact (Q8_0: a scale of 512 or more) or leak-safe (F16: an Inf/NaN K or V) one
  // for a marked piece, the fast one otherwise.
  if (any_marks) {
    if (blocks_marked(g, table, jbeg, jend) != (MODE != kPfFast)) return;
  }
  // A table entry outside the pool raises the fault flag, stages block 0 and is
  // skipped. Blocks are staged by direct loads into LDS (dma_block_at below).
  const uint8_t* kbase = tile_ptr(g, 0, layer, 0, kvh);
  // F16 stages with loads straight into LDS: no staging registers, and a block's data
  // lands while the step computes. An instruction writes 64 lanes' 16 bytes
  // contiguously (1 KiB); the lanes' sources give the layout (pf_k_row, pf_v_unit):
  // instruction n of the K tile fills runs 4n .. 4n + 3, lane l row l % 16 of run
  // 4n + l / 16; instruction n of the V tile fills units 64n + l. The K tile's
  // instructions come first, then the V tile's, and wave w issues w, w + 4, ... A lane's
  // source offset within its instruction's KiB is the same for every n (the K rows'
  // permutation depends on the block's place b in the step: two offsets).
  constexpr int kKIns = kTile / 1024, kFIns = 2 * kKIns;
  uint32_t dma_k0 = 0, dma_k1 = 0, dma_v = 0;
  if constexpr (DT == kDtypeF16) {
    const uint32_t l = ln.lane;
    dma_k0 = ((l >> 4) * B + pf_k_token(l & 15u, 0u)) * 16u;
    dma_k1 = ((l >> 4) * B + pf_k_token(l & 15u, 1u)) * 16u;
    // unit 64n' + l: half (l / 2 + 32n', l % 2 ^ swap) of the stored tile (pf_v_unit)
    const uint32_t n = l >> 1, h = (l & 1u) ^ (MODE == kPfLeakSafe ? (n >> 3) & 1u : 0u);
    dma_v = (uint32_t)(g.n_kv_heads * g.tile_bytes) + n * 32u + h * 16u;
  }
  // The pool's block count clamped to 2^31: one unsigned compare tests p >= 0 and
  // p < num_blocks for any int32 p. A block's bytes fit 32 bits (the API checks), so
  // its offset is one 32 x 32-bit product.
  const uint32_t nblk32 = g.num_blocks > 0x80000000ull ? 0x80000000u : (uint32_t)g.num_blocks;
  // Block p to staging buffer buf as its block b (K tile to slot b, V interleaved with
  // the other block's). The loads go through a buffer resource based at the block's K
  // tile: the lane's offset is a register worked out once, the instruction's a scalar or
  // an immediate, so issuing them costs no vector instruction.
  auto dma_block_at = [&](int32_t p, uint8_t(*buf)[kBlk], int b) {
    uint8_t* const dst = buf[b];
    p = __builtin_amdgcn_readfirstlane(p);
    const bool ok = (uint32_t)p < nblk32;
    // The tile address is wave-uniform; passed through readfirstlane (and worked out
    // before the fault branch below) the compiler keeps the resource in scalar
    // registers instead of looping over lanes.
    const uint64_t ka = (uint64_t)(uintptr_t)kbase + (uint64_t)(ok ? (uint32_t)p : 0u) * (uint32_t)g.block_bytes;
    const uint64_t kau = ((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((int)(ka >> 32)) << 32) |
                         (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)ka);
    const uint8_t* kt = (const uint8_t*)(uintptr_t)kau;
    if (__builtin_expect(!ok, 0)) {  // wave-uniform: the common path is one branch
      if (threadIdx.x == 0) raise_fault(g.fault, kFaultBlock);
    }
    const __amdgpu_buffer_rsrc_t rs =
        __builtin_amdgcn_make_buffer_rsrc((void*)kt, (short)0, 0x7fffffff, 0x00020000);
    if constexpr (DT == kDtypeF16) {
#pragma unroll
      for (int k = 0; k < (kFIns + 3) / 4; k++) {
        const int i = wave + 4 * k;  // wave-uniform
        if (kFIns % 4 == 0 || i < kFIns) {
          const bool isv = i >= kKIns;
          const uint32_t n = (uint32_t)(isv ? i - kKIns : i);
          __builtin_amdgcn_raw_ptr_buffer_load_lds(
              rs, (__attribute__((address_space(3))) void*)(dst + (isv ? kTile : 0) + n * 1024u),
              16, (isv ? dma_v : (b == 0 ? dma_k0 : dma_k1)) + n * 1024u, 0, 0, 0);
        }
      }
    } else {
      // Q8_0 tiles as stored, K to dst and V to dst + kTile: 16-byte units, instruction
      // i of the block (wave w takes i = w, w + 4, ...) = 64 units of the K tile (i' = i)
      // or of the V tile (i' = i - kQIns) from unit min(64i', units - 64): every lane
      // loads a unit of the tile, the last instruction overlapping the one before with
      // the same bytes.
      constexpr int kUnits = kTile / 16, kQIns = (kUnits + 63) / 64;
      static_assert(kUnits >= 64, "a Q8_0 tile holds at least 64 units");
      const uint32_t vsrc = (uint32_t)(g.n_kv_heads * g.tile_bytes);
#pragma unroll
      for (int k = 0; k < (2 * kQIns + 3) / 4; k++) {
        const int i = wave + 4 * k;  // wave-uniform
        if (i < 2 * kQIns) {
          const bool isv = i >= kQIns;
          const int ip = isv ? i - kQIns : i;
          const int u0 = ip * 64 < kUnits - 64 ? ip * 64 : kUnits - 64;
          __builtin_amdgcn_raw_ptr_buffer_load_lds(
              rs, (__attribute__((address_space(3))) void*)(dst + (isv ? kTile : 0) + u0 * 16),
              16, (isv ? vsrc : 0u) + ((uint32_t)u0 + ln.lane) * 16u, 0, 0, 0);
        }
      }
    }
    return ok;
  };
  // Fast instances: scores from mixed-block rows and P.V of a step's two blocks in one
  // MFMA, over binary16 tiles in the F16 layout (below).
  constexpr bool kPair = MODE == kPfFast;
  // every load this wave issued has landed (vmcnt 0; expcnt and lgkmcnt left alone)
  auto dma_wait = [] { __builtin_amdgcn_s_waitcnt(0x0F70); };

  bool lv[kStep] = {false, false};   // blocks of the step being computed: in the pool
  bool nlv[kStep] = {false, false};  // and of the next step
  int32_t pn[kStep] = {0, 0};        // table entries of the next step's blocks
#pragma unroll
  for (int bb = 0; bb < kStep; bb++) {
    if (jbeg + bb < jend) lv[bb] = dma_block_at(table[jbeg + bb], s_kv0, bb);
    if (jbeg + kStep + bb < jend) pn[bb] = table[jbeg + kStep + bb];
  }
  // blocks this wave computes: the piece's, up to the wave's furthest causal end
  const int32_t jw_end = nblk_w < jend ? nblk_w : jend;
  f16x8 qh[NC], qlo[NC];
  float hscale;
  prep_q<D>(q + row_of(ln.real ? ln.col : 0), ln, scale * kLog2e, qh, qlo, hscale);
  Accum<D> st;
  st.reset();
  dma_wait();
  __syncthreads();

  int32_t j0 = jbeg;
  PfQ8Lane q8l{};
  if constexpr (kQ8F) q8l = pf_q8_lane<D>(ln.lane);
  // Issue priority by work left: a wave whose workgroup has more than 1/2, 1/4, 1/8 of
  // the longest range of the launch (prio_blocks) left issues ahead of the other waves
  // on its SIMD (workgroups of other sequences and tiles). The hardware otherwise
  // favours the oldest wave: workgroups drift apart, and the launch ends with laggards
  // alone on their SIMDs, where one wave reaches well under half the SIMD's rate.
  // prio_blocks 0 (launches cut into pieces, whose later pieces queue for slots): off.
  const int32_t prio3 = (int32_t)(prio_blocks / 2u), prio2 = (int32_t)(prio_blocks / 4u),
                prio1 = (int32_t)(prio_blocks / 8u);
  // One step: blocks j0, j0 + 1 from buffer BUF; the next step's go to the other.
  auto step = [&](auto bufc) __attribute__((always_inline)) {
    constexpr int BUF = decltype(bufc)::value;
    uint8_t(*const cur)[kBlk] = BUF == 0 ? s_kv0 : s_kv1;
    uint8_t(*const nxt)[kBlk] = BUF == 0 ? s_kv1 : s_kv0;
    const bool more = j0 + kStep < jend;      // the workgroup has a next step
    const bool more2 = j0 + kStep + 1 < jend;  // with a second block
    // the next step's blocks into the other buffer (its readers passed the barrier that
    // ended the last step), and the table entries of the step after
    if (more) nlv[0] = dma_block_at(pn[0], nxt, 0);
    if (more2) nlv[1] = dma_block_at(pn[1], nxt, 1);
    if (prio_blocks != 0) {
      const int32_t left = jend - j0;  // wave-uniform
      if (left > prio3) __builtin_amdgcn_s_setprio(3);
      else if (left > prio2) __builtin_amdgcn_s_setprio(2);
      else if (left > prio1) __builtin_amdgcn_s_setprio(1);
      else __builtin_amdgcn_s_setprio(0);
    }
    // the tiles the fast instances compute from: F16 as staged; Q8_0 dequantised into
    // s_f16 (every thread a share, then a barrier; the barrier that ended the last step
    // follows every wave's reads of s_f16)
    const uint8_t* const cf = kQ8F ? &s_f16[0][0] : &cur[0][0];
    if constexpr (kQ8F) {
      pf_q8_to_f16<D>(&cur[0][0], &s_f16[0][0], q8l, (uint32_t)wave);
      __syncthreads();
    }
    float sc[kStep][4];
    if constexpr (kPair) {
      // The step's 32 tokens as two score MFMAs X = 0, 1 whose rows mix the blocks: row
      // r of X is token 8 * (r / 4 % 2) + 4X + r % 4 of block r / 8, K row r ^ 8X of that
      // block (pf_k_row). Lane (col, grp) then holds the scores of tokens 8 * (grp % 2)
      // + 4X + 0..3 of block grp / 2: its 8 weights are 8 consecutive tokens of one
      // block, whose V is one 16-byte half-row (pf_v_unit) for the paired P.V below.
      // Both chains are issued back to back, then one wave-uniform test for the causal
      // mask of the step.
      f32x4 a[kStep];
#pragma unroll
      for (int x = 0; x < kStep; x++) {
        const uint8_t* ks = cf + (ln.col >> 3) * kBlkF;
        uint4 kr[NC];
#pragma unroll
        for (int c = 0; c < NC; c++)
          kr[c] = *(const uint4*)(ks + ((c * 4 + ln.grp) * B + (ln.col ^ (8 * x))) * 16);
        a[x] = qk_mfma_pf1<D>(kr, qh, qlo);
      }
      // a block past a column's causal end (or past the wave's tile, or not in the
      // pool) is masked; the step's blocks both lie before every end in the common case
      const bool full2 = lv[0] & lv[1] & ((j0 + kStep) * B <= end_min);
#pragma unroll
      for (int x = 0; x < kStep; x++)
#pragma unroll
        for (int r = 0; r < 4; r++) sc[x][r] = a[x][r];
      if (!full2) {
        const bool lvb = (ln.grp >> 1) ? lv[1] : lv[0];
        const int32_t tb = (j0 + (ln.grp >> 1)) * B + (ln.grp & 1) * 8;
#pragma unroll
        for (int x = 0; x < kStep; x++) {
#pragma unroll
          for (int r = 0; r < 4; r++) {
            const bool ok = ln.real && lvb && tb + 4 * x + r < end_col;
            sc[x][r] = ok ? sc[x][r] : -__builtin_inff();
          }
        }
      }
    } else {
#pragma unroll
    for (int bb = 0; bb < kStep; bb++) {
      const int32_t j = j0 + bb;
      const int32_t t0 = j * B;
      const uint8_t* ks = cur[bb];
      // F16 (leak-safe): every wave scores both blocks. One past the wave's tile (at most
      // the last of the workgroup's range, or a slot holding an earlier step's block)
      // lies past every column's causal end, so the causal mask gives it -inf
      // throughout. Q8_0 (exact) skips it.
      if (DT == kDtypeF16 || j < jw_end) {  // wave-uniform
        if constexpr (DT == kDtypeF16) {
          uint4 kr[NC];  // token col's K row (pf_k_row): the scores in token order
          const uint32_t kro = pf_k_row((uint32_t)ln.col, (uint32_t)bb);
#pragma unroll
          for (int c = 0; c < NC; c++)
            kr[c] = *(const uint4*)(ks + ((c * 4 + ln.grp) * B + kro) * 16);
          qk_block_pf<D, MODE != kPfFast>(kr, qh, qlo, ln, lv[bb], t0 + B <= end_min, t0,
                                          end_col, sc[bb]);
        } else {
          static_assert(DT == kDtypeF16 || EXACT, "fast Q8_0 takes the paired path");
          BlockRegs<kDtypeQ8, D> rg;
          rg.template load_k_tile<true>(ks, ln);
          qk_block_q8x<D>(rg, qh, qlo, 1.0f, ln, lv[bb], t0, end_col, sc[bb]);
        }
      } else {
#pragma unroll
        for (int r = 0; r < 4; r++) sc[bb][r] = -__builtin_inff();
      }
    }
    }  // !kPair
    f16x4 pw[kStep];
    float ef[kStep][4];
    softmax_step_pf<D, kStep>(sc, hscale, ln, st, pw, ef);
    if constexpr (kPair) {
      // P.V of both blocks: one 16x16x32 MFMA per 16 dims. Lane (col, grp)'s 8 weights
      // (score MFMAs 0 then 1) are tokens 8 * (grp % 2) + 0..7 of block grp / 2, and so
      // is its V operand: half grp % 2 of dim 16m + col of that block, one 16-byte read
      // (pf_v_unit). The pool holds no Inf/NaN here, so V needs zeroing only where P's
      // zeros could meet unwritten bytes: tokens at or past the wave's furthest causal
      // end, and a block not in the pool or not staged (a slot not staged this step
      // holds an earlier block's bytes, or nothing written yet).
      if (j0 < jw_end) {  // wave-uniform
        const f16x8 pa = {pw[0][0], pw[0][1], pw[0][2], pw[0][3],
                          pw[1][0], pw[1][1], pw[1][2], pw[1][3]};
        const uint8_t* vc = cf + (ln.grp >> 1) * kBlkF + kTileF +
                            pf_v_unit<false>((uint32_t)ln.col, (uint32_t)(ln.grp & 1)) * 16u;
        // Masks (wave-uniform branch) change only the V operands: MFMAs in common code
        // keep the accumulators in place (MFMAs on both sides of a branch made the
        // compiler move them between registers, and spill). Operands half at a time.
        const bool vmask = !(lv[0] & lv[1] & ((j0 + kStep) * B <= end_max));
#pragma unroll
        for (int h = 0; h < 2; h++) {
          uint4 v[NM / 2];
#pragma unroll
          for (int i = 0; i < NM / 2; i++)
            v[i] = *(const uint4*)(vc + (h * (NM / 2) + i) * 512);
          if (vmask) {
            const int32_t t0 = (j0 + (ln.grp >> 1)) * B + (ln.grp & 1) * 8;
            const int32_t n = ((ln.grp >> 1) ? lv[1] : lv[0]) ? end_max - t0 : 0;
            const uint32_t k0 = n >= 2 ? ~0u : (n == 1 ? 0xffffu : 0u);
            const uint32_t k1 = n >= 4 ? ~0u : (n == 3 ? 0xffffu : 0u);
            const uint32_t k2 = n >= 6 ? ~0u : (n == 5 ? 0xffffu : 0u);
            const uint32_t k3 = n >= 8 ? ~0u : (n == 7 ? 0xffffu : 0u);
#pragma unroll
            for (int i = 0; i < NM / 2; i++) {
              v[i].x &= k0;
              v[i].y &= k1;
              v[i].z &= k2;
              v[i].w &= k3;
            }
          }
#pragma unroll
          for (int i = 0; i < NM / 2; i++)
            st.acc[h * (NM / 2) + i] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                pa, __builtin_bit_cast(f16x8, v[i]), st.acc[h * (NM / 2) + i], 0, 0, 0);
        }
      }
    } else {
#pragma unroll
    for (int bb = 0; bb < kStep; bb++) {
      const int32_t j = j0 + bb;
      const int32_t t0 = j * B;
      if (j < jw_end && lv[bb]) {
        const uint8_t* vs = cur[bb] + kTile;
        if constexpr (DT == kDtypeF16) {
          // tokens grp*4 .. +3 of dim 16m + col: 8 bytes of half grp / 2 (pf_v_unit<true>)
          const uint8_t* vl =
              vs + pf_v_unit<true>((uint32_t)ln.col, (uint32_t)(ln.grp >> 1)) * 16u + (ln.grp & 1) * 8;
          u32x2_t vr[NM];
#pragma unroll
          for (int m = 0; m < NM; m++) vr[m] = *(const u32x2_t*)(vl + m * 512);
          // Leak-safe instance: a block where a non-finite V lies past the tile's
          // nearest causal end takes one P.V per query token jt of the tile, V cut at
          // that token's causal end, into a zeroed temporary; only the rows (columns)
          // of token jt are added to the accumulators (a shared V operand would give
          // every other row 0 * NaN). The check costs the fast instance a wave per
          // SIMD, which is why it has none and the pool mark picks the instance.
          bool leak = false;
          if constexpr (MODE == kPfLeakSafe)
            leak = t0 + B > end_min &&
                   __builtin_amdgcn_ballot_w64(v_nonfinite_in<D>(vr, ln, t0, end_min, end_max)) != 0;
          if (!leak) {
            pv_block<D>(vr, pw[bb], ln, t0, end_max, st);
          } else if constexpr (MODE == kPfLeakSafe) {
            for (int32_t jt = 0; jt < T; jt++) {
#pragma unroll
              for (int m = 0; m < NM; m++) vr[m] = *(const u32x2_t*)(vl + m * 512);
              mask_v_tail<D>(vr, ln, t0, p0 + tile * T + jt + 1);
#pragma unroll
              for (int m = 0; m < NM; m++) {
                const f32x4 t = __builtin_amdgcn_mfma_f32_16x16x16f16(
                    pw[bb], __builtin_bit_cast(f16x4, vr[m]), (f32x4){0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
#pragma unroll
                for (int r = 0; r < 4; r++)
                  if ((ln.grp * 4 + r) / (int32_t)G == jt) st.acc[m][r] += t[r];
              }
            }
          }
        } else {
          BlockRegs<kDtypeQ8, D> rg;
          rg.template load_v_tile<true>(vs, ln);
          pv_block_q8x<D>(rg, ef[bb], ln, t0, end_col, st);
        }
      }
    }
    }  // !kPair
    // The table entries of the step after next, loaded after this step's last LDS read:
    // a scalar load and an LDS read share one wait counter, so issued at the top it
    // held up the step's first K operands; here its wait falls after the barrier.
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int bb = 0; bb < kStep; bb++)
      pn[bb] = j0 + 2 * kStep + bb < jend ? table[j0 + 2 * kStep + bb] : 0;
    if (more) {
      dma_wait();
      __syncthreads();
      lv[0] = nlv[0];
      lv[1] = more2 ? nlv[1] : false;
    }
  };
  while (j0 < jend) {
    step(PfBuf<0>{});
    j0 += kStep;
    if (j0 >= jend) break;
    step(PfBuf<1>{});
    j0 += kStep;
  }
  if (!wave_on) return;

  float lsum = st.l_part;
  lsum += __shfl_xor(lsum, 16);
  lsum += __shfl_xor(lsum, 32);
  // Piece partials: slot ((sk * gridDim.y + y) * max_splits + z) holds the workgroup's
  // 64 columns (wave * 16 + column) x (unnormalised output [D], then max and sum in
  // the log2 domain).
  const uint64_t pslot = (((uint64_t)sk * gridDim.y + blockIdx.y) * max_splits + blockIdx.z) *
                             (uint64_t)(kAttnWaves * 16) + (uint64_t)wave * 16u;
  // accumulator row r of this lane is column grp*4 + r; its M and L live in lane grp*4 + r
#pragma unroll
  for (int r = 0; r < 4; r++) {
    const int c = ln.grp * 4 + r;
    const float M = __shfl(st.m_ref, c);
    const float L = __shfl(lsum, c);
    const int32_t jc = tile * T + c / (int32_t)G;
    if (c < T * (int32_t)G && jc < ql) {
      // one piece: the normalised output; several: this piece's partial (the same
      // stores, selected, so the accumulators need no second path)
      const bool whole = npiece == 1;
      const float inv = 1.0f / L;
      float* o = whole ? out + row_of(c) : ws_o + (pslot + (uint64_t)c) * D;
#pragma unroll
      for (int m = 0; m < NM; m++)
        o[m * 16 + ln.col] =
            whole ? (__builtin_isfinite(M) ? st.acc[m][r] * inv : 0.0f) : st.acc[m][r];
      if (!whole && ln.col == 0) {
        ws_ml[(pslot + (uint64_t)c) * 2] = M;
        ws_ml[(pslot + (uint64_t)c) * 2 + 1] = L;
      }
    }
  }
}

// Q8_0 prefill through a staging area: the blocks of the calling sequences dequantised
// once per call into binary16 tiles in the F16 pool layout (K [D/8][B][8], V [D][B]),
// staged block s * nblk + j holding block j of sequence s (contexts clamped to nblk
// blocks) in a one-layer staging pool. The staging table maps (s, j) to it (-1 where the
// pool's entry lies outside the pool: the prefill kernel faults and skips it) and the
// staging marks copy the pool block's mark. A value is f16(scale x quant) with one
// rounding (v_pk_mul_f16): the operand the fast Q8_0 instance forms in LDS from the
// same bytes, so the F16 fast instance over the staging computes what it would. In
// the fast Q8_0 instance every workgroup dequantises every block it stages, and up to
// max_q_len / 16 workgroups of a (sequence, KV head) stage the same block; here each
// block is converted once. Marked blocks (scales of 512 or more, whose products can
// overflow binary16) are computed by the exact instance from the pool itself.
// Grid (n_seqs * nblk, n_kv_heads); thread t writes K unit t (run t / 16, token t %
// 16) and V unit t (dim t / 2, tokens 8 (t % 2) .. + 7), twice at head_dim 128.
template <int D>
__global__ void __launch_bounds__(256) pf_stage_q8_kernel(
    Geom g, uint32_t layer, const int32_t* __restrict__ tables, uint32_t max_blocks,
    const int32_t* __restrict__ ctx_lens, uint32_t nblk, uint8_t* __restrict__ stage,
    int32_t* __restrict__ stab, uint32_t* __restrict__ smark) {
  constexpr uint32_t NG = D / 32, kTileF = B * D * 2;
  const uint32_t sj = blockIdx.x, h = blockIdx.y;
  const uint32_t sq = sj / nblk, j = sj % nblk;
  int32_t c = ctx_lens[sq];
  const int32_t cap = (int32_t)(nblk * B);
  c = c < 0 ? 0 : (c > cap ? cap : c);
  if ((int32_t)(j * B) >= c) return;  // past the context: never read
  const int32_t p = tables[(uint64_t)sq * max_blocks + j];
  const bool ok = p >= 0 && (uint64_t)p < g.num_blocks;
  if (h == 0 && threadIdx.x == 0) {
    stab[sj] = ok ? (int32_t)sj : -1;
    smark[sj] = ok ? g.bmark[p] : 0u;
  }
  if (!ok) return;
  const uint8_t* kq = tile_ptr(g, (uint64_t)p, layer, 0, h);
  const uint8_t* vq = tile_ptr(g, (uint64_t)p, layer, 1, h);
  uint8_t* kf = stage + (uint64_t)sj * (2u * g.n_kv_heads * kTileF) + (uint64_t)h * kTileF;
  uint8_t* vf = kf + (uint64_t)g.n_kv_heads * kTileF;
  // K units: dims 8r .. 8r + 7 of token tt (q8_quant_offset: chunk cc, group gg)
  for (uint32_t u = threadIdx.x; u < (uint32_t)D / 8u * 16u; u += 256u) {
    {
      const uint32_t r = u / 16u, tt = u % 16u, cc = r / 4u, gg = r % 4u;
      const uint2 qq = *(const uint2*)(kq + (cc / 2u) * 1024u + (gg * 16u + tt) * 16u + (cc % 2u) * 8u);
      const uint32_t sb = *(const uint16_t*)(kq + B * D + (tt * NG + cc) * 2u);
      const f16x2 s2 = __builtin_bit_cast(f16x2, sb | (sb << 16));
      const uint32_t w0 = qq.x ^ 0x80808080u, w1 = qq.y ^ 0x80808080u;
      *(uint4*)(kf + (r * 16u + tt) * 16u) =
          make_uint4(__builtin_bit_cast(uint32_t, i8_pair_to_f16(w0, kSelLo) * s2),
                     __builtin_bit_cast(uint32_t, i8_pair_to_f16(w0, kSelHi) * s2),
                     __builtin_bit_cast(uint32_t, i8_pair_to_f16(w1, kSelLo) * s2),
                     __builtin_bit_cast(uint32_t, i8_pair_to_f16(w1, kSelHi) * s2));
    }
  }
  // V units: tokens 8hh .. 8hh + 7 of dim n, each with its token's scale of group n / 32
  for (uint32_t u = threadIdx.x; u < (uint32_t)D * 2u; u += 256u) {
    {
      const uint32_t n = u / 2u, hh = u % 2u, m = n / 16u, jj = n % 16u;
      const uint8_t* src = vq + (m / 4u) * 1024u + (2u * hh * 16u + jj) * 16u + (m % 4u) * 4u;
      const uint32_t qa = *(const uint32_t*)src ^ 0x80808080u;          // tokens 8hh .. +3
      const uint32_t qb = *(const uint32_t*)(src + 256) ^ 0x80808080u;  // tokens 8hh + 4 .. +7
      const uint8_t* sp = vq + B * D + ((8u * hh) * NG + n / 32u) * 2u;
      uint32_t sc[8];
#pragma unroll
      for (int i = 0; i < 8; i++) sc[i] = *(const uint16_t*)(sp + i * NG * 2u);
      auto pr = [&](int i) { return __builtin_bit_cast(f16x2, sc[i] | (sc[i + 1] << 16)); };
      *(uint4*)(vf + n * 32u + hh * 16u) =
          make_uint4(__builtin_bit_cast(uint32_t, i8_pair_to_f16(qa, kSelLo) * pr(0)),
                     __builtin_bit_cast(uint32_t, i8_pair_to_f16(qa, kSelHi) * pr(2)),
                     __builtin_bit_cast(uint32_t, i8_pair_to_f16(qb, kSelLo) * pr(4)),
                     __builtin_bit_cast(uint32_t, i8_pair_to_f16(qb, kSelHi) * pr(6)));
    }
  }
}

// Merges the key-range pieces of every prefill workgroup cut into more than one:
// out = sum_z 2^(m_z - M) o_z / sum_z 2^(m_z - M) l_z with M = max_z m_z (0 where M is
// not finite, as the single-piece path writes). Grid (n_seqs * n_kv_heads, tile
// groups): one workgroup per prefill workgroup, thread t on dim t % D of columns
// t / D, t / D + 256 / D, ...
template <int D>
__global__ void __launch_bounds__(256) attn_prefill_combine_kernel(
    uint32_t n_kv_heads, uint32_t n_heads, uint32_t G, uint32_t max_blocks,
    const int32_t* __restrict__ ctx_lens, const int32_t* __restrict__ q_lens,
    const int64_t* __restrict__ q_offsets, uint32_t max_q_len, uint32_t split_blocks,
    uint32_t max_splits, const float* __restrict__ ws_o, const float* __restrict__ ws_ml,
    float* __restrict__ out) {
  const uint32_t sk = blockIdx.x;
  const uint32_t seq = sk / n_kv_heads, kvh = sk % n_kv_heads;
  const int32_t T = 16 / (int32_t)G;
  const PfSeq sq = pf_seq(ctx_lens, q_lens, seq, (int32_t)(max_blocks * B), max_q_len);
  const int32_t tile0 = (int32_t)blockIdx.y * kAttnWaves;
  if (tile0 * T >= sq.ql) return;
  const int32_t npiece = pf_pieces(pf_wg_blocks(sq, tile0, T), split_blocks, max_splits);
  if (npiece <= 1) return;
  const uint64_t slot0 = ((uint64_t)sk * gridDim.y + blockIdx.y) * max_splits;
  constexpr uint32_t kCols = kAttnWaves * 16, kStride = 256 / D;
  const uint32_t d = threadIdx.x % D;
  const int64_t qrow0 = q_offsets[seq];
  for (uint32_t cc = threadIdx.x / D; cc < kCols; cc += kStride) {
    const int32_t c = (int32_t)(cc % 16u);
    const int32_t jc = (tile0 + (int32_t)(cc / 16u)) * T + c / (int32_t)G;
    if (c >= T * (int32_t)G || jc >= sq.ql) continue;
    float M = -__builtin_inff();
    for (int32_t z = 0; z < npiece; z++)
      M = __builtin_fmaxf(M, ws_ml[((slot0 + z) * kCols + cc) * 2]);
    float o = 0.0f, L = 0.0f;
    if (__builtin_isfinite(M)) {
      for (int32_t z = 0; z < npiece; z++) {
        const uint64_t i = (slot0 + z) * kCols + cc;
        const float w = __builtin_amdgcn_exp2f(ws_ml[i * 2] - M);
        o = __builtin_fmaf(w, ws_o[i * D + d], o);
        L = __builtin_fmaf(w, ws_ml[i * 2 + 1], L);
      }
    }
    const uint64_t row = ((uint64_t)(qrow0 + jc) * n_heads + (uint64_t)kvh * G + (uint64_t)(c % (int32_t)G)) * D;
    out[row + d] = __builtin_isfinite(M) ? o * (1.0f / L) : 0.0f;
  }
}

// Workgroups of the stream kernel one CU holds at once (0 if it cannot launch).
template <int D>
int stream_wgs_per_cu(size_t lds_bytes) {
  int n = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, attn_mfma_stream_kernel<D>, 256,
                                                   lds_bytes) != hipSuccess)
    return 0;
  return n;
}

}  // namespace

bool stream_attention_supported(uint32_t n_seqs) {
  return n_seqs >= 1 && n_seqs <= kStreamMaxSeqs;
}

uint32_t stream_attention_waves(uint32_t head_dim, uint32_t n_seqs, uint32_t n_cus) {
  const size_t lds = ((size_t)n_seqs + 1) * 4;
  const int per_cu = head_dim == 128 ? stream_wgs_per_cu<128>(lds) : stream_wgs_per_cu<64>(lds);
  if (per_cu <= 0 || n_cus == 0) return 0;
  return (uint32_t)per_cu * n_cus * kAttnWaves;
}

hipError_t launch_attention_stream(const Geom& g, uint32_t layer, uint32_t n_heads,
                                   const float* q, float* out, const int32_t* tables,
                                   uint32_t max_blocks, const int32_t* ctx_lens,
                                   uint32_t n_seqs, float scale, uint32_t n_waves,
                                   uint32_t* ws_pre, float* ws_o, float* ws_ml, hipStream_t s) {
  const uint32_t G = n_heads / g.n_kv_heads;
  const uint32_t grid = n_waves / kAttnWaves;
  const size_t lds = ((size_t)n_seqs + 1) * 4;
  if (g.head_dim == 128)
    attn_mfma_stream_kernel<128><<<grid, 256, lds, s>>>(g, layer, n_heads, G, q, out, tables,
                                                        max_blocks, ctx_lens, n_seqs, scale,
                                                        ws_pre, ws_o, ws_ml);
  else
    attn_mfma_stream_kernel<64><<<grid, 256, lds, s>>>(g, layer, n_heads, G, q, out, tables,
                                                       max_blocks, ctx_lens, n_seqs, scale,
                                                       ws_pre, ws_o, ws_ml);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  const uint32_t cgrid = n_seqs * g.n_kv_heads * G;
  if (g.head_dim == 128)
    attn_stream_combine_kernel<128><<<cgrid, 256, 0, s>>>(n_seqs, g.n_kv_heads, G, n_waves,
                                                          ws_pre, ws_o, ws_ml, out);
  else
    attn_stream_combine_kernel<64><<<cgrid, 256, 0, s>>>(n_seqs, g.n_kv_heads, G, n_waves,
                                                         ws_pre, ws_o, ws_ml, out);
  return hipGetLastError();
}

namespace {
PrefillPlan prefill_plan_pieces(const Geom& g, uint32_t n_heads, uint32_t n_seqs,
                                uint32_t max_q_len, uint32_t max_ctx_len) {
  PrefillPlan p{};
  const uint32_t G = n_heads / g.n_kv_heads;
  const uint32_t T = 16 / G;
  const uint64_t tiles = ((uint64_t)max_q_len + T - 1) / T;
  p.tile_groups = (uint32_t)((tiles + kAttnWaves - 1) / kAttnWaves);
  const uint64_t max_nblk = ((uint64_t)max_ctx_len + B - 1) / B;
  // Pieces pay only where the grid leaves workgroup slots idle (each piece restages q
  // and writes a partial): split so that about twice the slots have work, into pieces
  // of at least kPrefillMinPieceBlocks. FKV_PREFILL_SPLIT_BLOCKS sets the piece length
  // (0: no split).
  uint64_t split = 0;
  if (const int64_t v = tuning().prefill_split.load(std::memory_order_relaxed); v >= 0) {
    split = (uint64_t)v;
  } else {
    const uint64_t cus = g.n_cus;
    const uint64_t wgs = (uint64_t)n_seqs * g.n_kv_heads * p.tile_groups;
    if (cus > 0 && wgs < cus * kPrefillWgsPerCu) {
      const uint64_t want = (cus * kPrefillWgsPerCu * 2 + wgs - 1) / wgs;
      split = std::max<uint64_t>(kPrefillMinPieceBlocks, (max_nblk + want - 1) / want);
    }
  }
  p.prio_blocks = (uint32_t)max_nblk;
  if (split == 0 || max_nblk <= split) return p;  // one piece per workgroup
  split = std::max<uint64_t>(split, (max_nblk + kPrefillMaxSplits - 1) / kPrefillMaxSplits);
  if (max_nblk <= split) return p;
  p.split_blocks = (uint32_t)split;
  p.max_splits = (uint32_t)((max_nblk + split - 1) / split);
  p.prio_blocks = 0;  // pieces queue for slots: issue priority measured slower there
  const uint64_t slots = (uint64_t)n_seqs * g.n_kv_heads * p.tile_groups * p.max_splits *
                         (uint64_t)(kAttnWaves * 16);
  p.ws_o_floats = slots * g.head_dim;
  p.ws_bytes = (p.ws_o_floats + slots * 2) * sizeof(float);
  return p;
}
}  // namespace

// The key-range pieces, then for Q8_0 pools the staging area of pf_stage_q8_kernel after
// the partials: n_seqs x ceil(max_ctx_len / 16) blocks of binary16 K and V tiles of every
// KV head (one layer), the staging table and the staging marks.
PrefillPlan prefill_plan(const Geom& g, uint32_t n_heads, uint32_t n_seqs, uint32_t max_q_len,
                         uint32_t max_ctx_len) {
  PrefillPlan p = prefill_plan_pieces(g, n_heads, n_seqs, max_q_len, max_ctx_len);
  const uint64_t nblk = ((uint64_t)max_ctx_len + B - 1) / B;
  p.cap_blocks = (uint32_t)nblk;
  if (g.dtype != kDtypeQ8) return p;
  const uint64_t n = (uint64_t)n_seqs * nblk;
  if (nblk == 0 || n > 0x7fffffffull) return p;
  auto al = [](uint64_t x) { return (x + 255) / 256 * 256; };
  p.stage_nblk = (uint32_t)nblk;
  p.stage_off = al(p.ws_bytes);
  p.stage_tab_off = p.stage_off + al(n * 2u * g.n_kv_heads * B * g.head_dim * 2u);
  p.stage_mark_off = p.stage_tab_off + al(n * 4u);
  p.ws_bytes = p.stage_mark_off + al(n * 4u);
  return p;
}

hipError_t launch_prefill_attention(const Geom& g, uint32_t layer, uint32_t n_heads,
                                    const float* q, float* out, const int32_t* tables,
                                    uint32_t max_blocks, const int32_t* ctx_lens,
                                    const int32_t* q_lens, const int64_t* q_offsets,
                                    uint32_t n_seqs, uint32_t max_q_len, float scale,
                                    const PrefillPlan& plan, void* workspace, hipStream_t s) {
  const uint32_t G = n_heads / g.n_kv_heads;
  // Without a workspace every workgroup is one piece.
  const bool split = plan.split_blocks != 0 && workspace != nullptr;
  const uint32_t split_blocks = split ? plan.split_blocks : 0u;
  const uint32_t max_splits = split ? plan.max_splits : 1u;
  float* ws_o = split ? (float*)workspace : nullptr;
  float* ws_ml = split ? ws_o + plan.ws_o_floats : nullptr;
  dim3 grid(n_seqs * g.n_kv_heads, plan.tile_groups, max_splits);
  // Contexts past max_ctx_len (whole blocks) are clamped to it with FKV_FAULT_CTX_RANGE
  // by every kernel of the call. Q8_0 with a workspace: the calling sequences' blocks
  // dequantised once into the staging area (which holds that many blocks a sequence),
  // the F16 fast instance over it, the exact instance over the pool for marked blocks.
  const uint32_t cap_blocks =
      plan.cap_blocks != 0 && plan.cap_blocks < max_blocks ? plan.cap_blocks : max_blocks;
  const bool staged = g.dtype == kDtypeQ8 && workspace != nullptr && plan.stage_nblk != 0 &&
                      plan.stage_nblk == cap_blocks;
  Geom gs = g;
  int32_t* stab = nullptr;
  if (staged) {
    uint8_t* wsb = (uint8_t*)workspace;
    stab = (int32_t*)(wsb + plan.stage_tab_off);
    gs.base = wsb + plan.stage_off;
    gs.tile_bytes = (uint64_t)B * g.head_dim * 2u;
    gs.block_bytes = 2u * g.n_kv_heads * gs.tile_bytes;
    gs.num_blocks = (uint64_t)n_seqs * plan.stage_nblk;
    gs.n_layers = 1;
    gs.dtype = kDtypeF16;
    gs.bmark = (uint32_t*)(wsb + plan.stage_mark_off);
    gs.hmark = nullptr;
    const dim3 sgrid(n_seqs * plan.stage_nblk, g.n_kv_heads);
    if (g.head_dim == 128)
      pf_stage_q8_kernel<128><<<sgrid, 256, 0, s>>>(g, layer, tables, max_blocks, ctx_lens,
                                                    plan.stage_nblk, gs.base, stab, gs.bmark);
    else
      pf_stage_q8_kernel<64><<<sgrid, 256, 0, s>>>(g, layer, tables, max_blocks, ctx_lens,
                                                   plan.stage_nblk, gs.base, stab, gs.bmark);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
#define FKV_LAUNCH_PF(DT_, D_, X_)                                                          \
  attn_prefill_kernel<DT_, D_, X_><<<grid, 256, 0, s>>>(g, layer, n_heads, G, q, out, tables, \
                                                        max_blocks, cap_blocks, ctx_lens,     \
                                                        q_lens, q_offsets, max_q_len, scale,  \
                                                        split_blocks, max_splits, ws_o, ws_ml, \
                                                        plan.prio_blocks)
  // The fast instance, then the one for workgroups whose blocks' marks say the fast one
  // cannot compute them: Q8_0 the exact instance (a scale of 512 or more was stored),
  // F16 the leak-safe one (an Inf/NaN K or V was stored). Each exits where the other works.
  const int dt = g.dtype == kDtypeQ8 ? kDtypeQ8 : kDtypeF16;
  if (staged) {
    if (g.head_dim == 128)
      attn_prefill_kernel<kDtypeF16, 128, kPfFast><<<grid, 256, 0, s>>>(
          gs, 0, n_heads, G, q, out, stab, plan.stage_nblk, cap_blocks, ctx_lens, q_lens,
          q_offsets, max_q_len, scale, split_blocks, max_splits, ws_o, ws_ml, plan.prio_blocks);
    else
      attn_prefill_kernel<kDtypeF16, 64, kPfFast><<<grid, 256, 0, s>>>(
          gs, 0, n_heads, G, q, out, stab, plan.stage_nblk, cap_blocks, ctx_lens, q_lens,
          q_offsets, max_q_len, scale, split_blocks, max_splits, ws_o, ws_ml, plan.prio_blocks);
  } else if (dt == kDtypeQ8) {
    if (g.head_dim == 128) FKV_LAUNCH_PF(kDtypeQ8, 128, kPfFast);
    else FKV_LAUNCH_PF(kDtypeQ8, 64, kPfFast);
  } else {
    if (g.head_dim == 128) FKV_LAUNCH_PF(kDtypeF16, 128, kPfFast);
    else FKV_LAUNCH_PF(kDtypeF16, 64, kPfFast);
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  if (dt == kDtypeQ8) {
    if (g.head_dim == 128) FKV_LAUNCH_PF(kDtypeQ8, 128, kPfExact);
    else FKV_LAUNCH_PF(kDtypeQ8, 64, kPfExact);
  } else {
    if (g.head_dim == 128) FKV_LAUNCH_PF(kDtypeF16, 128, kPfLeakSafe);
    else FKV_LAUNCH_PF(kDtypeF16, 64, kPfLeakSafe);
  }
#undef FKV_LAUNCH_PF
  e = hipGetLastError();
  if (e != hipSuccess || !split) return e;
  // the combine reads the table width only as the context cap
  const dim3 cgrid(n_seqs * g.n_kv_heads, plan.tile_groups);
  if (g.head_dim == 128)
    attn_prefill_combine_kernel<128><<<cgrid, 256, 0, s>>>(g.n_kv_heads, n_heads, G, cap_blocks,
                                                           ctx_lens, q_lens, q_offsets, max_q_len,
                                                           split_blocks, max_splits, ws_o, ws_ml,
                                                           out);
  else
    attn_prefill_combine_kernel<64><<<cgrid, 256, 0, s>>>(g.n_kv_heads, n_heads, G, cap_blocks,
                                                          ctx_lens, q_lens, q_offsets, max_q_len,
                                                          split_blocks, max_splits, ws_o, ws_ml,
                                                          out);
  return hipGetLastError();
}

// Dynamic LDS that holds a decode launch to at most tuning().attn_wgs_per_cu workgroups
// a CU (0: none asked for): more than a (cap + 1)-th of the CU's 160 KiB in all, at most
// a cap-th. The instance's static LDS is read once per instance (on the first capped
// launch of the first device that runs it; the instance's static LDS is the same on
// every gfx950 device).
template <int DT, int D, int NB, bool R, bool X>
size_t decode_lds_pad() {
  const int32_t cap = tuning().attn_wgs_per_cu.load(std::memory_order_relaxed);
  if (cap <= 0) return 0;
  static const size_t fixed = [] {
    hipFuncAttributes a;
    return hipFuncGetAttributes(&a, (const void*)&attn_mfma_kernel<DT, D, NB, R, X>) ==
                   hipSuccess
               ? (size_t)a.sharedSizeBytes
               : (size_t)0;
  }();
  constexpr size_t kCuLds = 160u * 1024u;
  const size_t want = kCuLds / (size_t)(cap + 1) + 1u;
  return want > fixed ? want - fixed : 0u;
}

hipError_t launch_attention_mfma(const Geom& g, uint32_t layer, uint32_t n_heads,
                                 const float* q, float* out, const int32_t* tables,
                                 uint32_t max_blocks, const int32_t* ctx_lens, uint32_t n_seqs,
                                 uint32_t max_splits, uint32_t split_tokens, float scale,
                                 float* ws_o, float* ws_ml, const float* k_new,
                                 const float* v_new, hipStream_t s, const RopeTable* rope) {
  const uint32_t G = n_heads / g.n_kv_heads;
  const dim3 grid(n_seqs * g.n_kv_heads * max_splits);
  constexpr int NBUF = FKV_MFMA_RING;
  const int32_t st = (int32_t)split_tokens;
  // Longest-first order when the batch is small enough for every workgroup to
  // rank it; FKV_ATTN_ORDER=0/1/2 forces grid / full-first / longest-first.
  uint32_t order = n_seqs <= kOrderSortSeqs   ? kOrderLongestFirst
                   : n_seqs <= kOrderMaxSeqs ? kOrderFullFirst
                                             : kOrderGrid;
  if (const int32_t v = tuning().attn_order.load(std::memory_order_relaxed); v >= 0) {
    if (v == 0 || (v == 1 && n_seqs <= kOrderMaxSeqs) || (v == 2 && n_seqs <= kOrderSortSeqs))
      order = (uint32_t)v;
  }
  // RoPE in the kernel for F16 and Q8_0 storage.
  const bool roped = rope != nullptr && rope->rope_dim > 0;
  RopeTable rt{};
  if (roped) rt = *rope;
#define FKV_LAUNCH_MFMA(DT_, D_, R_, X_)                                                         \
  attn_mfma_kernel<DT_, D_, NBUF, R_, X_>                                                        \
      <<<grid, 256, decode_lds_pad<DT_, D_, NBUF, R_, X_>(), s>>>(                              \
          g, layer, n_heads, G, q, out, tables, max_blocks, ctx_lens, n_seqs, max_splits, st,   \
          order, scale, ws_o, ws_ml, k_new, v_new, rt)
  // Q8_0: the fast instance, then the exact one (each workgroup of which exits at once
  // unless its split reads a block marked as holding a scale of 512 or more).
  if (g.dtype == kDtypeQ8 && roped) {
    if (g.head_dim == 128) FKV_LAUNCH_MFMA(kDtypeQ8, 128, true, false);
    else FKV_LAUNCH_MFMA(kDtypeQ8, 64, true, false);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    if (g.head_dim == 128) FKV_LAUNCH_MFMA(kDtypeQ8, 128, true, true);
    else FKV_LAUNCH_MFMA(kDtypeQ8, 64, true, true);
  } else if (g.dtype == kDtypeQ8) {
    if (g.head_dim == 128) FKV_LAUNCH_MFMA(kDtypeQ8, 128, false, false);
    else FKV_LAUNCH_MFMA(kDtypeQ8, 64, false, false);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    if (g.head_dim == 128) FKV_LAUNCH_MFMA(kDtypeQ8, 128, false, true);
    else FKV_LAUNCH_MFMA(kDtypeQ8, 64, false, true);
  } else if (roped) {
    if (g.head_dim == 128) FKV_LAUNCH_MFMA(kDtypeF16, 128, true, false);
    else FKV_LAUNCH_MFMA(kDtypeF16, 64, true, false);
  } else {
    if (g.head_dim == 128) FKV_LAUNCH_MFMA(kDtypeF16, 128, false, false);
    else FKV_LAUNCH_MFMA(kDtypeF16, 64, false, false);
  }
#undef FKV_LAUNCH_MFMA
  return hipGetLastError();
}

}  // namespace fkv
