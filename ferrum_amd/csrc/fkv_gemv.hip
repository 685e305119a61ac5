// Q8_0 weight GEMV/GEMM on gfx950: Ferrum's ggml q8_0 x q8_0 product
// (crates/kernels/src/q8_dot.rs:35-109; scalar.rs:84-116,191-204), bit for bit.
//
// Per token the f32 activation row is quantized as Q8Activation::quantize_into
// (q8_dot.rs:35-61): per 32 values amax = max|v| (NaN ignored), d = amax/127,
// id = d != 0 ? 1/d : 0, q = clamp(round_half_away(v * id)), and the scale kept is
// f16(d) through the reference's own ties-away encoder (q8_dot.rs:111-139). Every
// output is then dot_q8_row_q8_act (q8_dot.rs:72-109):
//   acc = 0; for b = 0, 1, ...: acc += f32(sumi_b) * (w_scale_b * x_scale_b)
// where sumi_b is the int32 dot of the two 32-byte runs. The integer dots have no
// rounding, so any order gives the same sumi_b; w_scale * x_scale is exact (two
// binary16 significands fit in 22 bits); f32(sumi_b) * that rounds once, as in the
// reference (no FMA anywhere: -ffp-contract=off); and the f32 sum keeps the
// reference's left-to-right block order through a DPP broadcast chain.
//
// Layout: weights row-major, row r = cols/32 blocks of 34 bytes ([f16 scale LE]
// [32 x i8]) at w + r * (cols/32) * 34 (Ferrum's tensor bytes, dtype.rs:19-21); x is
// [n_tokens][cols] f32, y is [n_tokens][rows] f32 (GemmArgs, par.rs:9-26).
//
// Work split: a workgroup of 4 waves owns 16 consecutive rows of one of the launch's
// matrices (up to four that share the activation), a wave 4 rows, one per 16-lane DPP
// row. Lane l of a row group takes blocks l, l+16, l+32, ... of its
// row, so a 16-block step of the wave reads four runs of 544 contiguous bytes.
// Up to kPipe steps of loads are in flight per wave.
//
// Alignment without realignment: a block is only 2-byte aligned (34 = 2 mod 4), and
// the parity of its address is the same for every step of a lane (16 * 34 = 0 mod
// 4). A lane reads the 8 dwords that start at the first dword boundary of its block
// and the 16-bit word they leave out, and dots those 9 dwords as they are against
// one of two copies of the quantized activation block kept in LDS:
//   block at 2 mod 4: dwords = q0..q31, word = scale -> aligned copy (x0..x31, 0)
//   block at 0 mod 4: dwords = (scale, q0 q1), (q2..q5) ... (q26..q29), word = (q30,
//                     q31) -> copy shifted by two bytes ((0, 0, x0, x1), ..., (x30,
//                     x31, 0, 0)); the scale bytes meet zeros.
// The activation is quantized into LDS by each workgroup; its loads are issued
// before any weight load (loads retire in issue order, so activation loads behind
// a wave's weight prefetch would wait for all of it).
#include <utility>

#include "fkv_device.h"

namespace fkv {
namespace {

typedef float f32x4a __attribute__((ext_vector_type(4), aligned(4)));
typedef int v4i __attribute__((ext_vector_type(4)));

constexpr uint32_t kQ8Bytes = 34;
constexpr int kGemvWaves = 4;
constexpr int kGemvThreads = 64 * kGemvWaves;
constexpr int kRowsPerWave = 4;                             // 16 lanes per row
constexpr uint32_t kRowsPerWg = kGemvWaves * kRowsPerWave;  // 16
constexpr int kPipe = 4;                                    // 16-block steps in flight
// LDS dwords per (token, block): aligned q[0..8) | shifted q[0..8) | two tail pairs,
// aligned (q[8] = 0, xs) and shifted (q[8], xs). Each copy's first 8 dwords are
// 16-byte aligned. The tail pairs trade places in blocks with bit 3 set
// (kTailDw): lanes l and l + 8 read blocks 8 records = 160 dwords apart, a multiple
// of 32 banks, and would otherwise hit the same banks with their 8-byte tail reads.
constexpr uint32_t kXDw = 20;
__device__ __forceinline__ uint32_t tail_dw(bool aligned, uint32_t block) {
  const uint32_t swap = (block >> 3) & 1u;
  return aligned ? 16u + 2u * swap : 18u - 2u * swap;
}
// Activation passes (8 values a lane) loaded up front: 2 by default, 4 for two-token
// launches and 8 for one-token launches of more than 4096 columns (measured: more
// passes up front slowed the 3- and 4-token launches).
constexpr int kXRegs = 2;
constexpr int kXRegsWide = 8;

// LDS blocks a token: the step count rounded up to whole groups of kPipe iterations
// (an iteration is S steps of 16 blocks), so every step a group runs reads inside the
// array.
__host__ __device__ constexpr uint32_t gemv_padded_blocks(uint32_t nb, uint32_t S = 1) {
  return (nb + 16u * S * kPipe - 1u) / (16u * S * kPipe) * (16u * S * kPipe);
}

struct RawBlock {
  uint32_t d[8];
  uint32_t tail;
};

typedef unsigned int v4u __attribute__((ext_vector_type(4)));
// Buffer descriptor word 3 for raw 32-bit access on gfx9 (the data format that
// makes out-of-range reads return zero); offsets at or past kOobOffset are out of
// range (the resource never spans more than kOobOffset - 1 bytes).
constexpr int kBufferWord3 = 0x00020000;
constexpr uint32_t kOobOffset = 0x80000000u;

template <int L>
__device__ __forceinline__ float row_bcast(float v) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x150 + L, 0xf, 0xf, true));
}

// acc + p(lane 0) + p(lane 1) + ... + p(lane 15) of this lane's 16-lane row, in that
// order, one rounding per add (one v_add_f32_dpp row_newbcast each).
template <int... L>
__device__ __forceinline__ float chain16(float acc, float p, std::integer_sequence<int, L...>) {
  ((acc = acc + row_bcast<L>(p)), ...);
  return acc;
}

// amax / 127 correctly rounded for every amax >= 0: q = amax * RN(1/127) corrected
// once by its FMA residual equals the IEEE quotient for all finite amax (checked
// exhaustively over all 2^31 of them); +Inf, where the residual is NaN, maps to +Inf.
__device__ __forceinline__ float div127(float a) {
  const float c = 1.0f / 127.0f;
  const float q = a * c;
  const float r = __builtin_fmaf(-q, 127.0f, a);
  const float q1 = __builtin_fmaf(r, c, q);
  return a == __builtin_inff() ? a : q1;
}

// Rust's round (half away from zero) as trunc(y + copysign(0.5 - 2^-25, y)): equal
// for every f32 y (checked exhaustively over all 2^32).
__device__ __forceinline__ float round_away(float y) {
  return __builtin_truncf(y + __builtin_copysignf(0.49999997f, y));
}

// clamp(round(y) as i32, -128, 127) as a byte. v_cvt_i32_f32 is Rust's `as i32`:
// it saturates and takes NaN to 0 (written as asm: the C++ cast of NaN is undefined).
__device__ __forceinline__ uint32_t q8_byte(float y) {
  int q;
  __asm__("v_cvt_i32_f32 %0, %1" : "=v"(q) : "v"(round_away(y)));
  q = q < -128 ? -128 : (q > 127 ? 127 : q);  // v_med3_i32
  return (uint32_t)q & 0xffu;
}

// binary16 bits of d >= 0 (never NaN), ties away from zero (q8_dot.rs:111-139): the
// round-toward-zero neighbour and the next binary16 up, compared by distance (both
// differences exact near a tie). 65504 < d < 65520 stays 65504; d >= 65520 -> Inf.
__device__ __forceinline__ uint32_t f16_bits_away(float d) {
  auto pk = __builtin_amdgcn_cvt_pkrtz(d, 0.0f);
  const uint32_t lo = __builtin_bit_cast(uint32_t, pk) & 0xffffu;
  const float lo_v = dev::f16_bits_to_f32(lo);
  const float hi_v = (lo == 0x7bffu) ? 65536.0f : dev::f16_bits_to_f32(lo + 1u);
  return (hi_v - d <= d - lo_v) ? lo + 1u : lo;
}

// Activation quantization into LDS. Pass q covers token t = q / C of the launch
// (C = ceil((cols/8) / 256) passes a token), items j = (q % C) * 256 + thread:
// values 8j .. 8j+8 of the token; four consecutive lanes (a quad) own one 32-value
// block. Token and chunk are uniform, so no lane divides.
template <int XR>
struct XRegs {
  f32x4a v[2 * XR];
};

struct XPlan {
  uint32_t per_tok;  // cols / 8 items a token
  uint32_t chunks;   // passes a token
  uint32_t passes;   // nt * chunks
};

// Issues the loads of passes [q0, q0 + XR) (none past the last pass: a uniform
// test). Items past a token's end read its last item (in bounds; never stored).
template <int XR>
__device__ __forceinline__ void load_x(const float* x, uint32_t cols, uint32_t t0,
                                       const XPlan& pl, uint32_t q0, XRegs<XR>& r) {
#pragma unroll
  for (int k = 0; k < XR; ++k) {
    const uint32_t q = q0 + (uint32_t)k;
    if (q >= pl.passes) break;  // uniform
    const uint32_t t = q / pl.chunks, c = q - t * pl.chunks;
    uint32_t j = c * kGemvThreads + threadIdx.x;
    j = j < pl.per_tok ? j : pl.per_tok - 1u;
    const float* src = x + (uint64_t)(t0 + t) * cols + 8u * j;
    r.v[2 * k] = *(const f32x4a*)src;
    r.v[2 * k + 1] = *(const f32x4a*)(src + 4);
  }
}

template <int XR>
__device__ __forceinline__ void quantize_x(const XRegs<XR>& r, uint32_t nb, const XPlan& pl,
                                           uint32_t q0, uint32_t* lds) {
#pragma unroll
  for (int k = 0; k < XR; ++k) {
    const uint32_t q = q0 + (uint32_t)k;
    if (q >= pl.passes) break;  // uniform
    const uint32_t t = q / pl.chunks, c = q - t * pl.chunks;
    const uint32_t j = c * kGemvThreads + threadIdx.x;
    const f32x4a a = r.v[2 * k], b = r.v[2 * k + 1];
    // Rust's max ignores NaN; so does fmaxf (maxnum: a NaN operand, quiet or
    // signaling, yields the other one).
    float m = __builtin_fmaxf(__builtin_fabsf(a.x), __builtin_fabsf(a.y));
    m = __builtin_fmaxf(m, __builtin_fabsf(a.z));
    m = __builtin_fmaxf(m, __builtin_fabsf(a.w));
    m = __builtin_fmaxf(m, __builtin_fabsf(b.x));
    m = __builtin_fmaxf(m, __builtin_fabsf(b.y));
    m = __builtin_fmaxf(m, __builtin_fabsf(b.z));
    m = __builtin_fmaxf(m, __builtin_fabsf(b.w));
    m = __builtin_fmaxf(m, 0.0f);  // all NaN: 0, as the reference's amax = 0 start
    // max over the quad; a quad is entirely below or past per_tok (a multiple of 4)
    m = __builtin_fmaxf(m, dev::dpp<0xB1>(m));
    m = __builtin_fmaxf(m, dev::dpp<0x4E>(m));
    const float d = div127(m);
    const float id = (d != 0.0f) ? 1.0f / d : 0.0f;
    const uint32_t qa = q8_byte(a.x * id) | (q8_byte(a.y * id) << 8) |
                        (q8_byte(a.z * id) << 16) | (q8_byte(a.w * id) << 24);
    const uint32_t qb = q8_byte(b.x * id) | (q8_byte(b.y * id) << 8) |
                        (q8_byte(b.z * id) << 16) | (q8_byte(b.w * id) << 24);
    // the previous lane's qb (quad_perm [0,0,1,2]); nothing before the first lane
    const uint32_t sub = threadIdx.x & 3u;
    uint32_t prev = (uint32_t)__builtin_amdgcn_mov_dpp((int)qb, 0x90, 0xf, 0xf, true);
    prev = sub == 0u ? 0u : prev;
    if (j < pl.per_tok) {
      uint32_t* blk = lds + ((uint64_t)t * nb + j / 4u) * kXDw;
      *(uint2*)(blk + 2u * sub) = make_uint2(qa, qb);
      *(uint2*)(blk + 8u + 2u * sub) = make_uint2(__builtin_amdgcn_alignbit(qa, prev, 16),
                                                  __builtin_amdgcn_alignbit(qb, qa, 16));
      const uint32_t ta = tail_dw(true, j / 4u), ts = tail_dw(false, j / 4u);
      if (sub == 0u) {
        const float xs = dev::f16_bits_to_f32(f16_bits_away(d));
        *(uint2*)(blk + ta) = make_uint2(0u, __float_as_uint(xs));
        blk[ts + 1u] = __float_as_uint(xs);
      }
      if (sub == 3u) blk[ts] = qb >> 16;
    }
  }
}

// Four waves a SIMD (at most 128 VGPRs) keep every wave of a 14336-row matrix
// resident at once, so its weight stream never pauses between rounds of waves.
// S = 2 (launches with few rows): a weight row takes two 16-lane DPP rows, h = 0 the
// even 16-block steps and h = 1 the odd ones, so a wave holds 2 weight rows and the
// launch twice the waves. Each iteration's two steps are added in order by both DPP
// rows (the products of the other one brought over by a lane swap), so the sum is
// the same as S = 1's, bit for bit.
template <int T, int S, int XR>
__global__ __launch_bounds__(kGemvThreads) void gemv_q8_kernel(const GemvBatch bat, uint32_t cols,
                                                               const float* x, uint32_t n_tokens) {
  // This workgroup's matrix (uniform: scalar selects over the launch's few matrices).
  uint32_t mi = 0;
#pragma unroll
  for (int j = 1; j < kGemvMaxMats; ++j)
    if ((uint32_t)j < bat.n && blockIdx.x >= bat.m[j].wg0) mi = (uint32_t)j;
  const GemvMat M = mi == 0u ? bat.m[0] : mi == 1u ? bat.m[1] : mi == 2u ? bat.m[2] : bat.m[3];
  const uint8_t* __restrict__ w = M.w;
  float* __restrict__ y = M.y;
  const uint32_t rows = M.rows;
  const uint32_t wg = blockIdx.x - M.wg0;
  extern __shared__ uint32_t lds[];  // [T][nb][kXDw]
  const uint32_t nb = cols / 32u;
  const uint32_t t0 = blockIdx.y * T;
  const uint32_t nt = n_tokens - t0 < (uint32_t)T ? n_tokens - t0 : (uint32_t)T;

  const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
  const uint32_t l = lane & 15u;
  const uint32_t h = (lane >> 4) % (uint32_t)S;  // which steps of its row this DPP row takes
  constexpr uint32_t kRowsWg = kRowsPerWg / S;
  const uint32_t row = wg * kRowsWg + wave * (kRowsPerWave / S) + (lane >> 4) / S;
  const bool row_ok = row < rows;
  const uint32_t n_it = (nb + 16u * S - 1u) / (16u * S);  // iterations (S steps) a row
  const uint32_t nbp = gemv_padded_blocks(nb, S);         // LDS blocks a token (whole groups)

  // Weights through a buffer resource based at this workgroup's first row: a lane
  // whose block lies past its row's end asks for an offset beyond the resource, which
  // reads zeros without touching memory. So no load is clamped or branched around,
  // and every step's loads are a lane offset plus an immediate.
  const uint64_t row_bytes = (uint64_t)nb * kQ8Bytes;
  const uint32_t row0 = wg * kRowsWg;
  const uint64_t base = (uint64_t)(uintptr_t)w + row0 * row_bytes;
  const uint64_t left = (uint64_t)rows * row_bytes - row0 * row_bytes;
  const __amdgpu_buffer_rsrc_t rsrc = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(uintptr_t)base, (short)0, (int)(left < kOobOffset ? left : kOobOffset - 1u),
      kBufferWord3);
  // A row past the end reads the last row (its results are not stored).
  const uint32_t lane_off = (uint32_t)((uint64_t)((row_ok ? row : rows - 1u) - row0) * row_bytes) +
                            (h * 16u + l) * kQ8Bytes;
  // Which activation copy this lane's blocks pair with (the parity of a lane's block
  // addresses is the same at every step), as LDS dword offsets of its 8 quant dwords
  // and of its (9th dword, scale) pair; and its byte offsets of the 8 dwords and of
  // the 16-bit word.
  const bool aligned = ((base + lane_off) & 2u) != 0u;
  // a step's blocks start at a multiple of 16, so bit 3 of lane l's block is bit 3 of l
  const uint32_t q_dw = aligned ? 0u : 8u, t_dw = tail_dw(aligned, l);
  const uint32_t dw_off = lane_off + (aligned ? 2u : 0u);
  const uint32_t tail_off = lane_off + (aligned ? 0u : 32u);

  XPlan pl;
  pl.per_tok = cols / 8u;
  pl.chunks = (pl.per_tok + kGemvThreads - 1u) / kGemvThreads;
  pl.passes = nt * pl.chunks;
  XRegs<XR> xr;
  load_x<XR>(x, cols, t0, pl, 0, xr);
  // Keep these loads ahead of the weight prefetch: no load moves across an asm
  // statement that may touch memory (x is not __restrict__, so that covers it).
  __asm__ volatile("" ::: "memory");

  // Iteration it's loads: blocks (it*S + h)*16 + l; beyond the row (or the step count)
  // none.
  auto load_step = [&](uint32_t it, RawBlock& rb) {
    const bool in = (it * S + h) * 16u + l < nb;
    const uint32_t o = it * (16u * S * kQ8Bytes);
    const uint32_t od = in ? dw_off + o : kOobOffset;
    const uint32_t ot = in ? tail_off + o : kOobOffset;
    const v4u a = __builtin_amdgcn_raw_buffer_load_b128(rsrc, od, 0, 0);
    const v4u b = __builtin_amdgcn_raw_buffer_load_b128(rsrc, od + 16u, 0, 0);
    rb.d[0] = a[0]; rb.d[1] = a[1]; rb.d[2] = a[2]; rb.d[3] = a[3];
    rb.d[4] = b[0]; rb.d[5] = b[1]; rb.d[6] = b[2]; rb.d[7] = b[3];
    rb.tail = __builtin_amdgcn_raw_buffer_load_b16(rsrc, ot, 0, 0);
  };

  RawBlock buf[kPipe];
#pragma unroll
  for (int k = 0; k < kPipe; ++k) load_step((uint32_t)k, buf[k]);

  quantize_x<XR>(xr, nbp, pl, 0, lds);
  for (uint32_t q0 = XR; q0 < pl.passes; q0 += XR) {
    load_x<XR>(x, cols, t0, pl, q0, xr);
    quantize_x<XR>(xr, nbp, pl, q0, lds);
  }
  __syncthreads();

  float acc[T];
#pragma unroll
  for (int t = 0; t < T; ++t) acc[t] = 0.0f;

  // Step it into acc: lane L's block is the L-th added. Blocks past the row's end
  // (loaded as zeros, paired with LDS padding) add +0: acc starts at +0 and a zero
  // sum is +0 under round-to-nearest, so acc is never -0 and acc + 0 == acc.
  const uint32_t* lane_x = lds + (uint64_t)(h * 16u + l) * kXDw;
  auto consume = [&](uint32_t it, const RawBlock& rb) {
    const bool ok = (it * S + h) * 16u + l < nb;
    const float ws = dev::f16_bits_to_f32(aligned ? rb.tail : rb.d[0]);
#pragma unroll
    for (int t = 0; t < T; ++t) {
      const uint32_t* xb = lane_x + ((uint64_t)t * nbp + it * 16u * S) * kXDw;
      const uint4 x0 = *(const uint4*)(xb + q_dw);
      const uint4 x1 = *(const uint4*)(xb + q_dw + 4u);
      const uint2 xt = *(const uint2*)(xb + t_dw);
      int s = 0;
      s = __builtin_amdgcn_sdot4((int)rb.d[0], (int)x0.x, s, false);
      s = __builtin_amdgcn_sdot4((int)rb.d[1], (int)x0.y, s, false);
      s = __builtin_amdgcn_sdot4((int)rb.d[2], (int)x0.z, s, false);
      s = __builtin_amdgcn_sdot4((int)rb.d[3], (int)x0.w, s, false);
      s = __builtin_amdgcn_sdot4((int)rb.d[4], (int)x1.x, s, false);
      s = __builtin_amdgcn_sdot4((int)rb.d[5], (int)x1.y, s, false);
      s = __builtin_amdgcn_sdot4((int)rb.d[6], (int)x1.z, s, false);
      s = __builtin_amdgcn_sdot4((int)rb.d[7], (int)x1.w, s, false);
      s = __builtin_amdgcn_sdot4((int)rb.tail, (int)xt.x, s, false);
      float p = (float)s * (ws * __uint_as_float(xt.y));
      p = ok ? p : 0.0f;
      if constexpr (S == 1) {
        acc[t] = chain16(acc[t], p, std::make_integer_sequence<int, 16>{});
      } else {
        // this lane's product and the other DPP row's for the same lane index: step
        // it*2 (h = 0's) first, then step it*2 + 1 (h = 1's)
        const float o = __shfl_xor(p, 16);
        const float first = h == 0u ? p : o, second = h == 0u ? o : p;
        acc[t] = chain16(acc[t], first, std::make_integer_sequence<int, 16>{});
        acc[t] = chain16(acc[t], second, std::make_integer_sequence<int, 16>{});
      }
    }
  };

  // Groups of kPipe steps: consume each step, then load the step kPipe ahead into
  // its buffer (loads past the last step read nothing).
  for (uint32_t g = 0; g < n_it; g += kPipe) {
#pragma unroll
    for (int k = 0; k < kPipe; ++k) {
      consume(g + (uint32_t)k, buf[k]);
      load_step(g + (uint32_t)k + kPipe, buf[k]);
    }
  }

  if (row_ok && l == 0u && h == 0u) {
#pragma unroll
    for (int t = 0; t < T; ++t)
      if ((uint32_t)t < nt) y[(uint64_t)(t0 + t) * rows + row] = acc[t];
  }
}

template <int T, int S, int XR = kXRegs>
hipError_t launch_t(const GemvBatch& b, uint32_t n_wg, uint32_t cols, const float* x,
                    uint32_t n_tokens, hipStream_t s) {
  const dim3 grid(n_wg, (n_tokens + T - 1u) / T);
  const size_t lds = (size_t)T * gemv_padded_blocks(cols / 32u, S) * kXDw * 4u;
  if (lds > 65536u) {
    const hipError_t e = hipFuncSetAttribute((const void*)gemv_q8_kernel<T, S, XR>,
                                             hipFuncAttributeMaxDynamicSharedMemorySize,
                                             (int)lds);
    if (e != hipSuccess) return e;
  }
  hipLaunchKernelGGL((gemv_q8_kernel<T, S, XR>), grid, dim3(kGemvThreads), lds, s, b, cols, x,
                     n_tokens);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Batched Q8_0 GEMM on the matrix cores
// ---------------------------------------------------------------------------
//
// For a batch of activation rows (a decode step's sequences, a prefill chunk) the GEMV
// above takes 4 tokens a launch row, so a 64-token batch reads every weight 16 times.
// Here the activation is quantized once, into a workspace (q8_act_kernel, the same
// arithmetic as quantize_x), and gemm_q8_mfma_kernel takes each 32-value block's
// integer dots of 16 weight rows x 16 tokens from one v_mfma_i32_16x16x32_i8: the int32
// sums are exact, so they are the reference's sumi whatever the order inside the
// instruction. Each output then takes acc = acc + f32(sumi) * (w_scale * x_scale) block
// by block in order from +0, which is dot_q8_row_q8_act (q8_dot.rs:72-109) bit for bit.
//
// Workspace, per 16-token tile tt of the batch (tokens past n_tokens quantize to zeros):
//   quants: 16-byte unit (tt, block pair p, lane) at ((tt * nb/2 + p) * 64 + lane) * 16;
//           lane = grp*16 + c holds quants grp*8 .. +7 of token tt*16 + c of block 2p
//           (bytes 0..7) and of block 2p + 1 (bytes 8..15): the MFMA B operand order,
//           1 KiB per load instruction.
//   scales: f32 (the binary16 scale's value); token c's scales of blocks 4u .. 4u + 3
//           in the 16-byte unit (tt * nb/4 + u) * 16 + c after the quants.
// Needs cols % 1024 == 0 (whole pairs of 16-block chunks) and 16-byte aligned weights.

constexpr uint32_t kMmSub = 16;  // blocks of one set of B operands (a sub-chunk)

// Weight staging of a chunk of CH blocks (CH = 16 or 32): a row's CH * 34 bytes go
// to LDS at a row stride of CH * 34 + 8 (at CH = 16, 138 dwords: the 16 rows' reads start
// in 16 distinct even banks). Thread t stages row t / 16: its 16-byte units (t % 16) +
// 16j and the scales of blocks (t % 16) + 16m.
template <uint32_t CH>
struct MmShape {
  static constexpr uint32_t kRowBytes = CH * kQ8Bytes;
  static constexpr uint32_t kStride = kRowBytes + 8u;
  static constexpr uint32_t kRowUnits = kRowBytes / 16u;
  static constexpr uint32_t kRuns = (kRowUnits + 15u) / 16u;
  static constexpr uint32_t kScales = CH / 16u;
};

__host__ __device__ constexpr uint64_t mm_quant_bytes(uint32_t n_tiles, uint32_t nb) {
  return (uint64_t)n_tiles * nb * 16u * 32u;  // 16 tokens x 32 quants a block
}

// 64-thread workgroups: measured 1.0-1.4% faster steps than 256 at the same kernel time
// (Llama-3-8B projections, 64 tokens).
constexpr uint32_t kActThreads = 64;

__global__ __launch_bounds__(kActThreads) void q8_act_kernel(const float* __restrict__ x,
                                                             uint32_t cols, uint32_t n_tokens,
                                                             uint32_t n_tiles,
                                                             uint8_t* __restrict__ ws) {
  // Item i: token t = i / (cols/8), values 8j .. 8j + 7 with j = i % (cols/8): piece
  // grp = j % 4 of block j / 4. The four pieces of a block are a quad of lanes (the
  // item count per token is a multiple of 4), which exits or stays as a whole.
  const uint32_t per = cols / 8u, nb = cols / 32u;
  const uint64_t i = (uint64_t)blockIdx.x * kActThreads + threadIdx.x;
  if (i >= (uint64_t)n_tiles * 16u * per) return;
  const uint32_t t = (uint32_t)(i / per), j = (uint32_t)(i % per);
  f32x4a a = {0.0f, 0.0f, 0.0f, 0.0f}, b = {0.0f, 0.0f, 0.0f, 0.0f};
  if (t < n_tokens) {
    const float* src = x + (uint64_t)t * cols + 8u * j;
    a = *(const f32x4a*)src;
    b = *(const f32x4a*)(src + 4);
  }
  float m = __builtin_fmaxf(__builtin_fabsf(a.x), __builtin_fabsf(a.y));
  m = __builtin_fmaxf(m, __builtin_fabsf(a.z));
  m = __builtin_fmaxf(m, __builtin_fabsf(a.w));
  m = __builtin_fmaxf(m, __builtin_fabsf(b.x));
  m = __builtin_fmaxf(m, __builtin_fabsf(b.y));
  m = __builtin_fmaxf(m, __builtin_fabsf(b.z));
  m = __builtin_fmaxf(m, __builtin_fabsf(b.w));
  m = __builtin_fmaxf(m, 0.0f);  // all NaN: 0, as the reference's amax = 0 start
  m = __builtin_fmaxf(m, dev::dpp<0xB1>(m));
  m = __builtin_fmaxf(m, dev::dpp<0x4E>(m));
  const float d = div127(m);
  const float id = (d != 0.0f) ? 1.0f / d : 0.0f;
  const uint32_t qa = q8_byte(a.x * id) | (q8_byte(a.y * id) << 8) |
                      (q8_byte(a.z * id) << 16) | (q8_byte(a.w * id) << 24);
  const uint32_t qb = q8_byte(b.x * id) | (q8_byte(b.y * id) << 8) |
                      (q8_byte(b.z * id) << 16) | (q8_byte(b.w * id) << 24);
  const uint32_t tt = t / 16u, c = t % 16u, blk = j / 4u, grp = j % 4u;
  const uint64_t unit = ((uint64_t)tt * (nb / 2u) + blk / 2u) * 64u + grp * 16u + c;
  *(uint2*)(ws + unit * 16u + (blk % 2u) * 8u) = make_uint2(qa, qb);
  if (grp == 0u) {
    float* xs = (float*)(ws + mm_quant_bytes(n_tiles, nb));
    xs[(((uint64_t)tt * (nb / 4u) + blk / 4u) * 16u + c) * 4u + blk % 4u] =
        dev::f16_bits_to_f32(f16_bits_away(d));
  }
}

// A workgroup: 16 weight rows of one of the launch's matrices x 4 token tiles (wave w:
// tile blockIdx.y * 4 + w). The 16 rows' Q8_0 bytes are staged chunk by chunk (CH
// blocks) into LDS as stored, with their scales as f32 [block][row]; a lane (c, grp)
// reads its A operand, quants grp*8 .. +7 of row c, from there (one 16-bit realignment
// for blocks at 2 mod 4). The B operands load one 16-block sub-chunk ahead. The weights:
// chunk k + 1 loads while chunk k is computed, staged by the four computing waves
// (without PROD), or by a fifth wave two chunks ahead (PROD: launches that leave one
// workgroup a CU, where a chunk's weight loads would otherwise hold up the computing
// waves' B-operand waits). Chunks are 32 blocks wherever the chunk count is even, else 16.
struct MmB {
  uint4 q[kMmSub / 2];  // block pairs
  uint4 s[kMmSub / 4];  // scales of 4 blocks
};

template <uint32_t CH, bool PF, bool PROD>
__global__ __launch_bounds__(PROD ? 320 : 256)
__attribute__((amdgpu_waves_per_eu(CH == 16 ? 4 : 1, 8)))
void gemm_q8_mfma_kernel(const GemvBatch bat, uint32_t cols, uint32_t n_tokens,
                         uint32_t n_tiles, const uint8_t* __restrict__ ws) {
  using S = MmShape<CH>;
  uint32_t mi = 0;
#pragma unroll
  for (int j = 1; j < kGemvMaxMats; ++j)
    if ((uint32_t)j < bat.n && blockIdx.x >= bat.m[j].wg0) mi = (uint32_t)j;
  const GemvMat M = mi == 0u ? bat.m[0] : mi == 1u ? bat.m[1] : mi == 2u ? bat.m[2] : bat.m[3];
  const uint32_t rows = M.rows;
  const uint32_t row0 = (blockIdx.x - M.wg0) * 16u;
  const uint32_t nb = cols / 32u;
  const uint64_t row_bytes = (uint64_t)nb * kQ8Bytes;
  const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
  const uint32_t c = lane & 15u, grp = lane >> 4;
  const uint32_t tt = blockIdx.y * 4u + wave;
  const bool on = tt < n_tiles;  // wave-uniform; an idle wave still stages
  const uint32_t ttc = on ? tt : n_tiles - 1u;

  __shared__ __align__(16) uint8_t s_w[2][16 * S::kStride];
  __shared__ __align__(16) float s_ws[2][CH][16];

  // Staging (MmShape): a row past the matrix stages its last row (never stored).
  const uint32_t sr = tid / 16u, sc = tid % 16u;
  const uint8_t* wsrc = M.w + (uint64_t)(row0 + sr < rows ? row0 + sr : rows - 1u) * row_bytes;
  uint4 stg[S::kRuns];
  uint32_t sbits[S::kScales];
  auto stage_load = [&](uint32_t k) {
    const uint8_t* p = wsrc + (uint64_t)k * S::kRowBytes;
#pragma unroll
    for (uint32_t j = 0; j < S::kRuns; ++j)
      if (sc + 16u * j < S::kRowUnits) stg[j] = *(const uint4*)(p + (sc + 16u * j) * 16u);
#pragma unroll
    for (uint32_t m = 0; m < S::kScales; ++m)
      sbits[m] = *(const uint16_t*)(p + (sc + 16u * m) * kQ8Bytes);
  };
  auto stage_store = [&](uint32_t buf) {
    uint8_t* d = &s_w[buf][sr * S::kStride + sc * 16u];
#pragma unroll
    for (uint32_t j = 0; j < S::kRuns; ++j)
      if (sc + 16u * j < S::kRowUnits) {
        uint2* dst = (uint2*)(d + 256u * j);  // 8-byte aligned rows
        dst[0] = make_uint2(stg[j].x, stg[j].y);
        dst[1] = make_uint2(stg[j].z, stg[j].w);
      }
#pragma unroll
    for (uint32_t m = 0; m < S::kScales; ++m)
      s_ws[buf][sc + 16u * m][sr] = dev::f16_bits_to_f32(sbits[m]);
  };
  // B operands and x scales of sub-chunk g (blocks 16g .. 16g + 15) for this wave's
  // token tile.
  const uint8_t* bq = ws + (((uint64_t)ttc * (nb / 2u)) * 64u + lane) * 16u;
  const uint8_t* bs = ws + mm_quant_bytes(n_tiles, nb) + (((uint64_t)ttc * (nb / 4u)) * 16u + c) * 16u;
  auto bq_load = [&](uint32_t g, int p) {
    return *(const uint4*)(bq + ((uint64_t)g * (kMmSub / 2u) + (uint32_t)p) * 1024u);
  };
  auto bs_load = [&](uint32_t g, int u) {
    return *(const uint4*)(bs + ((uint64_t)g * (kMmSub / 4u) + (uint32_t)u) * 256u);
  };
  auto b_load = [&](uint32_t g, MmB& o) {
#pragma unroll
    for (int p = 0; p < (int)kMmSub / 2; ++p) o.q[p] = bq_load(g, p);
#pragma unroll
    for (int u = 0; u < (int)kMmSub / 4; ++u) o.s[u] = bs_load(g, u);
  };

  float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  const uint32_t nsub = nb / kMmSub;
  // One block's epilogue for this lane's 4 outputs: the reference's
  // acc + f32(sumi) * (w_scale * x_scale), no fused multiply-add.
  auto epilogue = [&](const v4i& si, const float4& w4, float xs) {
    acc[0] = acc[0] + (float)si[0] * (w4.x * xs);
    acc[1] = acc[1] + (float)si[1] * (w4.y * xs);
    acc[2] = acc[2] + (float)si[2] * (w4.z * xs);
    acc[3] = acc[3] + (float)si[3] * (w4.w * xs);
  };
  // Chunk k from LDS buffer `buf`, in groups of 4 blocks with B operands o. A group's
  // four integer dots are issued before its epilogues, which then run in block order.
  // Each register of o is reloaded with the next sub-chunk's operand
  // once its last use has issued (one set of registers, a sub-chunk ahead); past the
  // last sub-chunk the reloads read it again (in bounds, never used), so the loop has no
  // branch. With PF the next group's A operands and weight scales are read from LDS
  // before this group's dots, so their latency passes under the epilogues (a lone
  // wave on its SIMD has nothing else to cover it); without PF each group reads its own
  // just before use (fewer registers, for launches where several waves share a SIMD).
  auto compute = [&](uint32_t buf, MmB& o, uint32_t k) {
    constexpr int kGroups = (int)CH / 4;
    const uint8_t* wl = &s_w[buf][c * S::kStride + grp * 8u];
    uint32_t ra[2][4][3];  // a group's A operand dwords as stored (3 at 2 mod 4, else 2)
    float4 rw[2][4];       // its weight scales of rows grp*4 .. +3
    auto group_read = [&](int g, int slot) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int b = 4 * g + i;  // the block's parity is its parity in the chunk
        if (b % 2 == 0) {         // quants at 34b + 2 + 8grp: 2 mod 4
          const uint32_t* p = (const uint32_t*)(wl + 34 * b);
          ra[slot][i][0] = p[0];
          ra[slot][i][1] = p[1];
          ra[slot][i][2] = p[2];
        } else {  // 0 mod 4
          const uint32_t* p = (const uint32_t*)(wl + 34 * b + 2);
          ra[slot][i][0] = p[0];
          ra[slot][i][1] = p[1];
        }
        if (PF) rw[slot][i] = *(const float4*)&s_ws[buf][b][grp * 4u];
      }
    };
    if (PF) group_read(0, 0);
#pragma unroll
    for (int g = 0; g < kGroups; ++g) {
      const int cur = PF ? (g & 1) : 0;
      const uint32_t sub = (uint32_t)g / 4u;
      const int b0 = (4 * g) % (int)kMmSub;  // first block of the group in its sub-chunk
      const uint32_t gn = k * (CH / kMmSub) + sub + 1u;
      const uint32_t kn = gn < nsub ? gn : nsub - 1u;
      if (!PF) group_read(g, cur);
      long av[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int b = b0 + i;
        uint32_t lo, hi;
        if (b % 2 == 0) {
          lo = __builtin_amdgcn_alignbit(ra[cur][i][1], ra[cur][i][0], 16);
          hi = __builtin_amdgcn_alignbit(ra[cur][i][2], ra[cur][i][1], 16);
        } else {
          lo = ra[cur][i][0];
          hi = ra[cur][i][1];
        }
        av[i] = (long)(((uint64_t)hi << 32) | lo);
      }
      // the next group's reads go out before this group's dots and epilogues
      if (PF && g + 1 < kGroups) group_read(g + 1, cur ^ 1);
      v4i si[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int b = b0 + i;
        const uint4 u = o.q[b / 2];
        const long bv = (b % 2 == 0) ? (long)(((uint64_t)u.y << 32) | u.x)
                                     : (long)(((uint64_t)u.w << 32) | u.z);
        const v4i zero = {0, 0, 0, 0};
        si[i] = __builtin_amdgcn_mfma_i32_16x16x32_i8(av[i], bv, zero, 0, 0, 0);
      }
      // the reloads stay after the dots that read the registers they overwrite
      __builtin_amdgcn_sched_barrier(0);
      o.q[b0 / 2] = bq_load(kn, b0 / 2);
      o.q[b0 / 2 + 1] = bq_load(kn, b0 / 2 + 1);
      const uint4 s4 = o.s[b0 / 4];
      o.s[b0 / 4] = bs_load(kn, b0 / 4);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int i = 0; i < 4; ++i)
        epilogue(si[i], PF ? rw[cur][i] : *(const float4*)&s_ws[buf][4 * g + i][grp * 4u],
                 __uint_as_float(i == 0 ? s4.x : i == 1 ? s4.y : i == 2 ? s4.z : s4.w));
    }
  };

  const uint32_t nc = nb / CH;  // even (launch_gemm_q8_mfma picks CH so)
  MmB bo;
  if (PROD) {
    // A fifth wave stages the weights: two chunks in flight in its registers, one chunk
    // into the LDS buffer the four computing waves read next, their scales converted
    // from there. Its waits on HBM are its own: the computing waves' load counters hold
    // only their B operands, which a weight load issued before them would otherwise
    // hold back (loads retire in issue order).
    // Lane l stages units (l % 4) + 4j of row l / 4; it converts the scales of row l % 16,
    // blocks l / 16 + 4i.
    constexpr uint32_t kPer = (S::kRowUnits + 3u) / 4u;
    constexpr uint32_t kSc = CH / 4u;
    if (wave == 4u) {
      const uint32_t pr = lane / 4u, pu = lane % 4u;
      const uint8_t* psrc =
          M.w + (uint64_t)(row0 + pr < rows ? row0 + pr : rows - 1u) * row_bytes + pu * 16u;
      uint4 pst[2][kPer];
      auto p_load = [&](uint32_t k, int set) {
        const uint8_t* p = psrc + (uint64_t)k * S::kRowBytes;
#pragma unroll
        for (uint32_t j = 0; j < kPer; ++j)
          if (S::kRowUnits % 4u == 0u || pu + 4u * j < S::kRowUnits)
            pst[set][j] = *(const uint4*)(p + 64u * j);
      };
      auto p_store = [&](int set, uint32_t buf) {
        uint8_t* d = &s_w[buf][pr * S::kStride + pu * 16u];
#pragma unroll
        for (uint32_t j = 0; j < kPer; ++j)
          if (S::kRowUnits % 4u == 0u || pu + 4u * j < S::kRowUnits) {
            uint2* dst = (uint2*)(d + 64u * j);  // 8-byte aligned rows
            dst[0] = make_uint2(pst[set][j].x, pst[set][j].y);
            dst[1] = make_uint2(pst[set][j].z, pst[set][j].w);
          }
        const uint32_t sr = lane % 16u, sb0 = lane / 16u;
        uint32_t sb[kSc];
#pragma unroll
        for (uint32_t i = 0; i < kSc; ++i)
          sb[i] = *(const uint16_t*)&s_w[buf][sr * S::kStride + (sb0 + 4u * i) * kQ8Bytes];
#pragma unroll
        for (uint32_t i = 0; i < kSc; ++i) s_ws[buf][sb0 + 4u * i][sr] = dev::f16_bits_to_f32(sb[i]);
      };
      // Loads past the last chunk read the last chunk again (in bounds, never stored),
      // so every iteration issues set 1's loads before set 0's and the wait before a
      // set's stores leaves the other set in flight.
      const uint32_t last = nc - 1u;
      p_load(0, 0);
      p_load(1, 1);  // nc >= 2
      p_store(0, 0);
      p_load(2u < last ? 2u : last, 0);
      __syncthreads();  // buffer 0 holds chunk 0
      for (uint32_t k = 0; k < nc; k += 2) {
        // set 1 holds chunk k + 1, set 0 chunk k + 2
        p_store(1, 1);
        p_load(k + 3u < last ? k + 3u : last, 1);
        __syncthreads();
        if (k + 2u < nc) p_store(0, 0);
        p_load(k + 4u < last ? k + 4u : last, 0);
        __syncthreads();
      }
      return;  // after the last barrier
    }
    if (on) b_load(0, bo);
    __syncthreads();
    for (uint32_t k = 0; k < nc; k += 2) {
      if (on) compute(0, bo, k);
      __syncthreads();
      if (on) compute(1, bo, k + 1);
      __syncthreads();
    }
  } else {
  if (on) b_load(0, bo);
  stage_load(0);
  stage_store(0);
  __syncthreads();
  for (uint32_t k = 0; k < nc; k += 2) {
    // chunk k (buffer 0) while chunk k + 1's weights load; then chunk k + 1 (buffer 1)
    stage_load(k + 1);
    if (on) compute(0, bo, k);
    stage_store(1);
    __syncthreads();
    if (k + 2 < nc) stage_load(k + 2);
    if (on) compute(1, bo, k + 1);
    if (k + 2 < nc) stage_store(0);
    __syncthreads();
  }
  }

  if (!on) return;
  const uint32_t tok = tt * 16u + c;
  if (tok < n_tokens) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const uint32_t row = row0 + grp * 4u + (uint32_t)r;
      if (row < rows) M.y[(uint64_t)tok * rows + row] = acc[r];
    }
  }
}

}  // namespace

bool gemm_mfma_eligible(const GemvBatch& b, uint32_t cols, uint32_t n_tokens) {
  if (n_tokens < kGemmMfmaMinTokens || cols % 1024u != 0u) return false;
  for (uint32_t m = 0; m < b.n; ++m)
    if ((uintptr_t)b.m[m].w % 16u != 0u) return false;
  return true;
}

uint64_t gemm_mfma_workspace_bytes(uint32_t cols, uint32_t n_tokens) {
  const uint32_t n_tiles = (n_tokens + 15u) / 16u, nb = cols / 32u;
  return mm_quant_bytes(n_tiles, nb) + (uint64_t)n_tiles * nb * 16u * 4u;
}

// Batched launches of at most this many workgroups (one a CU on MI355X's 256 CUs) stage
// their weights by a fifth wave (gemm_q8_mfma_kernel with PROD).
#ifndef FKV_GEMM_PRODUCER_WGS
#define FKV_GEMM_PRODUCER_WGS 256
#endif
constexpr uint32_t kGemmProducerWgs = FKV_GEMM_PRODUCER_WGS;

hipError_t launch_gemm_q8_mfma(GemvBatch b, uint32_t cols, const float* x, uint32_t n_tokens,
                               void* workspace, hipStream_t s) {
  uint32_t n_wg = 0;
  for (uint32_t m = 0; m < b.n; ++m) {
    b.m[m].wg0 = n_wg;
    n_wg += (b.m[m].rows + 15u) / 16u;
  }
  for (uint32_t m = b.n; m < (uint32_t)kGemvMaxMats; ++m) b.m[m] = b.m[0];
  const uint32_t n_tiles = (n_tokens + 15u) / 16u;
  const uint64_t items = (uint64_t)n_tiles * 16u * (cols / 8u);
  q8_act_kernel<<<(uint32_t)((items + kActThreads - 1u) / kActThreads), kActThreads, 0, s>>>(
      x, cols, n_tokens, n_tiles, (uint8_t*)workspace);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  // 32-block chunks with the A operands and weight scales read a group ahead wherever
  // the chunk count is even (columns a multiple of 2048), staged by a producer wave
  // where the launch leaves one workgroup a CU; otherwise 16-block chunks. Measured at
  // 64 tokens (Llama-3-8B projections, one box, us a call): q/k/v 18.0 (producer 20.7,
  // 16-block chunks 21.1), attn_output 12.2, gate/up 56.9 (16-block chunks 60.0,
  // producer 72.1), down 32.0 (no producer 33.6).
  const uint32_t nb = cols / 32u;
  const dim3 grid(n_wg, (n_tiles + 3u) / 4u);
  const bool one_a_cu = (uint64_t)grid.x * grid.y <= kGemmProducerWgs;
  const uint8_t* wsp = (const uint8_t*)workspace;
  if (nb % 64u != 0u)
    gemm_q8_mfma_kernel<16, false, false><<<grid, 256, 0, s>>>(b, cols, n_tokens, n_tiles, wsp);
  else if (one_a_cu)
    gemm_q8_mfma_kernel<32, true, true><<<grid, 320, 0, s>>>(b, cols, n_tokens, n_tiles, wsp);
  else
    gemm_q8_mfma_kernel<32, true, false><<<grid, 256, 0, s>>>(b, cols, n_tokens, n_tiles, wsp);
  return hipGetLastError();
}

size_t gemv_lds_bytes(uint32_t tokens, uint32_t cols) {
  return (size_t)tokens * gemv_padded_blocks(cols / 32u) * kXDw * 4u;
}

// Launches of one token whose S = 1 grid would leave SIMDs with fewer than two waves
// (under 512 workgroups of 4 waves on 256 CUs) take S = 2, when its LDS fits as well.
constexpr uint32_t kGemvSplitBelowWgs = 512;

uint32_t gemv_tokens_per_launch(uint32_t n_tokens, uint32_t cols) {
  uint32_t t = n_tokens >= 3u ? 4u : (n_tokens == 2u ? 2u : 1u);
  while (t > 1u && gemv_lds_bytes(t, cols) > 65536u) t /= 2u;
  return t;
}

hipError_t launch_gemv_q8(GemvBatch b, uint32_t cols, const float* x, uint32_t n_tokens,
                          hipStream_t s) {
  uint32_t n_wg = 0;
  for (uint32_t m = 0; m < b.n; ++m) n_wg += (b.m[m].rows + kRowsPerWg - 1u) / kRowsPerWg;
  const uint32_t tpl = gemv_tokens_per_launch(n_tokens, cols);
  const uint32_t S = (tpl == 1u && n_wg < kGemvSplitBelowWgs &&
                      (size_t)gemv_padded_blocks(cols / 32u, 2) * kXDw * 4u <= 65536u)
                         ? 2u
                         : 1u;
  n_wg = 0;
  for (uint32_t m = 0; m < b.n; ++m) {
    b.m[m].wg0 = n_wg;
    n_wg += (b.m[m].rows + kRowsPerWg / S - 1u) / (kRowsPerWg / S);
  }
  for (uint32_t m = b.n; m < (uint32_t)kGemvMaxMats; ++m) b.m[m] = b.m[0];
  switch (tpl) {
    case 4: return launch_t<4, 1>(b, n_wg, cols, x, n_tokens, s);
    case 2: return launch_t<2, 1, 4>(b, n_wg, cols, x, n_tokens, s);
    default:
      if (cols > 4096u)
        return S == 2u ? launch_t<1, 2, kXRegsWide>(b, n_wg, cols, x, n_tokens, s)
                       : launch_t<1, 1, kXRegsWide>(b, n_wg, cols, x, n_tokens, s);
      return S == 2u ? launch_t<1, 2>(b, n_wg, cols, x, n_tokens, s)
                     : launch_t<1, 1>(b, n_wg, cols, x, n_tokens, s);
  }
}

}  // namespace fkv
