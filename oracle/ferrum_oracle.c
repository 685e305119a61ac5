/*
 * ferrum_oracle.c — CPU restatement of Ferrum's KV-cache path (TEST INFRASTRUCTURE).
 *
 * Loaded only by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
 * leg, as the checker. Compiled with -ffp-contract=off so that every a*b+c is
 * two roundings, as in Rust (rustc never contracts to FMA); the AVX2 section
 * uses FMA only where crates/kernels/src/avx2.rs calls an FMA intrinsic.
 * See ferrum_oracle.h for what pins each function.
 */
#include "ferrum_oracle.h"

#include <float.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include <immintrin.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ------------------------------------------------------------------------- */
/* Layout (include/ferrum_kv.h): pool[block][layer][kv][head][tile].          */
/* F32 tiles are token-major [B][D]. F16 K tiles are [D/8][B][8] and F16 V     */
/* tiles are [D][B]: the operand orders of the MFMA decode kernel.             */
/* ------------------------------------------------------------------------- */

/* Tiles are padded to a multiple of 16 bytes so every tile starts 16-byte aligned. */
uint64_t fo_tile_bytes(const fo_layout* l) {
  uint64_t elems = (uint64_t)l->block_size * l->head_dim, raw;
  switch (l->dtype) {
    case 0: raw = elems * 4; break;
    case 1: raw = (uint64_t)l->block_size * ((l->head_dim + 7) / 8 * 8) * 2; break;  /* K runs of 8 */
    case 8: raw = elems + (elems / 32) * 2; break;
    default: return 0;
  }
  return (raw + 15) / 16 * 16;
}

uint64_t fo_block_bytes(const fo_layout* l) {
  return (uint64_t)l->n_layers * 2 * l->n_kv_heads * fo_tile_bytes(l);
}

static uint64_t tile_offset(const fo_layout* l, uint64_t block, uint32_t layer, int kv,
                            uint32_t head) {
  uint64_t t = fo_tile_bytes(l);
  return block * fo_block_bytes(l) + (((uint64_t)layer * 2 + kv) * l->n_kv_heads + head) * t;
}

/* ------------------------------------------------------------------------- */
/* binary16 codec                                                              */
/* ------------------------------------------------------------------------- */

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* f16_to_f32, crates/core-types/src/dtype.rs:135-154. */
float fo_f16_to_f32(uint16_t bits) {
  uint32_t sign = (uint32_t)(bits >> 15) & 1u;
  uint32_t exp = (uint32_t)(bits >> 10) & 0x1fu;
  uint32_t frac = (uint32_t)bits & 0x3ffu;
  uint32_t out;
  if (exp == 0) {
    if (frac == 0) {
      out = sign << 31;
    } else {
      float scale = u2f((127u - 24u) << 23); /* 2^-24 */
      float mag = (float)frac * scale;        /* exact: frac < 2^10 */
      out = f2u(mag) | (sign << 31);
    }
  } else if (exp == 31) {
    out = (sign << 31) | (0xffu << 23) | (frac << 13);
  } else {
    out = (sign << 31) | ((exp + (127u - 15u)) << 23) | (frac << 13);
  }
  return u2f(out);
}

/* f32 -> binary16. Written from IEEE 754-2008 section 4.3 (rounding) and 3.4
 * (binary16 encoding), with two tie rules:
 *   rounding 0: roundTiesToEven (the north-star rule for f16 KV storage);
 *   rounding 1: ties away from zero, the behaviour of Ferrum's only encoder
 *               `f32_to_f16_bits` (crates/kernels/src/q8_dot.rs:111-139).
 * NaN keeps the top 10 payload bits and stays a NaN (the rule of
 * q8_dot.rs:118-121); +-Inf and overflow give +-Inf. */
uint16_t fo_f32_to_f16(float x, int32_t rounding) {
  uint32_t u = f2u(x);
  uint32_t sign = (u >> 16) & 0x8000u;
  uint32_t ax = u & 0x7fffffffu;
  if (ax >= 0x7f800000u) {
    if (ax == 0x7f800000u) return (uint16_t)(sign | 0x7c00u);
    uint32_t hf = (ax & 0x7fffffu) >> 13;
    return (uint16_t)(sign | 0x7c00u | hf | (hf == 0 ? 1u : 0u));
  }
  /* 65520 = 65504 + half an ulp: both rules round it (and above) to Inf. */
  if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);
  if (ax >= 0x38800000u) { /* result is a normal binary16 (>= 2^-14) */
    uint32_t add = (rounding == 0) ? (0x0fffu + ((ax >> 13) & 1u)) : 0x1000u;
    uint32_t r = ax + add;
    return (uint16_t)(sign | ((r - 0x38000000u) >> 13));
  }
  /* Below 2^-14: result is subnormal (units of 2^-24) or zero. */
  if (ax < 0x33000000u) return (uint16_t)sign; /* < 2^-25: rounds to 0 either way */
  uint32_t e = ax >> 23;                       /* 102..112 */
  uint32_t mant = (ax & 0x7fffffu) | 0x800000u;
  uint32_t shift = 126u - e;                   /* 14..24 */
  uint32_t q = mant >> shift;
  uint32_t rem = mant & ((1u << shift) - 1u);
  uint32_t half = 1u << (shift - 1u);
  if (rounding == 0) {
    if (rem > half || (rem == half && (q & 1u))) q++;
  } else {
    if (rem >= half) q++;
  }
  return (uint16_t)(sign | q);
}

void fo_f32_to_f16_array(const float* x, uint16_t* out, uint64_t n, int32_t rounding) {
  for (uint64_t i = 0; i < n; i++) out[i] = fo_f32_to_f16(x[i], rounding);
}

void fo_f16_to_f32_array(const uint16_t* x, float* out, uint64_t n) {
  for (uint64_t i = 0; i < n; i++) out[i] = fo_f16_to_f32(x[i]);
}

/* ------------------------------------------------------------------------- */
/* Q8_0 codec                                                                  */
/* ------------------------------------------------------------------------- */

/* Rust `f32::max`: a NaN argument yields the other argument (as fmaxf). */
static inline float rust_max(float a, float b) { return fmaxf(a, b); }

/* Rust `f as i32`: saturating, NaN -> 0. */
static inline int32_t rust_as_i32(float f) {
  if (isnan(f)) return 0;
  if (f >= 2147483648.0f) return INT32_MAX;
  if (f <= -2147483648.0f) return INT32_MIN;
  return (int32_t)f;
}

/* One block of Q8Activation::quantize_into (crates/kernels/src/q8_dot.rs:46-59):
 * amax = max|v|; d = amax/127; id = d != 0 ? 1/d : 0; q = clamp(round(v*id))
 * (Rust round = half away from zero, `as i32` saturates); the stored scale is
 * f16(d) while q uses the pre-f16 id (q8_dot.rs:54-55). */
void fo_q8_quantize_block(const float* x32, int32_t rounding, uint16_t* scale_out,
                          int8_t* q_out) {
  float amax = 0.0f;
  for (int j = 0; j < 32; j++) amax = rust_max(amax, fabsf(x32[j]));
  float d = amax / 127.0f;
  float id = (d != 0.0f) ? 1.0f / d : 0.0f;
  *scale_out = fo_f32_to_f16(d, rounding);
  for (int j = 0; j < 32; j++) {
    int32_t q = rust_as_i32(roundf(x32[j] * id));
    if (q < -128) q = -128;
    if (q > 127) q = 127;
    q_out[j] = (int8_t)q;
  }
}

void fo_q8_quantize_row(const float* x, uint64_t n, int32_t rounding, uint8_t* out) {
  for (uint64_t b = 0; b < n / 32; b++) {
    uint16_t s;
    int8_t q[32];
    fo_q8_quantize_block(x + b * 32, rounding, &s, q);
    out[b * 34 + 0] = (uint8_t)(s & 0xff);
    out[b * 34 + 1] = (uint8_t)(s >> 8);
    memcpy(out + b * 34 + 2, q, 32);
  }
}

/* dequant, DType::Q8_0 arm (crates/kernels/src/scalar.rs:261-279, pack.rs:23-34):
 * out = f16_to_f32(scale) * (i8 as f32). */
void fo_q8_dequant(const uint8_t* blocks, uint64_t n, float* out) {
  for (uint64_t b = 0; b < n / 32; b++) {
    const uint8_t* blk = blocks + b * 34;
    float scale = fo_f16_to_f32((uint16_t)(blk[0] | (blk[1] << 8)));
    for (int j = 0; j < 32; j++) out[b * 32 + j] = scale * (float)(int8_t)blk[2 + j];
  }
}

/* Kernels::gemm for DType::Q8_0 (crates/kernels/src/scalar.rs:98-116,191-204 through
 * par.rs:9-26; Kernels::gemv is n_tokens = 1, scalar.rs:84-96). For every token the
 * activation row is quantized by Q8Activation::quantize_into (q8_dot.rs:35-61):
 * fo_q8_quantize_block with the reference's ties-away f32_to_f16_bits
 * (q8_dot.rs:111-139), the scale kept as f16_to_f32 of those bits. Each weight row
 * is then dot_q8_row_q8_act (q8_dot.rs:72-109): acc = 0, and for every block in
 * order acc += (float)sumi * (w_scale * x_scale), sumi the int32 dot of the two i8
 * runs. y[t * rows + r]. The caller has validated the shapes (cols % 32 == 0,
 * w holds rows * (cols/32) * 34 bytes). */
void fo_q8_gemm(const uint8_t* w, uint64_t rows, uint64_t cols, const float* x,
                uint64_t n_tokens, float* y, int32_t threads) {
  if (threads <= 0) threads = omp_get_max_threads();
  const uint64_t nb = cols / 32;
  int8_t* xq = (int8_t*)malloc(cols ? cols : 1);
  float* xs = (float*)malloc((nb ? nb : 1) * sizeof(float));
  for (uint64_t t = 0; t < n_tokens; t++) {
    for (uint64_t b = 0; b < nb; b++) {
      uint16_t bits;
      fo_q8_quantize_block(x + t * cols + b * 32, 1, &bits, xq + b * 32);
      xs[b] = fo_f16_to_f32(bits);
    }
#pragma omp parallel for schedule(static) num_threads(threads)
    for (uint64_t r = 0; r < rows; r++) {
      const uint8_t* row = w + r * nb * 34;
      float acc = 0.0f;
      for (uint64_t b = 0; b < nb; b++) {
        const uint8_t* blk = row + b * 34;
        const float ws = fo_f16_to_f32((uint16_t)(blk[0] | (blk[1] << 8)));
        int32_t sumi = 0;
        for (int j = 0; j < 32; j++) sumi += (int32_t)(int8_t)blk[2 + j] * (int32_t)xq[b * 32 + j];
        acc += (float)sumi * (ws * xs[b]);
      }
      y[t * rows + r] = acc;
    }
  }
  free(xq);
  free(xs);
}

/* ------------------------------------------------------------------------- */
/* dot / softmax (scalar reference backend)                                    */
/* ------------------------------------------------------------------------- */

/* scalar dot, crates/kernels/src/scalar.rs:158-165: left to right, no FMA. */
float fo_dot(const float* a, const float* b, uint64_t n) {
  float acc = 0.0f;
  for (uint64_t i = 0; i < n; i++) acc += a[i] * b[i];
  return acc;
}

/* softmax_max, crates/kernels/src/math.rs:17-25: NaN never compares greater. */
static float softmax_max(const float* x, uint64_t n) {
  float max = -INFINITY;
  for (uint64_t i = 0; i < n; i++)
    if (x[i] > max) max = x[i];
  return max;
}

/* rope_tensor, crates/kernels/src/scalar.rs:167-189, with the angle of
 * math.rs:31-34: in every head_dim row, dims (2i, 2i+1) with 2i < rope_dim
 * (GGML_ROPE_TYPE_NORMAL) rotate by f = pos / theta^(2i / rope_dim), everything in
 * f32 and each product rounded (a' = a cos f - b sin f, b' = a sin f + b cos f).
 * Returns without change when head_dim == 0, rope_dim == 0 or rope_dim > head_dim
 * (scalar.rs:174-176). */
void fo_rope(float* data, uint64_t n_rows, uint32_t head_dim, uint32_t rope_dim, uint32_t pos,
             float theta) {
  if (head_dim == 0 || rope_dim == 0 || rope_dim > head_dim) return;
  for (uint64_t r = 0; r < n_rows; r++) {
    float* h = data + r * head_dim;
    for (uint32_t i = 0; i < rope_dim; i += 2) {
      const uint32_t pair = i / 2;
      const float freq = (float)pos / powf(theta, (float)(2 * pair) / (float)rope_dim);
      const float sn = sinf(freq), cs = cosf(freq);
      const float a = h[i], b = h[i + 1];
      h[i] = a * cs - b * sn;
      h[i + 1] = a * sn + b * cs;
    }
  }
}

/* scalar softmax, crates/kernels/src/scalar.rs:125-141. */
void fo_softmax(float* x, uint64_t n) {
  float max = softmax_max(x, n);
  if (!isfinite(max)) {
    for (uint64_t i = 0; i < n; i++) x[i] = 0.0f;
    return;
  }
  float sum = 0.0f;
  for (uint64_t i = 0; i < n; i++) {
    float e = expf(x[i] - max);
    x[i] = e;
    sum += e;
  }
  float inv = 1.0f / sum;
  for (uint64_t i = 0; i < n; i++) x[i] *= inv;
}

/* ------------------------------------------------------------------------- */
/* Paged pool image operations                                                 */
/* ------------------------------------------------------------------------- */

/* Element index of (token off, dim d) inside an F16 tile of kind kv:
 * K [D/8][B][8] (16-byte runs of 8 dims, token-contiguous per run), V [D][B]. */
static uint64_t f16_index(const fo_layout* l, int kv, uint32_t off, uint32_t d) {
  if (kv) return (uint64_t)d * l->block_size + off;
  return ((uint64_t)(d / 8) * l->block_size + off) * 8 + d % 8;
}

/* Byte index of the int8 quant of (token off, dim d) inside a Q8_0 tile of kind
 * kv. The quants come in 16-token sub-tiles of 16*D bytes, each in 1 KiB runs;
 * with t = off % 16:
 *   K: d = c*32 + g*8 + e -> (c/2)*1024 + (g*16 + t)*16 + (c%2)*8 + e
 *   V: d = m*16 + j, t = q*4 + r -> (m/4)*1024 + (q*16 + j)*16 + (m%4)*4 + r
 * (needs D % 64 == 0 and B % 16 == 0). The f16 scales of both follow the quants
 * as [B][D/32]. */
static uint64_t q8_index(const fo_layout* l, int kv, uint32_t off, uint32_t d) {
  const uint64_t sub = (uint64_t)(off / 16) * 16 * l->head_dim;
  const uint32_t t = off % 16;
  if (kv) {
    const uint32_t m = d / 16, j = d % 16, q = t / 4, r = t % 4;
    return sub + (uint64_t)(m / 4) * 1024 + (uint64_t)(q * 16 + j) * 16 + (m % 4) * 4 + r;
  }
  const uint32_t c = d / 32, g = (d % 32) / 8, e = d % 8;
  return sub + (uint64_t)(c / 2) * 1024 + (uint64_t)(g * 16 + t) * 16 + (c % 2) * 8 + e;
}

/* Encode one row of D values into token `off` of a tile of kind kv (0 K, 1 V). */
static void encode_row(const fo_layout* l, int kv, uint8_t* tile, uint32_t off, const float* src) {
  uint32_t D = l->head_dim;
  if (l->dtype == 0) {
    memcpy(tile + (uint64_t)off * D * 4, src, (size_t)D * 4);
  } else if (l->dtype == 1) {
    uint16_t* dst = (uint16_t*)tile;
    for (uint32_t d = 0; d < D; d++) dst[f16_index(l, kv, off, d)] = fo_f32_to_f16(src[d], l->rounding);
  } else {
    uint8_t* sc = tile + (uint64_t)l->block_size * D + (uint64_t)off * (D / 32) * 2;
    for (uint32_t g = 0; g < D / 32; g++) {
      uint16_t s;
      int8_t q[32];
      fo_q8_quantize_block(src + g * 32, l->rounding, &s, q);
      for (uint32_t j = 0; j < 32; j++) tile[q8_index(l, kv, off, g * 32 + j)] = (uint8_t)q[j];
      sc[g * 2] = (uint8_t)(s & 0xff);
      sc[g * 2 + 1] = (uint8_t)(s >> 8);
    }
  }
}

/* Decode token `off` of a tile of kind kv to f32 (dtype.rs:135-154 / scalar.rs:261-279). */
static void decode_row(const fo_layout* l, int kv, const uint8_t* tile, uint32_t off, float* dst) {
  uint32_t D = l->head_dim;
  if (l->dtype == 0) {
    memcpy(dst, tile + (uint64_t)off * D * 4, (size_t)D * 4);
  } else if (l->dtype == 1) {
    const uint16_t* src = (const uint16_t*)tile;
    for (uint32_t d = 0; d < D; d++) dst[d] = fo_f16_to_f32(src[f16_index(l, kv, off, d)]);
  } else {
    const uint8_t* sc = tile + (uint64_t)l->block_size * D + (uint64_t)off * (D / 32) * 2;
    for (uint32_t g = 0; g < D / 32; g++) {
      float scale = fo_f16_to_f32((uint16_t)(sc[g * 2] | (sc[g * 2 + 1] << 8)));
      for (uint32_t j = 0; j < 32; j++)
        dst[g * 32 + j] = scale * (float)(int8_t)tile[q8_index(l, kv, off, g * 32 + j)];
    }
  }
}

/* Raw storage values of one token row (binary16 bits in dim order for F16); Q8_0 is
 * re-packed into Ferrum's 34-byte blocks. */
static void raw_row(const fo_layout* l, int kv, const uint8_t* tile, uint32_t off, uint8_t* dst) {
  uint32_t D = l->head_dim;
  if (l->dtype == 0) {
    memcpy(dst, tile + (uint64_t)off * D * 4, (size_t)D * 4);
  } else if (l->dtype == 1) {
    const uint16_t* src = (const uint16_t*)tile;
    for (uint32_t d = 0; d < D; d++) ((uint16_t*)dst)[d] = src[f16_index(l, kv, off, d)];
  } else {
    const uint8_t* sc = tile + (uint64_t)l->block_size * D + (uint64_t)off * (D / 32) * 2;
    for (uint32_t g = 0; g < D / 32; g++) {
      dst[g * 34] = sc[g * 2];
      dst[g * 34 + 1] = sc[g * 2 + 1];
      for (uint32_t j = 0; j < 32; j++) dst[g * 34 + 2 + j] = tile[q8_index(l, kv, off, g * 32 + j)];
    }
  }
}

static uint64_t raw_row_bytes(const fo_layout* l) {
  uint64_t D = l->head_dim;
  if (l->dtype == 0) return D * 4;
  if (l->dtype == 1) return D * 2;
  return D / 32 * 34;
}

/* Paged append: pool.rs:122-153 stores K then V for one position; here each
 * token goes to slot = block*B + offset of its slot mapping. */
uint64_t fo_append(const fo_layout* l, uint8_t* pool, uint32_t layer, const float* k,
                   const float* v, const int64_t* slots, uint64_t n_tokens) {
  uint64_t cap = l->num_blocks * l->block_size, skipped = 0;
  uint64_t row = (uint64_t)l->n_kv_heads * l->head_dim;
  for (uint64_t i = 0; i < n_tokens; i++) {
    int64_t s = slots[i];
    if (s < 0) continue;
    if ((uint64_t)s >= cap) { skipped++; continue; }
    uint64_t blk = (uint64_t)s / l->block_size;
    uint32_t off = (uint32_t)((uint64_t)s % l->block_size);
    for (uint32_t h = 0; h < l->n_kv_heads; h++) {
      encode_row(l, 0, pool + tile_offset(l, blk, layer, 0, h), off, k + i * row + h * l->head_dim);
      encode_row(l, 1, pool + tile_offset(l, blk, layer, 1, h), off, v + i * row + h * l->head_dim);
    }
  }
  return skipped;
}

static void gather_one(const fo_layout* l, const uint8_t* pool, uint32_t layer, uint64_t blk,
                       uint32_t off, int32_t format, uint8_t* ok, uint8_t* ov) {
  for (uint32_t h = 0; h < l->n_kv_heads; h++) {
    const uint8_t* tk = pool + tile_offset(l, blk, layer, 0, h);
    const uint8_t* tv = pool + tile_offset(l, blk, layer, 1, h);
    if (format == 0) {
      decode_row(l, 0, tk, off, (float*)ok + (uint64_t)h * l->head_dim);
      decode_row(l, 1, tv, off, (float*)ov + (uint64_t)h * l->head_dim);
    } else {
      raw_row(l, 0, tk, off, ok + h * raw_row_bytes(l));
      raw_row(l, 1, tv, off, ov + h * raw_row_bytes(l));
    }
  }
}

static uint64_t out_row_bytes(const fo_layout* l, int32_t format) {
  return format == 0 ? (uint64_t)l->n_kv_heads * l->head_dim * 4
                     : (uint64_t)l->n_kv_heads * raw_row_bytes(l);
}

/* Gather by slot: KvPool::k / KvPool::v (pool.rs:174-204) for many positions. */
void fo_gather_slots(const fo_layout* l, const uint8_t* pool, uint32_t layer,
                     const int64_t* slots, uint64_t n_tokens, int32_t format, void* out_k,
                     void* out_v) {
  uint64_t cap = l->num_blocks * l->block_size, rb = out_row_bytes(l, format);
  for (uint64_t i = 0; i < n_tokens; i++) {
    int64_t s = slots[i];
    if (s < 0 || (uint64_t)s >= cap) continue;
    gather_one(l, pool, layer, (uint64_t)s / l->block_size,
               (uint32_t)((uint64_t)s % l->block_size), format, (uint8_t*)out_k + i * rb,
               (uint8_t*)out_v + i * rb);
  }
}

void fo_gather_tables(const fo_layout* l, const uint8_t* pool, uint32_t layer,
                      const int32_t* block_tables, uint32_t max_blocks, const int32_t* ctx_lens,
                      const int64_t* out_offsets, uint32_t n_seqs, int32_t format,
                      void* out_k, void* out_v) {
  uint64_t rb = out_row_bytes(l, format);
  for (uint32_t s = 0; s < n_seqs; s++) {
    for (int32_t p = 0; p < ctx_lens[s]; p++) {
      int32_t blk = block_tables[(uint64_t)s * max_blocks + (uint32_t)p / l->block_size];
      if (blk < 0 || (uint64_t)blk >= l->num_blocks) continue;
      uint64_t row = (uint64_t)out_offsets[s] + (uint64_t)p;
      gather_one(l, pool, layer, (uint64_t)blk, (uint32_t)p % l->block_size, format,
                 (uint8_t*)out_k + row * rb, (uint8_t*)out_v + row * rb);
    }
  }
}

void fo_copy_blocks(const fo_layout* l, uint8_t* pool, const int64_t* pairs, uint64_t n_pairs) {
  uint64_t bb = fo_block_bytes(l);
  for (uint64_t i = 0; i < n_pairs; i++) {
    int64_t s = pairs[2 * i], d = pairs[2 * i + 1];
    if (s < 0 || d < 0 || (uint64_t)s >= l->num_blocks || (uint64_t)d >= l->num_blocks) continue;
    memmove(pool + (uint64_t)d * bb, pool + (uint64_t)s * bb, bb);
  }
}

/* Attention loop of Llama::forward_one_token, crates/model/src/llama.rs:220-247,
 * for every (sequence, query head): kv_h = h / g (:168,223); score = dot * scale
 * (:229-233, scale after the dot); softmax_inplace (:234); acc += w * v serially
 * over positions (:236-245). The reference reads its current token's K/V from
 * the work buffer; here every position, the newest included, comes from the pool
 * (for F32 storage the two are the same bits). */
static void attention_one(const fo_layout* l, const uint8_t* pool, uint32_t layer,
                          uint32_t n_heads, const float* q, float* out,
                          const int32_t* table, int32_t ctx, float scale, float* scores,
                          float* row) {
  uint32_t D = l->head_dim, g = n_heads / l->n_kv_heads;
  for (uint32_t h = 0; h < n_heads; h++) {
    uint32_t kvh = h / g;
    const float* qh = q + (uint64_t)h * D;
    float* oh = out + (uint64_t)h * D;
    for (uint32_t d = 0; d < D; d++) oh[d] = 0.0f;
    if (ctx <= 0) continue; /* empty: softmax_max is -inf, non-finite -> zeros */
    for (int32_t p = 0; p < ctx; p++) {
      int32_t blk = table[(uint32_t)p / l->block_size];
      decode_row(l, 0, pool + tile_offset(l, (uint64_t)blk, layer, 0, kvh),
                 (uint32_t)p % l->block_size, row);
      scores[p] = fo_dot(qh, row, D) * scale;
    }
    fo_softmax(scores, (uint64_t)ctx);
    for (int32_t p = 0; p < ctx; p++) {
      int32_t blk = table[(uint32_t)p / l->block_size];
      decode_row(l, 1, pool + tile_offset(l, (uint64_t)blk, layer, 1, kvh),
                 (uint32_t)p % l->block_size, row);
      float w = scores[p];
      for (uint32_t d = 0; d < D; d++) oh[d] += w * row[d];
    }
  }
}

void fo_attention(const fo_layout* l, const uint8_t* pool, uint32_t layer, uint32_t n_heads,
                  const float* q, float* out, const int32_t* block_tables, uint32_t max_blocks,
                  const int32_t* ctx_lens, uint32_t n_seqs, float scale) {
  int32_t maxctx = 1;
  for (uint32_t s = 0; s < n_seqs; s++)
    if (ctx_lens[s] > maxctx) maxctx = ctx_lens[s];
  float* scores = (float*)malloc((size_t)maxctx * 4);
  float* row = (float*)malloc((size_t)l->head_dim * 4);
  uint64_t qs = (uint64_t)n_heads * l->head_dim;
  for (uint32_t s = 0; s < n_seqs; s++)
    attention_one(l, pool, layer, n_heads, q + s * qs, out + s * qs,
                  block_tables + (uint64_t)s * max_blocks, ctx_lens[s], scale, scores, row);
  free(scores);
  free(row);
}

/* Prefill, Llama::forward llama.rs:363-378: tokens run one at a time, and the
 * token at position p attends to positions 0 ..= p (:220-247 with pos = p). The
 * chunk of sequence s is its last q_lens[s] positions, already in the pool; its
 * queries are rows q_offsets[s] .. of q and out. */
void fo_prefill_attention(const fo_layout* l, const uint8_t* pool, uint32_t layer,
                          uint32_t n_heads, const float* q, float* out,
                          const int32_t* block_tables, uint32_t max_blocks,
                          const int32_t* ctx_lens, const int32_t* q_lens,
                          const int64_t* q_offsets, uint32_t n_seqs, float scale) {
  int32_t maxctx = 1;
  for (uint32_t s = 0; s < n_seqs; s++)
    if (ctx_lens[s] > maxctx) maxctx = ctx_lens[s];
  float* scores = (float*)malloc((size_t)maxctx * 4);
  float* row = (float*)malloc((size_t)l->head_dim * 4);
  uint64_t qs = (uint64_t)n_heads * l->head_dim;
  for (uint32_t s = 0; s < n_seqs; s++) {
    int32_t p0 = ctx_lens[s] - q_lens[s];
    for (int32_t i = 0; i < q_lens[s]; i++) {
      uint64_t r = (uint64_t)q_offsets[s] + (uint64_t)i;
      attention_one(l, pool, layer, n_heads, q + r * qs, out + r * qs,
                    block_tables + (uint64_t)s * max_blocks, p0 + i + 1, scale, scores, row);
    }
  }
  free(scores);
  free(row);
}

/* ------------------------------------------------------------------------- */
/* AVX2 restatement (timed CPU baseline)                                       */
/* ------------------------------------------------------------------------- */

int32_t fo_avx2_available(void) {
  __builtin_cpu_init();
  return __builtin_cpu_supports("avx2") && __builtin_cpu_supports("fma") &&
         __builtin_cpu_supports("f16c");
}

int32_t fo_max_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}

#define AVX2_FN __attribute__((target("avx2,fma,f16c")))

AVX2_FN static inline int all_finite256(__m256 v) {
  return _mm256_movemask_ps(_mm256_cmp_ps(v, v, _CMP_ORD_Q)) == 0xff;
}

/* accumulate_products, crates/kernels/src/avx2.rs:194-230: 8 products per step,
 * added to the accumulator one lane at a time (bit-identical to the scalar dot). */
AVX2_FN float fo_avx2_dot(const float* a, const float* b, uint64_t n) {
  float acc = 0.0f;
  uint64_t i = 0;
  float prod[8];
  while (i + 8 <= n) {
    __m256 va = _mm256_loadu_ps(a + i), vb = _mm256_loadu_ps(b + i);
    if (all_finite256(va) && all_finite256(vb)) {
      _mm256_storeu_ps(prod, _mm256_mul_ps(va, vb));
      for (int k = 0; k < 8; k++) acc += prod[k];
    } else {
      for (int k = 0; k < 8; k++) acc += a[i + k] * b[i + k];
    }
    i += 8;
  }
  for (; i < n; i++) acc += a[i] * b[i];
  return acc;
}

/* exp256, crates/kernels/src/avx2.rs:366-418: the Cephes expf polynomial as
 * published in sse_mathfun (range reduction by ln2 split C1+C2, degree-5 poly). */
AVX2_FN static __m256 exp256(__m256 x) {
  const __m256 one = _mm256_set1_ps(1.0f);
  __m256 original = x;
  x = _mm256_min_ps(x, _mm256_set1_ps(88.3762626647949f));
  x = _mm256_max_ps(x, _mm256_set1_ps(-88.3762626647949f));
  __m256 n = _mm256_mul_ps(x, _mm256_set1_ps(1.44269504088896341f));
  n = _mm256_add_ps(n, _mm256_set1_ps(0.5f));
  __m256 nf = _mm256_floor_ps(n);
  __m256 adjust = _mm256_and_ps(_mm256_cmp_ps(nf, n, _CMP_GT_OQ), one);
  n = _mm256_sub_ps(nf, adjust);
  x = _mm256_fnmadd_ps(n, _mm256_set1_ps(0.693359375f), x);
  x = _mm256_fnmadd_ps(n, _mm256_set1_ps(-2.12194440e-4f), x);
  __m256 z = _mm256_mul_ps(x, x);
  __m256 y = _mm256_fmadd_ps(x, _mm256_set1_ps(1.9875691500e-4f), _mm256_set1_ps(1.3981999507e-3f));
  y = _mm256_fmadd_ps(y, x, _mm256_set1_ps(8.3334519073e-3f));
  y = _mm256_fmadd_ps(y, x, _mm256_set1_ps(4.1665795894e-2f));
  y = _mm256_fmadd_ps(y, x, _mm256_set1_ps(1.6666665459e-1f));
  y = _mm256_fmadd_ps(y, x, _mm256_set1_ps(5.0000001201e-1f));
  y = _mm256_fmadd_ps(y, z, x);
  y = _mm256_add_ps(y, one);
  __m256i imm = _mm256_cvttps_epi32(n);
  imm = _mm256_add_epi32(imm, _mm256_set1_epi32(0x7f));
  imm = _mm256_slli_epi32(imm, 23);
  y = _mm256_mul_ps(y, _mm256_castsi256_ps(imm));
  __m256 nan = _mm256_cmp_ps(original, original, _CMP_UNORD_Q);
  return _mm256_blendv_ps(y, original, nan);
}

/* softmax_avx2, crates/kernels/src/avx2.rs:457-492 (falls back to the scalar
 * softmax on a non-finite max or any NaN). */
AVX2_FN void fo_avx2_softmax(float* x, uint64_t n) {
  float max = softmax_max(x, n);
  int any_nan = 0;
  for (uint64_t i = 0; i < n; i++) any_nan |= isnan(x[i]);
  if (!isfinite(max) || any_nan) {
    fo_softmax(x, n);
    return;
  }
  __m256 mv = _mm256_set1_ps(max);
  float sum = 0.0f, ex[8];
  uint64_t i = 0;
  while (i + 8 <= n) {
    __m256 e = exp256(_mm256_sub_ps(_mm256_loadu_ps(x + i), mv));
    _mm256_storeu_ps(x + i, e);
    _mm256_storeu_ps(ex, e);
    for (int k = 0; k < 8; k++) sum += ex[k];
    i += 8;
  }
  for (; i < n; i++) {
    float e = expf(x[i] - max);
    x[i] = e;
    sum += e;
  }
  float inv = 1.0f / sum;
  __m256 iv = _mm256_set1_ps(inv);
  i = 0;
  while (i + 8 <= n) {
    _mm256_storeu_ps(x + i, _mm256_mul_ps(_mm256_loadu_ps(x + i), iv));
    i += 8;
  }
  for (; i < n; i++) x[i] *= inv;
}

/* Row decode with the x86 conversions the AVX2 backend would use: F16C for
 * binary16 (exact), and avx2.rs:660-694's i8 -> f32 * scale for Q8_0. */
AVX2_FN static void decode_row_avx2(const fo_layout* l, int kv, const uint8_t* tile, uint32_t off,
                                    float* dst) {
  uint32_t D = l->head_dim;
  if (l->dtype == 1 && D % 8 == 0 && kv == 0) {
    const uint16_t* src = (const uint16_t*)tile + (uint64_t)off * 8;  /* K [D/8][B][8] */
    for (uint32_t d = 0; d < D; d += 8)
      _mm256_storeu_ps(dst + d, _mm256_cvtph_ps(_mm_loadu_si128(
                                    (const __m128i*)(src + (uint64_t)(d / 8) * l->block_size * 8))));
  } else if (l->dtype == 8) {
    const uint8_t* sc = tile + (uint64_t)l->block_size * D + (uint64_t)off * (D / 32) * 2;
    for (uint32_t g = 0; g < D / 32; g++) {
      /* the block's 32 quants, gathered from the tile's operand order (q8_index) into
       * the contiguous block the reference's loop reads */
      uint8_t qs[32];
      for (uint32_t j = 0; j < 32; j++) qs[j] = tile[q8_index(l, kv, off, g * 32 + j)];
      float scale = fo_f16_to_f32((uint16_t)(sc[g * 2] | (sc[g * 2 + 1] << 8)));
      if (!isfinite(scale)) {
        for (int j = 0; j < 32; j++) dst[g * 32 + j] = scale * (float)(int8_t)qs[j];
        continue;
      }
      __m256 sv = _mm256_set1_ps(scale);
      for (int j = 0; j < 32; j += 8) {
        __m128i qv = _mm_loadl_epi64((const __m128i*)(qs + j));
        __m256 qf = _mm256_cvtepi32_ps(_mm256_cvtepi8_epi32(qv));
        _mm256_storeu_ps(dst + g * 32 + j, _mm256_mul_ps(qf, sv));
      }
    }
  } else {
    decode_row(l, kv, tile, off, dst);
  }
}

/* The same llama.rs:220-247 loop with the AVX2 kernels: per query head (no GQA
 * reuse), dot via fo_avx2_dot, softmax via fo_avx2_softmax, V accumulated 8 lanes
 * at a time with a separate multiply and add (what rustc emits for :240-242).
 * Parallelised over (sequence, head) pairs with OpenMP when n_threads > 1. */
AVX2_FN void fo_avx2_attention(const fo_layout* l, const uint8_t* pool, uint32_t layer,
                               uint32_t n_heads, const float* q, float* out,
                               const int32_t* block_tables, uint32_t max_blocks,
                               const int32_t* ctx_lens, uint32_t n_seqs, float scale,
                               int32_t n_threads) {
  uint32_t D = l->head_dim, g = n_heads / l->n_kv_heads;
  int32_t maxctx = 1;
  for (uint32_t s = 0; s < n_seqs; s++)
    if (ctx_lens[s] > maxctx) maxctx = ctx_lens[s];
  int64_t total = (int64_t)n_seqs * n_heads;
  if (n_threads < 1) n_threads = 1;
#pragma omp parallel num_threads(n_threads)
  {
    float* scores = (float*)malloc((size_t)maxctx * 4);
    float* row = (float*)aligned_alloc(32, ((size_t)D * 4 + 31) / 32 * 32);
#pragma omp for schedule(dynamic, 1)
    for (int64_t item = 0; item < total; item++) {
      uint32_t s = (uint32_t)(item / n_heads), h = (uint32_t)(item % n_heads);
      uint32_t kvh = h / g;
      const int32_t* table = block_tables + (uint64_t)s * max_blocks;
      const float* qh = q + ((uint64_t)s * n_heads + h) * D;
      float* oh = out + ((uint64_t)s * n_heads + h) * D;
      int32_t ctx = ctx_lens[s];
      for (uint32_t d = 0; d < D; d++) oh[d] = 0.0f;
      if (ctx <= 0) continue;
      for (int32_t p = 0; p < ctx; p++) {
        int32_t blk = table[(uint32_t)p / l->block_size];
        decode_row_avx2(l, 0, pool + tile_offset(l, (uint64_t)blk, layer, 0, kvh),
                        (uint32_t)p % l->block_size, row);
        scores[p] = fo_avx2_dot(qh, row, D) * scale;
      }
      fo_avx2_softmax(scores, (uint64_t)ctx);
      for (int32_t p = 0; p < ctx; p++) {
        int32_t blk = table[(uint32_t)p / l->block_size];
        decode_row_avx2(l, 1, pool + tile_offset(l, (uint64_t)blk, layer, 1, kvh),
                        (uint32_t)p % l->block_size, row);
        __m256 w = _mm256_set1_ps(scores[p]);
        uint32_t d = 0;
        for (; d + 8 <= D; d += 8)
          _mm256_storeu_ps(oh + d, _mm256_add_ps(_mm256_loadu_ps(oh + d),
                                                 _mm256_mul_ps(w, _mm256_loadu_ps(row + d))));
        for (; d < D; d++) oh[d] += scores[p] * row[d];
      }
    }
    free(scores);
    free(row);
  }
}

/* ------------------------------------------------------------------------- */
/* Dense revision-1 pool: crates/kvcache/src/pool.rs restated                  */
/* ------------------------------------------------------------------------- */

struct fo_dense {
  uint64_t n_layers, n_kv_heads, head_dim, max_seq_len, max_slots;
  uint8_t* free_;
  uint64_t* seq_len;
  uint64_t* layers_appended;
  float* storage;
  uint64_t storage_len;
};

#define CACHE(m) (*msg = "cache: " m, 1)

static int mul_ovf(uint64_t a, uint64_t b, uint64_t* r) { return __builtin_mul_overflow(a, b, r); }

/* PreallocatedKvPool::new, pool.rs:21-46. */
int32_t fo_dense_new(uint64_t n_layers, uint64_t n_kv_heads, uint64_t head_dim,
                     uint64_t max_seq_len, uint64_t max_slots, fo_dense** out,
                     const char** msg) {
  *out = NULL;
  if (!n_layers || !n_kv_heads || !head_dim || !max_seq_len || !max_slots)
    return CACHE("kv pool dimension is zero");
  uint64_t block, per_slot, total;
  if (mul_ovf(n_kv_heads, head_dim, &block) || mul_ovf(block, 2, &block))
    return CACHE("kv pool size overflow");
  if (mul_ovf(n_layers, max_seq_len, &per_slot) || mul_ovf(per_slot, block, &per_slot))
    return CACHE("kv pool size overflow");
  if (mul_ovf(per_slot, max_slots, &total)) return CACHE("kv pool size overflow");
  fo_dense* p = (fo_dense*)calloc(1, sizeof(fo_dense));
  p->n_layers = n_layers; p->n_kv_heads = n_kv_heads; p->head_dim = head_dim;
  p->max_seq_len = max_seq_len; p->max_slots = max_slots;
  p->free_ = (uint8_t*)malloc(max_slots);
  memset(p->free_, 1, max_slots);
  p->seq_len = (uint64_t*)calloc(max_slots, 8);
  p->layers_appended = (uint64_t*)calloc(max_slots, 8);
  p->storage = (float*)calloc(total ? total : 1, 4);
  p->storage_len = total;
  *out = p;
  *msg = "";
  return 0;
}

void fo_dense_destroy(fo_dense* p) {
  if (!p) return;
  free(p->free_); free(p->seq_len); free(p->layers_appended); free(p->storage); free(p);
}

uint64_t fo_dense_storage_len(const fo_dense* p) { return p->storage_len; }

static uint64_t kv_block_len(const fo_dense* p) { return p->n_kv_heads * p->head_dim * 2; }

/* block_offset, pool.rs:52-71 (sizes here never overflow once `new` succeeded). */
static uint64_t block_offset(const fo_dense* p, uint64_t slot, uint64_t layer, uint64_t pos) {
  uint64_t block = kv_block_len(p);
  return slot * (p->n_layers * p->max_seq_len * block) + layer * p->max_seq_len * block +
         pos * block;
}

/* alloc, pool.rs:83-101: first free slot, zero-filled. */
int32_t fo_dense_alloc(fo_dense* p, uint32_t* slot, const char** msg) {
  for (uint64_t i = 0; i < p->max_slots; i++) {
    if (p->free_[i]) {
      p->free_[i] = 0;
      p->seq_len[i] = 0;
      p->layers_appended[i] = 0;
      uint64_t per_slot = p->n_layers * p->max_seq_len * kv_block_len(p);
      memset(p->storage + i * per_slot, 0, per_slot * 4);
      *slot = (uint32_t)i;
      *msg = "";
      return 0;
    }
  }
  *msg = "no free kv slots";
  return 2;
}

/* free, pool.rs:103-112. */
int32_t fo_dense_free(fo_dense* p, uint32_t slot, const char** msg) {
  if (slot >= p->max_slots || p->free_[slot]) return CACHE("free of unallocated slot");
  p->free_[slot] = 1;
  p->seq_len[slot] = 0;
  p->layers_appended[slot] = 0;
  *msg = "";
  return 0;
}

/* seq_len, pool.rs:114-120. */
int32_t fo_dense_seq_len(const fo_dense* p, uint32_t slot, uint64_t* out, const char** msg) {
  if (slot >= p->max_slots) return CACHE("unknown slot");
  *out = p->seq_len[slot];
  *msg = "";
  return 0;
}

/* append_layer, pool.rs:122-153. The reference indexes `free[index]` unchecked
 * and would panic on an out-of-range slot; that case is "unknown slot" here. */
int32_t fo_dense_append_layer(fo_dense* p, uint32_t slot, uint64_t layer, const float* k,
                              uint64_t k_len, const float* v, uint64_t v_len,
                              const char** msg) {
  if (slot >= p->max_slots) return CACHE("unknown slot");
  if (p->free_[slot]) return CACHE("append on free slot");
  if (layer >= p->n_layers) return CACHE("layer out of range");
  uint64_t expected = p->n_kv_heads * p->head_dim;
  if (k_len != expected || v_len != expected) return CACHE("kv vector length mismatch");
  uint64_t pos = p->seq_len[slot];
  if (pos >= p->max_seq_len) return CACHE("sequence length exceeds max");
  if (p->layers_appended[slot] != layer) return CACHE("layers must append in order");
  uint64_t off = block_offset(p, slot, layer, pos);
  memcpy(p->storage + off, k, expected * 4);
  memcpy(p->storage + off + expected, v, expected * 4);
  p->layers_appended[slot] += 1;
  *msg = "";
  return 0;
}

/* commit_token, pool.rs:155-172. */
int32_t fo_dense_commit_token(fo_dense* p, uint32_t slot, const char** msg) {
  if (slot >= p->max_slots) return CACHE("unknown slot");
  if (p->free_[slot]) return CACHE("commit on free slot");
  if (p->layers_appended[slot] != p->n_layers) return CACHE("not every layer appended");
  uint64_t next = p->seq_len[slot] + 1;
  if (next > p->max_seq_len) return CACHE("sequence length exceeds max");
  p->seq_len[slot] = next;
  p->layers_appended[slot] = 0;
  *msg = "";
  return 0;
}

/* k / v, pool.rs:174-204. */
static int32_t dense_read(const fo_dense* p, uint32_t slot, uint64_t layer, uint64_t pos,
                          float* out, int which, const char** msg) {
  if (slot >= p->max_slots) return CACHE("unknown slot");
  if (p->free_[slot]) return CACHE("read on free slot");
  if (pos >= p->seq_len[slot]) return CACHE("position not yet committed");
  if (layer >= p->n_layers) return CACHE("layer out of range");
  uint64_t n = p->n_kv_heads * p->head_dim;
  uint64_t off = block_offset(p, slot, layer, pos) + (which ? n : 0);
  memcpy(out, p->storage + off, n * 4);
  *msg = "";
  return 0;
}

int32_t fo_dense_k(const fo_dense* p, uint32_t slot, uint64_t layer, uint64_t pos, float* out,
                   const char** msg) {
  return dense_read(p, slot, layer, pos, out, 0, msg);
}

int32_t fo_dense_v(const fo_dense* p, uint32_t slot, uint64_t layer, uint64_t pos, float* out,
                   const char** msg) {
  return dense_read(p, slot, layer, pos, out, 1, msg);
}

/* abandon_partial, pool.rs:207-216. */
int32_t fo_dense_abandon_partial(fo_dense* p, uint32_t slot, const char** msg) {
  if (slot >= p->max_slots || p->free_[slot]) return CACHE("abandon on free slot");
  p->layers_appended[slot] = 0;
  *msg = "";
  return 0;
}

/* uncommit_token, pool.rs:218-231. */
int32_t fo_dense_uncommit_token(fo_dense* p, uint32_t slot, const char** msg) {
  if (slot >= p->max_slots || p->free_[slot]) return CACHE("uncommit on free slot");
  if (p->seq_len[slot] == 0) return CACHE("nothing to uncommit");
  p->seq_len[slot] -= 1;
  p->layers_appended[slot] = 0;
  *msg = "";
  return 0;
}

/* ------------------------------------------------------------------------- */
/* Exhaustive self-checks of the binary16 encoder                              */
/* ------------------------------------------------------------------------- */

/* Nearest binary16 to x found by f64 arithmetic on the value grid (no bit
 * manipulation): grid spacing 2^(e-10) in binade [2^e, 2^(e+1)), 2^-24 below
 * 2^-14, Inf from 65520 up. Returns the expected value (signed). */
static double f64_nearest_half(float xf, int ties_even) {
  double x = (double)xf, a = fabs(x);
  if (a >= 65520.0) return copysign(INFINITY, x);
  double ulp;
  if (a < 0x1p-14) {
    ulp = 0x1p-24;
  } else {
    int e;
    frexp(a, &e); /* a = m * 2^e, m in [0.5, 1) */
    ulp = ldexp(1.0, e - 11);
  }
  double lo = floor(a / ulp) * ulp, hi = lo + ulp;
  double dl = a - lo, dh = hi - a, r;
  if (dl < dh) r = lo;
  else if (dh < dl) r = hi;
  else if (!ties_even) r = hi;
  else r = (fmod(lo / ulp, 2.0) == 0.0) ? lo : hi;
  return copysign(r, x);
}

AVX2_FN static uint16_t f16c_rne(float x) {
  __m128i h = _mm_cvtps_ph(_mm_set_ss(x), _MM_FROUND_TO_NEAREST_INT | _MM_FROUND_NO_EXC);
  return (uint16_t)_mm_extract_epi16(h, 0);
}

uint64_t fo_selftest_f16(int32_t which, uint32_t stride, uint32_t* first_bad) {
  uint64_t bad = 0;
  uint32_t first = 0;
  int have_first = 0;
  if (stride == 0) stride = 1;
  int64_t n = (int64_t)((0x100000000ull + stride - 1) / stride);
#pragma omp parallel for schedule(static) reduction(+ : bad)
  for (int64_t i = 0; i < n; i++) {
    uint32_t u = (uint32_t)((uint64_t)i * stride);
    float x = u2f(u);
    int ok;
    if (isnan(x)) {
      /* NaN rule: sign kept, exponent all ones, payload = top 10 bits, non-zero. */
      int32_t r = (which == 1) ? 1 : 0;
      uint16_t h = fo_f32_to_f16(x, r);
      uint32_t hf = (u & 0x7fffffu) >> 13;
      uint16_t want = (uint16_t)(((u >> 16) & 0x8000u) | 0x7c00u | hf | (hf == 0));
      ok = (h == want);
    } else if (which == 0) {
      ok = (fo_f32_to_f16(x, 0) == f16c_rne(x));
    } else {
      int ties_even = (which == 2);
      uint16_t h = fo_f32_to_f16(x, ties_even ? 0 : 1);
      double want = f64_nearest_half(x, ties_even);
      double got = (double)fo_f16_to_f32(h);
      ok = (got == want) && (signbit(got) == signbit(want));
    }
    if (!ok) {
      bad++;
#pragma omp critical
      {
        if (!have_first || u < first) { first = u; have_first = 1; }
      }
    }
  }
  if (first_bad) *first_bad = first;
  return bad;
}
