/*
 * CPU oracle: plain-C restatement of the reference numerics for the
 * quantized-linear path. TEST INFRASTRUCTURE ONLY (see oracle.h).
 *
 * Build: oracle/Makefile (gcc -O2 -ffp-contract=off, no fast-math).
 *
 * How each part is pinned (tests/test_oracle_*.py):
 *  - f16 conversions: exhaustively against numpy's IEEE binary16 for all 65536
 *    half values and for f32 inputs around every rounding boundary; plus the
 *    reference vector 0.5 -> 0x3800 (format gguf/tests.rs:191).
 *  - dequantizers / per-element values: reference known answers
 *    (backends/cpu/src/tests.rs:17-133), closed forms of Appendix-style block
 *    formulas evaluated independently in numpy, and wire round trips
 *    (format gguf/tests.rs:163-231).
 *  - quantizers: the reference's exhaustive nearest-codebook oracle
 *    (quant schemes/k_grid_tests.rs:35-145) restated as a brute-force check,
 *    d == f16(d), rejection of f32::MAX (:148-155), sub-grid loss (:158-179),
 *    subnormal d (:182-196), round-trip bounds (quant/src/lib.rs tests).
 *  - matmuls: f64 brute force over the dequantized weights with the reference
 *    bound |a-e| < 1e-4 + 1e-5|e| (runtime/src/linear/tests.rs:137-155),
 *    output-rows == row-major bit equality (cpu tests.rs:63-114), threaded ==
 *    scalar (tests.rs:156-177, 259-278), the known answers 64.0 and 0.0, and an
 *    independent sequential-f32 numpy restatement on small inputs.
 *  - cpu-simd variants: within 1e-4 of scalar (cpu tests.rs:209-257). The
 *    horizontal-sum order of _mm512_reduce_add_ps as Rust compiles it is
 *    parity unpinned (only a tolerance is checked, as in the reference).
 */
#include "oracle.h"

#include <math.h>
#include <pthread.h>
#include <string.h>

#if defined(__x86_64__)
#include <immintrin.h>
#endif

static const float F32_EPSILON = 1.1920929e-7f; /* f32::EPSILON */

size_t qo_block_bytes(int qtype) {
  switch (qtype) {
    case QO_F32: return 4;
    case QO_Q8_0: return sizeof(qo_q8_0_block);
    case QO_Q4_0: return sizeof(qo_q4_0_block);
    case QO_Q4_K: return sizeof(qo_q4_k_block);
    case QO_Q5_K: return sizeof(qo_q5_k_block);
    case QO_Q6_K: return sizeof(qo_q6_k_block);
    default: return 0;
  }
}

/* format gguf/encoding.rs:126-195 */
size_t qo_wire_bytes(int qtype) {
  switch (qtype) {
    case QO_F32: return 4;
    case QO_Q8_0: return 34;
    case QO_Q4_0: return 18;
    case QO_Q4_K: return 144;
    case QO_Q5_K: return 176;
    case QO_Q6_K: return 210;
    default: return 0;
  }
}

/* core quantized/mod.rs:8-12 */
size_t qo_block_elems(int qtype) {
  switch (qtype) {
    case QO_F32: return 1;
    case QO_Q8_0:
    case QO_Q4_0: return 32;
    case QO_Q4_K:
    case QO_Q5_K:
    case QO_Q6_K: return 256;
    default: return 0;
  }
}

/* ------------------------------------------------------------------ f16 */

static uint32_t f32_bits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static float bits_f32(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* IEEE-754 binary32 -> binary16, round to nearest, ties to even; overflow to
 * infinity; NaN stays NaN (quiet). This is the conversion `half` 2.7.1 performs
 * for f16::from_f32 (the reference's only f32->f16 path). */
uint16_t qo_f32_to_f16(float value) {
  uint32_t x = f32_bits(value);
  uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
  uint32_t exp = (x >> 23) & 0xFFu;
  uint32_t man = x & 0x7FFFFFu;
  if (exp == 0xFFu) {
    if (man != 0) return (uint16_t)(sign | 0x7E00u | (man >> 13));
    return (uint16_t)(sign | 0x7C00u);
  }
  if (exp == 0) return sign; /* f32 zero or subnormal: far below half's range */
  int e = (int)exp - 127 + 15;
  if (e >= 31) return (uint16_t)(sign | 0x7C00u);
  if (e >= 1) {
    uint32_t h = ((uint32_t)e << 10) | (man >> 13);
    uint32_t rem = man & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h += 1; /* carry may reach inf: correct */
    return (uint16_t)(sign | h);
  }
  /* Result is subnormal (or rounds up to the smallest normal). The value is
   * full * 2^(exp-150) with full a 24-bit significand; in units of 2^-24 that
   * is full >> (126 - exp). */
  uint32_t full = man | 0x800000u;
  uint32_t shift = 126u - exp; /* >= 14 */
  if (shift > 24) return sign;  /* < half of the smallest subnormal */
  uint32_t q = full >> shift;
  uint32_t rem = full & ((1u << shift) - 1u);
  uint32_t halfway = 1u << (shift - 1u);
  if (rem > halfway || (rem == halfway && (q & 1u))) q += 1;
  return (uint16_t)(sign | q);
}

float qo_f16_to_f32(uint16_t bits) {
  uint32_t sign = ((uint32_t)bits & 0x8000u) << 16;
  uint32_t e = ((uint32_t)bits >> 10) & 0x1Fu;
  uint32_t m = (uint32_t)bits & 0x3FFu;
  if (e == 0) {
    if (m == 0) return bits_f32(sign);
    /* subnormal: m * 2^-24, exact in binary32 */
    float v = (float)m * 5.9604644775390625e-8f;
    return sign ? -v : v;
  }
  if (e == 31) return bits_f32(sign | 0x7F800000u | (m << 13));
  return bits_f32(sign | ((e - 15 + 127) << 23) | (m << 13));
}

void qo_f32_to_f16_array(const float *in, size_t n, uint16_t *out) {
  for (size_t i = 0; i < n; ++i) out[i] = qo_f32_to_f16(in[i]);
}

void qo_f16_to_f32_array(const uint16_t *in, size_t n, float *out) {
  for (size_t i = 0; i < n; ++i) out[i] = qo_f16_to_f32(in[i]);
}

static float f16_round(float v) { return qo_f16_to_f32(qo_f32_to_f16(v)); }

/* quant schemes/mod.rs:27-40 */
int qo_stored_f16_scale(float value, float *out) {
  float stored = f16_round(value);
  if (!isfinite(stored)) return QO_INVALID;
  if (stored == 0.0f && value > 0.0f) stored = qo_f16_to_f32(1);
  *out = stored;
  return QO_OK;
}

/* quant schemes/mod.rs:18-25 */
static int validate_finite(const float *values, size_t n) {
  for (size_t i = 0; i < n; ++i)
    if (!isfinite(values[i])) return QO_INVALID;
  return QO_OK;
}

/* Rust f32::clamp / f64::clamp on finite inputs */
static float clampf_(float v, float lo, float hi) { return v < lo ? lo : (v > hi ? hi : v); }
static double clampd_(double v, double lo, double hi) { return v < lo ? lo : (v > hi ? hi : v); }

/* ------------------------------------------------------------ quantizers */

/* quant schemes/q8.rs:8-31 */
int qo_quantize_q8_0(const float *values, size_t n, qo_q8_0_block *out) {
  if (validate_finite(values, n) != QO_OK || n % 32 != 0) return QO_INVALID;
  for (size_t b = 0; b < n / 32; ++b) {
    const float *chunk = values + 32 * b;
    float maximum = 0.0f;
    for (int i = 0; i < 32; ++i) maximum = fmaxf(maximum, fabsf(chunk[i]));
    float scale = maximum == 0.0f ? 1.0f : maximum / 127.0f;
    out[b].scale = scale;
    for (int i = 0; i < 32; ++i) {
      float rounded = clampf_(roundf(chunk[i] / scale), -127.0f, 127.0f);
      out[b].values[i] = (int8_t)rounded;
    }
  }
  return QO_OK;
}

/* quant schemes/q4.rs:8-33 */
int qo_quantize_q4_0(const float *values, size_t n, qo_q4_0_block *out) {
  if (validate_finite(values, n) != QO_OK || n % 32 != 0) return QO_INVALID;
  for (size_t b = 0; b < n / 32; ++b) {
    const float *chunk = values + 32 * b;
    float maximum = 0.0f;
    for (int i = 0; i < 32; ++i) maximum = fmaxf(maximum, fabsf(chunk[i]));
    float scale = maximum == 0.0f ? 1.0f : maximum / 7.0f;
    out[b].scale = scale;
    for (int i = 0; i < 32; ++i) {
      int code = (int)clampf_(roundf(chunk[i] / scale), -8.0f, 7.0f) + 8;
      out[b].values[i] = (uint8_t)code;
    }
  }
  return QO_OK;
}

/* Shared first stage of the Q4_K / Q5_K quantizers: per-sub-block affine range,
 * then the two-level scale quantization (q4_k.rs:21-45, q5_k.rs:21-45). */
static int kquant_affine_scales(const float *chunk, float levels, float *d_out, float *dmin_out,
                                uint8_t sv[8], uint8_t mv[8]) {
  float scales[8], mins[8];
  for (int sub = 0; sub < 8; ++sub) {
    const float *v = chunk + 32 * sub;
    float mn = INFINITY, mx = -INFINITY;
    for (int i = 0; i < 32; ++i) { mn = fminf(mn, v[i]); mx = fmaxf(mx, v[i]); }
    mn = fminf(mn, 0.0f);
    float scale = fmaxf((mx - mn) / levels, F32_EPSILON);
    scales[sub] = scale;
    mins[sub] = -mn;
  }
  float scale_max = 0.0f, min_max = 0.0f;
  for (int sub = 0; sub < 8; ++sub) { scale_max = fmaxf(scale_max, scales[sub]); }
  scale_max = fmaxf(scale_max, F32_EPSILON);
  for (int sub = 0; sub < 8; ++sub) { min_max = fmaxf(min_max, mins[sub]); }
  float d, dmin;
  if (qo_stored_f16_scale(scale_max / 63.0f, &d) != QO_OK) return QO_INVALID;
  if (qo_stored_f16_scale(min_max == 0.0f ? 1.0f : min_max / 63.0f, &dmin) != QO_OK)
    return QO_INVALID;
  for (int sub = 0; sub < 8; ++sub) {
    sv[sub] = d == 0.0f ? 0 : (uint8_t)clampf_(roundf(scales[sub] / d), 1.0f, 63.0f);
    mv[sub] = dmin == 0.0f ? 0 : (uint8_t)clampf_(roundf(mins[sub] / dmin), 0.0f, 63.0f);
  }
  *d_out = d;
  *dmin_out = dmin;
  return QO_OK;
}

/* 6-bit scale/min packing (q4_k.rs:60-68, q5_k.rs:58-65) */
static void kquant_pack_scales(const uint8_t sv[8], const uint8_t mv[8], uint8_t packed[12]) {
  for (int i = 0; i < 4; ++i) { packed[i] = sv[i]; packed[4 + i] = mv[i]; }
  for (int i = 0; i < 4; ++i) {
    packed[8 + i] = (uint8_t)((sv[4 + i] & 0x0F) | ((mv[4 + i] & 0x0F) << 4));
    packed[i] |= (uint8_t)((sv[4 + i] >> 4) << 6);
    packed[4 + i] |= (uint8_t)((mv[4 + i] >> 4) << 6);
  }
}

/* Codes chosen in f64 after both scale levels (q4_k.rs:46-59, q5_k.rs:46-57) */
static void kquant_codes(const float *chunk, float d, float dmin, const uint8_t sv[8],
                         const uint8_t mv[8], double maxcode, uint8_t q[256]) {
  for (int index = 0; index < 256; ++index) {
    int sub = index / 32;
    double scale = (double)d * (double)sv[sub];
    double minimum = (double)dmin * (double)mv[sub];
    q[index] = scale == 0.0 ? 0
        : (uint8_t)clampd_(round(((double)chunk[index] + minimum) / scale), 0.0, maxcode);
  }
}

/* quant schemes/q4_k.rs:8-88 */
int qo_quantize_q4_k(const float *values, size_t n, qo_q4_k_block *out) {
  if (validate_finite(values, n) != QO_OK || n % 256 != 0) return QO_INVALID;
  for (size_t b = 0; b < n / 256; ++b) {
    const float *chunk = values + 256 * b;
    float d, dmin;
    uint8_t sv[8], mv[8], q[256];
    if (kquant_affine_scales(chunk, 15.0f, &d, &dmin, sv, mv) != QO_OK) return QO_INVALID;
    kquant_codes(chunk, d, dmin, sv, mv, 15.0, q);
    qo_q4_k_block *blk = &out[b];
    blk->scale = d;
    blk->min_scale = dmin;
    kquant_pack_scales(sv, mv, blk->scales);
    for (int g = 0; g < 4; ++g)
      for (int i = 0; i < 32; ++i)
        blk->values[g * 32 + i] = (uint8_t)(q[g * 64 + i] | (q[g * 64 + 32 + i] << 4));
  }
  return QO_OK;
}

/* quant schemes/q5_k.rs:8-94 */
int qo_quantize_q5_k(const float *values, size_t n, qo_q5_k_block *out) {
  if (validate_finite(values, n) != QO_OK || n % 256 != 0) return QO_INVALID;
  for (size_t b = 0; b < n / 256; ++b) {
    const float *chunk = values + 256 * b;
    float d, dmin;
    uint8_t sv[8], mv[8], q[256];
    if (kquant_affine_scales(chunk, 31.0f, &d, &dmin, sv, mv) != QO_OK) return QO_INVALID;
    kquant_codes(chunk, d, dmin, sv, mv, 31.0, q);
    qo_q5_k_block *blk = &out[b];
    blk->scale = d;
    blk->min_scale = dmin;
    kquant_pack_scales(sv, mv, blk->scales);
    memset(blk->high_bits, 0, sizeof blk->high_bits);
    for (int g = 0; g < 4; ++g) {
      for (int i = 0; i < 32; ++i) {
        uint8_t first = q[g * 64 + i], second = q[g * 64 + 32 + i];
        blk->values[g * 32 + i] = (uint8_t)((first & 0x0F) | ((second & 0x0F) << 4));
        if (first & 0x10) blk->high_bits[i] |= (uint8_t)(1u << (2 * g));
        if (second & 0x10) blk->high_bits[i] |= (uint8_t)(1u << (2 * g + 1));
      }
    }
  }
  return QO_OK;
}

/* quant schemes/q6_k.rs:8-72 */
int qo_quantize_q6_k(const float *values, size_t n, qo_q6_k_block *out) {
  if (validate_finite(values, n) != QO_OK || n % 256 != 0) return QO_INVALID;
  for (size_t b = 0; b < n / 256; ++b) {
    const float *chunk = values + 256 * b;
    float scales_f[16];
    for (int sub = 0; sub < 16; ++sub) {
      float max_abs = 0.0f;
      for (int i = 0; i < 16; ++i) max_abs = fmaxf(max_abs, fabsf(chunk[16 * sub + i]));
      scales_f[sub] = fmaxf(max_abs / 31.0f, F32_EPSILON);
    }
    float max_scale = 0.0f;
    for (int sub = 0; sub < 16; ++sub) max_scale = fmaxf(max_scale, scales_f[sub]);
    max_scale = fmaxf(max_scale, F32_EPSILON);
    float d;
    if (qo_stored_f16_scale(max_scale / 127.0f, &d) != QO_OK) return QO_INVALID;
    qo_q6_k_block *blk = &out[b];
    for (int sub = 0; sub < 16; ++sub)
      blk->scales[sub] = d == 0.0f ? 0 : (int8_t)clampf_(roundf(scales_f[sub] / d), 1.0f, 127.0f);
    uint8_t q[256];
    for (int index = 0; index < 256; ++index) {
      double scale = (double)d * (double)blk->scales[index / 16];
      int sgn = scale == 0.0 ? 0 : (int)clampd_(round((double)chunk[index] / scale), -32.0, 31.0);
      q[index] = (uint8_t)(sgn + 32);
    }
    blk->scale = d;
    for (int ip = 0; ip < 2; ++ip) {
      for (int il = 0; il < 32; ++il) {
        uint8_t q0 = q[ip * 128 + il], q1 = q[ip * 128 + 32 + il];
        uint8_t q2 = q[ip * 128 + 64 + il], q3 = q[ip * 128 + 96 + il];
        blk->low_bits[ip * 64 + il] = (uint8_t)((q0 & 0x0F) | ((q2 & 0x0F) << 4));
        blk->low_bits[ip * 64 + 32 + il] = (uint8_t)((q1 & 0x0F) | ((q3 & 0x0F) << 4));
        blk->high_bits[ip * 32 + il] = (uint8_t)(((q0 >> 4) & 3) | (((q1 >> 4) & 3) << 2) |
                                                 (((q2 >> 4) & 3) << 4) | (((q3 >> 4) & 3) << 6));
      }
    }
  }
  return QO_OK;
}

/* quant providers/storage.rs:10-18 */
static int storage_round(float *v) {
  float rounded = f16_round(*v);
  if (!isfinite(*v) || !isfinite(rounded)) return QO_INVALID;
  *v = rounded;
  return QO_OK;
}

/* quant providers/storage.rs:28-87: scales/mins round to f16 (including
 * underflow to zero); integer codes untouched. */
int qo_storage_precision(int qtype, void *blocks, size_t count) {
  for (size_t i = 0; i < count; ++i) {
    switch (qtype) {
      case QO_Q8_0:
        if (storage_round(&((qo_q8_0_block *)blocks)[i].scale)) return QO_INVALID;
        break;
      case QO_Q4_0:
        if (storage_round(&((qo_q4_0_block *)blocks)[i].scale)) return QO_INVALID;
        break;
      case QO_Q4_K:
        if (storage_round(&((qo_q4_k_block *)blocks)[i].scale) ||
            storage_round(&((qo_q4_k_block *)blocks)[i].min_scale))
          return QO_INVALID;
        break;
      case QO_Q5_K:
        if (storage_round(&((qo_q5_k_block *)blocks)[i].scale) ||
            storage_round(&((qo_q5_k_block *)blocks)[i].min_scale))
          return QO_INVALID;
        break;
      case QO_Q6_K:
        if (storage_round(&((qo_q6_k_block *)blocks)[i].scale)) return QO_INVALID;
        break;
      default: return QO_INVALID;
    }
  }
  return QO_OK;
}

/* core quantized/q8.rs:20-40, q4.rs:22-51 and :87-120, k.rs:23-41 and :70-85 */
int qo_validate_blocks(int qtype, const void *blocks, size_t count, size_t elements) {
  size_t bs = qo_block_elems(qtype);
  if (bs == 0 || qtype == QO_F32 || elements == 0) return QO_INVALID;
  if (elements % bs != 0 || count * bs != elements) return QO_INVALID;
  for (size_t i = 0; i < count; ++i) {
    switch (qtype) {
      case QO_Q8_0:
        if (!isfinite(((const qo_q8_0_block *)blocks)[i].scale)) return QO_INVALID;
        break;
      case QO_Q4_0: {
        const qo_q4_0_block *b = &((const qo_q4_0_block *)blocks)[i];
        for (int j = 0; j < 32; ++j)
          if (b->values[j] > 15) return QO_INVALID;
        if (!isfinite(b->scale)) return QO_INVALID;
        break;
      }
      case QO_Q4_K: {
        const qo_q4_k_block *b = &((const qo_q4_k_block *)blocks)[i];
        if (!isfinite(b->scale) || !isfinite(b->min_scale)) return QO_INVALID;
        break;
      }
      case QO_Q5_K: {
        const qo_q5_k_block *b = &((const qo_q5_k_block *)blocks)[i];
        if (!isfinite(b->scale) || !isfinite(b->min_scale)) return QO_INVALID;
        break;
      }
      case QO_Q6_K:
        if (!isfinite(((const qo_q6_k_block *)blocks)[i].scale)) return QO_INVALID;
        break;
    }
  }
  return QO_OK;
}

/* -------------------------------------------- per-element reference values */

/* 6-bit sub-block scale and min of a Q4_K/Q5_K block (matmul.rs:192-201) */
static void kquant_scale_min(const uint8_t s[12], int sub, uint8_t *sc, uint8_t *mn) {
  if (sub < 4) {
    *sc = s[sub] & 0x3F;
    *mn = s[4 + sub] & 0x3F;
  } else {
    int i = sub - 4;
    *sc = (uint8_t)((s[8 + i] & 0x0F) | ((s[i] >> 6) << 4));
    *mn = (uint8_t)((s[8 + i] >> 4) | ((s[4 + i] >> 6) << 4));
  }
}

static float value_q8_0(const qo_q8_0_block *b, size_t local) {
  return b->scale * (float)b->values[local]; /* matmul.rs:167 */
}
static float value_q4_0(const qo_q4_0_block *b, size_t local) {
  return b->scale * ((float)b->values[local] - 8.0f); /* matmul.rs:179 */
}
static float value_q4_k(const qo_q4_k_block *b, size_t local) { /* matmul.rs:182-215 */
  uint8_t sc, mn;
  kquant_scale_min(b->scales, (int)(local / 32), &sc, &mn);
  size_t group = local / 64, within = local % 64;
  uint8_t packed = b->values[group * 32 + within % 32];
  uint8_t q = within < 32 ? (packed & 0x0F) : (packed >> 4);
  return b->scale * (float)sc * (float)q - b->min_scale * (float)mn;
}
static float value_q5_k(const qo_q5_k_block *b, size_t local) { /* matmul.rs:217-258 */
  uint8_t sc, mn;
  kquant_scale_min(b->scales, (int)(local / 32), &sc, &mn);
  size_t group = local / 64, within = local % 64;
  uint8_t packed = b->values[group * 32 + within % 32];
  uint8_t q = within < 32 ? (packed & 0x0F) : (packed >> 4);
  unsigned bit = within < 32 ? (unsigned)(2 * group) : (unsigned)(2 * group + 1);
  if (b->high_bits[within % 32] & (1u << bit)) q = (uint8_t)(q + 16);
  return b->scale * (float)sc * (float)q - b->min_scale * (float)mn;
}
static float value_q6_k(const qo_q6_k_block *b, size_t local) { /* matmul.rs:260-280 */
  size_t ip = local / 128, within = local % 128, chunk = within / 32, il = within % 32;
  uint8_t packed = b->low_bits[ip * 64 + (chunk % 2 == 0 ? il : 32 + il)];
  uint8_t low = chunk < 2 ? (packed & 0x0F) : (packed >> 4);
  uint8_t high = b->high_bits[ip * 32 + il];
  uint8_t q = (uint8_t)(low | (((high >> (chunk * 2)) & 3) << 4));
  return b->scale * (float)b->scales[local / 16] * (float)((int)q - 32);
}

float qo_value(int qtype, const void *blocks, size_t index) {
  switch (qtype) {
    case QO_Q8_0: return value_q8_0(&((const qo_q8_0_block *)blocks)[index / 32], index % 32);
    case QO_Q4_0: return value_q4_0(&((const qo_q4_0_block *)blocks)[index / 32], index % 32);
    case QO_Q4_K: return value_q4_k(&((const qo_q4_k_block *)blocks)[index / 256], index % 256);
    case QO_Q5_K: return value_q5_k(&((const qo_q5_k_block *)blocks)[index / 256], index % 256);
    case QO_Q6_K: return value_q6_k(&((const qo_q6_k_block *)blocks)[index / 256], index % 256);
    default: return NAN;
  }
}

/* ------------------------------------------------------------ dequantizers */

/* quant schemes/q8.rs:33-45, q4.rs:35-47, q4_k.rs:90-121, q5_k.rs:96-135,
 * q6_k.rs:74-103. Each produces exactly the per-element values above; the Q4_K
 * path hoists (d*sc) and (dmin*m) as the reference does (q4_k.rs:115-117),
 * which is the same sequence of f32 operations. */
int qo_dequantize(int qtype, const void *blocks, size_t count, float *out) {
  size_t bs = qo_block_elems(qtype);
  if (bs == 0 || qtype == QO_F32) return QO_INVALID;
  for (size_t b = 0; b < count; ++b) {
    switch (qtype) {
      case QO_Q4_K: {
        const qo_q4_k_block *blk = &((const qo_q4_k_block *)blocks)[b];
        for (int index = 0; index < 256; ++index) {
          uint8_t sc, mn;
          kquant_scale_min(blk->scales, index / 32, &sc, &mn);
          int group = index / 64, within = index % 64;
          uint8_t packed = blk->values[group * 32 + within % 32];
          uint8_t q = within < 32 ? (packed & 0x0F) : (packed >> 4);
          float scale = blk->scale * (float)sc;
          float minimum = blk->min_scale * (float)mn;
          out[b * 256 + (size_t)index] = scale * (float)q - minimum;
        }
        break;
      }
      default:
        for (size_t l = 0; l < bs; ++l) out[b * bs + l] = qo_value(qtype, blocks, b * bs + l);
    }
  }
  return QO_OK;
}

/* ------------------------------------------------------ CpuScalar matmuls */

static int check_blocks(int qtype, size_t nblocks, size_t k, size_t n) {
  size_t bs = qo_block_elems(qtype);
  if (bs == 0 || qtype == QO_F32) return QO_INVALID;
  if (k == 0 || n == 0) return QO_INVALID;
  if ((k * n) % bs != 0 || nblocks * bs != k * n) return QO_INVALID; /* from_blocks invariant */
  return QO_OK;
}

/* Output rows: backends/cpu/src/matmul.rs:119-160 (Q8_0/Q4_0) and :282-332
 * (K-quants). Per output: sum = 0; for k: sum += x[k] * value(n, k), f32,
 * no FMA, k ascending. */
static void output_rows_range(int qtype, const float *x, size_t k, const void *blocks,
                              size_t n, float *y, size_t row_begin, size_t row_end) {
  size_t bs = qo_block_elems(qtype);
  size_t row_blocks = k / bs;
  for (size_t r = row_begin; r < row_end; ++r) {
    const float *left = x + r * k;
    for (size_t o = 0; o < n; ++o) {
      float sum = 0.0f;
      switch (qtype) {
        case QO_Q8_0: {
          const qo_q8_0_block *row = (const qo_q8_0_block *)blocks + o * row_blocks;
          for (size_t b = 0; b < row_blocks; ++b) {
            float scale = row[b].scale;
            for (int i = 0; i < 32; ++i)
              sum += left[32 * b + (size_t)i] * (scale * (float)row[b].values[i]);
          }
          break;
        }
        case QO_Q4_0: {
          const qo_q4_0_block *row = (const qo_q4_0_block *)blocks + o * row_blocks;
          for (size_t b = 0; b < row_blocks; ++b) {
            float scale = row[b].scale;
            for (int i = 0; i < 32; ++i)
              sum += left[32 * b + (size_t)i] * (scale * ((float)row[b].values[i] - 8.0f));
          }
          break;
        }
        default: {
          for (size_t b = 0; b < row_blocks; ++b) {
            size_t base = (o * row_blocks + b) * bs;
            for (size_t l = 0; l < bs; ++l) sum += left[b * bs + l] * qo_value(qtype, blocks, base + l);
          }
        }
      }
      y[r * n + o] = sum;
    }
  }
}

int qo_matmul_output_rows(int qtype, const float *x, size_t m, size_t k, const void *blocks,
                          size_t nblocks, size_t n, float *y) {
  size_t bs = qo_block_elems(qtype);
  if (check_blocks(qtype, nblocks, k, n) != QO_OK || m == 0 || k % bs != 0) return QO_INVALID;
  output_rows_range(qtype, x, k, blocks, n, y, 0, m);
  return QO_OK;
}

typedef struct {
  int qtype;
  const float *x;
  size_t k, n;
  const void *blocks;
  float *y;
  size_t begin, end;
} rows_job;

static void *rows_worker(void *arg) {
  rows_job *j = (rows_job *)arg;
  output_rows_range(j->qtype, j->x, j->k, j->blocks, j->n, j->y, j->begin, j->end);
  return NULL;
}

/* Rows split across workers as matmul.rs:62-88 does for the row-major path. */
int qo_matmul_output_rows_threaded(int qtype, const float *x, size_t m, size_t k,
                                   const void *blocks, size_t nblocks, size_t n, float *y,
                                   int threads) {
  size_t bs = qo_block_elems(qtype);
  if (check_blocks(qtype, nblocks, k, n) != QO_OK || m == 0 || k % bs != 0) return QO_INVALID;
  size_t workers = threads < 1 ? 1 : (size_t)threads;
  if (workers > m) workers = m;
  if (workers > 64) workers = 64;
  size_t per = (m + workers - 1) / workers;
  pthread_t tid[64];
  rows_job jobs[64];
  size_t started = 0;
  for (size_t w = 0; w < workers; ++w) {
    size_t b = w * per, e = b + per < m ? b + per : m;
    if (b >= e) break;
    jobs[w] = (rows_job){qtype, x, k, n, blocks, y, b, e};
    if (pthread_create(&tid[w], NULL, rows_worker, &jobs[w]) != 0) {
      rows_worker(&jobs[w]);
      tid[w] = 0;
    }
    started = w + 1;
  }
  for (size_t w = 0; w < started; ++w)
    if (tid[w]) pthread_join(tid[w], NULL);
  return QO_OK;
}

/* Row-major: matmul.rs:14-32 (matmul_rows_with) over quantized_value* with
 * flat index k*N + n. The accumulation loop nest is (row, k, column) with
 * result[column] += left * value, i.e. per output the same ascending-k order. */
int qo_matmul_row_major(int qtype, const float *x, size_t m, size_t k, const void *blocks,
                        size_t nblocks, size_t n, float *y) {
  if (check_blocks(qtype, nblocks, k, n) != QO_OK || m == 0) return QO_INVALID;
  for (size_t r = 0; r < m; ++r) {
    float *out = y + r * n;
    for (size_t c = 0; c < n; ++c) out[c] = 0.0f;
    for (size_t i = 0; i < k; ++i) {
      float left = x[r * k + i];
      size_t off = i * n;
      for (size_t c = 0; c < n; ++c) out[c] += left * qo_value(qtype, blocks, off + c);
    }
  }
  return QO_OK;
}

/* F32 matmul: backends/cpu/src/backend.rs:48-60 -> matmul.rs:92-117 */
int qo_matmul_f32(const float *x, size_t m, size_t k, const float *w, size_t n, float *y) {
  if (m == 0 || k == 0 || n == 0) return QO_INVALID;
  for (size_t r = 0; r < m; ++r) {
    float *out = y + r * n;
    for (size_t c = 0; c < n; ++c) out[c] = 0.0f;
    for (size_t i = 0; i < k; ++i) {
      float left = x[r * k + i];
      const float *wr = w + i * n;
      for (size_t c = 0; c < n; ++c) out[c] += left * wr[c];
    }
  }
  return QO_OK;
}

/* ---------------------------------------------------------------- cpu-simd */

#if defined(__x86_64__)
/* cpu-simd lib.rs:100-113 */
__attribute__((target("avx2"))) static float q8_avx2(const float *in, float scale,
                                                      const int8_t *values) {
  __m256 sum = _mm256_setzero_ps();
  for (int index = 0; index < 32; index += 8) {
    __m256 lhs = _mm256_loadu_ps(in + index);
    __m128i codes = _mm_loadl_epi64((const __m128i *)(values + index));
    __m256 c = _mm256_cvtepi32_ps(_mm256_cvtepi8_epi32(codes));
    sum = _mm256_add_ps(sum, _mm256_mul_ps(lhs, c));
  }
  /* horizontal sum, cpu-simd lib.rs:131-143 */
  __m128 high = _mm256_extractf128_ps(sum, 1);
  __m128 low = _mm256_castps256_ps128(sum);
  __m128 s = _mm_add_ps(low, high);
  s = _mm_add_ps(s, _mm_movehl_ps(s, s));
  s = _mm_add_ss(s, _mm_shuffle_ps(s, s, 1));
  return _mm_cvtss_f32(s) * scale;
}

/* cpu-simd lib.rs:115-129 */
__attribute__((target("avx2"))) static float q4_avx2(const float *in, float scale,
                                                      const uint8_t *values) {
  __m256 sum = _mm256_setzero_ps();
  __m256 offset = _mm256_set1_ps(8.0f);
  for (int index = 0; index < 32; index += 8) {
    __m256 lhs = _mm256_loadu_ps(in + index);
    __m128i codes = _mm_loadl_epi64((const __m128i *)(values + index));
    __m256 c = _mm256_sub_ps(_mm256_cvtepi32_ps(_mm256_cvtepu8_epi32(codes)), offset);
    sum = _mm256_add_ps(sum, _mm256_mul_ps(lhs, c));
  }
  __m128 high = _mm256_extractf128_ps(sum, 1);
  __m128 low = _mm256_castps256_ps128(sum);
  __m128 s = _mm_add_ps(low, high);
  s = _mm_add_ps(s, _mm_movehl_ps(s, s));
  s = _mm_add_ss(s, _mm_shuffle_ps(s, s, 1));
  return _mm_cvtss_f32(s) * scale;
}

/* cpu-simd lib.rs:179-190 */
__attribute__((target("avx512f"))) static float q8_avx512(const float *in, float scale,
                                                           const int8_t *values) {
  __m512 sum = _mm512_setzero_ps();
  for (int index = 0; index < 32; index += 16) {
    __m512 lhs = _mm512_loadu_ps(in + index);
    __m128i codes = _mm_loadu_si128((const __m128i *)(values + index));
    __m512 c = _mm512_cvtepi32_ps(_mm512_cvtepi8_epi32(codes));
    sum = _mm512_add_ps(sum, _mm512_mul_ps(lhs, c));
  }
  return _mm512_reduce_add_ps(sum) * scale;
}

/* cpu-simd lib.rs:192-204 */
__attribute__((target("avx512f"))) static float q4_avx512(const float *in, float scale,
                                                           const uint8_t *values) {
  __m512 sum = _mm512_setzero_ps();
  __m512 offset = _mm512_set1_ps(8.0f);
  for (int index = 0; index < 32; index += 16) {
    __m512 lhs = _mm512_loadu_ps(in + index);
    __m128i codes = _mm_loadu_si128((const __m128i *)(values + index));
    __m512 c = _mm512_sub_ps(_mm512_cvtepi32_ps(_mm512_cvtepu8_epi32(codes)), offset);
    sum = _mm512_add_ps(sum, _mm512_mul_ps(lhs, c));
  }
  return _mm512_reduce_add_ps(sum) * scale;
}
#endif

int qo_simd_isa_available(int isa) {
#if defined(__x86_64__)
  __builtin_cpu_init();
  if (isa == 1) return __builtin_cpu_supports("avx2") ? 1 : 0;
  if (isa == 2) return __builtin_cpu_supports("avx512f") ? 1 : 0;
#else
  (void)isa;
#endif
  return 0;
}

/* backends/cpu/src/matmul.rs:334-412: per block a SIMD dot times scale, blocks
 * summed left to right (Iterator::sum). */
int qo_matmul_output_rows_simd(int qtype, int isa, const float *x, size_t m, size_t k,
                               const void *blocks, size_t nblocks, size_t n, float *y) {
  if ((qtype != QO_Q8_0 && qtype != QO_Q4_0) || !qo_simd_isa_available(isa)) return QO_INVALID;
  if (check_blocks(qtype, nblocks, k, n) != QO_OK || m == 0 || k % 32 != 0) return QO_INVALID;
#if defined(__x86_64__)
  size_t row_blocks = k / 32;
  for (size_t r = 0; r < m; ++r) {
    const float *left = x + r * k;
    for (size_t o = 0; o < n; ++o) {
      float sum = -0.0f;
      for (size_t b = 0; b < row_blocks; ++b) {
        const float *in = left + 32 * b;
        float dot;
        if (qtype == QO_Q8_0) {
          const qo_q8_0_block *blk = (const qo_q8_0_block *)blocks + o * row_blocks + b;
          dot = isa == 2 ? q8_avx512(in, blk->scale, blk->values)
                         : q8_avx2(in, blk->scale, blk->values);
        } else {
          const qo_q4_0_block *blk = (const qo_q4_0_block *)blocks + o * row_blocks + b;
          dot = isa == 2 ? q4_avx512(in, blk->scale, blk->values)
                         : q4_avx2(in, blk->scale, blk->values);
        }
        sum += dot;
      }
      y[r * n + o] = sum;
    }
  }
  return QO_OK;
#else
  (void)x; (void)y;
  return QO_INVALID;
#endif
}

/* ---------------------------------------------------------- wire codecs */

static void put_f16(uint8_t *p, float v) {
  uint16_t h = qo_f32_to_f16(v);
  p[0] = (uint8_t)(h & 0xFF);
  p[1] = (uint8_t)(h >> 8);
}
static float get_f16(const uint8_t *p) { return qo_f16_to_f32((uint16_t)(p[0] | (p[1] << 8))); }

/* format gguf/writer.rs:183-261 (standard GGML layouts) */
int qo_wire_pack(int qtype, const void *blocks, size_t count, uint8_t *out) {
  size_t wb = qo_wire_bytes(qtype);
  if (wb == 0 || qtype == QO_F32) return QO_INVALID;
  for (size_t i = 0; i < count; ++i) {
    uint8_t *p = out + i * wb;
    switch (qtype) {
      case QO_Q8_0: {
        const qo_q8_0_block *b = &((const qo_q8_0_block *)blocks)[i];
        put_f16(p, b->scale);
        memcpy(p + 2, b->values, 32);
        break;
      }
      case QO_Q4_0: {
        const qo_q4_0_block *b = &((const qo_q4_0_block *)blocks)[i];
        put_f16(p, b->scale);
        for (int j = 0; j < 16; ++j) p[2 + j] = (uint8_t)(b->values[j] | (b->values[j + 16] << 4));
        break;
      }
      case QO_Q4_K: {
        const qo_q4_k_block *b = &((const qo_q4_k_block *)blocks)[i];
        put_f16(p, b->scale);
        put_f16(p + 2, b->min_scale);
        memcpy(p + 4, b->scales, 12);
        memcpy(p + 16, b->values, 128);
        break;
      }
      case QO_Q5_K: {
        const qo_q5_k_block *b = &((const qo_q5_k_block *)blocks)[i];
        put_f16(p, b->scale);
        put_f16(p + 2, b->min_scale);
        memcpy(p + 4, b->scales, 12);
        memcpy(p + 16, b->high_bits, 32);
        memcpy(p + 48, b->values, 128);
        break;
      }
      case QO_Q6_K: {
        const qo_q6_k_block *b = &((const qo_q6_k_block *)blocks)[i];
        memcpy(p, b->low_bits, 128);
        memcpy(p + 128, b->high_bits, 64);
        memcpy(p + 192, b->scales, 16);
        put_f16(p + 208, b->scale);
        break;
      }
    }
  }
  return QO_OK;
}

/* format gguf/decode.rs:90-312; `legacy` selects the pre-GGML pair order for
 * Q4_0 (:168-172) and the scale-first Q6_K layout (:288-290). Non-finite
 * scales are rejected as the reader does. */
int qo_wire_unpack(int qtype, const uint8_t *bytes, size_t count, int legacy, void *blocks) {
  size_t wb = qo_wire_bytes(qtype);
  if (wb == 0 || qtype == QO_F32) return QO_INVALID;
  for (size_t i = 0; i < count; ++i) {
    const uint8_t *p = bytes + i * wb;
    switch (qtype) {
      case QO_Q8_0: {
        qo_q8_0_block *b = &((qo_q8_0_block *)blocks)[i];
        b->scale = get_f16(p);
        if (!isfinite(b->scale)) return QO_INVALID;
        memcpy(b->values, p + 2, 32);
        break;
      }
      case QO_Q4_0: {
        qo_q4_0_block *b = &((qo_q4_0_block *)blocks)[i];
        b->scale = get_f16(p);
        if (!isfinite(b->scale)) return QO_INVALID;
        for (int j = 0; j < 16; ++j) {
          uint8_t packed = p[2 + j];
          int lo = legacy ? 2 * j : j, hi = legacy ? 2 * j + 1 : j + 16;
          b->values[lo] = packed & 0x0F;
          b->values[hi] = packed >> 4;
        }
        break;
      }
      case QO_Q4_K: {
        qo_q4_k_block *b = &((qo_q4_k_block *)blocks)[i];
        b->scale = get_f16(p);
        b->min_scale = get_f16(p + 2);
        if (!isfinite(b->scale) || !isfinite(b->min_scale)) return QO_INVALID;
        memcpy(b->scales, p + 4, 12);
        memcpy(b->values, p + 16, 128);
        break;
      }
      case QO_Q5_K: {
        qo_q5_k_block *b = &((qo_q5_k_block *)blocks)[i];
        b->scale = get_f16(p);
        b->min_scale = get_f16(p + 2);
        if (!isfinite(b->scale) || !isfinite(b->min_scale)) return QO_INVALID;
        memcpy(b->scales, p + 4, 12);
        memcpy(b->high_bits, p + 16, 32);
        memcpy(b->values, p + 48, 128);
        break;
      }
      case QO_Q6_K: {
        qo_q6_k_block *b = &((qo_q6_k_block *)blocks)[i];
        if (legacy) {
          b->scale = get_f16(p);
          memcpy(b->scales, p + 2, 16);
          memcpy(b->low_bits, p + 18, 128);
          memcpy(b->high_bits, p + 146, 64);
        } else {
          memcpy(b->low_bits, p, 128);
          memcpy(b->high_bits, p + 128, 64);
          memcpy(b->scales, p + 192, 16);
          b->scale = get_f16(p + 208);
        }
        if (!isfinite(b->scale)) return QO_INVALID;
        break;
      }
    }
  }
  return QO_OK;
}

/* --------------------------------------------------------------- inputs */

/* SplitMix64 (Steele, Lea, Flood 2014; constants as published by Vigna),
 * used counter-style: draw c of a stream is the SplitMix64 output for state
 * seed + c*gamma, i.e. exactly the c-th output of the sequential generator. */
static uint64_t splitmix64_at(uint64_t seed, uint64_t counter) {
  uint64_t z = seed + (counter + 1) * 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

static double unit_open(uint64_t seed, uint64_t counter) { /* (0, 1] */
  return ((double)(splitmix64_at(seed, counter) >> 11) + 1.0) * (1.0 / 9007199254740992.0);
}

typedef struct {
  uint64_t seed;
  size_t begin, end;
  double std, outlier_rate, outlier_std;
  float *out;
} fill_job;

/* Element i consumes draws 3i, 3i+1 (Box-Muller in double precision) and 3i+2
 * (the outlier decision), so any chunking gives the same tensor. */
static void *fill_worker(void *arg) {
  const fill_job *j = (const fill_job *)arg;
  const double two_pi = 6.283185307179586476925286766559;
  for (size_t i = j->begin; i < j->end; ++i) {
    double u1 = unit_open(j->seed, 3 * (uint64_t)i);
    double u2 = unit_open(j->seed, 3 * (uint64_t)i + 1);
    double u3 = unit_open(j->seed, 3 * (uint64_t)i + 2);
    double z = sqrt(-2.0 * log(u1)) * cos(two_pi * u2);
    double s = (j->outlier_rate > 0.0 && u3 <= j->outlier_rate) ? j->outlier_std : j->std;
    j->out[i] = (float)(z * s);
  }
  return NULL;
}

void qo_fill_normal(uint64_t seed, size_t n, double std, double outlier_rate,
                    double outlier_std, float *out) {
  enum { MAXW = 16 };
  size_t workers = n >= (1u << 20) ? MAXW : 1;
  size_t per = (n + workers - 1) / workers;
  pthread_t tid[MAXW];
  fill_job jobs[MAXW];
  int started[MAXW] = {0};
  for (size_t w = 0; w < workers; ++w) {
    size_t b = w * per, e = b + per < n ? b + per : n;
    jobs[w] = (fill_job){seed, b < n ? b : n, e > b ? e : b, std, outlier_rate, outlier_std, out};
    if (workers > 1 && pthread_create(&tid[w], NULL, fill_worker, &jobs[w]) == 0)
      started[w] = 1;
    else
      fill_worker(&jobs[w]);
  }
  for (size_t w = 0; w < workers; ++w)
    if (started[w]) pthread_join(tid[w], NULL);
}
