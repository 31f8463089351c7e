// Host-side block quantizers: f32 values -> the reference's logical blocks.
//
// The reference quantizes offline (crates/quantinfer-quant/src/schemes):
// round-to-nearest block quantization with per-block scales, the K-quants
// with a second level of 6-bit (Q4_K/Q5_K) or int8 (Q6_K) sub-block scales
// under an f16 super-block scale, their codes chosen in f64 after both scale
// levels are fixed. These functions produce the same blocks bit for bit, so a
// caller can build weights of a given distribution without the Rust crate,
// and split the work over host threads (blocks are independent).
//
// Rust semantics kept here: f32::round rounds half away from zero (roundf /
// round); f32::max/min ignore a NaN operand (fmaxf/fminf); `as u8` / `as i8`
// after clamp are exact conversions; half::f16::from_f32 rounds to nearest
// even (the _Float16 conversion).
#include <math.h>
#include <string.h>

#include <algorithm>
#include <atomic>
#include <thread>
#include <vector>

#include "../../include/qi_hip.h"
#include "qi_ctx.h"
#include "qi_image.h"

namespace qi {
namespace {

constexpr float kEps = 1.1920929e-07f;  // f32::EPSILON

float f16_round(float v) { return static_cast<float>(static_cast<_Float16>(v)); }

// quant/src/schemes/mod.rs:27-40 (stored_f16_scale): false when the f16 value
// is not finite; a positive value that rounds to zero keeps the smallest f16
// subnormal.
bool stored_f16_scale(float v, float* out) {
  float s = f16_round(v);
  if (!isfinite(s)) return false;
  if (s == 0.0f && v > 0.0f) s = 5.9604645e-08f;  // f16 bits 0x0001 = 2^-24
  *out = s;
  return true;
}

// quant/src/schemes/q8.rs:17-29
void quantize_q8_0(const float* v, qi_hip_q8_0_block* b) {
  float mx = 0.0f;
  for (int i = 0; i < 32; ++i) mx = fmaxf(mx, fabsf(v[i]));
  const float scale = mx == 0.0f ? 1.0f : mx / 127.0f;
  for (int i = 0; i < 32; ++i) {
    const float r = std::min(std::max(roundf(v[i] / scale), -127.0f), 127.0f);
    b->values[i] = static_cast<int8_t>(r);
  }
  b->scale = scale;
}

// quant/src/schemes/q4.rs:17-27
void quantize_q4_0(const float* v, qi_hip_q4_0_block* b) {
  float mx = 0.0f;
  for (int i = 0; i < 32; ++i) mx = fmaxf(mx, fabsf(v[i]));
  const float scale = mx == 0.0f ? 1.0f : mx / 7.0f;
  for (int i = 0; i < 32; ++i) {
    const float r = std::min(std::max(roundf(v[i] / scale), -8.0f), 7.0f);
    b->values[i] = static_cast<uint8_t>(static_cast<int32_t>(r) + 8);
  }
  b->scale = scale;
}

// Q4_K / Q5_K (quant/src/schemes/q4_k.rs:17-83, q5_k.rs:17-93): per 32-element
// sub-block range [min(0, lo), hi] over `top` steps, the sub-block scales and
// mins quantized to 6 bits under f16 d and dmin, codes in f64 against the
// resulting grid. Writes d, dmin, the 12 packed scale bytes and the codes.
bool quantize_k_affine(const float* v, int top, float* d_out, float* dmin_out, uint8_t packed[12],
                       uint8_t codes[256]) {
  float scales[8], mins[8];
  for (int s = 0; s < 8; ++s) {
    float lo = INFINITY, hi = -INFINITY;
    for (int i = 0; i < 32; ++i) {
      lo = fminf(lo, v[32 * s + i]);
      hi = fmaxf(hi, v[32 * s + i]);
    }
    lo = fminf(lo, 0.0f);
    scales[s] = fmaxf((hi - lo) / static_cast<float>(top), kEps);
    mins[s] = -lo;
  }
  float scale_max = 0.0f, min_max = 0.0f;
  for (int s = 0; s < 8; ++s) {
    scale_max = fmaxf(scale_max, scales[s]);
    min_max = fmaxf(min_max, mins[s]);
  }
  scale_max = fmaxf(scale_max, kEps);
  float d, dmin;
  if (!stored_f16_scale(scale_max / 63.0f, &d)) return false;
  if (!stored_f16_scale(min_max == 0.0f ? 1.0f : min_max / 63.0f, &dmin)) return false;
  uint8_t sv[8], mv[8];
  for (int s = 0; s < 8; ++s) {
    sv[s] = d == 0.0f ? 0 : static_cast<uint8_t>(std::min(std::max(roundf(scales[s] / d), 1.0f), 63.0f));
    mv[s] = dmin == 0.0f ? 0 : static_cast<uint8_t>(std::min(std::max(roundf(mins[s] / dmin), 0.0f), 63.0f));
  }
  for (int i = 0; i < 256; ++i) {
    const double scale = static_cast<double>(d) * static_cast<double>(sv[i / 32]);
    const double minimum = static_cast<double>(dmin) * static_cast<double>(mv[i / 32]);
    codes[i] = scale == 0.0
                   ? 0
                   : static_cast<uint8_t>(std::min(
                         std::max(round((static_cast<double>(v[i]) + minimum) / scale), 0.0),
                         static_cast<double>(top)));
  }
  // 6-bit packing: sub-blocks 0-3 in the low six bits of bytes 0-3 (scales)
  // and 4-7 (mins); sub-blocks 4-7 in bytes 8-11 (scale low nibble, min high
  // nibble) with their top two bits in bits 6-7 of bytes 0-7
  for (int i = 0; i < 4; ++i) {
    packed[i] = static_cast<uint8_t>(sv[i] | ((sv[4 + i] >> 4) << 6));
    packed[4 + i] = static_cast<uint8_t>(mv[i] | ((mv[4 + i] >> 4) << 6));
    packed[8 + i] = static_cast<uint8_t>((sv[4 + i] & 15) | ((mv[4 + i] & 15) << 4));
  }
  *d_out = d;
  *dmin_out = dmin;
  return true;
}

bool quantize_q4_k(const float* v, qi_hip_q4_k_block* b) {
  uint8_t codes[256];
  if (!quantize_k_affine(v, 15, &b->scale, &b->min_scale, b->scales, codes)) return false;
  // group g of 64 elements: byte 32g + i = element 64g + i | element 64g + 32 + i << 4
  for (int g = 0; g < 4; ++g)
    for (int i = 0; i < 32; ++i)
      b->values[32 * g + i] = static_cast<uint8_t>(codes[64 * g + i] | (codes[64 * g + 32 + i] << 4));
  return true;
}

bool quantize_q5_k(const float* v, qi_hip_q5_k_block* b) {
  uint8_t codes[256];
  if (!quantize_k_affine(v, 31, &b->scale, &b->min_scale, b->scales, codes)) return false;
  memset(b->high_bits, 0, sizeof b->high_bits);
  for (int g = 0; g < 4; ++g) {
    for (int i = 0; i < 32; ++i) {
      const uint8_t lo = codes[64 * g + i], hi = codes[64 * g + 32 + i];
      b->values[32 * g + i] = static_cast<uint8_t>((lo & 15) | ((hi & 15) << 4));
      // the fifth bits of group g's two halves: bits 2g and 2g + 1 of byte i
      b->high_bits[i] = static_cast<uint8_t>(b->high_bits[i] | ((lo >> 4) << (2 * g)) |
                                             ((hi >> 4) << (2 * g + 1)));
    }
  }
  return true;
}

// quant/src/schemes/q6_k.rs:17-67
bool quantize_q6_k(const float* v, qi_hip_q6_k_block* b) {
  float sub[16];
  for (int s = 0; s < 16; ++s) {
    float mx = 0.0f;
    for (int i = 0; i < 16; ++i) mx = fmaxf(mx, fabsf(v[16 * s + i]));
    sub[s] = fmaxf(mx / 31.0f, kEps);
  }
  float max_scale = 0.0f;
  for (int s = 0; s < 16; ++s) max_scale = fmaxf(max_scale, sub[s]);
  max_scale = fmaxf(max_scale, kEps);
  float d;
  if (!stored_f16_scale(max_scale / 127.0f, &d)) return false;
  for (int s = 0; s < 16; ++s)
    b->scales[s] = d == 0.0f ? 0 : static_cast<int8_t>(std::min(std::max(roundf(sub[s] / d), 1.0f), 127.0f));
  uint8_t q[256];
  for (int i = 0; i < 256; ++i) {
    const double scale = static_cast<double>(d) * static_cast<double>(b->scales[i / 16]);
    const int32_t c = scale == 0.0 ? 0
                                   : static_cast<int32_t>(std::min(
                                         std::max(round(static_cast<double>(v[i]) / scale), -32.0), 31.0));
    q[i] = static_cast<uint8_t>(c + 32);
  }
  // half ip of 128 elements, quarter c of 32: low nibbles in bytes 64ip + il
  // (quarters 0 | 2 << 4) and 64ip + 32 + il (1 | 3 << 4); the top two bits of
  // quarter c at bits 2c of byte 32ip + il
  for (int ip = 0; ip < 2; ++ip) {
    for (int il = 0; il < 32; ++il) {
      const uint8_t q0 = q[128 * ip + il], q1 = q[128 * ip + 32 + il];
      const uint8_t q2 = q[128 * ip + 64 + il], q3 = q[128 * ip + 96 + il];
      b->low_bits[64 * ip + il] = static_cast<uint8_t>((q0 & 15) | ((q2 & 15) << 4));
      b->low_bits[64 * ip + 32 + il] = static_cast<uint8_t>((q1 & 15) | ((q3 & 15) << 4));
      b->high_bits[32 * ip + il] = static_cast<uint8_t>(((q0 >> 4) & 3) | (((q1 >> 4) & 3) << 2) |
                                                        (((q2 >> 4) & 3) << 4) | (((q3 >> 4) & 3) << 6));
    }
  }
  b->scale = d;
  return true;
}

// quant/src/providers/storage.rs:10-18: the f16 storage value of a scale
bool storage_round(float* v) {
  const float r = f16_round(*v);
  if (!isfinite(*v) || !isfinite(r)) return false;
  *v = r;
  return true;
}

// Blocks [b0, b1) of `qtype`; false on the first value or scale the
// reference rejects.
bool quantize_range(int32_t qtype, const float* values, uint64_t b0, uint64_t b1, bool storage_f16,
                    void* out) {
  const uint64_t bs = qtype == kQ8_0 || qtype == kQ4_0 ? 32 : 256;
  for (uint64_t i = b0 * bs; i < b1 * bs; ++i)
    if (!isfinite(values[i])) return false;  // validate_finite, schemes/mod.rs:18-25
  for (uint64_t b = b0; b < b1; ++b) {
    const float* v = values + b * bs;
    bool ok = true;
    switch (qtype) {
      case kQ8_0: {
        auto* blk = static_cast<qi_hip_q8_0_block*>(out) + b;
        quantize_q8_0(v, blk);
        if (storage_f16) ok = storage_round(&blk->scale);
        break;
      }
      case kQ4_0: {
        auto* blk = static_cast<qi_hip_q4_0_block*>(out) + b;
        quantize_q4_0(v, blk);
        if (storage_f16) ok = storage_round(&blk->scale);
        break;
      }
      // the K-quant scales are f16 values already: storage rounding keeps them
      case kQ4_K: ok = quantize_q4_k(v, static_cast<qi_hip_q4_k_block*>(out) + b); break;
      case kQ5_K: ok = quantize_q5_k(v, static_cast<qi_hip_q5_k_block*>(out) + b); break;
      case kQ6_K: ok = quantize_q6_k(v, static_cast<qi_hip_q6_k_block*>(out) + b); break;
      default: return false;
    }
    if (!ok) return false;
  }
  return true;
}

}  // namespace
}  // namespace qi

extern "C" qi_hip_status qi_hip_quantize(int32_t qtype, const float* values, uint64_t n,
                                         int32_t storage_f16, void* out, uint64_t out_count,
                                         int32_t threads) {
  using namespace qi;
  using qi_abi::fail;
  if (qtype < kQ8_0 || qtype > kQ6_K) return fail(QI_HIP_INVALID_INPUT, "quantize: unknown block type");
  if (values == nullptr || out == nullptr) return fail(QI_HIP_INVALID_INPUT, "quantize: null buffer");
  const uint64_t bs = qtype == kQ8_0 || qtype == kQ4_0 ? 32 : 256;
  // the reference's element-count rule (q8.rs:11-16, q4.rs:11-16, q4_k.rs:11-16, ...)
  if (n == 0 || n % bs != 0)
    return fail(QI_HIP_INVALID_INPUT, bs == 32 ? "quantize: requires a multiple of 32 elements"
                                               : "quantize: requires a multiple of 256 elements");
  if (out_count != n / bs) return fail(QI_HIP_INVALID_INPUT, "quantize: output block count differs from n / block size");
  const uint64_t blocks = n / bs;
  const uint64_t hw = std::max(1u, std::thread::hardware_concurrency());
  uint64_t nt = threads > 0 ? static_cast<uint64_t>(threads) : hw;
  nt = std::min<uint64_t>(std::min<uint64_t>(nt, 64), std::max<uint64_t>(1, blocks / 64));
  std::atomic<bool> ok{true};
  auto work = [&](uint64_t t) {
    const uint64_t b0 = blocks * t / nt, b1 = blocks * (t + 1) / nt;
    if (!quantize_range(qtype, values, b0, b1, storage_f16 != 0, out)) ok = false;
  };
  std::vector<std::thread> pool;
  for (uint64_t t = 1; t < nt; ++t) pool.emplace_back(work, t);
  work(0);
  for (auto& th : pool) th.join();
  if (!ok)
    return fail(QI_HIP_INVALID_INPUT,
                "quantize: input values must be finite and every scale representable as a finite f16");
  return QI_HIP_OK;
}

// Synthetic inputs for benchmarks: normal draws from counter-based SplitMix64
// (Steele, Lea and Flood 2014, with Vigna's published constants) and
// Box-Muller in double precision. Element i uses draws 3i, 3i + 1 (the
// normal) and 3i + 2 (outlier or not), so the tensor does not depend on how
// the elements are split over threads.
namespace {

uint64_t mix64(uint64_t seed, uint64_t draw) {
  uint64_t z = seed + (draw + 1) * 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

// uniform on (0, 1]: the top 53 bits, plus one, times 2^-53
double uniform(uint64_t seed, uint64_t draw) {
  return (static_cast<double>(mix64(seed, draw) >> 11) + 1.0) * 0x1p-53;
}

}  // namespace

extern "C" qi_hip_status qi_hip_synth_normal(uint64_t seed, uint64_t n, double std, double outlier_rate,
                                             double outlier_std, float* out, int32_t threads) {
  if (out == nullptr && n > 0) return qi_abi::fail(QI_HIP_INVALID_INPUT, "synth_normal: null output");
  const uint64_t hw = std::max(1u, std::thread::hardware_concurrency());
  uint64_t nt = threads > 0 ? static_cast<uint64_t>(threads) : hw;
  nt = std::min<uint64_t>(std::min<uint64_t>(nt, 64), std::max<uint64_t>(1, n >> 16));
  auto work = [&](uint64_t t) {
    const double two_pi = 6.283185307179586476925286766559;
    const uint64_t i0 = n * t / nt, i1 = n * (t + 1) / nt;
    for (uint64_t i = i0; i < i1; ++i) {
      const double u1 = uniform(seed, 3 * i), u2 = uniform(seed, 3 * i + 1), u3 = uniform(seed, 3 * i + 2);
      const double z = sqrt(-2.0 * log(u1)) * cos(two_pi * u2);
      const double s = outlier_rate > 0.0 && u3 <= outlier_rate ? outlier_std : std;
      out[i] = static_cast<float>(z * s);
    }
  };
  std::vector<std::thread> pool;
  for (uint64_t t = 1; t < nt; ++t) pool.emplace_back(work, t);
  work(0);
  for (auto& th : pool) th.join();
  return QI_HIP_OK;
}
