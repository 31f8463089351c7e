// Host-side validation and packing of logical blocks into the device image.
#include <math.h>
#include <string.h>

#include "../../include/qi_hip.h"
#include "qi_image.h"

namespace qi {
namespace {

bool f16_exact(float v) {
  // IEEE binary16 round trip (round to nearest even). A scale survives it
  // unchanged exactly when it is representable as f16.
  _Float16 h = static_cast<_Float16>(v);
  return static_cast<float>(h) == v || (v != v);
}

uint64_t align256(uint64_t x) { return (x + 255u) & ~static_cast<uint64_t>(255u); }

template <class B>
const B* as_blocks(const void* p) {
  return static_cast<const B*>(p);
}

// Scale fields of block i: writes up to two scales, returns false when a scale
// is not finite (core quantized/*.rs from_blocks reject those).
bool block_scales(int32_t qtype, const void* blocks, uint64_t i, float* d, float* dmin) {
  *dmin = 0.0f;
  switch (qtype) {
    case kQ8_0: *d = as_blocks<qi_hip_q8_0_block>(blocks)[i].scale; break;
    case kQ4_0: *d = as_blocks<qi_hip_q4_0_block>(blocks)[i].scale; break;
    case kQ4_K:
      *d = as_blocks<qi_hip_q4_k_block>(blocks)[i].scale;
      *dmin = as_blocks<qi_hip_q4_k_block>(blocks)[i].min_scale;
      break;
    case kQ5_K:
      *d = as_blocks<qi_hip_q5_k_block>(blocks)[i].scale;
      *dmin = as_blocks<qi_hip_q5_k_block>(blocks)[i].min_scale;
      break;
    case kQ6_K: *d = as_blocks<qi_hip_q6_k_block>(blocks)[i].scale; break;
    default: return false;
  }
  return isfinite(*d) && isfinite(*dmin);
}

}  // namespace

int32_t plan_image(int32_t qtype, int32_t layout, uint64_t k, uint64_t n, const void* blocks,
                   uint64_t count, Image* out, const char** why) {
  *why = "";
  if (qtype < kF32 || qtype > kQ6_K) { *why = "unknown weight type"; return QI_HIP_INVALID_INPUT; }
  if (layout != kRowMajor && layout != kOutputRows) { *why = "unknown layout"; return QI_HIP_INVALID_INPUT; }
  // tensor dimensions must be greater than zero (core tensor.rs:85-93)
  if (k == 0 || n == 0) { *why = "matrix dimensions must be greater than zero"; return QI_HIP_INVALID_INPUT; }
  if (k > 0x7FFFFFFFull || n > 0x7FFFFFFFull) { *why = "matrix dimension exceeds kernel indexing"; return QI_HIP_INVALID_INPUT; }
  uint64_t elements = 0;
  if (__builtin_mul_overflow(k, n, &elements) || elements > (1ull << 40)) {
    *why = "matrix element count overflows"; return QI_HIP_INVALID_INPUT;
  }
  if (blocks == nullptr) { *why = "null block pointer"; return QI_HIP_INVALID_INPUT; }
  Image im;
  im.qtype = qtype;
  im.layout = layout;
  im.k = k;
  im.n = n;
  if (qtype == kF32) {
    if (layout != kRowMajor) { *why = "F32 weights are row-major [K, N]"; return QI_HIP_INVALID_INPUT; }
    if (count != elements) { *why = "F32 weight element count does not match K*N"; return QI_HIP_INVALID_INPUT; }
    im.nblocks = elements;
    im.off_qs = 0;
    im.bytes = align256(elements * 4);
    *out = im;
    return QI_HIP_OK;
  }
  const uint64_t be = block_elems(qtype);
  // element count a multiple of the block size and block count matching the
  // shape (core quantized/q8.rs:24-33, q4.rs:26-35, q4.rs:91-100, k.rs:23-28, k.rs:70-75)
  if (elements % be != 0) { *why = "tensor element count is not a multiple of the block size"; return QI_HIP_INVALID_INPUT; }
  if (count != elements / be) { *why = "block count does not match tensor shape"; return QI_HIP_INVALID_INPUT; }
  // output rows need whole blocks per output (backends/cpu/src/matmul.rs:136-140, 299-314)
  if (layout == kOutputRows && k % be != 0) {
    *why = "invalid quantized output rows: K is not a multiple of the block size";
    return QI_HIP_INVALID_INPUT;
  }
  bool all_f16 = true;
  for (uint64_t i = 0; i < count; ++i) {
    float d, dmin;
    if (!block_scales(qtype, blocks, i, &d, &dmin)) { *why = "block scales must be finite"; return QI_HIP_INVALID_INPUT; }
    if (all_f16 && !(f16_exact(d) && f16_exact(dmin))) all_f16 = false;
    if (qtype == kQ4_0) {
      const uint8_t* v = as_blocks<qi_hip_q4_0_block>(blocks)[i].values;
      for (int j = 0; j < 32; ++j)
        if (v[j] > 15) { *why = "Q4_0 values must fit in four bits"; return QI_HIP_INVALID_INPUT; }
    }
  }
  const PlaneSizes ps = plane_sizes(qtype);
  const uint64_t scale_bytes = all_f16 ? 2 : 4;
  im.nblocks = count;
  im.wide = all_f16 ? 0 : 1;
  uint64_t off = 0;
  im.off_qs = off;
  off = align256(off + count * ps.qs);
  im.off_qh = off;
  off = align256(off + count * ps.qh);
  im.off_sc = off;
  off = align256(off + count * ps.sc);
  im.off_d = off;
  off = align256(off + count * scale_bytes);
  im.off_dmin = off;
  off = align256(off + (ps.has_dmin ? count * scale_bytes : 0));
  im.bytes = off + 256;  // slack: 16-byte vector loads never leave the allocation
  *out = im;
  return QI_HIP_OK;
}

namespace {

void put_scale(uint8_t* plane, uint64_t i, float v, bool wide) {
  if (wide) {
    memcpy(plane + 4 * i, &v, 4);
  } else {
    _Float16 h = static_cast<_Float16>(v);
    memcpy(plane + 2 * i, &h, 2);
  }
}

}  // namespace

void fill_image(const Image& im, const void* blocks, void* out) {
  uint8_t* base = static_cast<uint8_t*>(out);
  memset(base, 0, im.bytes);
  if (im.qtype == kF32) {
    memcpy(base, blocks, im.nblocks * 4);
    return;
  }
  uint8_t* qs = base + im.off_qs;
  uint8_t* qh = base + im.off_qh;
  uint8_t* sc = base + im.off_sc;
  uint8_t* d = base + im.off_d;
  uint8_t* dmin = base + im.off_dmin;
  const bool wide = im.wide != 0;
  for (uint64_t i = 0; i < im.nblocks; ++i) {
    switch (im.qtype) {
      case kQ8_0: {
        const auto& b = as_blocks<qi_hip_q8_0_block>(blocks)[i];
        memcpy(qs + 32 * i, b.values, 32);
        put_scale(d, i, b.scale, wide);
        break;
      }
      case kQ4_0: {
        // GGML split-half nibble order (format gguf/writer.rs:201-203)
        const auto& b = as_blocks<qi_hip_q4_0_block>(blocks)[i];
        for (int j = 0; j < 16; ++j)
          qs[16 * i + j] = static_cast<uint8_t>(b.values[j] | (b.values[j + 16] << 4));
        put_scale(d, i, b.scale, wide);
        break;
      }
      case kQ4_K: {
        const auto& b = as_blocks<qi_hip_q4_k_block>(blocks)[i];
        memcpy(qs + 128 * i, b.values, 128);
        memcpy(sc + 12 * i, b.scales, 12);
        put_scale(d, i, b.scale, wide);
        put_scale(dmin, i, b.min_scale, wide);
        break;
      }
      case kQ5_K: {
        const auto& b = as_blocks<qi_hip_q5_k_block>(blocks)[i];
        memcpy(qs + 128 * i, b.values, 128);
        memcpy(qh + 32 * i, b.high_bits, 32);
        memcpy(sc + 12 * i, b.scales, 12);
        put_scale(d, i, b.scale, wide);
        put_scale(dmin, i, b.min_scale, wide);
        break;
      }
      case kQ6_K: {
        const auto& b = as_blocks<qi_hip_q6_k_block>(blocks)[i];
        memcpy(qs + 128 * i, b.low_bits, 128);
        memcpy(qh + 64 * i, b.high_bits, 64);
        memcpy(sc + 16 * i, b.scales, 16);
        put_scale(d, i, b.scale, wide);
        break;
      }
    }
  }
}

}  // namespace qi
