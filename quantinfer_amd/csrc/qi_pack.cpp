// Host-side validation and packing of logical blocks into the device image.
#include <math.h>
#include <string.h>

#include <vector>

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
  // The matrix-core GEMM rounds every weight (Q8_0/Q4_0: code times the f16
  // scale) to an f16 operand. It is used only when that loses nothing beyond
  // f16's relative precision: the largest possible weight magnitude stays
  // below 2^15 (no overflow to infinity), Q8_0/Q4_0 scales are f16 normals
  // (>= 2^-14; a subnormal scale would be rounded with an error of up to 2^-25
  // absolute, hundreds of times f16's relative step for such a scale), and the
  // K-quant weights are not all below 2^-10 (so their f16 subnormal floor of
  // 2^-25 stays far below the tensor's scale). Other weights take the f32
  // kernels in AUTO mode.
  bool all_f16 = true, f16_gemm = true;
  float wmax = 0.0f;
  for (uint64_t i = 0; i < count; ++i) {
    float d, dmin;
    if (!block_scales(qtype, blocks, i, &d, &dmin)) { *why = "block scales must be finite"; return QI_HIP_INVALID_INPUT; }
    if (all_f16 && !(f16_exact(d) && f16_exact(dmin))) all_f16 = false;
    const float ad = fabsf(d), am = fabsf(dmin);
    switch (qtype) {
      case kQ8_0:
      case kQ4_0:
        if (ad != 0.0f && (ad < 0x1p-14f || ad > 256.0f)) f16_gemm = false;
        wmax = fmaxf(wmax, ad * 128.0f);
        break;
      case kQ4_K: wmax = fmaxf(wmax, ad * (63.0f * 15.0f) + am * 63.0f); break;
      case kQ5_K: wmax = fmaxf(wmax, ad * (63.0f * 31.0f) + am * 63.0f); break;
      case kQ6_K: wmax = fmaxf(wmax, ad * (127.0f * 32.0f)); break;
    }
    if (qtype == kQ4_0) {
      const uint8_t* v = as_blocks<qi_hip_q4_0_block>(blocks)[i].values;
      for (int j = 0; j < 32; ++j)
        if (v[j] > 15) { *why = "Q4_0 values must fit in four bits"; return QI_HIP_INVALID_INPUT; }
    }
  }
  const PlaneSizes ps = plane_sizes(qtype);
  const uint64_t scale_bytes = all_f16 ? 2 : 4;
  if (qtype >= kQ4_K && wmax < 0x1p-10f) f16_gemm = false;
  if (wmax > 32768.0f) f16_gemm = false;
  im.nblocks = count;
  im.wide = all_f16 ? 0 : 1;
  im.f16_gemm = f16_gemm ? 1 : 0;
  if ((layout == kOutputRows && k % 256 == 0) || (layout == kRowMajor && n % 256 == 0)) {
    // tiled records: 16-row tiles x 256-element units, a row being one
    // output's K elements (output rows) or one k's N elements (row major)
    const uint64_t rows = layout == kOutputRows ? n : k, cols = layout == kOutputRows ? k : n;
    im.tiled = 1;
    im.tiles = (rows + 15) / 16;
    im.units = cols / 256;
    im.rec = record_geometry(qtype, im.wide != 0);
    im.off_qs = im.off_qh = im.off_sc = im.off_d = im.off_dmin = 0;
    im.bytes = im.tiles * im.units * im.rec.bytes + 256;
    *out = im;
    return QI_HIP_OK;
  }
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

// Byte destinations of one block (n, b) in the image, for either arrangement.
struct Dest {
  const Image* im;
  uint8_t* base;
  uint64_t blk = 0;      // planar block index
  uint8_t* rec = nullptr;  // tiled record
  uint32_t col = 0, bi = 0;

  void at(uint64_t n, uint64_t b) {
    if (!im->tiled) {
      blk = n * (im->k / block_elems(im->qtype)) + b;
      return;
    }
    const uint64_t tile = n / 16, u = b / im->rec.bpu;
    col = static_cast<uint32_t>(n % 16);
    bi = static_cast<uint32_t>(b % im->rec.bpu);
    rec = base + (tile * im->units + u) * im->rec.bytes;
  }
  uint8_t* code(uint32_t o) const {
    const PlaneSizes ps = plane_sizes(im->qtype);
    if (!im->tiled) return base + im->off_qs + blk * ps.qs + o;
    const uint32_t s = bi * ps.qs + o, quarter = im->rec.slice / 4;
    const uint32_t g = s / quarter, q = (s % quarter) / 16, r = s % 16;
    return rec + im->rec.qs + q * 1024 + (16 * g + col) * 16 + r;
  }
  uint8_t* qh(uint32_t o) const {
    if (!im->tiled) return base + im->off_qh + blk * plane_sizes(im->qtype).qh + o;
    return rec + im->rec.qh + (o / 16) * 256 + col * 16 + o % 16;
  }
  uint8_t* sc(uint32_t o) const {
    const uint32_t scb = plane_sizes(im->qtype).sc;
    if (!im->tiled) return base + im->off_sc + blk * scb + o;
    return rec + im->rec.sc + col * scb + o;
  }
  void scale(float v, bool min_plane) const {
    const bool wide = im->wide != 0;
    uint8_t* p;
    const uint32_t ss = wide ? 4 : 2;
    if (!im->tiled) {
      p = base + (min_plane ? im->off_dmin : im->off_d) + blk * ss;
    } else if (min_plane) {
      p = rec + im->rec.dmin + col * ss;
    } else {
      p = rec + im->rec.d + (col * im->rec.bpu + bi) * ss;
    }
    if (wide) {
      memcpy(p, &v, 4);
    } else {
      _Float16 h = static_cast<_Float16>(v);
      memcpy(p, &h, 2);
    }
  }
};

// 6-bit scale and min of sub-block j from a Q4_K/Q5_K block's 12 packed
// bytes (backends/cpu/src/matmul.rs:192-201).
void kq_unpack(const uint8_t s[12], int j, uint32_t* sc, uint32_t* m) {
  if (j < 4) {
    *sc = s[j] & 63u;
    *m = s[j + 4] & 63u;
  } else {
    *sc = (s[j + 4] & 15u) | ((static_cast<uint32_t>(s[j - 4]) >> 6) << 4);
    *m = (static_cast<uint32_t>(s[j + 4]) >> 4) | ((static_cast<uint32_t>(s[j]) >> 6) << 4);
  }
}

// Scale bytes of a K-quant block: reference order in planar images, the
// per-lane-group arrangement of the tiled records (qi_image.h).
void put_kq_scales(const Dest& dst, const uint8_t s[12]) {
  if (!dst.im->tiled) {
    for (uint32_t o = 0; o < 12; ++o) *dst.sc(o) = s[o];
    return;
  }
  for (int g = 0; g < 4; ++g) {
    uint32_t sc0, m0, sc1, m1;
    kq_unpack(s, 2 * g, &sc0, &m0);
    kq_unpack(s, 2 * g + 1, &sc1, &m1);
    const uint32_t f = sc0 | (m0 << 6) | (sc1 << 12) | (m1 << 18);
    for (int b = 0; b < 3; ++b) *dst.sc(3 * g + b) = static_cast<uint8_t>(f >> (8 * b));
  }
}

void put_q6_scales(const Dest& dst, const int8_t s[16]) {
  for (uint32_t i = 0; i < 16; ++i)
    *dst.sc(dst.im->tiled ? q6_scale_pos(i) : i) = static_cast<uint8_t>(s[i]);
}

}  // namespace

void fill_image(const Image& im, const void* blocks, void* out) {
  uint8_t* base = static_cast<uint8_t*>(out);
  memset(base, 0, im.bytes);
  if (im.qtype == kF32) {
    memcpy(base, blocks, im.nblocks * 4);
    return;
  }
  const uint64_t be = block_elems(im.qtype);
  // block order of the reference: output rows (n, b) -> n*NB + b; row major is
  // flat, (k, b) -> k*(N/bs) + b, taken per k (a record row) when tiled
  const uint64_t nb = im.layout == kOutputRows ? im.k / be : im.tiled ? im.n / be : im.nblocks;
  Dest dst{&im, base};
  for (uint64_t i = 0; i < im.nblocks; ++i) {
    dst.at(i / nb, i % nb);
    switch (im.qtype) {
      case kQ8_0: {
        const auto& b = as_blocks<qi_hip_q8_0_block>(blocks)[i];
        for (uint32_t o = 0; o < 32; ++o) *dst.code(o) = static_cast<uint8_t>(b.values[o]);
        dst.scale(b.scale, false);
        break;
      }
      case kQ4_0: {
        // GGML split-half nibble order (format gguf/writer.rs:201-203)
        const auto& b = as_blocks<qi_hip_q4_0_block>(blocks)[i];
        for (uint32_t j = 0; j < 16; ++j)
          *dst.code(j) = static_cast<uint8_t>(b.values[j] | (b.values[j + 16] << 4));
        dst.scale(b.scale, false);
        break;
      }
      case kQ4_K: {
        const auto& b = as_blocks<qi_hip_q4_k_block>(blocks)[i];
        for (uint32_t o = 0; o < 128; ++o) *dst.code(o) = b.values[o];
        put_kq_scales(dst, b.scales);
        dst.scale(b.scale, false);
        dst.scale(b.min_scale, true);
        break;
      }
      case kQ5_K: {
        const auto& b = as_blocks<qi_hip_q5_k_block>(blocks)[i];
        for (uint32_t o = 0; o < 128; ++o) *dst.code(o) = b.values[o];
        for (uint32_t o = 0; o < 32; ++o) *dst.qh(o) = b.high_bits[o];
        put_kq_scales(dst, b.scales);
        dst.scale(b.scale, false);
        dst.scale(b.min_scale, true);
        break;
      }
      case kQ6_K: {
        const auto& b = as_blocks<qi_hip_q6_k_block>(blocks)[i];
        for (uint32_t o = 0; o < 128; ++o) *dst.code(o) = b.low_bits[o];
        for (uint32_t o = 0; o < 64; ++o) *dst.qh(o) = b.high_bits[o];
        put_q6_scales(dst, b.scales);
        dst.scale(b.scale, false);
        break;
      }
    }
  }
}

}  // namespace qi

namespace qi {

namespace {

// f16 little-endian to f32 (exact); false for inf/NaN, which the GGUF block
// readers reject (format/src/gguf/decode.rs:110-116 and the other types).
bool wire_f16(const uint8_t* p, float* out) {
  _Float16 h;
  memcpy(&h, p, 2);
  *out = static_cast<float>(h);
  return isfinite(*out);
}

}  // namespace

// The GGUF block readers of format/src/gguf/decode.rs: tensor_q8_0 (:90-130),
// tensor_q4_0 (:132-179, legacy nibble pairs :168-172), tensor_q4_k
// (:181-227), tensor_q5_k (:229-268), tensor_q6_k (:270-312, legacy field
// order :288-290), writing the logical blocks of include/qi_hip.h.
int32_t gguf_decode(int32_t qtype, const void* wire, uint64_t bytes, int32_t legacy, void* out_vec,
                    uint64_t* count, const char** why) {
  std::vector<uint8_t>& out = *static_cast<std::vector<uint8_t>*>(out_vec);
  const uint8_t* in = static_cast<const uint8_t*>(wire);
  if (wire == nullptr && bytes != 0) {
    *why = "null wire data";
    return QI_HIP_INVALID_INPUT;
  }
  uint64_t wb = 0, lb = 0;
  switch (qtype) {
    case kF32: wb = lb = 4; break;
    case kQ8_0: wb = 34; lb = sizeof(qi_hip_q8_0_block); break;
    case kQ4_0: wb = 18; lb = sizeof(qi_hip_q4_0_block); break;
    case kQ4_K: wb = 144; lb = sizeof(qi_hip_q4_k_block); break;
    case kQ5_K: wb = 176; lb = sizeof(qi_hip_q5_k_block); break;
    case kQ6_K: wb = 210; lb = sizeof(qi_hip_q6_k_block); break;
    default: *why = "unknown weight type"; return QI_HIP_UNSUPPORTED;
  }
  if (bytes % wb != 0) {
    *why = "GGUF tensor has an invalid byte length";
    return QI_HIP_INVALID_INPUT;
  }
  const uint64_t nb = bytes / wb;
  *count = nb;
  out.assign(nb * lb, 0);
  if (qtype == kF32) {
    if (bytes) memcpy(out.data(), in, bytes);
    return QI_HIP_OK;
  }
  for (uint64_t i = 0; i < nb; ++i) {
    const uint8_t* c = in + i * wb;
    uint8_t* o = out.data() + i * lb;
    bool ok = true;
    switch (qtype) {
      case kQ8_0: {
        qi_hip_q8_0_block b;
        ok = wire_f16(c, &b.scale);
        memcpy(b.values, c + 2, 32);
        memcpy(o, &b, sizeof b);
        break;
      }
      case kQ4_0: {
        qi_hip_q4_0_block b;
        ok = wire_f16(c, &b.scale);
        for (int j = 0; j < 16; ++j) {
          const uint8_t packed = c[2 + j];
          const int lo = legacy ? 2 * j : j, hi = legacy ? 2 * j + 1 : j + 16;
          b.values[lo] = packed & 0x0F;
          b.values[hi] = packed >> 4;
        }
        memcpy(o, &b, sizeof b);
        break;
      }
      case kQ4_K: {
        qi_hip_q4_k_block b;
        ok = wire_f16(c, &b.scale) & wire_f16(c + 2, &b.min_scale);
        memcpy(b.scales, c + 4, 12);
        memcpy(b.values, c + 16, 128);
        memcpy(o, &b, sizeof b);
        break;
      }
      case kQ5_K: {
        qi_hip_q5_k_block b;
        ok = wire_f16(c, &b.scale) & wire_f16(c + 2, &b.min_scale);
        memcpy(b.scales, c + 4, 12);
        memcpy(b.high_bits, c + 16, 32);
        memcpy(b.values, c + 48, 128);
        memcpy(o, &b, sizeof b);
        break;
      }
      default: {  // kQ6_K
        qi_hip_q6_k_block b;
        const uint8_t *d, *sc, *ql, *qh;
        if (legacy) {
          d = c; sc = c + 2; ql = c + 18; qh = c + 146;
        } else {
          ql = c; qh = c + 128; sc = c + 192; d = c + 208;
        }
        ok = wire_f16(d, &b.scale);
        memcpy(b.scales, sc, 16);
        memcpy(b.low_bits, ql, 128);
        memcpy(b.high_bits, qh, 64);
        memcpy(o, &b, sizeof b);
        break;
      }
    }
    if (!ok) {
      *why = "GGUF tensor contains a non-finite scale";
      return QI_HIP_INVALID_INPUT;
    }
  }
  return QI_HIP_OK;
}

}  // namespace qi
