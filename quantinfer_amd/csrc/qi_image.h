// Device image of a resident weight: the logical blocks split into planes
// ("structure of arrays"), each plane contiguous in block order.
//
// Block order is the reference's: for the output-rows layout output n owns
// blocks [n*NB, n*NB+NB) with NB = K / block_elems, so every plane is
// row-contiguous and a wavefront's 16-byte loads of one plane are coalesced.
// The planes hold exactly the bytes of the GGUF wire block (codes, high bits,
// packed 6-bit scales, f16 d/dmin), so the image of an f16-scale tensor has
// wire size: Q8_0 34, Q4_0 18, Q4_K 144, Q5_K 176, Q6_K 210 bytes per block.
// Scales that are not f16-exact (hand-built blocks, unrounded Q8_0/Q4_0
// quantizer output) switch the whole tensor to f32 scale planes ("wide").
//
//   plane   Q8_0        Q4_0              Q4_K        Q5_K        Q6_K
//   qs      32 B i8     16 B split-half   128 B       128 B       128 B ql
//   qh      -           -                 -           32 B        64 B
//   sc      -           -                 12 B 6-bit  12 B 6-bit  16 B i8
//   d       f16|f32     f16|f32           f16|f32     f16|f32     f16|f32
//   dmin    -           -                 f16|f32     f16|f32     -
// F32 weights keep the row-major [K, N] f32 matrix in qs.
#pragma once
#include <stdint.h>

namespace qi {

enum QType : int32_t { kF32 = 0, kQ8_0 = 1, kQ4_0 = 2, kQ4_K = 3, kQ5_K = 4, kQ6_K = 5 };
enum Layout : int32_t { kRowMajor = 0, kOutputRows = 1 };

struct PlaneSizes {
  uint32_t qs, qh, sc;  // bytes per block
  bool has_dmin;
};

inline PlaneSizes plane_sizes(int32_t qtype) {
  switch (qtype) {
    case kQ8_0: return {32, 0, 0, false};
    case kQ4_0: return {16, 0, 0, false};
    case kQ4_K: return {128, 0, 12, true};
    case kQ5_K: return {128, 32, 12, true};
    case kQ6_K: return {128, 64, 16, false};
    default: return {0, 0, 0, false};
  }
}

inline uint32_t block_elems(int32_t qtype) {
  switch (qtype) {
    case kQ8_0:
    case kQ4_0: return 32;
    case kQ4_K:
    case kQ5_K:
    case kQ6_K: return 256;
    case kF32: return 1;
    default: return 0;
  }
}

struct Image {
  int32_t qtype = 0, layout = 0;
  uint64_t k = 0, n = 0, nblocks = 0;
  int32_t wide = 0;  // 1: f32 scale planes
  uint64_t off_qs = 0, off_qh = 0, off_sc = 0, off_d = 0, off_dmin = 0;
  uint64_t bytes = 0;
};

// Device-side view of an image (plain pointers, passed by value to kernels).
struct View {
  const uint8_t* qs;
  const uint8_t* qh;
  const uint8_t* sc;
  const void* d;
  const void* dmin;
  uint64_t k, n;
  uint32_t nb;  // blocks per output row (output-rows layout)
};

inline View make_view(const Image& im, const void* base) {
  const uint8_t* b = static_cast<const uint8_t*>(base);
  View v;
  v.qs = b + im.off_qs;
  v.qh = b + im.off_qh;
  v.sc = b + im.off_sc;
  v.d = b + im.off_d;
  v.dmin = b + im.off_dmin;
  v.k = im.k;
  v.n = im.n;
  uint32_t be = block_elems(im.qtype);
  v.nb = be ? static_cast<uint32_t>(im.k / be) : 0;
  return v;
}

// Validation + layout of the image (no device). Returns 0 or an ABI status
// with a message in *why.
int32_t plan_image(int32_t qtype, int32_t layout, uint64_t k, uint64_t n, const void* blocks,
                   uint64_t count, Image* out, const char** why);
// Write the planes of a planned image into host memory of im.bytes bytes.
void fill_image(const Image& im, const void* blocks, void* out);

}  // namespace qi
