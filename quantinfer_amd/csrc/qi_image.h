// Device image of a resident weight.
//
// Every image holds exactly the bytes of the GGUF wire blocks (codes, high
// bits, packed 6-bit scales, f16 d/dmin): Q8_0 34, Q4_0 18, Q4_K 144, Q5_K 176,
// Q6_K 210 bytes per block. Scales that are not all f16-exact (hand-built
// blocks, unrounded Q8_0/Q4_0 quantizer output) switch the tensor to f32 scale
// entries ("wide"). Two arrangements:
//
// planar (row major with N not a multiple of 256, output rows with K not a
//   multiple of 256): one plane per field
//   in the reference block order, each plane contiguous.
//
//   plane   Q8_0        Q4_0              Q4_K        Q5_K        Q6_K
//   qs      32 B i8     16 B split-half   128 B       128 B       128 B ql
//   qh      -           -                 -           32 B        64 B
//   sc      -           -                 12 B 6-bit  12 B 6-bit  16 B i8
//   d       f16|f32     f16|f32           f16|f32     f16|f32     f16|f32
//   dmin    -           -                 f16|f32     f16|f32     -
//
// tiled (output rows with K a multiple of 256, what the decode GEMV streams;
//   row major with N a multiple of 256): the rows are grouped in tiles of 16
//   (the last tile zero-padded) and each row in units of 256 elements; one
//   record per (tile, unit) holds the 16 rows' bytes of that unit, records
//   ordered [tile][unit]. A row is one output's K elements (output rows) or
//   one k's N elements (row major, blocks along N). Inside a record:
//     codes  the row slice of S code bytes (Q8_0 S=256, others 128) is split
//            in four lane groups of S/4 bytes and 16-byte chunks; chunk q of
//            lane group g of row c sits at q*1024 + (16g + c)*16, so a
//            wavefront load (lane 16g + c) of chunk q reads 1 KB contiguous;
//     qh     16-byte chunk h of row c at h*256 + c*16 (Q5_K 2, Q6_K 4 chunks);
//     sc     Q4_K/Q5_K: row c's 12 bytes at c*12 hold the same 96 bits as the
//            GGUF packed 6-bit scales, regrouped per lane group: field g at
//            bytes 3g..3g+2 (little endian) = sc[2g] | m[2g] << 6 |
//            sc[2g+1] << 12 | m[2g+1] << 18, sub-block j's (sc, m) being what
//            the reference unpacks (backends/cpu/src/matmul.rs:192-201);
//            Q6_K: row c's 16 int8 sub-scales at c*16, lane group g = 2ip + h
//            holding sub-scales 8ip + 2h + {0, 1, 4, 5} at bytes 4g..4g+3;
//     d      row c's scales: c*8 + block (Q8_0/Q4_0) or c (K-quants) entries;
//     dmin   row c at c (Q4_K/Q5_K).
//   F32 weights keep the row-major [K, N] f32 matrix in qs.
#pragma once
#include <stdint.h>

namespace qi {

enum QType : int32_t { kF32 = 0, kQ8_0 = 1, kQ4_0 = 2, kQ4_K = 3, kQ5_K = 4, kQ6_K = 5 };
enum Layout : int32_t { kRowMajor = 0, kOutputRows = 1 };

struct PlaneSizes {
  uint32_t qs, qh, sc;  // bytes per block
  bool has_dmin;
};

constexpr PlaneSizes plane_sizes(int32_t qtype) {
  switch (qtype) {
    case kQ8_0: return {32, 0, 0, false};
    case kQ4_0: return {16, 0, 0, false};
    case kQ4_K: return {128, 0, 12, true};
    case kQ5_K: return {128, 32, 12, true};
    case kQ6_K: return {128, 64, 16, false};
    default: return {0, 0, 0, false};
  }
}

constexpr uint32_t block_elems(int32_t qtype) {
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

// Record geometry of the tiled arrangement (per 16-row tile, 256-element unit).
struct Record {
  uint32_t bytes = 0;                              // record size
  uint32_t qs = 0, qh = 0, sc = 0, d = 0, dmin = 0;  // section offsets
  uint32_t bpu = 0;                                // blocks per unit per row (8 or 1)
  uint32_t slice = 0;                              // code bytes per row per unit
};

constexpr Record record_geometry(int32_t qtype, bool wide) {
  Record r;
  const PlaneSizes ps = plane_sizes(qtype);
  const uint32_t be = block_elems(qtype);
  if (be == 0 || qtype == kF32) return r;
  r.bpu = 256 / be;
  r.slice = ps.qs * r.bpu;
  const uint32_t ss = wide ? 4 : 2;
  uint32_t off = 16 * r.slice;
  r.qs = 0;
  r.qh = off;
  off += 16 * ps.qh;
  r.sc = off;
  off += 16 * ps.sc;
  r.d = off;
  off += 16 * r.bpu * ss;
  r.dmin = off;
  off += ps.has_dmin ? 16 * ss : 0;
  r.bytes = (off + 15) & ~15u;
  return r;
}

struct Image {
  int32_t qtype = 0, layout = 0;
  uint64_t k = 0, n = 0, nblocks = 0;
  int32_t wide = 0;   // 1: f32 scale entries
  int32_t tiled = 0;  // 1: tiled arrangement
  // 1: every weight value and scale fits the f16 operands of the matrix-core
  // GEMM (no overflow, no scale in f16's subnormal range; see plan_image)
  int32_t f16_gemm = 1;
  uint64_t off_qs = 0, off_qh = 0, off_sc = 0, off_d = 0, off_dmin = 0;  // planar
  uint64_t tiles = 0, units = 0;  // tiled: 16-row tiles, 256-element units per row
  Record rec;
  uint64_t bytes = 0;
};

// Device-side view of an image (plain pointers, passed by value to kernels).
struct View {
  const uint8_t* qs;  // planar qs plane, or the first record
  const uint8_t* qh;
  const uint8_t* sc;
  const void* d;
  const void* dmin;
  uint64_t k, n;
  uint32_t nb;     // blocks per output row (output rows), per k (tiled row major)
  uint32_t tiled;  // 1: records
  uint32_t units;  // tiled: units per row
  uint32_t tiles;  // tiled: tiles
  Record rec;
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
  const uint32_t be = block_elems(im.qtype);
  const uint64_t row = im.layout == kRowMajor && im.tiled ? im.n : im.k;
  v.nb = be ? static_cast<uint32_t>(row / be) : 0;
  v.tiled = static_cast<uint32_t>(im.tiled);
  v.units = static_cast<uint32_t>(im.units);
  v.tiles = static_cast<uint32_t>(im.tiles);
  v.rec = im.rec;
  return v;
}

// Validation + layout of the image (no device). Returns 0 or an ABI status
// with a message in *why.
int32_t plan_image(int32_t qtype, int32_t layout, uint64_t k, uint64_t n, const void* blocks,
                   uint64_t count, Image* out, const char** why);
// Write the image into host memory of im.bytes bytes.
void fill_image(const Image& im, const void* blocks, void* out);
// GGUF wire blocks (`bytes` bytes) to logical blocks in `out` (resized), the
// block count in *count; legacy selects the old Q4_0 nibble pairs and Q6_K
// field order (others have one layout); QI_HIP_F32 passes f32 values through.
// Returns 0 or an ABI status with a message in *why.
int32_t gguf_decode(int32_t qtype, const void* wire, uint64_t bytes, int32_t legacy, void* out_vec,
                    uint64_t* count, const char** why);

// Tiled Q6_K record: byte position (0..15) of sub-scale i within a row's 16.
constexpr uint32_t q6_scale_pos(uint32_t i) {
  return 4 * (2 * (i / 8) + ((i % 8) % 4) / 2) + (i % 2) + 2 * ((i % 8) / 4);
}

}  // namespace qi
