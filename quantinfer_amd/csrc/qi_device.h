// Device-side block decoding shared by the dequantize, exact-order and GEMV
// kernels. Every translation unit is compiled with -ffp-contract=off: a
// multiply-add is fused only where fmaf() is written explicitly.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "qi_image.h"

namespace qi {

template <bool WIDE>
__device__ __forceinline__ float load_scale(const void* plane, uint64_t i) {
  if constexpr (WIDE) {
    return static_cast<const float*>(plane)[i];
  } else {
    return static_cast<float>(static_cast<const _Float16*>(plane)[i]);
  }
}

// 6-bit sub-block scale and min of a Q4_K/Q5_K block from its 12 packed bytes
// held as three little-endian words (backends/cpu/src/matmul.rs:192-201).
__device__ __forceinline__ void kquant_sc_m(uint32_t w0, uint32_t w1, uint32_t w2, int sub,
                                            uint32_t& sc, uint32_t& mn) {
  const int i = sub & 3;
  const uint32_t s_lo = (w0 >> (8 * i)) & 0xFFu;  // scales[i]
  const uint32_t m_lo = (w1 >> (8 * i)) & 0xFFu;  // scales[4 + i]
  if (sub < 4) {
    sc = s_lo & 63u;
    mn = m_lo & 63u;
  } else {
    const uint32_t hi = (w2 >> (8 * i)) & 0xFFu;  // scales[8 + i]
    sc = (hi & 15u) | ((s_lo >> 6) << 4);
    mn = (hi >> 4) | ((m_lo >> 6) << 4);
  }
}

// ---------------------------------------------------------------------------
// Block byte access for either image arrangement (planar or tiled records).

template <int QT>
struct Geo {
  static constexpr uint32_t kCode = QT == kQ8_0 ? 32 : QT == kQ4_0 ? 16 : 128;  // code bytes/block
  static constexpr uint32_t kQh = QT == kQ5_K ? 32 : QT == kQ6_K ? 64 : 0;
  static constexpr uint32_t kSc = (QT == kQ4_K || QT == kQ5_K) ? 12 : QT == kQ6_K ? 16 : 0;
  static constexpr uint32_t kBpu = (QT == kQ8_0 || QT == kQ4_0) ? 8 : 1;  // blocks per unit
  static constexpr uint32_t kSlice = kCode * kBpu;                          // code bytes/unit/row
};

struct BlockLoc {
  const uint8_t* rec;  // tiled: the record; planar: nullptr
  uint64_t blk;        // planar block index
  uint32_t col, bi;    // tiled: row within the tile, block within the unit
};

// Block b of output row n (output-rows layout), or flat block b (n = 0; row
// major, where a tiled image's record row is one k of v.nb blocks).
template <int QT>
__device__ __forceinline__ BlockLoc locate(const View& v, uint64_t n, uint64_t b) {
  BlockLoc L;
  if (v.tiled) {
    if (b >= v.nb) {
      n += b / v.nb;
      b %= v.nb;
    }
    const uint64_t u = b / Geo<QT>::kBpu;
    L.rec = v.qs + ((n / 16) * v.units + u) * v.rec.bytes;
    L.col = static_cast<uint32_t>(n % 16);
    L.bi = static_cast<uint32_t>(b % Geo<QT>::kBpu);
    L.blk = 0;
  } else {
    L.rec = nullptr;
    L.blk = n * v.nb + b;
    L.col = L.bi = 0;
  }
  return L;
}

template <int QT>
__device__ __forceinline__ uint8_t code_byte(const View& v, const BlockLoc& L, uint32_t o) {
  if (L.rec == nullptr) return v.qs[L.blk * Geo<QT>::kCode + o];
  const uint32_t s = L.bi * Geo<QT>::kCode + o, quarter = Geo<QT>::kSlice / 4;
  const uint32_t g = s / quarter, q = (s % quarter) / 16, r = s % 16;
  return L.rec[v.rec.qs + q * 1024 + (16 * g + L.col) * 16 + r];
}

template <int QT>
__device__ __forceinline__ uint8_t qh_byte(const View& v, const BlockLoc& L, uint32_t o) {
  if (L.rec == nullptr) return v.qh[L.blk * Geo<QT>::kQh + o];
  return L.rec[v.rec.qh + (o / 16) * 256 + L.col * 16 + o % 16];
}

template <int QT>
__device__ __forceinline__ uint8_t sc_byte(const View& v, const BlockLoc& L, uint32_t o) {
  if (L.rec == nullptr) return v.sc[L.blk * Geo<QT>::kSc + o];
  return L.rec[v.rec.sc + L.col * Geo<QT>::kSc + o];
}

template <int QT, bool WIDE>
__device__ __forceinline__ float scale_d(const View& v, const BlockLoc& L) {
  if (L.rec == nullptr) return load_scale<WIDE>(v.d, L.blk);
  return load_scale<WIDE>(L.rec + v.rec.d, L.col * Geo<QT>::kBpu + L.bi);
}

template <int QT, bool WIDE>
__device__ __forceinline__ float scale_dmin(const View& v, const BlockLoc& L) {
  if (L.rec == nullptr) return load_scale<WIDE>(v.dmin, L.blk);
  return load_scale<WIDE>(L.rec + v.rec.dmin, L.col);
}

// ---------------------------------------------------------------------------
// Exact per-element values: the reference's f32 operation sequence
// (backends/cpu/src/matmul.rs:162-280, identical to dequantize_* in
// quant/src/schemes). `L` locates the block, `l` is the element within it.

template <int QT, bool WIDE>
struct Exact;

template <bool WIDE>
struct Exact<kQ8_0, WIDE> {
  __device__ static float value(const View& v, const BlockLoc& L, uint32_t l) {
    const float d = scale_d<kQ8_0, WIDE>(v, L);
    const float q = static_cast<float>(static_cast<int8_t>(code_byte<kQ8_0>(v, L, l)));
    return d * q;  // matmul.rs:167
  }
};

template <bool WIDE>
struct Exact<kQ4_0, WIDE> {
  __device__ static float value(const View& v, const BlockLoc& L, uint32_t l) {
    const float d = scale_d<kQ4_0, WIDE>(v, L);
    const uint8_t byte = code_byte<kQ4_0>(v, L, l & 15);
    const uint32_t code = l < 16 ? (byte & 15u) : (byte >> 4);
    return d * (static_cast<float>(code) - 8.0f);  // matmul.rs:179
  }
};

// (sc, m) of sub-block `sub` of a Q4_K/Q5_K block: the reference's packed
// bytes in planar images, the lane-group field in tiled records (qi_image.h).
template <int QT>
__device__ __forceinline__ void kq_scale_min(const View& v, const BlockLoc& L, uint32_t sub,
                                             uint32_t& sc, uint32_t& mn) {
  if (L.rec == nullptr) {
    uint32_t w[3];
#pragma unroll
    for (int i = 0; i < 3; ++i)
      w[i] = static_cast<uint32_t>(sc_byte<QT>(v, L, 4 * i)) |
             (static_cast<uint32_t>(sc_byte<QT>(v, L, 4 * i + 1)) << 8) |
             (static_cast<uint32_t>(sc_byte<QT>(v, L, 4 * i + 2)) << 16) |
             (static_cast<uint32_t>(sc_byte<QT>(v, L, 4 * i + 3)) << 24);
    kquant_sc_m(w[0], w[1], w[2], static_cast<int>(sub), sc, mn);
    return;
  }
  const uint32_t g = sub / 2;
  const uint32_t f = static_cast<uint32_t>(sc_byte<QT>(v, L, 3 * g)) |
                     (static_cast<uint32_t>(sc_byte<QT>(v, L, 3 * g + 1)) << 8) |
                     (static_cast<uint32_t>(sc_byte<QT>(v, L, 3 * g + 2)) << 16);
  const uint32_t sh = (sub & 1) ? 12 : 0;
  sc = (f >> sh) & 63u;
  mn = (f >> (sh + 6)) & 63u;
}

template <int QT, bool WIDE>
__device__ __forceinline__ float exact_q45k(const View& v, const BlockLoc& L, uint32_t l) {
  uint32_t sc, mn;
  kq_scale_min<QT>(v, L, l / 32, sc, mn);
  const uint32_t group = l / 64, within = l % 64;
  const uint8_t packed = code_byte<QT>(v, L, group * 32 + within % 32);
  uint32_t q = within < 32 ? (packed & 15u) : (packed >> 4);
  if constexpr (QT == kQ5_K) {
    const uint32_t bit = within < 32 ? 2 * group : 2 * group + 1;
    if ((qh_byte<QT>(v, L, within % 32) >> bit) & 1u) q += 16;
  }
  const float d = scale_d<QT, WIDE>(v, L);
  const float dmin = scale_dmin<QT, WIDE>(v, L);
  // block.scale * f32(sc) * f32(q) - block.min_scale * f32(m)  (matmul.rs:211-214)
  return d * static_cast<float>(sc) * static_cast<float>(q) - dmin * static_cast<float>(mn);
}

template <bool WIDE>
struct Exact<kQ4_K, WIDE> {
  __device__ static float value(const View& v, const BlockLoc& L, uint32_t l) {
    return exact_q45k<kQ4_K, WIDE>(v, L, l);
  }
};

template <bool WIDE>
struct Exact<kQ5_K, WIDE> {
  __device__ static float value(const View& v, const BlockLoc& L, uint32_t l) {
    return exact_q45k<kQ5_K, WIDE>(v, L, l);
  }
};

template <bool WIDE>
struct Exact<kQ6_K, WIDE> {
  __device__ static float value(const View& v, const BlockLoc& L, uint32_t l) {
    const uint32_t ip = l / 128, within = l % 128, chunk = within / 32, il = within % 32;
    const uint8_t packed = code_byte<kQ6_K>(v, L, ip * 64 + ((chunk & 1) == 0 ? il : 32 + il));
    const uint32_t low = chunk < 2 ? (packed & 15u) : (packed >> 4);
    const uint32_t high = qh_byte<kQ6_K>(v, L, ip * 32 + il);
    const int32_t q = static_cast<int32_t>(low | (((high >> (chunk * 2)) & 3u) << 4));
    const uint32_t si = L.rec == nullptr ? l / 16 : q6_scale_pos(l / 16);
    const float sc = static_cast<float>(static_cast<int8_t>(sc_byte<kQ6_K>(v, L, si)));
    const float d = scale_d<kQ6_K, WIDE>(v, L);
    return d * sc * static_cast<float>(q - 32);  // matmul.rs:279
  }
};

// The CpuScalar sum of output n for one activation row x (k elements):
// acc = acc + x[k] * w(k) in f32, k ascending, no FMA (backends/cpu/src/
// matmul.rs:146-157, 319-330 output rows; :25-31 row major). The fast
// kernels call it for an output whose fast result is not finite: a NaN or
// infinite activation (or an overflow) then yields exactly the reference's
// value, where the fast arithmetic (digit splits, affine pieces, f16
// operands) cannot reproduce which outputs are NaN and which +-Inf.
template <int QT, bool WIDE>
__device__ __forceinline__ float exact_output_row(const View& w, const float* x, uint64_t n) {
  constexpr uint32_t bs = (QT == kQ8_0 || QT == kQ4_0) ? 32 : 256;
  float sum = 0.0f;
  for (uint32_t b = 0; b < w.nb; ++b) {
    const BlockLoc L = locate<QT>(w, n, b);
    const float* lb = x + static_cast<uint64_t>(b) * bs;
    // (a partial unroll: where n is wave-uniform, a full one would load a
    // whole block through scalar registers)
#pragma unroll 8
    for (uint32_t l = 0; l < bs; ++l) sum += lb[l] * Exact<QT, WIDE>::value(w, L, l);
  }
  return sum;
}

template <int QT, bool WIDE>
__device__ __forceinline__ float exact_row_major_col(const View& w, const float* x, uint64_t n) {
  constexpr uint32_t bs = (QT == kQ8_0 || QT == kQ4_0) ? 32 : 256;
  float sum = 0.0f;
  for (uint64_t k = 0; k < w.k; ++k) {
    // element (k, n): in a tiled image (N a multiple of 256) element n % bs of
    // block n / bs of record row k, else of flat block (k N + n) / bs
    const uint64_t f = w.tiled ? n : k * w.n + n;
    sum += x[k] * Exact<QT, WIDE>::value(w, locate<QT>(w, w.tiled ? k : 0, f / bs), static_cast<uint32_t>(f % bs));
  }
  return sum;
}

// ---------------------------------------------------------------------------
// Fast-path slot decoders (GEMV). A slot is the unit one lane handles per
// output row: 32 elements (Q8_0/Q4_0: one block) or 64 elements (K-quants:
// two sub-blocks of 32 / four of 16), split into 16-element pieces. Each
// piece has one affine scale: w = a*q - b with integer code q, so
//   sum_k x_k w_k = a * sum_k x_k q_k - b * sum_k x_k.
// This factoring reorders the reference arithmetic and is judged by tolerance.

__device__ __forceinline__ void nibbles16(uint4 src, int shift, float q[16]) {
  const uint32_t w[4] = {src.x, src.y, src.z, src.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t v = (w[i] >> shift) & 0x0F0F0F0Fu;
    q[4 * i + 0] = static_cast<float>(v & 0xFFu);
    q[4 * i + 1] = static_cast<float>((v >> 8) & 0xFFu);
    q[4 * i + 2] = static_cast<float>((v >> 16) & 0xFFu);
    q[4 * i + 3] = static_cast<float>(v >> 24);
  }
}

__device__ __forceinline__ void bytes16_u(uint4 src, float q[16]) {
  const uint32_t w[4] = {src.x, src.y, src.z, src.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    q[4 * i + 0] = static_cast<float>(w[i] & 0xFFu);
    q[4 * i + 1] = static_cast<float>((w[i] >> 8) & 0xFFu);
    q[4 * i + 2] = static_cast<float>((w[i] >> 16) & 0xFFu);
    q[4 * i + 3] = static_cast<float>(w[i] >> 24);
  }
}

__device__ __forceinline__ void bytes16_s(uint4 src, float q[16]) {
  const uint32_t w[4] = {src.x, src.y, src.z, src.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    q[4 * i + 0] = static_cast<float>(static_cast<int32_t>(w[i] << 24) >> 24);
    q[4 * i + 1] = static_cast<float>(static_cast<int32_t>(w[i] << 16) >> 24);
    q[4 * i + 2] = static_cast<float>(static_cast<int32_t>(w[i] << 8) >> 24);
    q[4 * i + 3] = static_cast<float>(static_cast<int32_t>(w[i]) >> 24);
  }
}

__device__ __forceinline__ uint4 or4(uint4 a, uint4 b) {
  return make_uint4(a.x | b.x, a.y | b.y, a.z | b.z, a.w | b.w);
}
__device__ __forceinline__ uint4 bits4(uint4 src, int shift, uint32_t mask, int up) {
  return make_uint4(((src.x >> shift) & mask) << up, ((src.y >> shift) & mask) << up,
                    ((src.z >> shift) & mask) << up, ((src.w >> shift) & mask) << up);
}

template <int QT, bool WIDE>
struct Fast;

template <bool WIDE>
struct Fast<kQ8_0, WIDE> {
  static constexpr int kSlotElems = 32, kPieces = 2;
  static constexpr bool kHasMin = false;
  struct Slot {
    uint4 q0, q1;
    float a;
  };
  __device__ static void load(const View& v, uint64_t row, uint32_t s, Slot& o) {
    const uint64_t blk = row * v.nb + s;
    const uint4* p = reinterpret_cast<const uint4*>(v.qs + blk * 32);
    o.q0 = p[0];
    o.q1 = p[1];
    o.a = load_scale<WIDE>(v.d, blk);
  }
  __device__ static uint32_t x_offset(uint32_t s, int p) { return s * 32 + 16 * p; }
  __device__ static void codes(const Slot& o, int p, float q[16]) { bytes16_s(p ? o.q1 : o.q0, q); }
  __device__ static float a(const Slot& o, int) { return o.a; }
  __device__ static float b(const Slot&, int) { return 0.0f; }
};

template <bool WIDE>
struct Fast<kQ4_0, WIDE> {
  static constexpr int kSlotElems = 32, kPieces = 2;
  // the offset enters the codes (q - 8, exact small integers), not a separate
  // -8d * sum(x) term: a*sum(x q) - 8a*sum(x) cancels when the codes sit near
  // 8, which costs f32 bits the reference's sum of x * d(q - 8) keeps
  static constexpr bool kHasMin = false;
  struct Slot {
    uint4 q;
    float a;
  };
  __device__ static void load(const View& v, uint64_t row, uint32_t s, Slot& o) {
    const uint64_t blk = row * v.nb + s;
    o.q = *reinterpret_cast<const uint4*>(v.qs + blk * 16);
    o.a = load_scale<WIDE>(v.d, blk);
  }
  // byte j holds element j (low nibble) and j+16 (high nibble)
  __device__ static uint32_t x_offset(uint32_t s, int p) { return s * 32 + 16 * p; }
  __device__ static void codes(const Slot& o, int p, float q[16]) {
    nibbles16(o.q, p ? 4 : 0, q);
#pragma unroll
    for (int j = 0; j < 16; ++j) q[j] -= 8.0f;
  }
  __device__ static float a(const Slot& o, int) { return o.a; }
  __device__ static float b(const Slot&, int) { return 0.0f; }
};

// Q4_K / Q5_K slot s = (super-block s/4, group g = s%4): 32 code bytes
// qs[32g, 32g+32) cover elements 64g + [0, 64): low nibbles -> sub-block 2g,
// high nibbles -> sub-block 2g+1. Q5_K adds bit 2g / 2g+1 of qh[0..32).
template <bool WIDE, bool FIVE>
struct FastQ45K {
  static constexpr int kSlotElems = 64, kPieces = 4;
  static constexpr bool kHasMin = true;
  struct Slot {
    uint4 q0, q1;
    uint4 h0, h1;
    float a_lo, b_lo, a_hi, b_hi;
    uint32_t g;
  };
  __device__ static void load(const View& v, uint64_t row, uint32_t s, Slot& o) {
    const uint32_t sb = s >> 2, g = s & 3;
    const uint64_t blk = row * v.nb + sb;
    const uint4* p = reinterpret_cast<const uint4*>(v.qs + blk * 128 + g * 32);
    o.q0 = p[0];
    o.q1 = p[1];
    if constexpr (FIVE) {
      const uint4* h = reinterpret_cast<const uint4*>(v.qh + blk * 32);
      o.h0 = h[0];
      o.h1 = h[1];
    }
    const uint32_t* scw = reinterpret_cast<const uint32_t*>(v.sc + blk * 12);
    const uint32_t w0 = scw[0], w1 = scw[1], w2 = scw[2];
    uint32_t sc_lo, m_lo, sc_hi, m_hi;
    kquant_sc_m(w0, w1, w2, static_cast<int>(2 * g), sc_lo, m_lo);
    kquant_sc_m(w0, w1, w2, static_cast<int>(2 * g + 1), sc_hi, m_hi);
    const float d = load_scale<WIDE>(v.d, blk);
    const float dmin = load_scale<WIDE>(v.dmin, blk);
    o.a_lo = d * static_cast<float>(sc_lo);
    o.b_lo = dmin * static_cast<float>(m_lo);
    o.a_hi = d * static_cast<float>(sc_hi);
    o.b_hi = dmin * static_cast<float>(m_hi);
    o.g = g;
  }
  __device__ static uint32_t x_offset(uint32_t s, int p) {
    return (s >> 2) * 256 + (s & 3) * 64 + 16 * p;
  }
  __device__ static void codes(const Slot& o, int p, float q[16]) {
    // pieces: 0 = low nibbles of bytes 0-15, 1 = low of 16-31,
    //         2 = high nibbles of bytes 0-15, 3 = high of 16-31
    uint4 src = (p & 1) ? o.q1 : o.q0;
    const int shift = p >= 2 ? 4 : 0;
    uint4 v = make_uint4((src.x >> shift) & 0x0F0F0F0Fu, (src.y >> shift) & 0x0F0F0F0Fu,
                         (src.z >> shift) & 0x0F0F0F0Fu, (src.w >> shift) & 0x0F0F0F0Fu);
    if constexpr (FIVE) {
      // fifth bit: bit 2g (low nibbles) or 2g+1 (high nibbles) of qh[i], to bit 4
      const uint4 h = (p & 1) ? o.h1 : o.h0;
      v = or4(v, bits4(h, static_cast<int>(2 * o.g) + (p >= 2 ? 1 : 0), 0x01010101u, 4));
    }
    bytes16_u(v, q);
  }
  __device__ static float a(const Slot& o, int p) { return p >= 2 ? o.a_hi : o.a_lo; }
  __device__ static float b(const Slot& o, int p) { return p >= 2 ? o.b_hi : o.b_lo; }
};

template <bool WIDE>
struct Fast<kQ4_K, WIDE> : FastQ45K<WIDE, false> {};
template <bool WIDE>
struct Fast<kQ5_K, WIDE> : FastQ45K<WIDE, true> {};

// Q6_K slot s = (super-block s/4, ip = (s%4)/2, c = s%2): ql bytes
// [64ip + 32c, +32) and qh bytes [32ip, +32) cover elements
// 128ip + 32c + [0, 32) (low nibbles, qh bits 2c) and 128ip + 32c + 64 + [0, 32)
// (high nibbles, qh bits 2c+4); each 16-element piece is one int8 sub-scale.
template <bool WIDE>
struct Fast<kQ6_K, WIDE> {
  static constexpr int kSlotElems = 64, kPieces = 4;
  static constexpr bool kHasMin = true;
  struct Slot {
    uint4 q0, q1, h0, h1;
    float a[4];
    uint32_t c;
  };
  __device__ static void load(const View& v, uint64_t row, uint32_t s, Slot& o) {
    const uint32_t sb = s >> 2, ip = (s >> 1) & 1, c = s & 1;
    const uint64_t blk = row * v.nb + sb;
    const uint4* p = reinterpret_cast<const uint4*>(v.qs + blk * 128 + ip * 64 + c * 32);
    o.q0 = p[0];
    o.q1 = p[1];
    const uint4* h = reinterpret_cast<const uint4*>(v.qh + blk * 64 + ip * 32);
    o.h0 = h[0];
    o.h1 = h[1];
    o.c = c;
    // sub-scales 8ip + 2c + {0, 1, 4, 5}
    const uint2 scv = *reinterpret_cast<const uint2*>(v.sc + blk * 16 + ip * 8);
    const uint32_t lo = c ? (scv.x >> 16) : scv.x;   // bytes 2c, 2c+1
    const uint32_t hi = c ? (scv.y >> 16) : scv.y;   // bytes 2c+4, 2c+5
    const float d = load_scale<WIDE>(v.d, blk);
    o.a[0] = d * static_cast<float>(static_cast<int8_t>(lo & 0xFFu));
    o.a[1] = d * static_cast<float>(static_cast<int8_t>((lo >> 8) & 0xFFu));
    o.a[2] = d * static_cast<float>(static_cast<int8_t>(hi & 0xFFu));
    o.a[3] = d * static_cast<float>(static_cast<int8_t>((hi >> 8) & 0xFFu));
  }
  __device__ static uint32_t x_offset(uint32_t s, int p) {
    const uint32_t sb = s >> 2, ip = (s >> 1) & 1, c = s & 1;
    return sb * 256 + ip * 128 + c * 32 + (p >= 2 ? 64 : 0) + 16 * (p & 1);
  }
  __device__ static void codes(const Slot& o, int p, float q[16]) {
    const uint4 src = (p & 1) ? o.q1 : o.q0;
    const uint4 h = (p & 1) ? o.h1 : o.h0;
    const int shift = p >= 2 ? 4 : 0;
    const int hs = 2 * static_cast<int>(o.c) + (p >= 2 ? 4 : 0);
    const uint4 v = or4(bits4(src, shift, 0x0F0F0F0Fu, 0), bits4(h, hs, 0x03030303u, 4));
    bytes16_u(v, q);
  }
  __device__ static float a(const Slot& o, int p) { return o.a[p]; }
  __device__ static float b(const Slot& o, int p) { return 32.0f * o.a[p]; }
};

// ---------------------------------------------------------------------------
// Wavefront (64-lane) sum with DPP row operations, then the four row sums.
__device__ __forceinline__ float wave_sum(float v) {
  v += __builtin_amdgcn_update_dpp(0.0f, v, 0xB1, 0xF, 0xF, false);   // quad_perm [1,0,3,2]
  v += __builtin_amdgcn_update_dpp(0.0f, v, 0x4E, 0xF, 0xF, false);   // quad_perm [2,3,0,1]
  v += __builtin_amdgcn_update_dpp(0.0f, v, 0x141, 0xF, 0xF, false);  // row_half_mirror
  v += __builtin_amdgcn_update_dpp(0.0f, v, 0x140, 0xF, 0xF, false);  // row_mirror
  const float r0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 0));
  const float r1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 16));
  const float r2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 32));
  const float r3 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 48));
  return (r0 + r1) + (r2 + r3);
}

}  // namespace qi
