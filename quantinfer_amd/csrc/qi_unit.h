// Per-format access to one unit (256 elements) of one output row of a tiled
// weight record, shared by the matrix-core GEMV and GEMM: a wavefront's lane
// 16g + c loads row c's lane-group-g bytes of the record (layout in
// qi_image.h), decodes the affine scales of its windows and hands out, per
// step t (0..7), the 8 codes of elements window_first(g, t / 4) + 8 (t % 4) +
// [0, 8) as bytes (Q8_0 signed, the other formats unsigned).
#pragma once
#include "qi_device.h"

namespace qi {
// 16 bytes of weight codes. NT: a non-temporal (streaming) load, for kernels
// that read every weight byte once (the GEMV: 3.97-4.02 against 3.73-3.84
// TB/s at Q4_K 4096 x 14336 on MI355X, alternating runs); the GEMMs re-read a
// weight tile for every row block and keep ordinary loads.
template <bool NT>
__device__ __forceinline__ uint4 ld_codes(const uint4* p) {
  static_assert(NT, "ordinary loads index the record directly");
  typedef unsigned int v4 __attribute__((ext_vector_type(4)));
  const v4 v = __builtin_nontemporal_load(reinterpret_cast<const v4*>(p));
  return make_uint4(v.x, v.y, v.z, v.w);
}


template <int QT>
struct Unit;  // per-format code/scale access for one (output n, lane group g, unit u)

// Loads read one (tile, unit) record (layout in qi_image.h): lane 16g + c
// takes row c's lane-group-g code chunks at q*1024 + lane*16 (each wavefront
// load is 1 KB contiguous), its scales from the record's scale sections.

template <>
struct Unit<kQ8_0> {
  static constexpr int kWindows = 2, kSteps = 4;  // two 32-element blocks per lane
  static constexpr bool kMin = false;
  struct Raw {
    uint4 q[4];
    uint32_t s0, s1;  // f16 pair in s0, or two f32 scales
  };
  template <bool W, bool NT = false>
  __device__ static void load(const uint8_t* rec, uint32_t lane, Raw& r) {
    constexpr Record R = record_geometry(kQ8_0, W);
    const uint4* p = reinterpret_cast<const uint4*>(rec + R.qs) + lane;
    if constexpr (NT) {
      r.q[0] = ld_codes<true>(p); r.q[1] = ld_codes<true>(p + 64);
      r.q[2] = ld_codes<true>(p + 128); r.q[3] = ld_codes<true>(p + 192);
    } else {
      r.q[0] = p[0]; r.q[1] = p[64]; r.q[2] = p[128]; r.q[3] = p[192];
    }
    const uint32_t e = (lane & 15) * 8 + 2 * (lane >> 4);  // blocks 2g, 2g+1 of row c
    if constexpr (W) {
      const uint2 d = *reinterpret_cast<const uint2*>(rec + R.d + e * 4);
      r.s0 = d.x; r.s1 = d.y;
    } else {
      r.s0 = *reinterpret_cast<const uint32_t*>(rec + R.d + e * 2);
      r.s1 = 0;
    }
  }
  template <bool W>
  __device__ static void scales(uint32_t, const Raw& r, float a[2], float b[2]) {
    if constexpr (W) {
      a[0] = __builtin_bit_cast(float, r.s0);
      a[1] = __builtin_bit_cast(float, r.s1);
    } else {
      a[0] = static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(r.s0 & 0xFFFFu)));
      a[1] = static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(r.s0 >> 16)));
    }
    b[0] = b[1] = 0.0f;
  }
  // step t (0..7): block h = t/4, bytes 8*(t%4) .. +8 of that block
  __device__ static long codes(const Raw& r, uint32_t, int t) {
    const uint4 q = r.q[(t >> 2) * 2 + ((t & 3) >> 1)];
    const uint32_t lo = (t & 1) ? q.z : q.x, hi = (t & 1) ? q.w : q.y;
    return static_cast<long>((static_cast<uint64_t>(hi) << 32) | lo);
  }
};

template <>
struct Unit<kQ4_0> {
  static constexpr int kWindows = 2, kSteps = 4;
  static constexpr bool kMin = true;  // w = d*q - 8d
  struct Raw {
    uint4 q[2];
    uint32_t s0, s1;
  };
  template <bool W, bool NT = false>
  __device__ static void load(const uint8_t* rec, uint32_t lane, Raw& r) {
    constexpr Record R = record_geometry(kQ4_0, W);
    const uint4* p = reinterpret_cast<const uint4*>(rec + R.qs) + lane;
    if constexpr (NT) {
      r.q[0] = ld_codes<true>(p); r.q[1] = ld_codes<true>(p + 64);
    } else {
      r.q[0] = p[0]; r.q[1] = p[64];
    }
    const uint32_t e = (lane & 15) * 8 + 2 * (lane >> 4);
    if constexpr (W) {
      const uint2 d = *reinterpret_cast<const uint2*>(rec + R.d + e * 4);
      r.s0 = d.x; r.s1 = d.y;
    } else {
      r.s0 = *reinterpret_cast<const uint32_t*>(rec + R.d + e * 2);
      r.s1 = 0;
    }
  }
  template <bool W>
  __device__ static void scales(uint32_t, const Raw& r, float a[2], float b[2]) {
    if constexpr (W) {
      a[0] = __builtin_bit_cast(float, r.s0);
      a[1] = __builtin_bit_cast(float, r.s1);
    } else {
      a[0] = static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(r.s0 & 0xFFFFu)));
      a[1] = static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(r.s0 >> 16)));
    }
    b[0] = 8.0f * a[0];
    b[1] = 8.0f * a[1];
  }
  // block h = t/4 (16 bytes: byte i = element i | element i+16 << 4);
  // quarter t%4: 0 = low nibbles of bytes 0-7, 1 = low of 8-15, 2 = high of 0-7, 3 = high of 8-15
  __device__ static long codes(const Raw& r, uint32_t, int t) {
    const uint4 q = r.q[t >> 2];
    const int qq = t & 3;
    const uint32_t lo = (qq & 1) ? q.z : q.x, hi = (qq & 1) ? q.w : q.y;
    const int sh = qq >= 2 ? 4 : 0;
    const uint32_t l2 = (lo >> sh) & 0x0F0F0F0Fu, h2 = (hi >> sh) & 0x0F0F0F0Fu;
    return static_cast<long>((static_cast<uint64_t>(h2) << 32) | l2);
  }
  // the same codes as 16 (q - 8), signed bytes: with bit 3 of each nibble
  // flipped, the nibble is q - 8 in 4-bit two's complement, and in the high
  // half of a byte it reads as 16 times that
  __device__ static long centred_codes(const Raw& r, uint32_t, int t) {
    const uint4 q = r.q[t >> 2];
    const int qq = t & 3;
    const uint32_t lo = ((qq & 1) ? q.z : q.x) ^ 0x88888888u, hi = ((qq & 1) ? q.w : q.y) ^ 0x88888888u;
    const uint32_t l2 = (qq >= 2 ? lo : lo << 4) & 0xF0F0F0F0u, h2 = (qq >= 2 ? hi : hi << 4) & 0xF0F0F0F0u;
    return static_cast<long>((static_cast<uint64_t>(h2) << 32) | l2);
  }
};

// Q4_K / Q5_K: lane group g holds code bytes [32g, 32g+32) of the super-block:
// step t < 4 takes the low nibbles of bytes 8t..8t+7 (sub-block 2g), t >= 4 the
// high nibbles of bytes 8(t-4).. (sub-block 2g+1); Q5_K adds bit 2g (low) or
// 2g+1 (high) of qh[byte] as bit 4.
template <bool FIVE>
struct UnitQ45K {
  static constexpr int kQT = FIVE ? kQ5_K : kQ4_K;
  static constexpr int kWindows = 2, kSteps = 4;
  static constexpr bool kMin = true;
  struct Raw {
    uint4 q[2];
    uint4 h[2];
    uint32_t sc[3];
    uint32_t s0, s1;  // d and dmin: f16 bits (zero-extended) or f32 bits
  };
  template <bool W, bool NT = false>
  __device__ static void load(const uint8_t* rec, uint32_t lane, Raw& r) {
    constexpr Record R = record_geometry(kQT, W);
    const uint32_t col = lane & 15;
    const uint4* p = reinterpret_cast<const uint4*>(rec + R.qs) + lane;
    if constexpr (NT) {
      r.q[0] = ld_codes<true>(p); r.q[1] = ld_codes<true>(p + 64);
    } else {
      r.q[0] = p[0]; r.q[1] = p[64];
    }
    if constexpr (FIVE) {
      const uint4* h = reinterpret_cast<const uint4*>(rec + R.qh) + col;
      r.h[0] = h[0]; r.h[1] = h[16];
    }
    const uint32_t* s = reinterpret_cast<const uint32_t*>(rec + R.sc + col * 12);
    r.sc[0] = s[0]; r.sc[1] = s[1]; r.sc[2] = s[2];
    if constexpr (W) {
      r.s0 = reinterpret_cast<const uint32_t*>(rec + R.d)[col];
      r.s1 = reinterpret_cast<const uint32_t*>(rec + R.dmin)[col];
    } else {
      // kept apart until scales(): combining them here would wait for the loads
      r.s0 = reinterpret_cast<const uint16_t*>(rec + R.d)[col];
      r.s1 = reinterpret_cast<const uint16_t*>(rec + R.dmin)[col];
    }
  }
  // the super-block's d and dmin
  template <bool W>
  __device__ static void dmins(const Raw& r, float& d, float& dmin) {
    if constexpr (W) {
      d = __builtin_bit_cast(float, r.s0);
      dmin = __builtin_bit_cast(float, r.s1);
    } else {
      d = static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(r.s0)));
      dmin = static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(r.s1)));
    }
  }
  // lane group g's 24-bit field sc[2g] | m[2g] << 6 | sc[2g+1] << 12 |
  // m[2g+1] << 18, at bytes 3g..3g+2 of the 12 scale bytes: one byte permute
  // from the word pair that holds it
  __device__ static uint32_t field(uint32_t g, const Raw& r) {
    const uint32_t lo = g < 2 ? r.sc[0] : r.sc[1];
    const uint32_t hi = g < 2 ? r.sc[1] : r.sc[2];
    const uint32_t first = (0x5230u >> (4 * g)) & 15u;  // g = 0..3: bytes 0, 3, 2, 5 (no branch)
    return __builtin_amdgcn_perm(hi, lo, first * 0x00010101u + 0x0C020100u);
  }
  template <bool W>
  __device__ static void scales(uint32_t g, const Raw& r, float a[2], float b[2]) {
    float d, dmin;
    dmins<W>(r, d, dmin);
    const uint32_t f = field(g, r);
    a[0] = d * static_cast<float>(f & 63u);
    b[0] = dmin * static_cast<float>((f >> 6) & 63u);
    a[1] = d * static_cast<float>((f >> 12) & 63u);
    b[1] = dmin * static_cast<float>(f >> 18);
  }
  __device__ static long codes(const Raw& r, uint32_t g, int t) {
    const int tt = t & 3;
    const uint4 q = r.q[tt >> 1];
    const uint32_t lo = (tt & 1) ? q.z : q.x, hi = (tt & 1) ? q.w : q.y;
    const int sh = t >= 4 ? 4 : 0;
    uint32_t l2 = (lo >> sh) & 0x0F0F0F0Fu, h2 = (hi >> sh) & 0x0F0F0F0Fu;
    if constexpr (FIVE) {
      const uint4 h = r.h[tt >> 1];
      const uint32_t hl = (tt & 1) ? h.z : h.x, hh = (tt & 1) ? h.w : h.y;
      const int bit = static_cast<int>(2 * g) + (t >= 4 ? 1 : 0);
      l2 |= ((hl >> bit) & 0x01010101u) << 4;
      h2 |= ((hh >> bit) & 0x01010101u) << 4;
    }
    return static_cast<long>((static_cast<uint64_t>(h2) << 32) | l2);
  }
  // The same codes centred, as signed bytes. Q4_K: 16 (q - 8), the nibble
  // with bit 3 flipped (q - 8 in 4-bit two's complement) in the byte's high
  // half. Q5_K: 8 (q - 16), the nibble in bits 3-6 and the high bit in bit 7
  // (disjoint, so joined by xor), bit 7 flipped (subtracting 128 = 8 * 16).
  __device__ static long centred_codes(const Raw& r, uint32_t g, int t) {
    const int tt = t & 3;
    const uint4 q = r.q[tt >> 1];
    const uint32_t lo = (tt & 1) ? q.z : q.x, hi = (tt & 1) ? q.w : q.y;
    uint32_t l2, h2;
    if constexpr (FIVE) {
      const uint4 h = r.h[tt >> 1];
      const uint32_t hl = (tt & 1) ? h.z : h.x, hh = (tt & 1) ? h.w : h.y;
      const int up = 7 - static_cast<int>(2 * g) - (t >= 4 ? 1 : 0);  // 7 - (bit of the pair)
      const uint32_t nl = (t >= 4 ? lo >> 1 : lo << 3) & 0x78787878u, nh = (t >= 4 ? hi >> 1 : hi << 3) & 0x78787878u;
      l2 = nl ^ ((hl << up) & 0x80808080u) ^ 0x80808080u;
      h2 = nh ^ ((hh << up) & 0x80808080u) ^ 0x80808080u;
    } else {
      const uint32_t fl = lo ^ 0x88888888u, fh = hi ^ 0x88888888u;
      l2 = (t >= 4 ? fl : fl << 4) & 0xF0F0F0F0u;
      h2 = (t >= 4 ? fh : fh << 4) & 0xF0F0F0F0u;
    }
    return static_cast<long>((static_cast<uint64_t>(h2) << 32) | l2);
  }
};

template <>
struct Unit<kQ4_K> : UnitQ45K<false> {};
template <>
struct Unit<kQ5_K> : UnitQ45K<true> {};

// Four Q6_K codes as 4 (q - 32) in signed bytes, from the low nibbles placed
// in bits 2-5 of `n` and the two high bits in bits 6-7 of `h` (the other bits
// of both are ignored): 4q takes bits 2-5 from n and 6-7 from h (one bit
// select), and clearing bits 0-1 while flipping bit 7 (subtracting 128 =
// 4 * 32) is one more bitwise operation.
__device__ __forceinline__ uint32_t q6_centred(uint32_t n, uint32_t h) {
  const uint32_t v = (n & 0x3C3C3C3Cu) | (h & ~0x3C3C3C3Cu);
  return (v & 0xFCFCFCFCu) ^ 0x80808080u;
}

// Q6_K: lane group g = 2*ip + c holds ql bytes [64ip + 32c, +32) and qh bytes
// [32ip, +32). Step t < 4: low nibbles of ql bytes 8t.. with qh bits 2c (elements
// 128ip + 32c + 8t + j); t >= 4: high nibbles of ql bytes 8(t-4).. with qh bits
// 2c+4 (elements 128ip + 32c + 64 + 8(t-4) + j). Windows are pairs of steps
// (16-element sub-blocks 8ip + 2c + {0, 1, 4, 5}); w = a*q - 32a.
template <>
struct Unit<kQ6_K> {
  static constexpr int kWindows = 4, kSteps = 2;
  static constexpr bool kMin = true;
  struct Raw {
    uint4 q[2];
    uint4 h[2];
    uint32_t sc;  // this lane group's four int8 sub-scales
    uint32_t d;   // f16 in the low half, or f32
  };
  template <bool W, bool NT = false>
  __device__ static void load(const uint8_t* rec, uint32_t lane, Raw& r) {
    constexpr Record R = record_geometry(kQ6_K, W);
    const uint32_t col = lane & 15, ip = lane >> 5;
    const uint4* p = reinterpret_cast<const uint4*>(rec + R.qs) + lane;
    if constexpr (NT) {
      r.q[0] = ld_codes<true>(p); r.q[1] = ld_codes<true>(p + 64);
    } else {
      r.q[0] = p[0]; r.q[1] = p[64];
    }
    const uint4* h = reinterpret_cast<const uint4*>(rec + R.qh) + 32 * ip + col;
    r.h[0] = h[0]; r.h[1] = h[16];
    r.sc = *reinterpret_cast<const uint32_t*>(rec + R.sc + col * 16 + 4 * (lane >> 4));
    if constexpr (W) r.d = reinterpret_cast<const uint32_t*>(rec + R.d)[col];
    else r.d = reinterpret_cast<const uint16_t*>(rec + R.d)[col];
  }
  template <bool W>
  __device__ static void scales(uint32_t, const Raw& r, float a[4], float b[4]) {
    float d;
    if constexpr (W) d = __builtin_bit_cast(float, r.d);
    else d = static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(r.d)));
    // sub-scales 8ip + 2c + {0, 1, 4, 5} of lane group g = 2ip + c
#pragma unroll
    for (int i = 0; i < 4; ++i)
      a[i] = d * static_cast<float>(static_cast<int32_t>(r.sc << (24 - 8 * i)) >> 24);
#pragma unroll
    for (int i = 0; i < 4; ++i) b[i] = 32.0f * a[i];
  }
  __device__ static long codes(const Raw& r, uint32_t g, int t) {
    const int tt = t & 3;
    const uint4 q = r.q[tt >> 1];
    const uint4 h = r.h[tt >> 1];
    const uint32_t lo = (tt & 1) ? q.z : q.x, hi = (tt & 1) ? q.w : q.y;
    const uint32_t hl = (tt & 1) ? h.z : h.x, hh = (tt & 1) ? h.w : h.y;
    const int sh = t >= 4 ? 4 : 0;
    const int hs = 2 * static_cast<int>(g & 1) + (t >= 4 ? 4 : 0);
    const uint32_t l2 = ((lo >> sh) & 0x0F0F0F0Fu) | (((hl >> hs) & 0x03030303u) << 4);
    const uint32_t h2 = ((hi >> sh) & 0x0F0F0F0Fu) | (((hh >> hs) & 0x03030303u) << 4);
    return static_cast<long>((static_cast<uint64_t>(h2) << 32) | l2);
  }
  // the same codes as 4 (q - 32), signed bytes (q6_centred)
  __device__ static long centred_codes(const Raw& r, uint32_t g, int t) {
    const int tt = t & 3;
    const uint4 q = r.q[tt >> 1];
    const uint4 h = r.h[tt >> 1];
    const uint32_t lo = (tt & 1) ? q.z : q.x, hi = (tt & 1) ? q.w : q.y;
    const uint32_t hl = (tt & 1) ? h.z : h.x, hh = (tt & 1) ? h.w : h.y;
    const int hs = 6 - 2 * static_cast<int>(g & 1) - (t >= 4 ? 4 : 0);  // 6 - (bit of the pair)
    const uint32_t l2 = q6_centred(t >= 4 ? lo >> 2 : lo << 2, hl << hs);
    const uint32_t h2 = q6_centred(t >= 4 ? hi >> 2 : hi << 2, hh << hs);
    return static_cast<long>((static_cast<uint64_t>(h2) << 32) | l2);
  }
};

// First unit element of window (g, h): Q6_K lane group g = 2*ip + c holds
// elements 128ip + 32c + [0, 32) (h = 0) and + 64 (h = 1); the other formats'
// lane group g holds elements 64g + [0, 64).
template <int QT>
__device__ __forceinline__ uint32_t window_first(uint32_t g, uint32_t h) {
  if constexpr (QT == kQ6_K) return 128 * (g >> 1) + 32 * (g & 1) + 64 * h;
  return 64 * g + 32 * h;
}

// Code centring of the decode GEMVs. With w = a q - b they compute
// a * sum x (q - z) - (b - a z) * sum x with the integer dot products of
// (q - z) exact, so that a sum x q and b sum x, of similar size, do not cancel
// in f32 (they cancelled to below their own rounding at small K).
// - The one-row kernel takes the codes centred on the middle of their range,
//   z = code_centre, as c (q - z) in signed bytes (centred_codes, c =
//   code_scale: 16 for Q4_0 and Q4_K, 8 for Q5_K, 4 for Q6_K), and scales
//   its sums back by 1 / c at the end (a power of two: exact). Q4_0 (b = 8a)
//   and Q6_K (b = 32a) are left with no offset; Q4_K and Q5_K with b - z a,
//   over a window sum added pairwise.
// - The 2-16 row kernel, which subtracts all offsets once at the end, centres
//   Q4_0 the same way and Q4_K / Q5_K on a zero point per output and window
//   (window_zero_point), subtracted by the matrix cores themselves: a second
//   instruction on the same activations with -z in every byte of B.
// - Q8_0: signed codes, no offset.
template <int QT>
constexpr int code_centre() {
  return QT == kQ4_0 || QT == kQ4_K ? 8 : QT == kQ5_K ? 16 : QT == kQ6_K ? 32 : 0;
}
template <int QT>
constexpr int code_scale() {
  return QT == kQ4_0 || QT == kQ4_K ? 16 : QT == kQ5_K ? 8 : QT == kQ6_K ? 4 : 1;
}
template <int QT>
constexpr bool window_centered() {
  return QT == kQ4_K || QT == kQ5_K;
}
// The codes of step t as the GEMV's matrix instructions take them.
template <int QT>
__device__ __forceinline__ long gemv_codes(const typename Unit<QT>::Raw& r, uint32_t g, int t) {
  if constexpr (code_scale<QT>() != 1) return Unit<QT>::centred_codes(r, g, t);
  else return Unit<QT>::codes(r, g, t);
}
// A lane's value moved by a DPP pattern (all lanes of the wavefront active):
// kDppSwap1 from lane i ^ 1, kDppRor4 / kDppRor8 from lane (i + 4) / (i + 8)
// mod 16 within each row of 16 lanes. VALU operand modifiers, no LDS round
// trip (unlike __shfl_xor).
constexpr int kDppSwap1 = 0xB1;  // quad_perm [1, 0, 3, 2]
constexpr int kDppRor4 = 0x124;  // row_ror:4
constexpr int kDppRor8 = 0x128;  // row_ror:8
template <int CTRL>
__device__ __forceinline__ float dpp_move(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}

// Zero point of an affine window (w = a q - b), as a float holding an
// integer: the integer nearest b / a (by the hardware reciprocal, so within
// one of it), clamped to [-127, 127] so that -z is an int8. Any integer keeps
// the centring exact; one near b / a leaves an offset b - z a of about a / 2
// at most. (a = 0 gives an infinite or NaN quotient; the clamps, which return
// their other operand for NaN, map both into the range.)
__device__ __forceinline__ float window_zero_point(float a, float b) {
  return fminf(fmaxf(rintf(b * __builtin_amdgcn_rcpf(a)), -127.0f), 127.0f);
}

// Weight access of one unit for the 2-16 row GEMVs: the one-row loaders,
// except that Q5_K loads only the 8 qh bytes of slice g (not all 32 of the
// output), which keeps the 16-wavefront register budget, and Q6_K (below).
template <int QT>
struct RowsUnit : Unit<QT> {};

template <>
struct RowsUnit<kQ5_K> {
  static constexpr bool kMin = true;
  struct Raw {
    uint4 q[2];
    uint32_t hl, hh;  // qh bytes 8g..8g+7 of this output
    uint32_t sc[3];
    uint32_t s0, s1;
  };
  template <bool W, bool NT>
  __device__ static void load(const uint8_t* rec, uint32_t lane, Raw& r) {
    constexpr Record R = record_geometry(kQ5_K, W);
    const uint32_t col = lane & 15, g = lane >> 4;
    const uint4* p = reinterpret_cast<const uint4*>(rec + R.qs) + lane;
    r.q[0] = ld_codes<true>(p);
    r.q[1] = ld_codes<true>(p + 64);
    // 16-byte chunk g / 2 of row col's qh, its half g % 2
    const uint2 h = *reinterpret_cast<const uint2*>(rec + R.qh + (g >> 1) * 256 + col * 16 + (g & 1) * 8);
    r.hl = h.x;
    r.hh = h.y;
    const uint32_t* s = reinterpret_cast<const uint32_t*>(rec + R.sc + col * 12);
    r.sc[0] = s[0];
    r.sc[1] = s[1];
    r.sc[2] = s[2];
    if constexpr (W) {
      r.s0 = reinterpret_cast<const uint32_t*>(rec + R.d)[col];
      r.s1 = reinterpret_cast<const uint32_t*>(rec + R.dmin)[col];
    } else {
      r.s0 = reinterpret_cast<const uint16_t*>(rec + R.d)[col];
      r.s1 = reinterpret_cast<const uint16_t*>(rec + R.dmin)[col];
    }
  }
  template <bool W>
  __device__ static void scales(uint32_t g, const Raw& r, float a[2], float b[2]) {
    typename Unit<kQ5_K>::Raw u;
    u.sc[0] = r.sc[0];
    u.sc[1] = r.sc[1];
    u.sc[2] = r.sc[2];
    u.s0 = r.s0;
    u.s1 = r.s1;
    Unit<kQ5_K>::template scales<W>(g, u, a, b);
  }
};

// Q6_K: the ql chunks as the one-row kernel loads them; the qh bytes of slice
// g of both halves (bytes 8g..8g+7 of 32ip + [0, 32), ip = 0, 1) instead of
// the lane group's own 32, and the row's 16 sub-scales (tiled order,
// q6_scale_pos: window w's two at bytes 2hf, 2hf + 1 of word 2ip + c).
template <>
struct RowsUnit<kQ6_K> {
  struct Raw {
    uint4 q[2];
    uint32_t h[4];
    uint4 sc;
    uint32_t d;  // f16 in the low half, or f32
  };
  template <bool W, bool NT>
  __device__ static void load(const uint8_t* rec, uint32_t lane, Raw& r) {
    constexpr Record R = record_geometry(kQ6_K, W);
    const uint32_t col = lane & 15, g = lane >> 4;
    const uint4* p = reinterpret_cast<const uint4*>(rec + R.qs) + lane;
    r.q[0] = ld_codes<true>(p);
    r.q[1] = ld_codes<true>(p + 64);
    // 16-byte chunk 2ip + g / 2 of row col's qh, its half g % 2
#pragma unroll
    for (int ip = 0; ip < 2; ++ip) {
      const uint2 h = *reinterpret_cast<const uint2*>(rec + R.qh + (2 * ip + (g >> 1)) * 256 + col * 16 + (g & 1) * 8);
      r.h[2 * ip] = h.x;
      r.h[2 * ip + 1] = h.y;
    }
    r.sc = *reinterpret_cast<const uint4*>(rec + R.sc + col * 16);
    if constexpr (W) r.d = reinterpret_cast<const uint32_t*>(rec + R.d)[col];
    else r.d = reinterpret_cast<const uint16_t*>(rec + R.d)[col];
  }
  template <bool W>
  __device__ static float d(const Raw& r) {
    if constexpr (W) return __builtin_bit_cast(float, r.d);
    else return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(r.d)));
  }
  // the sub-scales of window w, word 2ip + c of the row's 16
  __device__ static uint32_t window_scales(const Raw& r, int w) {
    const int word = 2 * (w >> 2) + (w & 1);
    return word == 0 ? r.sc.x : word == 1 ? r.sc.y : word == 2 ? r.sc.z : r.sc.w;
  }
};

}  // namespace qi
