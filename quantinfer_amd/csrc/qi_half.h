// Split-half activations for the f16 matrix cores, shared by the 9-16 row
// decode GEMV (qi_gemv_half.hip) and the F32-mode prefill GEMM
// (qi_gemm_split.hip): the conversion of eight activations of one (row,
// unit) into the hi / lo f16 halves, and the exact f16 weight codes built
// from code bytes under the exponent of 1024.
#pragma once
#include "qi_device.h"
#include "qi_unit.h"

namespace qi {
namespace half {

typedef float v4f __attribute__((ext_vector_type(4)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));

// All-gather across the lane groups: v is V[g] in lane group g; out[g'] = V[g'].
__device__ __forceinline__ void gather4u(uint32_t u, uint32_t out[4]) {
  const auto a = __builtin_amdgcn_permlane16_swap(u, u, false, false);
  const auto b = __builtin_amdgcn_permlane32_swap(a[0], a[0], false, false);
  const auto c = __builtin_amdgcn_permlane32_swap(a[1], a[1], false, false);
  out[0] = b[0];
  out[1] = c[0];
  out[2] = b[1];
  out[3] = c[1];
}

__device__ __forceinline__ uint32_t h2u(h2 v) { return __builtin_bit_cast(uint32_t, v); }
__device__ __forceinline__ h2 u2h(uint32_t v) { return __builtin_bit_cast(h2, v); }
// (a & m) | o in one v_and_or_b32: m from a scalar register, o from a vector
// register (gfx950 reads one scalar operand per VALU instruction, so with both
// constants scalar the compiler splits it in two)
__device__ __forceinline__ uint32_t and_or(uint32_t a, uint32_t m, uint32_t o) {
  uint32_t r;
  asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "s"(m), "v"(o));
  return r;
}
// centre a pair: v + c (exact on the integers these hold)
__device__ __forceinline__ uint32_t pk_add(uint32_t v, h2 c) { return h2u(u2h(v) + c); }
// centre a pair of 1024 + 16 q / 1024 + 4 q: v * s + c (exact likewise)
__device__ __forceinline__ uint32_t pk_fma(uint32_t v, h2 s, h2 c) {
  return h2u(__builtin_elementwise_fma(u2h(v), s, c));
}
// keep a value computed where it stands (an empty asm the compiler cannot move work across)
__device__ __forceinline__ void pin(v4f& v) {
  float a = v[0], b = v[1], c = v[2], d = v[3];
  asm volatile("" : "+v"(a), "+v"(b), "+v"(c), "+v"(d));
  v = v4f{a, b, c, d};
}
__device__ __forceinline__ h2 splat(float f) { return h2{static_cast<_Float16>(f), static_cast<_Float16>(f)}; }

constexpr uint32_t kExp1024 = 0x64006400u;  // f16 1024.0 in both halves

// B operand of one window from a slice's two code words: lo (elements 0..3),
// hi (elements 4..7), one code per byte in its low nibble (kMaskLo) or high
// nibble (kMaskHi), or as a whole byte (kMaskByte).
constexpr uint32_t kMaskLo = 0x000F000Fu, kMaskHi = 0x00F000F0u, kMaskByte = 0x00FF00FFu;
template <uint32_t MASK>
__device__ __forceinline__ void raw_pairs(uint32_t lo, uint32_t hi, uint32_t lo8, uint32_t hi8, uint32_t out[4]) {
  out[0] = and_or(lo, MASK, kExp1024);   // elements 0, 2
  out[1] = and_or(lo8, MASK, kExp1024);  // 1, 3
  out[2] = and_or(hi, MASK, kExp1024);   // 4, 6
  out[3] = and_or(hi8, MASK, kExp1024);  // 5, 7
}

// Convert one item (window w, slice g of one (row, unit)) of the values v[8]
// (zeros past M): the (row, unit) scale from its 32 items (the 32 lanes of a
// half wavefront), the window sum from its 4 items (adjacent lanes), the
// halves in the operand order. Every lane takes part.
__device__ __forceinline__ void half_convert(const float v[8], uint8_t* hi_slot, uint8_t* lo_slot, float* xsum_w,
                                             float* unsc_mu, uint32_t w, uint32_t g) {
  // the (row, unit) max over the 32 lanes: 16-lane rows by DPP, then the
  // pair of rows (a NaN is passed over here; it reaches the sums below)
  float mx = 0.0f;
#pragma unroll
  for (int j = 0; j < 8; ++j) mx = fmaxf(mx, fabsf(v[j]));
  mx = fmaxf(mx, dpp_move<0x121>(mx));  // row_ror:1
  mx = fmaxf(mx, dpp_move<0x122>(mx));  // row_ror:2
  mx = fmaxf(mx, dpp_move<kDppRor4>(mx));
  mx = fmaxf(mx, dpp_move<kDppRor8>(mx));
  {
    const auto p = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(uint32_t, mx), __builtin_bit_cast(uint32_t, mx),
                                                    false, false);
    mx = fmaxf(__builtin_bit_cast(float, static_cast<uint32_t>(p[0])), __builtin_bit_cast(float, static_cast<uint32_t>(p[1])));
  }
  // max |x| * 2^sh < 2^15, bounded so that 2^-sh stays a normal f32. A NaN
  // or infinite activation is not caught here: it stays non-finite through
  // the halves and the matrix sums (inf * 0 is NaN), so every output of its
  // row is non-finite and the epilogue recomputes it in the reference's order.
  const int e = __builtin_isfinite(mx) && mx > 0.0f ? __builtin_amdgcn_frexp_expf(mx) : 0;
  const int sh = min(15 - e, 125);
  const float scale = __builtin_bit_cast(float, static_cast<uint32_t>(127 + sh) << 23);  // 2^sh
  // hi: x' truncated to 11 significant bits (exact in f16 in this range); lo:
  // the rest, exactly x' - hi in f32, rounded to f16
  constexpr int kOrd[8] = {0, 2, 1, 3, 4, 6, 5, 7};  // operand order: (0, 2), (1, 3), (4, 6), (5, 7)
  float xh[8], xl[8], sum = 0.0f;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const float xs = v[kOrd[j]] * scale;
    xh[j] = __builtin_bit_cast(float, __builtin_bit_cast(uint32_t, xs) & 0xFFFFE000u);
    xl[j] = xs - xh[j];
    sum += xs;
  }
  uint32_t hi[4], lo[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    hi[j] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(xh[2 * j], xh[2 * j + 1]));  // exact
    lo[j] = h2u(h2{static_cast<_Float16>(xl[2 * j]), static_cast<_Float16>(xl[2 * j + 1])});
  }
  // the window's four slices are lanes 4w'..4w'+3
  sum += dpp_move<kDppSwap1>(sum);
  sum += dpp_move<0x4E>(sum);  // quad_perm [2, 3, 0, 1]
  *reinterpret_cast<uint4*>(hi_slot) = make_uint4(hi[0], hi[1], hi[2], hi[3]);
  *reinterpret_cast<uint4*>(lo_slot) = make_uint4(lo[0], lo[1], lo[2], lo[3]);
  if (g == 0) *xsum_w = sum;
  if (g == 0 && w == 0) *unsc_mu = __builtin_bit_cast(float, static_cast<uint32_t>(127 - sh) << 23);  // 2^-sh
}


// ---------------------------------------------------------------------------
// Split-half operands in the lane groups' own element order (the split-half
// GEMM, qi_gemm_split.hip, and the K-quant 9-16 row GEMV, qi_gemv_half.hip).
//
// A stage holds one unit of 256 elements for a tile of R activation rows:
// the hi and lo halves [half][step][16-row tile][lane] x 16 B, where step t
// (0..7) and lane 16 g + r hold row r's elements of lane group g at step t;
// the 8 window sums [window][row] and the unscales 2^-s [row] (f32). For
// Q8_0 / Q4_0 / Q4_K / Q5_K lane group g holds windows 2g, 2g + 1 (step t:
// window 2g + t / 4, slice t % 4); Q6_K (ORDER6) lane group g = 2 ip + c
// holds elements 128 ip + 32 c + 64 (t / 4) + 8 (t % 4) + [0, 8)
// (Unit<kQ6_K>).
template <uint32_t R>
struct SplitStage {
  static_assert(R % 16 == 0, "whole 16-row tiles");
  static constexpr uint32_t kHalf = 8 * (R / 16) * 64 * 16;
  static constexpr uint32_t kSums = 2 * kHalf;
  static constexpr uint32_t kUnsc = kSums + 8 * R * 4;
  static constexpr uint32_t kBytes = kUnsc + R * 4;
};

// The stage of rows row0 .. row0 + R - 1 (zeros past M) and unit u, by a
// 256-thread workgroup: each half wavefront converts one row per pass (item
// 4 w + s of its 32 lanes: window w, slice s, elements 32 w + 8 s + [0, 8));
// passes p0 .. p1 - 1 (rows 8 p0 .. 8 p1 - 1 of the stage).
template <uint32_t R, bool ORDER6>
__device__ __forceinline__ void split_stage(const float* __restrict__ x, uint32_t K, uint64_t M, uint64_t row0,
                                            uint32_t u, uint8_t* __restrict__ st, uint32_t p0 = 0,
                                            uint32_t p1 = R / 8) {
  using S = SplitStage<R>;
  const uint32_t i32 = threadIdx.x & 31, w = i32 >> 2, s = i32 & 3, hw = threadIdx.x >> 5;
  // the step and lane group that use this slice
  const uint32_t t = ORDER6 ? 4 * ((w >> 1) & 1) + s : 4 * (w & 1) + s;
  const uint32_t g = ORDER6 ? 2 * (w >> 2) + (w & 1) : w >> 1;
  float* const sums = reinterpret_cast<float*>(st + S::kSums);
  float* const unsc = reinterpret_cast<float*>(st + S::kUnsc);
#pragma unroll 1
  for (uint32_t pass = p0; pass < p1; ++pass) {
    const uint32_t r = pass * 8 + hw;
    const uint64_t row = row0 + r;
    float4 v0 = make_float4(0.0f, 0.0f, 0.0f, 0.0f), v1 = v0;
    if (row < M) {
      const float4* p = reinterpret_cast<const float4*>(x + row * K + u * 256 + 32 * w + 8 * s);
      v0 = p[0];
      v1 = p[1];
    }
    const float v[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
    uint8_t* const hs = st + ((t * (R / 16) + (r >> 4)) * 64 + 16 * g + (r & 15)) * 16;
    half_convert(v, hs, hs + S::kHalf, sums + w * R + r, unsc + r, w, s);
  }
}

// Per-format choices. Q4_K / Q5_K fold the 6-bit sub-block scale into an
// exact f16 code (one weight plane, offsets through the window sums). The
// other formats' per-block factors do not fold exactly into one f16 number
// (Q8_0 d q: up to 19 bits; Q6_K sc (q - 32): up to 12), so the weight enters
// as two f16 planes, hi = f16(w') and lo = w' - hi (exact, one fused
// multiply-add), and every product takes three instructions: x_hi w_hi,
// x_lo w_hi, x_hi w_lo (x_lo w_lo, below 2^-22 of the product, is left out).
// Q8_0 / Q4_0: w' = 2^e d (q - bias), e per (output, unit) from the largest
// of its eight block scales; Q6_K: w' = sc (q - 32), d applied in the
// combine. Wavefronts hold 2 output tiles (two units of records in registers
// and two wavefronts per SIMD).
template <int QT>
struct SplitFmt {
  static constexpr bool kK45 = QT == kQ4_K || QT == kQ5_K;
  static constexpr int kPlanes = kK45 ? 1 : 2;
  static constexpr int kTiles = 2;  // output tiles per wavefront
  static constexpr bool kOrder6 = QT == kQ6_K;
};

// Per (output, unit) factors for lane group g. K45: the unit's d, the
// windows' integer scales and centring constants, the offsets' operand.
// Q8_0 / Q4_0: d = 2^-e, sc[h] = 2^e times block 2g + h's scale. Q6_K: d, and
// sc[] the lane group's four sub-scales.
struct SplitScales {
  float d;
  h2 sc[4], c[2];
  uint4 bo;  // K45: the offsets' B operand: -b' of windows 2g, 2g+1 as f16 halves, scaled by 2^e
  float fo;  // K45: 2^(6 - e), the offsets' matrix sum back to the f32 scale
};

// x as hi (x truncated to 11 significant bits, exact in f16) + lo (the rest
// rounded to f16)
__device__ __forceinline__ void split_f16(float x, float& hi, float& lo) {
  hi = __builtin_bit_cast(float, __builtin_bit_cast(uint32_t, x) & 0xFFFFE000u);
  lo = x - hi;
}
__device__ __forceinline__ uint32_t pack_rtz(float a, float b) {
  return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(a, b));
}
__device__ __forceinline__ float f16_bits(uint32_t v) {
  return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(v & 0xFFFFu)));
}

template <int QT, bool WIDE>
__device__ __forceinline__ void split_scales(const typename Unit<QT>::Raw& r, uint32_t g, SplitScales& o) {
  using U = Unit<QT>;
  if constexpr (QT == kQ8_0 || QT == kQ4_0) {
    static_assert(!WIDE, "f32 block scales are not exact in f16");
    const float d0 = f16_bits(r.s0), d1 = f16_bits(r.s0 >> 16);
    // the largest scale of the output's eight blocks (two per lane group)
    uint32_t all[4];
    gather4u(__builtin_bit_cast(uint32_t, fmaxf(fabsf(d0), fabsf(d1))), all);
    const float dm = fmaxf(fmaxf(__builtin_bit_cast(float, all[0]), __builtin_bit_cast(float, all[1])),
                           fmaxf(__builtin_bit_cast(float, all[2]), __builtin_bit_cast(float, all[3])));
    // 2^e d_max in [2^7, 2^8): |w'| < 2^15 (Q8_0 codes up to 128 in magnitude)
    const int e = dm > 0.0f ? 8 - __builtin_amdgcn_frexp_expf(dm) : 0;
    o.d = __builtin_ldexpf(1.0f, -e);
    o.sc[0] = splat(__builtin_ldexpf(d0, e));
    o.sc[1] = splat(__builtin_ldexpf(d1, e));
  } else if constexpr (QT == kQ6_K) {
    o.d = WIDE ? __builtin_bit_cast(float, r.d) : f16_bits(r.d);
#pragma unroll
    for (int i = 0; i < 4; ++i) o.sc[i] = splat(static_cast<float>(static_cast<int32_t>(r.sc << (24 - 8 * i)) >> 24));
  } else {
    constexpr float kQMax = QT == kQ5_K ? 31.0f : 15.0f;
    float d, dmin;
    U::template dmins<WIDE>(r, d, dmin);
    const uint32_t f = U::field(g, r);
    o.d = d;
    // |b'| <= max(d sc / 2, dmin m) < max(32 d, 64 dmin) = B: scaled by 2^e
    // with B 2^e < 2^15 the offsets fit f16 (the same e in every lane group of
    // the output, as its four lane groups' offsets enter one sum)
    const float bound = fmaxf(32.0f * d, 64.0f * dmin);
    const int eb = bound > 0.0f ? __builtin_amdgcn_frexp_expf(bound) : 0;
    const float up = __builtin_ldexpf(1.0f, 15 - eb);
    o.fo = __builtin_ldexpf(1.0f, eb - 9);
    float nh[2], nl[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const float sc = static_cast<float>((f >> (12 * h)) & 63u), mn = static_cast<float>((f >> (12 * h + 6)) & 63u);
      const float a = d * sc, b = dmin * mn;  // both exact in f32
      // any integer z keeps the arithmetic exact; the nearest one keeps b'
      // small (a = 0 gives z = kQMax or 0 and b' = b, with codes times sc = 0)
      const float z = fminf(fmaxf(rintf(b * __builtin_amdgcn_rcpf(a)), 0.0f), kQMax);
      split_f16(fmaf(a, z, -b) * up, nh[h], nl[h]);
      o.sc[h] = splat(sc);
      o.c[h] = splat(h == 0 ? -(1024.0f + z) : -(64.0f + z));
    }
    // slots 8g..8g+7: hi(2g), hi(2g+1), lo(2g), lo(2g+1), hi(2g), hi(2g+1), 0, 0
    const uint32_t hh = pack_rtz(nh[0], nh[1]);
    o.bo = make_uint4(hh, pack_rtz(nl[0], nl[1]), hh, 0u);
  }
}

// The B operand(s) of step t: the lane's 8 codes in the operand order (0, 2),
// (1, 3), (4, 6), (5, 7). K45: sc (q - z), one plane. Other formats: the
// centred code c times the factor f as hi = f16(c f) and lo = c f - hi.
template <int QT>
__device__ __forceinline__ void split_codes(const typename Unit<QT>::Raw& r, uint32_t g, int t, const SplitScales& s,
                                            uint32_t out[SplitFmt<QT>::kPlanes][4]) {
  const int h = t >> 2, p = t & 3;
  if constexpr (SplitFmt<QT>::kK45) {
    const uint4 q = r.q[p >> 1];
    const uint32_t lo = (p & 1) ? q.z : q.x, hi = (p & 1) ? q.w : q.y;
    if (h == 0) raw_pairs<kMaskLo>(lo, hi, lo >> 8, hi >> 8, out[0]);
    else raw_pairs<kMaskHi>(lo, hi, lo >> 8, hi >> 8, out[0]);
    if constexpr (QT == kQ5_K) {
      // bit 2g + h of qh byte e is bit 4 of element e's code
      const uint4 qh = r.h[p >> 1];
      const uint32_t bit = 2 * g + static_cast<uint32_t>(h);
      const uint32_t l = ((p & 1) ? qh.z : qh.x) >> bit, u = ((p & 1) ? qh.w : qh.y) >> bit;
      if (h == 0) {
        out[0][0] |= (l << 4) & 0x00100010u;
        out[0][1] |= (l >> 4) & 0x00100010u;
        out[0][2] |= (u << 4) & 0x00100010u;
        out[0][3] |= (u >> 4) & 0x00100010u;
      } else {
        out[0][0] |= (l << 8) & 0x01000100u;
        out[0][1] |= l & 0x01000100u;
        out[0][2] |= (u << 8) & 0x01000100u;
        out[0][3] |= u & 0x01000100u;
      }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t centred = h == 0 ? pk_add(out[0][i], s.c[0]) : pk_fma(out[0][i], splat(0.0625f), s.c[1]);
      out[0][i] = h2u(u2h(centred) * s.sc[h]);
    }
  } else {
    // the step's 8 codes, one per byte (Q8_0 signed: + 128 by flipping bit 7)
    const uint64_t w = static_cast<uint64_t>(Unit<QT>::codes(r, g, t));
    uint32_t lo = static_cast<uint32_t>(w), hi = static_cast<uint32_t>(w >> 32);
    if constexpr (QT == kQ8_0) {
      lo ^= 0x80808080u;
      hi ^= 0x80808080u;
    }
    uint32_t v[4];
    raw_pairs<kMaskByte>(lo, hi, lo >> 8, hi >> 8, v);  // 1024 + byte
    constexpr float kBias = QT == kQ8_0 ? 1152.0f : QT == kQ4_0 ? 1032.0f : 1056.0f;
    // Q8_0 / Q4_0: block 2g + h's factor; Q6_K: sub-block 2 h + p / 2 of the lane group
    const h2 f = QT == kQ6_K ? s.sc[2 * h + (p >> 1)] : s.sc[h];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const h2 cc = u2h(pk_add(v[i], splat(-kBias)));  // the centred code, exact
      const h2 whi = cc * f;
      out[0][i] = h2u(whi);
      out[1][i] = h2u(__builtin_elementwise_fma(cc, f, -whi));  // exact: c f - f16(c f)
    }
  }
}


}  // namespace half
}  // namespace qi
