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

}  // namespace half
}  // namespace qi
