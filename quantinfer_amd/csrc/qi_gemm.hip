// Prefill GEMM on the f16 matrix cores (v_mfma_f32_16x16x32_f16), output-rows
// layout, K a multiple of 256, any M (meant for M >= 128).
//
// Arithmetic. The activations are rounded once to f16 (x_to_f16_kernel, rows
// padded to the 128-row tile with zeros). Each weight is rounded once to f16:
// Q8_0 / Q4_0 as (code - bias) * d, an exact f16 integer times the stored f16
// scale; the K-quants from the reference's own f32 value (d * sc) * q -
// dmin * m (Q6_K (d * sc) * (q - 32)), so no rounding is shared by the 32
// weights of a sub-block (rounding d * sc or dmin * m to f16 would be, and
// cancels badly in blocks whose range an outlier stretched). Q4_K computes
// that value as a * (1024 + q) + c with c = -(1024 a + b) rounded once to f32
// per window (q4k_affine), an extra error below 2^-14 a, far under the f16
// rounding of the weight. Products accumulate in f32 on the matrix cores.
// This is the tolerance-judged MFMA mode (f16 operands, f32 accumulation).
//
// Tiling. A workgroup of 8 wavefronts owns 128 activation rows x 256
// outputs, split by role (gemm_ws_kernel): 4 compute wavefronts each own all
// 128 rows and 64 outputs (8 x 4 MFMA tiles of 16 x 16, so a weight fragment
// feeds 8 MFMAs); 4 producer wavefronts stage the activations and dequantize
// the weight fragments into LDS one 2-step stage ahead. Step t of a unit
// covers, for lane group g, elements window_first(g, t / 4) + 8 (t % 4) +
// [0, 8) on both operands, the element order the weight records store, so
// neither operand is reshuffled; LDS blocks are laid out [step][tile][lane] x
// 16 bytes, so every fragment read and every staging write is 1 KB contiguous.
#include "qi_device.h"
#include "qi_internal.h"
#include "qi_unit.h"

#include <stdlib.h>

#include <type_traits>

namespace qi {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kTileM = 128;

__global__ __launch_bounds__(256) void x_to_f16_kernel(const float* __restrict__ x, uint64_t m,
                                                       uint64_t k, uint64_t m_pad,
                                                       _Float16* __restrict__ xh) {
  const uint64_t i = (static_cast<uint64_t>(blockIdx.x) * 256 + threadIdx.x) * 8;
  if (i >= m_pad * k) return;
  h8 o;
  if (i / k < m) {
    const float4* p = reinterpret_cast<const float4*>(x + i);
    const float4 a = p[0], b = p[1];
    o = h8{static_cast<_Float16>(a.x), static_cast<_Float16>(a.y), static_cast<_Float16>(a.z),
           static_cast<_Float16>(a.w), static_cast<_Float16>(b.x), static_cast<_Float16>(b.y),
           static_cast<_Float16>(b.z), static_cast<_Float16>(b.w)};
  } else {
    o = h8{0, 0, 0, 0, 0, 0, 0, 0};
  }
  *reinterpret_cast<h8*>(xh + i) = o;
}

// 8 codes (bytes of a long) -> 8 exact f16 integers q - bias (Q8_0, Q4_0).
template <int QT>
__device__ __forceinline__ void codes_to_f16(long codes, h2 out[4]) {
  uint32_t w[2] = {static_cast<uint32_t>(codes), static_cast<uint32_t>(static_cast<uint64_t>(codes) >> 32)};
  // Q8_0 codes are signed: flip the sign bit so the byte is code + 128
  if constexpr (QT == kQ8_0) {
    w[0] ^= 0x80808080u;
    w[1] ^= 0x80808080u;
  }
  constexpr float bias = QT == kQ8_0 ? 1152.0f : 1032.0f;
  const h2 sub = {static_cast<_Float16>(bias), static_cast<_Float16>(bias)};
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    out[2 * i] = __builtin_bit_cast(h2, __builtin_amdgcn_perm(0x64646464u, w[i], 0x04010400u)) - sub;
    out[2 * i + 1] = __builtin_bit_cast(h2, __builtin_amdgcn_perm(0x64646464u, w[i], 0x04030402u)) - sub;
  }
}

// f16 weight fragment of 8 codes. Q8_0 / Q4_0: w = (q - bias) * d with d the
// stored f16 scale, one rounding. K-quants: the reference's f32 value
// (d * sc) * q - dmin * m (Q6_K: (d * sc) * (q - 32)), then one rounding to
// f16, so no rounding error is shared by the weights of a sub-block.
template <int QT>
__device__ __forceinline__ h8 weight_fragment(long codes, float a, float b) {
  if constexpr (QT == kQ8_0 || QT == kQ4_0) {
    h2 q[4];
    codes_to_f16<QT>(codes, q);
    const _Float16 ha = static_cast<_Float16>(a);
    const h2 a2 = {ha, ha};
    h2 w[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) w[i] = q[i] * a2;
    return h8{w[0][0], w[0][1], w[1][0], w[1][1], w[2][0], w[2][1], w[3][0], w[3][1]};
  } else {
    // codes (0..63) -> exact f16 integers by the exponent-pattern permute, then
    // one f32 fma per weight rounded once to f16 (a mixed-precision fma that
    // writes an f16 half: one instruction per weight)
    const uint32_t w[2] = {static_cast<uint32_t>(codes),
                           static_cast<uint32_t>(static_cast<uint64_t>(codes) >> 32)};
    const float nb = QT == kQ6_K ? -32.0f * a : -b;  // Q6_K: (d * sc) * (q - 32) = a * q - 32 a
    const h2 k1024 = {static_cast<_Float16>(1024.0f), static_cast<_Float16>(1024.0f)};
    h8 out;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const h2 q01 = __builtin_bit_cast(h2, __builtin_amdgcn_perm(0x64646464u, w[i], 0x04010400u)) - k1024;
      const h2 q23 = __builtin_bit_cast(h2, __builtin_amdgcn_perm(0x64646464u, w[i], 0x04030402u)) - k1024;
      out[4 * i + 0] = static_cast<_Float16>(fmaf(a, static_cast<float>(q01[0]), nb));
      out[4 * i + 1] = static_cast<_Float16>(fmaf(a, static_cast<float>(q01[1]), nb));
      out[4 * i + 2] = static_cast<_Float16>(fmaf(a, static_cast<float>(q23[0]), nb));
      out[4 * i + 3] = static_cast<_Float16>(fmaf(a, static_cast<float>(q23[1]), nb));
    }
    return out;
  }
}

// Outputs of a lane's tile whose f16 result is not finite (a NaN or infinite
// activation, |x| beyond f16's range) are recomputed in the reference's order
// (exact_output_row), which decides which are NaN and which +-Inf. The lane
// owns rows row0 + 16 rt + r (rt < rts, r < 4) of columns col0 + 16 ct
// (ct < CT); its values are already stored in y.
template <int QT, bool WIDE, int CT = 4>
__device__ __forceinline__ void gemm_fix_nonfinite(const GemmArgs& a, uint64_t row0, int rts, uint64_t col0) {
#pragma unroll 1
  for (int i = 0; i < 4 * CT * rts; ++i) {
    const uint64_t n = col0 + 16 * static_cast<uint64_t>(i / (4 * rts));
    const uint64_t m = row0 + 16 * static_cast<uint64_t>((i / 4) % rts) + (i % 4);
    if (n >= a.w.n || m >= a.m) continue;
    float* const p = a.y + m * a.w.n + n;
    if (!__builtin_isfinite(*p)) *p = exact_output_row<QT, WIDE>(a.w, a.x + m * a.w.k, n);
  }
}

// SiLU-pairs epilogue of a 128-row block (GemmArgs::act): lane (g, c16) holds
// acc[rt][ct][r], row m0 + 16 rt + 4 g + r of output tile tile0 + ct, column
// c16; columns c16 and c16 ^ 8 are a gate and its up value. The two lanes of
// a pair swap their four rows and each finishes two of them (the gate lane
// rows 0-1, the up lane rows 2-3), writing gate / (1 + e^-gate) * up
// (backends/cpu/src/backend.rs:224-237) to act[m][8 T + c16 % 8].
template <int CT = 4>
__device__ __forceinline__ void gemm_store_silu(const GemmArgs& a, const f4 (&acc)[8][CT], uint32_t tile0,
                                                uint64_t m0, uint32_t g, uint32_t c16) {
  const uint64_t lda = a.w.n / 2;
  const bool up = c16 >= 8;
  const uint32_t c8 = c16 & 7;
#pragma unroll
  for (int ct = 0; ct < CT; ++ct) {
    const uint64_t T = tile0 + ct;
#pragma unroll
    for (int rt = 0; rt < 8; ++rt) {
      f4 other;
#pragma unroll
      for (int r = 0; r < 4; ++r) other[r] = __shfl_xor(acc[rt][ct][r], 8);
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int r = up ? 2 + h : h;
        const float gate = up ? other[r] : acc[rt][ct][r], upv = up ? acc[rt][ct][r] : other[r];
        const uint64_t m = m0 + 16 * rt + 4 * g + r;
        if (T * 16 < a.w.n && m < a.m) a.act[m * lda + T * 8 + c8] = gate / (1.0f + expf(-gate)) * upv;
      }
    }
  }
}

// (v & mask) | pattern in one instruction: a VOP3 encoding on gfx9 holds no
// literal and reads at most one scalar register, so the mask comes from a
// scalar and the pattern from a vector register (the compiler otherwise
// splits it into an and and an or).
__device__ __forceinline__ uint32_t and_or(uint32_t v, uint32_t mask, uint32_t pattern) {
  uint32_t r;
  asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(v), "s"(mask), "v"(pattern));
  return r;
}

// Q4_K fragment straight from the record words (no byte unpacking): the
// nibble mask and the f16 exponent pattern 0x6400 give 1024 + q per half
// (low nibbles, steps t < 4) or 1024 + 16 q (high nibbles, t >= 4), and the
// per-window affine (a, c) has the offset folded in (q4k_affine), so each
// weight is one f32 fma of the exact f16 code, rounded once to f16.
// Element order within the fragment is the natural one (bytes 0..7).
__device__ __forceinline__ h8 q4k_fragment(const Unit<kQ4_K>::Raw& r, int t, float a, float c) {
  const int tt = t & 3;
  const uint4 q = r.q[tt >> 1];
  const uint32_t lo = (tt & 1) ? q.z : q.x, hi = (tt & 1) ? q.w : q.y;
  const uint32_t mask = t >= 4 ? 0x00F000F0u : 0x000F000Fu;
  const h2 e0 = __builtin_bit_cast(h2, and_or(lo, mask, 0x64006400u));       // elements 0, 2
  const h2 e1 = __builtin_bit_cast(h2, and_or(lo >> 8, mask, 0x64006400u));  // 1, 3
  const h2 e2 = __builtin_bit_cast(h2, and_or(hi, mask, 0x64006400u));       // 4, 6
  const h2 e3 = __builtin_bit_cast(h2, and_or(hi >> 8, mask, 0x64006400u));  // 5, 7
  auto w = [&](_Float16 v) { return static_cast<_Float16>(fmaf(a, static_cast<float>(v), c)); };
  return h8{w(e0[0]), w(e1[0]), w(e0[1]), w(e1[1]), w(e2[0]), w(e3[0]), w(e2[1]), w(e3[1])};
}

// (a, b) of a Q4_K window -> the (scale, offset) q4k_fragment applies to the
// biased codes: window 0 (low nibbles, 1024 + q): (a, -(1024 a + b));
// window 1 (high nibbles, 1024 + 16 q): (a / 16, -(64 a + b)).
__device__ __forceinline__ void q4k_affine(float sa[2], float sb[2]) {
  sb[0] = -fmaf(1024.0f, sa[0], sb[0]);
  sb[1] = -fmaf(64.0f, sa[1], sb[1]);
  sa[1] = sa[1] * 0.0625f;
}

// Warp-specialized variant: 8 wavefronts, two roles on every SIMD.
//   compute wavefronts 0-3 own 128 rows x 64 outputs each (8 x 4 MFMA tiles)
//     and only read fragments from LDS and issue MFMAs;
//   producer wavefronts 4-7 stage the activations (global -> LDS) and
//     dequantize the weight fragments of compute wavefront (w - 4)'s 4 output
//     tiles into LDS, one 2-step stage ahead.
// Wavefronts w and w + 4 share a SIMD, so the matrix core (compute) and the
// VALU (producer) overlap across wavefronts instead of within one.
// LDS: two slots of [A: 2 steps x 8 row tiles x 64 lanes x 16 B = 16 KB |
// B: 2 steps x 16 output tiles x 64 lanes x 16 B = 32 KB]; one barrier per
// stage, executed the same number of times by both roles.
template <int QT, bool WIDE>
__global__ __launch_bounds__(512) void gemm_ws_kernel(GemmArgs a) {
  using U = Unit<QT>;
  constexpr Record R = record_geometry(QT, WIDE);
  constexpr uint32_t kA = 2 * 8 * 64 * 16, kB = 2 * 16 * 64 * 16, kSlot = kA + kB;
  constexpr uint32_t kHalf = QT == kQ6_K ? 64 : 32;
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];

  const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const uint32_t g = lane >> 4, c16 = lane & 15;
  const uint32_t units = a.w.units;
  const uint32_t K = static_cast<uint32_t>(a.w.k);
  const uint64_t m0 = static_cast<uint64_t>(blockIdx.y) * kTileM;
  const uint32_t stages = 4 * units;

  if (wave < 4) {
    // ------------------------------------------------------------ compute
    f4 acc[8][4];
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[i][j] = f4{0, 0, 0, 0};
    for (uint32_t st = 0; st < stages; ++st) {
      __syncthreads();  // stage st is in slot st % 2
      const uint8_t* A = lds + (st & 1) * kSlot;
      const uint8_t* B = A + kA;
#pragma unroll
      for (int tt = 0; tt < 2; ++tt) {
        h8 af[8], bf[4];
#pragma unroll
        for (int rt = 0; rt < 8; ++rt) af[rt] = *reinterpret_cast<const h8*>(A + ((tt * 8 + rt) * 64 + lane) * 16);
#pragma unroll
        for (int ct = 0; ct < 4; ++ct)
          bf[ct] = *reinterpret_cast<const h8*>(B + ((tt * 16 + 4 * wave + ct) * 64 + lane) * 16);
#pragma unroll
        for (int ct = 0; ct < 4; ++ct)
#pragma unroll
          for (int rt = 0; rt < 8; ++rt)
            acc[rt][ct] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[rt], bf[ct], acc[rt][ct], 0, 0, 0);
      }
    }
    // C[i][j]: lane j + 16 (i / 4), element i % 4
    const uint64_t ld = a.w.n;
    float* yrow = a.y + (m0 + 4 * g) * ld;
    bool bad = false;
#pragma unroll
    for (int ct = 0; ct < 4; ++ct) {
      const uint64_t n = static_cast<uint64_t>((blockIdx.x * 4 + wave) * 4 + ct) * 16 + c16;
      if (n >= a.w.n) continue;
#pragma unroll
      for (int rt = 0; rt < 8; ++rt) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const uint64_t m = m0 + rt * 16 + 4 * g + r;
          if (m < a.m) {
            yrow[(rt * 16 + r) * ld + n] = acc[rt][ct][r];
            bad |= !__builtin_isfinite(acc[rt][ct][r]);
          }
        }
      }
    }
    if (bad) gemm_fix_nonfinite<QT, WIDE>(a, m0 + 4 * g, 8, static_cast<uint64_t>((blockIdx.x * 4 + wave) * 4) * 16 + c16);
    return;
  }

  // -------------------------------------------------------------- producer
  const uint32_t pw = wave - 4, pt = tid - 256;
  const uint8_t* trec[4];
#pragma unroll
  for (int ct = 0; ct < 4; ++ct) {
    const uint32_t t = min((blockIdx.x * 4 + pw) * 4 + ct, a.w.tiles - 1);
    trec[ct] = a.w.qs + static_cast<uint64_t>(t) * units * R.bytes;
  }
  // activation staging: thread pt owns row 16 rt + si (rt = pt / 64 + 4 p) and
  // lane group sg; a stage holds its 16 elements window_first(sg, q / 2) +
  // 16 (q % 2) + [0, 16) as two chunks (tt), chunk (p, tt) to slot 16 sg + si
  // of block (tt, rt): one store instruction fills one contiguous 1 KB block
  const uint32_t si = pt & 15, sg = (pt >> 4) & 3, srt = pt >> 6;
  const _Float16* abase = a.xh + (m0 + 16 * srt + si) * K + window_first<QT>(sg, 0);
  const uint64_t apass = static_cast<uint64_t>(64) * K;
  const uint32_t sbase = (srt * 64 + sg * 16 + si) * 16;
  u32x4 areg[4];
  auto a_load = [&](uint32_t u, uint32_t q) {
    const _Float16* p = abase + 256 * u + kHalf * (q >> 1) + 16 * (q & 1);
#pragma unroll
    for (int i = 0; i < 4; ++i) areg[i] = *reinterpret_cast<const u32x4*>(p + (i >> 1) * apass + 8 * (i & 1));
  };
  auto a_store = [&](uint32_t slot) {
    uint8_t* p = lds + slot * kSlot + sbase;
#pragma unroll
    for (int i = 0; i < 4; ++i) *reinterpret_cast<u32x4*>(p + ((i & 1) * 8 + 4 * (i >> 1)) * 64 * 16) = areg[i];
  };

  typename U::Raw cur[4], nxt[4];
  float sa[4][U::kWindows], sb[4][U::kWindows];
  // weight fragments of steps 2q, 2q+1 of the current unit into a slot
  auto b_store = [&](auto qc, uint32_t slot) {
    constexpr int q = decltype(qc)::value;
    uint8_t* B = lds + slot * kSlot + kA;
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) {
      const int t = 2 * q + tt, w = t / U::kSteps;
#pragma unroll
      for (int ct = 0; ct < 4; ++ct) {
        const h8 f = weight_fragment<QT>(U::codes(cur[ct], g, t), sa[ct][w], sb[ct][w]);
        *reinterpret_cast<h8*>(B + ((tt * 16 + 4 * pw + ct) * 64 + lane) * 16) = f;
      }
    }
  };
  auto new_unit = [&](uint32_t u) {
    // cur holds unit u: its scales, then the prefetch of unit u + 1
#pragma unroll
    for (int ct = 0; ct < 4; ++ct) U::template scales<WIDE>(g, cur[ct], sa[ct], sb[ct]);
    const uint32_t un = min(u + 1, units - 1);
#pragma unroll
    for (int ct = 0; ct < 4; ++ct)
      U::template load<WIDE>(trec[ct] + static_cast<uint64_t>(un) * R.bytes, lane, nxt[ct]);
  };

  // prologue: stage 0 into slot 0
#pragma unroll
  for (int ct = 0; ct < 4; ++ct) U::template load<WIDE>(trec[ct], lane, cur[ct]);
  a_load(0, 0);
  new_unit(0);
  a_store(0);
  a_load(0, 1);
  b_store(std::integral_constant<int, 0>{}, 0);

  for (uint32_t u = 0; u < units; ++u) {
    // iteration (u, q): barrier of stage 4u + q, then produce stage 4u + q + 1
    auto step = [&](auto qc) {
      constexpr int q = decltype(qc)::value;
      __syncthreads();
      const uint32_t st = 4 * u + q;
      if (st + 1 < stages) {
        const uint32_t slot = (st + 1) & 1;
        a_store(slot);
        constexpr int qn = (q + 1) & 3;
        const uint32_t un = qn == 0 ? u + 1 : u;
        // activations of the stage after
        if (st + 2 < stages) a_load(qn == 3 ? un + 1 : un, (qn + 1) & 3);
        if constexpr (qn == 0) {
#pragma unroll
          for (int ct = 0; ct < 4; ++ct) cur[ct] = nxt[ct];
          new_unit(un);
        }
        b_store(std::integral_constant<int, qn>{}, slot);
      }
    };
    step(std::integral_constant<int, 0>{});
    step(std::integral_constant<int, 1>{});
    step(std::integral_constant<int, 2>{});
    step(std::integral_constant<int, 3>{});
  }
}

// Activations to f16 in MFMA fragment order for gemm_reg_kernel:
// xa[mt][u][t][rt][lane] x 8 halves (mt: 128-row tile, u: 256-element unit,
// t: step, rt: 16-row tile); lane l holds row 16 rt + (l & 15), elements
// window_first(l >> 4, t / 4) + 8 (t % 4) + [0, 8) of unit u, the order the
// weight fragments of step t use. A 2-step stage is 16 KB contiguous. Rows
// past m are zero.
// One workgroup per (128-row tile mt, unit u, 32-row quarter rq): rows
// mt * 128 + 32 rq + [0, 32) of unit u. Loads take 64 contiguous bytes of
// each of 16 rows per wavefront instruction; the f16 values are placed in
// fragment order in LDS (two-way bank conflicts at most) and leave as 1 KB
// contiguous runs: the 16 KB of (mt, u, steps 0-7, row tiles 2 rq, 2 rq + 1).
// Not for Q6_K, whose windows interleave differently (gemm_ws_kernel reads
// plain f16 rows).
template <int QT>
__global__ __launch_bounds__(256) void x_to_frag_kernel(const float* __restrict__ x, uint64_t m, uint32_t K,
                                                        _Float16* __restrict__ xa) {
  static_assert(QT != kQ6_K, "Q6_K activations use x_to_f16_kernel");
  __shared__ __attribute__((aligned(16))) uint8_t tile[16384];  // [t][rt2][lane] x 16 B
  const uint32_t units = K / 256, tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const uint32_t r = lane & 15, c = lane >> 4;
  const uint32_t rq = blockIdx.x & 3;
  const uint64_t rest = blockIdx.x >> 2;  // mt * units + u
  const uint64_t mt = rest / units;
  const uint32_t u = static_cast<uint32_t>(rest % units);
  const float4* x4 = reinterpret_cast<const float4*>(x);
  float4 v[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const uint32_t I = 4 * j + w, rt2 = I >> 4, cblk = I & 15;
    const uint64_t row = mt * kTileM + 32 * rq + 16 * rt2 + r;
    v[j] = row < m ? x4[(row * K + 256 * u) / 4 + 4 * cblk + c] : float4{0, 0, 0, 0};
  }
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const uint32_t I = 4 * j + w, rt2 = I >> 4, cblk = I & 15;
    // element k = 16 cblk + 4 c of the unit: window (g, h) = (k / 64, k / 32 % 2),
    // step t = 4 h + k / 8 % 4, half k / 4 % 2 of the 8-element piece
    const uint32_t g = cblk >> 2, h = (cblk >> 1) & 1, t = 4 * h + (((cblk & 1) << 1) | (c >> 1));
    const uint32_t off = ((t * 2 + rt2) * 64 + 16 * g + r) * 16 + (c & 1) * 8;
    typedef _Float16 h4 __attribute__((ext_vector_type(4)));
    *reinterpret_cast<h4*>(tile + off) = h4{static_cast<_Float16>(v[j].x), static_cast<_Float16>(v[j].y),
                                            static_cast<_Float16>(v[j].z), static_cast<_Float16>(v[j].w)};
  }
  __syncthreads();
  u32x4* out = reinterpret_cast<u32x4*>(xa) + rest * 4096;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t q = 256 * i + tid, t = q >> 7, rt2 = (q >> 6) & 1, l = q & 63;
    out[(t * 8 + 2 * rq + rt2) * 64 + l] = reinterpret_cast<const u32x4*>(tile)[q];
  }
}

// Weights in registers: the workgroup's 128 x 256 block is split over W = 8
// wavefronts (two per SIMD), each owning all 8 row tiles (128 rows) and 2
// output tiles (32 outputs); against 4 wavefronts of 4 tiles (one per SIMD)
// Q8_0 2048x4096x12288 270.5 -> 259.5 us, Q4_0 236.5 -> 228.3. A wavefront
// streams its tiles' weight records from global memory (one unit ahead) and
// dequantizes each step's fragments itself, between its MFMA issues, so
// weights never pass through LDS. The activations of a 2-step
// stage (16 KB, fragment order) go global -> registers (kAhead stages in
// flight) -> one of two LDS slots, one barrier per stage; a fragment read is
// 1 KB contiguous across the wavefront. Split-K (a.splits > 1): workgroup z
// takes units [z units / splits, (z + 1) units / splits) and writes its
// partial tile to a.part[z].
constexpr int kRegWaves = 8;  // wavefronts per workgroup (16 output tiles over them)

template <int QT, bool WIDE, int W>
__global__ __launch_bounds__(64 * W) void gemm_reg_kernel(GemmArgs a) {
  using U = Unit<QT>;
  constexpr Record R = record_geometry(QT, WIDE);
  constexpr int RT = 8;  // row tiles per wavefront
  constexpr int kThreads = 64 * W;
  constexpr int CT = 16 / W;  // output tiles per wavefront
  constexpr int kPer = 1024 / kThreads;  // 16-byte activation pieces per thread per stage
  constexpr uint32_t kStage = 2 * 8 * 64 * 16;  // bytes: 2 steps x 8 row tiles x 64 lanes x 16 B
  __shared__ __attribute__((aligned(16))) uint8_t lds[2 * kStage];

  const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const uint32_t g = lane >> 4, c16 = lane & 15;
  const uint32_t cw = wave;  // column group: output tiles CT cw .. CT cw + CT - 1
  constexpr uint32_t rt0 = 0;
  const uint32_t units = a.w.units;
  const uint32_t ub = blockIdx.z * units / a.splits, ue = (blockIdx.z + 1) * units / a.splits;
  const uint64_t m0 = static_cast<uint64_t>(blockIdx.y) * kTileM;
  const uint32_t stages = 4 * ue;  // one past this workgroup's last stage
  // this row tile's activation pieces (16 B each): stage s is pieces [1024 s, 1024 s + 1024)
  const u32x4* xa = reinterpret_cast<const u32x4*>(a.xh) + static_cast<uint64_t>(blockIdx.y) * units * 4096;

  const uint32_t tile0 = (blockIdx.x * W + cw) * CT;
  const uint8_t* trec[CT];
#pragma unroll
  for (int ct = 0; ct < CT; ++ct) {
    const uint32_t t = min(tile0 + ct, a.w.tiles - 1);
    trec[ct] = a.w.qs + static_cast<uint64_t>(t) * units * R.bytes;
  }

  constexpr int kAhead = 2;  // activation stages in flight (register ring, stage s in ar[s % kAhead])
  u32x4 ar[kAhead][kPer];
  auto a_load = [&](auto pc, uint32_t st) {
    constexpr int par = decltype(pc)::value;
    const uint32_t sl = st < stages ? st : stages - 1;
#pragma unroll
    for (int i = 0; i < kPer; ++i) ar[par][i] = xa[static_cast<uint64_t>(sl) * 1024 + tid + kThreads * i];
  };
  auto a_store = [&](auto pc, uint32_t slot) {
    constexpr int par = decltype(pc)::value;
    u32x4* dst = reinterpret_cast<u32x4*>(lds + slot * kStage);
#pragma unroll
    for (int i = 0; i < kPer; ++i) dst[tid + kThreads * i] = ar[par][i];
  };

  // the next unit's weight records are prefetched into registers
  typename U::Raw cur[CT], nxt[CT];
  float sa[CT][U::kWindows], sb[CT][U::kWindows];
  auto b_load = [&](uint32_t u) {
    const uint32_t ul = u < ue ? u : ue - 1;
#pragma unroll
    for (int ct = 0; ct < CT; ++ct)
      U::template load<WIDE>(trec[ct] + static_cast<uint64_t>(ul) * R.bytes, lane, nxt[ct]);
  };

  f4 acc[RT][CT];
#pragma unroll
  for (int i = 0; i < RT; ++i)
#pragma unroll
    for (int j = 0; j < CT; ++j) acc[i][j] = f4{0, 0, 0, 0};

  // prologue: stage 4 ub into slot 0, the next kAhead stages in registers,
  // unit ub's weights current and unit ub + 1's in flight (stage parity is
  // that of q, the stage within its unit)
#pragma unroll
  for (int ct = 0; ct < CT; ++ct)
    U::template load<WIDE>(trec[ct] + static_cast<uint64_t>(ub) * R.bytes, lane, cur[ct]);
  a_load(std::integral_constant<int, 0>{}, 4 * ub);
  a_load(std::integral_constant<int, 1>{}, 4 * ub + 1);
  a_store(std::integral_constant<int, 0>{}, 0);
  a_load(std::integral_constant<int, 0>{}, 4 * ub + 2);
  b_load(ub + 1);
#pragma unroll
  for (int ct = 0; ct < CT; ++ct) U::template scales<WIDE>(g, cur[ct], sa[ct], sb[ct]);
  if constexpr (QT == kQ4_K) {
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) q4k_affine(sa[ct], sb[ct]);
  }

  for (uint32_t u = ub; u < ue; ++u) {
    // stage s = 4u + q: its activations are in slot q & 1; stages s + 1 ..
    // s + kAhead are in registers, stage s + 1 in ar[(q + 1) % kAhead]
    static_assert(4 % kAhead == 0, "the ring index below assumes kAhead divides 4");
    auto step = [&](auto qc) {
      constexpr int q = decltype(qc)::value;
      constexpr int p1 = (q + 1) % kAhead;
      const uint32_t s = 4 * u + q;
      __syncthreads();
      if (s + 1 < stages) {
        a_store(std::integral_constant<int, p1>{}, (q + 1) & 1);
        a_load(std::integral_constant<int, p1>{}, s + 1 + kAhead);
      }
      const uint8_t* A = lds + (q & 1) * kStage;
#pragma unroll
      for (int tt = 0; tt < 2; ++tt) {
        const int t = 2 * q + tt, w = t / U::kSteps;
        h8 af[RT], bf[CT];
#pragma unroll
        for (int rt = 0; rt < RT; ++rt)
          af[rt] = *reinterpret_cast<const h8*>(A + ((tt * 8 + rt0 + rt) * 64 + lane) * 16);
#pragma unroll
        for (int ct = 0; ct < CT; ++ct) {
          if constexpr (QT == kQ4_K) bf[ct] = q4k_fragment(cur[ct], t, sa[ct][w], sb[ct][w]);
          else bf[ct] = weight_fragment<QT>(U::codes(cur[ct], g, t), sa[ct][w], sb[ct][w]);
        }
#pragma unroll
        for (int ct = 0; ct < CT; ++ct)
#pragma unroll
          for (int rt = 0; rt < RT; ++rt)
            acc[rt][ct] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[rt], bf[ct], acc[rt][ct], 0, 0, 0);
      }
      if constexpr (q == 3) {
        // unit u + 1 becomes current; the next records are loaded after this
        // stage's activation loads, so waiting for those never waits for these
#pragma unroll
        for (int ct = 0; ct < CT; ++ct) cur[ct] = nxt[ct];
#pragma unroll
        for (int ct = 0; ct < CT; ++ct) U::template scales<WIDE>(g, cur[ct], sa[ct], sb[ct]);
        if constexpr (QT == kQ4_K) {
#pragma unroll
          for (int ct = 0; ct < CT; ++ct) q4k_affine(sa[ct], sb[ct]);
        }
        b_load(u + 2);
      }
    };
    step(std::integral_constant<int, 0>{});
    step(std::integral_constant<int, 1>{});
    step(std::integral_constant<int, 2>{});
    step(std::integral_constant<int, 3>{});
  }

  // C[i][j]: lane j + 16 (i / 4), element i % 4
  static_assert(RT == 8 && rt0 == 0, "the SiLU epilogue takes the whole 128-row block");
  if (a.act != nullptr) {
    gemm_store_silu<CT>(a, acc, tile0, m0, g, c16);
    return;
  }
  const uint64_t ld = a.w.n;
  float* const out = a.splits > 1 ? a.part + static_cast<uint64_t>(blockIdx.z) * a.m_pad * ld : a.y;
  float* yrow = out + (m0 + 16 * rt0 + 4 * g) * ld;
  bool bad = false;
#pragma unroll
  for (int ct = 0; ct < CT; ++ct) {
    const uint64_t n = static_cast<uint64_t>(tile0 + ct) * 16 + c16;
    if (n >= a.w.n) continue;
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const uint64_t m = m0 + 16 * (rt0 + rt) + 4 * g + r;
        if (m < a.m) {
          yrow[(rt * 16 + r) * ld + n] = acc[rt][ct][r];
          bad |= !__builtin_isfinite(acc[rt][ct][r]);
        }
      }
    }
  }
  // with a K split the partial sums are checked by gemm_splitk_sum_kernel
  if (bad && a.splits == 1)
    gemm_fix_nonfinite<QT, WIDE, CT>(a, m0 + 16 * rt0 + 4 * g, RT, static_cast<uint64_t>(tile0) * 16 + c16);
}

// s_waitcnt with vmcnt <= n (0..63) and lgkmcnt 0 (gfx9 encoding: vmcnt in
// bits 3:0 and 15:14, expcnt 6:4 left at its maximum, lgkmcnt 11:8).
template <int N>
__device__ __forceinline__ void wait_vm_lgkm0() {
  static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | ((N >> 4) << 14));
}

// Q4_K and Q5_K (f16 scales) with both operands staged in LDS by direct
// global-to-LDS loads, so no register holds data in flight and every
// vector-memory instruction of the main loop is one of these copies, a known
// number per stage, which lets a stage wait for exactly the copy it needs:
//   activations: 2-step stages (16 KB, fragment order) in a ring of 4 LDS
//     slots, stage s + 3 requested at the top of stage s (P = 16 / W copies
//     of 1 KB per wavefront, W wavefronts per workgroup);
//   weights: each wavefront copies its CT = 16 / W tiles' records of unit
//     u + 1 (LdsRec<QT>::kCopies instructions per record) into the other of
//     its two LDS buffers at the top of unit u, and reads its code words and
//     scales from there when the unit becomes current.
// Waits at the top of stage s = 4u + q (copies issued after the one needed
// stay in flight): q = 0: the stage's activations, 2 P younger copies
// (stages s + 1, s + 2); q = 1, 2: 2 P + the unit's record copies; q = 3: the
// next unit's records, 2 P younger copies. The raw s_barrier (no fence) keeps
// the other copies in flight; the wait before it also drains this
// wavefront's LDS reads, so the slot the new copy overwrites is free.
// W = 8: a wavefront owns 128 rows x 2 output tiles (about 170 registers),
// two wavefronts per SIMD; measured against W = 4 (4 tiles each, one per
// SIMD): Q4_K 2048x4096x12288 245.5 -> 240.6 us, 512x4096x4096 50.1 -> 46.2,
// Q5_K 2048x4096x12288 295.1 -> 272.7. Tiling, arithmetic and split-K as
// gemm_reg_kernel. Each step dequantizes its fragments before its matrix
// instructions (dequantizing one step ahead measured slower here: the second
// fragment set costs registers).
constexpr uint32_t kLdsSlots = 4, kLdsStage = 2 * 8 * 64 * 16;
constexpr int kLdsWaves = 8;  // wavefronts per workgroup (16 output tiles over them)

typedef __attribute__((address_space(3))) void* lds_ptr;

template <int QT>
struct LdsRec;  // record copy into LDS and read-back for gemm_lds_kernel

// The record reads use inline assembly: the compiler tracks all global-to-LDS
// copies as one group and would otherwise wait for every copy in flight (the
// prefetched activation stages too) before them. The copy they need was
// waited for at the top of the stage; the closing wait passes every result
// through, so no use can move above it. Tile CT's record sits at CT * kBytes.
template <>
struct LdsRec<kQ4_K> {
  static constexpr Record R = record_geometry(kQ4_K, false);
  static constexpr uint32_t kBytes = R.bytes, kCopies = 3;
  static_assert(kBytes == 2304 && R.sc == 2048 && R.d == 2240 && R.dmin == 2272,
                "the copies and reads below hard-code the Q4_K record layout");
  // 2 x 1 KB + 256 B (64 lanes x 4 B)
  __device__ static void copy(const uint8_t* src, uint8_t* dst, uint32_t lane) {
    __builtin_amdgcn_global_load_lds(src + static_cast<uint32_t>(lane * 16), (lds_ptr)dst, 16, 0, 0);
    __builtin_amdgcn_global_load_lds(src + static_cast<uint32_t>(1024 + lane * 16), (lds_ptr)(dst + 1024), 16, 0,
                                     0);
    __builtin_amdgcn_global_load_lds(src + static_cast<uint32_t>(2048 + lane * 4), (lds_ptr)(dst + 2048), 4, 0, 0);
  }
  template <int CT>
  __device__ static void read(uint32_t base, uint32_t lane, Unit<kQ4_K>::Raw cur[CT]) {
    const uint32_t c16 = lane & 15;
    const uint32_t aq = base + lane * 16, asc = base + R.sc + c16 * 12, ad = base + R.d + c16 * 2;
    u32x4 q0[4], q1[4];
    uint32_t sc0[4], sc1[4], sc2[4], d0[4], d1[4];
#define QI_Q4K_TILE_READ(CT)                                                                         \
  asm volatile("ds_read_b128 %0, %7 offset:" #CT "*2304\n\t"                                       \
               "ds_read_b128 %1, %7 offset:" #CT "*2304+1024\n\t"                                  \
               "ds_read_b32 %2, %8 offset:" #CT "*2304\n\t"                                        \
               "ds_read_b32 %3, %8 offset:" #CT "*2304+4\n\t"                                      \
               "ds_read_b32 %4, %8 offset:" #CT "*2304+8\n\t"                                      \
               "ds_read_u16 %5, %9 offset:" #CT "*2304\n\t"                                        \
               "ds_read_u16 %6, %9 offset:" #CT "*2304+32"                                          \
               : "=&v"(q0[CT]), "=&v"(q1[CT]), "=&v"(sc0[CT]), "=&v"(sc1[CT]), "=&v"(sc2[CT]),     \
                 "=&v"(d0[CT]), "=&v"(d1[CT])                                                      \
               : "v"(aq), "v"(asc), "v"(ad))
    QI_Q4K_TILE_READ(0);
    QI_Q4K_TILE_READ(1);
    if constexpr (CT == 4) {
      QI_Q4K_TILE_READ(2);
      QI_Q4K_TILE_READ(3);
      asm volatile("s_waitcnt lgkmcnt(0)"
                   : "+v"(q0[0]), "+v"(q1[0]), "+v"(sc0[0]), "+v"(sc1[0]), "+v"(sc2[0]), "+v"(d0[0]), "+v"(d1[0]),
                     "+v"(q0[1]), "+v"(q1[1]), "+v"(sc0[1]), "+v"(sc1[1]), "+v"(sc2[1]), "+v"(d0[1]), "+v"(d1[1]),
                     "+v"(q0[2]), "+v"(q1[2]), "+v"(sc0[2]), "+v"(sc1[2]), "+v"(sc2[2]), "+v"(d0[2]), "+v"(d1[2]),
                     "+v"(q0[3]), "+v"(q1[3]), "+v"(sc0[3]), "+v"(sc1[3]), "+v"(sc2[3]), "+v"(d0[3]), "+v"(d1[3]));
    } else {
      static_assert(CT == 2, "2 or 4 tiles per wavefront");
      asm volatile("s_waitcnt lgkmcnt(0)"
                   : "+v"(q0[0]), "+v"(q1[0]), "+v"(sc0[0]), "+v"(sc1[0]), "+v"(sc2[0]), "+v"(d0[0]), "+v"(d1[0]),
                     "+v"(q0[1]), "+v"(q1[1]), "+v"(sc0[1]), "+v"(sc1[1]), "+v"(sc2[1]), "+v"(d0[1]), "+v"(d1[1]));
    }
#undef QI_Q4K_TILE_READ
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) {
      cur[ct].q[0] = __builtin_bit_cast(uint4, q0[ct]);
      cur[ct].q[1] = __builtin_bit_cast(uint4, q1[ct]);
      cur[ct].sc[0] = sc0[ct];
      cur[ct].sc[1] = sc1[ct];
      cur[ct].sc[2] = sc2[ct];
      cur[ct].s0 = d0[ct];
      cur[ct].s1 = d1[ct];
    }
  }
};

template <>
struct LdsRec<kQ5_K> {
  static constexpr Record R = record_geometry(kQ5_K, false);
  static constexpr uint32_t kBytes = R.bytes, kCopies = 5;
  static_assert(kBytes == 2816 && R.qh == 2048 && R.sc == 2560 && R.d == 2752 && R.dmin == 2784,
                "the copies and reads below hard-code the Q5_K record layout");
  // 2 x 1 KB + 3 x 256 B (64 lanes x 4 B)
  __device__ static void copy(const uint8_t* src, uint8_t* dst, uint32_t lane) {
    __builtin_amdgcn_global_load_lds(src + static_cast<uint32_t>(lane * 16), (lds_ptr)dst, 16, 0, 0);
    __builtin_amdgcn_global_load_lds(src + static_cast<uint32_t>(1024 + lane * 16), (lds_ptr)(dst + 1024), 16, 0,
                                     0);
#pragma unroll
    for (uint32_t i = 0; i < 3; ++i)
      __builtin_amdgcn_global_load_lds(src + static_cast<uint32_t>(2048 + 256 * i + lane * 4),
                                       (lds_ptr)(dst + 2048 + 256 * i), 4, 0, 0);
  }
  template <int CT>
  __device__ static void read(uint32_t base, uint32_t lane, Unit<kQ5_K>::Raw cur[CT]) {
    const uint32_t c16 = lane & 15;
    const uint32_t aq = base + lane * 16, ah = base + R.qh + c16 * 16, asc = base + R.sc + c16 * 12,
                   ad = base + R.d + c16 * 2;
    u32x4 q0[4], q1[4], h0[4], h1[4];
    uint32_t sc0[4], sc1[4], sc2[4], d0[4], d1[4];
#define QI_Q5K_TILE_READ(CT)                                                                         \
  asm volatile("ds_read_b128 %0, %9 offset:" #CT "*2816\n\t"                                       \
               "ds_read_b128 %1, %9 offset:" #CT "*2816+1024\n\t"                                  \
               "ds_read_b128 %2, %10 offset:" #CT "*2816\n\t"                                      \
               "ds_read_b128 %3, %10 offset:" #CT "*2816+256\n\t"                                  \
               "ds_read_b32 %4, %11 offset:" #CT "*2816\n\t"                                       \
               "ds_read_b32 %5, %11 offset:" #CT "*2816+4\n\t"                                     \
               "ds_read_b32 %6, %11 offset:" #CT "*2816+8\n\t"                                     \
               "ds_read_u16 %7, %12 offset:" #CT "*2816\n\t"                                       \
               "ds_read_u16 %8, %12 offset:" #CT "*2816+32"                                         \
               : "=&v"(q0[CT]), "=&v"(q1[CT]), "=&v"(h0[CT]), "=&v"(h1[CT]), "=&v"(sc0[CT]),       \
                 "=&v"(sc1[CT]), "=&v"(sc2[CT]), "=&v"(d0[CT]), "=&v"(d1[CT])                      \
               : "v"(aq), "v"(ah), "v"(asc), "v"(ad))
    QI_Q5K_TILE_READ(0);
    QI_Q5K_TILE_READ(1);
    if constexpr (CT == 4) {
      QI_Q5K_TILE_READ(2);
      QI_Q5K_TILE_READ(3);
      asm volatile("s_waitcnt lgkmcnt(0)"
                   : "+v"(q0[0]), "+v"(q1[0]), "+v"(h0[0]), "+v"(h1[0]), "+v"(sc0[0]), "+v"(sc1[0]), "+v"(sc2[0]),
                     "+v"(d0[0]), "+v"(d1[0]), "+v"(q0[1]), "+v"(q1[1]), "+v"(h0[1]), "+v"(h1[1]), "+v"(sc0[1]),
                     "+v"(sc1[1]), "+v"(sc2[1]), "+v"(d0[1]), "+v"(d1[1]), "+v"(q0[2]), "+v"(q1[2]), "+v"(h0[2]),
                     "+v"(h1[2]), "+v"(sc0[2]), "+v"(sc1[2]), "+v"(sc2[2]), "+v"(d0[2]), "+v"(d1[2]), "+v"(q0[3]),
                     "+v"(q1[3]), "+v"(h0[3]), "+v"(h1[3]), "+v"(sc0[3]), "+v"(sc1[3]), "+v"(sc2[3]), "+v"(d0[3]),
                     "+v"(d1[3]));
    } else {
      static_assert(CT == 2, "2 or 4 tiles per wavefront");
      asm volatile("s_waitcnt lgkmcnt(0)"
                   : "+v"(q0[0]), "+v"(q1[0]), "+v"(h0[0]), "+v"(h1[0]), "+v"(sc0[0]), "+v"(sc1[0]), "+v"(sc2[0]),
                     "+v"(d0[0]), "+v"(d1[0]), "+v"(q0[1]), "+v"(q1[1]), "+v"(h0[1]), "+v"(h1[1]), "+v"(sc0[1]),
                     "+v"(sc1[1]), "+v"(sc2[1]), "+v"(d0[1]), "+v"(d1[1]));
    }
#undef QI_Q5K_TILE_READ
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) {
      cur[ct].q[0] = __builtin_bit_cast(uint4, q0[ct]);
      cur[ct].q[1] = __builtin_bit_cast(uint4, q1[ct]);
      cur[ct].h[0] = __builtin_bit_cast(uint4, h0[ct]);
      cur[ct].h[1] = __builtin_bit_cast(uint4, h1[ct]);
      cur[ct].sc[0] = sc0[ct];
      cur[ct].sc[1] = sc1[ct];
      cur[ct].sc[2] = sc2[ct];
      cur[ct].s0 = d0[ct];
      cur[ct].s1 = d1[ct];
    }
  }
};

template <int QT>
constexpr uint32_t lds_gemm_bytes() {
  return kLdsSlots * kLdsStage + 4 * 2 * 4 * LdsRec<QT>::kBytes;
}

template <int QT, int W>
__global__ __launch_bounds__(64 * W) void gemm_lds_kernel(GemmArgs a) {
  using U = Unit<QT>;
  using L = LdsRec<QT>;
  static_assert(lds_gemm_bytes<QT>() <= 160 * 1024, "LDS per workgroup");
  constexpr int RT = 8;
  constexpr int CT = 16 / W;                  // output tiles per wavefront
  constexpr int P = 4 * 4 / W;                // activation copies per stage and wavefront
  constexpr uint32_t kWBuf = CT * L::kBytes;  // one wavefront's CT records of a unit
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  uint8_t* const abuf = lds;

  const uint32_t tid = threadIdx.x, lane = tid & 63;
  const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: scalar addressing
  const uint32_t g = lane >> 4, c16 = lane & 15;
  uint8_t* const wbuf = lds + kLdsSlots * kLdsStage + wave * 2 * kWBuf;
  const uint32_t units = a.w.units;
  const uint32_t ub = blockIdx.z * units / a.splits, ue = (blockIdx.z + 1) * units / a.splits;
  const uint64_t m0 = static_cast<uint64_t>(blockIdx.y) * kTileM;
  const uint32_t stages = 4 * ue;
  const u32x4* xa = reinterpret_cast<const u32x4*>(a.xh) + static_cast<uint64_t>(blockIdx.y) * units * 4096;

  const uint32_t tile0 = (blockIdx.x * W + wave) * CT;
  const uint8_t* trec[CT];
#pragma unroll
  for (int ct = 0; ct < CT; ++ct) {
    const uint32_t t = min(tile0 + ct, a.w.tiles - 1);
    trec[ct] = a.w.qs + static_cast<uint64_t>(t) * units * L::kBytes;
  }

  // stage st's activations (clamped to the last stage) into slot st % 4
  auto copy_stage = [&](uint32_t st) {
    const uint32_t sl = st < stages ? st : stages - 1;
    uint8_t* dst = abuf + (st % kLdsSlots) * kLdsStage;
    // uniform base plus a 32-bit lane offset: the scalar-base addressing form
    const uint8_t* src = reinterpret_cast<const uint8_t*>(xa + static_cast<uint64_t>(sl) * 1024);
#pragma unroll
    for (int i = 0; i < P; ++i)
      __builtin_amdgcn_global_load_lds(src + static_cast<uint32_t>((tid + 64 * W * i) * 16),
                                       (lds_ptr)(dst + (64 * W * i + 64 * wave) * 16), 16, 0, 0);
  };
  // this wavefront's records of unit u (clamped) into its buffer (u - ub) & 1
  auto copy_unit = [&](uint32_t u) {
    const uint32_t ul = u < ue ? u : ue - 1;
    uint8_t* dst = wbuf + ((u - ub) & 1) * kWBuf;
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) L::copy(trec[ct] + static_cast<uint64_t>(ul) * L::kBytes, dst + ct * L::kBytes, lane);
  };

  typename U::Raw cur[CT];
  float sa[CT][U::kWindows], sb[CT][U::kWindows];
  auto take_unit = [&](uint32_t u) {
    typedef __attribute__((address_space(3))) uint8_t* lds_u8;
    L::template read<CT>(static_cast<uint32_t>(reinterpret_cast<uintptr_t>((lds_u8)wbuf)) + ((u - ub) & 1) * kWBuf,
                         lane, cur);
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) {
      U::template scales<false>(g, cur[ct], sa[ct], sb[ct]);
      if constexpr (QT == kQ4_K) q4k_affine(sa[ct], sb[ct]);
    }
  };
  auto frags = [&](auto tc, h8 out[CT]) {
    constexpr int t = decltype(tc)::value, w = t / U::kSteps;
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) {
      if constexpr (QT == kQ4_K) out[ct] = q4k_fragment(cur[ct], t, sa[ct][w], sb[ct][w]);
      else out[ct] = weight_fragment<QT>(U::codes(cur[ct], g, t), sa[ct][w], sb[ct][w]);
    }
  };

  f4 acc[RT][CT];
#pragma unroll
  for (int i = 0; i < RT; ++i)
#pragma unroll
    for (int j = 0; j < CT; ++j) acc[i][j] = f4{0, 0, 0, 0};

  // prologue: stages 4 ub .. 4 ub + 2 and unit ub, all complete
  copy_stage(4 * ub);
  copy_stage(4 * ub + 1);
  copy_stage(4 * ub + 2);
  copy_unit(ub);
  wait_vm_lgkm0<0>();
  __builtin_amdgcn_s_barrier();
  take_unit(ub);

  // copies younger than the one a stage needs: the two next stages' (2 P),
  // at q = 1, 2 also the next unit's records (CT per record copy count)
  constexpr int kMid = 2 * P + CT * static_cast<int>(L::kCopies);
  for (uint32_t u = ub; u < ue; ++u) {
    auto step = [&](auto qc) {
      constexpr int q = decltype(qc)::value;
      const uint32_t s = 4 * u + q;
      if constexpr (q == 1 || q == 2) wait_vm_lgkm0<kMid>();
      else wait_vm_lgkm0<2 * P>();
      __builtin_amdgcn_s_barrier();
      copy_stage(s + 3);
      if constexpr (q == 0) copy_unit(u + 1);
      const uint8_t* A = abuf + (s % kLdsSlots) * kLdsStage;
      auto sub = [&](auto ttc) {
        constexpr int tt = decltype(ttc)::value, t = 2 * q + tt;
        h8 af[RT], bf[CT];
#pragma unroll
        for (int rt = 0; rt < RT; ++rt)
          af[rt] = *reinterpret_cast<const h8*>(A + ((tt * 8 + rt) * 64 + lane) * 16);
        frags(std::integral_constant<int, t>{}, bf);
#pragma unroll
        for (int ct = 0; ct < CT; ++ct)
#pragma unroll
          for (int rt = 0; rt < RT; ++rt)
            acc[rt][ct] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[rt], bf[ct], acc[rt][ct], 0, 0, 0);
        // the next unit's records (waited for at the top of this stage)
        if constexpr (t == 7) take_unit(u + 1);
      };
      sub(std::integral_constant<int, 0>{});
      sub(std::integral_constant<int, 1>{});
    };
    step(std::integral_constant<int, 0>{});
    step(std::integral_constant<int, 1>{});
    step(std::integral_constant<int, 2>{});
    step(std::integral_constant<int, 3>{});
  }
  // the clamped copies past the last stage and unit must land before the
  // workgroup's LDS is released
  wait_vm_lgkm0<0>();

  if (a.act != nullptr) {
    gemm_store_silu<CT>(a, acc, tile0, m0, g, c16);
    return;
  }
  const uint64_t ld = a.w.n;
  float* const out = a.splits > 1 ? a.part + static_cast<uint64_t>(blockIdx.z) * a.m_pad * ld : a.y;
  float* yrow = out + (m0 + 4 * g) * ld;
  bool bad = false;
#pragma unroll
  for (int ct = 0; ct < CT; ++ct) {
    const uint64_t n = static_cast<uint64_t>(tile0 + ct) * 16 + c16;
    if (n >= a.w.n) continue;
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const uint64_t m = m0 + 16 * rt + 4 * g + r;
        if (m < a.m) {
          yrow[(rt * 16 + r) * ld + n] = acc[rt][ct][r];
          bad |= !__builtin_isfinite(acc[rt][ct][r]);
        }
      }
    }
  }
  // with a K split the partial sums are checked by gemm_splitk_sum_kernel
  if (bad && a.splits == 1)
    gemm_fix_nonfinite<QT, false, CT>(a, m0 + 4 * g, RT, static_cast<uint64_t>(tile0) * 16 + c16);
}

// y = sum of the split-K partial products, in split order (deterministic);
// a sum that is not finite is recomputed in the reference's order. The
// partials are loaded eight at a time ahead of their additions, so a thread
// waits for one memory round trip per eight splits (the 2-16 row GEMV's
// four-part sums: Q4_0 4096 x 4096 M=16 15.5 -> 15.0 us per call on MI355X;
// the 16-part sums of 128-row GEMMs are bound by the partials' bytes).
template <int QT, bool WIDE>
__global__ __launch_bounds__(256) void gemm_splitk_sum_kernel(const float* __restrict__ part, uint32_t splits,
                                                              uint64_t count, uint64_t stride,
                                                              float* __restrict__ y, View w,
                                                              const float* __restrict__ x) {
  const uint64_t i = static_cast<uint64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i >= count) return;
  float v = part[i];
  uint32_t s = 1;
  for (; s + 8 <= splits; s += 8) {
    float t[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) t[j] = part[(s + j) * stride + i];
#pragma unroll
    for (int j = 0; j < 8; ++j) v += t[j];
  }
  for (; s < splits; ++s) v += part[s * stride + i];
  if (!__builtin_isfinite(v)) v = exact_output_row<QT, WIDE>(w, x + (i / w.n) * w.k, i % w.n);
  y[i] = v;
}

namespace {

template <int QT, bool WIDE>
hipError_t launch_reg(const Image& im, const GemmArgs& a, hipStream_t st) {
  const uint32_t nblk = static_cast<uint32_t>((im.tiles + 15) / 16);
  const uint32_t mblk = static_cast<uint32_t>(a.m_pad / kTileM);
  if (a.splits < 1 || a.splits > im.k / 256 || (a.splits > 1 && a.part == nullptr)) return hipErrorInvalidValue;
  hipLaunchKernelGGL((gemm_reg_kernel<QT, WIDE, kRegWaves>), dim3(nblk, mblk, a.splits), dim3(64 * kRegWaves), 0, st,
                     a);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || a.splits == 1) return e;
  // rows of y and of each partial block share the row stride n
  const uint64_t count = a.m * im.n;
  hipLaunchKernelGGL((gemm_splitk_sum_kernel<QT, WIDE>), dim3(static_cast<uint32_t>((count + 255) / 256)),
                     dim3(256), 0, st, a.part, a.splits, count, a.m_pad * im.n, a.y, a.w, a.x);
  return hipGetLastError();
}

template <int QT>
hipError_t launch_lds(const Image& im, const GemmArgs& a, hipStream_t st) {
  const uint32_t nblk = static_cast<uint32_t>((im.tiles + 15) / 16);
  const uint32_t mblk = static_cast<uint32_t>(a.m_pad / kTileM);
  if (a.splits < 1 || a.splits > im.k / 256 || (a.splits > 1 && a.part == nullptr)) return hipErrorInvalidValue;
  auto kern = gemm_lds_kernel<QT, kLdsWaves>;
  constexpr uint32_t bytes = lds_gemm_bytes<QT>();
  hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                     hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(bytes));
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(kern, dim3(nblk, mblk, a.splits), dim3(64 * kLdsWaves), bytes, st, a);
  e = hipGetLastError();
  if (e != hipSuccess || a.splits == 1) return e;
  const uint64_t count = a.m * im.n;
  hipLaunchKernelGGL((gemm_splitk_sum_kernel<QT, false>), dim3(static_cast<uint32_t>((count + 255) / 256)),
                     dim3(256), 0, st, a.part, a.splits, count, a.m_pad * im.n, a.y, a.w, a.x);
  return hipGetLastError();
}

template <int QT, bool WIDE>
hipError_t launch_ws(const Image& im, const GemmArgs& a, hipStream_t st) {
  const uint32_t nblk = static_cast<uint32_t>((im.tiles + 15) / 16);
  const uint32_t mblk = static_cast<uint32_t>(a.m_pad / kTileM);
  constexpr uint32_t bytes = 2 * (2 * 8 * 64 * 16 + 2 * 16 * 64 * 16);
  auto kern = gemm_ws_kernel<QT, WIDE>;
  hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                     hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(bytes));
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(kern, dim3(nblk, mblk), dim3(512), bytes, st, a);
  return hipGetLastError();
}

// Q6_K's dequantization (low nibble + 2 high bits, signed 8-bit scales) is
// the heaviest; the kernel with dedicated dequantizing wavefronts runs it
// faster (660 vs 631 TFLOP/s at 2048 x 4096 x 12288 on MI355X). The other
// types run faster with each wavefront dequantizing its own fragments.
constexpr bool use_ws(int qtype) { return qtype == kQ6_K; }

template <int QT>
hipError_t launch_q(const Image& im, const GemmArgs& a, hipStream_t st) {
  if constexpr (use_ws(QT)) {
    return im.wide ? launch_ws<QT, true>(im, a, st) : launch_ws<QT, false>(im, a, st);
  } else {
    // activations in fragment order, then the register-weight kernel
    const uint32_t blocks = static_cast<uint32_t>(a.m_pad / kTileM * (im.k / 256) * 4);
    hipLaunchKernelGGL((x_to_frag_kernel<QT>), dim3(blocks), dim3(256), 0, st, a.x, a.m,
                       static_cast<uint32_t>(im.k), a.xh);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    // Q4_K and Q5_K with f16 scales: both operands staged in LDS (faster on
    // MI355X: Q4_K 743 against 681 TFLOP/s at 2048 x 4096 x 12288);
    // QI_HIP_GEMM_REG=1 selects the register-weight kernel instead
    if constexpr (QT == kQ4_K || QT == kQ5_K) {
      if (!im.wide && getenv("QI_HIP_GEMM_REG") == nullptr) return launch_lds<QT>(im, a, st);
    }
    return im.wide ? launch_reg<QT, true>(im, a, st) : launch_reg<QT, false>(im, a, st);
  }
}

}  // namespace

hipError_t launch_splitk_sum(const Image& im, const View& v, const float* part, uint32_t splits,
                             uint64_t count, uint64_t stride, float* y, const float* x, hipStream_t st) {
  const dim3 grid(static_cast<uint32_t>((count + 255) / 256));
  auto go = [&](auto kern) {
    hipLaunchKernelGGL(kern, grid, dim3(256), 0, st, part, splits, count, stride, y, v, x);
    return hipGetLastError();
  };
  const bool w = im.wide != 0;
  switch (im.qtype) {
    case kQ8_0: return w ? go(gemm_splitk_sum_kernel<kQ8_0, true>) : go(gemm_splitk_sum_kernel<kQ8_0, false>);
    case kQ4_0: return w ? go(gemm_splitk_sum_kernel<kQ4_0, true>) : go(gemm_splitk_sum_kernel<kQ4_0, false>);
    case kQ4_K: return w ? go(gemm_splitk_sum_kernel<kQ4_K, true>) : go(gemm_splitk_sum_kernel<kQ4_K, false>);
    case kQ5_K: return w ? go(gemm_splitk_sum_kernel<kQ5_K, true>) : go(gemm_splitk_sum_kernel<kQ5_K, false>);
    case kQ6_K: return w ? go(gemm_splitk_sum_kernel<kQ6_K, true>) : go(gemm_splitk_sum_kernel<kQ6_K, false>);
    default: return hipErrorInvalidValue;
  }
}

bool gemm_supported(int32_t qtype, int32_t layout, uint64_t k, uint64_t n) {
  (void)n;
  return layout == kOutputRows && qtype >= kQ8_0 && qtype <= kQ6_K && k % 256 == 0 && k > 0;
}

uint64_t gemm_padded_rows(uint64_t m) { return (m + kTileM - 1) / kTileM * kTileM; }

bool gemm_silu_supported(const Image& im) { return im.tiled && !use_ws(im.qtype) && im.n % 16 == 0; }

uint32_t gemm_splits(const Image& im, uint64_t m) {
  // The register-weight kernel runs one workgroup per CU (256 on MI355X),
  // each walking its K range at the latency of one workgroup; with fewer row
  // x column blocks than CUs, split K so the launch fills the CUs once
  // (M = 512, N = 4096: 64 blocks x 4 splits). The Q6_K kernel does not split.
  if (use_ws(im.qtype) || !im.tiled) return 1;
  const uint64_t blocks = (im.tiles + 15) / 16 * (gemm_padded_rows(m) / kTileM);
  const uint64_t units = im.k / 256;
  uint64_t s = blocks >= 256 ? 1 : 256 / blocks;
  if (s > units) s = units;
  return static_cast<uint32_t>(s < 1 ? 1 : s);
}

hipError_t launch_gemm(const Image& im, const GemmArgs& a, hipStream_t st) {
  if (!im.tiled || a.xh == nullptr || a.m_pad != gemm_padded_rows(a.m)) return hipErrorInvalidValue;
  if (use_ws(im.qtype)) {
    const uint64_t elems = a.m_pad * im.k;
    const uint32_t blocks = static_cast<uint32_t>((elems / 8 + 255) / 256);
    hipLaunchKernelGGL(x_to_f16_kernel, dim3(blocks), dim3(256), 0, st, a.x, a.m, im.k, a.m_pad, a.xh);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  switch (im.qtype) {
    case kQ8_0: return launch_q<kQ8_0>(im, a, st);
    case kQ4_0: return launch_q<kQ4_0>(im, a, st);
    case kQ4_K: return launch_q<kQ4_K>(im, a, st);
    case kQ5_K: return launch_q<kQ5_K>(im, a, st);
    case kQ6_K: return launch_q<kQ6_K>(im, a, st);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace qi
