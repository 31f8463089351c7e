// Prefill GEMM on the f16 matrix cores (v_mfma_f32_16x16x32_f16), output-rows
// layout, K a multiple of 256, any M (meant for M >= 128).
//
// Arithmetic. The activations are rounded once to f16 (x_to_f16_kernel, rows
// padded to the 128-row tile with zeros). Each weight is rounded once to f16:
// Q8_0 / Q4_0 as (code - bias) * d, an exact f16 integer times the stored f16
// scale; the K-quants from the reference's own f32 value (d * sc) * q -
// dmin * m (Q6_K (d * sc) * (q - 32)), so no rounding is shared by the 32
// weights of a sub-block (rounding d * sc or dmin * m to f16 would be, and
// cancels badly in blocks whose range an outlier stretched). Products
// accumulate in f32 on the matrix cores. This is the tolerance-judged MFMA
// mode (f16 operands, f32 accumulation).
//
// Tiling. A workgroup of WN wavefronts owns 128 activation rows x 64 WN
// outputs; each wavefront owns all 128 rows and its own 64 outputs, i.e. 8 x 4
// MFMA tiles of 16 x 16 (128 f32 accumulators per lane), so a weight fragment
// feeds 8 MFMAs. K runs in units of 256, each as two stages of 4 MFMA steps.
// Step t of a unit covers, for lane group g, elements window_first(g, t / 4) +
// 8 (t % 4) + [0, 8) on both operands, the element order the weight records
// store, so neither operand is reshuffled:
//   A (activations) is staged per stage through LDS, double buffered, laid out
//     [step][row tile][lane] x 16 bytes so that a fragment read is 1 KB
//     contiguous, shared by the workgroup's wavefronts;
//   B (weights) never touches LDS: each wavefront streams its 4 output tiles'
//     records of the next unit into registers (the GEMV's coalesced loads)
//     while it computes the current one, and dequantizes the 8 codes of a
//     step into an f16 fragment right before the 8 MFMAs that use it.
#include "qi_device.h"
#include "qi_internal.h"
#include "qi_unit.h"

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
    const uint32_t w[2] = {static_cast<uint32_t>(codes),
                           static_cast<uint32_t>(static_cast<uint64_t>(codes) >> 32)};
    const float nb = QT == kQ6_K ? -32.0f * a : -b;  // Q6_K: (d * sc) * (q - 32) = a * q - 32 a
    h8 out;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float q = static_cast<float>((w[j >> 2] >> (8 * (j & 3))) & 0xFFu);
      out[j] = static_cast<_Float16>(fmaf(a, q, nb));
    }
    return out;
  }
}

// Two elements (2p, 2p + 1) of a step's f16 weight fragment, as one packed
// register, from the step's 8 code bytes w[2]: the same arithmetic as
// weight_fragment, split so that it can be spread between MFMA issues.
template <int QT>
__device__ __forceinline__ uint32_t weight_pair(const uint32_t w[2], float a, float b, int p) {
  uint32_t word = w[p >> 1];
  if constexpr (QT == kQ8_0 || QT == kQ4_0) {
    if constexpr (QT == kQ8_0) word ^= 0x80808080u;
    constexpr float bias = QT == kQ8_0 ? 1152.0f : 1032.0f;
    const h2 sub = {static_cast<_Float16>(bias), static_cast<_Float16>(bias)};
    const h2 q = __builtin_bit_cast(h2, __builtin_amdgcn_perm(0x64646464u, word, (p & 1) ? 0x04030402u
                                                                                   : 0x04010400u)) - sub;
    const _Float16 ha = static_cast<_Float16>(a);
    return __builtin_bit_cast(uint32_t, q * h2{ha, ha});
  } else {
    // the codes as exact f16 integers, then fma in f32 with one rounding to
    // f16 (v_fma_mix: f16 code, f32 scale and offset)
    const float nb = QT == kQ6_K ? -32.0f * a : -b;
    const h2 sub = {static_cast<_Float16>(1024.0f), static_cast<_Float16>(1024.0f)};
    const h2 q = __builtin_bit_cast(h2, __builtin_amdgcn_perm(0x64646464u, word, (p & 1) ? 0x04030402u
                                                                                   : 0x04010400u)) - sub;
    const h2 r = {static_cast<_Float16>(fmaf(a, static_cast<float>(q[0]), nb)),
                  static_cast<_Float16>(fmaf(a, static_cast<float>(q[1]), nb))};
    return __builtin_bit_cast(uint32_t, r);
  }
}

// Workgroup: WN wavefronts side by side, each owning 128 activation rows x 64
// outputs (8 x 4 MFMA tiles); the workgroup covers 128 rows x 64 WN outputs.
// Activations are staged four MFMA steps (half a unit) at a time.
//
// Load order per unit (vector loads complete in order, so a wait for one load
// is a wait for every older one): the activations of the next stage first,
// then the next unit's weights. The wait at the end of stage 0 (for the stage
// 1 activations) then leaves the weights in flight; they are waited for only
// at the end of stage 1, two stages after they were issued.
template <int QT, bool WIDE, int WN>
__global__ __launch_bounds__(64 * WN) void gemm_kernel(GemmArgs a) {
  using U = Unit<QT>;
  constexpr Record R = record_geometry(QT, WIDE);
  constexpr uint32_t kStage = 4 * 8 * 64 * 16;  // [step][row tile][lane] x 16 B = 32 KB
  // element offset of stage h (0/1) within a unit: window_first(g, h) - window_first(g, 0)
  constexpr uint32_t kHalf = QT == kQ6_K ? 64 : 32;
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];

  const uint32_t tid = threadIdx.x, lane = tid & 63, wn = tid >> 6;
  const uint32_t g = lane >> 4, c16 = lane & 15;
  const uint32_t units = a.w.units;
  const uint32_t K = static_cast<uint32_t>(a.w.k);
  const uint64_t m0 = static_cast<uint64_t>(blockIdx.y) * kTileM;

  // this wavefront's 4 output tiles (clamped: past-the-end tiles re-read the
  // last tile and store nothing)
  const uint8_t* trec[4];
  uint32_t tile_raw[4];
#pragma unroll
  for (int ct = 0; ct < 4; ++ct) {
    tile_raw[ct] = (blockIdx.x * WN + wn) * 4 + ct;
    const uint32_t t = min(tile_raw[ct], a.w.tiles - 1);
    trec[ct] = a.w.qs + static_cast<uint64_t>(t) * units * R.bytes;
  }

  // Staging of one stage (128 rows x 4 lane groups x 32 elements, 32 KB):
  // thread t owns row 16 rt + i with i = t % 16, lane group sg = (t / 16) % 4
  // and row tiles rt = t / 64 + 4 p (p = 0, 1); it loads that row's 32
  // elements window_first(sg, h) + [0, 32) as four 16-byte chunks (steps tt)
  // and writes chunk tt to slot 16 sg + i of block (tt, rt). One store
  // instruction of a wavefront thus fills one contiguous 1 KB block (no LDS
  // bank conflicts), the same pattern the fragment reads use.
  static_assert(WN == 4, "staging assumes 4 wavefronts");
  constexpr int kChunks = 8;
  const uint32_t si = tid & 15, sg = (tid >> 4) & 3, srt = tid >> 6;
  const _Float16* abase = a.xh + (m0 + 16 * srt + si) * K + window_first<QT>(sg, 0);
  const uint64_t apass = static_cast<uint64_t>(64) * K;  // 4 row tiles further down
  const uint32_t sbase = (srt * 64 + sg * 16 + si) * 16;

  // staging registers: a native vector array (HIP's uint4 wraps a union,
  // which keeps a returned copy out of registers); index 4 p + tt
  u32x4 areg[kChunks];
#define QI_STAGE_LOAD(U_, H_)                                                           \
  do {                                                                                  \
    const _Float16* p_ = abase + 256 * (U_) + kHalf * (H_);                             \
    _Pragma("unroll") for (int i_ = 0; i_ < kChunks; ++i_) areg[i_] =                   \
        *reinterpret_cast<const u32x4*>(p_ + (i_ >> 2) * apass + 8 * (i_ & 3));         \
  } while (0)
#define QI_STAGE_STORE(BUF_)                                                            \
  do {                                                                                  \
    uint8_t* p_ = lds + (BUF_) * kStage + sbase;                                        \
    _Pragma("unroll") for (int i_ = 0; i_ < kChunks; ++i_)                              \
        *reinterpret_cast<u32x4*>(p_ + ((i_ & 3) * 8 + 4 * (i_ >> 2)) * 64 * 16) = areg[i_]; \
  } while (0)

  f4 acc[8][4];
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f4{0, 0, 0, 0};

  typename U::Raw cur[4], nxt[4];
  QI_STAGE_LOAD(0u, 0u);
#pragma unroll
  for (int ct = 0; ct < 4; ++ct) U::template load<WIDE>(trec[ct], lane, cur[ct]);
  QI_STAGE_STORE(0u);
  __syncthreads();

  // Software pipeline: while the 32 MFMAs of a step issue, the operands of
  // the next step are prepared in between them (one MFMA, then a slice of the
  // LDS reads and of the weight dequantization, fenced by sched_barrier so
  // that the matrix core and the VALU overlap), including across stages and
  // into the next unit (whose weights were prefetched two stages earlier).
  float sa[4][U::kWindows], sb[4][U::kWindows];
#pragma unroll
  for (int ct = 0; ct < 4; ++ct) U::template scales<WIDE>(g, cur[ct], sa[ct], sb[ct]);
  uint32_t bk[4][4];  // the current step's weight fragments, packed f16 pairs
#pragma unroll
  for (int ct = 0; ct < 4; ++ct) {
    const uint64_t c = static_cast<uint64_t>(U::codes(cur[ct], g, 0));
    const uint32_t w[2] = {static_cast<uint32_t>(c), static_cast<uint32_t>(c >> 32)};
#pragma unroll
    for (int p = 0; p < 4; ++p) bk[ct][p] = weight_pair<QT>(w, sa[ct][0], sb[ct][0], p);
  }

  uint32_t buf = 0;
  for (uint32_t u = 0; u < units; ++u) {
    const bool next_unit = u + 1 < units;
    // after the last unit the prefetches re-read it (unused, always in bounds)
    const uint32_t un = next_unit ? u + 1 : u;
    float nsa[4][U::kWindows], nsb[4][U::kWindows];
    // the two stages of the unit, with the stage index a compile-time constant
    // (a runtime step index would put the per-window arrays in scratch memory)
    auto stage = [&](auto hc) {
      constexpr uint32_t h = decltype(hc)::value;
      QI_STAGE_LOAD(h == 0 ? u : un, h ^ 1);
      if constexpr (h == 0) {
#pragma unroll
        for (int ct = 0; ct < 4; ++ct)
          U::template load<WIDE>(trec[ct] + static_cast<uint64_t>(un) * R.bytes, lane, nxt[ct]);
      } else {
#pragma unroll
        for (int ct = 0; ct < 4; ++ct) U::template scales<WIDE>(g, nxt[ct], nsa[ct], nsb[ct]);
      }
      const uint8_t* sb_ = lds + buf * kStage;
      h8 af[8];
#pragma unroll
      for (int rt = 0; rt < 8; ++rt)
        af[rt] = *reinterpret_cast<const h8*>(sb_ + (rt * 64 + lane) * 16);
#pragma unroll
      for (int tt = 0; tt < 4; ++tt) {
        const int t = 4 * static_cast<int>(h) + tt;
        const bool to_next_unit = t == 7;  // the next step is the next unit's step 0
        h8 afn[8];
        uint32_t bn[4][4];
        uint32_t cw[2] = {0, 0};
        float ca = 0.0f, cb = 0.0f;
#pragma unroll
        for (int i = 0; i < 32; ++i) {
          const int ct = i >> 3, rt = i & 7;
          acc[rt][ct] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[rt], __builtin_bit_cast(h8, bk[ct]),
                                                              acc[rt][ct], 0, 0, 0);
          if (tt < 3 && i < 8)
            afn[i] = *reinterpret_cast<const h8*>(sb_ + (((tt + 1) * 8 + i) * 64 + lane) * 16);
          const int j = i & 7;
          if (j == 0) {
            const int tn = to_next_unit ? 0 : t + 1;
            const uint64_t c = static_cast<uint64_t>(to_next_unit ? U::codes(nxt[ct], g, 0)
                                                                  : U::codes(cur[ct], g, tn));
            cw[0] = static_cast<uint32_t>(c);
            cw[1] = static_cast<uint32_t>(c >> 32);
            const int w = tn / U::kSteps;
            ca = to_next_unit ? nsa[ct][0] : sa[ct][w];
            cb = to_next_unit ? nsb[ct][0] : sb[ct][w];
          }
          if (j & 1) bn[ct][j >> 1] = weight_pair<QT>(cw, ca, cb, j >> 1);
          __builtin_amdgcn_sched_barrier(0);
        }
        if (tt < 3) {
#pragma unroll
          for (int i = 0; i < 8; ++i) af[i] = afn[i];
        }
#pragma unroll
        for (int ct = 0; ct < 4; ++ct)
#pragma unroll
          for (int p = 0; p < 4; ++p) bk[ct][p] = bn[ct][p];
      }
      QI_STAGE_STORE(buf ^ 1);
      __syncthreads();
      buf ^= 1;
    };
    stage(std::integral_constant<uint32_t, 0>{});
    stage(std::integral_constant<uint32_t, 1>{});
#pragma unroll
    for (int ct = 0; ct < 4; ++ct) {
      cur[ct] = nxt[ct];
#pragma unroll
      for (int w = 0; w < U::kWindows; ++w) {
        sa[ct][w] = nsa[ct][w];
        sb[ct][w] = nsb[ct][w];
      }
    }
  }

  // C[i][j]: lane j + 16 (i / 4), element i % 4
  const uint64_t ld = a.w.n;
  float* yrow = a.y + (m0 + 4 * g) * ld;
#pragma unroll
  for (int ct = 0; ct < 4; ++ct) {
    const uint64_t n = static_cast<uint64_t>(tile_raw[ct]) * 16 + c16;
    if (n >= a.w.n) continue;
#pragma unroll
    for (int rt = 0; rt < 8; ++rt) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const uint64_t m = m0 + rt * 16 + 4 * g + r;
        if (m < a.m) yrow[(rt * 16 + r) * ld + n] = acc[rt][ct][r];
      }
    }
  }
}

#undef QI_STAGE_LOAD
#undef QI_STAGE_STORE

namespace {

template <int QT, bool WIDE, int WN>
hipError_t launch_wn(const Image& im, const GemmArgs& a, hipStream_t st) {
  const uint32_t nblk = static_cast<uint32_t>((im.tiles + 4 * WN - 1) / (4 * WN));
  const uint32_t mblk = static_cast<uint32_t>(a.m_pad / kTileM);
  hipLaunchKernelGGL((gemm_kernel<QT, WIDE, WN>), dim3(nblk, mblk), dim3(64 * WN), 2 * 4 * 8 * 64 * 16,
                     st, a);
  return hipGetLastError();
}

template <int QT>
hipError_t launch_q(const Image& im, const GemmArgs& a, hipStream_t st) {
  return im.wide ? launch_wn<QT, true, 4>(im, a, st) : launch_wn<QT, false, 4>(im, a, st);
}

}  // namespace

bool gemm_supported(int32_t qtype, int32_t layout, uint64_t k, uint64_t n) {
  (void)n;
  return layout == kOutputRows && qtype >= kQ8_0 && qtype <= kQ6_K && k % 256 == 0 && k > 0;
}

uint64_t gemm_padded_rows(uint64_t m) { return (m + kTileM - 1) / kTileM * kTileM; }

hipError_t launch_gemm(const Image& im, const GemmArgs& a, hipStream_t st) {
  if (!im.tiled || a.xh == nullptr || a.m_pad != gemm_padded_rows(a.m)) return hipErrorInvalidValue;
  const uint64_t elems = a.m_pad * im.k;
  const uint32_t blocks = static_cast<uint32_t>((elems / 8 + 255) / 256);
  hipLaunchKernelGGL(x_to_f16_kernel, dim3(blocks), dim3(256), 0, st, a.x, a.m, im.k, a.m_pad, a.xh);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
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
