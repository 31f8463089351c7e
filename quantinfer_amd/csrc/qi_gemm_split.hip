// Prefill GEMM of F32 mode on the f16 matrix cores (v_mfma_f32_16x16x32_f16):
// output rows of every format (Q8_0 / Q4_0 with f16 block scales), K a
// multiple of 256, any M (planned for prompts of 48 rows and more). Its
// results meet the f32 GEMV's bars (1e-5 componentwise and normwise), unlike
// the f16-operand GEMM of qi_gemm.hip. The arithmetic below is that of Q4_K /
// Q5_K; the other formats' weights enter as two f16 planes (SplitFmt).
//
// Arithmetic (the split halves of the 9-16 row GEMV, qi_gemv_half.hip, with
// the sub-block scales folded into the codes). Per (row, unit of 256
// elements) the activations are scaled by a power of two 2^s that brings the
// unit's largest |x| under 2^15 and held as two f16 numbers, hi (x' truncated
// to 11 significant bits) and lo = f16(x' - hi): 22 significant bits of x'.
// A Q4_K / Q5_K weight is w = d sc q - dmin m with d, dmin per unit and the
// 6-bit (sc, m) per 32-element sub-block. With a zero point z per (output,
// sub-block), the integer nearest dmin m / (d sc),
//   w = d * [sc (q - z)] - b',   b' = dmin m - d sc z  (|b'| <= d sc / 2),
// and sc (q - z) is an integer of at most 63 * 31 = 1953 in magnitude, exact
// in f16. So the matrix cores sum exact products x'_hi * sc (q - z) and
// x'_lo * sc (q - z) over the whole unit (both halves into one f32
// accumulator, 16 instructions per 16 x 16 block), and per unit
//   sum_k x_k w_k = 2^-s * (d * C + sum_j S_j * (-b'_j)),
// C the unit's matrix sum, S_j the sum of x' over sub-block j: the eight
// offsets go through one more f16 instruction (window sums and offsets each
// as two f16 halves, scaled by powers of two into f16 range; the three
// products that carry 22 bits), then three f32 operations per output fold
// the unit into the running sum.
// The rounding is that of f32 sums of exact products plus x to 22 bits, as in
// the GEMV, so the same bars hold at every K.
//
// Operands. Step t (0..7) of a unit covers, for lane group g, elements
// 64 g + 32 (t / 4) + 8 (t % 4) + [0, 8): sub-block 2 g + t / 4, the
// record's own code bytes of the lane (qi_image.h), so a lane's B operand
// needs no lane moves and each lane group applies its own sub-block's sc and
// z. A pair of codes becomes 1024 + q (low nibble) or 1024 + 16 q (high) by
// one v_and_or_b32, is centred by one packed f16 add or fma and scaled by
// sc with one packed multiply, all exact. The activation records
// (split_prep_kernel) hold, per (64-row tile, unit), the hi and lo halves in
// this operand order ([half][step][row tile][lane] x 16 B), the 8 window sums
// per row and the unscales 2^-s: one contiguous 66.25 KB stage.
//
// Tiling. A workgroup of 8 wavefronts owns 64 rows x 256 outputs; wavefront
// w holds 4 row tiles x 2 output tiles (tiles 2 w, 2 w + 1), about 200
// registers, so two wavefronts share each SIMD (one workgroup per CU, its
// double-buffered stage taking 133 KB of LDS) and one's matrix instructions
// overlap the other's code construction. Per unit the stage is copied
// global -> LDS (1 KB direct copies, double-buffered, one unit ahead) while
// each wavefront loads its 2 tiles' weight records of the next unit into
// registers. The grid's blocks are dealt XCD-aware (logical
// block (b % 8) * ceil(B / 8) + b / 8, row tiles fastest), so the row tiles
// that share a weight panel run on one XCD's L2. K parts over the grid (for
// shapes with few blocks) write partial sums that launch_splitk_sum adds in
// order. A non-finite output (a NaN or infinite activation) is recomputed in
// the reference's order.
#include "qi_device.h"
#include "qi_half.h"
#include "qi_internal.h"
#include "qi_unit.h"

namespace qi {

namespace {

using namespace half;

constexpr int kSThreads = 512;
constexpr uint32_t kSRows = 64;   // activation rows of a workgroup (4 row tiles)
constexpr uint32_t kSHalf = SplitStage<kSRows>::kHalf;   // one half plane: [step][row tile][lane] x 16 B
constexpr uint32_t kSSums = SplitStage<kSRows>::kSums;   // offset of the window sums [window][row] (f32)
constexpr uint32_t kSUnsc = SplitStage<kSRows>::kUnsc;   // offset of the unscales [row] (f32)
constexpr uint32_t kSStage = SplitStage<kSRows>::kBytes; // bytes of one (row tile, unit) stage
constexpr uint32_t kSCopies = (kSStage + 1023) / 1024;   // 1 KB copies per stage
constexpr uint32_t kSCUs = 256;                          // compute units of an MI355X (gfx950)
static_assert(kSStage % 16 == 0 && 2 * kSStage <= 160 * 1024, "two stages fit LDS");

// One (64-row tile, unit) stage per workgroup (split_stage).
template <bool ORDER6>
__global__ __launch_bounds__(256) void split_prep_kernel(const float* __restrict__ x, uint32_t K, uint64_t M,
                                                         uint8_t* __restrict__ rec) {
  const uint32_t units = K / 256;
  const uint64_t mt = blockIdx.x / units;
  const uint32_t u = blockIdx.x % units;
  split_stage<kSRows, ORDER6>(x, K, M, mt * kSRows, u, rec + (mt * units + u) * kSStage);
}

struct SplitArgs {
  View w;
  const float* x;  // [m, k]: only for the recompute of non-finite outputs
  float* y;        // [m, n]
  uint64_t m;
  const uint8_t* rec;  // the activation stages [row tile][unit]
  uint32_t mtiles, groups, splits;
  float* part;  // [splits][m][n] when splits > 1
};

template <int QT, bool WIDE>
__global__ __launch_bounds__(kSThreads) void gemm_split_kernel(SplitArgs a) {
  using U = Unit<QT>;
  using F = SplitFmt<QT>;
  constexpr int TW = F::kTiles, NP = F::kPlanes;
  constexpr Record R = record_geometry(QT, WIDE);
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];  // two stages

  const uint32_t blocks = a.mtiles * a.groups * a.splits;
  const uint32_t per = (blocks + 7) / 8;
  const uint32_t logical = (blockIdx.x % 8) * per + blockIdx.x / 8;
  if (logical >= blocks) return;
  const uint32_t mt = logical % a.mtiles, rest = logical / a.mtiles;
  const uint32_t grp = rest % a.groups, z = rest / a.groups;

  const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const uint32_t g = lane >> 4, c = lane & 15;
  const uint32_t units = a.w.units;
  const uint32_t ub = z * units / a.splits, ue = (z + 1) * units / a.splits;
  const uint32_t tile0 = (grp * (kSThreads / 64) + wave) * TW;
  const uint8_t* trec[TW];
#pragma unroll
  for (int j = 0; j < TW; ++j) {
    const uint32_t t = min(tile0 + j, a.w.tiles - 1);
    trec[j] = a.w.qs + static_cast<uint64_t>(t) * units * R.bytes;
  }
  const uint8_t* const xrec = a.rec + static_cast<uint64_t>(mt) * units * kSStage;
  auto copy_stage = [&](uint32_t u, uint32_t slot) {
    const uint8_t* const src = xrec + static_cast<uint64_t>(u) * kSStage;
    uint8_t* const dst = lds + slot * kSStage;
    for (uint32_t j = wave; j < kSCopies; j += kSThreads / 64)
      if (1024 * j + 16 * lane < kSStage)
        __builtin_amdgcn_global_load_lds(src + 1024 * j + 16 * lane,
                                         (__attribute__((address_space(3))) void*)(dst + 1024 * j), 16, 0, 0);
  };

  typename U::Raw cur[TW], nxt[TW];
  copy_stage(ub, 0);
#pragma unroll
  for (int j = 0; j < TW; ++j) U::template load<WIDE>(trec[j] + static_cast<uint64_t>(ub) * R.bytes, lane, cur[j]);

  v4f total[4][TW];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < TW; ++j) total[i][j] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
  const v4f zero = {0.0f, 0.0f, 0.0f, 0.0f};

#pragma unroll 1
  for (uint32_t u = ub; u < ue; ++u) {
    const uint32_t slot = (u - ub) & 1;
    // this unit's stage and records have landed (the only loads in flight),
    // and every wavefront is done with the other slot
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
    __syncthreads();
    if (u + 1 < ue) {
      copy_stage(u + 1, slot ^ 1);
#pragma unroll
      for (int j = 0; j < TW; ++j)
        U::template load<WIDE>(trec[j] + static_cast<uint64_t>(u + 1) * R.bytes, lane, nxt[j]);
    }
    const uint8_t* const st = lds + slot * kSStage;
    SplitScales sc[TW];
#pragma unroll
    for (int j = 0; j < TW; ++j) split_scales<QT, WIDE>(cur[j], g, sc[j]);

    v4f tmp[4][TW];
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      uint32_t b[TW][NP][4];
#pragma unroll
      for (int j = 0; j < TW; ++j) split_codes<QT>(cur[j], g, t, sc[j], b[j]);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint8_t* const ap = st + ((t * 4 + i) * 64 + lane) * 16;
        const h8 ahi = *reinterpret_cast<const h8*>(ap);
        const h8 alo = *reinterpret_cast<const h8*>(ap + kSHalf);
#pragma unroll
        for (int j = 0; j < TW; ++j) {
          const h8 b0 = __builtin_bit_cast(h8, make_uint4(b[j][0][0], b[j][0][1], b[j][0][2], b[j][0][3]));
          tmp[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ahi, b0, t == 0 ? zero : tmp[i][j], 0, 0, 0);
          tmp[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(alo, b0, tmp[i][j], 0, 0, 0);
          if constexpr (NP == 2) {
            const h8 b1 = __builtin_bit_cast(h8, make_uint4(b[j][1][0], b[j][1][1], b[j][1][2], b[j][1][3]));
            tmp[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ahi, b1, tmp[i][j], 0, 0, 0);
          }
        }
      }
    }
    // fold the unit in: total += 2^-s (d C [+ window sums x offsets])
    const float* const sums = reinterpret_cast<const float*>(st + kSSums);
    const float* const unsc = reinterpret_cast<const float*>(st + kSUnsc);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float4 us = *reinterpret_cast<const float4*>(unsc + 16 * i + 4 * g);
      const float uu[4] = {us.x, us.y, us.z, us.w};
      if constexpr (F::kK45) {
        // offsets on one f16 instruction: lane (row c, lane group g)
        // supplies S / 64 of windows 2g, 2g+1 (|S| < 2^20) as halves in the
        // slots hi, hi, hi, hi, lo, lo, 0, 0 against the B slots of
        // split_scales: S_hi b_hi + S_hi b_lo + S_lo b_hi of both windows
        float sh[2], sl[2];
        split_f16(sums[(2 * g) * kSRows + 16 * i + c] * 0x1p-6f, sh[0], sl[0]);
        split_f16(sums[(2 * g + 1) * kSRows + 16 * i + c] * 0x1p-6f, sh[1], sl[1]);
        const uint32_t ah = pack_rtz(sh[0], sh[1]);
        const h8 ao = __builtin_bit_cast(h8, make_uint4(ah, ah, pack_rtz(sl[0], sl[1]), 0u));
#pragma unroll
        for (int j = 0; j < TW; ++j) {
          const v4f off = __builtin_amdgcn_mfma_f32_16x16x32_f16(ao, __builtin_bit_cast(h8, sc[j].bo), zero, 0, 0, 0);
#pragma unroll
          for (int r = 0; r < 4; ++r)
            total[i][j][r] = fmaf(uu[r], fmaf(sc[j].fo, off[r], sc[j].d * tmp[i][j][r]), total[i][j][r]);
        }
      } else {
#pragma unroll
        for (int j = 0; j < TW; ++j)
#pragma unroll
          for (int r = 0; r < 4; ++r) total[i][j][r] = fmaf(uu[r], sc[j].d * tmp[i][j][r], total[i][j][r]);
      }
    }
    if (u + 1 < ue) {
#pragma unroll
      for (int j = 0; j < TW; ++j) cur[j] = nxt[j];
    }
  }

  // lane (g, c) holds rows 16 i + 4 g + r of output 16 (tile0 + j) + c
  const uint64_t n = a.w.n;
  float* const out = a.splits > 1 ? a.part + static_cast<uint64_t>(z) * a.m * n : a.y;
  bool bad = false;
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const uint64_t row = static_cast<uint64_t>(mt) * kSRows + 16 * i + 4 * g + r;
#pragma unroll
      for (int j = 0; j < TW; ++j) {
        const uint64_t col = static_cast<uint64_t>(tile0 + j) * 16 + c;
        if (row < a.m && col < n) {
          out[row * n + col] = total[i][j][r];
          bad |= !__builtin_isfinite(total[i][j][r]);
        }
      }
    }
  // with a K split the partial sums are checked by the split-K sum
  if (a.splits == 1 && bad) {
    for (int i = 0; i < 16; ++i) {
      const uint64_t row = static_cast<uint64_t>(mt) * kSRows + 16 * (i >> 2) + 4 * g + (i & 3);
      for (int j = 0; j < TW; ++j) {
        const uint64_t col = static_cast<uint64_t>(tile0 + j) * 16 + c;
        if (row < a.m && col < n && !__builtin_isfinite(a.y[row * n + col]))
          a.y[row * n + col] = exact_output_row<QT, WIDE>(a.w, a.x + row * a.w.k, col);
      }
    }
  }
}

template <int QT, bool WIDE>
hipError_t launch_split_t(const SplitArgs& a, hipStream_t st) {
  auto kern = gemm_split_kernel<QT, WIDE>;
  constexpr uint32_t bytes = 2 * kSStage;
  const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(bytes));
  if (e != hipSuccess) {
    (void)hipGetLastError();
    return e;
  }
  const uint64_t blocks = static_cast<uint64_t>(a.mtiles) * a.groups * a.splits;
  if (blocks > 0x7fffff00ull) return hipErrorInvalidValue;
  hipLaunchKernelGGL(kern, dim3(static_cast<uint32_t>((blocks + 7) / 8 * 8)), dim3(kSThreads), bytes, st, a);
  return hipGetLastError();
}

// 16-output tiles per workgroup (every format: SplitFmt<QT>::kTiles = 2)
uint32_t split_group_tiles() { return (kSThreads / 64) * 2u; }

}  // namespace

bool gemm_split_supported(const Image& im) {
  if (im.tiled == 0 || im.layout != kOutputRows || im.k % 256 != 0 || im.k / 256 > 0xFFFFu) return false;
  switch (im.qtype) {
    case kQ4_K:
    case kQ5_K:
    case kQ6_K: return true;
    case kQ8_0:
    case kQ4_0: return im.wide == 0;  // f16 block scales: exact in the weight halves
    default: return false;
  }
}

uint64_t gemm_split_records_bytes(uint64_t m, uint64_t k) {
  return (m + kSRows - 1) / kSRows * (k / 256) * kSStage;
}

uint32_t gemm_split_splits(const Image& im, uint64_t m) {
  // fill the CUs once when the row and column blocks alone do not, keeping
  // at least 4 units per part; the count returned is the one the launch
  // runs (every part holds units)
  const uint64_t gt = split_group_tiles();
  const uint64_t blocks = (m + kSRows - 1) / kSRows * ((im.tiles + gt - 1) / gt);
  const uint64_t units = im.k / 256;
  if (blocks >= kSCUs || units < 8) return 1;
  uint64_t s = (kSCUs + blocks - 1) / blocks;
  const uint64_t most = units / 4;
  if (s > most) s = most;
  if (s < 1) s = 1;
  const uint64_t part_units = (units + s - 1) / s;
  return static_cast<uint32_t>((units + part_units - 1) / part_units);
}

hipError_t launch_gemm_split(const Image& im, const View& v, const float* x, uint64_t m, float* y, float* part,
                             uint32_t splits, uint8_t* rec, hipStream_t st) {
  if (!gemm_split_supported(im) || m == 0 || rec == nullptr || splits < 1 || splits > im.k / 256 ||
      (splits > 1 && part == nullptr))
    return hipErrorInvalidValue;
  const uint64_t units = im.k / 256, mtiles = (m + kSRows - 1) / kSRows;
  const uint64_t gt = split_group_tiles();
  const uint64_t groups = (im.tiles + gt - 1) / gt;
  if (mtiles * units > 0x7fffffffull || mtiles > 0xFFFFFFu || groups > 0xFFFFFFu) return hipErrorInvalidValue;
  if (im.qtype == kQ6_K)
    hipLaunchKernelGGL(split_prep_kernel<true>, dim3(static_cast<uint32_t>(mtiles * units)), dim3(256), 0, st, x,
                       static_cast<uint32_t>(im.k), m, rec);
  else
    hipLaunchKernelGGL(split_prep_kernel<false>, dim3(static_cast<uint32_t>(mtiles * units)), dim3(256), 0, st, x,
                       static_cast<uint32_t>(im.k), m, rec);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  const SplitArgs a{v, x, y, m, rec, static_cast<uint32_t>(mtiles), static_cast<uint32_t>(groups), splits, part};
  switch (im.qtype) {
    case kQ8_0: e = launch_split_t<kQ8_0, false>(a, st); break;
    case kQ4_0: e = launch_split_t<kQ4_0, false>(a, st); break;
    case kQ4_K: e = im.wide ? launch_split_t<kQ4_K, true>(a, st) : launch_split_t<kQ4_K, false>(a, st); break;
    case kQ5_K: e = im.wide ? launch_split_t<kQ5_K, true>(a, st) : launch_split_t<kQ5_K, false>(a, st); break;
    case kQ6_K: e = im.wide ? launch_split_t<kQ6_K, true>(a, st) : launch_split_t<kQ6_K, false>(a, st); break;
    default: return hipErrorInvalidValue;
  }
  if (e != hipSuccess || splits == 1) return e;
  const uint64_t count = m * im.n;
  return launch_splitk_sum(im, v, part, splits, count, count, y, x, st);
}

}  // namespace qi
