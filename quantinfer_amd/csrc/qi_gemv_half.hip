// Decode GEMV of 9-16 activation rows on the f16 matrix cores
// (v_mfma_f32_16x16x32_f16), output-rows layout, K a multiple of 256; one
// kernel per call after one activation-record kernel (K parts over the grid
// only for shapes with few tiles).
//
// Arithmetic ("split halves"). Per (row, unit of 256 elements) the
// activations are scaled by a power of two 2^s that brings the unit's largest
// |x| just under 2^15, and each scaled value x' is held as two f16 numbers,
// hi = x' truncated to 11 significant bits and lo = f16(x' - hi), which carry
// 22 significant bits of it. The weight codes enter the matrix cores as exact
// small f16 integers, centred: q - z with z the middle of the code range
// (Q4_0 8, Q6_K 32), a zero point per (output, window) for Q4_K / Q5_K (the
// integer nearest b / a), Q8_0's signed codes as they are. All products are
// exact in f32; per (row, window of 32, output), with w = a q - b,
//   sum_k x'_k w_k = a * (C_hi + C_lo) - (b - z a) * sum_k x'_k,
// where C_hi / C_lo are the matrix-core sums of the two halves against the
// centred codes, and the unit's sum is multiplied by 2^-s once. The rounding
// is that of f32 sums of exact products, plus x to 22 bits: within the 1e-5
// bars of the f32 GEMV at every K (no cancellation: the centred codes leave
// an offset of at most a / 2 for the K-quants).
//
// Q8_0 / Q4_0 / Q6_K. One 16x16x32 instruction covers one window for all 16
// rows (A: lane (m, g) = lane m + 16 g supplies 8 values of row m, k-slots
// 8g..8g+7) and the tile's 16 outputs (B: lane (n, g) supplies output n's
// codes of the same slots); lane (n, g) receives rows 4g..4g+3 of output n.
// The weight record gives lane group g two whole windows of its output; the B
// operand needs slice g of every window, so the code words are transposed
// across the four lane groups with v_permlane32_swap / v_permlane16_swap, and
// the window scales, decoded by their owning lane group, are gathered the same
// way; the window scale a is applied by one f32 fma per window and output.
// Q6_K's 16-element sub-blocks (two per window) take two instructions per
// half, each with the other sub-block's codes zeroed, weighted by their own
// int8 scales. A 16-bit pair of the B operand is made from two code bytes with
// one v_and_or_b32 (the code in the low mantissa bits under the exponent of
// 1024: 1024 + q, or 1024 + 16 q for a high nibble) and centred with one
// packed f16 add or fma (exact: integers below 2048); the slots of a lane
// group hold elements (0, 2), (1, 3), (4, 6), (5, 7) of its slice in that
// order, and the activation halves are stored in the same order.
//
// Q4_K / Q5_K take the split GEMM's operand order instead (qi_half.h): the
// activations in each lane group's own element order, so that no codes move
// between lanes, B = sc (q - z) with the 6-bit window scale folded in (exact
// in f16), one combine per unit (d times the matrix sum), and the offsets of
// the unit's eight windows on one more f16 instruction.
//
// Work split: a workgroup is 16 wavefronts, 4 tiles of 16 outputs x 4 K
// slices (or, for shapes of up to one tile per CU, one tile x 16 K slices,
// so that no K part leaves the workgroup). The record kernel converts the
// call's activations once; each workgroup copies those of its K range into
// LDS (chunk by chunk when they do not fit), each wavefront streams its
// tile's units of its slice, and the slices are summed in order through LDS.
// The copies are waited for before the weight loads are issued (vector loads
// complete in order), so that the copies are not queued behind the weights.
// No state is shared between workgroups. Rows past M hold zeros and are never
// stored. A NaN or infinite activation (or a sum of |x| that overflows) makes
// its (row, unit) scale NaN, so every output of the row comes out non-finite
// and is recomputed in the reference's order.
#include "qi_device.h"
#include "qi_internal.h"
#include "qi_half.h"
#include "qi_unit.h"

namespace qi {

namespace {

using namespace half;


constexpr int kHThreads = 1024;  // 16 wavefronts
constexpr int kHWaves = 16;
constexpr uint32_t kHCUs = 256;  // compute units of an MI355X (gfx950)
constexpr int kHRows = 16;      // rows of the A operand (9-16 activation rows)

// LDS of a chunk of `cu` units for MR rows, the records' layout: Q8_0 /
// Q4_0 / Q6_K the halves [unit][window][half][row][lane group] x 16 B, then
// the window sums [unit][row][window] and the unscales 2^-s [unit][row] as
// f32; Q4_K / Q5_K the units' stages (SplitStage<MR>), of the same size.
constexpr uint32_t half_lds(int mr, uint32_t cu) { return cu * static_cast<uint32_t>(mr) * (1024 + 32 + 4); }
constexpr uint32_t half_chunk_cap(int mr) { return 128 / static_cast<uint32_t>(mr); }
static_assert(half_lds(16, 8) <= 160 * 1024 && half_lds(4, 32) <= 160 * 1024, "chunks fit LDS");

// A workgroup barrier that waits for this wavefront's LDS accesses but not
// for its vector-memory loads (weights may stay in flight); the compiler moves
// no memory access across it.
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

__device__ __forceinline__ void xpose4(uint32_t r[4]) {
  const auto a = __builtin_amdgcn_permlane32_swap(r[0], r[2], false, false);
  const auto b = __builtin_amdgcn_permlane32_swap(r[1], r[3], false, false);
  const auto c = __builtin_amdgcn_permlane16_swap(a[0], b[0], false, false);
  const auto d = __builtin_amdgcn_permlane16_swap(a[1], b[1], false, false);
  r[0] = c[0];
  r[1] = c[1];
  r[2] = d[0];
  r[3] = d[1];
}


// Per-format weight access of one unit: load() the record bytes (the
// one-row kernel's loaders), prepare() the transposes, then for window w the
// centred f16 codes of slice g and, from the scales, the window's factor and
// offset.
template <int QT>
struct Half;

template <>
struct Half<kQ8_0> {
  using U = Unit<kQ8_0>;
  static constexpr bool kSplit = false;
  struct T {
    uint32_t lo[2][4], hi[2][4];
  };
  __device__ static void prepare(const U::Raw& r, T& t) {
#pragma unroll
    for (int b = 0; b < 2; ++b) {
      t.lo[b][0] = r.q[2 * b].x; t.lo[b][1] = r.q[2 * b].z; t.lo[b][2] = r.q[2 * b + 1].x; t.lo[b][3] = r.q[2 * b + 1].z;
      t.hi[b][0] = r.q[2 * b].y; t.hi[b][1] = r.q[2 * b].w; t.hi[b][2] = r.q[2 * b + 1].y; t.hi[b][3] = r.q[2 * b + 1].w;
      xpose4(t.lo[b]);
      xpose4(t.hi[b]);
    }
  }
  // signed bytes s: 1024 + (s ^ 128) - 1152 = s
  __device__ static void codes(const T& t, int w, uint32_t out[4]) {
    const uint32_t lo = t.lo[w & 1][w >> 1] ^ 0x80808080u, hi = t.hi[w & 1][w >> 1] ^ 0x80808080u;
    raw_pairs<kMaskByte>(lo, hi, lo >> 8, hi >> 8, out);
    const h2 c = splat(-1152.0f);
#pragma unroll
    for (int i = 0; i < 4; ++i) out[i] = pk_add(out[i], c);
  }
};

template <>
struct Half<kQ4_0> {
  using U = Unit<kQ4_0>;
  static constexpr bool kSplit = false;
  static constexpr uint32_t kM = 0x0F0F0F0Fu;
  struct T {
    uint32_t w[2][4];
  };
  // block 2g + b in q[b] (byte i = element i | element i+16 << 4); slice s as
  // one word, byte k = element 8s+k | element 8s+4+k << 4
  __device__ static void prepare(const U::Raw& r, T& t) {
#pragma unroll
    for (int b = 0; b < 2; ++b) {
      const uint4 q = r.q[b];
      t.w[b][0] = (q.x & kM) | ((q.y << 4) & ~kM);
      t.w[b][1] = (q.z & kM) | ((q.w << 4) & ~kM);
      t.w[b][2] = ((q.x >> 4) & kM) | (q.y & ~kM);
      t.w[b][3] = ((q.z >> 4) & kM) | (q.w & ~kM);
      xpose4(t.w[b]);
    }
  }
  __device__ static void codes(const T& t, int w, uint32_t out[4]) {
    const uint32_t v = t.w[w & 1][w >> 1], v8 = v >> 8;
    out[0] = pk_add(and_or(v, kMaskLo, kExp1024), splat(-1032.0f));                     // elements 0, 2: q - 8
    out[1] = pk_add(and_or(v8, kMaskLo, kExp1024), splat(-1032.0f));                    // 1, 3
    out[2] = pk_fma(and_or(v, kMaskHi, kExp1024), splat(0.0625f), splat(-72.0f));       // 4, 6: (1024 + 16q) / 16 - 72
    out[3] = pk_fma(and_or(v8, kMaskHi, kExp1024), splat(0.0625f), splat(-72.0f));      // 5, 7
  }
};

// Q4_K / Q5_K take the split GEMM's operands (split_stage, split_scales,
// split_codes): activations in each lane group's own element order, so that
// the weight codes need no lane transposes, with the 6-bit window scales
// folded into exact f16 codes sc (q - z) and one combine per unit.
template <int QT>
struct HalfSplit {
  using U = Unit<QT>;
  static constexpr bool kSplit = true;
};
template <>
struct Half<kQ4_K> : HalfSplit<kQ4_K> {};
template <>
struct Half<kQ5_K> : HalfSplit<kQ5_K> {};

// Q6_K: lane group g' = 2ip + c holds ql bytes [64ip + 32c, +32); window
// w = 4ip + 2hf + c is their low (hf = 0) or high (hf = 1) nibbles, its two
// high bits bits 2c + 4hf of qh bytes 32ip + 8g..8g+7 (RowsUnit<kQ6_K>).
template <>
struct Half<kQ6_K> {
  using U = RowsUnit<kQ6_K>;
  static constexpr bool kSplit = false;
  struct T {
    uint32_t lo[4], hi[4];
    uint32_t h[4];
  };
  __device__ static void prepare(const U::Raw& r, T& t) {
    t.lo[0] = r.q[0].x; t.lo[1] = r.q[0].z; t.lo[2] = r.q[1].x; t.lo[3] = r.q[1].z;
    t.hi[0] = r.q[0].y; t.hi[1] = r.q[0].w; t.hi[2] = r.q[1].y; t.hi[3] = r.q[1].w;
    xpose4(t.lo);
    xpose4(t.hi);
#pragma unroll
    for (int i = 0; i < 4; ++i) t.h[i] = r.h[i];
  }
  // 4q in each byte (nibble to bits 2-5, high bits to 6-7), as 1024 + 4q pairs
  __device__ static void raw(const T& t, int w, uint32_t out[4]) {
    const int ip = w >> 2, hf = (w >> 1) & 1, c = w & 1, gp = 2 * ip + c;
    const int up = 6 - 2 * c - 4 * hf;
    const uint32_t lo = (((hf ? t.lo[gp] >> 2 : t.lo[gp] << 2)) & 0x3C3C3C3Cu) | ((t.h[2 * ip] << up) & 0xC0C0C0C0u);
    const uint32_t hi = (((hf ? t.hi[gp] >> 2 : t.hi[gp] << 2)) & 0x3C3C3C3Cu) | ((t.h[2 * ip + 1] << up) & 0xC0C0C0C0u);
    raw_pairs<kMaskByte>(lo, hi, lo >> 8, hi >> 8, out);
  }
};

struct HalfArgs {
  View w;
  const float* x;  // [m, k]
  float* y;        // [m, n]
  int m;
  uint32_t chunk_units;  // units per LDS chunk
  uint32_t part_units;   // units per K part (grid.y)
  float* part;           // [grid.y][m][n] when grid.y > 1
  const uint8_t* rec;    // the call's activation records (half_prep_kernel / half_stage_kernel)
  const float* rsum;     // half_prep_kernel's window sums, then unscales
};


// The call's activation records, built once. Q8_0 / Q4_0 / Q6_K
// (half_prep_kernel): for all K / 256 units, the halves [unit][window][half]
// [row < MR][lane group] x 16 B, then the window sums [unit][row][window] and
// the unscales [unit][row] (f32) -- the LDS layout of a chunk, so that a chunk
// is three contiguous copies. Q4_K / Q5_K (half_stage_kernel): the units'
// stages (SplitStage<MR>) in order, of the same size.
constexpr uint64_t half_records_size(uint64_t units, int mr) {
  return units * static_cast<uint64_t>(mr) * (1024 + 32 + 4);
}

// One (row, unit) per 32 threads: item r = 4 w + g of the 32.
template <int MR>
__global__ __launch_bounds__(256) void half_prep_kernel(const float* __restrict__ x, uint32_t K, int M,
                                                        uint8_t* __restrict__ rec) {
  const uint32_t units = K / 256;
  const uint32_t pair = blockIdx.x * 8 + (threadIdx.x >> 5);  // u * MR + m
  const uint32_t r = threadIdx.x & 31, w = r >> 2, g = r & 3;
  // whole half-wavefronts are in or out (the lane moves stay within them)
  if (pair >= units * MR) return;
  const uint32_t u = pair / MR, m = pair % MR;
  float4 v0 = make_float4(0.0f, 0.0f, 0.0f, 0.0f), v1 = v0;
  if (static_cast<int>(m) < M) {
    const float4* p = reinterpret_cast<const float4*>(x + static_cast<uint64_t>(m) * K + u * 256 + 32 * w + 8 * g);
    v0 = p[0];
    v1 = p[1];
  }
  const float v[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
  uint8_t* const hs = rec + ((((u * 8 + w) * 2) * MR + m) * 4 + g) * 16;
  float* const xsum = reinterpret_cast<float*>(rec + static_cast<uint64_t>(units) * MR * 1024);
  float* const unsc = xsum + units * MR * 8;
  half_convert(v, hs, hs + MR * 64, xsum + pair * 8 + w, unsc + pair, w, g);
}

// Q4_K / Q5_K: one stage (split_stage) of rows 0..MR-1 per unit, the units in
// order; a workgroup converts 8 rows of one unit (grid: units x MR / 8).
template <int MR>
__global__ __launch_bounds__(256) void half_stage_kernel(const float* __restrict__ x, uint32_t K, int M,
                                                         uint8_t* __restrict__ rec) {
  split_stage<MR, false>(x, K, static_cast<uint64_t>(M), 0, blockIdx.x,
                         rec + static_cast<uint64_t>(blockIdx.x) * SplitStage<MR>::kBytes, blockIdx.y, blockIdx.y + 1);
}
static_assert(SplitStage<kHRows>::kBytes == kHRows * (1024 + 32 + 4), "stages and records of one size");

// MR rows held (M <= MR), D units of weights in flight per wavefront, TL
// tiles per workgroup (4, or 1 with 16 K slices).
template <int QT, bool WIDE, int MR, int D, int TL>
__global__ __launch_bounds__(kHThreads) void gemv_half_kernel(HalfArgs a) {
  constexpr int SL = kHWaves / TL;  // K slices per tile
  using H = Half<QT>;
  using U = typename H::U;
  constexpr Record R = record_geometry(QT, WIDE);
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  const uint32_t cu = a.chunk_units;
  uint8_t* const planes = lds;
  float* const xsum = reinterpret_cast<float*>(lds + cu * MR * 1024);
  float* const unsc = xsum + cu * MR * 8;

  const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const uint32_t sw = wave % SL, wc = wave / SL;
  const uint32_t col = lane & 15, g = lane >> 4;
  const uint32_t tile_raw = blockIdx.x * TL + wc;
  const uint32_t tile = min(tile_raw, a.w.tiles - 1);
  const uint32_t units_total = a.w.units;
  const uint8_t* const trec = a.w.qs + static_cast<uint64_t>(tile) * units_total * R.bytes;
  const uint32_t K = static_cast<uint32_t>(a.w.k);
  const int M = a.m;
  const uint32_t u_lo = blockIdx.y * a.part_units;
  const uint32_t u_hi = min(units_total, u_lo + a.part_units);

  v4f acc = {0.0f, 0.0f, 0.0f, 0.0f};
  typename U::Raw ring[D];

  for (uint32_t ku0 = u_lo; ku0 < u_hi; ku0 += cu) {
    const uint32_t units = min(cu, u_hi - ku0);
    const uint32_t u_begin = (units * sw) / SL;
    const uint32_t u_count = (units * (sw + 1)) / SL - u_begin;
    if (ku0 != u_lo) __syncthreads();  // the previous chunk is consumed

    // ---- the chunk's activation records: Q4_K / Q5_K stages (split_stage)
    // as one contiguous copy; otherwise (half_prep_kernel) the halves by 1 KB
    // global-to-LDS copies, the window sums and unscales by 256 B ones
    if constexpr (H::kSplit) {
      const uint8_t* const src = a.rec + static_cast<uint64_t>(ku0) * SplitStage<MR>::kBytes;
      const uint32_t bytes = units * SplitStage<MR>::kBytes;
      for (uint32_t j = wave; 1024 * j < bytes; j += kHWaves)
        if (1024 * j + 16 * lane < bytes)
          __builtin_amdgcn_global_load_lds(src + 1024 * j + 16 * lane,
                                           (__attribute__((address_space(3))) void*)(planes + 1024 * j), 16, 0, 0);
    } else {
      const uint8_t* const src = a.rec + static_cast<uint64_t>(ku0) * MR * 1024;
      const uint32_t kb = units * MR;  // KB of halves
      for (uint32_t j = wave; j < kb; j += kHWaves)
        __builtin_amdgcn_global_load_lds(src + 1024 * j + 16 * lane,
                                         (__attribute__((address_space(3))) void*)(planes + 1024 * j), 16, 0, 0);
      const float* const ssrc = a.rsum + static_cast<uint64_t>(ku0) * MR * 8;
      const float* const usrc = a.rsum + static_cast<uint64_t>(units_total) * MR * 8 + ku0 * MR;
      const uint32_t nsum = units * MR * 8, nun = units * MR;  // floats
      for (uint32_t j = wave; j * 64 < nsum; j += kHWaves)
        if (j * 64 + lane < nsum)
          __builtin_amdgcn_global_load_lds(ssrc + 64 * j + lane,
                                           (__attribute__((address_space(3))) void*)(xsum + 64 * j), 4, 0, 0);
      for (uint32_t j = wave; j * 64 < nun; j += kHWaves)
        if (j * 64 + lane < nun)
          __builtin_amdgcn_global_load_lds(usrc + 64 * j + lane,
                                           (__attribute__((address_space(3))) void*)(unsc + 64 * j), 4, 0, 0);
    }
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): the weights queue behind nothing
#pragma unroll
    for (int i = 0; i < D; ++i)
      if (i < static_cast<int>(u_count))
        U::template load<WIDE, true>(trec + (ku0 + u_begin + i) * R.bytes, lane, ring[i]);
    // every wavefront's copies have landed; a barrier with no wait for the
    // weight loads (a fenced one would wait for them)
    lds_barrier();
    auto consume = [&](uint32_t j) {
#pragma unroll
      for (int i = 0; i < D; ++i) {
        if (j + i >= u_count) break;
        const uint32_t u = u_begin + j + i;  // chunk-relative unit
        const typename U::Raw& r = ring[i];
        if constexpr (H::kSplit) {
          // lane (row col, lane group g) of step t's A operand at stage lane
          // 16 g + col; B: sc (q - z) of the lane group's windows; the two
          // nibble halves' chains interleaved
          using S = SplitStage<MR>;
          const uint8_t* const st = planes + u * S::kBytes;
          SplitScales sc;
          split_scales<QT, WIDE>(r, g, sc);
          v4f tmp[2] = {{0.0f, 0.0f, 0.0f, 0.0f}, {0.0f, 0.0f, 0.0f, 0.0f}};
#pragma unroll
          for (int p = 0; p < 4; ++p)
#pragma unroll
            for (int h = 0; h < 2; ++h) {
              const int t = 4 * h + p;
              uint32_t b[1][4];
              split_codes<QT>(r, g, t, sc, b);
              const uint8_t* const ap = st + (t * 64 + lane) * 16;
              const h8 ahi = *reinterpret_cast<const h8*>(ap);
              const h8 alo = *reinterpret_cast<const h8*>(ap + S::kHalf);
              const h8 b0 = __builtin_bit_cast(h8, make_uint4(b[0][0], b[0][1], b[0][2], b[0][3]));
              tmp[h] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ahi, b0, tmp[h], 0, 0, 0);
              tmp[h] = __builtin_amdgcn_mfma_f32_16x16x32_f16(alo, b0, tmp[h], 0, 0, 0);
            }
          // offsets on one f16 instruction (as in the split GEMM): S / 64 of
          // windows 2g, 2g + 1 of row col as halves against sc.bo
          const float* const sums = reinterpret_cast<const float*>(st + S::kSums);
          float sh[2], sl[2];
          split_f16(sums[(2 * g) * MR + col] * 0x1p-6f, sh[0], sl[0]);
          split_f16(sums[(2 * g + 1) * MR + col] * 0x1p-6f, sh[1], sl[1]);
          const uint32_t ah = pack_rtz(sh[0], sh[1]);
          const h8 ao = __builtin_bit_cast(h8, make_uint4(ah, ah, pack_rtz(sl[0], sl[1]), 0u));
          const v4f off = __builtin_amdgcn_mfma_f32_16x16x32_f16(ao, __builtin_bit_cast(h8, sc.bo),
                                                                 v4f{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
          const float4 us = *reinterpret_cast<const float4*>(st + S::kUnsc + 16 * g);
          const float uu[4] = {us.x, us.y, us.z, us.w};
#pragma unroll
          for (int q = 0; q < 4; ++q) acc[q] = fmaf(uu[q], fmaf(sc.fo, off[q], sc.d * (tmp[0][q] + tmp[1][q])), acc[q]);
        } else {
          typename H::T ct;
          H::prepare(r, ct);
          v4f ua = {0.0f, 0.0f, 0.0f, 0.0f};
          // rows past MR read row MR - 1 (their sums are never stored)
          const uint32_t arow = col < static_cast<uint32_t>(MR) ? col : MR - 1;
          const uint8_t* const ab = planes + ((u * 16) * MR + arow) * 64 + g * 16;  // window 0, hi
          if constexpr (QT == kQ6_K) {
            const float d = U::template d<WIDE>(r);
            const h2 k0 = splat(g < 2 ? 0.25f : 0.0f), c0 = splat(g < 2 ? -288.0f : 0.0f);
            const h2 k1 = splat(g < 2 ? 0.0f : 0.25f), c1 = splat(g < 2 ? 0.0f : -288.0f);
#pragma unroll
            for (int w = 0; w < 8; ++w) {
              uint32_t raw[4], b0[4], b1[4];
              H::raw(ct, w, raw);
#pragma unroll
              for (int q = 0; q < 4; ++q) {
                b0[q] = pk_fma(raw[q], k0, c0);
                b1[q] = pk_fma(raw[q], k1, c1);
              }
              const uint32_t swd = U::window_scales(r, w);
              const int hf = (w >> 1) & 1;
              const float a0 = d * static_cast<float>(static_cast<int32_t>(swd << (24 - 16 * hf)) >> 24);
              const float a1 = d * static_cast<float>(static_cast<int32_t>(swd << (16 - 16 * hf)) >> 24);
              const h8 ahi = *reinterpret_cast<const h8*>(ab + w * 2 * MR * 64);
              const h8 alo = *reinterpret_cast<const h8*>(ab + (w * 2 + 1) * MR * 64);
              const h8 bb0 = __builtin_bit_cast(h8, make_uint4(b0[0], b0[1], b0[2], b0[3]));
              const h8 bb1 = __builtin_bit_cast(h8, make_uint4(b1[0], b1[1], b1[2], b1[3]));
              v4f c0v = __builtin_amdgcn_mfma_f32_16x16x32_f16(ahi, bb0, v4f{0, 0, 0, 0}, 0, 0, 0);
              c0v = __builtin_amdgcn_mfma_f32_16x16x32_f16(alo, bb0, c0v, 0, 0, 0);
              v4f c1v = __builtin_amdgcn_mfma_f32_16x16x32_f16(ahi, bb1, v4f{0, 0, 0, 0}, 0, 0, 0);
              c1v = __builtin_amdgcn_mfma_f32_16x16x32_f16(alo, bb1, c1v, 0, 0, 0);
#pragma unroll
              for (int q = 0; q < 4; ++q) ua[q] = fmaf(a1, c1v[q], fmaf(a0, c0v[q], ua[q]));
              // the window's sums are combined here, not after the last window
              // (the compiler would otherwise keep every window's sums live)
              pin(ua);
              __builtin_amdgcn_sched_barrier(0);
            }
          } else {
            // window factors of this lane group's windows 2g, 2g + 1, gathered
            // for all eight: the windows of one h (w = 2g' + h) at a time
            float sa_own[2], sb_own[2];
            U::template scales<WIDE>(g, r, sa_own, sb_own);
#pragma unroll
            for (int h = 0; h < 2; ++h) {
              uint32_t fa[4];
              gather4u(__builtin_bit_cast(uint32_t, sa_own[h]), fa);
              // two windows at a time, their instruction chains interleaved
#pragma unroll
              for (int pp = 0; pp < 2; ++pp) {
                h8 ahi[2], alo[2], bb[2];
#pragma unroll
                for (int e = 0; e < 2; ++e) {
                  const int w = 2 * (2 * pp + e) + h;
                  ahi[e] = *reinterpret_cast<const h8*>(ab + w * 2 * MR * 64);
                  alo[e] = *reinterpret_cast<const h8*>(ab + (w * 2 + 1) * MR * 64);
                }
#pragma unroll
                for (int e = 0; e < 2; ++e) {
                  const int w = 2 * (2 * pp + e) + h;
                  uint32_t bq[4];
                  H::codes(ct, w, bq);
                  bb[e] = __builtin_bit_cast(h8, make_uint4(bq[0], bq[1], bq[2], bq[3]));
                }
                v4f c0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(ahi[0], bb[0], v4f{0, 0, 0, 0}, 0, 0, 0);
                v4f c1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(ahi[1], bb[1], v4f{0, 0, 0, 0}, 0, 0, 0);
                c0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(alo[0], bb[0], c0, 0, 0, 0);
                c1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(alo[1], bb[1], c1, 0, 0, 0);
                const float f0 = __builtin_bit_cast(float, fa[2 * pp]), f1 = __builtin_bit_cast(float, fa[2 * pp + 1]);
#pragma unroll
                for (int q = 0; q < 4; ++q) ua[q] = fmaf(f1, c1[q], fmaf(f0, c0[q], ua[q]));
                // the pair's sums are combined here, not after the last window
                // (the compiler would otherwise keep every window's sums live)
                pin(ua);
                __builtin_amdgcn_sched_barrier(0);
              }
            }
          }
          // the unit's sums of rows 4g..4g+3, unscaled
          const float4 us = *reinterpret_cast<const float4*>(unsc + u * MR + min(4 * g, static_cast<uint32_t>(MR) - 4));
          acc[0] = fmaf(us.x, ua[0], acc[0]);
          acc[1] = fmaf(us.y, ua[1], acc[1]);
          acc[2] = fmaf(us.z, ua[2], acc[2]);
          acc[3] = fmaf(us.w, ua[3], acc[3]);
        }
      }
    };
    consume(0);
    for (uint32_t j = D; j < u_count; j += D) {
#pragma unroll
      for (int i = 0; i < D; ++i)
        if (j + i < u_count) U::template load<WIDE, true>(trec + (ku0 + u_begin + j + i) * R.bytes, lane, ring[i]);
      consume(j);
    }
  }

  // ---- the K slices of each tile, in order ----
  __syncthreads();  // the chunk is no longer read
  float* red = reinterpret_cast<float*>(lds);  // [tile][slice][4][64]
#pragma unroll
  for (int q = 0; q < 4; ++q) red[((wc * SL + sw) * 4 + q) * 64 + lane] = acc[q];
  __syncthreads();
  if (sw != 0) return;
  const uint64_t n_out = static_cast<uint64_t>(tile_raw) * 16 + col;
  if (tile_raw >= a.w.tiles || n_out >= a.w.n) return;
  float* const yout = gridDim.y > 1 ? a.part + static_cast<uint64_t>(blockIdx.y) * M * a.w.n : a.y;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int m = 4 * static_cast<int>(g) + q;
    if (m >= M) continue;
    float v = red[((wc * SL) * 4 + q) * 64 + lane];
#pragma unroll
    for (int p = 1; p < SL; ++p) v += red[((wc * SL + p) * 4 + q) * 64 + lane];
    // NaN or infinite activations (or an overflow): the reference's own order
    // decides which outputs are NaN and which +-Inf
    if (!__builtin_isfinite(v) && gridDim.y == 1)
      v = exact_output_row<QT, WIDE>(a.w, a.x + static_cast<uint64_t>(m) * K, n_out);
    yout[static_cast<uint64_t>(m) * a.w.n + n_out] = v;
  }
}

template <int QT, bool WIDE, int MR, int TL>
hipError_t launch_half_t(HalfArgs a, uint32_t ksplit, hipStream_t st) {
  constexpr int D = 2;
  const uint32_t cap = half_chunk_cap(MR);
  a.chunk_units = a.part_units < cap ? a.part_units : cap;
  const uint32_t main = half_lds(MR, a.chunk_units);
  const uint32_t red = kHWaves * 4 * 64 * 4;
  const uint32_t bytes = main > red ? main : red;
  auto kern = gemv_half_kernel<QT, WIDE, MR, D, TL>;
  if (bytes > 65536) {
    const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                             hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(bytes));
    if (e != hipSuccess) {
      (void)hipGetLastError();
      return e;
    }
  }
  if (ksplit > 1 && a.part == nullptr) return hipErrorInvalidValue;
  hipLaunchKernelGGL(kern, dim3((a.w.tiles + TL - 1) / TL, ksplit), dim3(kHThreads), bytes, st, a);
  return hipGetLastError();
}

// One-tile workgroups (16 K slices, no K split) for shapes of up to one tile
// per CU whose whole K range fits one LDS chunk.
bool half_one_tile(uint64_t k, uint64_t n) {
  return (n + 15) / 16 <= kHCUs && k / 256 <= half_chunk_cap(kHRows);
}

template <int QT, bool WIDE>
hipError_t launch_half_w(const HalfArgs& a, uint32_t ksplit, hipStream_t st) {
  const bool one = half_one_tile(a.w.k, a.w.n);
  if (one && ksplit != 1) return hipErrorInvalidValue;
  return one ? launch_half_t<QT, WIDE, kHRows, 1>(a, ksplit, st) : launch_half_t<QT, WIDE, kHRows, 4>(a, ksplit, st);
}

}  // namespace

uint32_t gemv_half_splits(uint64_t k, uint64_t n, uint32_t m) {
  (void)m;
  if (half_one_tile(k, n)) return 1;
  // one four-tile workgroup per CU; split K only when the tile groups leave
  // most CUs idle, keeping at least 4 units (one per K slice) per part, and
  // return the count the launch runs (every part holds units)
  const uint64_t tiles = (n + 15) / 16, units = k / 256, groups = (tiles + 3) / 4;
  uint64_t s = kHCUs / (groups ? groups : 1);
  const uint64_t most = units / 4 ? units / 4 : 1;
  if (s > most) s = most;
  if (s < 1) s = 1;
  const uint64_t part_units = (units + s - 1) / s;
  return static_cast<uint32_t>((units + part_units - 1) / part_units);
}

uint64_t gemv_half_records_bytes(uint64_t k) { return half_records_size(k / 256, kHRows); }

hipError_t launch_gemv_half_records(int32_t qtype, const float* x, uint64_t k, int m, uint8_t* rec, hipStream_t st) {
  if (m < 9 || m > 16 || k == 0 || k % 256 != 0 || rec == nullptr) return hipErrorInvalidValue;
  if (qtype == kQ4_K || qtype == kQ5_K) {
    hipLaunchKernelGGL(half_stage_kernel<kHRows>, dim3(static_cast<uint32_t>(k / 256), kHRows / 8), dim3(256), 0, st, x,
                       static_cast<uint32_t>(k), m, rec);
    return hipGetLastError();
  }
  const uint32_t pairs = static_cast<uint32_t>(k / 256) * kHRows;
  hipLaunchKernelGGL(half_prep_kernel<kHRows>, dim3((pairs + 7) / 8), dim3(256), 0, st, x,
                     static_cast<uint32_t>(k), m, rec);
  return hipGetLastError();
}

hipError_t launch_gemv_half(int32_t qtype, bool wide, const View& w, const float* x, int m, float* y, float* part,
                            uint32_t ksplit, const uint8_t* rec, hipStream_t st) {
  if (m < 9 || m > 16 || ksplit < 1 || w.k == 0 || w.k % 256 != 0 || rec == nullptr) return hipErrorInvalidValue;
  HalfArgs a{w, x, y, m, 0, 0, part, rec, nullptr};
  const uint32_t units = w.units;
  a.rsum = reinterpret_cast<const float*>(rec + static_cast<uint64_t>(units) * kHRows * 1024);
  a.part_units = (units + ksplit - 1) / ksplit;
  if ((units + a.part_units - 1) / a.part_units != ksplit) return hipErrorInvalidValue;  // every K part holds units
  switch (qtype) {
    case kQ8_0: return wide ? launch_half_w<kQ8_0, true>(a, ksplit, st) : launch_half_w<kQ8_0, false>(a, ksplit, st);
    case kQ4_0: return wide ? launch_half_w<kQ4_0, true>(a, ksplit, st) : launch_half_w<kQ4_0, false>(a, ksplit, st);
    case kQ4_K: return wide ? launch_half_w<kQ4_K, true>(a, ksplit, st) : launch_half_w<kQ4_K, false>(a, ksplit, st);
    case kQ5_K: return wide ? launch_half_w<kQ5_K, true>(a, ksplit, st) : launch_half_w<kQ5_K, false>(a, ksplit, st);
    case kQ6_K: return wide ? launch_half_w<kQ6_K, true>(a, ksplit, st) : launch_half_w<kQ6_K, false>(a, ksplit, st);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace qi
