// Decode GEMV on the int8 matrix cores (v_mfma_i32_16x16x64_i8), output-rows
// layout, one activation row, K a multiple of 256.
//
// Arithmetic. The activations are cut into windows of 32 consecutive
// elements. Each activation x of a window becomes a 30-bit fixed-point
// integer F = rint(x * 2^s), with one power of two 2^s per (activation row,
// window) chosen from the window's max |x|, written as four signed 8-bit
// digits F = d0 + d1*2^8 + d2*2^16 + d3*2^24. The weight codes enter the
// matrix cores as signed bytes centred on the middle of their range (Q8_0's
// int8 codes as they are; Q4_0 and Q4_K as 16 (q - 8), Q5_K as 8 (q - 16),
// Q6_K as 4 (q - 32); qi_unit.h), so every product digit*code is exact in
// int32, and over a window
//   sum_k x_k (q_k - z) = 2^-s * (C0 + C1*2^8 + C2*2^16 + C3*2^24),  Ci = sum_k di_k (q_k - z)
// up to the 2^-30-of-window-max rounding of x. The sub-block scale a and the
// offset left, b' = b - z a, of the format (w = a*q - b) are applied in f32
// once per window (Q6_K: per 16-element half window, one int8 sub-scale
// each): y += a * 2^-s * combine(C) - b' * sum_k x_k, with b' = 0 for Q4_0
// and Q6_K; the sums are scaled back by the codes' 1/16, 1/8 or 1/4 once at
// the end. Centring keeps a sum x q and b sum x, of similar size, from
// cancelling in f32.
// This reorders the reference arithmetic and is judged by tolerance.
//
// Operand layout (v_mfma_i32_16x16x64_i8: A[i][k] lane i+16*(k/16), B[k][j]
// lane j+16*(k/16), 16 bytes per lane; C[i][j] lane j+16*(i/4) element i%4).
// For a tile of 16 outputs (B columns) the 4 lane groups g = lane/16 each
// stream their own codes: a step is 8 codes per lane group and one matrix
// instruction takes a pair of steps (16 codes). A row i = 4*sigma + digit
// carries digit `digit` of lane group sigma's 16 activations and is zero
// elsewhere, so C row 4*sigma + digit holds lane group sigma's own digit sums:
// after a window of steps, lane (n, g) holds the four digit sums of its own
// codes in its four C registers, next to its own scale. A 256-element unit is
// 8 steps x 4 groups x 8 codes, 4 instructions. (The 16x16x32 instruction
// takes as many cycles for half the products on gfx950.)
//
// Work split: WC tiles of 16 outputs per workgroup, SW wavefronts per tile
// splitting its K range (contiguous runs of units, reduced through LDS at the
// end). The activation digits of a K chunk are built once per workgroup into
// LDS and shared by its WC tiles (half a window per thread, the window max
// from the neighbouring lane: a single barrier).
// Each wavefront issues its activation loads, then the loads of up to D
// units, before it waits for anything (vector loads complete in order, so
// waiting for the activations never waits for the weights). Two to sixteen
// rows run in the dense-operand kernel of qi_gemv_rows.hip.
// No state is shared between workgroups, so there are no device-scope fences.
#include <type_traits>

#include "qi_device.h"
#include "qi_internal.h"
#include "qi_unit.h"

namespace qi {

typedef int v4i __attribute__((ext_vector_type(4)));

constexpr uint32_t kZeroBytes = 1024;  // zero A operand for the lanes of other lane groups
// Activation record of one (row, unit): 256 activations x 4 digits (1024 B,
// [step pair p][lane group g][digit d] x 16 B: digit d of the pair's 16
// activations, steps 2p and 2p + 1), then 8 windows x float4 {2^-s, window
// sum, 0, 0} (128 B, [g][h]), built in LDS by the workgroup.
constexpr uint32_t kUnitDigitBytes = 1024;
constexpr uint32_t kUnitAuxBytes = 128;
constexpr uint32_t kUnitRecBytes = kUnitDigitBytes + kUnitAuxBytes;
constexpr uint32_t kMaxLds = 160 * 1024;
constexpr uint64_t kCUs = 256;  // compute units of an MI355X (gfx950), for the work split

// Profiling build only (quantinfer_amd/build.py --timeline makes
// libqi_hip_timeline.so with QI_TIMELINE defined): per workgroup of the last
// GEMV launch, the 100 MHz constant clock at kernel entry, once the
// activation records are in LDS, after the first batch of units, after the
// last unit and before the epilogue, plus the hardware and XCD ids; read back
// with qi_timeline_read. In the product build the stamps compile to nothing.
#ifdef QI_TIMELINE
constexpr uint32_t kTimelineSlots = 8192;
__device__ uint64_t g_timeline[kTimelineSlots * 8];
__device__ __forceinline__ void stamp(uint32_t slot, int i) {
  g_timeline[(slot % kTimelineSlots) * 8 + i] = __builtin_amdgcn_s_memrealtime();
}
__device__ __forceinline__ void stamp_where(uint32_t slot) {
  uint32_t hw, xcc;
  asm volatile("s_getreg_b32 %0, hwreg(HW_REG_HW_ID)" : "=s"(hw));
  asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(xcc));
  g_timeline[(slot % kTimelineSlots) * 8 + 5] = hw;
  g_timeline[(slot % kTimelineSlots) * 8 + 6] = xcc;
}
#else
__device__ __forceinline__ void stamp(uint32_t, int) {}
__device__ __forceinline__ void stamp_where(uint32_t) {}
#endif

// Byte transpose of four digit words (one per activation) into four words
// (one per digit): out[i] byte e = in[e] byte i.
__device__ __forceinline__ void transpose4(const uint32_t in[4], uint32_t out[4]) {
  const uint32_t t0 = __builtin_amdgcn_perm(in[1], in[0], 0x05010400u);
  const uint32_t t1 = __builtin_amdgcn_perm(in[1], in[0], 0x07030602u);
  const uint32_t t2 = __builtin_amdgcn_perm(in[3], in[2], 0x05010400u);
  const uint32_t t3 = __builtin_amdgcn_perm(in[3], in[2], 0x07030602u);
  out[0] = __builtin_amdgcn_perm(t2, t0, 0x05040100u);
  out[1] = __builtin_amdgcn_perm(t2, t0, 0x07060302u);
  out[2] = __builtin_amdgcn_perm(t3, t1, 0x05040100u);
  out[3] = __builtin_amdgcn_perm(t3, t1, 0x07060302u);
}

// Half window item hi of a chunk of `units` units: window (row m, unit u,
// lane group g, half h) = hi / 2, elements 16 * (hi % 2) + [0, 16) of it.
// The two halves of a window sit in adjacent lanes.
struct Item {
  uint32_t m, u, g, h, half;
};
__device__ __forceinline__ Item item_of(uint32_t hi, uint32_t units) {
  Item it;
  const uint32_t w = hi >> 1;
  it.half = hi & 1;
  it.m = w / (units * 8);
  const uint32_t r = w % (units * 8);
  it.u = r >> 3;
  it.g = (r >> 1) & 3;
  it.h = r & 1;
  return it;
}

struct HalfX {
  float4 v[4];
};

template <int QT>
__device__ __forceinline__ void load_half(const float* x, uint32_t K, uint32_t k0, const Item& it,
                                          HalfX& o) {
  const float4* p = reinterpret_cast<const float4*>(
      x + static_cast<uint64_t>(it.m) * K + k0 + 256 * it.u + window_first<QT>(it.g, it.h) + 16 * it.half);
#pragma unroll
  for (int i = 0; i < 4; ++i) o.v[i] = p[i];
}

// Digits and sums of one half window into the activation records
// recs[m][u] (cu units per row). Every lane of the wavefront takes part (the
// window max and the other half's sum come from the neighbouring lane); only
// `valid` items store.
__device__ __forceinline__ void store_half(const HalfX& o, const Item& it, bool valid, uint8_t* recs,
                                           uint32_t cu) {
  const float xs[16] = {o.v[0].x, o.v[0].y, o.v[0].z, o.v[0].w, o.v[1].x, o.v[1].y, o.v[1].z, o.v[1].w,
                        o.v[2].x, o.v[2].y, o.v[2].z, o.v[2].w, o.v[3].x, o.v[3].y, o.v[3].z, o.v[3].w};
  float mx = 0.0f;
#pragma unroll
  for (int j = 0; j < 16; ++j) mx = fmaxf(mx, fabsf(xs[j]));
  // the half window's sum, pairwise (the offset term's error scales with it)
  float ps[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) ps[j] = xs[2 * j] + xs[2 * j + 1];
#pragma unroll
  for (int j = 0; j < 4; ++j) ps[j] = ps[2 * j] + ps[2 * j + 1];
  const float sum = (ps[0] + ps[1]) + (ps[2] + ps[3]);
  mx = fmaxf(mx, dpp_move<kDppSwap1>(mx));
  const float other = dpp_move<kDppSwap1>(sum);
  // A NaN or infinite activation makes the window sum non-finite. Its scale
  // is then NaN, so every output of the row comes out NaN and the GEMV's
  // epilogue recomputes it in the reference's order; the digits are built
  // from zeros (no float-to-int conversion of a non-finite value).
  const bool finite = __builtin_isfinite(sum + other);
  // 2^s with max|x| * 2^s < 2^29: F = rint(x * 2^s) keeps 30 bits with headroom
  const int e = finite && mx > 0.0f ? __builtin_amdgcn_frexp_expf(mx) : 0;
  const int sh = 29 - e;
  const float inv = !finite ? __builtin_nanf("") : mx > 0.0f ? ldexpf(1.0f, e - 29) : 0.0f;
  if (!valid) return;
  // this half window is the step pair p = 2h + half (steps 2p and 2p + 1)
  const uint32_t p = 2 * it.h + it.half;
  uint8_t* const rec = recs + (static_cast<uint64_t>(it.m) * cu + it.u) * kUnitRecBytes;
  uint32_t lo[2][4], hi[2][4];
#pragma unroll
  for (int tt = 0; tt < 2; ++tt) {
    uint32_t dig[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int F = finite ? static_cast<int>(rintf(ldexpf(xs[8 * tt + j], sh))) : 0;
      // signed base-256 digits: byte i of (F + 0x808080) ^ 0x808080
      dig[j] = (static_cast<uint32_t>(F) + 0x00808080u) ^ 0x00808080u;
    }
    transpose4(dig, lo[tt]);
    transpose4(dig + 4, hi[tt]);
  }
  // digit d of the pair's 16 activations: 16 contiguous bytes
  uint4* const dst = reinterpret_cast<uint4*>(rec + (p * 4 + it.g) * 64);
#pragma unroll
  for (int d = 0; d < 4; ++d) dst[d] = make_uint4(lo[0][d], hi[0][d], lo[1][d], hi[1][d]);
  if (it.half == 0)
    reinterpret_cast<float4*>(rec + kUnitDigitBytes)[it.g * 2 + it.h] = make_float4(inv, sum + other, 0.0f, 0.0f);
}

// WC tiles of 16 outputs per workgroup, SW wavefronts per tile splitting its
// K range, D units in flight per wavefront, XP half windows of activations
// preloaded per thread (the WC tiles share one activation prep).
// XS: the activation source, see XSource. kXNorm keeps each
// thread's share of sum(v^2) in a register; the wavefront sums reach LDS only
// in the final reduction, so the norm adds no barrier. a.radd adds the
// residual to the outputs, a.silu_pairs combines gate/up output pairs.
template <int QT, bool WIDE, int SW, int D, int WC, int XS = kXPlain>
__global__ __launch_bounds__(64 * SW * WC, (QT == kQ4_K && SW == 4) ? 4 : 1)
void gemv_mfma_kernel(GemvMfmaArgs a) {
  using U = Unit<QT>;
  constexpr int kThreads = 64 * SW * WC;
  constexpr int XP = SW == 8 ? 2 : 1;
  constexpr Record R = record_geometry(QT, WIDE);
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  // [0, kZeroBytes) zeros | activation records [m][chunk unit]
  const uint32_t cu = a.chunk_units;
  uint8_t* const recs = lds + kZeroBytes;

  const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const uint32_t sw = wave % SW, wc = wave / SW;
  const uint32_t slot = blockIdx.y * gridDim.x + blockIdx.x;
  if (tid == 0) {
    stamp(slot, 0);
    stamp_where(slot);
  }
  const uint32_t col = lane & 15, g = lane >> 4;
  // the grid's last workgroup may hold a tile past the end: it streams the
  // last tile again and stores nothing
  const uint32_t tile_raw = blockIdx.x * WC + wc;
  const uint32_t tile = min(tile_raw, a.w.tiles - 1);
  const uint64_t n_out = static_cast<uint64_t>(tile_raw) * 16 + col;
  const uint32_t units_total = a.w.units;
  const uint8_t* trec = a.w.qs + static_cast<uint64_t>(tile) * units_total * R.bytes;
  const uint32_t K = static_cast<uint32_t>(a.w.k);

  // A-operand lane role: row (sigma, digit) is live for lane group g == sigma
  const uint32_t arow = lane & 15, sigma = arow >> 2, digit = arow & 3;
  const bool a_live = sigma == g;

  for (uint32_t i = tid; i < kZeroBytes / 4; i += kThreads) reinterpret_cast<uint32_t*>(lds)[i] = 0;

  float acc = 0.0f;
  [[maybe_unused]] float ssq = 0.0f;  // kXNorm: this thread's part of sum(v^2)

  typename U::Raw ring[D];

  for (uint32_t ku0 = 0; ku0 < units_total; ku0 += cu) {
    const uint32_t units = min(cu, units_total - ku0);
    const uint32_t k0 = ku0 * 256;
    const uint32_t halves = units * 16;
    // this wavefront's contiguous run of the chunk's units (balanced split)
    const uint32_t u_begin = (units * sw) / SW;
    const uint32_t u_count = (units * (sw + 1)) / SW - u_begin;
    const uint32_t u_last = ku0 + (u_count ? u_begin + u_count - 1 : 0);

    // activations first (so that waiting for them never waits for the
    // weights), then this wavefront's first D units, unconditionally (slots
    // past the run re-read its last unit)
    HalfX xp[XP];
    Item ip[XP];
    [[maybe_unused]] HalfX up[XP];  // kXNorm: the norm weights
#pragma unroll
    for (int i = 0; i < XP; ++i) {
      const uint32_t hi = tid + kThreads * i;
      ip[i] = item_of(hi < halves ? hi : 0, units);
      if constexpr (XS == kXNorm) {
        load_half<QT>(a.hres, K, k0, ip[i], xp[i]);
        load_half<QT>(a.nw, K, k0, ip[i], up[i]);
      } else {
        load_half<QT>(a.x, K, k0, ip[i], xp[i]);
      }
    }
    // fused sources: keep every activation load ahead of the weight loads
    // (the scheduler hoisted weight scale loads above them, so the in-order
    // wait for the activations waited for HBM); the plain source already
    // keeps that order, and the barrier measured slower there
    if constexpr (XS != kXPlain) __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < D; ++i)
      U::template load<WIDE, true>(trec + min(ku0 + u_begin + i, u_last) * R.bytes, lane, ring[i]);

    // kXNorm: sum(v^2) over valid items, x = v * w
    [[maybe_unused]] auto norm = [&](HalfX& vx, const HalfX& wx, bool valid) {
      float s2 = 0.0f;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const float4 v = vx.v[q];
        s2 += v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
        vx.v[q] = make_float4(v.x * wx.v[q].x, v.y * wx.v[q].y, v.z * wx.v[q].z, v.w * wx.v[q].w);
      }
      if (valid) ssq += s2;
    };
#pragma unroll
    for (int i = 0; i < XP; ++i) {
      const bool valid = tid + kThreads * i < halves;
      if constexpr (XS == kXNorm) norm(xp[i], up[i], valid);
      store_half(xp[i], ip[i], valid, recs, cu);
    }
    for (uint32_t h0 = XP * kThreads; h0 < halves; h0 += kThreads) {
      const uint32_t hi = h0 + tid;
      Item it = item_of(hi < halves ? hi : 0, units);
      HalfX xh;
      if constexpr (XS == kXNorm) {
        HalfX wh;
        load_half<QT>(a.hres, K, k0, it, xh);
        load_half<QT>(a.nw, K, k0, it, wh);
        norm(xh, wh, hi < halves);
      } else {
        load_half<QT>(a.x, K, k0, it, xh);
      }
      store_half(xh, it, hi < halves, recs, cu);
    }
    __syncthreads();
    if (tid == 0) stamp(slot, 1);

    // ---- main: this wavefront's units, D in flight ----
    // The first batch is straight-line code on the registers loaded above (a
    // loop over it would copy the ring into loop-carried registers, waiting
    // for every load); later batches reload the ring and consume it.
    auto consume = [&](uint32_t j) {
#pragma unroll
      for (int i = 0; i < D; ++i) {
        if (j + i >= u_count) break;
        const uint32_t u = u_begin + j + i;  // chunk-relative unit
        float sa[U::kWindows], sb[U::kWindows];
        U::template scales<WIDE>(g, ring[i], sa, sb);
        // Q4_K / Q5_K: the offsets left by the centred codes, b - z a
        // (exactly rounded), in the codes' scale (times a power of two)
        if constexpr (window_centered<QT>()) {
#pragma unroll
          for (int w = 0; w < U::kWindows; ++w)
            sb[w] = fmaf(-static_cast<float>(code_centre<QT>()), sa[w], sb[w]) * static_cast<float>(code_scale<QT>());
        }
        const uint8_t* const rec = recs + u * kUnitRecBytes;
        const uint8_t* const abase = a_live ? rec + g * 64 + digit * 16 : lds;
        const float4* const ax = reinterpret_cast<const float4*>(rec + kUnitDigitBytes) + g * 2;
#pragma unroll
        for (int w = 0; w < U::kWindows; ++w) {
          v4i c = {0, 0, 0, 0};
#pragma unroll
          for (int s = 0; s < U::kSteps; s += 2) {
            // one 16x16x64 instruction per step pair: 16 activations (digit
            // bytes) and 16 codes per lane
            const int t = w * U::kSteps + s;
            const v4i av = *reinterpret_cast<const v4i*>(abase + (t >> 1) * 256);
            const long c0 = gemv_codes<QT>(ring[i], g, t), c1 = gemv_codes<QT>(ring[i], g, t + 1);
            const v4i cb = {static_cast<int>(c0), static_cast<int>(c0 >> 32), static_cast<int>(c1),
                            static_cast<int>(c1 >> 32)};
            c = __builtin_amdgcn_mfma_i32_16x16x64_i8(av, cb, c, 0, 0, 0);
          }
          const int h = U::kSteps == 4 ? w : (w >> 1);
          // combine the digit sums: pairs exactly in int32 (|C0| < 2^20,
          // |C1 * 256| < 2^28), the two halves in f32
          const float comb = fmaf(static_cast<float>(c[2] + c[3] * 256), 65536.0f,
                                  static_cast<float>(c[0] + c[1] * 256));
          const float4 wx = ax[h];
          acc = fmaf(sa[w] * wx.x, comb, acc);
          if constexpr (window_centered<QT>()) acc = fmaf(-sb[w], wx.y, acc);
        }
      }
    };
    consume(0);
    if (tid == 0) stamp(slot, 2);
    for (uint32_t j = D; j < u_count; j += D) {
#pragma unroll
      for (int i = 0; i < D; ++i)
        U::template load<WIDE, true>(trec + min(ku0 + u_begin + j + i, u_last) * R.bytes, lane, ring[i]);
      consume(j);
    }
    __syncthreads();  // LDS reused by the next chunk / the reduction
  }

  if (tid == 0) stamp(slot, 3);
  // ---- reduce: 4 lane groups of a column, then the SW K-parts ----
  acc *= 1.0f / code_scale<QT>();  // centred codes' scale (exact)
  acc += __shfl_xor(acc, 16);
  acc += __shfl_xor(acc, 32);
  float* red = reinterpret_cast<float*>(recs);  // [WC][SW][16], then kXNorm: [waves]
  if (g == 0) red[(wc * SW + sw) * 16 + col] = acc;
  if constexpr (XS == kXNorm) {
    float s2 = ssq;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) s2 += __shfl_xor(s2, o);
    if (lane == 0) red[WC * SW * 16 + wave] = s2;
  }
  __syncthreads();
  [[maybe_unused]] float inv = 1.0f;
  if constexpr (XS == kXNorm) {
    float total = 0.0f;
    for (int w = 0; w < SW * WC; ++w) total += red[WC * SW * 16 + w];
    inv = 1.0f / sqrtf(total / static_cast<float>(K) + a.eps);
  }
  if (a.silu_pairs) {
    // lanes 0-7 of the tile hold gate rows, lanes 8-15 the matching up rows
    if (sw == 0 && g == 0) {
      float v = red[(wc * SW) * 16 + col];
#pragma unroll
      for (int p = 1; p < SW; ++p) v += red[(wc * SW + p) * 16 + col];
      if constexpr (XS == kXNorm) v *= inv;
      const float u = __shfl(v, static_cast<int>(lane) + 8, 16);
      if (col < 8 && tile_raw < a.w.tiles) a.y[static_cast<uint64_t>(tile_raw) * 8 + col] = v / (1.0f + expf(-v)) * u;
    }
    return;
  }
  if (tid == 0) stamp(slot, 4);
  if (sw == 0 && g == 0 && n_out < a.w.n) {
    float v = red[(wc * SW) * 16 + col];
#pragma unroll
    for (int p = 1; p < SW; ++p) v += red[(wc * SW + p) * 16 + col];
    if constexpr (XS == kXNorm) v *= inv;
    const float rv = a.radd != nullptr ? a.radd[n_out] : 0.0f;
    if (a.radd != nullptr) v = rv + v;
    // NaN or infinite activations (or an overflow): the reference's own order
    // decides which outputs are NaN and which +-Inf
    if constexpr (XS == kXPlain) {
      if (!__builtin_isfinite(v)) {
        v = exact_output_row<QT, WIDE>(a.w, a.x, n_out);
        if (a.radd != nullptr) v = rv + v;
      }
    }
    a.y[n_out] = v;
  }
}


namespace {

uint32_t lds_bytes(uint32_t chunk_units, int waves) {
  const uint32_t main = kZeroBytes + chunk_units * kUnitRecBytes;
  const uint32_t red = kZeroBytes + static_cast<uint32_t>(waves * 16 * 4 + waves * 4);
  return main > red ? main : red;
}

template <int QT, bool WIDE, int SW, int D, int WC, int XS = kXPlain>
hipError_t launch4(GemvMfmaArgs a, hipStream_t st) {
  const uint32_t cap = (kMaxLds - kZeroBytes) / kUnitRecBytes;
  a.chunk_units = a.w.units < cap ? a.w.units : cap;
  const uint32_t bytes = lds_bytes(a.chunk_units, SW * WC);
  auto kern = gemv_mfma_kernel<QT, WIDE, SW, D, WC, XS>;
  if (bytes > 65536) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(bytes));
    if (e != hipSuccess) {
      (void)hipGetLastError();  // the next launch's check must not see this call's error
      return e;
    }
  }
  hipLaunchKernelGGL(kern, dim3((a.w.tiles + WC - 1) / WC), dim3(64 * SW * WC), bytes, st, a);
  return hipGetLastError();
}

// (wavefronts per workgroup, units in flight per wavefront) for `sw` and the
// units each wavefront holds
template <int QT, bool WIDE, int XS = kXPlain>
hipError_t launch_split(const GemvMfmaArgs& a, int sw, hipStream_t st) {
  const uint32_t cap = (kMaxLds - kZeroBytes) / kUnitRecBytes;
  const uint32_t chunk = a.w.units < cap ? a.w.units : cap;
  if (sw == 4) {
    // Two tiles share the activation prep (an 8-wavefront workgroup) where
    // that does not raise the most tiles any CU streams, with workgroups
    // spread evenly over the CUs: ceil(tiles / 256) one-tile workgroups
    // against 2 ceil(tiles / 512) two-tile ones (896 tiles: 4 and 4, so
    // the shared prep wins; 768: 3 against 4); above 1024 tiles the
    // workgroups no longer all fit at once. With two workgroups on a CU
    // the second one's activation loads queue behind the first one's
    // weight loads, so the 4-bit K-quants then keep two units in flight per
    // wavefront, not four (measured on MI355X at 896 tiles: Q4_K 7.9
    // against 8.2 us, Q5_K 10.0 against 10.6, Q6_K 10.7 against 11.4; the
    // 8-bit and Q4_0 codes do not gain).
    const uint64_t t = a.w.tiles;
    const uint64_t one = (t + kCUs - 1) / kCUs, two = 2 * ((t + 2 * kCUs - 1) / (2 * kCUs));
    if (two <= one && t <= 4 * kCUs) {
      if constexpr (QT == kQ4_K || QT == kQ5_K || QT == kQ6_K) {
        if (t > 2 * kCUs) return launch4<QT, WIDE, 4, 2, 2, XS>(a, st);
      }
      return launch4<QT, WIDE, 4, 4, 2, XS>(a, st);
    }
    if constexpr (QT == kQ4_K) {
      // 1281-1536 tiles (the decoder's fused gate|up, N = 24576): four
      // one-tile workgroups fit a CU at once, so the one-tile launch runs
      // in two rounds and the second pays the activation round trip again.
      // Six tiles per workgroup with two wavefronts each (8 units per
      // wavefront, two in flight; 12 wavefronts, one workgroup per CU) run
      // in one. Measured on MI355X: decode step of the Qwen3-8B-shape
      // decoder 1.671 -> 1.626 ms; plain 4096 x 24576 11.6-11.9 -> 11.4 us.
      if (t > 5 * kCUs && t <= 6 * kCUs) return launch4<QT, WIDE, 2, 2, 6, XS>(a, st);
    }
    return launch4<QT, WIDE, 4, 4, 1, XS>(a, st);
  }
  const uint32_t upw = (chunk + 7) / 8;
  if (upw <= 2) return launch4<QT, WIDE, 8, 2, 1, XS>(a, st);
  // up to two tiles per CU: 16 wavefronts per tile with two units in
  // flight each, reloaded per batch (K = 12288 on MI355X: N = 4096 8.5 us
  // against 8.9 for 8 wavefronts x 2 units and 9.2-9.5 for 8 x 8; N = 6144
  // 14.1 against 15.7); more tiles: 8 wavefronts with the whole run in
  // flight (N = 14336: 21.9 against 24.1 us for 8 x 2)
  if (a.w.tiles <= 2 * kCUs) return launch4<QT, WIDE, 16, 2, 1, XS>(a, st);
  // (Q5_K, and Q6_K with the norm prep, spill registers at 8 units deep)
  constexpr bool deep = QT != kQ5_K && (XS != kXNorm || QT != kQ6_K);
  if constexpr (deep) {
    if (upw > 4) return launch4<QT, WIDE, 8, 8, 1, XS>(a, st);
  }
  return launch4<QT, WIDE, 8, 4, 1, XS>(a, st);
}

template <int QT, bool WIDE>
hipError_t launch_m(const GemvMfmaArgs& a, int sw, hipStream_t st) {
  if (a.m != 1) return hipErrorInvalidValue;
  if (a.silu_pairs && (a.radd != nullptr || a.w.n % 16 != 0)) return hipErrorInvalidValue;
  if (a.xs != kXPlain) {
    // the decoder's fused projections: f16-scale images
    if constexpr (WIDE) {
      return hipErrorInvalidValue;
    } else {
      if (a.xs == kXNorm && a.hres != nullptr && a.nw != nullptr) return launch_split<QT, WIDE, kXNorm>(a, sw, st);
      return hipErrorInvalidValue;
    }
  }
  return launch_split<QT, WIDE>(a, sw, st);
}

template <int QT>
hipError_t launch_w(const GemvMfmaArgs& a, bool wide, int sw, hipStream_t st) {
  return wide ? launch_m<QT, true>(a, sw, st) : launch_m<QT, false>(a, sw, st);
}

}  // namespace

bool gemv_mfma_supported(int32_t qtype, int32_t layout, uint64_t k) {
  return layout == kOutputRows && qtype >= kQ8_0 && qtype <= kQ6_K && k % 256 == 0 && k > 0;
}

int gemv_mfma_split(uint64_t k, uint64_t n) {
  // Wavefronts per tile (K parts of one 16-output tile): 4 up to 16 units
  // (K <= 4096: at most 4 units per wavefront, all in flight), 8 above.
  // Measured on MI355X at K = 4096 the 4-way split beats the 8-way one at
  // every N tried (256 to 1536 tiles).
  (void)n;
  return k <= 4096 ? 4 : 8;
}

hipError_t launch_gemv_mfma(int32_t qtype, bool wide, int sw, const GemvMfmaArgs& a, hipStream_t st) {
  if (sw != 4 && sw != 8) return hipErrorInvalidValue;
  switch (qtype) {
    case kQ8_0: return launch_w<kQ8_0>(a, wide, sw, st);
    case kQ4_0: return launch_w<kQ4_0>(a, wide, sw, st);
    case kQ4_K: return launch_w<kQ4_K>(a, wide, sw, st);
    case kQ5_K: return launch_w<kQ5_K>(a, wide, sw, st);
    case kQ6_K: return launch_w<kQ6_K>(a, wide, sw, st);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace qi

#ifdef QI_TIMELINE
// Copy the first n words of the timeline ([slot][8]) to host memory, or zero it.
extern "C" int qi_timeline_read(uint64_t* host, uint64_t n) {
  if (n > qi::kTimelineSlots * 8) return static_cast<int>(hipErrorInvalidValue);
  return static_cast<int>(hipMemcpyFromSymbol(host, HIP_SYMBOL(qi::g_timeline), n * 8, 0, hipMemcpyDeviceToHost));
}
extern "C" int qi_timeline_clear(void) {
  static uint64_t zeros[qi::kTimelineSlots * 8];
  return static_cast<int>(hipMemcpyToSymbol(HIP_SYMBOL(qi::g_timeline), zeros, sizeof(zeros), 0, hipMemcpyHostToDevice));
}
#endif
