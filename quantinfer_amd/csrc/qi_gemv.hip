// Decode GEMV for the output-rows layout when K is a multiple of 32 but not
// of 256 (Q8_0/Q4_0; the matrix-core GEMV needs 256-element units), M <= 16
// activation rows, f32 arithmetic (the "F32" mode; judged by tolerance
// against the CPU reference).
//
// Mapping (one wavefront per workgroup):
//   blockIdx.x -> RW consecutive output rows (register-blocked),
//   lane       -> blocks s = lane, lane+64, ... of the row.
// Each lane streams its blocks' code bytes with 16-byte loads (coalesced: the
// 64 lanes of a load read consecutive blocks of one row), decodes them in
// registers and accumulates sum_i x_i q_i per 16-element piece; the piece's
// affine scale is applied once per piece. The activations come through L1/L2
// (they are shared by every row) and are reused from registers across the RW
// rows. Lane partials are reduced with DPP. An output whose sum is not
// finite (a NaN or infinite activation) is recomputed in the reference's
// order (exact_output_row), which fixes which outputs are NaN and which +-Inf.
#include "qi_device.h"
#include "qi_internal.h"

namespace qi {

template <int QT, bool WIDE, int MT, int RW>
__global__ __launch_bounds__(64) void gemv_kernel(GemvArgs a) {
  using F = Fast<QT, WIDE>;
  const uint32_t lane = threadIdx.x;
  const uint64_t row0 = static_cast<uint64_t>(blockIdx.x) * RW;
  const uint32_t slots = static_cast<uint32_t>(a.w.k / F::kSlotElems);

  uint64_t rows[RW];
#pragma unroll
  for (int i = 0; i < RW; ++i) rows[i] = min(row0 + i, a.w.n - 1);

  float acc[RW][MT];
#pragma unroll
  for (int i = 0; i < RW; ++i)
#pragma unroll
    for (int m = 0; m < MT; ++m) acc[i][m] = 0.0f;

  for (uint32_t s = lane; s < slots; s += 64) {
    typename F::Slot sl[RW];
#pragma unroll
    for (int i = 0; i < RW; ++i) F::load(a.w, rows[i], s, sl[i]);
#pragma unroll
    for (int p = 0; p < F::kPieces; ++p) {
      const uint32_t xo = F::x_offset(s, p);
      float q[RW][16];
#pragma unroll
      for (int i = 0; i < RW; ++i) F::codes(sl[i], p, q[i]);
#pragma unroll
      for (int m = 0; m < MT; ++m) {
        const int mr = m < a.m ? m : a.m - 1;
        const float4* xp = reinterpret_cast<const float4*>(a.x + static_cast<uint64_t>(mr) * a.w.k + xo);
        const float4 x0 = xp[0], x1 = xp[1], x2 = xp[2], x3 = xp[3];
        const float xs[16] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w,
                              x2.x, x2.y, x2.z, x2.w, x3.x, x3.y, x3.z, x3.w};
        float xsum = 0.0f;
        if constexpr (F::kHasMin) {
#pragma unroll
          for (int j = 0; j < 16; ++j) xsum += xs[j];
        }
#pragma unroll
        for (int i = 0; i < RW; ++i) {
          float dot = 0.0f;
#pragma unroll
          for (int j = 0; j < 16; ++j) dot = fmaf(xs[j], q[i][j], dot);
          acc[i][m] = fmaf(F::a(sl[i], p), dot, acc[i][m]);
          if constexpr (F::kHasMin) acc[i][m] = fmaf(-F::b(sl[i], p), xsum, acc[i][m]);
        }
      }
    }
  }

  float tot[RW][MT];
#pragma unroll
  for (int i = 0; i < RW; ++i)
#pragma unroll
    for (int m = 0; m < MT; ++m) tot[i][m] = wave_sum(acc[i][m]);

  if (lane == 0) {
    bool bad = false;
#pragma unroll
    for (int i = 0; i < RW; ++i) {
      if (row0 + i >= a.w.n) break;
#pragma unroll
      for (int m = 0; m < MT; ++m) {
        if (m < a.m) {
          a.y[static_cast<uint64_t>(m) * a.w.n + row0 + i] = tot[i][m];
          bad |= !__builtin_isfinite(tot[i][m]);
        }
      }
    }
    if (bad) {
#pragma unroll 1
      for (int o = 0; o < RW * a.m; ++o) {
        const uint64_t n = row0 + o / a.m, m = o % a.m;
        if (n >= a.w.n) break;
        float* y = a.y + m * a.w.n + n;
        if (!__builtin_isfinite(*y)) *y = exact_output_row<QT, WIDE>(a.w, a.x + m * a.w.k, n);
      }
    }
  }
}

namespace {

template <int QT, bool WIDE, int MT, int RW>
hipError_t launch_one(const GemvArgs& a, hipStream_t st) {
  const uint32_t row_tiles = static_cast<uint32_t>((a.w.n + RW - 1) / RW);
  hipLaunchKernelGGL((gemv_kernel<QT, WIDE, MT, RW>), dim3(row_tiles), dim3(64), 0, st, a);
  return hipGetLastError();
}

template <int QT, bool WIDE>
hipError_t launch_mt(GemvArgs a, int mt, hipStream_t st) {
  switch (mt) {
    case 1: return launch_one<QT, WIDE, 1, 4>(a, st);
    case 2: return launch_one<QT, WIDE, 2, 4>(a, st);
    case 4: return launch_one<QT, WIDE, 4, 2>(a, st);
    case 8: return launch_one<QT, WIDE, 8, 2>(a, st);
    case 16: return launch_one<QT, WIDE, 16, 1>(a, st);
    default: return hipErrorInvalidValue;
  }
}

template <int QT>
hipError_t launch_wide(GemvArgs a, int mt, bool wide, hipStream_t st) {
  return wide ? launch_mt<QT, true>(a, mt, st) : launch_mt<QT, false>(a, mt, st);
}

}  // namespace

bool gemv_supported(int32_t qtype, int32_t layout, uint64_t k) {
  return layout == kOutputRows && (qtype == kQ8_0 || qtype == kQ4_0) && k % 32 == 0 && k > 0;
}

hipError_t launch_gemv(int32_t qtype, bool wide, int mt, const GemvArgs& a, hipStream_t st) {
  if (a.m < 1 || a.m > mt) return hipErrorInvalidValue;
  switch (qtype) {
    case kQ8_0: return launch_wide<kQ8_0>(a, mt, wide, st);
    case kQ4_0: return launch_wide<kQ4_0>(a, mt, wide, st);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace qi
