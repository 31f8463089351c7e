// Decode GEMV for the output-rows layout, M <= 16 activation rows, f32
// arithmetic (the "F32" mode; judged by tolerance against the CPU reference).
//
// Mapping (one wavefront per workgroup):
//   blockIdx.x -> RW consecutive output rows (register-blocked),
//   blockIdx.y -> one split of the K range (split-K for short grids),
//   lane       -> slots s = lane, lane+64, ... of the split; a slot is one
//                 Q8_0/Q4_0 block or 64 elements of a K-quant super-block.
// Each lane streams its slots' code bytes with 16-byte loads (coalesced: the
// 64 lanes of a load read consecutive slots of one row), decodes them in
// registers and accumulates sum_i x_i q_i per 16-element piece; the piece's
// affine scale is applied once per piece. The activations come through L1/L2
// (they are shared by every row) and are reused from registers across the RW
// rows. Lane partials are reduced with DPP; with split-K, the partial row
// sums go to a workspace and the last workgroup of a row tile (atomic ticket)
// adds them in split order, so results do not depend on scheduling.
#include "qi_device.h"
#include "qi_internal.h"

namespace qi {

template <int QT, bool WIDE, int MT, int RW>
__global__ __launch_bounds__(64) void gemv_kernel(GemvArgs a) {
  using F = Fast<QT, WIDE>;
  const uint32_t lane = threadIdx.x;
  const uint64_t row0 = static_cast<uint64_t>(blockIdx.x) * RW;
  const uint32_t split = blockIdx.y;
  const uint32_t slots = static_cast<uint32_t>(a.w.k / F::kSlotElems);
  const uint32_t s_begin = split * a.slots_per_split;
  const uint32_t s_end = min(slots, s_begin + a.slots_per_split);

  uint64_t rows[RW];
#pragma unroll
  for (int i = 0; i < RW; ++i) rows[i] = min(row0 + i, a.w.n - 1);

  float acc[RW][MT];
#pragma unroll
  for (int i = 0; i < RW; ++i)
#pragma unroll
    for (int m = 0; m < MT; ++m) acc[i][m] = 0.0f;

  for (uint32_t s = s_begin + lane; s < s_end; s += 64) {
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

  if (gridDim.y == 1) {
    if (lane == 0) {
#pragma unroll
      for (int i = 0; i < RW; ++i) {
        if (row0 + i >= a.w.n) break;
#pragma unroll
        for (int m = 0; m < MT; ++m)
          if (m < a.m) a.y[static_cast<uint64_t>(m) * a.w.n + row0 + i] = tot[i][m];
      }
    }
    return;
  }

  // split-K: publish partials, then the last arriving split reduces in order
  float* ws = a.partials;
  if (lane == 0) {
#pragma unroll
    for (int i = 0; i < RW; ++i) {
      if (row0 + i >= a.w.n) break;
#pragma unroll
      for (int m = 0; m < MT; ++m)
        if (m < a.m)
          ws[(static_cast<uint64_t>(split) * a.m + m) * a.w.n + row0 + i] = tot[i][m];
    }
  }
  __threadfence();
  uint32_t ticket = 0;
  if (lane == 0) ticket = atomicAdd(&a.tickets[blockIdx.x], 1u);
  ticket = __builtin_amdgcn_readfirstlane(ticket);
  if (ticket != gridDim.y - 1) return;
  __threadfence();
  // lanes < RW*MT each own one (row, m) output
  const uint32_t i = lane / MT, m = lane % MT;
  if (lane < RW * MT && row0 + i < a.w.n && m < static_cast<uint32_t>(a.m)) {
    float sum = 0.0f;
    for (uint32_t sp = 0; sp < gridDim.y; ++sp)
      sum += __builtin_nontemporal_load(&ws[(static_cast<uint64_t>(sp) * a.m + m) * a.w.n + row0 + i]);
    a.y[static_cast<uint64_t>(m) * a.w.n + row0 + i] = sum;
  }
  if (lane == 0) a.tickets[blockIdx.x] = 0;  // ready for the next launch
}

namespace {

template <int QT, bool WIDE, int MT, int RW>
hipError_t launch_one(const GemvArgs& a, uint32_t row_tiles, uint32_t splits, hipStream_t st) {
  hipLaunchKernelGGL((gemv_kernel<QT, WIDE, MT, RW>), dim3(row_tiles, splits), dim3(64), 0, st, a);
  return hipGetLastError();
}

template <int QT, bool WIDE>
hipError_t launch_mt(GemvArgs a, int mt, const GemvPlan& plan, hipStream_t st) {
  switch (mt) {
    case 1: return launch_one<QT, WIDE, 1, 4>(a, plan.row_tiles, plan.splits, st);
    case 2: return launch_one<QT, WIDE, 2, 4>(a, plan.row_tiles, plan.splits, st);
    case 4: return launch_one<QT, WIDE, 4, 2>(a, plan.row_tiles, plan.splits, st);
    case 8: return launch_one<QT, WIDE, 8, 2>(a, plan.row_tiles, plan.splits, st);
    case 16: return launch_one<QT, WIDE, 16, 1>(a, plan.row_tiles, plan.splits, st);
    default: return hipErrorInvalidValue;
  }
}

template <int QT>
hipError_t launch_wide(GemvArgs a, int mt, bool wide, const GemvPlan& plan, hipStream_t st) {
  return wide ? launch_mt<QT, true>(a, mt, plan, st) : launch_mt<QT, false>(a, mt, plan, st);
}

}  // namespace

int gemv_tile_rows(int mt) { return mt <= 2 ? 4 : (mt <= 8 ? 2 : 1); }

int gemv_slot_elems(int32_t qtype) { return (qtype == kQ8_0 || qtype == kQ4_0) ? 32 : 64; }

GemvPlan plan_gemv(int32_t qtype, uint64_t k, uint64_t n, int mt, uint64_t max_partials) {
  GemvPlan p;
  const uint64_t rw = static_cast<uint64_t>(gemv_tile_rows(mt));
  p.row_tiles = static_cast<uint32_t>((n + rw - 1) / rw);
  const uint32_t slots = static_cast<uint32_t>(k / static_cast<uint64_t>(gemv_slot_elems(qtype)));
  // This kernel only serves shapes the matrix-core GEMV does not (K not a
  // multiple of 256): short rows, no split of K across workgroups (a
  // cross-workgroup reduction needs device-scope fences, which write back the
  // per-XCD L2 on MI355X).
  uint32_t splits = 1;
  (void)max_partials;
  (void)mt;
  p.slots_per_split = (slots + splits - 1) / splits;
  p.splits = (slots + p.slots_per_split - 1) / p.slots_per_split;
  return p;
}

hipError_t launch_gemv(int32_t qtype, bool wide, int mt, const GemvArgs& a, const GemvPlan& plan,
                       hipStream_t st) {
  switch (qtype) {
    case kQ8_0: return launch_wide<kQ8_0>(a, mt, wide, plan, st);
    case kQ4_0: return launch_wide<kQ4_0>(a, mt, wide, plan, st);
    case kQ4_K: return launch_wide<kQ4_K>(a, mt, wide, plan, st);
    case kQ5_K: return launch_wide<kQ5_K>(a, mt, wide, plan, st);
    case kQ6_K: return launch_wide<kQ6_K>(a, mt, wide, plan, st);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace qi
