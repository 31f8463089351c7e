// Row-major (blocks along N) GEMV and GEMM, F32 mode: y[m, n] = sum_k x[m, k]
// w(k, n) for QuantInfer-layout weights (backends/cpu/src/backend.rs:62-140 ->
// matmul.rs:14-90; element values matmul.rs:162-280). From 3 rows on a tiled
// image with K a multiple of 4 the call is rm_gemm_kernel (its comment below):
// the records dequantized into LDS for the f32 matrix cores. The GEMV takes 1
// and 2 rows, two kernels by image:
//
// Tiled image (N a multiple of 256; gemv_rmt_kernel): record (t, u) holds
// rows k = 16t + c (c = 0..15) of outputs n = 256u + [0, 256), in the
// arrangement of the output-rows records. Lane 16g + c of a wavefront loads row
// c's lane group g with the GEMV's record loader (Unit<QT>, non-temporal): the
// codes of 64 outputs at one k and the scales of their windows. The lane keeps
// one f32 accumulator per output and activation row and adds x[k] w per code
// (rmt_consume: the codes centred as the one-row output-rows GEMV takes them,
// the weight formed in one multiply-add where an offset is left).
// A workgroup of four wavefronts takes one unit and one K split, each
// wavefront every fourth tile of the split: at most rmt_max_slots records,
// all loaded before the first is consumed.
// The 16 rows of a lane group are summed by two DPP steps (lanes c, c + 4,
// c + 8, c + 12) and through LDS for the last four and the four wavefronts, in
// a fixed order.
//
// Planar image (gemv_rm_kernel): flat block index k * (N / bs) + nb, so at
// one k the code bytes of consecutive output blocks are contiguous. A lane
// owns one column unit: the outputs one 4-byte code word decodes to
// (Q8_0: 4 outputs; Q4_0 and Q4_K/Q5_K: 8, low and high nibbles; Q6_K: 16 from
// two ql words and one qh word). 64 consecutive column units per workgroup
// column, the four wavefronts split the workgroup's K range, and the grid's
// y dimension splits K further; every k a lane loads its code word(s) and its
// block's scales (the activations are wavefront-uniform loads), forms the
// weights in f32 and accumulates x * w for up to MT activation rows.
// Partials of the K parts are summed in a fixed order: the four wavefronts
// through LDS, the K splits by rm_sum_kernel. Results are deterministic; the
// summation order differs from the reference's sequential k, so the mode is
// judged by tolerance like the output-rows F32 GEMV.
#include "qi_device.h"
#include "qi_internal.h"
#include "qi_unit.h"

namespace qi {

namespace {

template <int QT>
struct RmGeo {
  static constexpr uint32_t kBs = (QT == kQ8_0 || QT == kQ4_0) ? 32 : 256;   // outputs per block
  static constexpr int kOut = QT == kQ8_0 ? 4 : QT == kQ6_K ? 16 : 8;        // outputs per lane
  static constexpr uint32_t kCus = kBs / kOut;                              // column units per block
};

__device__ __forceinline__ uint32_t load_u32(const uint8_t* p) { return *reinterpret_cast<const uint32_t*>(p); }

// Weights of column unit c of flat block blk: w[j] for the lane's outputs
// (their positions within the block: rm_offset).
template <int QT, bool WIDE>
__device__ __forceinline__ void rm_weights(const View& v, uint64_t blk, uint32_t c, float w[RmGeo<QT>::kOut]) {
  const float d = load_scale<WIDE>(v.d, blk);
  if constexpr (QT == kQ8_0) {
    const uint32_t q = load_u32(v.qs + blk * 32 + 4 * c);
#pragma unroll
    for (int j = 0; j < 4; ++j) w[j] = d * static_cast<float>(static_cast<int8_t>(q >> (8 * j)));
  } else if constexpr (QT == kQ4_0) {
    const uint32_t q = load_u32(v.qs + blk * 16 + 4 * c);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      w[j] = d * (static_cast<float>((q >> (8 * j)) & 15u) - 8.0f);
      w[4 + j] = d * (static_cast<float>((q >> (8 * j + 4)) & 15u) - 8.0f);
    }
  } else if constexpr (QT == kQ4_K || QT == kQ5_K) {
    const uint32_t g = c / 8, i = c % 8;
    const uint32_t q = load_u32(v.qs + blk * 128 + 32 * g + 4 * i);
    const uint8_t* s = v.sc + blk * 12;
    uint32_t sc0, m0, sc1, m1;
    const uint32_t w0 = load_u32(s), w1 = load_u32(s + 4), w2 = load_u32(s + 8);
    kquant_sc_m(w0, w1, w2, static_cast<int>(2 * g), sc0, m0);
    kquant_sc_m(w0, w1, w2, static_cast<int>(2 * g + 1), sc1, m1);
    const float dmin = load_scale<WIDE>(v.dmin, blk);
    const float a0 = d * static_cast<float>(sc0), b0 = dmin * static_cast<float>(m0);
    const float a1 = d * static_cast<float>(sc1), b1 = dmin * static_cast<float>(m1);
    [[maybe_unused]] uint32_t h = 0;
    if constexpr (QT == kQ5_K) h = load_u32(v.qh + blk * 32 + 4 * i);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      uint32_t lo = (q >> (8 * j)) & 15u, hi = (q >> (8 * j + 4)) & 15u;
      if constexpr (QT == kQ5_K) {
        lo += ((h >> (8 * j + 2 * g)) & 1u) << 4;
        hi += ((h >> (8 * j + 2 * g + 1)) & 1u) << 4;
      }
      w[j] = a0 * static_cast<float>(lo) - b0;
      w[4 + j] = a1 * static_cast<float>(hi) - b1;
    }
  } else {  // kQ6_K
    const uint32_t ip = c / 8, i = c % 8;
    const uint32_t A = load_u32(v.qs + blk * 128 + 64 * ip + 4 * i);
    const uint32_t B = load_u32(v.qs + blk * 128 + 64 * ip + 32 + 4 * i);
    const uint32_t H = load_u32(v.qh + blk * 64 + 32 * ip + 4 * i);
    const int8_t* s = reinterpret_cast<const int8_t*>(v.sc + blk * 16) + 8 * ip + i / 4;
#pragma unroll
    for (int ch = 0; ch < 4; ++ch) {
      const uint32_t src = (ch & 1) ? B : A;
      const int sh = ch < 2 ? 0 : 4;
      const float a = d * static_cast<float>(s[2 * ch]);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint32_t low = (src >> (8 * j + sh)) & 15u;
        const uint32_t high = (H >> (8 * j + 2 * ch)) & 3u;
        w[4 * ch + j] = a * static_cast<float>(static_cast<int>(low | (high << 4)) - 32);
      }
    }
  }
}

// output offset within the block of the lane's output j
template <int QT>
__device__ __forceinline__ uint32_t rm_offset(uint32_t c, int j) {
  if constexpr (QT == kQ8_0) return 4 * c + j;
  else if constexpr (QT == kQ4_0) return j < 4 ? 4 * c + j : 16 + 4 * c + (j - 4);
  else if constexpr (QT == kQ4_K || QT == kQ5_K) return 64 * (c / 8) + 4 * (c % 8) + (j < 4 ? j : 32 + j - 4);
  else return 128 * (c / 8) + 32 * (j / 4) + 4 * (c % 8) + (j % 4);
}

template <int QT, bool WIDE, int MT>
__global__ __launch_bounds__(256) void gemv_rm_kernel(View v, const float* __restrict__ x, uint32_t m,
                                                      uint32_t ksplit, float* __restrict__ out) {
  using G = RmGeo<QT>;
  constexpr int OUT = G::kOut;
  __shared__ float red[3][MT][OUT][64];
  const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const uint32_t nb_count = static_cast<uint32_t>(v.n / G::kBs);
  const uint32_t cu = blockIdx.x * 64 + lane;  // global column unit
  const uint32_t nb = cu / G::kCus, c = cu % G::kCus;
  const bool live = nb < nb_count;
  const uint32_t K = static_cast<uint32_t>(v.k);
  // this workgroup's K range, then this wavefront's quarter of it
  const uint32_t kb = static_cast<uint32_t>((static_cast<uint64_t>(blockIdx.y) * K) / ksplit);
  const uint32_t ke = static_cast<uint32_t>((static_cast<uint64_t>(blockIdx.y + 1) * K) / ksplit);
  const uint32_t k0 = kb + (ke - kb) * wave / 4, k1 = kb + (ke - kb) * (wave + 1) / 4;

  float acc[MT][OUT];
#pragma unroll
  for (int r = 0; r < MT; ++r)
#pragma unroll
    for (int j = 0; j < OUT; ++j) acc[r][j] = 0.0f;
  const uint64_t blk_nb = live ? nb : 0;  // lanes past N read block 0 and store nothing
#pragma unroll 4
  for (uint32_t k = k0; k < k1; ++k) {
    float w[OUT];
    rm_weights<QT, WIDE>(v, static_cast<uint64_t>(k) * nb_count + blk_nb, c, w);
#pragma unroll
    for (int r = 0; r < MT; ++r) {
      const float xv = static_cast<uint32_t>(r) < m ? x[static_cast<uint64_t>(r) * K + k] : 0.0f;
#pragma unroll
      for (int j = 0; j < OUT; ++j) acc[r][j] = fmaf(xv, w[j], acc[r][j]);
    }
  }
  // the four K quarters, in order
  if (wave > 0) {
#pragma unroll
    for (int r = 0; r < MT; ++r)
#pragma unroll
      for (int j = 0; j < OUT; ++j) red[wave - 1][r][j][lane] = acc[r][j];
  }
  __syncthreads();
  if (wave != 0 || !live) return;
  float* dst = out + static_cast<uint64_t>(blockIdx.y) * m * v.n;
#pragma unroll
  for (int r = 0; r < MT; ++r) {
    if (static_cast<uint32_t>(r) >= m) break;
#pragma unroll
    for (int j = 0; j < OUT; ++j) {
      float s = ((acc[r][j] + red[0][r][j][lane]) + red[1][r][j][lane]) + red[2][r][j][lane];
      const uint64_t col = static_cast<uint64_t>(nb) * G::kBs + rm_offset<QT>(c, j);
      // a NaN or infinite activation: the reference's order decides NaN or
      // +-Inf (with a K split, rm_sum_kernel checks the sum instead)
      if (ksplit == 1 && !__builtin_isfinite(s)) s = exact_row_major_col<QT, WIDE>(v, x + static_cast<uint64_t>(r) * K, col);
      dst[static_cast<uint64_t>(r) * v.n + col] = s;
    }
  }
}

// y = sum of the K-split partials in split order; a sum that is not finite
// is recomputed in the reference's order
template <int QT, bool WIDE>
__global__ __launch_bounds__(256) void rm_sum_kernel(const float* __restrict__ part, uint32_t splits,
                                                     uint64_t count, float* __restrict__ y, View v,
                                                     const float* __restrict__ x) {
  const uint64_t i = static_cast<uint64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i >= count) return;
  // loads issued 8 at a time with no condition (past the last split the last
  // one is read again and not added), ahead of the in-order adds
  float s = 0.0f;
  for (uint32_t p0 = 0; p0 < splits; p0 += 8) {
    float t[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const uint32_t pj = p0 + j < splits ? p0 + j : splits - 1;
      t[j] = part[static_cast<uint64_t>(pj) * count + i];
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) s = p0 + j == 0 ? t[j] : p0 + j < splits ? s + t[j] : s;
  }
  if (!__builtin_isfinite(s)) s = exact_row_major_col<QT, WIDE>(v, x + (i / v.n) * v.k, i % v.n);
  y[i] = s;
}

// ------------------------------------------------------------ tiled image

constexpr int kRmtRows = 2;     // activation rows per launch
constexpr int kRmtStride = 17;  // float4s per summed lane in LDS: 64 outputs and one of padding

// Records per wavefront, all loaded before the first is consumed (a record
// in registers with its activation: Q4_0 11, Q4_K 14, Q8_0 and Q6_K 19, Q5_K
// 22 VGPRs). Q4_0/Q4_K take 8 at two wavefronts per SIMD; the others 4 at
// three, as 6 leaves them at two: Q5_K 4096 x 14336 M=1 24.4 us with 6 slots,
// 19.0 with 4; Q6_K 23.6 / 19.1; Q4_K with 4 slots 16.6 against 15.9 (MI355X).
constexpr uint32_t rmt_max_slots(int32_t qtype, uint32_t rows) {
  return rows > 1 ? 4u : (qtype == kQ4_0 || qtype == kQ4_K) ? 8u : 4u;
}

// Record of tile t into r, with the activations of its row k = 16t + c,
// read at min(k, K - 1) (rows past K are zero in the record and their
// activation is zeroed at use). No condition on loaded values here, so that
// nothing waits for the loads before the record is consumed.
template <int QT, bool WIDE, int MT>
__device__ __forceinline__ void rmt_fetch(const uint8_t* rec, uint32_t lane, uint32_t k, uint32_t K,
                                          const float* __restrict__ x, typename Unit<QT>::Raw& r,
                                          float (&xs)[MT]) {
  const uint32_t kk = k < K ? k : K - 1;
#pragma unroll
  for (int i = 0; i < MT; ++i) xs[i] = x[static_cast<uint64_t>(i) * K + kk];
  Unit<QT>::template load<WIDE, true>(rec, lane, r);
}

// One record's products, acc[i][8 st + e] += x_i w for step st's code e. The
// codes arrive centred, s (q - z) in a signed byte (one sign-extending
// conversion); a / s is exact. Q8_0, Q4_0 and Q6_K have no offset left (w =
// (a / s) s (q - z)): the lane forms x a / s once per window and multiplies.
// Q4_K/Q5_K keep b - a z: the lane forms each weight with one fused
// multiply-add, w = (a / s) s (q - z) - (b - a z), as a sum of x a q and of
// x b over K would cancel in f32 at small K.
template <int QT, bool WIDE, int MT>
__device__ __forceinline__ void rmt_consume(const typename Unit<QT>::Raw& r, uint32_t g, bool live,
                                            const float (&xr)[MT], float (&acc)[MT][64]) {
  using U = Unit<QT>;
  constexpr int kW = U::kWindows, kS = U::kSteps;
  constexpr bool kOff = window_centered<QT>();
  constexpr float kInv = 1.0f / static_cast<float>(code_scale<QT>());
  constexpr float kCentre = static_cast<float>(code_centre<QT>());
  float a[kW], b[kW], xa[MT][kW], xs[MT];
#pragma unroll
  for (int i = 0; i < MT; ++i) xs[i] = live ? xr[i] : 0.0f;
  U::template scales<WIDE>(g, r, a, b);
#pragma unroll
  for (int w = 0; w < kW; ++w) {
    if constexpr (kOff) {
      b[w] = a[w] * kCentre - b[w];  // -(b - a z)
      a[w] *= kInv;
    } else {
      const float as = a[w] * kInv;
#pragma unroll
      for (int i = 0; i < MT; ++i) xa[i][w] = xs[i] * as;
    }
  }
#pragma unroll
  for (int st = 0; st < 8; ++st) {
    const uint64_t q = static_cast<uint64_t>(gemv_codes<QT>(r, g, st));
    const uint32_t lo = static_cast<uint32_t>(q), hi = static_cast<uint32_t>(q >> 32);
    const int w = st / kS;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const uint32_t word = e < 4 ? lo : hi;
      const float qf = static_cast<float>(static_cast<int8_t>(word >> (8 * (e & 3))));
      if constexpr (kOff) {
        const float wt = fmaf(a[w], qf, b[w]);
#pragma unroll
        for (int i = 0; i < MT; ++i) acc[i][8 * st + e] = fmaf(xs[i], wt, acc[i][8 * st + e]);
      } else {
#pragma unroll
        for (int i = 0; i < MT; ++i) acc[i][8 * st + e] = fmaf(xa[i][w], qf, acc[i][8 * st + e]);
      }
    }
  }
}

template <int QT, bool WIDE, int MT, int R>
__global__ __launch_bounds__(256) void gemv_rmt_kernel(View v, const float* __restrict__ x, uint32_t m,
                                                       uint32_t ksplit, float* __restrict__ out) {
  using U = Unit<QT>;
  // [wavefront][row][lane group g * 4 + c, c < 4][64 outputs]
  __shared__ float4 red[4][MT][16][kRmtStride];
  const uint32_t lane = threadIdx.x & 63, g = lane >> 4, c = lane & 15;
  const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // uniform: scalar branches
  const uint32_t K = static_cast<uint32_t>(v.k), T = v.tiles;
  const uint32_t tb = static_cast<uint32_t>((static_cast<uint64_t>(blockIdx.y) * T) / ksplit);
  const uint32_t te = static_cast<uint32_t>((static_cast<uint64_t>(blockIdx.y + 1) * T) / ksplit);
  const uint8_t* base = v.qs + static_cast<uint64_t>(blockIdx.x) * v.rec.bytes;
  const uint64_t tile_bytes = static_cast<uint64_t>(v.units) * v.rec.bytes;

  float acc[MT][64];
#pragma unroll
  for (int i = 0; i < MT; ++i)
#pragma unroll
    for (int j = 0; j < 64; ++j) acc[i][j] = 0.0f;
  // this wavefront's records: tiles t0, t0 + 4, ... below te, n <= R of them
  // (the host picks the split count so). All R loads are issued first, with
  // no condition (slots past n load the last record again), so that each
  // record waits only for its own loads.
  const uint32_t t0 = tb + wave, n = t0 < te ? (te - t0 + 3) / 4 : 0;
  if (n > 0) {
    typename U::Raw r[R];
    float xs[R][MT];
#pragma unroll
    for (int j = 0; j < R; ++j) {
      const uint32_t t = t0 + 4 * (static_cast<uint32_t>(j) < n ? j : n - 1);
      rmt_fetch<QT, WIDE, MT>(base + t * tile_bytes, lane, 16 * t + c, K, x, r[j], xs[j]);
      // loads in record order, all before the first record's arithmetic
      __builtin_amdgcn_sched_barrier(0);
    }
    // every slot is consumed (no branch, so no load sinks into one): a slot
    // past n, or a row past K, adds zero
#pragma unroll
    for (int j = 0; j < R; ++j)
      rmt_consume<QT, WIDE, MT>(r[j], g, static_cast<uint32_t>(j) < n && 16 * (t0 + 4 * j) + c < K, xs[j], acc);
  }

  // rows c, c + 4, c + 8, c + 12 of each lane group, then lanes c < 4 to LDS
#pragma unroll
  for (int i = 0; i < MT; ++i)
#pragma unroll
    for (int j = 0; j < 64; ++j) {
      acc[i][j] += dpp_move<kDppRor8>(acc[i][j]);
      acc[i][j] += dpp_move<kDppRor4>(acc[i][j]);
    }
  if (c < 4) {
#pragma unroll
    for (int i = 0; i < MT; ++i) {
      float4* dst = red[wave][i][4 * g + c];
#pragma unroll
      for (int q = 0; q < 16; ++q)
        dst[q] = make_float4(acc[i][4 * q], acc[i][4 * q + 1], acc[i][4 * q + 2], acc[i][4 * q + 3]);
    }
  }
  __syncthreads();
  // wavefront i sums activation row i: lane 16g + h takes outputs 4h .. 4h + 3
  // of lane group g (step h / 2: elements window_first(g, h / 8) + 8 (h / 2 % 4)
  // + 4 (h % 2) + [0, 4))
  if (wave >= static_cast<uint32_t>(MT) || wave >= m) return;
  const uint32_t h = c, step = h / 2;
  float4 s = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
  for (int wv = 0; wv < 4; ++wv)
#pragma unroll
    for (int cc = 0; cc < 4; ++cc) {
      const float4 p = red[wv][wave][4 * g + cc][h];
      s.x += p.x; s.y += p.y; s.z += p.z; s.w += p.w;
    }
  const uint32_t e0 = window_first<QT>(g, step / 4) + 8 * (step % 4) + 4 * (h % 2);
  const uint64_t n0 = static_cast<uint64_t>(blockIdx.x) * 256 + e0;
  float* dst = out + (static_cast<uint64_t>(blockIdx.y) * m + wave) * v.n + n0;
  const float val[4] = {s.x, s.y, s.z, s.w};
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    float y = val[e];
    // a NaN or infinite activation: the reference's order decides NaN or
    // +-Inf (with a K split, rm_sum_kernel checks the sum instead)
    if (ksplit == 1 && !__builtin_isfinite(y))
      y = exact_row_major_col<QT, WIDE>(v, x + static_cast<uint64_t>(wave) * K, n0 + e);
    dst[e] = y;
  }
}

template <int QT, bool WIDE, int MT>
hipError_t launch_rmt_rows(const View& v, const float* x, uint32_t m, float* out, uint32_t splits, hipStream_t st) {
  // records per wavefront: ceil(ceil(T / splits) / 4), served by the smallest slot count that holds them
  const uint32_t per = static_cast<uint32_t>(((v.tiles + splits - 1) / splits + 3) / 4);
  const dim3 grid(v.units, splits);
  auto go = [&](auto kern) {
    hipLaunchKernelGGL(kern, grid, dim3(256), 0, st, v, x, m, splits, out);
    return hipGetLastError();
  };
  constexpr int kMax = static_cast<int>(rmt_max_slots(QT, MT));
  if (per <= 2) return go(gemv_rmt_kernel<QT, WIDE, MT, 2>);
  if (per <= 4) return go(gemv_rmt_kernel<QT, WIDE, MT, 4>);
  if constexpr (kMax > 4) {
    if (per <= kMax) return go(gemv_rmt_kernel<QT, WIDE, MT, kMax>);
  }
  return hipErrorInvalidValue;
}

template <int QT, bool WIDE>
hipError_t launch_rmt_q(const View& v, const float* x, uint32_t m, float* y, float* part, uint32_t splits,
                        hipStream_t st) {
  float* out = splits > 1 ? part : y;
  if (m != 1 && m != kRmtRows) return hipErrorInvalidValue;  // the kernel reads MT = m rows
  hipError_t e = m == 1 ? launch_rmt_rows<QT, WIDE, 1>(v, x, m, out, splits, st)
                        : launch_rmt_rows<QT, WIDE, kRmtRows>(v, x, m, out, splits, st);
  if (e != hipSuccess || splits == 1) return e;
  const uint64_t count = static_cast<uint64_t>(m) * v.n;
  hipLaunchKernelGGL((rm_sum_kernel<QT, WIDE>), dim3(static_cast<uint32_t>((count + 255) / 256)), dim3(256), 0,
                     st, part, splits, count, y, v, x);
  return hipGetLastError();
}

template <int QT, bool WIDE>
hipError_t launch_rm_q(const View& v, const float* x, uint32_t m, float* y, float* part, uint32_t splits,
                       hipStream_t st) {
  const uint64_t cus = (v.n / RmGeo<QT>::kBs) * RmGeo<QT>::kCus;
  float* out = splits > 1 ? part : y;
  const dim3 grid(static_cast<uint32_t>((cus + 63) / 64), splits);
  if (m == 1)
    hipLaunchKernelGGL((gemv_rm_kernel<QT, WIDE, 1>), grid, dim3(256), 0, st, v, x, m, splits, out);
  else
    hipLaunchKernelGGL((gemv_rm_kernel<QT, WIDE, 4>), grid, dim3(256), 0, st, v, x, m, splits, out);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || splits == 1) return e;
  const uint64_t count = static_cast<uint64_t>(m) * v.n;
  hipLaunchKernelGGL((rm_sum_kernel<QT, WIDE>), dim3(static_cast<uint32_t>((count + 255) / 256)), dim3(256), 0,
                     st, part, splits, count, y, v, x);
  return hipGetLastError();
}

}  // namespace

namespace {

// Row-major GEMM, 2 rows and more: y[m, n] = sum_k x[m, k] w(k, n) with the
// weights dequantized in LDS, never stored to HBM. Workgroup (u, mb, z) takes
// unit u (outputs 256u .. 256u + 255), rows 16 TM mb .. of x and K part z
// (tiles [z T / P, (z + 1) T / P)). A stage is 64 weight rows: wavefront w
// loads the record of the stage's tile w (Unit<QT>, lane 16g + c row c's lane
// group g) and writes its 64 weights per lane to LDS as f32, each by the
// reference's operation sequence, so bit-identical to dequantize
// (matmul.rs:162-280): Q8_0 d q; Q4_0 d (q - 8); Q4_K/Q5_K (d sc) q - dmin m,
// no fused multiply-add (the file is compiled with -ffp-contract=off); Q6_K
// (d sc) (q - 32). The stage's activations go to LDS beside it. The
// next stage's record and activations are loaded into registers while the
// matrix cores (v_mfma_f32_16x16x4f32, f32 products) take the current one:
// wavefront w owns outputs 64w .. 64w + 63 for all 16 TM rows. Each 32-row
// half of a stage is summed apart and then added to the running sums (the
// f32 matrix-core GEMM's staged order). One part stores y, recomputing a
// non-finite sum in the reference's order; more store partial sums, which
// rm_sum_kernel adds in part order.
constexpr uint32_t kRmgStageK = 64;       // weight rows per stage: one record per wavefront
constexpr uint32_t kRmgWs = 256 + 4;      // LDS row stride of the stage's weights (floats)
constexpr uint32_t kRmgXs = kRmgStageK + 4;  // LDS row stride of the stage's activations

typedef float rmg_f32x4 __attribute__((ext_vector_type(4)));

template <int QT, bool WIDE, int TM>
__global__ __launch_bounds__(256) void rm_gemm_kernel(View v, const float* __restrict__ x, uint32_t M,
                                                      uint32_t parts, float* __restrict__ out) {
  using U = Unit<QT>;
  constexpr int kW = U::kWindows, kS = U::kSteps;
  __shared__ __align__(16) float ws[kRmgStageK * kRmgWs];
  __shared__ __align__(16) float xs[TM * 16 * kRmgXs];
  const uint32_t lane = threadIdx.x & 63, g = lane >> 4, c = lane & 15;
  const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const uint32_t u = blockIdx.x, m0 = blockIdx.y * TM * 16, z = blockIdx.z;
  const uint32_t K = static_cast<uint32_t>(v.k), T = v.tiles;
  const uint32_t tb = static_cast<uint32_t>((static_cast<uint64_t>(z) * T) / parts);
  const uint32_t te = static_cast<uint32_t>((static_cast<uint64_t>(z + 1) * T) / parts);
  const uint32_t kend = 16 * te < K ? 16 * te : K;  // activations past it are zero
  const uint32_t stages = (te - tb + 3) / 4;
  const uint8_t* base = v.qs + static_cast<uint64_t>(u) * v.rec.bytes;
  const uint64_t tile_bytes = static_cast<uint64_t>(v.units) * v.rec.bytes;

  // two stages in flight: stage s's record and activations in registers
  // r[s % 2], xr[s % 2] (s + 1 loads while s is multiplied)
  typename U::Raw r[2];
  rmg_f32x4 xr[2][TM];
  // stage s: tile tb + 4s + wave (if below te) and activation columns
  // 16 tb + 64 s .. + 63 of rows m0 .. m0 + 16 TM - 1
  auto fetch = [&](uint32_t s, typename U::Raw& rr, rmg_f32x4 (&xx)[TM]) {
    const uint32_t t = tb + 4 * s + wave;
    if (t < te) U::template load<WIDE>(base + t * tile_bytes, lane, rr);
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      const uint32_t e = threadIdx.x + 256 * i, row = e / 16, k = 16 * tb + kRmgStageK * s + (e % 16) * 4;
      xx[i] = (m0 + row < M && k < kend)
                  ? *reinterpret_cast<const rmg_f32x4*>(x + static_cast<uint64_t>(m0 + row) * K + k)
                  : rmg_f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    }
  };
  auto put = [&](uint32_t s, const typename U::Raw& rr, const rmg_f32x4 (&xx)[TM]) {
    const uint32_t t = tb + 4 * s + wave;
    float* wrow = ws + (16 * wave + c) * kRmgWs;
    if (t < te) {
      float a[kW], b[kW];
      U::template scales<WIDE>(g, rr, a, b);
#pragma unroll
      for (int st = 0; st < 8; ++st) {
        const uint64_t q = static_cast<uint64_t>(U::codes(rr, g, st));
        const int w = st / kS;
        float o[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const uint32_t byte = static_cast<uint32_t>(q >> (8 * e)) & 0xFFu;
          if constexpr (QT == kQ8_0) {
            o[e] = a[w] * static_cast<float>(static_cast<int8_t>(byte));
          } else if constexpr (QT == kQ4_0) {
            o[e] = a[w] * (static_cast<float>(byte) - 8.0f);
          } else if constexpr (QT == kQ6_K) {
            o[e] = a[w] * static_cast<float>(static_cast<int32_t>(byte) - 32);
          } else {
            o[e] = a[w] * static_cast<float>(byte) - b[w];
          }
        }
        float4* dst = reinterpret_cast<float4*>(wrow + window_first<QT>(g, st / 4) + 8 * (st % 4));
        dst[0] = make_float4(o[0], o[1], o[2], o[3]);
        dst[1] = make_float4(o[4], o[5], o[6], o[7]);
      }
    } else {
#pragma unroll
      for (int st = 0; st < 8; ++st) {
        float4* dst = reinterpret_cast<float4*>(wrow + window_first<QT>(g, st / 4) + 8 * (st % 4));
        dst[0] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        dst[1] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
      }
    }
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      const uint32_t e = threadIdx.x + 256 * i;
      *reinterpret_cast<rmg_f32x4*>(xs + (e / 16) * kRmgXs + (e % 16) * 4) = xx[i];
    }
  };

  rmg_f32x4 acc[TM][4];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = rmg_f32x4{0.0f, 0.0f, 0.0f, 0.0f};

  // lane (c, g) supplies A[c][g] = x[row c][k] and B[g][c] = w(k, column c)
  // of each 16 x 16 x 4 product, k = 16 kk + 4 g + step
  const float* xb = xs + c * kRmgXs + 4 * g;
  const float* wb = ws + (4 * g) * kRmgWs + wave * 64 + c;
  auto multiply = [&]() {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      rmg_f32x4 part[TM][4];
#pragma unroll
      for (int k2 = 0; k2 < 2; ++k2) {
        const int kk = 2 * h + k2;
        rmg_f32x4 a[TM];
#pragma unroll
        for (int i = 0; i < TM; ++i) a[i] = *reinterpret_cast<const rmg_f32x4*>(xb + i * 16 * kRmgXs + kk * 16);
#pragma unroll
        for (int st = 0; st < 4; ++st) {
          float bv[4];
#pragma unroll
          for (int j = 0; j < 4; ++j) bv[j] = wb[(kk * 16 + st) * kRmgWs + j * 16];
#pragma unroll
          for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j)
              part[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(
                  a[i][st], bv[j], k2 == 0 && st == 0 ? rmg_f32x4{0.0f, 0.0f, 0.0f, 0.0f} : part[i][j], 0, 0, 0);
        }
      }
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] += part[i][j];
    }
  };
  if (stages > 0) fetch(0, r[0], xr[0]);
  if (stages > 1) fetch(1, r[1], xr[1]);
  for (uint32_t s = 0; s < stages; s += 2) {
    put(s, r[0], xr[0]);
    __syncthreads();
    if (s + 2 < stages) fetch(s + 2, r[0], xr[0]);
    multiply();
    __syncthreads();
    if (s + 1 < stages) {
      put(s + 1, r[1], xr[1]);
      __syncthreads();
      if (s + 3 < stages) fetch(s + 3, r[1], xr[1]);
      multiply();
      __syncthreads();
    }
  }

  // lane (c, g) holds rows 4g .. 4g + 3 of each 16 x 16 block, column c
  float* const dst = out + (parts == 1 ? 0 : static_cast<uint64_t>(z) * M * v.n);
  bool bad = false;
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint64_t n = static_cast<uint64_t>(u) * 256 + wave * 64 + j * 16 + c;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const uint32_t m = m0 + i * 16 + 4 * g + q;
        if (m >= M) continue;
        bad |= !__builtin_isfinite(acc[i][j][q]);
        dst[static_cast<uint64_t>(m) * v.n + n] = acc[i][j][q];
      }
    }
  // with one part, a non-finite sum (NaN or infinite activations) is
  // recomputed in the reference's order, which decides NaN or +-Inf; this
  // lane's own stores are read back (a loop of its own, so that the
  // accumulator tile above stays in registers)
  if (parts == 1 && bad) {
#pragma unroll 1
    for (int e = 0; e < TM * 16; ++e) {
      const uint32_t i = e / 16, j = (e / 4) % 4, q = e % 4, m = m0 + i * 16 + 4 * g + q;
      const uint64_t n = static_cast<uint64_t>(u) * 256 + wave * 64 + j * 16 + c;
      float* p = dst + static_cast<uint64_t>(m) * v.n + n;
      if (m < M && !__builtin_isfinite(*p)) *p = exact_row_major_col<QT, WIDE>(v, x + static_cast<uint64_t>(m) * K, n);
    }
  }
}

template <int QT, bool WIDE>
hipError_t launch_rm_gemm_q(const View& v, const float* x, uint32_t m, float* y, float* part, uint32_t parts,
                            hipStream_t st) {
  const uint32_t tm = rm_gemm_tile_rows(m) / 16;
  const dim3 grid(v.units, (m + 16 * tm - 1) / (16 * tm), parts);
  float* out = parts > 1 ? part : y;
  if (tm == 1)
    hipLaunchKernelGGL((rm_gemm_kernel<QT, WIDE, 1>), grid, dim3(256), 0, st, v, x, m, parts, out);
  else
    hipLaunchKernelGGL((rm_gemm_kernel<QT, WIDE, 2>), grid, dim3(256), 0, st, v, x, m, parts, out);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || parts == 1) return e;
  const uint64_t count = static_cast<uint64_t>(m) * v.n;
  hipLaunchKernelGGL((rm_sum_kernel<QT, WIDE>), dim3(static_cast<uint32_t>((count + 255) / 256)), dim3(256), 0,
                     st, part, parts, count, y, v, x);
  return hipGetLastError();
}

}  // namespace

// 16-row tiles up to 16 rows, 32 above: 64-row tiles (one wavefront per
// SIMD) ran 2-5% slower from 64 rows on (MI355X, Q4_K 4096 x 14336 M=512
// 684 against 660 us, M=2048 2388 against 2272; Q8_0 4096 x 4096 M=2048 682
// against 642)
uint32_t rm_gemm_tile_rows(uint64_t m) { return m <= 16 ? 16 : 32; }

uint32_t rm_gemm_parts(const Image& im, uint64_t m, uint64_t max_part_floats) {
  // The part count with the fewest rounds of resident workgroups per part
  // (two per CU, 256 CUs), the smaller count on a tie; each part at least two
  // stages (8 tiles), the partial sums within max_part_floats.
  const uint64_t rows = rm_gemm_tile_rows(m), slots = 512;
  const uint64_t groups = static_cast<uint64_t>(im.units) * ((m + rows - 1) / rows);
  uint64_t pmax = im.tiles / 8;
  const uint64_t by_space = max_part_floats / (m * im.n);
  if (pmax > by_space) pmax = by_space;
  if (pmax > 64) pmax = 64;
  uint64_t best = 1;
  for (uint64_t p = 2; p <= pmax; ++p) {
    // rounds(p) / p < rounds(best) / best
    const uint64_t rp = (groups * p + slots - 1) / slots, rb = (groups * best + slots - 1) / slots;
    if (rp * best < rb * p) best = p;
  }
  return static_cast<uint32_t>(best);
}

bool rm_gemm_supported(const Image& im) {
  return gemv_rm_supported(im) && im.tiled && im.k % 4 == 0 && im.k <= 0xFFFFFFF0ull;
}

hipError_t launch_rm_gemm(const Image& im, const View& v, const float* x, uint64_t m, float* y, float* part,
                          uint32_t parts, hipStream_t st) {
  // grid: units x row blocks (at most 0xFFFF) x parts; each part at least one tile
  if (!rm_gemm_supported(im) || m < 1 || (m + 31) / 32 > 0xFFFFu || parts < 1 || parts > 0xFFFFu ||
      parts > im.tiles || (parts > 1 && part == nullptr) || v.units != im.n / 256 || v.tiles != (im.k + 15) / 16 ||
      (m * im.n + 255) / 256 > 0x7fffffffull)
    return hipErrorInvalidValue;
  const uint32_t mm = static_cast<uint32_t>(m);
  const bool w = im.wide != 0;
  switch (im.qtype) {
    case kQ8_0: return w ? launch_rm_gemm_q<kQ8_0, true>(v, x, mm, y, part, parts, st)
                         : launch_rm_gemm_q<kQ8_0, false>(v, x, mm, y, part, parts, st);
    case kQ4_0: return w ? launch_rm_gemm_q<kQ4_0, true>(v, x, mm, y, part, parts, st)
                         : launch_rm_gemm_q<kQ4_0, false>(v, x, mm, y, part, parts, st);
    case kQ4_K: return w ? launch_rm_gemm_q<kQ4_K, true>(v, x, mm, y, part, parts, st)
                         : launch_rm_gemm_q<kQ4_K, false>(v, x, mm, y, part, parts, st);
    case kQ5_K: return w ? launch_rm_gemm_q<kQ5_K, true>(v, x, mm, y, part, parts, st)
                         : launch_rm_gemm_q<kQ5_K, false>(v, x, mm, y, part, parts, st);
    case kQ6_K: return w ? launch_rm_gemm_q<kQ6_K, true>(v, x, mm, y, part, parts, st)
                         : launch_rm_gemm_q<kQ6_K, false>(v, x, mm, y, part, parts, st);
    default: return hipErrorInvalidValue;
  }
}

bool gemv_rm_supported(const Image& im) {
  // tiled: grid x = units, grid y = splits of at most 4 * 4 records per workgroup
  return im.layout == kRowMajor && im.qtype >= kQ8_0 && im.qtype <= kQ6_K && im.n % block_elems(im.qtype) == 0 &&
         im.k > 0 && (!im.tiled || (im.units <= 0xFFFFu && im.tiles <= 16ull * 0xFFFFu));
}

uint32_t gemv_rm_rows(const Image& im) { return im.tiled ? kRmtRows : 4; }

uint32_t gemv_rm_splits(const Image& im, uint32_t m) {
  const uint32_t be = block_elems(im.qtype);
  if (im.tiled) {
    // About 512 workgroups (two wavefronts per SIMD on 256 CUs) give each
    // wavefront ceil(T / (4 s)) records; that count is rounded up to a slot
    // count of the kernel (2, 4 or the most), and s lowered to the fewest
    // splits that keep it.
    const uint64_t rmax = rmt_max_slots(im.qtype, m > 1 ? kRmtRows : 1);
    const uint64_t s0 = (512 + im.units - 1) / im.units;
    const uint64_t per = ((im.tiles + s0 - 1) / s0 + 3) / 4;
    const uint64_t slots = per <= 2 ? 2 : per <= 4 ? 4 : rmax;
    const uint64_t s = (im.tiles + 4 * slots - 1) / (4 * slots);
    return static_cast<uint32_t>(s < 1 ? 1 : s);
  }
  // enough K splits for about 1024 workgroups, keeping at least 16 k per
  // wavefront (4 wavefronts per workgroup) and at most 256 splits
  const uint64_t out = im.qtype == kQ8_0 ? 4 : im.qtype == kQ6_K ? 16 : 8;
  const uint64_t col_groups = ((im.n / be) * (be / out) + 63) / 64;
  uint64_t s = col_groups >= 1024 ? 1 : 1024 / col_groups;
  const uint64_t cap = im.k / 64 < 256 ? im.k / 64 : 256;
  if (s > cap) s = cap;
  return static_cast<uint32_t>(s < 1 ? 1 : s);
}

hipError_t launch_gemv_rm(const Image& im, const View& v, const float* x, uint32_t m, float* y, float* part,
                          uint32_t splits, hipStream_t st) {
  if (m < 1 || m > gemv_rm_rows(im) || splits < 1 || (splits > 1 && part == nullptr)) return hipErrorInvalidValue;
  const bool wide = im.wide != 0;
  if (im.tiled) {
    if (v.units != im.n / 256 || v.tiles != (im.k + 15) / 16 || !gemv_rm_supported(im)) return hipErrorInvalidValue;
    switch (im.qtype) {
      case kQ8_0: return wide ? launch_rmt_q<kQ8_0, true>(v, x, m, y, part, splits, st)
                              : launch_rmt_q<kQ8_0, false>(v, x, m, y, part, splits, st);
      case kQ4_0: return wide ? launch_rmt_q<kQ4_0, true>(v, x, m, y, part, splits, st)
                              : launch_rmt_q<kQ4_0, false>(v, x, m, y, part, splits, st);
      case kQ4_K: return wide ? launch_rmt_q<kQ4_K, true>(v, x, m, y, part, splits, st)
                              : launch_rmt_q<kQ4_K, false>(v, x, m, y, part, splits, st);
      case kQ5_K: return wide ? launch_rmt_q<kQ5_K, true>(v, x, m, y, part, splits, st)
                              : launch_rmt_q<kQ5_K, false>(v, x, m, y, part, splits, st);
      case kQ6_K: return wide ? launch_rmt_q<kQ6_K, true>(v, x, m, y, part, splits, st)
                              : launch_rmt_q<kQ6_K, false>(v, x, m, y, part, splits, st);
      default: return hipErrorInvalidValue;
    }
  }
  switch (im.qtype) {
    case kQ8_0: return wide ? launch_rm_q<kQ8_0, true>(v, x, m, y, part, splits, st)
                            : launch_rm_q<kQ8_0, false>(v, x, m, y, part, splits, st);
    case kQ4_0: return wide ? launch_rm_q<kQ4_0, true>(v, x, m, y, part, splits, st)
                            : launch_rm_q<kQ4_0, false>(v, x, m, y, part, splits, st);
    case kQ4_K: return wide ? launch_rm_q<kQ4_K, true>(v, x, m, y, part, splits, st)
                            : launch_rm_q<kQ4_K, false>(v, x, m, y, part, splits, st);
    case kQ5_K: return wide ? launch_rm_q<kQ5_K, true>(v, x, m, y, part, splits, st)
                            : launch_rm_q<kQ5_K, false>(v, x, m, y, part, splits, st);
    case kQ6_K: return wide ? launch_rm_q<kQ6_K, true>(v, x, m, y, part, splits, st)
                            : launch_rm_q<kQ6_K, false>(v, x, m, y, part, splits, st);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace qi
