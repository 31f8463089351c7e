// F32 weights: the reference's dense `matmul` (backends/cpu/src/backend.rs:
// 48-60 -> matmul.rs:92-117), y[m, n] = sum_k x[m, k] W[k, n] with W the
// row-major [K, N] f32 matrix (the unchanged runtime's LM head after a Q6_K
// head is dequantized at load, runtime/src/qwen3/loader.rs:47-61, is 2.49 GB
// of it). Two throughput paths, judged by the F32 tolerance (EXACT mode keeps
// the sequential-k kernel of qi_exact.hip):
//
// * up to 8 activation rows: a streaming GEMV (in 8-row launches for any
//   row count when K is not a multiple of 4). A lane owns 4 consecutive
//   columns and reads them with one 16-byte load per k (a wavefront reads
//   1 KB of a row), the activations are wavefront-uniform loads, and each k
//   adds x * w for every row with an FMA. The four wavefronts of a workgroup
//   split its K range and the grid's y dimension splits K further; the parts
//   are summed in a fixed order (through LDS, then f32w_sum_kernel), so
//   results do not depend on scheduling. HBM-bound: K * N * 4 bytes.
// * more rows: a GEMM on the f32 matrix cores (f32w_gemm_kernel below),
//   LDS-staged tiles of 32 to 128 rows by 128 or 256 columns.
//
// An output whose sum is not finite (a NaN or infinite activation, or an
// overflow) is recomputed in the reference's order, which fixes which outputs
// are NaN and which +-Inf.
#include "qi_device.h"
#include "qi_internal.h"

namespace qi {

namespace {

// the reference's per-output sum: acc = acc + x[k] * W[k, n], k ascending
__device__ __forceinline__ float f32w_exact(const float* W, uint32_t K, uint32_t N, const float* x, uint64_t n) {
  float s = 0.0f;
  for (uint32_t k = 0; k < K; ++k) s += x[k] * W[static_cast<uint64_t>(k) * N + n];
  return s;
}

template <int MT>
__global__ __launch_bounds__(256) void f32w_gemv_kernel(const float* __restrict__ W, uint32_t K, uint32_t N,
                                                        const float* __restrict__ x, uint32_t m,
                                                        uint32_t ksplit, float* __restrict__ out) {
  __shared__ float4 red[3][MT][64];
  const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const uint32_t n0 = (blockIdx.x * 64 + lane) * 4;
  const bool live = n0 < N;
  const uint32_t kb = static_cast<uint32_t>((static_cast<uint64_t>(blockIdx.y) * K) / ksplit);
  const uint32_t ke = static_cast<uint32_t>((static_cast<uint64_t>(blockIdx.y + 1) * K) / ksplit);
  const uint32_t k0 = kb + (ke - kb) * wave / 4, k1 = kb + (ke - kb) * (wave + 1) / 4;
  const float* col = W + (live ? n0 : 0);

  // rows past m repeat the last row (valid memory, never stored), so the
  // row loops have a fixed trip count and the accumulators stay in registers
  const float* xrow[MT];
#pragma unroll
  for (int r = 0; r < MT; ++r) xrow[r] = x + static_cast<uint64_t>(static_cast<uint32_t>(r) < m ? r : m - 1) * K;
  float4 acc[MT];
#pragma unroll
  for (int r = 0; r < MT; ++r) acc[r] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  uint32_t k = k0;
  // eight rows of W in flight ahead of their FMAs
  for (; k + 8 <= k1; k += 8) {
    float4 w[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) w[i] = *reinterpret_cast<const float4*>(col + static_cast<uint64_t>(k + i) * N);
#pragma unroll
    for (int r = 0; r < MT; ++r) {
      const float* xr = xrow[r] + k;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float xv = xr[i];
        acc[r].x = fmaf(xv, w[i].x, acc[r].x);
        acc[r].y = fmaf(xv, w[i].y, acc[r].y);
        acc[r].z = fmaf(xv, w[i].z, acc[r].z);
        acc[r].w = fmaf(xv, w[i].w, acc[r].w);
      }
    }
  }
  for (; k < k1; ++k) {
    const float4 w = *reinterpret_cast<const float4*>(col + static_cast<uint64_t>(k) * N);
#pragma unroll
    for (int r = 0; r < MT; ++r) {
      const float xv = xrow[r][k];
      acc[r].x = fmaf(xv, w.x, acc[r].x);
      acc[r].y = fmaf(xv, w.y, acc[r].y);
      acc[r].z = fmaf(xv, w.z, acc[r].z);
      acc[r].w = fmaf(xv, w.w, acc[r].w);
    }
  }
  // the four K quarters, in order
  if (wave > 0) {
#pragma unroll
    for (int r = 0; r < MT; ++r) red[wave - 1][r][lane] = acc[r];
  }
  __syncthreads();
  if (wave != 0 || !live) return;
  float* dst = out + static_cast<uint64_t>(blockIdx.y) * m * N;
#pragma unroll
  for (int r = 0; r < MT; ++r) {
    if (static_cast<uint32_t>(r) >= m) break;
    const float4 a = acc[r], b = red[0][r][lane], c = red[1][r][lane], d = red[2][r][lane];
    float v[4] = {((a.x + b.x) + c.x) + d.x, ((a.y + b.y) + c.y) + d.y, ((a.z + b.z) + c.z) + d.z,
                  ((a.w + b.w) + c.w) + d.w};
    if (ksplit == 1) {
#pragma unroll
      for (int j = 0; j < 4; ++j)
        if (!__builtin_isfinite(v[j])) v[j] = f32w_exact(W, K, N, x + static_cast<uint64_t>(r) * K, n0 + j);
    }
    *reinterpret_cast<float4*>(dst + static_cast<uint64_t>(r) * N + n0) = make_float4(v[0], v[1], v[2], v[3]);
  }
}

// y = sum of the K-split partials in split order; a non-finite sum is
// recomputed in the reference's order
__global__ __launch_bounds__(256) void f32w_sum_kernel(const float* __restrict__ part, uint32_t splits,
                                                       uint64_t count, float* __restrict__ y,
                                                       const float* __restrict__ W, uint32_t K, uint32_t N,
                                                       const float* __restrict__ x) {
  const uint64_t i = static_cast<uint64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i >= count) return;
  float s = part[i];
  uint32_t p = 1;
  for (; p + 8 <= splits; p += 8) {
    float t[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) t[j] = part[(p + j) * count + i];
#pragma unroll
    for (int j = 0; j < 8; ++j) s += t[j];
  }
  for (; p < splits; ++p) s += part[p * count + i];
  if (!__builtin_isfinite(s)) s = f32w_exact(W, K, N, x + (i / N) * K, i % N);
  y[i] = s;
}

}  // namespace

bool f32w_gemv_supported(const Image& im) {
  return im.qtype == kF32 && im.layout == kRowMajor && im.n % 4 == 0 && im.k > 0;
}

uint32_t f32w_splits(const Image& im) {
  // enough K splits for about 2048 workgroups (a few per CU at once, the
  // last wave of them short), keeping at least 64 rows of W per wavefront
  const uint64_t groups = (im.n / 4 + 63) / 64;
  uint64_t s = groups >= 2048 ? 1 : (2048 + groups - 1) / groups;
  const uint64_t cap = im.k / 256 < 256 ? im.k / 256 : 256;
  if (s > cap) s = cap;
  return static_cast<uint32_t>(s < 1 ? 1 : s);
}

hipError_t launch_f32w_gemv(const Image& im, const View& v, const float* x, uint32_t m, float* y, float* part,
                            uint32_t splits, hipStream_t st) {
  if (m < 1 || m > 8 || splits < 1 || (splits > 1 && part == nullptr) || !f32w_gemv_supported(im))
    return hipErrorInvalidValue;
  const float* W = reinterpret_cast<const float*>(v.qs);
  const uint32_t K = static_cast<uint32_t>(im.k), N = static_cast<uint32_t>(im.n);
  float* out = splits > 1 ? part : y;
  const dim3 grid(static_cast<uint32_t>((N / 4 + 63) / 64), splits);
  if (m == 1)
    hipLaunchKernelGGL((f32w_gemv_kernel<1>), grid, dim3(256), 0, st, W, K, N, x, m, splits, out);
  else if (m == 2)
    hipLaunchKernelGGL((f32w_gemv_kernel<2>), grid, dim3(256), 0, st, W, K, N, x, m, splits, out);
  else if (m <= 4)
    hipLaunchKernelGGL((f32w_gemv_kernel<4>), grid, dim3(256), 0, st, W, K, N, x, m, splits, out);
  else
    hipLaunchKernelGGL((f32w_gemv_kernel<8>), grid, dim3(256), 0, st, W, K, N, x, m, splits, out);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || splits == 1) return e;
  const uint64_t count = static_cast<uint64_t>(m) * N;
  hipLaunchKernelGGL(f32w_sum_kernel, dim3(static_cast<uint32_t>((count + 255) / 256)), dim3(256), 0, st, part,
                     splits, count, y, W, K, N, x);
  return hipGetLastError();
}

// ---------------------------------------------------------------- GEMM
//
// More rows: y[M, N] = x[M, K] W[K, N] on the f32 matrix cores
// (v_mfma_f32_16x16x4f32: f32 products, f32 sums). A workgroup owns an
// MT x NT tile of y (MT = WM*TM*16 rows, NT = WN*TN*16 columns), wavefront
// (wm, wn) a TM x TN grid of 16 x 16 blocks of it. K advances in stages of 32:
// the x stage (MT rows x 32, row stride 36 floats) and the W stage (32 rows x
// NT, row stride NT + 4) are loaded from HBM into registers with 16-byte
// loads while the previous stage is multiplied out of LDS, then stored into
// the other LDS buffer; one barrier per stage.
//
// Operands: for k-step s (0..3) of a 16-wide k slice, lane l (row or column
// l % 16, lane group g = l / 16) supplies k = 16 kk + 4 g + s. So an A operand
// for four k-steps is one 16-byte LDS read (x[row][16 kk + 4 g .. + 3]), and
// a B operand one 4-byte read of W[16 kk + 4 g + s][col]; the row strides put
// the four lane groups' rows in different LDS banks. Rows past M, k past K
// and columns past N load as zeros (K and N are multiples of 4, so a 16-byte
// load is all in or all out) and are never stored.
//
// Block order is XCD-aware: the hardware deals workgroups round-robin over
// the 8 XCDs, so workgroup b takes logical tile (b % 8) * ceil(B / 8) + b / 8
// and each XCD runs a contiguous run of logical tiles; M tiles vary fastest,
// so the workgroups sharing a W column panel run on one XCD's L2.
namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr uint32_t kF32Kt = 32;

// STAGED: per-stage sums, below (every launch takes them).
template <int WM, int WN, int TM, int TN, bool STAGED = false>
__global__ __launch_bounds__(WM * WN * 64) void f32w_gemm_kernel(const float* __restrict__ W, uint32_t K,
                                                                  uint32_t N, const float* __restrict__ x,
                                                                  uint32_t M, uint32_t mtiles,
                                                                  uint32_t ntiles, float* __restrict__ y) {
  constexpr int MT = WM * TM * 16, NT = WN * TN * 16, KT = kF32Kt, THREADS = WM * WN * 64;
  constexpr int XS = KT + 4, WS = NT + 4;
  constexpr int XL = MT * KT / 4 / THREADS, WL = KT * NT / 4 / THREADS;  // 16-byte loads per thread
  static_assert(XL >= 1 && WL >= 1 && MT * KT / 4 % THREADS == 0 && KT * NT / 4 % THREADS == 0, "tile");
  __shared__ __align__(16) float xs[2][MT * XS];
  __shared__ __align__(16) float ws[2][KT * WS];

  const uint32_t tiles = mtiles * ntiles;
  const uint32_t per = (tiles + 7) / 8;
  const uint32_t logical = (blockIdx.x % 8) * per + blockIdx.x / 8;
  if (logical >= tiles) return;
  const uint32_t m0 = (logical % mtiles) * MT, n0 = (logical / mtiles) * NT;
  const uint32_t t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const uint32_t wm = wave / WN, wn = wave % WN, r16 = lane & 15, g = lane >> 4;

  f32x4 xr[XL], wr[WL];
  auto load = [&](uint32_t k0) {
#pragma unroll
    for (int i = 0; i < XL; ++i) {
      const uint32_t e = t + i * THREADS, row = e / (KT / 4), k = k0 + (e % (KT / 4)) * 4;
      xr[i] = (m0 + row < M && k < K)
                  ? *reinterpret_cast<const f32x4*>(x + static_cast<uint64_t>(m0 + row) * K + k)
                  : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    }
#pragma unroll
    for (int i = 0; i < WL; ++i) {
      const uint32_t e = t + i * THREADS, kr = e / (NT / 4), n = n0 + (e % (NT / 4)) * 4;
      wr[i] = (k0 + kr < K && n < N)
                  ? __builtin_nontemporal_load(
                        reinterpret_cast<const f32x4*>(W + static_cast<uint64_t>(k0 + kr) * N + n))
                  : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    }
  };
  auto store = [&](int b) {
#pragma unroll
    for (int i = 0; i < XL; ++i) {
      const uint32_t e = t + i * THREADS;
      *reinterpret_cast<f32x4*>(&xs[b][(e / (KT / 4)) * XS + (e % (KT / 4)) * 4]) = xr[i];
    }
#pragma unroll
    for (int i = 0; i < WL; ++i) {
      const uint32_t e = t + i * THREADS;
      *reinterpret_cast<f32x4*>(&ws[b][(e / (NT / 4)) * WS + (e % (NT / 4)) * 4]) = wr[i];
    }
  };

  f32x4 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

  const uint32_t stages = (K + KT - 1) / KT;
  load(0);
  store(0);
  __syncthreads();
  for (uint32_t s = 0; s < stages; ++s) {
    const int b = s & 1;
    if (s + 1 < stages) load((s + 1) * KT);
    const float* xb = &xs[b][(wm * TM * 16 + r16) * XS + 4 * g];
    const float* wb = &ws[b][(4 * g) * WS + wn * TN * 16 + r16];
    // STAGED: the stage's KT products in sums of their own, added to the
    // running ones once per stage, so that each output's chain of dependent
    // matrix-instruction accumulations is KT / 4 long and then K / KT f32
    // additions. One chain over K missed the F32 bars wherever many outputs
    // were checked: F32 weights N(0, 0.02^2) at K = 4096, N = 4096, 130 and
    // 512 rows 1.06e-5 and 1.45e-5 componentwise, 2048 x 8192 x 300 rows
    // 1.15e-5; dequantized Q8_0 at 4096 x 4096 x 130 rows 1.09e-5. It
    // doubles the accumulator registers (one wavefront per SIMD for the
    // 128 x 128 tile).
    [[maybe_unused]] f32x4 part[TM][TN];
#pragma unroll
    for (int kk = 0; kk < KT / 16; ++kk) {
      f32x4 a[TM];
#pragma unroll
      for (int i = 0; i < TM; ++i) a[i] = *reinterpret_cast<const f32x4*>(xb + i * 16 * XS + kk * 16);
#pragma unroll
      for (int st = 0; st < 4; ++st) {
        float bv[TN];
#pragma unroll
        for (int j = 0; j < TN; ++j) bv[j] = wb[(kk * 16 + st) * WS + j * 16];
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
          for (int j = 0; j < TN; ++j) {
            if constexpr (STAGED)
              part[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(
                  a[i][st], bv[j], kk == 0 && st == 0 ? f32x4{0.0f, 0.0f, 0.0f, 0.0f} : part[i][j], 0, 0, 0);
            else
              acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[i][st], bv[j], acc[i][j], 0, 0, 0);
          }
      }
    }
    if constexpr (STAGED) {
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] += part[i][j];
    }
    if (s + 1 < stages) store(b ^ 1);
    __syncthreads();
  }

  // lane l holds rows 4 g + 0..3 of each block, column l % 16
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const uint32_t n = n0 + wn * TN * 16 + j * 16 + r16;
      if (n >= N) continue;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const uint32_t m = m0 + wm * TM * 16 + i * 16 + 4 * g + q;
        if (m >= M) continue;
        float v = acc[i][j][q];
        if (!__builtin_isfinite(v)) v = f32w_exact(W, K, N, x + static_cast<uint64_t>(m) * K, n);
        y[static_cast<uint64_t>(m) * N + n] = v;
      }
    }
}

template <int WM, int WN, int TM, int TN, bool STAGED>
hipError_t launch_f32w_gemm_t(const float* W, uint32_t K, uint32_t N, const float* x, uint32_t M, float* y,
                              hipStream_t st) {
  constexpr uint32_t MT = WM * TM * 16, NT = WN * TN * 16;
  const uint32_t mtiles = (M + MT - 1) / MT, ntiles = (N + NT - 1) / NT;
  const uint64_t tiles = static_cast<uint64_t>(mtiles) * ntiles;
  if (tiles > 0x7fffffffull) return hipErrorInvalidValue;
  const uint32_t grid = static_cast<uint32_t>((tiles + 7) / 8 * 8);
  hipLaunchKernelGGL((f32w_gemm_kernel<WM, WN, TM, TN, STAGED>), dim3(grid), dim3(WM * WN * 64), 0, st, W, K, N, x,
                     M, mtiles, ntiles, y);
  return hipGetLastError();
}

template <bool STAGED = false>
hipError_t launch_f32w_gemm_any(const float* W, uint32_t K, uint32_t N, const float* x, uint32_t M, float* y,
                                hipStream_t st) {
  // 32 x 256 tiles up to 32 rows, 64 x 128 above: with the staged sums the
  // 64 x 256 and 128 x 128 tiles ran at one wavefront per SIMD (LM head
  // 4096 x 151936, us per call: M=64 1122 against 933, M=512 6368 against
  // 5657 for 64 x 128)
  if (M <= 32) return launch_f32w_gemm_t<1, 4, 2, 4, STAGED>(W, K, N, x, M, y, st);
  return launch_f32w_gemm_t<2, 2, 2, 4, STAGED>(W, K, N, x, M, y, st);
}

}  // namespace

bool f32w_gemm_supported(const Image& im) { return f32w_gemv_supported(im) && im.k % 4 == 0; }

hipError_t launch_f32w_gemm(const Image& im, const View& v, const float* x, uint64_t m, float* y, hipStream_t st) {
  if (!f32w_gemm_supported(im) || m < 1 || m > 0x7fffffffull || im.k > 0x7fffffffull || im.n > 0x7fffffffull)
    return hipErrorInvalidValue;
  const float* W = reinterpret_cast<const float*>(v.qs);
  const uint32_t K = static_cast<uint32_t>(im.k), N = static_cast<uint32_t>(im.n), M = static_cast<uint32_t>(m);
  return launch_f32w_gemm_any<true>(W, K, N, x, M, y, st);
}

}  // namespace qi
