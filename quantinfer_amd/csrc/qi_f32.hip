// F32 weights: the reference's dense `matmul` (backends/cpu/src/backend.rs:
// 48-60 -> matmul.rs:92-117), y[m, n] = sum_k x[m, k] W[k, n] with W the
// row-major [K, N] f32 matrix (the unchanged runtime's LM head after a Q6_K
// head is dequantized at load, runtime/src/qwen3/loader.rs:47-61, is 2.49 GB
// of it). Two throughput paths, judged by the F32 tolerance (EXACT mode keeps
// the sequential-k kernel of qi_exact.hip):
//
// * up to 16 activation rows: a streaming GEMV, 8 rows per launch. A lane owns 4 consecutive
//   columns and reads them with one 16-byte load per k (a wavefront reads
//   1 KB of a row), the activations are wavefront-uniform loads, and each k
//   adds x * w for every row with an FMA. The four wavefronts of a workgroup
//   split its K range and the grid's y dimension splits K further; the parts
//   are summed in a fixed order (through LDS, then f32w_sum_kernel), so
//   results do not depend on scheduling. HBM-bound: K * N * 4 bytes.
// * more rows: rocBLAS sgemm (a plain f32 library GEMM on the matrix cores;
//   there is nothing to fuse into it).
//
// An output whose sum is not finite (a NaN or infinite activation, or an
// overflow) is recomputed in the reference's order, which fixes which outputs
// are NaN and which +-Inf.
#include <rocblas/rocblas.h>

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

// y[M, N] = x[M, K] W[K, N], all row-major: in rocBLAS's column-major terms
// y^T (N x M, ld N) = W^T (N x K, ld N) * x^T (K x M, ld K).
int f32w_sgemm(void* handle, const Image& im, const View& v, const float* x, uint64_t m, float* y,
               hipStream_t st) {
  rocblas_handle h = static_cast<rocblas_handle>(handle);
  if (rocblas_set_stream(h, st) != rocblas_status_success) return -1;
  const float one = 1.0f, zero = 0.0f;
  const rocblas_int n = static_cast<rocblas_int>(im.n), k = static_cast<rocblas_int>(im.k);
  const rocblas_int mm = static_cast<rocblas_int>(m);
  const rocblas_status s = rocblas_sgemm(h, rocblas_operation_none, rocblas_operation_none, n, mm, k, &one,
                                         reinterpret_cast<const float*>(v.qs), n, x, k, &zero, y, n);
  return s == rocblas_status_success ? 0 : static_cast<int>(s);
}

int f32w_blas_create(void** handle) {
  rocblas_handle h = nullptr;
  const rocblas_status s = rocblas_create_handle(&h);
  if (s != rocblas_status_success) return static_cast<int>(s);
  // host-side alpha/beta, default (non-atomic, deterministic) kernels
  rocblas_set_pointer_mode(h, rocblas_pointer_mode_host);
  rocblas_set_atomics_mode(h, rocblas_atomics_not_allowed);
  *handle = h;
  return 0;
}

void f32w_blas_destroy(void* handle) {
  if (handle) rocblas_destroy_handle(static_cast<rocblas_handle>(handle));
}

}  // namespace qi
