// Exact-order kernels: bit-identical to the reference CPU arithmetic.
//
// * dequant: every element computed with the reference's f32 operation
//   sequence (quant/src/schemes/*.rs dequantize_*), written in block order.
// * exact matmul: one thread per output keeps the CpuScalar accumulation
//   acc = acc + x[k] * w(k) in f32, k ascending, no FMA
//   (backends/cpu/src/matmul.rs:146-157, 319-330 for output rows; :25-31 for
//   row major). The whole file is compiled with -ffp-contract=off, so no
//   multiply-add below is fused.
// * F32 weights (row-major [K, N], the reference's `matmul`, matmul.rs:92-117)
//   use the same per-output sequential order; one thread per column streams
//   coalesced rows of W, up to 16 activation rows per thread.
#include "qi_device.h"
#include "qi_internal.h"

namespace qi {

// ------------------------------------------------------------------ dequant

template <int QT, bool WIDE>
__global__ __launch_bounds__(256) void dequant_kernel(View w, uint64_t elements, uint64_t nb,
                                                      float* out) {
  const uint64_t e0 = (static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x) * 8;
  if (e0 >= elements) return;
  constexpr uint32_t bs = (QT == kQ8_0 || QT == kQ4_0) ? 32 : 256;
  const uint64_t blk = e0 / bs;
  const uint32_t l0 = static_cast<uint32_t>(e0 % bs);  // 8 | bs, so all 8 share the block
  // block order: output n owns blocks [n*nb, n*nb+nb) (row major: k owns them
  // in a tiled image, nb = all blocks in a planar one)
  const BlockLoc L = locate<QT>(w, blk / nb, blk % nb);
  float v[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) v[j] = Exact<QT, WIDE>::value(w, L, l0 + j);
  float4* o = reinterpret_cast<float4*>(out + e0);
  o[0] = make_float4(v[0], v[1], v[2], v[3]);
  o[1] = make_float4(v[4], v[5], v[6], v[7]);
}

__global__ __launch_bounds__(256) void copy_f32_kernel(const float* in, uint64_t n, float* out) {
  const uint64_t i = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < n) out[i] = in[i];
}

// ------------------------------------------------------- exact: output rows

template <int QT, bool WIDE>
__global__ __launch_bounds__(256) void exact_output_rows_kernel(View w, const float* x, uint64_t m,
                                                                float* y) {
  const uint64_t n = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const uint64_t r = blockIdx.y;
  if (n >= w.n || r >= m) return;
  y[r * w.n + n] = exact_output_row<QT, WIDE>(w, x + r * w.k, n);
}

// --------------------------------------------------------- exact: row major

template <int QT, bool WIDE>
__global__ __launch_bounds__(256) void exact_row_major_kernel(View w, const float* x, uint64_t m,
                                                              float* y) {
  const uint64_t n = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const uint64_t r = blockIdx.y;
  if (n >= w.n || r >= m) return;
  y[r * w.n + n] = exact_row_major_col<QT, WIDE>(w, x + r * w.k, n);
}

// ------------------------------------------------------------------ F32 W

template <int MT>
__global__ __launch_bounds__(256) void f32_rows_kernel(const float* W, uint64_t k, uint64_t nn,
                                                       const float* x, uint64_t m0, uint64_t mcount,
                                                       float* y) {
  const uint64_t n = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (n >= nn) return;
  float acc[MT];
#pragma unroll
  for (int j = 0; j < MT; ++j) acc[j] = 0.0f;
  for (uint64_t i = 0; i < k; ++i) {
    const float wv = W[i * nn + n];
#pragma unroll
    for (int j = 0; j < MT; ++j) {
      const uint64_t r = m0 + (static_cast<uint64_t>(j) < mcount ? j : 0);
      acc[j] += x[r * k + i] * wv;
    }
  }
#pragma unroll
  for (int j = 0; j < MT; ++j)
    if (static_cast<uint64_t>(j) < mcount) y[(m0 + j) * nn + n] = acc[j];
}

// ---------------------------------------------------------------- launchers

namespace {

template <int QT, bool WIDE>
hipError_t dequant_one(const View& w, uint64_t elements, uint64_t nb, float* out, hipStream_t st) {
  const uint64_t threads = (elements + 7) / 8;
  const uint64_t grid = (threads + 255) / 256;
  hipLaunchKernelGGL((dequant_kernel<QT, WIDE>), dim3(static_cast<uint32_t>(grid)), dim3(256), 0, st,
                     w, elements, nb, out);
  return hipGetLastError();
}

template <int QT, bool WIDE>
hipError_t exact_one(const Image& im, const View& w, const float* x, uint64_t m, float* y,
                     hipStream_t st) {
  const dim3 grid(static_cast<uint32_t>((im.n + 255) / 256), static_cast<uint32_t>(m));
  if (im.layout == kOutputRows) {
    hipLaunchKernelGGL((exact_output_rows_kernel<QT, WIDE>), grid, dim3(256), 0, st, w, x, m, y);
  } else {
    hipLaunchKernelGGL((exact_row_major_kernel<QT, WIDE>), grid, dim3(256), 0, st, w, x, m, y);
  }
  return hipGetLastError();
}

template <int QT>
hipError_t exact_wide(const Image& im, const View& w, const float* x, uint64_t m, float* y,
                      hipStream_t st) {
  return im.wide ? exact_one<QT, true>(im, w, x, m, y, st) : exact_one<QT, false>(im, w, x, m, y, st);
}

template <int QT>
hipError_t dequant_wide(const Image& im, const View& w, float* out, hipStream_t st) {
  const uint64_t elements = im.k * im.n;
  const uint64_t nb = im.layout == kOutputRows ? im.k / block_elems(im.qtype)
                     : im.tiled                 ? im.n / block_elems(im.qtype)
                                                : im.nblocks;
  return im.wide ? dequant_one<QT, true>(w, elements, nb, out, st)
                 : dequant_one<QT, false>(w, elements, nb, out, st);
}

}  // namespace

hipError_t launch_dequant(const Image& im, const View& w, float* out, hipStream_t st) {
  switch (im.qtype) {
    case kF32: {
      const uint64_t n = im.k * im.n;
      hipLaunchKernelGGL(copy_f32_kernel, dim3(static_cast<uint32_t>((n + 255) / 256)), dim3(256), 0,
                         st, reinterpret_cast<const float*>(w.qs), n, out);
      return hipGetLastError();
    }
    case kQ8_0: return dequant_wide<kQ8_0>(im, w, out, st);
    case kQ4_0: return dequant_wide<kQ4_0>(im, w, out, st);
    case kQ4_K: return dequant_wide<kQ4_K>(im, w, out, st);
    case kQ5_K: return dequant_wide<kQ5_K>(im, w, out, st);
    case kQ6_K: return dequant_wide<kQ6_K>(im, w, out, st);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_exact(const Image& im, const View& w, const float* x, uint64_t m, float* y,
                        hipStream_t st) {
  switch (im.qtype) {
    case kF32: {
      const dim3 grid(static_cast<uint32_t>((im.n + 255) / 256));
      const float* W = reinterpret_cast<const float*>(w.qs);
      for (uint64_t m0 = 0; m0 < m; m0 += 16) {
        const uint64_t cnt = m - m0 < 16 ? m - m0 : 16;
        if (cnt == 1) {
          hipLaunchKernelGGL((f32_rows_kernel<1>), grid, dim3(256), 0, st, W, im.k, im.n, x, m0, cnt, y);
        } else if (cnt <= 4) {
          hipLaunchKernelGGL((f32_rows_kernel<4>), grid, dim3(256), 0, st, W, im.k, im.n, x, m0, cnt, y);
        } else {
          hipLaunchKernelGGL((f32_rows_kernel<16>), grid, dim3(256), 0, st, W, im.k, im.n, x, m0, cnt, y);
        }
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
      }
      return hipSuccess;
    }
    case kQ8_0: return exact_wide<kQ8_0>(im, w, x, m, y, st);
    case kQ4_0: return exact_wide<kQ4_0>(im, w, x, m, y, st);
    case kQ4_K: return exact_wide<kQ4_K>(im, w, x, m, y, st);
    case kQ5_K: return exact_wide<kQ5_K>(im, w, x, m, y, st);
    case kQ6_K: return exact_wide<kQ6_K>(im, w, x, m, y, st);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace qi
