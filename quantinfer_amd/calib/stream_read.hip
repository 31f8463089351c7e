// Measurement aid, not part of the product library: plain streaming reads of
// a device buffer, the ceiling a kernel that reads every byte once can reach
// at a given size. bench.py --workload calib times them back to back over
// resident buffers exactly as it times the GEMV.
//
// pattern 0: grid-stride; `param` workgroups of 256 threads, each thread
//            keeps 8 x 16-byte loads in flight (a workgroup reads 4 KB per
//            load instruction, consecutive workgroups adjacent 4 KB blocks).
// pattern 1: one contiguous chunk of `param` bytes per workgroup (a GEMV
//            weight tile's shape), 8 x 16-byte loads in flight per thread.
// Loads are non-temporal, like the GEMV's weight loads; the sum is stored
// only under a condition the zero-filled buffers never meet, which keeps the
// loads.
#include <hip/hip_runtime.h>

#include <cstdint>

namespace {

typedef float v4 __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(256) void grid_stride_read(const v4* __restrict__ p, uint64_t n4, float* sink) {
  const uint64_t stride = static_cast<uint64_t>(gridDim.x) * 256;
  uint64_t i = static_cast<uint64_t>(blockIdx.x) * 256 + threadIdx.x;
  v4 acc = {0, 0, 0, 0};
  for (; i + 7 * stride < n4; i += 8 * stride) {
    v4 r[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) r[j] = __builtin_nontemporal_load(p + i + j * stride);
#pragma unroll
    for (int j = 0; j < 8; ++j) acc += r[j];
  }
  for (; i < n4; i += stride) acc += __builtin_nontemporal_load(p + i);
  const float s = acc.x + acc.y + acc.z + acc.w;
  if (s == 1234.5f) sink[blockIdx.x & 1023] = s;
}

__global__ __launch_bounds__(256) void chunk_read(const v4* __restrict__ p, uint64_t n4, uint64_t chunk4,
                                                  float* sink) {
  const uint64_t b = static_cast<uint64_t>(blockIdx.x) * chunk4;
  const uint64_t e = b + chunk4 < n4 ? b + chunk4 : n4;
  v4 acc = {0, 0, 0, 0};
  uint64_t i = b + threadIdx.x;
  for (; i + 7 * 256 < e; i += 8 * 256) {
    v4 r[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) r[j] = __builtin_nontemporal_load(p + i + j * 256);
#pragma unroll
    for (int j = 0; j < 8; ++j) acc += r[j];
  }
  for (; i < e; i += 256) acc += __builtin_nontemporal_load(p + i);
  const float s = acc.x + acc.y + acc.z + acc.w;
  if (s == 1234.5f) sink[blockIdx.x & 1023] = s;
}

}  // namespace

// Enqueue one read of `bytes` (a multiple of 16) at `p` on `stream`; `sink`
// is a device buffer of at least 4 KB. Returns a hipError_t value.
extern "C" int qi_calib_stream_read(const void* p, uint64_t bytes, int32_t pattern, uint64_t param, float* sink,
                                    void* stream) {
  if (p == nullptr || sink == nullptr || bytes == 0 || bytes % 16 != 0 || param == 0)
    return static_cast<int>(hipErrorInvalidValue);
  hipStream_t st = static_cast<hipStream_t>(stream);
  const uint64_t n4 = bytes / 16;
  if (pattern == 0) {
    if (param > 65535) return static_cast<int>(hipErrorInvalidValue);
    hipLaunchKernelGGL(grid_stride_read, dim3(static_cast<uint32_t>(param)), dim3(256), 0, st,
                       static_cast<const v4*>(p), n4, sink);
  } else if (pattern == 1) {
    if (param % 16 != 0) return static_cast<int>(hipErrorInvalidValue);
    const uint64_t chunk4 = param / 16;
    const uint64_t groups = (n4 + chunk4 - 1) / chunk4;
    if (groups > 0x7fffffffull) return static_cast<int>(hipErrorInvalidValue);
    hipLaunchKernelGGL(chunk_read, dim3(static_cast<uint32_t>(groups)), dim3(256), 0, st,
                       static_cast<const v4*>(p), n4, chunk4, sink);
  } else {
    return static_cast<int>(hipErrorInvalidValue);
  }
  return static_cast<int>(hipGetLastError());
}
