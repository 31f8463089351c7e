// Kernel launchers shared between the ABI layer and the kernel translation units.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "qi_image.h"

namespace qi {

// Planar decode GEMV (Q8_0/Q4_0 output rows, K a multiple of 32 but not of
// 256), up to 16 rows per launch.
struct GemvArgs {
  View w;
  const float* x;  // [m, k] device
  float* y;        // [m, n] device
  int m;           // activation rows in this launch (<= compile-time tile)
};
bool gemv_supported(int32_t qtype, int32_t layout, uint64_t k);
hipError_t launch_gemv(int32_t qtype, bool wide, int mt, const GemvArgs& a, hipStream_t st);

// Matrix-core decode GEMV (int8 digits of the activations x raw weight codes).
// Activation source of a one-row GEMV. The decoder fuses the element-wise
// step before the down projection into the GEMV's activation prep:
//   kXPlain  x
//   kXNorm   RMSNorm in front of a projection (backends/cpu/src/backend.rs:172-190):
//            x = v * nw[k] with v = hres[k], and the outputs are scaled by
//            1/sqrt(mean(v^2) + eps) at the end (the norm's scalar moves past
//            the dot product)
enum XSource : int { kXPlain = 0, kXNorm = 3 };

struct GemvMfmaArgs {
  View w;
  const float* x;  // [m, k] device, 16-byte aligned rows
  float* y;        // [m, n]
  int m;           // rows in this launch: 1 (2-16 rows: launch_gemv_rows)
  uint32_t chunk_units = 0;  // set by the launcher: K units whose activation digits fit LDS
  int xs = kXPlain;  // one row, f16-scale images only
  // kXNorm: the residual row, the norm weight and epsilon
  const float* hres = nullptr;
  const float* nw = nullptr;
  float eps = 0.0f;
  // one row: y[n] = radd[n] + (x . w_n), the residual add after a projection
  // (runtime/src/linear.rs:129-142); y may be radd itself (each output is read
  // and written by the one lane that computes it)
  const float* radd = nullptr;
  // one row, N a multiple of 16: every 16-output tile holds 8 gate rows then
  // the 8 up rows of the same outputs, and y[8 t + c] = g / (1 + exp(-g)) * u
  // (backends/cpu/src/backend.rs:224-237), N / 2 outputs
  bool silu_pairs = false;
};
bool gemv_mfma_supported(int32_t qtype, int32_t layout, uint64_t k);
int gemv_mfma_split(uint64_t k, uint64_t n);
// y[i] = sum over s of part[s * stride + i] (i < count = m * n) in split order;
// a non-finite sum is recomputed in the reference's order
hipError_t launch_splitk_sum(const Image& im, const View& v, const float* part, uint32_t splits,
                             uint64_t count, uint64_t stride, float* y, const float* x, hipStream_t st);
hipError_t launch_gemv_mfma(int32_t qtype, bool wide, int split, const GemvMfmaArgs& a, hipStream_t st);

// Matrix-core decode GEMV of 2-8 rows with dense operands and int8
// activation digits (qi_gemv_rows.hip): one kernel, K parts over the grid
// (gemv_rows_splits, by shape and row count) only for shapes with few tiles;
// with ksplit > 1 the partial sums [ksplit][m][n] go to `part` and
// launch_splitk_sum adds them. Shapes: those of gemv_mfma_supported (every
// format, output rows, K a multiple of 256).
uint32_t gemv_rows_splits(uint64_t k, uint64_t n, uint32_t m);
hipError_t launch_gemv_rows(int32_t qtype, bool wide, const View& w, const float* x, int m, float* y, float* part,
                            uint32_t ksplit, hipStream_t st);

// Decode GEMV of 9-16 rows on the f16 matrix cores with split-half
// activations (qi_gemv_half.hip): launch_gemv_half_records converts the
// activations once per call into `records` (gemv_half_records_bytes bytes;
// their layout depends on the format: pass the GEMV's qtype),
// which the GEMV workgroups copy; one GEMV kernel, K parts over the grid
// (gemv_half_splits) only for shapes with few tiles; with ksplit > 1 the
// partial sums [ksplit][m][n] go to `part` and launch_splitk_sum adds them.
// Shapes: those of gemv_mfma_supported.
uint32_t gemv_half_splits(uint64_t k, uint64_t n, uint32_t m);
uint64_t gemv_half_records_bytes(uint64_t k);
hipError_t launch_gemv_half_records(int32_t qtype, const float* x, uint64_t k, int m, uint8_t* records,
                                    hipStream_t st);
hipError_t launch_gemv_half(int32_t qtype, bool wide, const View& w, const float* x, int m, float* y, float* part,
                            uint32_t ksplit, const uint8_t* records, hipStream_t st);

// F32-mode GEMM of output rows (qi_gemm_split.hip): split-half activations
// against exact f16 weight codes (Q4_K / Q5_K, sub-block scales folded in) or
// weights as two f16 halves (Q8_0 / Q4_0 with f16 scales, Q6_K), within the
// f32 GEMV's bars. launch_gemm_split converts the activations into
// `records` (gemm_split_records_bytes) and runs the GEMM; with splits > 1
// (gemm_split_splits) the partial sums [splits][m][n] go to `part` and are
// added in order.
bool gemm_split_supported(const Image& im);
uint64_t gemm_split_records_bytes(uint64_t m, uint64_t k);
uint32_t gemm_split_splits(const Image& im, uint64_t m);
hipError_t launch_gemm_split(const Image& im, const View& v, const float* x, uint64_t m, float* y, float* part,
                             uint32_t splits, uint8_t* records, hipStream_t st);

// Row-major (blocks along N) GEMV of up to gemv_rm_rows activation rows (4
// for planar images, 2 for tiled ones), f32 accumulation, K split over the
// grid; `part` holds splits * m * n floats when splits > 1.
bool gemv_rm_supported(const Image& im);
uint32_t gemv_rm_rows(const Image& im);
uint32_t gemv_rm_splits(const Image& im, uint32_t m);
hipError_t launch_gemv_rm(const Image& im, const View& v, const float* x, uint32_t m, float* y, float* part,
                          uint32_t splits, hipStream_t st);
// Row-major GEMM on a tiled image (K a multiple of 4), any row count: the
// weights dequantized into LDS for f32 matrix-core products, K split into
// `parts` (partial sums in `part`, parts * m * n floats, when parts > 1),
// non-finite outputs recomputed in the reference's order.
bool rm_gemm_supported(const Image& im);
uint32_t rm_gemm_tile_rows(uint64_t m);
uint32_t rm_gemm_parts(const Image& im, uint64_t m, uint64_t max_part_floats);
hipError_t launch_rm_gemm(const Image& im, const View& v, const float* x, uint64_t m, float* y, float* part,
                          uint32_t parts, hipStream_t st);

// F32 weights (row-major [K, N] f32, N a multiple of 4): the streaming GEMV
// for up to 8 rows per launch (K split over the grid; `part` holds splits * m * n floats
// when splits > 1), and the matrix-core GEMM for more rows (K a multiple of
// 4; no workspace).
// rows above which F32 weights take the GEMM: at the LM head shape
// (4096 x 151936) 9-16 rows take 0.55-0.64 ms on the 32-row GEMM tiles
// against 0.97-1.11 ms for two GEMV launches; 8 rows 0.56 ms on one GEMV
constexpr uint64_t kF32GemvMaxRows = 8;
bool f32w_gemv_supported(const Image& im);
uint32_t f32w_splits(const Image& im);
hipError_t launch_f32w_gemv(const Image& im, const View& v, const float* x, uint32_t m, float* y, float* part,
                            uint32_t splits, hipStream_t st);
bool f32w_gemm_supported(const Image& im);
hipError_t launch_f32w_gemm(const Image& im, const View& v, const float* x, uint64_t m, float* y, hipStream_t st);

// Exact-order matmul: bit-identical to CpuScalar (any M, either layout).
hipError_t launch_exact(const Image& im, const View& w, const float* x, uint64_t m, float* y,
                        hipStream_t st);
// Bit-exact dequantization in block order.
hipError_t launch_dequant(const Image& im, const View& w, float* out, hipStream_t st);

struct GemmArgs {
  View w;
  const float* x;  // [m, k] f32 device
  float* y;        // [m, n]
  uint64_t m;
  _Float16* xh;    // [m_pad, k] f16 workspace (the activations rounded once)
  uint64_t m_pad;  // gemm_padded_rows(m)
  // split-K (gemm_splits > 1): [splits][m_pad][n] f32 partial products,
  // summed in split order into y
  float* part = nullptr;
  uint32_t splits = 1;
  // non-null (splits == 1 only): the epilogue pairs output 16 T + c with
  // 16 T + 8 + c (c < 8) and writes SiLU(first) * second to act[m][8 T + c]
  // instead of y (a gate|up image interleaved in groups of 8)
  float* act = nullptr;
};
bool gemm_supported(int32_t qtype, int32_t layout, uint64_t k, uint64_t n);
uint64_t gemm_padded_rows(uint64_t m);
// K splits of a GEMM launch (1: no split): enough workgroups to fill the CUs
// once when the row and column blocks alone do not.
uint32_t gemm_splits(const Image& im, uint64_t m);
// The GEMM kernel this image runs on has the SiLU-pairs epilogue.
bool gemm_silu_supported(const Image& im);
hipError_t launch_gemm(const Image& im, const GemmArgs& a, hipStream_t st);

}  // namespace qi
