// Decode GEMV of 2-8 activation rows on the int8 matrix cores
// (v_mfma_i32_16x16x32_i8), output-rows layout, K a multiple of 256; one
// kernel per call (K parts over the grid only for shapes with few tiles);
// 9-16 rows take the split-half kernel (qi_gemv_half.hip).
//
// Arithmetic: as the one-row kernel (qi_gemv_mfma.hip). Each activation row
// is cut into windows of 32 elements; an element becomes the 30-bit integer
// F = rint(x * 2^s) (2^s per (row, window) from the window's max |x|), held
// as four signed 8-bit digits; weight codes enter the matrix cores as bytes,
// centred as there (Q4_0 as 16 (q - 8), Q6_K as 4 (q - 32); Q4_K and Q5_K as
// q - z with a zero point z per window, by a second matrix instruction with -z
// in every B byte), so every digit sum is exact in int32, and per (row,
// window, output)
//   sum_k x_k w_k = a * 2^-s * (C0 + C1*2^8 + C2*2^16 + C3*2^24) - b' * sum_k x_k
// with the format's sub-block scale a and the offset left, b' = b - z a
// (w = a*q - b). The offset terms of all windows go through f32 matrix
// instructions (v_mfma_f32_16x16x4_f32: window sums x per-output offsets).
// Q6_K's windows hold two 16-element sub-blocks of their own scales, whose
// digit sums two instructions per window keep apart (consume_q6).
//
// Dense operands. One 16x16x32 instruction covers one window for four
// activation rows and the tile's 16 outputs: A row 4r + d holds digit d of
// row 4q + r (row group q), lane group g (lanes 16g..16g+15) supplying
// elements 8g..8g+7 of the window (A[i][k] at lane i + 16(k/8)); B holds the
// window's codes (B[k][j] at lane j + 16(k/8)); lane (j, g) receives the four
// digit sums of row 4q + g for output j (C[i][j] at lane j + 16(i/4)). Every
// A row is live, against one in four in the one-row kernel's block-diagonal
// form. The weight record gives lane group g two whole windows of its
// output (elements 64g..64g+63 of a unit); the B operand needs slice g of
// every window, so the code words are transposed across the four lane groups
// with gfx950's v_permlane32_swap / v_permlane16_swap (four instructions per
// 4 x 4 dwords), and the window scales, decoded by their owning lane group,
// are broadcast to the others the same way.
//
// Work split: a workgroup is 16 wavefronts, 4 tiles of 16 outputs x 4 K
// slices (or, for shapes of up to one tile per CU, one tile x 16 K slices,
// so that no K part leaves the workgroup). The workgroup builds the digits of its K range for all rows into
// LDS (chunk by chunk when they do not fit), each wavefront streams its
// tile's units of its slice, and the slices are summed in order through LDS.
// Weight loads are issued before the activation prep so that the HBM latency
// overlaps it; the activation loads go first (vector loads complete in order).
// No state is shared between workgroups. Row-group indices past M hold zero
// digits and are never stored.
#include <type_traits>

#include "qi_device.h"
#include "qi_internal.h"
#include "qi_unit.h"

namespace qi {

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));

constexpr int kRowsThreads = 1024;   // 16 wavefronts
constexpr int kRowsWaves = 16;      // wavefronts per workgroup: TL tiles x (16 / TL) K slices
constexpr uint32_t kBlock = 512;     // LDS bytes per (row group, window) digit block
constexpr uint32_t kRowsCUs = 256;   // compute units of an MI355X (gfx950)

// LDS bytes of the activation records of `cu` units for `mg` row groups:
// digits [q][window] blocks of kBlock bytes (lane L's 8 bytes at 8L), then the
// activation scales 2^-s [row][window] and the window sums [row][window] as f32.
constexpr uint32_t rows_lds(int mg, uint32_t cu) {
  return static_cast<uint32_t>(mg) * 8 * cu * kBlock + 2 * (4 * static_cast<uint32_t>(mg) * 8 * cu * 4);
}
constexpr uint32_t kRowsLdsCap = 160 * 1024;
// units of a chunk: the LDS budget (32 / 16 / 8 for 1 / 2 / 4 row groups)
constexpr uint32_t rows_chunk_cap(int mg) { return 32 / static_cast<uint32_t>(mg); }
static_assert(rows_lds(1, 32) <= kRowsLdsCap && rows_lds(2, 16) <= kRowsLdsCap &&
              rows_lds(4, 8) <= kRowsLdsCap, "records fit LDS");

// 4 x 4 dword transpose across the lane groups: in lane group g, r[s] holds
// P[g][s] on entry and P[s][g] on return.
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

// All-gather across the lane groups: v is V[g] in lane group g; out[g'] = V[g'].
// (The swap results are copied to scalars before the bit casts: a bit cast
// of a vector element reads element 0 with this compiler.)
__device__ __forceinline__ void gather4(float v, float out[4]) {
  const uint32_t u = __builtin_bit_cast(uint32_t, v);
  const auto a = __builtin_amdgcn_permlane16_swap(u, u, false, false);       // [V0 V0 V2 V2], [V1 V1 V3 V3]
  const auto b = __builtin_amdgcn_permlane32_swap(a[0], a[0], false, false);  // [V0]x4, [V2]x4
  const auto c = __builtin_amdgcn_permlane32_swap(a[1], a[1], false, false);  // [V1]x4, [V3]x4
  const uint32_t r[4] = {b[0], c[0], b[1], c[1]};
#pragma unroll
  for (int i = 0; i < 4; ++i) out[i] = __builtin_bit_cast(float, r[i]);
}

__device__ __forceinline__ long pack2(uint32_t lo, uint32_t hi) {
  return static_cast<long>((static_cast<uint64_t>(hi) << 32) | lo);
}

// Per-format dense B operands of one unit. prepare() moves the code words
// across the lane groups; b(t, w) is then the 8 codes of slice g (elements
// 8g..8g+7) of window w (w = 2g' + h: window h of lane group g').
template <int QT>
struct Dense;

template <>
struct Dense<kQ8_0> {
  // lane group g: block 2g in q[0], q[1], block 2g+1 in q[2], q[3]; slice s
  // of a block = its dwords 2s, 2s+1
  struct T {
    uint32_t lo[2][4], hi[2][4];
  };
  template <bool C>
  __device__ static void prepare(const Unit<kQ8_0>::Raw& r, uint32_t, T& t) {
#pragma unroll
    for (int b = 0; b < 2; ++b) {
      t.lo[b][0] = r.q[2 * b].x; t.lo[b][1] = r.q[2 * b].z; t.lo[b][2] = r.q[2 * b + 1].x; t.lo[b][3] = r.q[2 * b + 1].z;
      t.hi[b][0] = r.q[2 * b].y; t.hi[b][1] = r.q[2 * b].w; t.hi[b][2] = r.q[2 * b + 1].y; t.hi[b][3] = r.q[2 * b + 1].w;
      xpose4(t.lo[b]);
      xpose4(t.hi[b]);
    }
  }
  __device__ static long b(const T& t, int w) { return pack2(t.lo[w & 1][w >> 1], t.hi[w & 1][w >> 1]); }
};

template <>
struct Dense<kQ4_0> {
  // lane group g: block 2g + b in q[b] (byte i = element i | element i+16 << 4).
  // Slice s as one word of 8 nibbles (byte k = element 8s+k | element 8s+4+k << 4)
  // before the transpose, so a lane group sends four words per block. The
  // codes go out centred, 16 (q - 8) as signed bytes (Unit<kQ4_0>::centred_codes,
  // qi_unit.h): bit 3 of every nibble flipped, each nibble moved to the high
  // half of its byte.
  static constexpr uint32_t kM = 0x0F0F0F0Fu;
  struct T {
    uint32_t w[2][4];
  };
  template <bool C>
  __device__ static void prepare(const Unit<kQ4_0>::Raw& r, uint32_t, T& t) {
#pragma unroll
    for (int b = 0; b < 2; ++b) {
      const uint4 q = r.q[b];
      t.w[b][0] = ((q.x & kM) | ((q.y << 4) & ~kM)) ^ 0x88888888u;
      t.w[b][1] = ((q.z & kM) | ((q.w << 4) & ~kM)) ^ 0x88888888u;
      t.w[b][2] = (((q.x >> 4) & kM) | (q.y & ~kM)) ^ 0x88888888u;
      t.w[b][3] = (((q.z >> 4) & kM) | (q.w & ~kM)) ^ 0x88888888u;
      xpose4(t.w[b]);
    }
  }
  __device__ static long b(const T& t, int w) {
    const uint32_t v = t.w[w & 1][w >> 1];
    return pack2((v << 4) & ~kM, v & ~kM);
  }
};

// Q4_K / Q5_K: lane group g holds code bytes [32g, 32g+32) of the
// super-block, bytes 8s..8s+7 (dwords 2s, 2s+1) carrying slice s of window
// 2g (low nibbles) and of window 2g+1 (high nibbles); Q5_K adds bit w of
// qh byte e as bit 4 of element e of window w. b() gives the codes as they
// are, bc() centred on the middle of their range as the one-row kernel takes
// them (qi_unit.h): Q4_K 16 (q - 8) (nibble bit 3 flipped, the nibble in the
// byte's high half; prepare() flips the bits when C), Q5_K 8 (q - 16).
template <bool FIVE>
struct DenseQ45K {
  static constexpr uint32_t kM = 0x0F0F0F0Fu;
  struct T {
    uint32_t lo[4], hi[4];
    uint32_t hl, hh;  // Q5_K: qh bytes 8g..8g+7 of this output
  };
  template <bool C, typename Raw>
  __device__ static void prepare(const Raw& r, uint32_t, T& t) {
    t.lo[0] = r.q[0].x; t.lo[1] = r.q[0].z; t.lo[2] = r.q[1].x; t.lo[3] = r.q[1].z;
    t.hi[0] = r.q[0].y; t.hi[1] = r.q[0].w; t.hi[2] = r.q[1].y; t.hi[3] = r.q[1].w;
    if constexpr (C && !FIVE) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        t.lo[i] ^= 0x88888888u;
        t.hi[i] ^= 0x88888888u;
      }
    }
    xpose4(t.lo);
    xpose4(t.hi);
    if constexpr (FIVE) {
      t.hl = r.hl;
      t.hh = r.hh;
    } else {
      t.hl = t.hh = 0;
    }
  }
  __device__ static long b(const T& t, int w) {
    const int gp = w >> 1, h = w & 1;
    uint32_t a = h ? (t.lo[gp] >> 4) & kM : t.lo[gp] & kM;
    uint32_t c = h ? (t.hi[gp] >> 4) & kM : t.hi[gp] & kM;
    if constexpr (FIVE) {
      // bit w of each qh byte to bit 4
      a |= (w <= 4 ? t.hl << (4 - w) : t.hl >> (w - 4)) & 0x10101010u;
      c |= (w <= 4 ? t.hh << (4 - w) : t.hh >> (w - 4)) & 0x10101010u;
    }
    return pack2(a, c);
  }
  __device__ static long bc(const T& t, int w) {
    const int gp = w >> 1, h = w & 1;
    if constexpr (FIVE) {
      // nibble to bits 3-6, bit w of the qh byte to bit 7, bit 7 flipped
      const uint32_t a = ((h ? t.lo[gp] >> 1 : t.lo[gp] << 3) & 0x78787878u) ^
                         ((t.hl << (7 - w)) & 0x80808080u) ^ 0x80808080u;
      const uint32_t c = ((h ? t.hi[gp] >> 1 : t.hi[gp] << 3) & 0x78787878u) ^
                         ((t.hh << (7 - w)) & 0x80808080u) ^ 0x80808080u;
      return pack2(a, c);
    } else {
      const uint32_t a = (h ? t.lo[gp] : t.lo[gp] << 4) & ~kM;
      const uint32_t c = (h ? t.hi[gp] : t.hi[gp] << 4) & ~kM;
      return pack2(a, c);
    }
  }
};
template <>
struct Dense<kQ4_K> : DenseQ45K<false> {};
template <>
struct Dense<kQ5_K> : DenseQ45K<true> {};

// Q6_K: lane group g' = 2ip + c holds ql bytes [64ip + 32c, +32) of the
// super-block, window w = 4ip + 2hf + c (elements 32w..32w+31) being the low
// (hf = 0) or high (hf = 1) nibbles of them, so the ql words cross the lane
// groups as Q4_K's do. Slice g of window w takes its two high bits from bits
// 2c + 4hf of qh bytes 32ip + 8g..8g+7, which each lane group loads for itself
// (h[2ip], h[2ip + 1]; RowsUnit<kQ6_K>). The codes go out as the one-row
// kernel takes them (Unit<kQ6_K>::centred_codes): 4 (q - 32) as signed bytes.
template <>
struct Dense<kQ6_K> {
  struct T {
    uint32_t lo[4], hi[4];
    uint32_t h[4];
  };
  template <bool C, typename Raw>
  __device__ static void prepare(const Raw& r, uint32_t, T& t) {
    t.lo[0] = r.q[0].x; t.lo[1] = r.q[0].z; t.lo[2] = r.q[1].x; t.lo[3] = r.q[1].z;
    t.hi[0] = r.q[0].y; t.hi[1] = r.q[0].w; t.hi[2] = r.q[1].y; t.hi[3] = r.q[1].w;
    xpose4(t.lo);
    xpose4(t.hi);
#pragma unroll
    for (int i = 0; i < 4; ++i) t.h[i] = r.h[i];
  }
  __device__ static long bc(const T& t, int w) {
    const int ip = w >> 2, hf = (w >> 1) & 1, c = w & 1, gp = 2 * ip + c;
    const int up = 6 - 2 * c - 4 * hf;  // qh bits 2c + 4hf to bits 6-7
    const uint32_t a = q6_centred(hf ? t.lo[gp] >> 2 : t.lo[gp] << 2, t.h[2 * ip] << up);
    const uint32_t b = q6_centred(hf ? t.hi[gp] >> 2 : t.hi[gp] << 2, t.h[2 * ip + 1] << up);
    return pack2(a, b);
  }
};

struct RowsArgs {
  View w;
  const float* x;  // [m, k]
  float* y;        // [m, n]
  int m;
  uint32_t chunk_units;  // units per LDS chunk
  uint32_t part_units;   // units per K part (grid.y)
  float* part;           // [grid.y][m][n] when grid.y > 1
};

// Activation prep, in place. Item (q, W, s, r) is slice s (elements 8s..8s+7)
// of window W of row 4q + r; its 32 bytes at 32 * item of the digit area
// (block (q, W) = items 16 (q cw + W) ..) first receive the item's 8 floats by
// global-to-LDS copies, then its 4 digit words (digit d at + 8 d: lane
// 16 s + 4 r + d of the A operand). A wavefront's items are 2 KB of LDS in a
// row, so neither the copies nor the conversion conflict on banks.

// Copy the chunk's activations (windows < cwin of rows < M) into the items;
// wave-uniform LDS destination, one 1 KB copy (two blocks) per instruction.
__device__ __forceinline__ void stage_x(const float* x, uint32_t K, uint32_t k0, int M, int mg, uint32_t cw,
                                        uint32_t cwin, uint8_t* dig, uint32_t wave, uint32_t lane) {
  const uint32_t copies = static_cast<uint32_t>(mg) * cw / 2;
  const uint32_t o = 16 * (lane & 31), s = o >> 7, r = (o >> 5) & 3, h = (o >> 4) & 1;
  for (uint32_t j = wave; j < copies; j += kRowsThreads / 64) {
    const uint32_t b = 2 * j + (lane >> 5), q = b / cw, W = b % cw;
    const uint32_t m = 4 * q + r;
    if (static_cast<int>(m) < M && W < cwin)
      __builtin_amdgcn_global_load_lds(x + static_cast<uint64_t>(m) * K + k0 + 32 * W + 8 * s + 4 * h,
                                       (__attribute__((address_space(3))) void*)(dig + 1024 * j), 16, 0, 0);
  }
}

// Convert item t (activations v0, v1; zeros for rows >= M) of row group q,
// window W: window max and sum over its four slices (lanes 4, 8 and 12
// apart), the power of two 2^-s, the digits, at 32 * t of `dig`; slice 0
// stores the window's scale and sum. Every lane of the wavefront takes part
// (the lane moves); only `valid` items store.
__device__ __forceinline__ void prep_convert(float4 v0, float4 v1, uint32_t t, uint32_t q, uint32_t W, uint32_t cw,
                                             bool valid, uint8_t* dig, float* xsc, float* xsum) {
  const uint32_t s = (t >> 2) & 3, m = 4 * q + (t & 3);
  const float xs[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
  float mx = 0.0f, sum = 0.0f;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    mx = fmaxf(mx, fabsf(xs[j]));
    sum += xs[j];
  }
  // the four slices of a window are lanes r, r + 4, r + 8, r + 12 of a row of 16
  mx = fmaxf(mx, dpp_move<kDppRor4>(mx));
  mx = fmaxf(mx, dpp_move<kDppRor8>(mx));
  sum += dpp_move<kDppRor4>(sum);
  sum += dpp_move<kDppRor8>(sum);
  // A NaN or infinite activation makes the window sum non-finite: the scale
  // is then NaN (every output of the row comes out NaN and the epilogue
  // recomputes it in the reference's order) and the digits are zero.
  const bool finite = __builtin_isfinite(sum);
  const int e = finite && mx > 0.0f ? __builtin_amdgcn_frexp_expf(mx) : 0;
  const int sh = 29 - e;  // max|x| * 2^sh < 2^29
  const float inv = !finite ? __builtin_nanf("") : mx > 0.0f ? ldexpf(1.0f, e - 29) : 0.0f;
  if (!valid) return;
  uint32_t dg[8] = {0, 0, 0, 0, 0, 0, 0, 0};  // zero digits for a non-finite window
  if (finite) {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int F = static_cast<int>(rintf(ldexpf(xs[j], sh)));
      // signed base-256 digits: byte i of (F + 0x808080) ^ 0x808080
      dg[j] = (static_cast<uint32_t>(F) + 0x00808080u) ^ 0x00808080u;
    }
  }
  // digit d of the 8 elements: byte d of dg[0..3] (low word), of dg[4..7] (high word)
  uint32_t lo[4], hi[4];
  {
    const uint32_t t0 = __builtin_amdgcn_perm(dg[1], dg[0], 0x05010400u);
    const uint32_t t1 = __builtin_amdgcn_perm(dg[1], dg[0], 0x07030602u);
    const uint32_t t2 = __builtin_amdgcn_perm(dg[3], dg[2], 0x05010400u);
    const uint32_t t3 = __builtin_amdgcn_perm(dg[3], dg[2], 0x07030602u);
    lo[0] = __builtin_amdgcn_perm(t2, t0, 0x05040100u);
    lo[1] = __builtin_amdgcn_perm(t2, t0, 0x07060302u);
    lo[2] = __builtin_amdgcn_perm(t3, t1, 0x05040100u);
    lo[3] = __builtin_amdgcn_perm(t3, t1, 0x07060302u);
  }
  {
    const uint32_t t0 = __builtin_amdgcn_perm(dg[5], dg[4], 0x05010400u);
    const uint32_t t1 = __builtin_amdgcn_perm(dg[5], dg[4], 0x07030602u);
    const uint32_t t2 = __builtin_amdgcn_perm(dg[7], dg[6], 0x05010400u);
    const uint32_t t3 = __builtin_amdgcn_perm(dg[7], dg[6], 0x07030602u);
    hi[0] = __builtin_amdgcn_perm(t2, t0, 0x05040100u);
    hi[1] = __builtin_amdgcn_perm(t2, t0, 0x07060302u);
    hi[2] = __builtin_amdgcn_perm(t3, t1, 0x05040100u);
    hi[3] = __builtin_amdgcn_perm(t3, t1, 0x07060302u);
  }
  uint4* const dst = reinterpret_cast<uint4*>(dig + 32 * t);
  dst[0] = make_uint4(lo[0], hi[0], lo[1], hi[1]);
  dst[1] = make_uint4(lo[2], hi[2], lo[3], hi[3]);
  if (s == 0) {
    xsc[m * cw + W] = inv;
    xsum[m * cw + W] = sum;
  }
}

// Convert item t (row group q, window W) of a chunk in place (its floats
// staged by stage_x).
__device__ __forceinline__ void prep_item(uint32_t t, uint32_t q, uint32_t W, uint32_t cw, uint32_t cwin, int M,
                                          uint8_t* dig, float* xsc, float* xsum) {
  const uint32_t m = 4 * q + (t & 3);
  const bool valid = W < cwin;
  float4 v0 = make_float4(0.0f, 0.0f, 0.0f, 0.0f), v1 = v0;
  if (valid && static_cast<int>(m) < M) {
    const float4* p = reinterpret_cast<const float4*>(dig + 32 * t);
    v0 = p[0];
    v1 = p[1];
  }
  prep_convert(v0, v1, t, q, W, cw, valid, dig, xsc, xsum);
}

// MG row groups (M <= 4 MG), D units of weights in flight per wavefront, TL
// tiles per workgroup (4, or 1 with 16 K slices for shapes of up to one tile
// per CU). ZP (Q4_K / Q5_K): the codes centred on a zero point per window
// (window_zero_point, kRowsZeroPointUnits); otherwise on the middle of their
// range. Given the call's activation records (a.rec; four row groups), the
// workgroups copy them; otherwise each converts its activations itself.
template <int QT, bool WIDE, int MG, int D, int TL, bool ZP>
__global__ __launch_bounds__(kRowsThreads) void gemv_rows_kernel(RowsArgs a) {
  // codes centred on the middle of their range, and their scale
  constexpr bool kFixed = QT == kQ4_0 || QT == kQ6_K || (window_centered<QT>() && !ZP);
  constexpr float kInvScale = kFixed ? 1.0f / static_cast<float>(code_scale<QT>()) : 1.0f;
  constexpr int SL = kRowsWaves / TL;  // K slices per tile
  using U = RowsUnit<QT>;
  constexpr Record R = record_geometry(QT, WIDE);
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  const uint32_t cu = a.chunk_units, cw = 8 * cu;
  uint8_t* const dig = lds;
  float* const xsc = reinterpret_cast<float*>(lds + MG * cw * kBlock);
  float* const xsum = xsc + 4 * MG * cw;

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

  float acc[MG];
#pragma unroll
  for (int q = 0; q < MG; ++q) acc[q] = 0.0f;
  v4f cmin = {0.0f, 0.0f, 0.0f, 0.0f};  // offset terms: element e = row group e
  // the offset MFMA's A rows: row i carries activation row pi(i) = 4 (i % 4) + i / 4,
  // so that C row 4g + e (lane group g, element e) is activation row 4e + g
  const uint32_t arow = lane & 15, mrow = 4 * (arow & 3) + (arow >> 2);

  typename U::Raw ring[D];

  for (uint32_t ku0 = u_lo; ku0 < u_hi; ku0 += cu) {
    const uint32_t units = min(cu, u_hi - ku0);
    const uint32_t cwin = 8 * units;  // windows of this chunk (records use the chunk stride cw)
    // this wavefront's contiguous run of the chunk's units
    const uint32_t u_begin = (units * sw) / SL;
    const uint32_t u_count = (units * (sw + 1)) / SL - u_begin;

    // the previous chunk's records are consumed before its blocks are reused
    if (ku0 != u_lo) __syncthreads();
    // Activation copies, then the first D units of weights. The copies are
    // waited for before the weight loads are issued: the compiler waits for
    // all outstanding vector memory before the first LDS read after a
    // global-to-LDS copy, and vector memory completes in order, so a copy
    // waited for after the weight loads would wait for the weights. The
    // weights' HBM latency then overlaps the prep instead.
    // this workgroup's own conversion of its activations
    stage_x(a.x, K, ku0 * 256, M, MG, cw, cwin, dig, wave, lane);
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
#pragma unroll
    for (int i = 0; i < D; ++i)
      if (i < static_cast<int>(u_count))
        U::template load<WIDE, true>(trec + (ku0 + u_begin + i) * R.bytes, lane, ring[i]);
    // every wavefront's copies have landed; a bare barrier (a fenced one
    // would wait for the weight loads)
    __builtin_amdgcn_s_barrier();
    // items t = tid + 1024 i: block t / 16 advances by 64 windows a step,
    // (row group, window) kept without a division per item
    const uint32_t items = 16u * MG * cw;
    uint32_t q = (tid >> 4) / cw, W = (tid >> 4) % cw;
    for (uint32_t t = tid; t < items; t += kRowsThreads) {
      prep_item(t, q, W, cw, cwin, M, dig, xsc, xsum);
      W += kRowsThreads / 16;
      while (W >= cw) {
        W -= cw;
        ++q;
      }
    }
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): this wavefront's records are written
    __builtin_amdgcn_s_barrier();

    // Q6_K: each 32-element window holds two 16-element sub-blocks of their
    // own scales. The window's codes go in twice, in one instruction with
    // lane groups 0-1 (elements 0-15) and in one with lane groups 2-3
    // (elements 16-31), the others zero, so each sub-block's digit sums come
    // out apart; the int8 sub-scales weight them per window and d per unit.
    [[maybe_unused]] auto consume_q6 = [&](uint32_t u, const typename U::Raw& r) __attribute__((always_inline)) {
      if constexpr (QT == kQ6_K) {
        typename Dense<QT>::T ct;
        Dense<QT>::template prepare<true>(r, g, ct);
        const uint32_t keep = g < 2 ? ~0u : 0u;  // this lane group's slice in the first sub-block
        const uint8_t* dq[MG];
        const float* xq[MG];
        float accu[MG];
#pragma unroll
        for (int q = 0; q < MG; ++q) {
          dq[q] = dig + (q * cw + u * 8) * kBlock + lane * 8;
          xq[q] = xsc + (4 * q + g) * cw + u * 8;
          accu[q] = 0.0f;
        }
#pragma unroll
        for (int w = 0; w < 8; ++w) {
          const long bw = Dense<QT>::bc(ct, w);
          const uint32_t b_lo = static_cast<uint32_t>(bw), b_hi = static_cast<uint32_t>(static_cast<uint64_t>(bw) >> 32);
          const long b0 = pack2(b_lo & keep, b_hi & keep);
          const long b1 = pack2(b_lo & ~keep, b_hi & ~keep);
          const uint32_t sw = U::window_scales(r, w);
          const int hf = (w >> 1) & 1;
          const float s0 = static_cast<float>(static_cast<int32_t>(sw << (24 - 16 * hf)) >> 24);
          const float s1 = static_cast<float>(static_cast<int32_t>(sw << (16 - 16 * hf)) >> 24);
#pragma unroll
          for (int q = 0; q < MG; ++q) {
            const long av = *reinterpret_cast<const long*>(dq[q] + w * kBlock);
            const float xw = xq[q][w];
            const v4i c0 = __builtin_amdgcn_mfma_i32_16x16x32_i8(av, b0, v4i{0, 0, 0, 0}, 0, 0, 0);
            const v4i c1 = __builtin_amdgcn_mfma_i32_16x16x32_i8(av, b1, v4i{0, 0, 0, 0}, 0, 0, 0);
            // pairs exactly in int32 (|C0| < 2^19, |C1 * 256| < 2^27), halves in f32
            const float comb0 = fmaf(static_cast<float>(c0[2] + c0[3] * 256), 65536.0f,
                                     static_cast<float>(c0[0] + c0[1] * 256));
            const float comb1 = fmaf(static_cast<float>(c1[2] + c1[3] * 256), 65536.0f,
                                     static_cast<float>(c1[0] + c1[1] * 256));
            accu[q] = fmaf(xw, fmaf(s1, comb1, s0 * comb0), accu[q]);
          }
          // the window's sums are combined here, not after the last window
          // (the compiler would otherwise keep every window's digit sums live)
#pragma unroll
          for (int q = 0; q < MG; ++q) asm volatile("" : "+v"(accu[q]));
          __builtin_amdgcn_sched_barrier(0);
        }
        const float d = U::template d<WIDE>(r);
#pragma unroll
        for (int q = 0; q < MG; ++q) acc[q] = fmaf(d, accu[q], acc[q]);
      }
    };

    auto consume = [&](uint32_t j) {
#pragma unroll
      for (int i = 0; i < D; ++i) {
        if (j + i >= u_count) break;
        const uint32_t u = u_begin + j + i;  // chunk-relative unit
        if constexpr (QT == kQ6_K) {
          consume_q6(u, ring[i]);
        } else {
          float sa_own[2], sb_own[2];
          U::template scales<WIDE>(g, ring[i], sa_own, sb_own);
          float sa[8];
          {
            float t[4];
            gather4(sa_own[0], t);
#pragma unroll
            for (int gp = 0; gp < 4; ++gp) sa[2 * gp] = t[gp];
            gather4(sa_own[1], t);
#pragma unroll
            for (int gp = 0; gp < 4; ++gp) sa[2 * gp + 1] = t[gp];
          }
          typename Dense<QT>::T ct;
          Dense<QT>::template prepare<kFixed>(ring[i], g, ct);
          if constexpr (window_centered<QT>() && !ZP) {
            // the offsets left by the centred codes, b - z a (exactly rounded),
            // of windows 2k + h (k = lane group) of this unit for the tile's
            // outputs, times the rows' window sums
            constexpr float z = static_cast<float>(code_centre<QT>());
            const float2 sx = mrow < 4 * MG
                                  ? *reinterpret_cast<const float2*>(xsum + mrow * cw + u * 8 + 2 * g)
                                  : make_float2(0.0f, 0.0f);
            cmin = __builtin_amdgcn_mfma_f32_16x16x4f32(sx.x, fmaf(-z, sa_own[0], sb_own[0]), cmin, 0, 0, 0);
            cmin = __builtin_amdgcn_mfma_f32_16x16x4f32(sx.y, fmaf(-z, sa_own[1], sb_own[1]), cmin, 0, 0, 0);
          }
          // ZP: -z of windows 2k and 2k + 1 of this output as bytes 0 and 1 of zg[k]
          [[maybe_unused]] uint32_t zg[4];
          if constexpr (window_centered<QT>() && ZP) {
            // zero points of windows 2g, 2g + 1 (window_zero_point) and the
            // offsets left, b - z a (exactly rounded); -z of both as bytes 0
            // and 1 of one word, gathered from the other lane groups
            const float z0 = window_zero_point(sa_own[0], sb_own[0]);
            const float z1 = window_zero_point(sa_own[1], sb_own[1]);
            sb_own[0] = fmaf(-z0, sa_own[0], sb_own[0]);
            sb_own[1] = fmaf(-z1, sa_own[1], sb_own[1]);
            const uint32_t nz = (static_cast<uint32_t>(-static_cast<int>(z0)) & 0xFFu) |
                                ((static_cast<uint32_t>(-static_cast<int>(z1)) & 0xFFu) << 8);
            float t[4];
            gather4(__builtin_bit_cast(float, nz), t);
#pragma unroll
            for (int gp = 0; gp < 4; ++gp) zg[gp] = __builtin_bit_cast(uint32_t, t[gp]);
            // offsets of windows 2k + h (k = lane group) of this unit for the
            // tile's outputs, times the rows' window sums
            const float2 sx = mrow < 4 * MG
                                  ? *reinterpret_cast<const float2*>(xsum + mrow * cw + u * 8 + 2 * g)
                                  : make_float2(0.0f, 0.0f);
            cmin = __builtin_amdgcn_mfma_f32_16x16x4f32(sx.x, sb_own[0], cmin, 0, 0, 0);
            cmin = __builtin_amdgcn_mfma_f32_16x16x4f32(sx.y, sb_own[1], cmin, 0, 0, 0);
          }
          // this unit's digit blocks and activation scales per row group; the
          // windows are then constant offsets from them
          const uint8_t* dq[MG];
          const float* xq[MG];
#pragma unroll
          for (int q = 0; q < MG; ++q) {
            dq[q] = dig + (q * cw + u * 8) * kBlock + lane * 8;
            xq[q] = xsc + (4 * q + g) * cw + u * 8;
          }
#pragma unroll
          for (int w = 0; w < 8; ++w) {
            long bw;
            if constexpr (window_centered<QT>() && !ZP) bw = Dense<QT>::bc(ct, w);
            else bw = Dense<QT>::b(ct, w);
#pragma unroll
            for (int q = 0; q < MG; ++q) {
              const long av = *reinterpret_cast<const long*>(dq[q] + w * kBlock);
              const float xw = xq[q][w];
              v4i c = __builtin_amdgcn_mfma_i32_16x16x32_i8(av, bw, v4i{0, 0, 0, 0}, 0, 0, 0);
              if constexpr (window_centered<QT>() && ZP) {
                // byte (w & 1) of zg[w / 2] everywhere
                const uint32_t zb = __builtin_amdgcn_perm(0u, zg[w >> 1], (w & 1) ? 0x01010101u : 0u);
                c = __builtin_amdgcn_mfma_i32_16x16x32_i8(av, pack2(zb, zb), c, 0, 0, 0);
              }
              // pairs exactly in int32 (|C0| < 2^20, |C1 * 256| < 2^28), halves in f32
              const float comb = fmaf(static_cast<float>(c[2] + c[3] * 256), 65536.0f,
                                      static_cast<float>(c[0] + c[1] * 256));
              acc[q] = fmaf(sa[w] * xw, comb, acc[q]);
            }
            // one window at a time: the scheduler would otherwise hoist every
            // window's operand reads and keep their results live
            __builtin_amdgcn_sched_barrier(0);
          }
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

  // ---- reduce the 4 K slices of each tile in order ----
  __syncthreads();  // records no longer read
  float* red = reinterpret_cast<float*>(lds);  // [tile][slice][q][64]
#pragma unroll
  for (int q = 0; q < MG; ++q) {
    float v = acc[q] * kInvScale;  // centred codes' scale (exact)
    if constexpr (window_centered<QT>()) v -= cmin[q];
    red[((wc * SL + sw) * MG + q) * 64 + lane] = v;
  }
  __syncthreads();
  if (sw != 0) return;
  const uint64_t n_out = static_cast<uint64_t>(tile_raw) * 16 + col;
  if (tile_raw >= a.w.tiles || n_out >= a.w.n) return;
  float* const yout = gridDim.y > 1 ? a.part + static_cast<uint64_t>(blockIdx.y) * M * a.w.n : a.y;
#pragma unroll
  for (int q = 0; q < MG; ++q) {
    const int m = 4 * q + static_cast<int>(g);
    if (m >= M) continue;
    float v = red[((wc * SL) * MG + q) * 64 + lane];
#pragma unroll
    for (int p = 1; p < SL; ++p) v += red[((wc * SL + p) * MG + q) * 64 + lane];
    // NaN or infinite activations (or an overflow): the reference's own order
    // decides which outputs are NaN and which +-Inf
    if (!__builtin_isfinite(v) && gridDim.y == 1)
      v = exact_output_row<QT, WIDE>(a.w, a.x + static_cast<uint64_t>(m) * K, n_out);
    yout[static_cast<uint64_t>(m) * a.w.n + n_out] = v;
  }
}

template <int QT, bool WIDE, int MG, int D, int TL, bool ZP>
hipError_t launch_rows_t(RowsArgs a, uint32_t ksplit, hipStream_t st) {
  const uint32_t cap = rows_chunk_cap(MG);
  a.chunk_units = a.part_units < cap ? a.part_units : cap;
  const uint32_t main = rows_lds(MG, a.chunk_units);
  const uint32_t red = kRowsWaves * MG * 64 * 4;
  const uint32_t bytes = main > red ? main : red;
  auto kern = gemv_rows_kernel<QT, WIDE, MG, D, TL, ZP>;
  if (bytes > 65536) {
    const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                             hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(bytes));
    if (e != hipSuccess) {
      (void)hipGetLastError();  // the next launch's check must not see this call's error
      return e;
    }
  }
  if (ksplit > 1 && a.part == nullptr) return hipErrorInvalidValue;
  hipLaunchKernelGGL(kern, dim3((a.w.tiles + TL - 1) / TL, ksplit), dim3(kRowsThreads), bytes, st,
                     a);
  return hipGetLastError();
}

template <int QT, bool WIDE, int TL, bool ZP>
hipError_t launch_rows_tz(const RowsArgs& a, uint32_t ksplit, hipStream_t st) {
  // two units in flight per wavefront: what the 128-register budget of a
  // 16-wavefront workgroup holds
  if (a.m <= 4) return launch_rows_t<QT, WIDE, 1, 2, TL, ZP>(a, ksplit, st);
  return launch_rows_t<QT, WIDE, 2, 2, TL, ZP>(a, ksplit, st);
}

// Q4_K / Q5_K centring. The offsets of all windows are summed apart from the
// code products and subtracted once at the end, so what the centring leaves
// of them cancels there; centred on the middle of the code range, the
// leftover of outlier windows (b / a far from the middle) still cancels to
// 1.7e-5 of sum |x w| at K = 256 (16 rows; a CPU model of this kernel's
// arithmetic, and MI355X). The cancellation error grows like sqrt(K) and
// sum |x w| like K, so zero points (window_zero_point, subtracted by a second
// matrix instruction per window: 10-16% slower at 4-16 rows) are taken for
// K <= 2048, where the fixed centre would leave more than 6e-6.
constexpr uint64_t kRowsZeroPointUnits = 8;

template <int QT, bool WIDE, int TL>
hipError_t launch_rows_tl(const RowsArgs& a, uint32_t ksplit, hipStream_t st) {
  if constexpr (window_centered<QT>()) {
    if (a.w.units <= kRowsZeroPointUnits) return launch_rows_tz<QT, WIDE, TL, true>(a, ksplit, st);
  }
  return launch_rows_tz<QT, WIDE, TL, false>(a, ksplit, st);
}

// One-tile workgroups (16 K slices, no K split) for shapes of up to one tile
// per CU whose whole K range of activation digits fits one LDS chunk: every
// workgroup then builds its digits once and streams straight through. With
// more K (more chunks, each built and consumed in turn) the four-tile
// workgroups with K parts over the grid build less per workgroup. Measured on
// MI355X (Q4_0, one launch plus the split-K sum where there is one): 4096 x
// 1024 M=4 13.9 -> 7.1 us, M=8 13.7 -> 10.8; 4096 x 4096 M=4 13.3 -> 7.4,
// M=8 13.0 -> 11.1; slower with two chunks or more (4096 x 4096 M=16 15.5 ->
// 21.7, 12288 x 4096 M=4 16.7 -> 18.7).
bool rows_one_tile(uint64_t k, uint64_t n, uint32_t m) {
  const int mg = m <= 4 ? 1 : 2;
  return (n + 15) / 16 <= kRowsCUs && k / 256 <= rows_chunk_cap(mg);
}

template <int QT, bool WIDE>
hipError_t launch_rows_w(const RowsArgs& a, uint32_t ksplit, hipStream_t st) {
  if (rows_one_tile(a.w.k, a.w.n, static_cast<uint32_t>(a.m))) {
    if (ksplit != 1) return hipErrorInvalidValue;
    return launch_rows_tl<QT, WIDE, 1>(a, ksplit, st);
  }
  return launch_rows_tl<QT, WIDE, 4>(a, ksplit, st);
}

}  // namespace

uint32_t gemv_rows_splits(uint64_t k, uint64_t n, uint32_t m) {
  // one-tile workgroups: no K split (launch_rows_w)
  if (rows_one_tile(k, n, m)) return 1;
  const uint64_t tiles = (n + 15) / 16;
  // one four-tile workgroup per CU (LDS and registers); split K only when the
  // tile groups leave most CUs idle, keeping at least 4 units (one per K
  // slice) per part
  const uint64_t units = k / 256, groups = (tiles + 3) / 4;
  uint64_t s = kRowsCUs / (groups ? groups : 1);
  const uint64_t most = units / 4 ? units / 4 : 1;
  if (s > most) s = most;
  if (s < 1) s = 1;
  // the launch gives every part ceil(units / s) units; with that part length
  // fewer parts may cover K (8960 / 256 = 35 units over s = 8 gives parts of
  // 5, so 7 parts): return the count the launch will actually run
  const uint64_t part_units = (units + s - 1) / s;
  return static_cast<uint32_t>((units + part_units - 1) / part_units);
}

hipError_t launch_gemv_rows(int32_t qtype, bool wide, const View& w, const float* x, int m, float* y, float* part,
                            uint32_t ksplit, hipStream_t st) {
  if (m < 1 || m > 8 || ksplit < 1 || w.k == 0 || w.k % 256 != 0) return hipErrorInvalidValue;
  RowsArgs a{w, x, y, m, 0, 0, part};
  const uint32_t units = w.units;
  a.part_units = (units + ksplit - 1) / ksplit;
  const uint32_t parts = (units + a.part_units - 1) / a.part_units;
  if (parts != ksplit) return hipErrorInvalidValue;  // every K part holds units
  switch (qtype) {
    case kQ8_0: return wide ? launch_rows_w<kQ8_0, true>(a, ksplit, st) : launch_rows_w<kQ8_0, false>(a, ksplit, st);
    case kQ4_0: return wide ? launch_rows_w<kQ4_0, true>(a, ksplit, st) : launch_rows_w<kQ4_0, false>(a, ksplit, st);
    case kQ4_K: return wide ? launch_rows_w<kQ4_K, true>(a, ksplit, st) : launch_rows_w<kQ4_K, false>(a, ksplit, st);
    case kQ5_K: return wide ? launch_rows_w<kQ5_K, true>(a, ksplit, st) : launch_rows_w<kQ5_K, false>(a, ksplit, st);
    case kQ6_K: return wide ? launch_rows_w<kQ6_K, true>(a, ksplit, st) : launch_rows_w<kQ6_K, false>(a, ksplit, st);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace qi
