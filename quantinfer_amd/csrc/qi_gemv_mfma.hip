// Decode GEMV on the int8 matrix cores (v_mfma_i32_16x16x32_i8), output-rows
// layout, M <= 16 activation rows, K a multiple of 256.
//
// Arithmetic. Each activation x is turned into a 30-bit fixed-point integer
// F = rint(x * 2^s) (one power-of-two s per activation row and K chunk, chosen
// from the chunk's max |x|) written as four signed 8-bit digits
// F = d0 + d1*2^8 + d2*2^16 + d3*2^24. The weight codes enter the matrix cores
// unchanged (Q8_0 int8 codes, Q4_0/Q4_K/Q5_K/Q6_K unsigned codes), so every
// product digit*code is exact in int32, and
//   sum_k x_k q_k = 2^-s * (C0 + C1*2^8 + C2*2^16 + C3*2^24),  Ci = sum_k di_k q_k
// up to the 2^-30-of-chunk-max rounding of x. Per sub-block scale a and
// offset b of the format (w = a*q - b) are applied in f32 once per window:
//   y += a * 2^-s * combine(C) - b * sum_k x_k.
// This reorders the reference arithmetic and is judged by tolerance.
//
// Operand layout (16x16x32, verified on gfx950: A[i][k] lane i+16*(k/8),
// B[k][j] lane j+16*(k/8), C[i][j] lane j+16*(i/4) element i%4). For a tile of
// 16 outputs (B columns) the 4 lane groups g = lane/16 each stream their own
// 8 codes per step; A row i = 4*sigma + digit carries digit `digit` of lane
// group sigma's 8 activations and is zero elsewhere, so C row 4*sigma + digit
// holds lane group sigma's own digit sums: after a window of steps, lane
// (n, g) holds the four digit sums of its own codes in its four C registers,
// next to its own scale. A 256-element unit is 8 steps x 4 groups x 8 codes.
//
// Work split: a workgroup of 4 wavefronts owns TILES_C x 16 outputs; its
// wavefronts split those tiles (WC per row of tiles) and the K range (SW
// parts, reduced through LDS at the end). The activation digits for a K chunk
// are built once per workgroup into LDS. No state is shared between
// workgroups, so there are no device-scope fences.
#include "qi_device.h"
#include "qi_internal.h"

namespace qi {

typedef int v4i __attribute__((ext_vector_type(4)));

constexpr int kLdsA = 32768;  // activation digit bytes per chunk (all rows)

template <int QT>
struct Unit;  // per-format code/scale access for one (output n, lane group g, unit u)

// Loads read one (tile, unit) record (layout in qi_image.h): lane 16g + c
// takes row c's lane-group-g code chunks at q*1024 + lane*16 (each wavefront
// load is 1 KB contiguous), its scales from the record's scale sections.

template <>
struct Unit<kQ8_0> {
  static constexpr int kWindows = 2, kSteps = 4;  // two 32-element blocks per lane
  static constexpr bool kMin = false;
  struct Raw {
    uint4 q[4];
    uint32_t s0, s1;  // f16 pair in s0, or two f32 scales
  };
  template <bool W>
  __device__ static void load(const uint8_t* rec, uint32_t lane, Raw& r) {
    constexpr Record R = record_geometry(kQ8_0, W);
    const uint4* p = reinterpret_cast<const uint4*>(rec + R.qs) + lane;
    r.q[0] = p[0]; r.q[1] = p[64]; r.q[2] = p[128]; r.q[3] = p[192];
    const uint32_t e = (lane & 15) * 8 + 2 * (lane >> 4);  // blocks 2g, 2g+1 of row c
    if constexpr (W) {
      const uint2 d = *reinterpret_cast<const uint2*>(rec + R.d + e * 4);
      r.s0 = d.x; r.s1 = d.y;
    } else {
      r.s0 = *reinterpret_cast<const uint32_t*>(rec + R.d + e * 2);
      r.s1 = 0;
    }
  }
  template <bool W>
  __device__ static void scales(uint32_t, const Raw& r, float a[2], float b[2]) {
    if constexpr (W) {
      a[0] = __builtin_bit_cast(float, r.s0);
      a[1] = __builtin_bit_cast(float, r.s1);
    } else {
      a[0] = static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(r.s0 & 0xFFFFu)));
      a[1] = static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(r.s0 >> 16)));
    }
    b[0] = b[1] = 0.0f;
  }
  // step t (0..7): block h = t/4, bytes 8*(t%4) .. +8 of that block
  __device__ static long codes(const Raw& r, uint32_t, int t) {
    const uint4 q = r.q[(t >> 2) * 2 + ((t & 3) >> 1)];
    const uint32_t lo = (t & 1) ? q.z : q.x, hi = (t & 1) ? q.w : q.y;
    return static_cast<long>((static_cast<uint64_t>(hi) << 32) | lo);
  }
};

template <>
struct Unit<kQ4_0> {
  static constexpr int kWindows = 2, kSteps = 4;
  static constexpr bool kMin = true;  // w = d*q - 8d
  struct Raw {
    uint4 q[2];
    uint32_t s0, s1;
  };
  template <bool W>
  __device__ static void load(const uint8_t* rec, uint32_t lane, Raw& r) {
    constexpr Record R = record_geometry(kQ4_0, W);
    const uint4* p = reinterpret_cast<const uint4*>(rec + R.qs) + lane;
    r.q[0] = p[0]; r.q[1] = p[64];
    const uint32_t e = (lane & 15) * 8 + 2 * (lane >> 4);
    if constexpr (W) {
      const uint2 d = *reinterpret_cast<const uint2*>(rec + R.d + e * 4);
      r.s0 = d.x; r.s1 = d.y;
    } else {
      r.s0 = *reinterpret_cast<const uint32_t*>(rec + R.d + e * 2);
      r.s1 = 0;
    }
  }
  template <bool W>
  __device__ static void scales(uint32_t, const Raw& r, float a[2], float b[2]) {
    if constexpr (W) {
      a[0] = __builtin_bit_cast(float, r.s0);
      a[1] = __builtin_bit_cast(float, r.s1);
    } else {
      a[0] = static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(r.s0 & 0xFFFFu)));
      a[1] = static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(r.s0 >> 16)));
    }
    b[0] = 8.0f * a[0];
    b[1] = 8.0f * a[1];
  }
  // block h = t/4 (16 bytes: byte i = element i | element i+16 << 4);
  // quarter t%4: 0 = low nibbles of bytes 0-7, 1 = low of 8-15, 2 = high of 0-7, 3 = high of 8-15
  __device__ static long codes(const Raw& r, uint32_t, int t) {
    const uint4 q = r.q[t >> 2];
    const int qq = t & 3;
    const uint32_t lo = (qq & 1) ? q.z : q.x, hi = (qq & 1) ? q.w : q.y;
    const int sh = qq >= 2 ? 4 : 0;
    const uint32_t l2 = (lo >> sh) & 0x0F0F0F0Fu, h2 = (hi >> sh) & 0x0F0F0F0Fu;
    return static_cast<long>((static_cast<uint64_t>(h2) << 32) | l2);
  }
};

// Q4_K / Q5_K: lane group g holds code bytes [32g, 32g+32) of the super-block:
// step t < 4 takes the low nibbles of bytes 8t..8t+7 (sub-block 2g), t >= 4 the
// high nibbles of bytes 8(t-4).. (sub-block 2g+1); Q5_K adds bit 2g (low) or
// 2g+1 (high) of qh[byte] as bit 4.
template <bool FIVE>
struct UnitQ45K {
  static constexpr int kQT = FIVE ? kQ5_K : kQ4_K;
  static constexpr int kWindows = 2, kSteps = 4;
  static constexpr bool kMin = true;
  struct Raw {
    uint4 q[2];
    uint4 h[2];
    uint32_t sc[3];
    uint32_t s0, s1;  // d | dmin << 16 in s0 (f16), or d and dmin (f32)
  };
  template <bool W>
  __device__ static void load(const uint8_t* rec, uint32_t lane, Raw& r) {
    constexpr Record R = record_geometry(kQT, W);
    const uint32_t col = lane & 15;
    const uint4* p = reinterpret_cast<const uint4*>(rec + R.qs) + lane;
    r.q[0] = p[0]; r.q[1] = p[64];
    if constexpr (FIVE) {
      const uint4* h = reinterpret_cast<const uint4*>(rec + R.qh) + col;
      r.h[0] = h[0]; r.h[1] = h[16];
    }
    const uint32_t* s = reinterpret_cast<const uint32_t*>(rec + R.sc + col * 12);
    r.sc[0] = s[0]; r.sc[1] = s[1]; r.sc[2] = s[2];
    if constexpr (W) {
      r.s0 = reinterpret_cast<const uint32_t*>(rec + R.d)[col];
      r.s1 = reinterpret_cast<const uint32_t*>(rec + R.dmin)[col];
    } else {
      const uint32_t d = reinterpret_cast<const uint16_t*>(rec + R.d)[col];
      const uint32_t dm = reinterpret_cast<const uint16_t*>(rec + R.dmin)[col];
      r.s0 = d | (dm << 16);
      r.s1 = 0;
    }
  }
  template <bool W>
  __device__ static void scales(uint32_t g, const Raw& r, float a[2], float b[2]) {
    float d, dmin;
    if constexpr (W) {
      d = __builtin_bit_cast(float, r.s0);
      dmin = __builtin_bit_cast(float, r.s1);
    } else {
      d = static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(r.s0 & 0xFFFFu)));
      dmin = static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(r.s0 >> 16)));
    }
    uint32_t s0, m0, s1, m1;
    kquant_sc_m(r.sc[0], r.sc[1], r.sc[2], static_cast<int>(2 * g), s0, m0);
    kquant_sc_m(r.sc[0], r.sc[1], r.sc[2], static_cast<int>(2 * g + 1), s1, m1);
    a[0] = d * static_cast<float>(s0);
    b[0] = dmin * static_cast<float>(m0);
    a[1] = d * static_cast<float>(s1);
    b[1] = dmin * static_cast<float>(m1);
  }
  __device__ static long codes(const Raw& r, uint32_t g, int t) {
    const int tt = t & 3;
    const uint4 q = r.q[tt >> 1];
    const uint32_t lo = (tt & 1) ? q.z : q.x, hi = (tt & 1) ? q.w : q.y;
    const int sh = t >= 4 ? 4 : 0;
    uint32_t l2 = (lo >> sh) & 0x0F0F0F0Fu, h2 = (hi >> sh) & 0x0F0F0F0Fu;
    if constexpr (FIVE) {
      const uint4 h = r.h[tt >> 1];
      const uint32_t hl = (tt & 1) ? h.z : h.x, hh = (tt & 1) ? h.w : h.y;
      const int bit = static_cast<int>(2 * g) + (t >= 4 ? 1 : 0);
      l2 |= ((hl >> bit) & 0x01010101u) << 4;
      h2 |= ((hh >> bit) & 0x01010101u) << 4;
    }
    return static_cast<long>((static_cast<uint64_t>(h2) << 32) | l2);
  }
};

template <>
struct Unit<kQ4_K> : UnitQ45K<false> {};
template <>
struct Unit<kQ5_K> : UnitQ45K<true> {};

// Q6_K: lane group g = 2*ip + c holds ql bytes [64ip + 32c, +32) and qh bytes
// [32ip, +32). Step t < 4: low nibbles of ql bytes 8t.. with qh bits 2c (elements
// 128ip + 32c + 8t + j); t >= 4: high nibbles of ql bytes 8(t-4).. with qh bits
// 2c+4 (elements 128ip + 32c + 64 + 8(t-4) + j). Windows are pairs of steps
// (16-element sub-blocks 8ip + 2c + {0, 1, 4, 5}); w = a*q - 32a.
template <>
struct Unit<kQ6_K> {
  static constexpr int kWindows = 4, kSteps = 2;
  static constexpr bool kMin = true;
  struct Raw {
    uint4 q[2];
    uint4 h[2];
    uint2 sc;
    uint32_t d;  // f16 in the low half, or f32
  };
  template <bool W>
  __device__ static void load(const uint8_t* rec, uint32_t lane, Raw& r) {
    constexpr Record R = record_geometry(kQ6_K, W);
    const uint32_t col = lane & 15, ip = lane >> 5;
    const uint4* p = reinterpret_cast<const uint4*>(rec + R.qs) + lane;
    r.q[0] = p[0]; r.q[1] = p[64];
    const uint4* h = reinterpret_cast<const uint4*>(rec + R.qh) + 32 * ip + col;
    r.h[0] = h[0]; r.h[1] = h[16];
    r.sc = *reinterpret_cast<const uint2*>(rec + R.sc + col * 16 + 8 * ip);
    if constexpr (W) r.d = reinterpret_cast<const uint32_t*>(rec + R.d)[col];
    else r.d = reinterpret_cast<const uint16_t*>(rec + R.d)[col];
  }
  template <bool W>
  __device__ static void scales(uint32_t g, const Raw& r, float a[4], float b[4]) {
    float d;
    if constexpr (W) d = __builtin_bit_cast(float, r.d);
    else d = static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(r.d)));
    const uint32_t c = g & 1;
    const uint32_t lo = c ? (r.sc.x >> 16) : r.sc.x;  // sub-scales 2c, 2c+1 of this half
    const uint32_t hi = c ? (r.sc.y >> 16) : r.sc.y;  // sub-scales 2c+4, 2c+5
    a[0] = d * static_cast<float>(static_cast<int8_t>(lo & 0xFFu));
    a[1] = d * static_cast<float>(static_cast<int8_t>((lo >> 8) & 0xFFu));
    a[2] = d * static_cast<float>(static_cast<int8_t>(hi & 0xFFu));
    a[3] = d * static_cast<float>(static_cast<int8_t>((hi >> 8) & 0xFFu));
#pragma unroll
    for (int i = 0; i < 4; ++i) b[i] = 32.0f * a[i];
  }
  __device__ static long codes(const Raw& r, uint32_t g, int t) {
    const int tt = t & 3;
    const uint4 q = r.q[tt >> 1];
    const uint4 h = r.h[tt >> 1];
    const uint32_t lo = (tt & 1) ? q.z : q.x, hi = (tt & 1) ? q.w : q.y;
    const uint32_t hl = (tt & 1) ? h.z : h.x, hh = (tt & 1) ? h.w : h.y;
    const int sh = t >= 4 ? 4 : 0;
    const int hs = 2 * static_cast<int>(g & 1) + (t >= 4 ? 4 : 0);
    const uint32_t l2 = ((lo >> sh) & 0x0F0F0F0Fu) | (((hl >> hs) & 0x03030303u) << 4);
    const uint32_t h2 = ((hi >> sh) & 0x0F0F0F0Fu) | (((hh >> hs) & 0x03030303u) << 4);
    return static_cast<long>((static_cast<uint64_t>(h2) << 32) | l2);
  }
};

// Unit-relative element of 8-element group p (0..31): the first element.
template <int QT>
__device__ __forceinline__ uint32_t group_first_element(uint32_t p) {
  if constexpr (QT == kQ6_K) {
    // p = 16ip + r; r < 8: c = r/4, t = r%4 (low nibbles); r >= 8: c = (r-8)/4, t = 4 + r%4
    const uint32_t ip = p >> 4, r = p & 15;
    const uint32_t c = (r & 7) >> 2, t = (r & 3) + (r >= 8 ? 4 : 0);
    return 128 * ip + 32 * c + 8 * (t & 3) + (t >= 4 ? 64 : 0);
  } else {
    return 8 * p;  // e = 64g + 8t + j with p = 8g + t
  }
}
// (lane group, step) of 8-element group p
template <int QT>
__device__ __forceinline__ void group_slot(uint32_t p, uint32_t& g, uint32_t& t) {
  if constexpr (QT == kQ6_K) {
    const uint32_t ip = p >> 4, r = p & 15;
    g = 2 * ip + ((r & 7) >> 2);
    t = (r & 3) + (r >= 8 ? 4 : 0);
  } else {
    g = p >> 3;
    t = p & 7;
  }
}

__device__ __forceinline__ float wave_max(float v) {
  v = fmaxf(v, __builtin_amdgcn_update_dpp(0.0f, v, 0xB1, 0xF, 0xF, false));
  v = fmaxf(v, __builtin_amdgcn_update_dpp(0.0f, v, 0x4E, 0xF, 0xF, false));
  v = fmaxf(v, __builtin_amdgcn_update_dpp(0.0f, v, 0x141, 0xF, 0xF, false));
  v = fmaxf(v, __builtin_amdgcn_update_dpp(0.0f, v, 0x140, 0xF, 0xF, false));
  const float r0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 0));
  const float r1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 16));
  const float r2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 32));
  const float r3 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 48));
  return fmaxf(fmaxf(r0, r1), fmaxf(r2, r3));
}

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

template <int QT, bool WIDE, int MT, int WC, int SW>
__global__ __launch_bounds__(64 * WC * SW) void gemv_mfma_kernel(GemvMfmaArgs a) {
  using U = Unit<QT>;
  constexpr int kThreads = 64 * WC * SW;
  constexpr int kWaves = WC * SW;
  constexpr int kChunk = kLdsA / (4 * MT);  // activations per row per chunk
  constexpr int kUnitsChunk = kChunk / 256;
  // digits [m][unit][t][g][digit] x 8 B, then 1 KB of zeros read by the lanes
  // whose A row belongs to another lane group
  __shared__ __attribute__((aligned(16))) uint8_t lds_a[kLdsA + 1024];
  __shared__ __attribute__((aligned(16))) float lds_gs[MT * kUnitsChunk * 32];  // [m][u][g][t] sums of 8
  __shared__ float lds_inv[MT];
  __shared__ int lds_shift[MT];
  __shared__ float lds_max[kWaves][MT];
  __shared__ float lds_red[SW > 1 ? SW : 1][MT][16 * WC];

  const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const uint32_t wc = wave % WC, sw = wave / WC;
  const uint32_t col = lane & 15, g = lane >> 4;
  const uint64_t n_raw = (static_cast<uint64_t>(blockIdx.x) * WC + wc) * 16 + col;
  // this wavefront's tile of 16 outputs (the grid's last tiles may be past
  // the end: they re-read the last tile, whose rows past n are zero padding)
  constexpr Record R = record_geometry(QT, WIDE);
  const uint32_t tile = min(blockIdx.x * WC + wc, a.w.tiles - 1);
  const uint8_t* trec = a.w.qs + static_cast<uint64_t>(tile) * a.w.units * R.bytes;
  const uint32_t K = static_cast<uint32_t>(a.w.k);
  const int M = a.m;

  // A-operand lane role: row (sigma, digit) is live for lane group g == sigma
  const uint32_t arow = lane & 15, sigma = arow >> 2, digit = arow & 3;
  const bool a_live = sigma == g;

  for (uint32_t i = tid; i < 256; i += kThreads) reinterpret_cast<uint32_t*>(lds_a + kLdsA)[i] = 0;

  float acc[MT];
#pragma unroll
  for (int m = 0; m < MT; ++m) acc[m] = 0.0f;

  // Units in flight per wavefront: their weight loads are issued before the
  // activation prep of the chunk and refilled as units are consumed.
  constexpr int D = (kWaves >= 16 || MT > 2) ? 2 : 4;
  typename U::Raw ring[D];

  for (uint32_t k0 = 0; k0 < K; k0 += kChunk) {
    const uint32_t kc = min(static_cast<uint32_t>(kChunk), K - k0);
    const uint32_t units = kc / 256;
    const uint32_t ku0 = k0 / 256;
    const uint32_t u_begin = (units * sw) / SW, u_end = (units * (sw + 1)) / SW;
#pragma unroll
    for (int i = 0; i < D; ++i)
      if (u_begin + i < u_end) U::template load<WIDE>(trec + (ku0 + u_begin + i) * R.bytes, lane, ring[i]);

    // ---- prep: 8-element groups (m, unit, t, g), g fastest across threads ----
    constexpr int kGroups = MT * kChunk / 8;
    constexpr int kPer = (kGroups + kThreads - 1) / kThreads;
    float xv[kPer][8];
    float mx[MT];
#pragma unroll
    for (int m = 0; m < MT; ++m) mx[m] = 0.0f;
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const uint32_t gi = tid + kThreads * i;
      const uint32_t m = gi / (units * 32), r = gi % (units * 32);
      const uint32_t u = r >> 5, t = (r & 31) >> 2, gg = r & 3;
      const bool ok = gi < static_cast<uint32_t>(MT) * units * 32 && static_cast<int>(m) < M;
      if (ok) {
        uint32_t e;
        if constexpr (QT == kQ6_K) {
          e = 128 * (gg >> 1) + 32 * (gg & 1) + 8 * (t & 3) + (t >= 4 ? 64 : 0);
        } else {
          e = 64 * gg + 8 * t;
        }
        const float4* xp = reinterpret_cast<const float4*>(a.x + static_cast<uint64_t>(m) * K + k0 + 256 * u + e);
        const float4 x0 = xp[0], x1 = xp[1];
        xv[i][0] = x0.x; xv[i][1] = x0.y; xv[i][2] = x0.z; xv[i][3] = x0.w;
        xv[i][4] = x1.x; xv[i][5] = x1.y; xv[i][6] = x1.z; xv[i][7] = x1.w;
      } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) xv[i][j] = 0.0f;
      }
      float lm = 0.0f;
#pragma unroll
      for (int j = 0; j < 8; ++j) lm = fmaxf(lm, fabsf(xv[i][j]));
#pragma unroll
      for (int mm = 0; mm < MT; ++mm)
        if (static_cast<uint32_t>(mm) == m) mx[mm] = fmaxf(mx[mm], lm);
    }
#pragma unroll
    for (int m = 0; m < MT; ++m) {
      const float w = wave_max(mx[m]);
      if (lane == 0) lds_max[wave][m] = w;
    }
    __syncthreads();
    if (tid < static_cast<uint32_t>(MT)) {
      float mm = 0.0f;
#pragma unroll
      for (int w = 0; w < kWaves; ++w) mm = fmaxf(mm, lds_max[w][tid]);
      // 2^s with max|x| * 2^s < 2^29: F = rint(x * 2^s) keeps 30 bits with headroom
      const int e = mm > 0.0f ? __builtin_amdgcn_frexp_expf(mm) : 0;
      lds_shift[tid] = 29 - e;
      lds_inv[tid] = mm > 0.0f ? ldexpf(1.0f, e - 29) : 0.0f;
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const uint32_t gi = tid + kThreads * i;
      const uint32_t m = gi / (units * 32), r = gi % (units * 32);
      const uint32_t u = r >> 5, t = (r & 31) >> 2, gg = r & 3;
      if (gi < static_cast<uint32_t>(MT) * units * 32 && static_cast<int>(m) < M) {
        const int sh = lds_shift[m];
        uint32_t dig[8];
        float s = 0.0f;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const int F = static_cast<int>(rintf(ldexpf(xv[i][j], sh)));
          dig[j] = (static_cast<uint32_t>(F) + 0x00808080u) ^ 0x00808080u;
          s += xv[i][j];
        }
        uint32_t lo[4], hi[4];
        transpose4(dig, lo);
        transpose4(dig + 4, hi);
        uint8_t* dst = lds_a + ((((m * kUnitsChunk + u) * 8 + t) * 4 + gg) * 32);
        *reinterpret_cast<uint4*>(dst) = make_uint4(lo[0], hi[0], lo[1], hi[1]);
        *reinterpret_cast<uint4*>(dst + 16) = make_uint4(lo[2], hi[2], lo[3], hi[3]);
        lds_gs[((m * kUnitsChunk + u) * 4 + gg) * 8 + t] = s;
      }
    }
    __syncthreads();

    // ---- main: this wavefront's units of the chunk, D in flight ----
    for (uint32_t ub = u_begin; ub < u_end; ub += D) {
#pragma unroll
      for (int i = 0; i < D; ++i) {
        const uint32_t u = ub + i;
        if (u >= u_end) break;
        float sa[U::kWindows], sb[U::kWindows];
        U::template scales<WIDE>(g, ring[i], sa, sb);
        const typename U::Raw cur = ring[i];
        if (u + D < u_end) U::template load<WIDE>(trec + (ku0 + u + D) * R.bytes, lane, ring[i]);
#pragma unroll
        for (int m = 0; m < MT; ++m) {
          if (m >= M) break;
          const uint8_t* abase = a_live ? lds_a + (((m * kUnitsChunk + u) * 8) * 4 + g) * 32 + digit * 8
                                        : lds_a + kLdsA;
          const float inv = lds_inv[m];
          const float* gs = lds_gs + ((m * kUnitsChunk + u) * 4 + g) * 8;
#pragma unroll
          for (int w = 0; w < U::kWindows; ++w) {
            v4i c = {0, 0, 0, 0};
#pragma unroll
            for (int s = 0; s < U::kSteps; ++s) {
              const int t = w * U::kSteps + s;
              const long av = *reinterpret_cast<const long*>(abase + t * 128);
              c = __builtin_amdgcn_mfma_i32_16x16x32_i8(av, U::codes(cur, g, t), c, 0, 0, 0);
            }
            // combine digit sums (exact int32) in f32
            const float comb = fmaf(fmaf(fmaf(static_cast<float>(c[3]), 256.0f, static_cast<float>(c[2])),
                                         256.0f, static_cast<float>(c[1])),
                                    256.0f, static_cast<float>(c[0]));
            acc[m] = fmaf(sa[w] * inv, comb, acc[m]);
            if constexpr (U::kMin) {
              float xs;
              if constexpr (U::kSteps == 4) {
                const float4 v = *reinterpret_cast<const float4*>(gs + 4 * w);
                xs = (v.x + v.y) + (v.z + v.w);
              } else {
                const float2 v = *reinterpret_cast<const float2*>(gs + 2 * w);
                xs = v.x + v.y;
              }
              acc[m] = fmaf(-sb[w], xs, acc[m]);
            }
          }
        }
      }
    }
    __syncthreads();  // LDS reused by the next chunk
  }

  // ---- reduce: 4 lane groups of a column, then the SW K-parts ----
#pragma unroll
  for (int m = 0; m < MT; ++m) {
    float v = acc[m];
    v += __shfl_xor(v, 16);
    v += __shfl_xor(v, 32);
    acc[m] = v;
  }
  if constexpr (SW > 1) {
    if (g == 0) {
#pragma unroll
      for (int m = 0; m < MT; ++m) lds_red[sw][m][wc * 16 + col] = acc[m];
    }
    __syncthreads();
    if (sw == 0 && g == 0 && n_raw < a.w.n) {
#pragma unroll
      for (int m = 0; m < MT; ++m) {
        if (m >= M) break;
        float v = lds_red[0][m][wc * 16 + col];
#pragma unroll
        for (int p = 1; p < SW; ++p) v += lds_red[p][m][wc * 16 + col];
        a.y[static_cast<uint64_t>(m) * a.w.n + n_raw] = v;
      }
    }
  } else {
    if (g == 0 && n_raw < a.w.n) {
#pragma unroll
      for (int m = 0; m < MT; ++m) {
        if (m >= M) break;
        a.y[static_cast<uint64_t>(m) * a.w.n + n_raw] = acc[m];
      }
    }
  }
}

namespace {

template <int QT, bool WIDE, int MT, int WC, int SW>
hipError_t launch4(const GemvMfmaArgs& a, hipStream_t st) {
  const uint64_t tiles = (a.w.n + 15) / 16;
  const uint32_t grid = static_cast<uint32_t>((tiles + WC - 1) / WC);
  hipLaunchKernelGGL((gemv_mfma_kernel<QT, WIDE, MT, WC, SW>), dim3(grid), dim3(64 * WC * SW), 0, st, a);
  return hipGetLastError();
}

// shape id -> (output tiles per workgroup WC, K parts SW)
template <int QT, bool WIDE, int MT>
hipError_t launch_split(const GemvMfmaArgs& a, int shape, hipStream_t st) {
  switch (shape) {
    case 0: return launch4<QT, WIDE, MT, 4, 1>(a, st);
    case 1: return launch4<QT, WIDE, MT, 4, 2>(a, st);
    case 2: return launch4<QT, WIDE, MT, 4, 4>(a, st);
    case 3: return launch4<QT, WIDE, MT, 2, 8>(a, st);
    case 4: return launch4<QT, WIDE, MT, 1, 16>(a, st);
    case 5: return launch4<QT, WIDE, MT, 2, 4>(a, st);
    default: return launch4<QT, WIDE, MT, 1, 8>(a, st);
  }
}

template <int QT, bool WIDE>
hipError_t launch_m(const GemvMfmaArgs& a, int mt, int split, hipStream_t st) {
  switch (mt) {
    case 1: return launch_split<QT, WIDE, 1>(a, split, st);
    case 2: return launch_split<QT, WIDE, 2>(a, split, st);
    case 4: return launch_split<QT, WIDE, 4>(a, split, st);
    case 8: return launch_split<QT, WIDE, 8>(a, split, st);
    default: return launch_split<QT, WIDE, 16>(a, split, st);
  }
}

template <int QT>
hipError_t launch_w(const GemvMfmaArgs& a, bool wide, int mt, int split, hipStream_t st) {
  return wide ? launch_m<QT, true>(a, mt, split, st) : launch_m<QT, false>(a, mt, split, st);
}

}  // namespace

bool gemv_mfma_supported(int32_t qtype, int32_t layout, uint64_t k) {
  return layout == kOutputRows && qtype >= kQ8_0 && qtype <= kQ6_K && k % 256 == 0 && k > 0;
}

int gemv_mfma_split(uint64_t n) {
  // Workgroup shape: 64 outputs and 4 K parts per workgroup when there are
  // enough outputs to give every CU one; fewer outputs and more K parts per
  // workgroup otherwise (the activation prep is shared by the workgroup).
  const uint64_t tiles = (n + 15) / 16;
  if (tiles / 4 >= 192) return 2;
  if (tiles / 2 >= 192) return 3;
  return 4;
}

hipError_t launch_gemv_mfma(int32_t qtype, bool wide, int mt, int split, const GemvMfmaArgs& a,
                            hipStream_t st) {
  switch (qtype) {
    case kQ8_0: return launch_w<kQ8_0>(a, wide, mt, split, st);
    case kQ4_0: return launch_w<kQ4_0>(a, wide, mt, split, st);
    case kQ4_K: return launch_w<kQ4_K>(a, wide, mt, split, st);
    case kQ5_K: return launch_w<kQ5_K>(a, wide, mt, split, st);
    case kQ6_K: return launch_w<kQ6_K>(a, wide, mt, split, st);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace qi
