// GPU-resident Qwen3 dense decoder (include/qi_hip.h, "GPU-resident Qwen3").
//
// The forward pass of crates/quantinfer-runtime/src/qwen3/mod.rs:117-378 with
// weights, activations and the KV cache in device memory:
//
//   embedding + RMSNorm           residual_norm_kernel<EMBED>
//   q|k|v projection              one fused GEMV/GEMM image (qi_gemv_mfma / qi_gemm)
//   q_norm/k_norm, RoPE, KV append qk_norm_rope_kernel
//   GQA attention                 attn_kernel (a 4-wavefront workgroup per 64 positions;
//                                 the last workgroup of a KV head combines the chunks);
//                                 prompt rows at head_dim 128: attn_mfma_kernel
//   o projection                  GEMV/GEMM
//   residual + RMSNorm            residual_norm_kernel<ADD>
//   gate|up projection            one fused image
//   SiLU(gate) * up               the gate|up GEMV epilogue (one row) or GEMM epilogue
//                                 (an un-split GEMM); silu_mul_kernel otherwise
//   down projection               GEMV/GEMM
//   residual + next RMSNorm       residual_norm_kernel<ADD> (the final norm after the last layer)
//   LM head on the last row       GEMV (a Q6_K head stays quantized)
//   greedy argmax                 argmax_partial_kernel + argmax_final_kernel
//
// Position bookkeeping lives on the device: the cache holds the token history
// (tok[p] = token at position p) and the current length. Every kernel reads
// the length from device memory, and the last kernel of a step writes the
// selected token at tok[len + rows] and advances the length. A decode step
// therefore has fixed launch arguments and is captured once as a HIP graph and
// replayed for every generated token.
//
// KV cache layout per layer (positions rounded up to 64):
//   keys   [kv_head][dim][position]  - lanes of a wavefront read 64 consecutive
//                                      positions of one dimension (256 B)
//   values [kv_head][position][dim]  - lanes read one position's dimensions
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include <atomic>
#include <memory>
#include <string>
#include <vector>

#include "qi_ctx.h"
#include "qi_internal.h"

using qi_abi::fail;
using qi_abi::hip_fail;

namespace {

constexpr uint32_t kChunk = 64;       // attention positions per wavefront
constexpr uint32_t kMaxRows = 512;    // prompt tokens per forward chunk
constexpr uint32_t kArgBlocks = 256;  // argmax partial blocks
constexpr uint64_t kPartialBudget = 64ull << 20;  // bytes of attention partials per row batch

// Wavefront reductions on DPP lane moves (no LDS round trips): swap lanes in
// pairs and quads, mirror within half rows and rows (every lane then holds its
// row of 16), broadcast lane 15 into rows 1 and 3 and lane 31 into rows 2 and
// 3; lane 63 ends with the total, read back as one value for every lane.
// Disabled rows keep `old` (the operation's identity).
template <int CTRL, int ROWS = 0xF>
__device__ __forceinline__ float dpp_move(float old, float v) {
  return __int_as_float(
      __builtin_amdgcn_update_dpp(__float_as_int(old), __float_as_int(v), CTRL, ROWS, 0xF, false));
}

__device__ __forceinline__ float wave_sum(float v) {
  v += dpp_move<0xB1>(0.0f, v);         // quad_perm [1,0,3,2]
  v += dpp_move<0x4E>(0.0f, v);         // quad_perm [2,3,0,1]
  v += dpp_move<0x141>(0.0f, v);        // row_half_mirror
  v += dpp_move<0x140>(0.0f, v);        // row_mirror
  v += dpp_move<0x142, 0xA>(0.0f, v);   // row_bcast:15
  v += dpp_move<0x143, 0xC>(0.0f, v);   // row_bcast:31
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

__device__ __forceinline__ float wave_max(float v) {
  v = fmaxf(v, dpp_move<0xB1>(-INFINITY, v));
  v = fmaxf(v, dpp_move<0x4E>(-INFINITY, v));
  v = fmaxf(v, dpp_move<0x141>(-INFINITY, v));
  v = fmaxf(v, dpp_move<0x140>(-INFINITY, v));
  v = fmaxf(v, dpp_move<0x142, 0xA>(-INFINITY, v));
  v = fmaxf(v, dpp_move<0x143, 0xC>(-INFINITY, v));
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

// ---------------------------------------------------------------- RMSNorm
// backends/cpu/src/backend.rs:172-190: out = v * (1/sqrt(mean(v^2) + eps)) * w.
// EMBED: h = embedding[tok[len + row]] (backend.rs:281-298). Otherwise h = h + y
// (runtime/src/linear.rs:129-142), or h unchanged when y is null (the residual
// add already done by the projection). Then x = RMSNorm(h) * w. A row is held in
// registers (NV float4 per thread), so every load is issued before the
// reduction and nothing is read twice.
template <bool EMBED, int NV>
__global__ __launch_bounds__(256) void residual_norm_kernel(
    float* __restrict__ h, const float* __restrict__ y, const float* __restrict__ table,
    const int32_t* __restrict__ tok, const uint32_t* __restrict__ len, float* __restrict__ x,
    const float* __restrict__ w, uint32_t hidden, float eps) {
  __shared__ float red[4];
  const uint32_t r = blockIdx.x;
  const uint32_t n4 = hidden / 4;
  float4* hr = reinterpret_cast<float4*>(h + static_cast<uint64_t>(r) * hidden);
  const float4* src;
  if constexpr (EMBED) {
    const int32_t t = tok[*len + r];
    src = reinterpret_cast<const float4*>(table + static_cast<uint64_t>(t) * hidden);
  } else {
    src = reinterpret_cast<const float4*>(y + static_cast<uint64_t>(r) * hidden);
  }
  const float4* wr = reinterpret_cast<const float4*>(w);
  float4 v[NV], g[NV];
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const uint32_t i = threadIdx.x + 256u * j;
    v[j] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    g[j] = v[j];
    if (i < n4) {
      g[j] = wr[i];
      if constexpr (EMBED) {
        v[j] = src[i];
      } else {
        const float4 o = hr[i];
        if (y != nullptr) {
          const float4 d = src[i];
          v[j] = make_float4(o.x + d.x, o.y + d.y, o.z + d.z, o.w + d.w);
        } else {
          v[j] = o;
        }
      }
    }
  }
  float ss = 0.0f;
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const uint32_t i = threadIdx.x + 256u * j;
    if (i < n4) hr[i] = v[j];
    ss += v[j].x * v[j].x + v[j].y * v[j].y + v[j].z * v[j].z + v[j].w * v[j].w;
  }
  ss = wave_sum(ss);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
  __syncthreads();
  const float total = (red[0] + red[1]) + (red[2] + red[3]);
  const float inv = 1.0f / sqrtf(total / static_cast<float>(hidden) + eps);
  float4* xr = reinterpret_cast<float4*>(x + static_cast<uint64_t>(r) * hidden);
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const uint32_t i = threadIdx.x + 256u * j;
    if (i < n4)
      xr[i] = make_float4(v[j].x * inv * g[j].x, v[j].y * inv * g[j].y, v[j].z * inv * g[j].z,
                          v[j].w * inv * g[j].w);
  }
}

// ------------------------------------------- head RMSNorm, RoPE, KV append
// One wavefront per (head, row). Heads [0, heads) are query heads, the next
// kv_heads are key heads (which also copy their value head into the cache).
// rms_norm_heads (backend.rs:192-198), then apply_rope with the pair (p,
// p + head_dim/2) (backend.rs:239-279) at position len + row, then
// KvCache::append (cache.rs:96-125) of the rotated key and the value.
struct HeadArgs {
  const float* qkv;  // [rows][row_stride]: q | k | v
  uint32_t row_stride, heads, kv_heads, head_dim;
  const float* q_norm;
  const float* k_norm;
  float eps;
  const float* rope_cos;  // [position][head_dim/2]
  const float* rope_sin;
  const uint32_t* len;
  float* q_out;  // [rows][heads*head_dim]
  float* keys;   // this layer: [kv_head][dim][cap]
  float* values; // this layer: [kv_head][cap][dim]
  uint32_t cap;
};

__global__ __launch_bounds__(64) void qk_norm_rope_kernel(HeadArgs a) {
  const uint32_t r = blockIdx.y, hidx = blockIdx.x, lane = threadIdx.x;
  const uint32_t pos = *a.len + r;
  const uint32_t hd = a.head_dim, pairs = hd / 2;
  const bool is_q = hidx < a.heads;
  const uint32_t g = is_q ? 0 : hidx - a.heads;
  const float* row = a.qkv + static_cast<uint64_t>(r) * a.row_stride;
  const float* src = is_q ? row + hidx * hd : row + a.heads * hd + g * hd;
  const float* wn = is_q ? a.q_norm : a.k_norm;
  // head_dim <= 128: at most one pair per lane
  const bool act = lane < pairs;
  const float x0 = act ? src[lane] : 0.0f;
  const float x1 = act ? src[lane + pairs] : 0.0f;
  const float ss = wave_sum(x0 * x0 + x1 * x1);
  const float inv = 1.0f / sqrtf(ss / static_cast<float>(hd) + a.eps);
  if (act) {
    const float f = x0 * inv * wn[lane];
    const float s = x1 * inv * wn[lane + pairs];
    const float c = a.rope_cos[static_cast<uint64_t>(pos) * pairs + lane];
    const float sn = a.rope_sin[static_cast<uint64_t>(pos) * pairs + lane];
    const float o0 = f * c - s * sn;
    const float o1 = f * sn + s * c;
    if (is_q) {
      float* q = a.q_out + static_cast<uint64_t>(r) * a.heads * hd + hidx * hd;
      q[lane] = o0;
      q[lane + pairs] = o1;
    } else {
      float* kt = a.keys + static_cast<uint64_t>(g) * hd * a.cap;
      kt[static_cast<uint64_t>(lane) * a.cap + pos] = o0;
      kt[static_cast<uint64_t>(lane + pairs) * a.cap + pos] = o1;
    }
  }
  if (!is_q) {
    const float* v = row + (a.heads + a.kv_heads) * hd + g * hd;
    float* vc = a.values + (static_cast<uint64_t>(g) * a.cap + pos) * hd;
    for (uint32_t d = lane; d < hd; d += 64) vc[d] = v[d];
  }
}

// ------------------------------------------------------------- attention
// runtime/src/attention.rs:37-141: for query token r at position p = len + r,
// head h of kv group g: scores s_j = (q . k_j) / sqrt(head_dim) for j <= p,
// weights softmax(s), output sum_j weight_j v_j. Split over chunks of 64
// positions: each wavefront keeps its chunk's max m, sum l = sum exp(s - m) and
// unnormalized output o = sum exp(s - m) v; the combine rescales the chunks by
// exp(m - max m) (the same softmax, evaluated in pieces).
struct AttnArgs {
  const float* q;  // [rows][heads*hd] (rotated queries; unfused path)
  const float* keys;
  const float* values;
  const uint32_t* len;
  float* pm;  // [batch row][heads][chunks]
  float* pl;
  float* po;  // [batch row][heads][chunks][hd]
  uint32_t heads, kv_heads, cap, chunks;
  uint32_t row0;   // first row of this batch (blockIdx row 0)
  uint32_t nrows;  // rows in this batch (the row-blocked prefill path)
  float scale;
  float* out;  // [rows][heads*hd]
  // fused path (one decode row): q/k/v straight from the projection
  const float* qkv;
  uint32_t row_stride;
  const float* q_norm;
  const float* k_norm;
  float eps;
  const float* rope_cos;
  const float* rope_sin;
  float* keys_w;    // writable views of the same cache (the new position)
  float* values_w;
  uint32_t* tickets;  // [batch row][kv head] chunk counters, zero between launches
};

// RMSNorm of one head from preloaded values (lane owns the pair (lane,
// lane + hd/2); head_dim <= 128) and RoPE: returns the rotated pair. Lanes past
// head_dim/2 (`act` false) hold clamped copies and add nothing to the sum.
__device__ __forceinline__ float2 norm_rope(float x0, float x1, float w0, float w1, float c, float sn,
                                            float hd, float eps, bool act) {
  const float ss = wave_sum(act ? x0 * x0 + x1 * x1 : 0.0f);
  const float inv = 1.0f / sqrtf(ss / hd + eps);
  const float f = x0 * inv * w0;
  const float s = x1 * inv * w1;
  return make_float2(f * c - s * sn, f * sn + s * c);
}

// Partials are exchanged between the workgroups of one (row, KV head) through
// device-coherent stores and loads (bypassing the non-coherent per-XCD L2
// copies), ordered by waiting for the stores before the ticket increment, so
// no cache-wide writeback or invalidate is needed.
__device__ __forceinline__ void store_coherent(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float load_coherent(const float* p) {
  return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

constexpr int kAttnWaves = 4;

// Query rows per prefill workgroup: 16 (row, head) pairs at head_dim 128 (the
// staged queries take 8 KB and two workgroups fit a CU's LDS), 4 at head_dim
// 64 (its fully unrolled loops keep every row's queries in registers and
// spilled at 8 pairs).
template <int HD, int G>
constexpr int attn_rows() { return HD == 128 ? 16 / G : (G >= 4 ? 1 : 4 / G); }

// LDS of one attention workgroup: keys [dim][64 positions], values [64][dim],
// the rotated queries of its RB rows x G heads, the new position's key and
// value, the softmax weights [row][head][64 positions].
template <int HD, int G, int RB>
constexpr uint32_t attn_lds_bytes() {
  return static_cast<uint32_t>((2 * HD * kChunk + RB * G * HD + 2 * HD + RB * G * kChunk) * sizeof(float) + 16);
}

// One 4-wavefront workgroup per (chunk of 64 positions, KV head, row). The
// workgroup copies the chunk's keys and values into LDS with global-to-LDS
// loads, issued before any arithmetic; wavefront w then handles query heads
// w, w + 4, ... of the KV group: lane t scores position t0 + t, the chunk's
// softmax pieces (max m, sum l of exp(s - m), unnormalized output o) are
// published, and the last workgroup of the (row, KV head) combines all chunks
// of its query heads and resets the ticket.
// FUSED (one decode row): the query heads are normalized and rotated here from
// the raw projection, and the workgroup whose chunk holds the new position
// also normalizes/rotates its key, appends key and value to the cache
// (KvCache::append, cache.rs:96-125) and uses them for that position.
// Otherwise (prompt rows, RB per workgroup): the rotated queries of RB
// consecutive rows share the staged chunk; the ticket and the merge are per
// (row block, KV head).
template <int HD, int G, bool FUSED, int RB = 1>
__global__ __launch_bounds__(64 * kAttnWaves) void attn_kernel(AttnArgs a) {
  static_assert(!FUSED || RB == 1, "the fused decode path takes one row");
  constexpr int DPL = HD / 64;  // value dimensions per lane
  constexpr uint32_t P = HD / 2;
  constexpr int HPW = (G + kAttnWaves - 1) / kAttnWaves;  // query heads per wavefront
  extern __shared__ __attribute__((aligned(16))) float attn_lds[];
  float* ks = attn_lds;                  // [HD][64]
  float* vs = ks + HD * kChunk;          // [64][HD]
  float* qs = vs + kChunk * HD;          // [RB][G][HD]
  float* kn = qs + RB * G * HD;          // [HD]
  float* vn = kn + HD;                   // [HD]
  float* pe = vn + HD;                   // [RB][G][64]
  uint32_t* flag = reinterpret_cast<uint32_t*>(pe + RB * G * kChunk);
  const uint32_t c = blockIdx.x, g = blockIdx.y;
  const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  // rows rb0 .. rb0 + nrb - 1 of the batch (one row on the fused path)
  const uint32_t rb0 = blockIdx.z * RB;
  const uint32_t nrb = FUSED ? 1u : (a.nrows - rb0 < static_cast<uint32_t>(RB) ? a.nrows - rb0 : RB);
  const uint32_t r = rb0 + a.row0;
  const uint32_t pos = *a.len + r;        // the first row's position
  const uint32_t pos_last = pos + nrb - 1;
  const uint32_t t0 = c * kChunk;
  if (t0 > pos_last) return;  // chunks past every row's position take no part
  const uint32_t tp = pos - t0;  // the query position within this chunk (if < 64)
  const bool owner = FUSED && tp < kChunk;
  const bool act = lane < P;
  const uint32_t pl = act ? lane : 0;
  const float* row = a.qkv + static_cast<uint64_t>(r) * a.row_stride;

  // 1. prologue operands of this wavefront's query heads (and the new key/value)
  [[maybe_unused]] float qx0[HPW], qx1[HPW], nq0 = 0, nq1 = 0, cs = 0, sn = 0;
  [[maybe_unused]] float kx0 = 0, kx1 = 0, nk0 = 0, nk1 = 0, vx[DPL];
  if constexpr (FUSED) {
#pragma unroll
    for (int i = 0; i < HPW; ++i) {
      const uint32_t h = wave + kAttnWaves * i;
      const uint32_t hc = h < G ? h : 0;
      qx0[i] = row[(g * G + hc) * HD + pl];
      qx1[i] = row[(g * G + hc) * HD + pl + P];
    }
    nq0 = a.q_norm[pl];
    nq1 = a.q_norm[pl + P];
    cs = a.rope_cos[static_cast<uint64_t>(pos) * P + pl];
    sn = a.rope_sin[static_cast<uint64_t>(pos) * P + pl];
    if (owner && wave == 0) {
      const float* ksrc = row + a.heads * HD + g * HD;
      const float* vsrc = row + (a.heads + a.kv_heads) * HD + g * HD;
      kx0 = ksrc[pl];
      kx1 = ksrc[pl + P];
      nk0 = a.k_norm[pl];
      nk1 = a.k_norm[pl + P];
#pragma unroll
      for (int j = 0; j < DPL; ++j) vx[j] = vsrc[lane * DPL + j];
    }
  }
  // 2. the chunk into LDS, 1 KB per instruction, instructions dealt round robin
  // to the wavefronts: keys rows 4i..4i+3 (64 positions each, rows cap apart),
  // values 256 contiguous floats
  {
    const float* kt = a.keys + static_cast<uint64_t>(g) * HD * a.cap + t0;
    const float* vchunk = a.values + (static_cast<uint64_t>(g) * a.cap + t0) * HD;
    const uint32_t kr = lane >> 4, kc = (lane & 15) * 4;
#pragma unroll
    for (int i = static_cast<int>(wave); i < HD / 4; i += kAttnWaves) {
      __builtin_amdgcn_global_load_lds(
          kt + static_cast<uint64_t>(4 * i + kr) * a.cap + kc,
          (__attribute__((address_space(3))) void*)(ks + i * 256), 16, 0, 0);
      __builtin_amdgcn_global_load_lds(
          vchunk + i * 256 + lane * 4, (__attribute__((address_space(3))) void*)(vs + i * 256), 16, 0,
          0);
    }
  }
  // 3. rotated queries (and the new key/value) while the chunk is in flight
  if constexpr (FUSED) {
#pragma unroll
    for (int i = 0; i < HPW; ++i) {
      const uint32_t h = wave + kAttnWaves * i;
      const float2 o =
          norm_rope(qx0[i], qx1[i], nq0, nq1, cs, sn, static_cast<float>(HD), a.eps, act);
      if (h < G && act) {
        qs[h * HD + lane] = o.x;
        qs[h * HD + lane + P] = o.y;
      }
    }
    if (owner && wave == 0) {
      const float2 o = norm_rope(kx0, kx1, nk0, nk1, cs, sn, static_cast<float>(HD), a.eps, act);
      float* kw = a.keys_w + static_cast<uint64_t>(g) * HD * a.cap;
      float* vw = a.values_w + (static_cast<uint64_t>(g) * a.cap + pos) * HD;
      if (act) {
        kn[lane] = o.x;
        kn[lane + P] = o.y;
        kw[static_cast<uint64_t>(lane) * a.cap + pos] = o.x;
        kw[static_cast<uint64_t>(lane + P) * a.cap + pos] = o.y;
      }
#pragma unroll
      for (int j = 0; j < DPL; ++j) {
        vn[lane * DPL + j] = vx[j];
        vw[lane * DPL + j] = vx[j];
      }
    }
  } else {
    for (uint32_t i = tid; i < RB * G * HD; i += 64 * kAttnWaves) {
      const uint32_t rr = i / (G * HD), j = i % (G * HD);
      qs[i] = rr < nrb ? a.q[(static_cast<uint64_t>(r + rr) * a.heads + g * G) * HD + j] : 0.0f;
    }
  }
  __syncthreads();  // LDS: queries, new key/value, and the DMA'd chunk (vmcnt drained)
  if (owner) {
    // the new position's key and value replace the chunk's stale copies
    for (uint32_t d = tid; d < HD; d += 64 * kAttnWaves) {
      ks[d * kChunk + tp] = kn[d];
      vs[tp * HD + d] = vn[d];
    }
    __syncthreads();
  }

  // 4. this wavefront's heads for every row of the block at once (each key
  // and value read from LDS serves all RB rows): scores (lane t: position
  // t0 + t; four partial sums over the dimensions), softmax pieces, value
  // sums. Positions past a row's query get weight 0; the cache holds finite
  // values there (zeroed at creation, earlier tokens after a reset), so their
  // products vanish. Rows past the block or before the chunk are not stored.
  float s[RB][HPW];
  {
    float sp[RB][HPW][4];
#pragma unroll
    for (int rr = 0; rr < RB; ++rr)
#pragma unroll
      for (int i = 0; i < HPW; ++i)
#pragma unroll
        for (int u = 0; u < 4; ++u) sp[rr][i][u] = 0.0f;
#pragma unroll 2
    for (int d0 = 0; d0 < HD; d0 += 32) {
      float kv[32];
#pragma unroll
      for (int u = 0; u < 32; ++u) kv[u] = ks[(d0 + u) * kChunk + lane];
#pragma unroll
      for (int rr = 0; rr < RB; ++rr)
#pragma unroll
        for (int i = 0; i < HPW; ++i) {
          const uint32_t h = wave + kAttnWaves * i;
          const float4* qv = reinterpret_cast<const float4*>(qs + (rr * G + (h < G ? h : 0)) * HD + d0);
#pragma unroll
          for (int u4 = 0; u4 < 8; ++u4) {
            const float4 q4 = qv[u4];
            sp[rr][i][0] = fmaf(q4.x, kv[4 * u4], sp[rr][i][0]);
            sp[rr][i][1] = fmaf(q4.y, kv[4 * u4 + 1], sp[rr][i][1]);
            sp[rr][i][2] = fmaf(q4.z, kv[4 * u4 + 2], sp[rr][i][2]);
            sp[rr][i][3] = fmaf(q4.w, kv[4 * u4 + 3], sp[rr][i][3]);
          }
        }
    }
#pragma unroll
    for (int rr = 0; rr < RB; ++rr)
#pragma unroll
      for (int i = 0; i < HPW; ++i) s[rr][i] = (sp[rr][i][0] + sp[rr][i][1]) + (sp[rr][i][2] + sp[rr][i][3]);
  }
  float m[RB][HPW], l[RB][HPW];
#pragma unroll
  for (int rr = 0; rr < RB; ++rr) {
    const bool valid = t0 + lane <= pos + rr;
#pragma unroll
    for (int i = 0; i < HPW; ++i) {
      const uint32_t h = wave + kAttnWaves * i;
      const float sc = valid ? s[rr][i] * a.scale : -INFINITY;
      m[rr][i] = wave_max(sc);
      const float e = valid ? expf(sc - m[rr][i]) : 0.0f;
      l[rr][i] = wave_sum(e);
      if (h < G) pe[(rr * G + h) * kChunk + lane] = e;  // read back by this wavefront only
    }
  }
  float acc[RB][HPW][DPL];
#pragma unroll
  for (int rr = 0; rr < RB; ++rr)
#pragma unroll
    for (int i = 0; i < HPW; ++i)
#pragma unroll
      for (int j = 0; j < DPL; ++j) acc[rr][i][j] = 0.0f;
  // all 64 positions: the weights come back from LDS four at a time (the same
  // address for every lane), lane l sums value dimensions l*DPL .. l*DPL+DPL-1
#pragma unroll 4
  for (int t4 = 0; t4 < static_cast<int>(kChunk) / 4; ++t4) {
    float v[4][DPL];
#pragma unroll
    for (int u = 0; u < 4; ++u)
#pragma unroll
      for (int j = 0; j < DPL; ++j) v[u][j] = vs[(4 * t4 + u) * HD + lane * DPL + j];
#pragma unroll
    for (int rr = 0; rr < RB; ++rr)
#pragma unroll
      for (int i = 0; i < HPW; ++i) {
        const uint32_t h = wave + kAttnWaves * i;
        const float4 w4 = reinterpret_cast<const float4*>(pe + (rr * G + (h < G ? h : 0)) * kChunk)[t4];
        const float wt[4] = {w4.x, w4.y, w4.z, w4.w};
#pragma unroll
        for (int u = 0; u < 4; ++u)
#pragma unroll
          for (int j = 0; j < DPL; ++j) acc[rr][i][j] = fmaf(wt[u], v[u][j], acc[rr][i][j]);
      }
  }
#pragma unroll
  for (int rr = 0; rr < RB; ++rr) {
    if (static_cast<uint32_t>(rr) >= nrb || t0 > pos + rr) continue;
#pragma unroll
    for (int i = 0; i < HPW; ++i) {
      const uint32_t h = wave + kAttnWaves * i;
      if (h >= G) continue;
      const uint64_t idx = (static_cast<uint64_t>(rb0 + rr) * a.heads + g * G + h) * a.chunks + c;
      if (lane == 0) {
        store_coherent(a.pm + idx, m[rr][i]);
        store_coherent(a.pl + idx, l[rr][i]);
      }
#pragma unroll
      for (int j = 0; j < DPL; ++j) store_coherent(a.po + idx * HD + lane * DPL + j, acc[rr][i][j]);
    }
  }

  // 5. the last workgroup of this (row block, KV head) combines its query heads
  const uint32_t nc = pos_last / kChunk + 1;
  __builtin_amdgcn_s_waitcnt(0);  // this thread's partial stores are complete
  __syncthreads();
  const uint64_t ticket = static_cast<uint64_t>(blockIdx.z) * a.kv_heads + g;
  if (tid == 0) *flag = atomicAdd(&a.tickets[ticket], 1u) == nc - 1 ? 1u : 0u;
  __syncthreads();
  if (*flag == 0) return;
  // Online combine over groups of 64 chunks: a group's maxima, sums and its
  // first 16 chunk outputs are loaded together (one round trip for up to 16
  // chunks), the running output and denominator are rescaled when the maximum
  // grows: out = sum_c e^(m_c - M) o_c / sum_c e^(m_c - M) l_c.
  for (uint32_t rr = 0; rr < nrb; ++rr)
#pragma unroll
  for (int i = 0; i < HPW; ++i) {
    const uint32_t hl = wave + kAttnWaves * i;
    if (hl >= G) continue;
    const uint32_t h = g * G + hl;
    const uint32_t ncr = (pos + rr) / kChunk + 1;  // chunks this row attends to
    const uint64_t base = (static_cast<uint64_t>(rb0 + rr) * a.heads + h) * a.chunks;
    float mx = -INFINITY, denom = 0.0f, out[DPL];
#pragma unroll
    for (int j = 0; j < DPL; ++j) out[j] = 0.0f;
    for (uint32_t c0 = 0; c0 < ncr; c0 += 64) {
      const uint32_t n = ncr - c0 < 64 ? ncr - c0 : 64;
      const bool have = lane < n;
      const float* o = a.po + (base + c0) * HD + lane * DPL;
      const float gm_l = have ? load_coherent(a.pm + base + c0 + lane) : -INFINITY;
      const float gl_l = have ? load_coherent(a.pl + base + c0 + lane) : 0.0f;
      float ov[16][DPL];
#pragma unroll
      for (int cc = 0; cc < 16; ++cc) {
        const uint32_t ci = static_cast<uint32_t>(cc) < n ? static_cast<uint32_t>(cc) : n - 1;
#pragma unroll
        for (int j = 0; j < DPL; ++j) ov[cc][j] = load_coherent(o + static_cast<uint64_t>(ci) * HD + j);
      }
      // every load above is issued before the maximum needs the first of them
      __builtin_amdgcn_sched_barrier(0);
      const float nm = fmaxf(mx, wave_max(gm_l));
      const float rs = expf(mx - nm);  // 0 on the first group (mx = -inf)
      const float f = have ? expf(gm_l - nm) : 0.0f;
      denom = denom * rs + wave_sum(f * gl_l);
#pragma unroll
      for (int j = 0; j < DPL; ++j) out[j] *= rs;
      mx = nm;
      for (uint32_t cb = 0; cb < n; cb += 16) {
        if (cb > 0) {
          // chunks past the first 16 of the group (contexts above 1024 positions)
#pragma unroll
          for (int cc = 0; cc < 16; ++cc) {
            const uint32_t ci = cb + cc < n ? cb + cc : n - 1;
#pragma unroll
            for (int j = 0; j < DPL; ++j) ov[cc][j] = load_coherent(o + static_cast<uint64_t>(ci) * HD + j);
          }
        }
        // indices past the group's last chunk re-read it with weight 0
#pragma unroll
        for (int cc = 0; cc < 16; ++cc) {
          const float fc = __int_as_float(
              __builtin_amdgcn_readlane(__float_as_int(f), static_cast<int>((cb + cc) & 63)));
          const float w = cb + cc < n ? fc : 0.0f;
#pragma unroll
          for (int j = 0; j < DPL; ++j) out[j] = fmaf(w, ov[cc][j], out[j]);
        }
      }
    }
    float* dst = a.out + (static_cast<uint64_t>(r + rr) * a.heads + h) * HD + lane * DPL;
#pragma unroll
    for (int j = 0; j < DPL; ++j) dst[j] = out[j] / denom;
  }
  if (tid == 0) atomicExch(&a.tickets[ticket], 0u);
}

// ------------------------------------------------- prompt attention (MFMA)
// Prompt rows of head_dim 128 on the f32 matrix cores
// (v_mfma_f32_16x16x4f32: f32 products, f32 sums, the same arithmetic class as
// the FMA kernel). One workgroup per (16 consecutive rows, KV head), one
// wavefront per query head of the group; the group's key/value chunks of 64
// positions are staged in LDS (double-buffered, 2 x 64 KB) and read by every
// wavefront. Per chunk, per 16-position tile:
//   S^T (16 positions x 16 rows) = K (positions x 128) . Q^T: A = K from LDS
//     (lane l: position l % 16, dimension 4 s + l / 16), B = Q^T from 32
//     registers; lane l ends with row l % 16, positions 4 (l / 16) + i;
//   online softmax per row (the 4 lanes of a row exchange by shuffles);
//   O^T (128 x 16 rows) += V^T . P^T: the score registers are the B operand
//     as they stand (k-step i pairs lane group j with position 4 j + i, and
//     the value operand is loaded for the same positions), so P needs no
//     transpose; output tile dt row r holds dimension 8 r + dt, which makes a
//     lane's 8 value operands of one k-step contiguous (two 16-byte reads) and
//     its 32 outputs contiguous.
// LDS rows are rotated (key row d by 16 (d % 4) positions, value row p by
// 16 ((p / 4) % 4) dimensions) so neither read pattern has bank conflicts.
// Masked positions (past a row's position) get zero weight; the cache is
// zeroed at creation, so positions never written hold finite values.
constexpr uint32_t kMmaChunk = 64;
constexpr uint32_t kMmaLds = 2 * 2 * 128 * kMmaChunk * 4;  // 2 buffers x (keys + values)

template <int G>
__global__ __launch_bounds__(64 * G) void attn_mfma_kernel(AttnArgs a) {
  constexpr uint32_t HD = 128, C = kMmaChunk;
  typedef float f4v __attribute__((ext_vector_type(4)));
  typedef __attribute__((address_space(3))) void* lds_ptr;
  extern __shared__ __attribute__((aligned(16))) float mma_lds[];
  const uint32_t g = blockIdx.y, lane = threadIdx.x & 63;
  const uint32_t w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const uint32_t h = g * G + w;
  const uint32_t rb = blockIdx.x * 16;  // first row of the block within the call
  const uint32_t nr = a.nrows - rb < 16u ? a.nrows - rb : 16u;
  const uint32_t pos0 = *a.len + rb;  // position of the block's first row
  const uint32_t nchunks = (pos0 + nr - 1) / C + 1;
  const uint32_t myrow = lane & 15, jg = lane >> 4;
  const bool rowok = myrow < nr;
  const uint32_t mypos = pos0 + myrow;
  const uint32_t ld = a.heads * HD;

  // Q^T operand: lane l holds Q[row l % 16][dimension 4 s + l / 16], s = 0..31
  float qreg[32];
  {
    const float* q = a.q + static_cast<uint64_t>(rb + (rowok ? myrow : 0)) * ld + h * HD + jg;
#pragma unroll
    for (int s = 0; s < 32; ++s) qreg[s] = q[4 * s];
  }
  const float* kg = a.keys + static_cast<uint64_t>(g) * HD * a.cap;
  const float* vg = a.values + static_cast<uint64_t>(g) * a.cap * HD;
  // chunk c into buffer b: keys [128][64] and values [64][128], rotated rows;
  // 16-byte global-to-LDS copies (4 key rows or 2 value rows each) dealt
  // round robin to the wavefronts
  auto copy_chunk = [&](uint32_t c, uint32_t b) {
    float* ks = mma_lds + b * 2 * HD * C;
    float* vs = ks + HD * C;
    const uint32_t t0 = c * C;
    for (uint32_t i = w; i < HD / 4; i += G) {
      const uint32_t jj = lane >> 4, qq = lane & 15;
      const float* src = kg + static_cast<uint64_t>(4 * i + jj) * a.cap + t0 + 4 * ((qq - 4 * jj) & 15);
      __builtin_amdgcn_global_load_lds(src, (lds_ptr)(ks + i * 256), 16, 0, 0);
    }
    for (uint32_t i = w; i < C / 2; i += G) {
      const uint32_t p = 2 * i + (lane >> 5), qq = lane & 31;
      const float* src = vg + static_cast<uint64_t>(t0 + p) * HD + ((4 * qq - 16 * ((p >> 2) & 3)) & 127);
      __builtin_amdgcn_global_load_lds(src, (lds_ptr)(vs + i * 256), 16, 0, 0);
    }
  };

  f4v o[8];
#pragma unroll
  for (int dt = 0; dt < 8; ++dt) o[dt] = f4v{0, 0, 0, 0};
  float m = -INFINITY, lsum = 0.0f;

  copy_chunk(0, 0);
  for (uint32_t c = 0; c < nchunks; ++c) {
    const uint32_t b = c & 1;
    // chunk c landed (this wavefront's copies, then everyone's), and every
    // wavefront is done with buffer b ^ 1 (chunk c - 1)
    __builtin_amdgcn_s_waitcnt(0);
    __builtin_amdgcn_s_barrier();
    if (c + 1 < nchunks) copy_chunk(c + 1, b ^ 1);
    const float* ks = mma_lds + b * 2 * HD * C;
    const float* vs = ks + HD * C;
    const uint32_t t0 = c * C;

    f4v sc[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      f4v acc = f4v{0, 0, 0, 0};
      // key row d = 4 s + jg (d % 4 = jg): position p sits at (p + 16 jg) % 64
      const float* kr = ks + jg * C + ((16 * t + myrow + 16 * jg) & (C - 1));
#pragma unroll
      for (int s = 0; s < 32; ++s) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(kr[4 * s * C], qreg[s], acc, 0, 0, 0);
      sc[t] = acc;
    }
    // scale and mask, then the online softmax of row myrow over this chunk
    float mx = -INFINITY;
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint32_t p = t0 + 16 * t + 4 * jg + i;
        const float v = (rowok && p <= mypos) ? sc[t][i] * a.scale : -INFINITY;
        sc[t][i] = v;
        mx = fmaxf(mx, v);
      }
    mx = fmaxf(mx, __shfl_xor(mx, 16));
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    const float mn = fmaxf(m, mx);
    const float f = mn == -INFINITY ? 1.0f : expf(m - mn);  // 0 while m = -inf
    m = mn;
    lsum *= f;
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) o[dt] *= f;
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float e = sc[t][i] == -INFINITY ? 0.0f : expf(sc[t][i] - mn);
        sc[t][i] = e;
        lsum += e;
      }
    // O^T += V^T . P^T: k-step i of tile t takes position 16 t + 4 jg + i
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint32_t p = 16 * t + 4 * jg + i;  // (p / 4) % 4 = jg
        const f4v* vr = reinterpret_cast<const f4v*>(vs + p * HD + ((8 * myrow + 16 * jg) & (HD - 1)));
        const f4v v0 = vr[0], v1 = vr[1];  // dimensions 8 myrow + 0..7
#pragma unroll
        for (int dt = 0; dt < 4; ++dt) o[dt] = __builtin_amdgcn_mfma_f32_16x16x4f32(v0[dt], sc[t][i], o[dt], 0, 0, 0);
#pragma unroll
        for (int dt = 0; dt < 4; ++dt)
          o[4 + dt] = __builtin_amdgcn_mfma_f32_16x16x4f32(v1[dt], sc[t][i], o[4 + dt], 0, 0, 0);
      }
  }
  lsum += __shfl_xor(lsum, 16);
  lsum += __shfl_xor(lsum, 32);
  if (!rowok) return;
  // lane l: row l % 16, dimensions 32 jg + 8 i + dt
  const float inv = 1.0f / lsum;
  float* out = a.out + static_cast<uint64_t>(rb + myrow) * ld + h * HD + 32 * jg;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    reinterpret_cast<f4v*>(out + 8 * i)[0] = f4v{o[0][i], o[1][i], o[2][i], o[3][i]} * inv;
    reinterpret_cast<f4v*>(out + 8 * i)[1] = f4v{o[4][i], o[5][i], o[6][i], o[7][i]} * inv;
  }
}

// --------------------------------------------------------------- SiLU*up
// backends/cpu/src/backend.rs:224-237: gate / (1 + exp(-gate)) * up from the
// fused gate|up output row: the two halves (group 0) or, for an interleaved
// image, groups of `group` gate outputs each followed by the same up outputs.
__global__ __launch_bounds__(256) void silu_mul_kernel(const float* __restrict__ gu,
                                                       float* __restrict__ out, uint32_t inter,
                                                       uint64_t total, uint32_t group) {
  const uint64_t i = static_cast<uint64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i >= total) return;
  const uint64_t r = i / inter, j = i % inter;
  const uint64_t gi = group ? (j / group) * 2 * group + j % group : j;
  const uint64_t ui = group ? gi + group : inter + j;
  const float g = gu[r * 2 * inter + gi];
  const float u = gu[r * 2 * inter + ui];
  out[i] = g / (1.0f + expf(-g)) * u;
}

// ----------------------------------------------------------------- argmax
// generation.rs:58-76: the first index of the largest logit; a non-finite
// logit is an error (flagged, reported by the host).
__device__ __forceinline__ void better(float& bv, uint32_t& bi, float v, uint32_t i) {
  if (v > bv || (v == bv && i < bi)) {
    bv = v;
    bi = i;
  }
}

__global__ __launch_bounds__(256) void argmax_partial_kernel(const float* __restrict__ logits,
                                                             uint32_t n, float* __restrict__ pv,
                                                             uint32_t* __restrict__ pi,
                                                             int32_t* __restrict__ bad) {
  __shared__ float sv[256];
  __shared__ uint32_t si[256];
  const uint32_t per = (n + kArgBlocks - 1) / kArgBlocks;
  const uint32_t b0 = blockIdx.x * per;
  const uint32_t b1 = b0 + per < n ? b0 + per : n;
  float bv = -INFINITY;
  uint32_t bi = 0xffffffffu;
  bool nonfinite = false;
  for (uint32_t i = b0 + threadIdx.x; i < b1; i += 256) {
    const float v = logits[i];
    nonfinite |= !isfinite(v);
    better(bv, bi, v, i);
  }
  if (nonfinite) *bad = 1;
  sv[threadIdx.x] = bv;
  si[threadIdx.x] = bi;
  __syncthreads();
  for (uint32_t s = 128; s > 0; s >>= 1) {
    if (threadIdx.x < s) {
      float v = sv[threadIdx.x];
      uint32_t i = si[threadIdx.x];
      better(v, i, sv[threadIdx.x + s], si[threadIdx.x + s]);
      sv[threadIdx.x] = v;
      si[threadIdx.x] = i;
    }
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    pv[blockIdx.x] = sv[0];
    pi[blockIdx.x] = si[0];
  }
}

// Reduce the partials, store the token at tok[len + rows] and advance len.
__global__ __launch_bounds__(256) void argmax_final_kernel(const float* __restrict__ pv,
                                                           const uint32_t* __restrict__ pi,
                                                           int32_t* __restrict__ tok,
                                                           uint32_t* __restrict__ len,
                                                           uint32_t rows) {
  __shared__ float sv[kArgBlocks];
  __shared__ uint32_t si[kArgBlocks];
  sv[threadIdx.x] = pv[threadIdx.x];
  si[threadIdx.x] = pi[threadIdx.x];
  __syncthreads();
  for (uint32_t s = kArgBlocks / 2; s > 0; s >>= 1) {
    if (threadIdx.x < s) {
      float v = sv[threadIdx.x];
      uint32_t i = si[threadIdx.x];
      better(v, i, sv[threadIdx.x + s], si[threadIdx.x + s]);
      sv[threadIdx.x] = v;
      si[threadIdx.x] = i;
    }
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    const uint32_t next = *len + rows;
    tok[next] = static_cast<int32_t>(si[0] == 0xffffffffu ? 0u : si[0]);
    *len = next;
  }
}

__global__ void advance_kernel(uint32_t* len, uint32_t rows) {
  if (threadIdx.x == 0) *len = *len + rows;
}

// ------------------------------------------------------------------ host

std::atomic<uint64_t> g_next_model_id{1};

struct Linear {
  qi_hip_weights* w = nullptr;
  uint64_t k = 0, n = 0;
  uint32_t pair_group = 0;  // two fused parts: 0 concatenated, else interleaved in groups of this many rows
};

struct Layer {
  float* norms = nullptr;  // input | q | k | post (device)
  Linear qkv, o, gate_up, down;
  bool set = false;
};

size_t logical_bytes(int32_t qtype) {
  switch (qtype) {
    case QI_HIP_F32: return 4;
    case QI_HIP_Q8_0: return sizeof(qi_hip_q8_0_block);
    case QI_HIP_Q4_0: return sizeof(qi_hip_q4_0_block);
    case QI_HIP_Q4_K: return sizeof(qi_hip_q4_k_block);
    case QI_HIP_Q5_K: return sizeof(qi_hip_q5_k_block);
    case QI_HIP_Q6_K: return sizeof(qi_hip_q6_k_block);
    default: return 0;
  }
}

uint32_t elems_per_block(int32_t qtype) {
  return qtype == QI_HIP_F32 ? 1u : qi::block_elems(qtype);
}

}  // namespace

struct qi_hip_qwen3 {
  qi_hip_ctx* ctx = nullptr;
  qi_hip_qwen3_config cfg{};
  int32_t mode = QI_HIP_MODE_F32;  // token-identical to the CPU run; AUTO trades that for prompt speed
  uint64_t id = 0;
  std::vector<Layer> layers;
  float* embedding = nullptr;
  float* final_norm = nullptr;
  Linear head;
  float* rope_cos = nullptr;
  float* rope_sin = nullptr;
  // activations for up to kMaxRows rows
  float *h = nullptr, *x = nullptr, *qkv = nullptr, *q = nullptr, *att = nullptr, *y = nullptr;
  float *gu = nullptr, *act = nullptr, *logits = nullptr, *apv = nullptr;
  uint32_t* api = nullptr;
  int32_t* bad = nullptr;
  hipEvent_t ev[3] = {nullptr, nullptr, nullptr};
  qi_hip_qwen3_timing timing{};
  bool eager = false;    // QI_HIP_QWEN3_EAGER=1: launch decode steps one by one (no graph)
  bool unfused = false;  // QI_HIP_QWEN3_UNFUSED=1: separate SiLU and norm kernels (decode and prompt)
  bool attn_fma = false;  // QI_HIP_QWEN3_ATTN_FMA=1: prompt attention on the FMA kernel (head_dim 128)
};

struct qi_hip_kv_cache {
  qi_hip_ctx* ctx = nullptr;
  uint32_t layers = 0, max_seq = 0, kv_heads = 0, head_dim = 0, cap = 0;
  float* keys = nullptr;    // [layer][kv_head][dim][cap]
  float* values = nullptr;  // [layer][kv_head][cap][dim]
  int32_t* tok = nullptr;   // [cap + 1]
  uint32_t* len_dev = nullptr;
  uint64_t len = 0;         // host mirror of *len_dev
  // attention partials for row batches of `rb` rows
  float *pm = nullptr, *pl = nullptr, *po = nullptr;
  uint32_t* tickets = nullptr;  // [rb][kv head], zero between launches
  uint32_t rb = 0, heads = 0;
  hipGraphExec_t exec = nullptr;
  uint64_t graph_model = 0, graph_ws = 0;
};

namespace {

void dev_free(void* p) {
  if (p) (void)hipFree(p);
}

qi_hip_status dev_alloc(void** p, uint64_t bytes, const char* what) {
  *p = nullptr;
  hipError_t e = hipMalloc(p, bytes ? bytes : 16);
  if (e != hipSuccess) return hip_fail(e, what);
  return QI_HIP_OK;
}

template <class T>
qi_hip_status dev_alloc_t(T** p, uint64_t count, const char* what) {
  return dev_alloc(reinterpret_cast<void**>(p), count * sizeof(T), what);
}

qi_hip_status upload(void* dst, const void* src, uint64_t bytes, hipStream_t st) {
  QI_HIP_TRY(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, st), "upload");
  QI_HIP_TRY(hipStreamSynchronize(st), "upload");
  return QI_HIP_OK;
}

// Concatenate linear weights along N (the output dimension) into one logical
// buffer and upload it as one image. Output rows: each part is [N_i][K/bs]
// blocks, so the parts follow one another. Row-major: each part is
// [K][N_i/bs] blocks, so row k of the result is row k of every part in turn.
// `interleave` (two equal output-rows parts): rows alternate in groups of that
// many, part 0's group then part 1's (a 16-output tile then holds 8 rows of
// each, for the GEMV epilogue that pairs them).
qi_hip_status make_linear(qi_hip_ctx* c, const qi_hip_linear_weight* const* parts, int count,
                          uint64_t k, const uint64_t* ns, const char* name, Linear* out,
                          uint32_t interleave = 0) {
  const int32_t qtype = parts[0]->qtype, layout = parts[0]->layout;
  const size_t lb = logical_bytes(qtype);
  if (lb == 0) return fail(QI_HIP_INVALID_INPUT, std::string(name) + ": unknown weight type");
  const uint32_t bs = elems_per_block(qtype);
  uint64_t n = 0;
  for (int i = 0; i < count; ++i) {
    if (parts[i]->qtype != qtype || parts[i]->layout != layout)
      return fail(QI_HIP_UNSUPPORTED,
                  std::string(name) + ": fused projections must share weight type and layout");
    if (parts[i]->data == nullptr) return fail(QI_HIP_INVALID_INPUT, std::string(name) + ": null weight");
    n += ns[i];
  }
  const bool rows = layout == QI_HIP_LAYOUT_OUTPUT_ROWS;
  for (int i = 0; i < count; ++i) {
    const uint64_t per = rows ? ns[i] * (k / bs) : k * (ns[i] / bs);
    if ((rows ? k % bs : ns[i] % bs) != 0 || parts[i]->count != per)
      return fail(QI_HIP_INVALID_INPUT, std::string(name) + ": block count does not match its shape");
  }
  std::vector<uint8_t> joined;
  const void* blocks = parts[0]->data;
  uint64_t total = parts[0]->count;
  const bool pair = interleave > 0 && count == 2 && rows && ns[0] == ns[1] && ns[0] % interleave == 0;
  if (count > 1) {
    total = 0;
    for (int i = 0; i < count; ++i) total += parts[i]->count;
    joined.resize(total * lb);
    uint8_t* dst = joined.data();
    if (pair) {
      const uint64_t grp = static_cast<uint64_t>(interleave) * (k / bs) * lb;  // bytes of one row group
      for (uint64_t r = 0; r < ns[0]; r += interleave) {
        for (int i = 0; i < 2; ++i) {
          memcpy(dst, static_cast<const uint8_t*>(parts[i]->data) + r / interleave * grp, grp);
          dst += grp;
        }
      }
    } else if (rows) {
      for (int i = 0; i < count; ++i) {
        memcpy(dst, parts[i]->data, parts[i]->count * lb);
        dst += parts[i]->count * lb;
      }
    } else {
      for (uint64_t kk = 0; kk < k; ++kk) {
        for (int i = 0; i < count; ++i) {
          const uint64_t row = ns[i] / bs * lb;
          memcpy(dst, static_cast<const uint8_t*>(parts[i]->data) + kk * row, row);
          dst += row;
        }
      }
    }
    blocks = joined.data();
  }
  qi::Image im;
  const char* why = "";
  qi_hip_status s = qi::plan_image(qtype, layout, k, n, blocks, total, &im, &why);
  if (s != QI_HIP_OK) return fail(s, std::string(name) + ": " + why);
  s = qi_abi::create_weights_locked(c, im, blocks, &out->w);
  if (s != QI_HIP_OK) return s;
  out->k = k;
  out->n = n;
  out->pair_group = pair ? interleave : 0;
  return QI_HIP_OK;
}

void free_linear(Linear* l) {
  if (l->w) qi_abi::free_weights_locked(l->w);
  l->w = nullptr;
}

bool model_ready(const qi_hip_qwen3* m) {
  if (!m->embedding || !m->final_norm || !m->head.w) return false;
  for (const Layer& l : m->layers)
    if (!l.set) return false;
  return true;
}

qi_hip_status linear(qi_hip_qwen3* m, const Linear& l, const float* x, uint32_t rows, float* y) {
  return qi_abi::run_linear(m->ctx, l.w, x, rows, y, m->mode, m->ctx->stream);
}

// Launch the attention of `rows` query rows (positions len .. len+rows-1).
// One row (a decode step) takes the fused path: query/key norms, RoPE and the
// cache append happen inside the attention kernel. Several rows need the keys
// of earlier rows of the same call, so they are appended by
// qk_norm_rope_kernel first.
qi_hip_status attention(qi_hip_qwen3* m, qi_hip_kv_cache* c, uint32_t layer, uint32_t rows) {
  const qi_hip_qwen3_config& k = m->cfg;
  const Layer& L = m->layers[layer];
  const uint32_t H = k.hidden_size, hd = k.head_dim;
  const uint32_t group = k.num_attention_heads / k.num_key_value_heads;
  const uint64_t lay = static_cast<uint64_t>(k.num_key_value_heads) * hd * c->cap;
  hipStream_t st = m->ctx->stream;
  const bool fused = rows == 1;
  if (!fused) {
    HeadArgs ha;
    ha.qkv = m->qkv;
    ha.row_stride = (k.num_attention_heads + 2 * k.num_key_value_heads) * hd;
    ha.heads = k.num_attention_heads;
    ha.kv_heads = k.num_key_value_heads;
    ha.head_dim = hd;
    ha.q_norm = L.norms + H;
    ha.k_norm = L.norms + H + hd;
    ha.eps = k.rms_norm_eps;
    ha.rope_cos = m->rope_cos;
    ha.rope_sin = m->rope_sin;
    ha.len = c->len_dev;
    ha.q_out = m->q;
    ha.keys = c->keys + layer * lay;
    ha.values = c->values + layer * lay;
    ha.cap = c->cap;
    hipLaunchKernelGGL(qk_norm_rope_kernel, dim3(ha.heads + ha.kv_heads, rows), dim3(64), 0, st, ha);
  }
  AttnArgs a;
  a.q = m->q;
  a.keys = c->keys + layer * lay;
  a.values = c->values + layer * lay;
  a.len = c->len_dev;
  a.pm = c->pm;
  a.pl = c->pl;
  a.po = c->po;
  a.heads = k.num_attention_heads;
  a.kv_heads = k.num_key_value_heads;
  a.cap = c->cap;
  a.chunks = c->cap / kChunk;
  a.row0 = 0;
  a.scale = 1.0f / sqrtf(static_cast<float>(hd));
  a.out = m->att;
  a.qkv = m->qkv;
  a.row_stride = (k.num_attention_heads + 2 * k.num_key_value_heads) * hd;
  a.q_norm = L.norms + H;
  a.k_norm = L.norms + H + hd;
  a.eps = k.rms_norm_eps;
  a.rope_cos = m->rope_cos;
  a.rope_sin = m->rope_sin;
  a.keys_w = c->keys + layer * lay;
  a.values_w = c->values + layer * lay;
  a.tickets = c->tickets;
  if (!fused && hd == 128 && !m->attn_fma) {
    // prompt rows on the matrix cores: every row in one launch
    a.row0 = 0;
    a.nrows = rows;
    const dim3 grid((rows + 15) / 16, a.kv_heads);
    switch (group) {
      case 1: hipLaunchKernelGGL(attn_mfma_kernel<1>, grid, dim3(64), kMmaLds, st, a); break;
      case 2: hipLaunchKernelGGL(attn_mfma_kernel<2>, grid, dim3(128), kMmaLds, st, a); break;
      case 4: hipLaunchKernelGGL(attn_mfma_kernel<4>, grid, dim3(256), kMmaLds, st, a); break;
      case 8: hipLaunchKernelGGL(attn_mfma_kernel<8>, grid, dim3(512), kMmaLds, st, a); break;
      default: return fail(QI_HIP_UNSUPPORTED, "attention supports 1/2/4/8 query heads per KV head");
    }
    QI_HIP_TRY(hipGetLastError(), "launch attention");
    return QI_HIP_OK;
  }
  for (uint32_t r0 = 0; r0 < rows; r0 += c->rb) {
    const uint32_t nr = rows - r0 < c->rb ? rows - r0 : c->rb;
    AttnArgs b = a;
    b.row0 = r0;
    b.nrows = nr;
#define QI_ATTN(HD_, G_)                                                                         \
  if (hd == HD_ && group == G_) {                                                                \
    constexpr int RB_ = attn_rows<HD_, G_>();                                                         \
    constexpr uint32_t one_ = attn_lds_bytes<HD_, G_, 1>();                                      \
    constexpr uint32_t blk_ = attn_lds_bytes<HD_, G_, RB_>();                                    \
    if (fused)                                                                                   \
      hipLaunchKernelGGL((attn_kernel<HD_, G_, true>), dim3(a.chunks, a.kv_heads, nr),           \
                         dim3(64 * kAttnWaves), one_, st, b);                                    \
    else                                                                                         \
      hipLaunchKernelGGL((attn_kernel<HD_, G_, false, RB_>),                                     \
                         dim3(a.chunks, a.kv_heads, (nr + RB_ - 1) / RB_), dim3(64 * kAttnWaves), \
                         blk_, st, b);                                                           \
  } else
    QI_ATTN(128, 1) QI_ATTN(128, 2) QI_ATTN(128, 4) QI_ATTN(128, 8)
    QI_ATTN(64, 1) QI_ATTN(64, 2) QI_ATTN(64, 4) QI_ATTN(64, 8)
    return fail(QI_HIP_UNSUPPORTED, "attention supports head_dim 64/128 and 1/2/4/8 query heads per KV head");
#undef QI_ATTN
    QI_HIP_TRY(hipGetLastError(), "launch attention");
  }
  return QI_HIP_OK;
}

// Attention workgroups of head_dim 128 hold more than 64 KB of LDS: raise the
// kernels' dynamic LDS limit once, outside any stream capture.
template <int HD, int G>
hipError_t attn_set_lds() {
  hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(attn_kernel<HD, G, true>),
                                     hipFuncAttributeMaxDynamicSharedMemorySize,
                                     static_cast<int>(attn_lds_bytes<HD, G, 1>()));
  if (e == hipSuccess)
    e = hipFuncSetAttribute(reinterpret_cast<const void*>(attn_kernel<HD, G, false, attn_rows<HD, G>()>),
                            hipFuncAttributeMaxDynamicSharedMemorySize,
                            static_cast<int>(attn_lds_bytes<HD, G, attn_rows<HD, G>()>()));
  if constexpr (HD == 128) {
    if (e == hipSuccess)
      e = hipFuncSetAttribute(reinterpret_cast<const void*>(attn_mfma_kernel<G>),
                              hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(kMmaLds));
  }
  return e;
}

hipError_t attn_prepare(uint32_t hd, uint32_t group) {
  if (hd == 128) {
    switch (group) {
      case 1: return attn_set_lds<128, 1>();
      case 2: return attn_set_lds<128, 2>();
      case 4: return attn_set_lds<128, 4>();
      case 8: return attn_set_lds<128, 8>();
    }
  }
  return hipSuccess;  // head_dim 64 stays within 64 KB
}

// x = RMSNorm(h (+ y)) for `rows` rows (h updated in place; add = false: the
// residual add is already in h); the row is held in registers.
qi_hip_status residual_norm(qi_hip_qwen3* m, bool embed, const qi_hip_kv_cache* c,
                            uint32_t rows, const float* w, bool add = true) {
  const uint32_t H = m->cfg.hidden_size;
  const uint32_t nv = (H / 4 + 255) / 256;
  hipStream_t st = m->ctx->stream;
  const float eps = m->cfg.rms_norm_eps;
#define QI_NORM(NV_)                                                                         \
  if (nv <= NV_) {                                                                           \
    if (embed)                                                                               \
      hipLaunchKernelGGL((residual_norm_kernel<true, NV_>), dim3(rows), dim3(256), 0, st,    \
                         m->h, nullptr, m->embedding, c->tok, c->len_dev, m->x, w, H, eps);  \
    else                                                                                     \
      hipLaunchKernelGGL((residual_norm_kernel<false, NV_>), dim3(rows), dim3(256), 0, st,   \
                         m->h, add ? m->y : nullptr, nullptr, nullptr, nullptr, m->x, w, H, eps); \
  } else
  QI_NORM(1) QI_NORM(2) QI_NORM(4) QI_NORM(8) QI_NORM(16)
  return fail(QI_HIP_UNSUPPORTED, "hidden_size above 16384");
#undef QI_NORM
  QI_HIP_TRY(hipGetLastError(), "launch norm");
  return QI_HIP_OK;
}

// A projection can take part in the decode fusions with the matrix-core GEMV
// (F32/AUTO modes, a tiled f16-scale image).
bool gemv_fusable(const qi_hip_qwen3* m, const Linear& l) {
  if (m->unfused || (m->mode != QI_HIP_MODE_AUTO && m->mode != QI_HIP_MODE_F32)) return false;
  const qi::Image& im = l.w->im;
  return im.tiled && !im.wide && qi::gemv_mfma_supported(im.qtype, im.layout, im.k);
}

// One-row matrix-core GEMV of the decoder: activation source xs (plain x,
// or kXNorm: x = RMSNorm(h) * w with the norm's 1/rms applied to the outputs);
// with `radd`, the residual add on the outputs (out may be radd); with
// `pairs`, SiLU(gate) * up of an interleaved gate|up image (I outputs).
qi_hip_status fused_linear(qi_hip_qwen3* m, const Linear& l, int xs, const float* x, const float* w,
                           float* out, const float* radd, bool pairs = false) {
  const qi::Image& im = l.w->im;
  qi::GemvMfmaArgs ga{qi::make_view(im, l.w->dev), x, out, 1};
  ga.xs = xs;
  if (xs == qi::kXNorm) {
    ga.hres = m->h;
    ga.nw = w;
    ga.eps = m->cfg.rms_norm_eps;
  }
  ga.radd = radd;
  ga.silu_pairs = pairs;
  const int split = m->ctx->gemv_split > 0 ? m->ctx->gemv_split : qi::gemv_mfma_split(im.k, im.n);
  QI_HIP_TRY(qi::launch_gemv_mfma(im.qtype, false, split, ga, m->ctx->stream), "launch fused gemv");
  return QI_HIP_OK;
}

// A decode step folds the residual adds into the o and down GEMVs (written
// into h), the RMSNorms into the activation prep of the q|k|v (from layer 1)
// and gate|up GEMVs, and SiLU(gate) * up into the gate|up GEMV epilogue, when
// all four have matrix-core images and gate|up is interleaved by 8.
bool decode_fusable(const qi_hip_qwen3* m) {
  if (m->unfused) return false;
  for (const Layer& L : m->layers)
    if (!gemv_fusable(m, L.qkv) || !gemv_fusable(m, L.o) || !gemv_fusable(m, L.gate_up) ||
        !gemv_fusable(m, L.down) || L.gate_up.pair_group != 8 || L.gate_up.n % 16 != 0)
      return false;
  return true;
}

// Enqueue the forward of `rows` tokens tok[len .. len+rows) on the context
// stream. With `project`, the last row goes through the final norm, the LM
// head and the argmax (token stored at tok[len+rows]); len advances by rows.
qi_hip_status enqueue_forward(qi_hip_qwen3* m, qi_hip_kv_cache* c, uint32_t rows, bool project) {
  const qi_hip_qwen3_config& k = m->cfg;
  hipStream_t st = m->ctx->stream;
  const uint32_t H = k.hidden_size, I = k.intermediate_size, hd = k.head_dim;
  qi_hip_status s;
  if ((s = residual_norm(m, true, c, rows, m->layers[0].norms)) != QI_HIP_OK) return s;
  if (rows == 1 && decode_fusable(m)) {
    // decode step: the residual row h is updated in place by the o and down
    // GEMVs; q|k|v (from layer 1) and gate|up normalize it in their prep
    for (uint32_t l = 0; l < k.num_hidden_layers; ++l) {
      Layer& L = m->layers[l];
      if (l == 0) s = fused_linear(m, L.qkv, qi::kXPlain, m->x, nullptr, m->qkv, nullptr);
      else s = fused_linear(m, L.qkv, qi::kXNorm, nullptr, L.norms, m->qkv, nullptr);
      if (s != QI_HIP_OK) return s;
      if ((s = attention(m, c, l, 1)) != QI_HIP_OK) return s;
      if ((s = fused_linear(m, L.o, qi::kXPlain, m->att, nullptr, m->h, m->h)) != QI_HIP_OK) return s;
      if ((s = fused_linear(m, L.gate_up, qi::kXNorm, nullptr, L.norms + H + 2 * hd, m->act, nullptr,
                            true)) != QI_HIP_OK)
        return s;
      if ((s = fused_linear(m, L.down, qi::kXPlain, m->act, nullptr, m->h, m->h)) != QI_HIP_OK) return s;
    }
    if ((s = residual_norm(m, false, c, 1, m->final_norm, false)) != QI_HIP_OK) return s;
  } else {
    for (uint32_t l = 0; l < k.num_hidden_layers; ++l) {
      Layer& L = m->layers[l];
      if ((s = linear(m, L.qkv, m->x, rows, m->qkv)) != QI_HIP_OK) return s;
      if ((s = attention(m, c, l, rows)) != QI_HIP_OK) return s;
      if ((s = linear(m, L.o, m->att, rows, m->y)) != QI_HIP_OK) return s;
      if ((s = residual_norm(m, false, c, rows, L.norms + H + 2 * hd)) != QI_HIP_OK) return s;
      // SiLU(gate) * up in the GEMM epilogue when the layer runs as one
      // un-split GEMM over an image interleaved in groups of 8; else a pass
      bool silu_done = false;
      float* act = L.gate_up.pair_group == 8 && !m->unfused ? m->act : nullptr;
      if ((s = qi_abi::run_linear(m->ctx, L.gate_up.w, m->x, rows, m->gu, m->mode, st, act, &silu_done)) !=
          QI_HIP_OK)
        return s;
      if (!silu_done) {
        const uint64_t total = static_cast<uint64_t>(rows) * I;
        hipLaunchKernelGGL(silu_mul_kernel, dim3(static_cast<uint32_t>((total + 255) / 256)), dim3(256), 0, st,
                           m->gu, m->act, I, total, L.gate_up.pair_group);
      }
      if ((s = linear(m, L.down, m->act, rows, m->y)) != QI_HIP_OK) return s;
      const float* next = l + 1 < k.num_hidden_layers ? m->layers[l + 1].norms : m->final_norm;
      if ((s = residual_norm(m, false, c, rows, next)) != QI_HIP_OK) return s;
    }
  }
  if (project) {
    const float* last = m->x + static_cast<uint64_t>(rows - 1) * H;
    if ((s = linear(m, m->head, last, 1, m->logits)) != QI_HIP_OK) return s;
    hipLaunchKernelGGL(argmax_partial_kernel, dim3(kArgBlocks), dim3(256), 0, st, m->logits,
                       k.vocab_size, m->apv, m->api, m->bad);
    hipLaunchKernelGGL(argmax_final_kernel, dim3(1), dim3(kArgBlocks), 0, st, m->apv, m->api,
                       c->tok, c->len_dev, rows);
  } else {
    hipLaunchKernelGGL(advance_kernel, dim3(1), dim3(64), 0, st, c->len_dev, rows);
  }
  QI_HIP_TRY(hipGetLastError(), "launch decoder kernels");
  return QI_HIP_OK;
}

qi_hip_status check_pair(qi_hip_qwen3* m, qi_hip_kv_cache* c) {
  if (m == nullptr || c == nullptr) return fail(QI_HIP_INVALID_INPUT, "null model or cache");
  if (m->ctx != c->ctx) return fail(QI_HIP_INVALID_INPUT, "model and cache belong to different contexts");
  if (m->ctx->closed) return fail(QI_HIP_INVALID_INPUT, "context is closed");
  if (!model_ready(m)) return fail(QI_HIP_INVALID_INPUT, "Qwen3 model weights are not all set");
  // KvCache::validate_layout (cache.rs:67-94)
  if (c->layers != m->cfg.num_hidden_layers || c->kv_heads != m->cfg.num_key_value_heads ||
      c->head_dim != m->cfg.head_dim)
    return fail(QI_HIP_INVALID_INPUT, "KV cache layout differs from model");
  return QI_HIP_OK;
}

// Size the cache's attention partials for this model's head count.
qi_hip_status ensure_partials(qi_hip_qwen3* m, qi_hip_kv_cache* c) {
  const uint32_t heads = m->cfg.num_attention_heads;
  if (c->pm && c->heads == heads) return QI_HIP_OK;
  QI_HIP_TRY(hipStreamSynchronize(m->ctx->stream), "synchronize before sizing partials");
  dev_free(c->pm);
  dev_free(c->pl);
  dev_free(c->po);
  dev_free(c->tickets);
  c->pm = c->pl = c->po = nullptr;
  c->tickets = nullptr;
  if (c->exec) (void)hipGraphExecDestroy(c->exec);
  c->exec = nullptr;
  const uint64_t chunks = c->cap / kChunk;
  const uint64_t per_row = static_cast<uint64_t>(heads) * chunks * (c->head_dim + 2) * 4;
  uint64_t rb = kPartialBudget / per_row;
  rb = rb < 1 ? 1 : (rb > kMaxRows ? kMaxRows : rb);
  const uint64_t hc = static_cast<uint64_t>(heads) * chunks * rb;
  qi_hip_status s;
  if ((s = dev_alloc_t(&c->pm, hc, "alloc attention partials")) != QI_HIP_OK) return s;
  if ((s = dev_alloc_t(&c->pl, hc, "alloc attention partials")) != QI_HIP_OK) return s;
  if ((s = dev_alloc_t(&c->po, hc * c->head_dim, "alloc attention partials")) != QI_HIP_OK) return s;
  const uint64_t nt = rb * c->kv_heads;
  if ((s = dev_alloc_t(&c->tickets, nt, "alloc attention tickets")) != QI_HIP_OK) return s;
  QI_HIP_TRY(hipMemset(c->tickets, 0, nt * 4), "zero attention tickets");
  QI_HIP_TRY(hipDeviceSynchronize(), "zero attention tickets");
  c->rb = static_cast<uint32_t>(rb);
  c->heads = heads;
  return QI_HIP_OK;
}

// Prompt forward: upload tokens, run chunks of kMaxRows, project the last row.
qi_hip_status forward_locked(qi_hip_qwen3* m, qi_hip_kv_cache* c, const int32_t* tokens,
                             uint64_t count) {
  hipStream_t st = m->ctx->stream;
  if (count == 0) return fail(QI_HIP_INVALID_INPUT, "Qwen3 forward requires at least one token");
  for (uint64_t i = 0; i < count; ++i)
    if (tokens[i] < 0 || static_cast<uint64_t>(tokens[i]) >= m->cfg.vocab_size)
      return fail(QI_HIP_INVALID_INPUT, "token id " + std::to_string(tokens[i]) +
                                            " is outside vocabulary size " +
                                            std::to_string(m->cfg.vocab_size));
  if (c->len + count > m->cfg.max_position_embeddings)
    return fail(QI_HIP_INVALID_INPUT, "input exceeds Qwen3 max_position_embeddings");
  if (c->len + count > c->max_seq)
    return fail(QI_HIP_INVALID_INPUT, "KV cache capacity is smaller than the requested sequence");
  qi_hip_status s = ensure_partials(m, c);
  if (s != QI_HIP_OK) return s;
  QI_HIP_TRY(hipMemcpyAsync(c->tok + c->len, tokens, count * 4, hipMemcpyHostToDevice, st),
             "upload tokens");
  QI_HIP_TRY(hipMemsetAsync(m->bad, 0, 4, st), "clear logits flag");
  for (uint64_t r0 = 0; r0 < count; r0 += kMaxRows) {
    const uint32_t rows = static_cast<uint32_t>(count - r0 < kMaxRows ? count - r0 : kMaxRows);
    const bool last = r0 + rows == count;
    if ((s = enqueue_forward(m, c, rows, last)) != QI_HIP_OK) return s;
  }
  c->len += count;
  return QI_HIP_OK;
}

qi_hip_status read_bad(qi_hip_qwen3* m) {
  int32_t bad = 0;
  QI_HIP_TRY(hipMemcpyAsync(&bad, m->bad, 4, hipMemcpyDeviceToHost, m->ctx->stream), "read flag");
  QI_HIP_TRY(hipStreamSynchronize(m->ctx->stream), "synchronize");
  if (bad) return fail(QI_HIP_INVALID_INPUT, "logits must contain only finite values");
  return QI_HIP_OK;
}

// One decode step (the token at tok[len]) as a replay of the cache's graph,
// captured on first use for this model and context workspace generation.
qi_hip_status decode_step(qi_hip_qwen3* m, qi_hip_kv_cache* c) {
  hipStream_t st = m->ctx->stream;
  if (m->eager) return enqueue_forward(m, c, 1, true);
  if (c->exec == nullptr || c->graph_model != m->id || c->graph_ws != qi_abi::workspace_version()) {
    if (c->exec) {
      QI_HIP_TRY(hipStreamSynchronize(st), "synchronize before recapture");
      (void)hipGraphExecDestroy(c->exec);
      c->exec = nullptr;
    }
    // An eager step first: it grows any context workspace the step needs, so
    // the capture below allocates nothing.
    qi_hip_status s = enqueue_forward(m, c, 1, true);
    if (s != QI_HIP_OK) return s;
    const uint64_t ws = qi_abi::workspace_version();
    hipGraph_t graph = nullptr;
    QI_HIP_TRY(hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal), "begin capture");
    s = enqueue_forward(m, c, 1, true);
    hipError_t e = hipStreamEndCapture(st, &graph);
    if (s != QI_HIP_OK) {
      if (graph) (void)hipGraphDestroy(graph);
      return s;
    }
    if (e != hipSuccess) return hip_fail(e, "capture decode step");
    e = hipGraphInstantiate(&c->exec, graph, nullptr, nullptr, 0);
    (void)hipGraphDestroy(graph);
    if (e != hipSuccess) {
      c->exec = nullptr;
      return hip_fail(e, "instantiate decode graph");
    }
    c->graph_model = m->id;
    c->graph_ws = ws;
    return QI_HIP_OK;  // the eager step was this step
  }
  // the step's graph may read the context workspaces (MFMA mode)
  qi_hip_status s = qi_abi::ws_before(m->ctx, st);
  if (s != QI_HIP_OK) return s;
  QI_HIP_TRY(hipGraphLaunch(c->exec, st), "launch decode graph");
  return qi_abi::ws_after(m->ctx, st);
}

void model_destroy(qi_hip_qwen3* m) {
  qi_hip_ctx* c = m->ctx;
  {
    std::lock_guard<std::mutex> lock(c->mu);
    (void)hipSetDevice(c->device);
    (void)hipStreamSynchronize(c->stream);
    for (Layer& l : m->layers) {
      dev_free(l.norms);
      free_linear(&l.qkv);
      free_linear(&l.o);
      free_linear(&l.gate_up);
      free_linear(&l.down);
    }
    free_linear(&m->head);
    for (void* p : {static_cast<void*>(m->embedding), static_cast<void*>(m->final_norm),
                    static_cast<void*>(m->rope_cos), static_cast<void*>(m->rope_sin),
                    static_cast<void*>(m->h), static_cast<void*>(m->x), static_cast<void*>(m->qkv),
                    static_cast<void*>(m->q), static_cast<void*>(m->att), static_cast<void*>(m->y),
                    static_cast<void*>(m->gu), static_cast<void*>(m->act),
                    static_cast<void*>(m->logits), static_cast<void*>(m->apv),
                    static_cast<void*>(m->api), static_cast<void*>(m->bad)})
      dev_free(p);
    for (hipEvent_t e : m->ev)
      if (e) (void)hipEventDestroy(e);
  }
  qi_abi::ctx_release(c);
  delete m;
}

}  // namespace

extern "C" {

qi_hip_status qi_hip_qwen3_create(qi_hip_ctx* ctx, const qi_hip_qwen3_config* cfg,
                                  qi_hip_qwen3** out) {
  if (ctx == nullptr || cfg == nullptr || out == nullptr) return fail(QI_HIP_INVALID_INPUT, "null argument");
  *out = nullptr;
  if (ctx->closed) return fail(QI_HIP_INVALID_INPUT, "context is closed");
  const qi_hip_qwen3_config& k = *cfg;
  // Qwen3Config::validate / LlamaConfig::validate (quantinfer-model llama.rs:64-100)
  if (k.vocab_size == 0 || k.hidden_size == 0 || k.intermediate_size == 0 ||
      k.num_hidden_layers == 0 || k.num_attention_heads == 0 || k.num_key_value_heads == 0 ||
      k.max_position_embeddings == 0)
    return fail(QI_HIP_INVALID_INPUT, "Qwen3 dimensions must be greater than zero");
  if (k.num_attention_heads % k.num_key_value_heads != 0)
    return fail(QI_HIP_INVALID_INPUT, "attention heads must be divisible by key/value heads");
  if (k.head_dim == 0 || k.head_dim % 2 != 0)
    return fail(QI_HIP_INVALID_INPUT, "head_dim must be positive and even for RoPE");
  if (!(k.rms_norm_eps > 0.0f) || !isfinite(k.rms_norm_eps) || !(k.rope_theta > 0.0f) ||
      !isfinite(k.rope_theta))
    return fail(QI_HIP_INVALID_INPUT, "rms_norm_eps and rope_theta must be positive and finite");
  // shapes this device implementation covers
  if (k.head_dim != 64 && k.head_dim != 128)
    return fail(QI_HIP_UNSUPPORTED, "the device decoder supports head_dim 64 and 128");
  const uint32_t group = k.num_attention_heads / k.num_key_value_heads;
  if (group != 1 && group != 2 && group != 4 && group != 8)
    return fail(QI_HIP_UNSUPPORTED, "the device decoder supports 1, 2, 4 or 8 query heads per KV head");
  if (k.hidden_size % 4 != 0 || k.hidden_size > 16384)
    return fail(QI_HIP_UNSUPPORTED, "hidden_size must be a multiple of 4, at most 16384");

  qi_hip_qwen3* m = new qi_hip_qwen3();
  m->cfg = k;
  m->layers.resize(k.num_hidden_layers);
  if (const char* env = getenv("QI_HIP_QWEN3_EAGER")) m->eager = atoi(env) != 0;
  if (const char* env = getenv("QI_HIP_QWEN3_UNFUSED")) m->unfused = atoi(env) != 0;
  if (const char* env = getenv("QI_HIP_QWEN3_ATTN_FMA")) m->attn_fma = atoi(env) != 0;
  std::lock_guard<std::mutex> lock(ctx->mu);
  ctx->refs.fetch_add(1, std::memory_order_relaxed);
  m->ctx = ctx;
  m->id = g_next_model_id++;
  auto bail = [&](qi_hip_status s) {
    ctx->mu.unlock();
    model_destroy(m);
    ctx->mu.lock();
    return s;
  };
  hipError_t e = hipSetDevice(ctx->device);
  if (e != hipSuccess) return bail(hip_fail(e, "set device"));
  e = attn_prepare(k.head_dim, group);
  if (e != hipSuccess) return bail(hip_fail(e, "attention LDS limit"));
  // RoPE tables for every position (attention.rs:7-35, evaluated once with
  // the same f32 library functions)
  const uint32_t pairs = k.head_dim / 2;
  std::vector<float> cs(static_cast<uint64_t>(k.max_position_embeddings) * pairs);
  std::vector<float> sn(cs.size());
  for (uint64_t p = 0; p < k.max_position_embeddings; ++p) {
    const float position = static_cast<float>(p);
    for (uint32_t i = 0; i < pairs; ++i) {
      const float exponent = (2.0f * static_cast<float>(i)) / static_cast<float>(k.head_dim);
      const float angle = position * powf(k.rope_theta, -exponent);
      cs[p * pairs + i] = cosf(angle);
      sn[p * pairs + i] = sinf(angle);
    }
  }
  const uint64_t H = k.hidden_size, I = k.intermediate_size;
  const uint64_t QS = static_cast<uint64_t>(k.num_attention_heads) * k.head_dim;
  const uint64_t KS = static_cast<uint64_t>(k.num_key_value_heads) * k.head_dim;
  qi_hip_status s;
  if ((s = dev_alloc_t(&m->rope_cos, cs.size(), "alloc rope tables")) != QI_HIP_OK) return bail(s);
  if ((s = dev_alloc_t(&m->rope_sin, sn.size(), "alloc rope tables")) != QI_HIP_OK) return bail(s);
  if ((s = upload(m->rope_cos, cs.data(), cs.size() * 4, ctx->stream)) != QI_HIP_OK) return bail(s);
  if ((s = upload(m->rope_sin, sn.data(), sn.size() * 4, ctx->stream)) != QI_HIP_OK) return bail(s);
  const uint64_t R = kMaxRows;
  if ((s = dev_alloc_t(&m->h, R * H, "alloc activations")) != QI_HIP_OK ||
      (s = dev_alloc_t(&m->x, R * H, "alloc activations")) != QI_HIP_OK ||
      (s = dev_alloc_t(&m->qkv, R * (QS + 2 * KS), "alloc activations")) != QI_HIP_OK ||
      (s = dev_alloc_t(&m->q, R * QS, "alloc activations")) != QI_HIP_OK ||
      (s = dev_alloc_t(&m->att, R * QS, "alloc activations")) != QI_HIP_OK ||
      (s = dev_alloc_t(&m->y, R * H, "alloc activations")) != QI_HIP_OK ||
      (s = dev_alloc_t(&m->gu, R * 2 * I, "alloc activations")) != QI_HIP_OK ||
      (s = dev_alloc_t(&m->act, R * I, "alloc activations")) != QI_HIP_OK ||
      (s = dev_alloc_t(&m->logits, k.vocab_size, "alloc logits")) != QI_HIP_OK ||
      (s = dev_alloc_t(&m->apv, kArgBlocks, "alloc argmax")) != QI_HIP_OK ||
      (s = dev_alloc_t(&m->api, kArgBlocks, "alloc argmax")) != QI_HIP_OK ||
      (s = dev_alloc_t(&m->bad, 1, "alloc flag")) != QI_HIP_OK)
    return bail(s);
  for (hipEvent_t& ev : m->ev) {
    e = hipEventCreate(&ev);
    if (e != hipSuccess) return bail(hip_fail(e, "create events"));
  }
  *out = m;
  return QI_HIP_OK;
}

qi_hip_status qi_hip_qwen3_set_embedding(qi_hip_qwen3* m, const float* table) {
  if (m == nullptr || table == nullptr) return fail(QI_HIP_INVALID_INPUT, "null argument");
  std::lock_guard<std::mutex> lock(m->ctx->mu);
  QI_HIP_TRY(hipSetDevice(m->ctx->device), "set device");
  const uint64_t n = static_cast<uint64_t>(m->cfg.vocab_size) * m->cfg.hidden_size;
  if (m->embedding == nullptr) {
    qi_hip_status s = dev_alloc_t(&m->embedding, n, "alloc embedding");
    if (s != QI_HIP_OK) return s;
  }
  return upload(m->embedding, table, n * 4, m->ctx->stream);
}

qi_hip_status qi_hip_qwen3_set_layer(qi_hip_qwen3* m, uint32_t index, const qi_hip_qwen3_layer* L) {
  if (m == nullptr || L == nullptr) return fail(QI_HIP_INVALID_INPUT, "null argument");
  const qi_hip_qwen3_config& k = m->cfg;
  if (index >= k.num_hidden_layers) return fail(QI_HIP_INVALID_INPUT, "layer index is out of bounds");
  if (!L->input_layernorm || !L->q_norm || !L->k_norm || !L->post_attention_layernorm)
    return fail(QI_HIP_INVALID_INPUT, "null norm weight");
  const uint64_t H = k.hidden_size, I = k.intermediate_size, hd = k.head_dim;
  const uint64_t QS = k.num_attention_heads * hd, KS = k.num_key_value_heads * hd;
  std::lock_guard<std::mutex> lock(m->ctx->mu);
  QI_HIP_TRY(hipSetDevice(m->ctx->device), "set device");
  QI_HIP_TRY(hipStreamSynchronize(m->ctx->stream), "synchronize");
  Layer fresh;
  qi_hip_status s = dev_alloc_t(&fresh.norms, 2 * H + 2 * hd, "alloc norms");
  auto cleanup = [&](qi_hip_status st) {
    dev_free(fresh.norms);
    free_linear(&fresh.qkv);
    free_linear(&fresh.o);
    free_linear(&fresh.gate_up);
    free_linear(&fresh.down);
    return st;
  };
  if (s != QI_HIP_OK) return cleanup(s);
  std::vector<float> norms(2 * H + 2 * hd);
  memcpy(norms.data(), L->input_layernorm, H * 4);
  memcpy(norms.data() + H, L->q_norm, hd * 4);
  memcpy(norms.data() + H + hd, L->k_norm, hd * 4);
  memcpy(norms.data() + H + 2 * hd, L->post_attention_layernorm, H * 4);
  if ((s = upload(fresh.norms, norms.data(), norms.size() * 4, m->ctx->stream)) != QI_HIP_OK)
    return cleanup(s);
  const qi_hip_linear_weight* qkv[3] = {&L->q_proj, &L->k_proj, &L->v_proj};
  const uint64_t nqkv[3] = {QS, KS, KS};
  const qi_hip_linear_weight* gu[2] = {&L->gate_proj, &L->up_proj};
  const uint64_t ngu[2] = {I, I};
  const qi_hip_linear_weight* o[1] = {&L->o_proj};
  const qi_hip_linear_weight* dn[1] = {&L->down_proj};
  const uint64_t nh[1] = {H};
  if ((s = make_linear(m->ctx, qkv, 3, H, nqkv, "q/k/v projection", &fresh.qkv)) != QI_HIP_OK ||
      (s = make_linear(m->ctx, o, 1, QS, nh, "o projection", &fresh.o)) != QI_HIP_OK ||
      (s = make_linear(m->ctx, gu, 2, H, ngu, "gate/up projection", &fresh.gate_up, 8)) != QI_HIP_OK ||
      (s = make_linear(m->ctx, dn, 1, I, nh, "down projection", &fresh.down)) != QI_HIP_OK)
    return cleanup(s);
  Layer& dst = m->layers[index];
  dev_free(dst.norms);
  free_linear(&dst.qkv);
  free_linear(&dst.o);
  free_linear(&dst.gate_up);
  free_linear(&dst.down);
  dst = fresh;
  dst.set = true;
  m->id = g_next_model_id++;  // captured decode graphs of this model are stale
  return QI_HIP_OK;
}

qi_hip_status qi_hip_qwen3_set_output(qi_hip_qwen3* m, const float* final_norm,
                                      const qi_hip_linear_weight* head) {
  if (m == nullptr || final_norm == nullptr || head == nullptr)
    return fail(QI_HIP_INVALID_INPUT, "null argument");
  const uint64_t H = m->cfg.hidden_size, V = m->cfg.vocab_size;
  std::lock_guard<std::mutex> lock(m->ctx->mu);
  QI_HIP_TRY(hipSetDevice(m->ctx->device), "set device");
  QI_HIP_TRY(hipStreamSynchronize(m->ctx->stream), "synchronize");
  Linear fresh;
  const qi_hip_linear_weight* parts[1] = {head};
  const uint64_t nv[1] = {V};
  qi_hip_status s = make_linear(m->ctx, parts, 1, H, nv, "lm_head", &fresh);
  if (s != QI_HIP_OK) return s;
  if (m->final_norm == nullptr && (s = dev_alloc_t(&m->final_norm, H, "alloc final norm")) != QI_HIP_OK) {
    free_linear(&fresh);
    return s;
  }
  if ((s = upload(m->final_norm, final_norm, H * 4, m->ctx->stream)) != QI_HIP_OK) {
    free_linear(&fresh);
    return s;
  }
  free_linear(&m->head);
  m->head = fresh;
  m->id = g_next_model_id++;
  return QI_HIP_OK;
}

qi_hip_status qi_hip_qwen3_set_mode(qi_hip_qwen3* m, int32_t mode) {
  if (m == nullptr) return fail(QI_HIP_INVALID_INPUT, "null model");
  if (mode < QI_HIP_MODE_AUTO || mode > QI_HIP_MODE_MFMA) return fail(QI_HIP_INVALID_INPUT, "unknown arithmetic mode");
  std::lock_guard<std::mutex> lock(m->ctx->mu);
  m->mode = mode;
  m->id = g_next_model_id++;
  return QI_HIP_OK;
}

void qi_hip_qwen3_free(qi_hip_qwen3* m) {
  if (m) model_destroy(m);
}

qi_hip_status qi_hip_kv_cache_create(qi_hip_ctx* ctx, uint32_t layers, uint32_t max_seq,
                                     uint32_t kv_heads, uint32_t head_dim, qi_hip_kv_cache** out) {
  if (ctx == nullptr || out == nullptr) return fail(QI_HIP_INVALID_INPUT, "null argument");
  *out = nullptr;
  if (ctx->closed) return fail(QI_HIP_INVALID_INPUT, "context is closed");
  // KvCache::new (cache.rs:25-60)
  if (layers == 0 || max_seq == 0 || kv_heads == 0 || head_dim == 0)
    return fail(QI_HIP_INVALID_INPUT, "KV cache dimensions must be greater than zero");
  qi_hip_kv_cache* c = new qi_hip_kv_cache();
  c->layers = layers;
  c->max_seq = max_seq;
  c->kv_heads = kv_heads;
  c->head_dim = head_dim;
  c->cap = (max_seq + kChunk - 1) / kChunk * kChunk;
  const uint64_t per = static_cast<uint64_t>(layers) * kv_heads * head_dim * c->cap;
  std::lock_guard<std::mutex> lock(ctx->mu);
  qi_hip_status s = QI_HIP_OK;
  hipError_t e = hipSetDevice(ctx->device);
  if (e != hipSuccess) s = hip_fail(e, "set device");
  if (s == QI_HIP_OK) s = dev_alloc_t(&c->keys, per, "alloc KV cache");
  if (s == QI_HIP_OK) s = dev_alloc_t(&c->values, per, "alloc KV cache");
  if (s == QI_HIP_OK) s = dev_alloc_t(&c->tok, c->cap + 1, "alloc token history");
  if (s == QI_HIP_OK) s = dev_alloc_t(&c->len_dev, 1, "alloc cache length");
  if (s == QI_HIP_OK) {
    // positions past the length are never read, but keep them finite
    e = hipMemsetAsync(c->keys, 0, per * 4, ctx->stream);
    if (e == hipSuccess) e = hipMemsetAsync(c->values, 0, per * 4, ctx->stream);
    if (e == hipSuccess) e = hipMemsetAsync(c->len_dev, 0, 4, ctx->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
    if (e != hipSuccess) s = hip_fail(e, "clear KV cache");
  }
  if (s != QI_HIP_OK) {
    dev_free(c->keys);
    dev_free(c->values);
    dev_free(c->tok);
    dev_free(c->len_dev);
    delete c;
    return s;
  }
  ctx->refs.fetch_add(1, std::memory_order_relaxed);
  c->ctx = ctx;
  *out = c;
  return QI_HIP_OK;
}

qi_hip_status qi_hip_kv_cache_length(const qi_hip_kv_cache* c, uint64_t* out) {
  if (c == nullptr || out == nullptr) return fail(QI_HIP_INVALID_INPUT, "null argument");
  *out = c->len;
  return QI_HIP_OK;
}

qi_hip_status qi_hip_kv_cache_reset(qi_hip_kv_cache* c) {
  if (c == nullptr) return fail(QI_HIP_INVALID_INPUT, "null cache");
  std::lock_guard<std::mutex> lock(c->ctx->mu);
  QI_HIP_TRY(hipSetDevice(c->ctx->device), "set device");
  QI_HIP_TRY(hipMemsetAsync(c->len_dev, 0, 4, c->ctx->stream), "reset cache");
  QI_HIP_TRY(hipStreamSynchronize(c->ctx->stream), "reset cache");
  c->len = 0;
  return QI_HIP_OK;
}

void qi_hip_kv_cache_free(qi_hip_kv_cache* c) {
  if (c == nullptr) return;
  qi_hip_ctx* ctx = c->ctx;
  {
    std::lock_guard<std::mutex> lock(ctx->mu);
    (void)hipSetDevice(ctx->device);
    (void)hipStreamSynchronize(ctx->stream);
    if (c->exec) (void)hipGraphExecDestroy(c->exec);
    for (void* p : {static_cast<void*>(c->keys), static_cast<void*>(c->values),
                    static_cast<void*>(c->tok), static_cast<void*>(c->len_dev),
                    static_cast<void*>(c->pm), static_cast<void*>(c->pl), static_cast<void*>(c->po),
                    static_cast<void*>(c->tickets)})
      dev_free(p);
  }
  qi_abi::ctx_release(ctx);
  delete c;
}

qi_hip_status qi_hip_qwen3_forward(qi_hip_qwen3* m, qi_hip_kv_cache* c, const int32_t* tokens,
                                   uint64_t count, float* last_logits, int32_t* next_token) {
  qi_hip_status s = check_pair(m, c);
  if (s != QI_HIP_OK) return s;
  if (tokens == nullptr && count > 0) return fail(QI_HIP_INVALID_INPUT, "null token array");
  std::lock_guard<std::mutex> lock(m->ctx->mu);
  QI_HIP_TRY(hipSetDevice(m->ctx->device), "set device");
  hipStream_t st = m->ctx->stream;
  const uint64_t start = c->len;
  if ((s = forward_locked(m, c, tokens, count)) != QI_HIP_OK) {
    (void)hipStreamSynchronize(st);
    return s;
  }
  if (last_logits)
    QI_HIP_TRY(hipMemcpyAsync(last_logits, m->logits, static_cast<uint64_t>(m->cfg.vocab_size) * 4,
                              hipMemcpyDeviceToHost, st), "read logits");
  int32_t tok = 0;
  QI_HIP_TRY(hipMemcpyAsync(&tok, c->tok + start + count, 4, hipMemcpyDeviceToHost, st), "read token");
  QI_HIP_TRY(hipStreamSynchronize(st), "synchronize");
  if (next_token) {
    if ((s = read_bad(m)) != QI_HIP_OK) return s;
    *next_token = tok;
  }
  return QI_HIP_OK;
}

qi_hip_status qi_hip_qwen3_generate(qi_hip_qwen3* m, qi_hip_kv_cache* c, const int32_t* prompt,
                                    uint64_t n, uint64_t max_new, int32_t eos, int32_t* out,
                                    uint64_t* out_count) {
  qi_hip_status s = check_pair(m, c);
  if (s != QI_HIP_OK) return s;
  if (out_count == nullptr || (out == nullptr && max_new > 0) || (prompt == nullptr && n > 0))
    return fail(QI_HIP_INVALID_INPUT, "null argument");
  *out_count = 0;
  if (n == 0) return fail(QI_HIP_INVALID_INPUT, "streaming generation requires a non-empty prompt");
  std::lock_guard<std::mutex> lock(m->ctx->mu);
  QI_HIP_TRY(hipSetDevice(m->ctx->device), "set device");
  hipStream_t st = m->ctx->stream;
  m->timing = qi_hip_qwen3_timing{};
  QI_HIP_TRY(hipEventRecord(m->ev[0], st), "record event");
  if ((s = forward_locked(m, c, prompt, n)) != QI_HIP_OK) {
    (void)hipStreamSynchronize(st);
    return s;
  }
  QI_HIP_TRY(hipEventRecord(m->ev[1], st), "record event");
  // Token i (i = 0..max_new-1) is tok[base + i]: token 0 comes from the prompt
  // forward and forwarding token i produces token i + 1. Every selected token
  // but an EOS is forwarded (generation.rs:189-199). Without an EOS all steps
  // are enqueued back to back; with one, steps run in batches of 16 and the
  // host looks at the tokens between batches, undoing the steps past an EOS
  // (their cache positions are dropped by resetting the length).
  const uint64_t base = c->len;
  const uint64_t limit = c->max_seq < m->cfg.max_position_embeddings ? c->max_seq
                                                                     : m->cfg.max_position_embeddings;
  std::vector<int32_t> toks(max_new + 1);
  uint64_t forwarded = 0, checked = 0, count = max_new;
  const uint64_t batch = eos < 0 ? (max_new ? max_new : 1) : 16;
  while (true) {
    if (eos >= 0 && checked < max_new) {
      const uint64_t upto = forwarded < max_new - 1 ? forwarded : max_new - 1;  // tokens 0..upto exist
      QI_HIP_TRY(hipMemcpyAsync(toks.data() + checked, c->tok + base + checked,
                                (upto + 1 - checked) * 4, hipMemcpyDeviceToHost, st), "read tokens");
      QI_HIP_TRY(hipStreamSynchronize(st), "synchronize");
      bool hit = false;
      for (uint64_t i = checked; i <= upto; ++i)
        if (toks[i] == eos) {
          count = i + 1;
          hit = true;
          break;
        }
      checked = upto + 1;
      if (hit) {
        if (forwarded > count - 1) {
          // only tokens 0..count-2 were to be forwarded
          c->len = base + (count - 1);
          const uint32_t len32 = static_cast<uint32_t>(c->len);
          QI_HIP_TRY(hipMemcpyAsync(c->len_dev, &len32, 4, hipMemcpyHostToDevice, st), "reset length");
          QI_HIP_TRY(hipStreamSynchronize(st), "synchronize");
          forwarded = count - 1;
        }
        break;
      }
    }
    if (forwarded >= max_new) break;
    uint64_t todo = max_new - forwarded < batch ? max_new - forwarded : batch;
    if (c->len + 1 > limit) {
      (void)hipStreamSynchronize(st);
      return fail(QI_HIP_INVALID_INPUT, "KV cache capacity is smaller than the requested sequence");
    }
    if (c->len + todo > limit) todo = limit - c->len;
    for (uint64_t i = 0; i < todo; ++i) {
      if ((s = decode_step(m, c)) != QI_HIP_OK) {
        (void)hipStreamSynchronize(st);
        return s;
      }
      c->len += 1;
      ++forwarded;
    }
  }
  QI_HIP_TRY(hipEventRecord(m->ev[2], st), "record event");
  if (count > checked)
    QI_HIP_TRY(hipMemcpyAsync(toks.data() + checked, c->tok + base + checked, (count - checked) * 4,
                              hipMemcpyDeviceToHost, st), "read tokens");
  QI_HIP_TRY(hipStreamSynchronize(st), "synchronize");
  if ((s = read_bad(m)) != QI_HIP_OK) return s;
  memcpy(out, toks.data(), count * 4);
  *out_count = count;
  float ms = 0.0f;
  if (hipEventElapsedTime(&ms, m->ev[0], m->ev[1]) == hipSuccess) m->timing.prefill_ms = ms;
  if (hipEventElapsedTime(&ms, m->ev[1], m->ev[2]) == hipSuccess) m->timing.decode_ms = ms;
  m->timing.prompt_tokens = n;
  m->timing.decode_steps = forwarded;
  return QI_HIP_OK;
}

qi_hip_status qi_hip_qwen3_last_timing(const qi_hip_qwen3* m, qi_hip_qwen3_timing* out) {
  if (m == nullptr || out == nullptr) return fail(QI_HIP_INVALID_INPUT, "null argument");
  *out = m->timing;
  return QI_HIP_OK;
}

}  // extern "C"
