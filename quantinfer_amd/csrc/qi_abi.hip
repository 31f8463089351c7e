// C ABI of the MI355X quantized-linear backend (include/qi_hip.h).
//
// The context owns one HIP stream (default priority), grow-only device
// workspaces (f16 activations and split-K partials of the prefill GEMM, the
// activation records of the multi-row GEMV) and the staging buffers of the
// synchronous host entry point. A mutex serializes calls on one context.
// Calls may enqueue on different caller streams; the device work of calls
// that use a workspace is ordered by an event (ws_before / ws_after), so two
// such calls never use a workspace at the same time. The event carries no
// system-scope fence: it orders work on one device and tells the host when a
// workspace is free, and a fence would write back the caches on every call.
#include <hip/hip_runtime.h>
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <atomic>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/qi_hip.h"
#include "qi_image.h"
#include "qi_internal.h"
#include "qi_ctx.h"

using qi::Image;

// Scratch memory of qi_hip_linear_device_noalloc: the workspaces of one call
// (the GEMM's f16 activations and split-K partials, the multi-row GEMV's
// activation records) carved out of this file-scope array instead of
// allocated. Each GPU the library runs on holds its own copy, at its own
// address, until the process ends. In host code `scratch` is a host-side
// stand-in, never a device address: qi_hip_open resolves the device address
// once per device (hipGetSymbolAddress) and only that address is used.
constexpr uint64_t kScratchBytes = 64ull << 20;
static __device__ __align__(256) uint8_t scratch[kScratchBytes];

namespace qi_abi {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch[kMaxDevices] = {};  // device address of `scratch`, per device ordinal

// With `device` current: the device address of its `scratch`, resolved once.
qi_hip_status scratch_setup(int device, void** out);

thread_local std::string g_last_error;
std::atomic<uint64_t> g_ws_version{0};

qi_hip_status fail(qi_hip_status st, const std::string& msg) {
  g_last_error = msg;
  return st;
}

qi_hip_status hip_fail(hipError_t e, const char* what) {
  return fail(QI_HIP_RUNTIME_ERROR, std::string("HIP ") + what + ": " + hipGetErrorString(e));
}


uint64_t workspace_version() { return g_ws_version.load(std::memory_order_relaxed); }

bool capturing(hipStream_t st) {
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  return hipStreamIsCapturing(st, &cs) == hipSuccess && cs != hipStreamCaptureStatusNone;
}

qi_hip_status ws_before(qi_hip_ctx* c, hipStream_t st) {
  // A stream under capture records only its own work; the decoder captures
  // on the context stream after an eager step, so nothing else is pending.
  if (!c->ws_used || c->ws_stream == st || capturing(st)) return QI_HIP_OK;
  QI_HIP_TRY(hipStreamWaitEvent(st, c->ws_event, 0), "order workspace use across streams");
  return QI_HIP_OK;
}

qi_hip_status ws_after(qi_hip_ctx* c, hipStream_t st) {
  if (capturing(st)) return QI_HIP_OK;
  QI_HIP_TRY(hipEventRecord(c->ws_event, st), "record workspace use");
  c->ws_stream = st;
  c->ws_used = true;
  return QI_HIP_OK;
}

// Wait until no queued work uses a workspace (before one is reallocated).
qi_hip_status ws_drain(qi_hip_ctx* c, hipStream_t st) {
  if (c->ws_used) QI_HIP_TRY(hipEventSynchronize(c->ws_event), "wait for workspace users");
  QI_HIP_TRY(hipStreamSynchronize(st), "synchronize before growing a workspace");
  return QI_HIP_OK;
}

qi_hip_status grow(float** buf, uint64_t* cap, uint64_t need, const char* what) {
  if (need <= *cap) return QI_HIP_OK;
  ++g_ws_version;
  if (*buf) (void)hipFree(*buf);
  *buf = nullptr;
  *cap = 0;
  QI_HIP_TRY(hipMalloc(reinterpret_cast<void**>(buf), need * sizeof(float)), what);
  *cap = need;
  return QI_HIP_OK;
}

// Pinned host staging buffer of at least `need` floats. Every qi_hip_linear
// call ends with a stream synchronize, so no copy still reads the old one.
qi_hip_status grow_pinned(float** buf, uint64_t* cap, uint64_t need) {
  if (need <= *cap) return QI_HIP_OK;
  if (*buf) (void)hipHostFree(*buf);
  *buf = nullptr;
  *cap = 0;
  QI_HIP_TRY(hipHostMalloc(reinterpret_cast<void**>(buf), need * sizeof(float), hipHostMallocDefault),
             "alloc pinned staging");
  *cap = need;
  return QI_HIP_OK;
}

qi_hip_status scratch_setup(int device, void** out) {
  if (device < 0 || device >= kMaxDevices) return fail(QI_HIP_UNSUPPORTED, "HIP device ordinal beyond 63");
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch[device] == nullptr) {
    void* ptr = nullptr;
    QI_HIP_TRY(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)), "device address of the scratch array");
    if (ptr == nullptr) return fail(QI_HIP_RUNTIME_ERROR, "device address of the scratch array is null");
    g_scratch[device] = ptr;
  }
  *out = g_scratch[device];
  return QI_HIP_OK;
}

void ctx_destroy(qi_hip_ctx* c) {
  (void)hipSetDevice(c->device);
  if (c->stream) (void)hipStreamSynchronize(c->stream);
  if (c->ws_event) {
    if (c->ws_used) (void)hipEventSynchronize(c->ws_event);
    (void)hipEventDestroy(c->ws_event);
  }
  if (c->xbuf) (void)hipFree(c->xbuf);
  if (c->ybuf) (void)hipFree(c->ybuf);
  if (c->hx) (void)hipHostFree(c->hx);
  if (c->hy) (void)hipHostFree(c->hy);
  if (c->hbuf) (void)hipFree(c->hbuf);
  if (c->sbuf) (void)hipFree(c->sbuf);
  if (c->dbuf) (void)hipFree(c->dbuf);
  if (c->stream) (void)hipStreamDestroy(c->stream);
  delete c;
}

void ctx_release(qi_hip_ctx* c) {
  if (c->refs.fetch_sub(1, std::memory_order_acq_rel) == 1) ctx_destroy(c);
}

qi_hip_status check_call(qi_hip_ctx* ctx, const qi_hip_weights* w, uint64_t m) {
  if (ctx == nullptr || w == nullptr) return fail(QI_HIP_INVALID_INPUT, "null context or weights");
  if (ctx->closed) return fail(QI_HIP_INVALID_INPUT, "context is closed");
  if (w->ctx != ctx) return fail(QI_HIP_INVALID_INPUT, "weights belong to another context");
  // lhs rows must be nonzero (core tensor.rs:85-93); grid.y limits exact-mode rows
  if (m == 0) return fail(QI_HIP_INVALID_INPUT, "matmul lhs must have at least one row");
  if (m > 65535) return fail(QI_HIP_INVALID_INPUT, "matmul lhs has more than 65535 rows");
  return QI_HIP_OK;
}

// Grow workspace `buf` to `need` floats, after every queued user is done.
qi_hip_status grow_ws(qi_hip_ctx* c, hipStream_t st, float** buf, uint64_t* cap, uint64_t need,
                      const char* what) {
  if (need <= *cap) return QI_HIP_OK;
  qi_hip_status s = ws_drain(c, st);
  if (s != QI_HIP_OK) return s;
  return grow(buf, cap, need, what);
}

// Which kernels a linear call runs and the workspace floats they need. One
// function decides, so that the growing path (run_linear) and the scratch
// path (qi_hip_linear_device_noalloc) take the same kernels.
struct LinearPlan {
  enum Kind { kGemm, kRowMajor, kRowMajorGemm, kMfma, kSplitGemm, kPlanar, kF32Gemv, kF32Gemm, kExact } kind = kExact;
  uint64_t m_pad = 0;
  uint32_t splits = 1;  // GEMM K splits, or row-major GEMV K splits per row chunk
  uint64_t h_floats = 0, s_floats = 0, d_floats = 0;  // f16 activations, partials, records
};

// Rows from which row-major weights (tiled image, K a multiple of 4) take
// the row-major GEMM (weights dequantized into LDS for the f32 matrix cores,
// K split into parts whose partial sums take at most kRmPartFloats) instead
// of the GEMV's 2-row launches, each of which reads and converts the whole
// weight. Calls run in chunks of kRmGemmChunkRows rows. Measured on MI355X,
// us per call, Q4_K 4096x14336, GEMV launches / GEMM: M=2 28.0 / 36.4,
// M=4 54.7 / 37.7, M=16 211.6 / 39.6, M=64 838 / 105 (the K-slice GEMM it
// replaced, f32 weight slices dequantized to HBM: 580), M=512 843 (K slices)
// / 660, M=2048 2446 (K slices) / 2272.
constexpr uint64_t kRmGemmMinRows = 3;
constexpr uint64_t kRmGemmChunkRows = 4096;
constexpr uint64_t kRmPartFloats = 8ull << 20;

// Rows of a chunk at which the 2-16 row GEMV switches from the int8-digit
// kernel (qi_gemv_rows.hip) to the split-half kernel (qi_gemv_half.hip): the
// digit kernel's work grows with the row count (a matrix instruction and a
// combine per four rows and window), the split-half kernel's does not (all 16
// rows in one f16 instruction per window half). Measured on MI355X, us per
// call, digit / split-half: Q4_K 4096x14336 M=2 12.5 / 14.8, M=8 17.7 / 17.1,
// M=16 29.5 / 23.8; Q4_0 12288x4096 M=4 16.6 / 18.0, M=16 28.1 / 22.9; Q4_K
// 4096x24576 M=16 49.6 / 38.3.
constexpr uint32_t kHalfMinRows = 9;

// Rows from which output rows take the split-half GEMM (qi_gemm_split.hip)
// in F32 mode, and in AUTO mode below the f16 GEMM's 128.
// Below it the 16-row GEMV chunks are faster. Measured on MI355X, us per
// call, GEMV chunks / split GEMM: Q4_K 4096x6144 M=17 22.9 / 31.9, M=24
// 30.3 / 33.0, M=32 31.0 / 33.1, M=40 43.7 / 34.1, M=48 34.7 (GEMM);
// at M=32 4096x24576 70.3 / 76.5, 12288x4096 43.2 / 36.9, Q8_0 4096x14336
// 47.6 / 42.8, Q6_K 52.4 / 42.2. From 33 rows the GEMV needs a third chunk.
constexpr uint64_t kSplitMinRows = 33;
// Rows per split-half GEMM launch: longer calls run in chunks, so that the
// activation records (about 4.1 bytes per activation) stay bounded.
constexpr uint64_t kSplitChunkRows = 4096;

qi_hip_status plan_linear(const Image& im, uint64_t m, int32_t mode, LinearPlan* p) {
  if (mode < QI_HIP_MODE_AUTO || mode > QI_HIP_MODE_MFMA)
    return fail(QI_HIP_INVALID_INPUT, "unknown arithmetic mode");
  bool use_gemm = false;
  if (mode == QI_HIP_MODE_MFMA) {
    if (!qi::gemm_supported(im.qtype, im.layout, im.k, im.n))
      return fail(QI_HIP_UNSUPPORTED, "MFMA GEMM does not support this weight type/layout/shape");
    if (!im.f16_gemm)
      return fail(QI_HIP_UNSUPPORTED,
                  "MFMA GEMM: the weight values or scales lie outside the range f16 operands hold");
    use_gemm = true;
  } else if (mode == QI_HIP_MODE_AUTO) {
    use_gemm = m >= 128 && im.f16_gemm && qi::gemm_supported(im.qtype, im.layout, im.k, im.n);
  }
  *p = LinearPlan{};
  if (use_gemm) {
    p->kind = LinearPlan::kGemm;
    p->m_pad = qi::gemm_padded_rows(m);
    p->h_floats = (p->m_pad * im.k + 1) / 2;
    p->splits = qi::gemm_splits(im, m);
    if (p->splits > 1) p->s_floats = p->splits * p->m_pad * im.n;
    return QI_HIP_OK;
  }
  if (mode != QI_HIP_MODE_EXACT && qi::f32w_gemv_supported(im)) {
    // F32 weights: the streaming GEMV in 8-row chunks, the matrix-core GEMM above
    if (m > qi::kF32GemvMaxRows && qi::f32w_gemm_supported(im)) {
      p->kind = LinearPlan::kF32Gemm;
      return QI_HIP_OK;
    }
    p->kind = LinearPlan::kF32Gemv;
    p->splits = qi::f32w_splits(im);
    if (p->splits > 1) p->s_floats = static_cast<uint64_t>(p->splits) * (m < 8 ? m : 8) * im.n;
    return QI_HIP_OK;
  }
  if (mode != QI_HIP_MODE_EXACT && qi::rm_gemm_supported(im) && m >= kRmGemmMinRows) {
    p->kind = LinearPlan::kRowMajorGemm;
    // chunks of kRmGemmChunkRows rows; a shorter last chunk takes its own
    // part count (enqueue_linear asks again)
    const uint64_t chunk = m < kRmGemmChunkRows ? m : kRmGemmChunkRows;
    for (uint64_t r : {chunk, m > chunk ? m % chunk : 0}) {
      if (r == 0) continue;
      const uint32_t parts = qi::rm_gemm_parts(im, r, kRmPartFloats);
      if (parts > 1) p->s_floats = std::max(p->s_floats, static_cast<uint64_t>(parts) * r * im.n);
    }
    p->splits = qi::rm_gemm_parts(im, chunk, kRmPartFloats);
    return QI_HIP_OK;
  }
  if (mode != QI_HIP_MODE_EXACT && qi::gemv_rm_supported(im)) {
    p->kind = LinearPlan::kRowMajor;
    const uint32_t rows = qi::gemv_rm_rows(im);
    const uint32_t chunk = m < rows ? static_cast<uint32_t>(m) : rows;
    p->splits = qi::gemv_rm_splits(im, chunk);
    if (p->splits > 1) p->s_floats = static_cast<uint64_t>(p->splits) * chunk * im.n;
    return QI_HIP_OK;
  }
  if (mode != QI_HIP_MODE_EXACT && m >= kSplitMinRows && qi::gemm_split_supported(im)) {
    p->kind = LinearPlan::kSplitGemm;
    // chunks of kSplitChunkRows rows; a shorter last chunk takes its own K
    // split count (enqueue_linear asks again)
    const uint64_t chunk = m < kSplitChunkRows ? m : kSplitChunkRows;
    uint64_t floats = 0;
    for (uint64_t r : {chunk, m > chunk ? m % chunk : 0}) {
      if (r == 0) continue;
      const uint32_t sp = qi::gemm_split_splits(im, r);
      if (sp > 1) floats = std::max(floats, static_cast<uint64_t>(sp) * r * im.n);
    }
    p->splits = qi::gemm_split_splits(im, chunk);
    p->s_floats = floats;
    p->d_floats = (qi::gemm_split_records_bytes(chunk, im.k) + 3) / 4;
    return QI_HIP_OK;
  }
  if (mode != QI_HIP_MODE_EXACT && qi::gemv_mfma_supported(im.qtype, im.layout, im.k)) {
    p->kind = LinearPlan::kMfma;
    if (m >= 2) {
      // two or more rows (launch_gemv_half, the same formats and shapes as
      // the one-row kernel): one kernel per 16-row chunk; K parts only for
      // shapes with few tiles, by the chunk's row count (a shorter last chunk
      // may take a different count; enqueue_linear asks again)
      uint64_t floats = 0, records = 0;
      for (uint64_t r : {static_cast<uint64_t>(m < 16 ? m : 16), m > 16 ? m % 16 : 0}) {
        if (r < 2) continue;
        const uint32_t rr = static_cast<uint32_t>(r);
        const bool half = rr >= kHalfMinRows;
        const uint32_t pr = half ? qi::gemv_half_splits(im.k, im.n, rr) : qi::gemv_rows_splits(im.k, im.n, rr);
        if (pr > 1) floats = std::max(floats, static_cast<uint64_t>(pr) * r * im.n);
        if (half) records = std::max(records, qi::gemv_half_records_bytes(im.k));
      }
      p->splits = 1;
      p->s_floats = floats;
      p->d_floats = (records + 3) / 4;
    }
    return QI_HIP_OK;
  }
  if (mode != QI_HIP_MODE_EXACT && qi::gemv_supported(im.qtype, im.layout, im.k)) {
    p->kind = LinearPlan::kPlanar;
    return QI_HIP_OK;
  }
  p->kind = LinearPlan::kExact;
  return QI_HIP_OK;
}

// Enqueue the kernels of `p` on `st` with the given workspaces (each at least
// the plan's size).
qi_hip_status enqueue_linear(const qi_hip_weights* w, const LinearPlan& p, const float* x, uint64_t m,
                             float* y, hipStream_t st, float* hws, float* sws, float* dws,
                             float* silu_act, bool* silu_done) {
  const Image& im = w->im;
  const qi::View v = qi::make_view(im, w->dev);
  switch (p.kind) {
    case LinearPlan::kGemm: {
      qi::GemmArgs ga{v, x, y, m, reinterpret_cast<_Float16*>(hws), p.m_pad};
      ga.splits = p.splits;
      if (silu_act != nullptr && silu_done != nullptr && ga.splits == 1 && qi::gemm_silu_supported(im)) {
        ga.act = silu_act;
        *silu_done = true;
      }
      if (ga.splits > 1) ga.part = sws;
      QI_HIP_TRY(qi::launch_gemm(im, ga, st), "launch gemm");
      return QI_HIP_OK;
    }
    case LinearPlan::kRowMajor: {
      // the blocks-along-N GEMV, gemv_rm_rows rows per launch; a last chunk
      // of fewer rows keeps at most the full chunk's split count
      const uint32_t per = qi::gemv_rm_rows(im);
      for (uint64_t m0 = 0; m0 < m; m0 += per) {
        const uint32_t rows = static_cast<uint32_t>(m - m0 < per ? m - m0 : per);
        const uint32_t chunk = m < per ? static_cast<uint32_t>(m) : per;
        const uint32_t sp = rows == chunk ? p.splits : qi::gemv_rm_splits(im, rows);
        QI_HIP_TRY(qi::launch_gemv_rm(im, v, x + m0 * im.k, rows, y + m0 * im.n, sws,
                                      sp <= p.splits ? sp : p.splits, st),
                   "launch row-major gemv");
      }
      return QI_HIP_OK;
    }
    case LinearPlan::kRowMajorGemm:
      for (uint64_t m0 = 0; m0 < m; m0 += kRmGemmChunkRows) {
        const uint64_t rows = m - m0 < kRmGemmChunkRows ? m - m0 : kRmGemmChunkRows;
        const uint32_t parts = qi::rm_gemm_parts(im, rows, kRmPartFloats);
        QI_HIP_TRY(qi::launch_rm_gemm(im, v, x + m0 * im.k, rows, y + m0 * im.n, sws, parts, st),
                   "launch row-major GEMM");
      }
      return QI_HIP_OK;
    case LinearPlan::kMfma:
    case LinearPlan::kPlanar:
      for (uint64_t m0 = 0; m0 < m; m0 += 16) {
        const int rows = static_cast<int>(m - m0 < 16 ? m - m0 : 16);
        if (p.kind == LinearPlan::kMfma && rows >= 2) {
          const float* xc = x + m0 * im.k;
          float* const yc = y + m0 * im.n;
          const uint32_t rr = static_cast<uint32_t>(rows);
          if (rr >= kHalfMinRows) {
            const uint32_t parts = qi::gemv_half_splits(im.k, im.n, rr);
            QI_HIP_TRY(qi::launch_gemv_half_records(im.qtype, xc, im.k, rows, reinterpret_cast<uint8_t*>(dws), st),
                       "launch gemv rows activation records");
            QI_HIP_TRY(qi::launch_gemv_half(im.qtype, im.wide != 0, v, xc, rows, yc, sws, parts,
                                            reinterpret_cast<const uint8_t*>(dws), st),
                       "launch gemv rows");
            if (parts > 1) {
              const uint64_t count = static_cast<uint64_t>(rows) * im.n;
              QI_HIP_TRY(qi::launch_splitk_sum(im, v, sws, parts, count, count, yc, xc, st),
                         "launch gemv split-K sum");
            }
            continue;
          }
          const uint32_t parts = qi::gemv_rows_splits(im.k, im.n, rr);
          QI_HIP_TRY(qi::launch_gemv_rows(im.qtype, im.wide != 0, v, xc, rows, yc, sws, parts, st),
                     "launch gemv rows");
          if (parts > 1) {
            const uint64_t count = static_cast<uint64_t>(rows) * im.n;
            QI_HIP_TRY(qi::launch_splitk_sum(im, v, sws, parts, count, count, yc, xc, st),
                       "launch gemv split-K sum");
          }
        } else if (p.kind == LinearPlan::kMfma) {
          // one row
          const qi::GemvMfmaArgs ga{v, x + m0 * im.k, y + m0 * im.n, rows};
          const int split = w->ctx->gemv_split > 0 ? w->ctx->gemv_split : qi::gemv_mfma_split(im.k, im.n);
          QI_HIP_TRY(qi::launch_gemv_mfma(im.qtype, im.wide != 0, split, ga, st), "launch gemv");
        } else {
          const int mt = rows == 1 ? 1 : rows == 2 ? 2 : rows <= 4 ? 4 : rows <= 8 ? 8 : 16;
          qi::GemvArgs ga{v, x + m0 * im.k, y + m0 * im.n, rows};
          QI_HIP_TRY(qi::launch_gemv(im.qtype, im.wide != 0, mt, ga, st), "launch gemv");
        }
      }
      return QI_HIP_OK;
    case LinearPlan::kSplitGemm:
      for (uint64_t m0 = 0; m0 < m; m0 += kSplitChunkRows) {
        const uint64_t rows = m - m0 < kSplitChunkRows ? m - m0 : kSplitChunkRows;
        QI_HIP_TRY(qi::launch_gemm_split(im, v, x + m0 * im.k, rows, y + m0 * im.n, sws,
                                         qi::gemm_split_splits(im, rows), reinterpret_cast<uint8_t*>(dws), st),
                   "launch split-half gemm");
      }
      return QI_HIP_OK;
    case LinearPlan::kF32Gemv:
      for (uint64_t m0 = 0; m0 < m; m0 += 8) {
        const uint32_t rows = static_cast<uint32_t>(m - m0 < 8 ? m - m0 : 8);
        QI_HIP_TRY(qi::launch_f32w_gemv(im, v, x + m0 * im.k, rows, y + m0 * im.n, sws, p.splits, st),
                   "launch f32 gemv");
      }
      return QI_HIP_OK;
    case LinearPlan::kF32Gemm:
      QI_HIP_TRY(qi::launch_f32w_gemm(im, v, x, m, y, st), "launch f32 gemm");
      return QI_HIP_OK;
    case LinearPlan::kExact:
      QI_HIP_TRY(qi::launch_exact(im, v, x, m, y, st), "launch exact matmul");
      return QI_HIP_OK;
  }
  return fail(QI_HIP_RUNTIME_ERROR, "unknown linear plan");
}

qi_hip_status run_linear(qi_hip_ctx* c, const qi_hip_weights* w, const float* x, uint64_t m,
                         float* y, int32_t mode, hipStream_t st, float* silu_act, bool* silu_done) {
  if (silu_done != nullptr) *silu_done = false;
  LinearPlan p;
  qi_hip_status s = plan_linear(w->im, m, mode, &p);
  if (s != QI_HIP_OK) return s;
  if ((s = grow_ws(c, st, &c->hbuf, &c->hcap, p.h_floats, "alloc GEMM workspace")) != QI_HIP_OK) return s;
  if ((s = grow_ws(c, st, &c->sbuf, &c->scap, p.s_floats, "alloc split-K workspace")) != QI_HIP_OK) return s;
  if ((s = grow_ws(c, st, &c->dbuf, &c->dcap, p.d_floats, "alloc GEMV workspace")) != QI_HIP_OK) return s;
  const bool uses_ws = p.h_floats + p.s_floats + p.d_floats > 0;
  if (uses_ws && (s = ws_before(c, st)) != QI_HIP_OK) return s;
  if ((s = enqueue_linear(w, p, x, m, y, st, c->hbuf, c->sbuf, c->dbuf, silu_act, silu_done)) != QI_HIP_OK)
    return s;
  return uses_ws ? ws_after(c, st) : QI_HIP_OK;
}

qi_hip_status create_weights_locked(qi_hip_ctx* c, const Image& im, const void* blocks,
                                    qi_hip_weights** out) {
  QI_HIP_TRY(hipSetDevice(c->device), "set device");
  void* host = nullptr;
  QI_HIP_TRY(hipHostMalloc(&host, im.bytes, hipHostMallocDefault), "pinned staging");
  qi::fill_image(im, blocks, host);
  void* dev = nullptr;
  hipError_t e = hipMalloc(&dev, im.bytes);
  if (e == hipSuccess) e = hipMemcpyAsync(dev, host, im.bytes, hipMemcpyHostToDevice, c->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
  (void)hipHostFree(host);
  if (e != hipSuccess) {
    if (dev) (void)hipFree(dev);
    return hip_fail(e, "upload weights");
  }
  qi_hip_weights* w = new qi_hip_weights();
  c->refs.fetch_add(1, std::memory_order_relaxed);
  w->ctx = c;
  w->im = im;
  w->dev = dev;
  *out = w;
  return QI_HIP_OK;
}

void free_weights_locked(qi_hip_weights* w) {
  if (w == nullptr) return;
  (void)hipSetDevice(w->ctx->device);
  (void)hipStreamSynchronize(w->ctx->stream);
  if (w->dev) (void)hipFree(w->dev);
  w->ctx->refs.fetch_sub(1, std::memory_order_acq_rel);  // the caller still holds its own reference
  delete w;
}

}  // namespace qi_abi

using namespace qi_abi;

extern "C" {

int32_t qi_hip_abi_version(void) { return QI_HIP_ABI_VERSION; }

const char* qi_hip_last_error(void) { return g_last_error.c_str(); }

qi_hip_status qi_hip_open(int32_t device, qi_hip_ctx** out) {
  if (out == nullptr) return fail(QI_HIP_INVALID_INPUT, "null output pointer");
  *out = nullptr;
  int count = 0;
  hipError_t e = hipGetDeviceCount(&count);
  if (e != hipSuccess || count == 0)
    return fail(QI_HIP_UNSUPPORTED, "no HIP device is available");
  if (device < 0 || device >= count) return fail(QI_HIP_UNSUPPORTED, "HIP device ordinal out of range");
  hipDeviceProp_t prop;
  e = hipGetDeviceProperties(&prop, device);
  if (e != hipSuccess) return hip_fail(e, "device properties");
  if (strncmp(prop.gcnArchName, "gfx950", 6) != 0)
    return fail(QI_HIP_UNSUPPORTED, std::string("device is ") + prop.gcnArchName + ", gfx950 is required");
  e = hipSetDevice(device);
  if (e != hipSuccess) return hip_fail(e, "set device");
  qi_hip_ctx* c = new qi_hip_ctx();
  c->device = device;
  if (const char* env = getenv("QI_HIP_GEMV_SPLIT")) c->gemv_split = atoi(env);
  c->name = prop.name[0] ? std::string(prop.name) : std::string("AMD ") + prop.gcnArchName;
  e = hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking);
  if (e == hipSuccess) e = hipEventCreateWithFlags(&c->ws_event, hipEventDisableTiming | hipEventDisableSystemFence);
  if (e == hipSuccess) {
    const qi_hip_status st = scratch_setup(device, &c->scratch);
    if (st != QI_HIP_OK) {
      ctx_destroy(c);
      return st;
    }
  }
  if (e != hipSuccess) {
    ctx_destroy(c);
    return hip_fail(e, "context setup");
  }
  *out = c;
  return QI_HIP_OK;
}

void qi_hip_close(qi_hip_ctx* c) {
  if (c == nullptr) return;
  {
    std::lock_guard<std::mutex> lock(c->mu);
    if (c->closed) return;  // a second close of the same handle is a no-op
    c->closed = true;
  }
  ctx_release(c);
}

qi_hip_status qi_hip_device_name(qi_hip_ctx* c, char* buf, size_t len) {
  if (c == nullptr || buf == nullptr || len == 0) return fail(QI_HIP_INVALID_INPUT, "null argument");
  strncpy(buf, c->name.c_str(), len - 1);
  buf[len - 1] = '\0';
  return QI_HIP_OK;
}

qi_hip_status qi_hip_pack_weights(int32_t qtype, int32_t layout, uint64_t k, uint64_t n,
                                  const void* blocks, uint64_t count, void* out, uint64_t* bytes,
                                  int32_t* f16_scales) {
  if (bytes == nullptr) return fail(QI_HIP_INVALID_INPUT, "null size pointer");
  Image im;
  const char* why = "";
  qi_hip_status s = qi::plan_image(qtype, layout, k, n, blocks, count, &im, &why);
  if (s != QI_HIP_OK) return fail(s, why);
  if (out != nullptr) {
    if (*bytes < im.bytes) return fail(QI_HIP_INVALID_INPUT, "output buffer too small");
    qi::fill_image(im, blocks, out);
  }
  *bytes = im.bytes;
  if (f16_scales) *f16_scales = im.wide ? 0 : 1;
  return QI_HIP_OK;
}

qi_hip_status qi_hip_pack_gguf(int32_t qtype, int32_t layout, uint64_t k, uint64_t n, const void* wire,
                               uint64_t wire_bytes, int32_t legacy, void* out, uint64_t* bytes,
                               int32_t* f16_scales) {
  std::vector<uint8_t> blocks;
  uint64_t count = 0;
  const char* why = "";
  const qi_hip_status s = qi::gguf_decode(qtype, wire, wire_bytes, legacy, &blocks, &count, &why);
  if (s != QI_HIP_OK) return fail(s, why);
  return qi_hip_pack_weights(qtype, layout, k, n, blocks.data(), count, out, bytes, f16_scales);
}

qi_hip_status qi_hip_weights_create_gguf(qi_hip_ctx* c, int32_t qtype, int32_t layout, uint64_t k,
                                         uint64_t n, const void* wire, uint64_t wire_bytes, int32_t legacy,
                                         qi_hip_weights** out) {
  if (c == nullptr || out == nullptr) return fail(QI_HIP_INVALID_INPUT, "null context or output");
  *out = nullptr;
  std::vector<uint8_t> blocks;
  uint64_t count = 0;
  const char* why = "";
  const qi_hip_status s = qi::gguf_decode(qtype, wire, wire_bytes, legacy, &blocks, &count, &why);
  if (s != QI_HIP_OK) return fail(s, why);
  return qi_hip_weights_create(c, qtype, layout, k, n, blocks.data(), count, out);
}

qi_hip_status qi_hip_weights_create(qi_hip_ctx* c, int32_t qtype, int32_t layout, uint64_t k,
                                    uint64_t n, const void* blocks, uint64_t count,
                                    qi_hip_weights** out) {
  if (c == nullptr || out == nullptr) return fail(QI_HIP_INVALID_INPUT, "null context or output");
  *out = nullptr;
  if (c->closed) return fail(QI_HIP_INVALID_INPUT, "context is closed");
  Image im;
  const char* why = "";
  qi_hip_status s = qi::plan_image(qtype, layout, k, n, blocks, count, &im, &why);
  if (s != QI_HIP_OK) return fail(s, why);
  std::lock_guard<std::mutex> lock(c->mu);
  return create_weights_locked(c, im, blocks, out);
}

void qi_hip_weights_free(qi_hip_weights* w) {
  if (w == nullptr) return;
  qi_hip_ctx* c = w->ctx;
  if (c) {
    {
      std::lock_guard<std::mutex> lock(c->mu);
      (void)hipSetDevice(c->device);
      (void)hipStreamSynchronize(c->stream);
      if (w->dev) (void)hipFree(w->dev);
    }
    ctx_release(c);
  }
  delete w;
}

qi_hip_status qi_hip_weights_info_get(const qi_hip_weights* w, qi_hip_weights_info* out) {
  if (w == nullptr || out == nullptr) return fail(QI_HIP_INVALID_INPUT, "null argument");
  out->qtype = w->im.qtype;
  out->layout = w->im.layout;
  out->k = w->im.k;
  out->n = w->im.n;
  out->device_bytes = w->im.bytes;
  out->f16_scales = w->im.wide ? 0 : 1;
  return QI_HIP_OK;
}

constexpr uint64_t kStageFloats = 16ull << 20;  // 64 MiB
constexpr uint64_t kDirectFloats = 1ull << 20;  // 4 MiB

qi_hip_status qi_hip_linear(qi_hip_ctx* c, const qi_hip_weights* w, const float* x_host, uint64_t m,
                            float* y_host, int32_t mode) {
  qi_hip_status s = check_call(c, w, m);
  if (s != QI_HIP_OK) return s;
  if (x_host == nullptr || y_host == nullptr) return fail(QI_HIP_INVALID_INPUT, "null activation buffer");
  std::lock_guard<std::mutex> lock(c->mu);
  QI_HIP_TRY(hipSetDevice(c->device), "set device");
  const uint64_t xn = m * w->im.k, yn = m * w->im.n;
  if ((s = grow(&c->xbuf, &c->xcap, xn + 64, "alloc activations")) != QI_HIP_OK) return s;
  if ((s = grow(&c->ybuf, &c->ycap, yn, "alloc outputs")) != QI_HIP_OK) return s;
  // Activations up to 64 MiB each way are staged through pinned host buffers
  // (a host memcpy, then an asynchronous DMA); larger ones are copied from the
  // caller's pageable memory directly.
  const bool staged = xn <= kStageFloats && yn <= kStageFloats;
  if (staged) {
    if ((s = grow_pinned(&c->hx, &c->hxcap, xn)) != QI_HIP_OK) return s;
    if ((s = grow_pinned(&c->hy, &c->hycap, yn)) != QI_HIP_OK) return s;
    memcpy(c->hx, x_host, xn * 4);
  }
  QI_HIP_TRY(hipMemcpyAsync(c->xbuf, staged ? c->hx : x_host, xn * 4, hipMemcpyHostToDevice, c->stream),
             "copy x");
  // Outputs up to 4 MiB go from the kernels straight into the pinned buffer
  // (device-mapped host memory, visible to the host once the stream is
  // synchronized), which saves the device-to-host copy.
  const bool direct = staged && yn <= kDirectFloats;
  s = run_linear(c, w, c->xbuf, m, direct ? c->hy : c->ybuf, mode, c->stream);
  if (s != QI_HIP_OK) return s;
  if (!direct)
    QI_HIP_TRY(hipMemcpyAsync(staged ? c->hy : y_host, c->ybuf, yn * 4, hipMemcpyDeviceToHost, c->stream),
               "copy y");
  QI_HIP_TRY(hipStreamSynchronize(c->stream), "synchronize");
  if (staged) memcpy(y_host, c->hy, yn * 4);
  return QI_HIP_OK;
}

qi_hip_status qi_hip_linear_device(qi_hip_ctx* c, const qi_hip_weights* w, const float* x_dev,
                                   uint64_t m, float* y_dev, int32_t mode, void* stream) {
  qi_hip_status s = check_call(c, w, m);
  if (s != QI_HIP_OK) return s;
  if (x_dev == nullptr || y_dev == nullptr) return fail(QI_HIP_INVALID_INPUT, "null activation buffer");
  // the kernels read activation rows with 16-byte loads
  if ((reinterpret_cast<uintptr_t>(x_dev) | reinterpret_cast<uintptr_t>(y_dev)) & 15u)
    return fail(QI_HIP_INVALID_INPUT, "device activation and output buffers must be 16-byte aligned");
  std::lock_guard<std::mutex> lock(c->mu);
  QI_HIP_TRY(hipSetDevice(c->device), "set device");
  hipStream_t st = stream ? static_cast<hipStream_t>(stream) : c->stream;
  return run_linear(c, w, x_dev, m, y_dev, mode, st);
}

qi_hip_status qi_hip_linear_device_noalloc(qi_hip_ctx* c, const qi_hip_weights* w, const float* x_dev,
                                           uint64_t m, float* y_dev, int32_t mode, void* stream) {
  qi_hip_status s = check_call(c, w, m);
  if (s != QI_HIP_OK) return s;
  if (x_dev == nullptr || y_dev == nullptr) return fail(QI_HIP_INVALID_INPUT, "null activation buffer");
  if ((reinterpret_cast<uintptr_t>(x_dev) | reinterpret_cast<uintptr_t>(y_dev)) & 15u)
    return fail(QI_HIP_INVALID_INPUT, "device activation and output buffers must be 16-byte aligned");
  std::lock_guard<std::mutex> lock(c->mu);
  QI_HIP_TRY(hipSetDevice(c->device), "set device");
  LinearPlan p;
  if ((s = plan_linear(w->im, m, mode, &p)) != QI_HIP_OK) return s;
  auto a256 = [](uint64_t floats) { return (floats * 4 + 255) & ~static_cast<uint64_t>(255); };
  const uint64_t hb = a256(p.h_floats), sb = a256(p.s_floats), db = a256(p.d_floats);
  if (hb + sb + db > kScratchBytes)
    return fail(QI_HIP_INVALID_INPUT, "this call needs " + std::to_string(hb + sb + db) +
                                          " bytes of scratch; the no-allocation entry point holds " +
                                          std::to_string(kScratchBytes));
  // every workspace is written in full before it is read: nothing to clear
  uint8_t* base = static_cast<uint8_t*>(c->scratch);
  float* hws = reinterpret_cast<float*>(base);
  float* sws = reinterpret_cast<float*>(base + hb);
  float* dws = reinterpret_cast<float*>(base + hb + sb);
  hipStream_t st = stream ? static_cast<hipStream_t>(stream) : c->stream;
  return enqueue_linear(w, p, x_dev, m, y_dev, st, hws, sws, dws, nullptr, nullptr);
}

qi_hip_status qi_hip_dequantize_device(qi_hip_ctx* c, const qi_hip_weights* w, float* out_dev,
                                       void* stream) {
  if (c == nullptr || w == nullptr || out_dev == nullptr) return fail(QI_HIP_INVALID_INPUT, "null argument");
  if (c->closed) return fail(QI_HIP_INVALID_INPUT, "context is closed");
  if (w->ctx != c) return fail(QI_HIP_INVALID_INPUT, "weights belong to another context");
  std::lock_guard<std::mutex> lock(c->mu);
  QI_HIP_TRY(hipSetDevice(c->device), "set device");
  hipStream_t st = stream ? static_cast<hipStream_t>(stream) : c->stream;
  QI_HIP_TRY(qi::launch_dequant(w->im, qi::make_view(w->im, w->dev), out_dev, st), "launch dequant");
  return QI_HIP_OK;
}

qi_hip_status qi_hip_dequantize(qi_hip_ctx* c, const qi_hip_weights* w, float* out_host) {
  if (c == nullptr || w == nullptr || out_host == nullptr) return fail(QI_HIP_INVALID_INPUT, "null argument");
  if (c->closed) return fail(QI_HIP_INVALID_INPUT, "context is closed");
  if (w->ctx != c) return fail(QI_HIP_INVALID_INPUT, "weights belong to another context");
  std::lock_guard<std::mutex> lock(c->mu);
  QI_HIP_TRY(hipSetDevice(c->device), "set device");
  const uint64_t n = w->im.k * w->im.n;
  float* tmp = nullptr;
  QI_HIP_TRY(hipMalloc(reinterpret_cast<void**>(&tmp), n * 4), "alloc dequant output");
  hipError_t e = qi::launch_dequant(w->im, qi::make_view(w->im, w->dev), tmp, c->stream);
  if (e == hipSuccess) e = hipMemcpyAsync(out_host, tmp, n * 4, hipMemcpyDeviceToHost, c->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
  (void)hipFree(tmp);
  if (e != hipSuccess) return hip_fail(e, "dequantize");
  return QI_HIP_OK;
}

}  // extern "C"
