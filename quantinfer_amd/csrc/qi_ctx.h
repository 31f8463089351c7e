// Internal: the context and weights handles behind include/qi_hip.h, shared by
// the C ABI (qi_abi.hip) and the Qwen3 decoder (qi_qwen3.hip).
#pragma once

#include <hip/hip_runtime.h>

#include <atomic>
#include <mutex>
#include <string>

#include "../../include/qi_hip.h"
#include "qi_image.h"

// A context is reference counted: the caller's handle and every live weights
// handle hold one reference, so qi_hip_close and qi_hip_weights_free may come
// in any order; the stream and workspace go away with the last reference.
struct qi_hip_ctx {
  std::atomic<int> refs{1};
  bool closed = false;
  int device = 0;
  hipStream_t stream = nullptr;
  std::mutex mu;
  std::string name;
  // Order of work that uses the workspaces below (hbuf, sbuf, dbuf): calls
  // may enqueue on different caller streams, so the launches of a call that
  // uses a workspace wait (hipStreamWaitEvent) for ws_event, recorded after
  // the previous such call's launches on ws_stream. A workspace is
  // reallocated only after ws_event has completed.
  hipEvent_t ws_event = nullptr;
  hipStream_t ws_stream = nullptr;
  bool ws_used = false;
  float* xbuf = nullptr;
  uint64_t xcap = 0;  // floats
  float* ybuf = nullptr;
  uint64_t ycap = 0;
  // pinned host staging of qi_hip_linear (hipHostMalloc), so that its copies
  // are asynchronous DMA transfers instead of pageable-memory copies
  float* hx = nullptr;
  uint64_t hxcap = 0;  // floats
  float* hy = nullptr;
  uint64_t hycap = 0;
  float* hbuf = nullptr;  // f16 activations of the prefill GEMM (capacity in floats)
  uint64_t hcap = 0;
  float* sbuf = nullptr;  // split-K partial products of the prefill GEMM (capacity in floats)
  uint64_t scap = 0;
  float* dbuf = nullptr;  // activation records of the decode GEMV, 2+ rows (capacity in floats)
  uint64_t dcap = 0;
  int gemv_split = 0;  // QI_HIP_GEMV_SPLIT tuning override (wavefronts per GEMV workgroup: 4 or 8)
  void* scratch = nullptr;  // device address of this device's scratch array (qi_abi.hip)
};

struct qi_hip_weights {
  qi_hip_ctx* ctx = nullptr;
  qi::Image im;
  void* dev = nullptr;
};

namespace qi_abi {

// Set the calling thread's last error and return `st`.
qi_hip_status fail(qi_hip_status st, const std::string& msg);
qi_hip_status hip_fail(hipError_t e, const char* what);
// Grow-only device buffer (capacity in floats); the caller synchronizes first
// when queued work may still read the old buffer.
qi_hip_status grow(float** buf, uint64_t* cap, uint64_t need, const char* what);
// One linear layer on device buffers, no locking (the caller holds c->mu).
// With `silu_act` (an image whose 16-output tiles hold 8 gate rows then the 8
// matching up rows): when the layer runs as one MFMA GEMM launch without a K
// split, the GEMM writes SiLU(gate) * up of each pair to silu_act ([m][n/2])
// instead of y and *silu_done is set; otherwise y is written as usual.
qi_hip_status run_linear(qi_hip_ctx* c, const qi_hip_weights* w, const float* x, uint64_t m,
                         float* y, int32_t mode, hipStream_t st, float* silu_act = nullptr,
                         bool* silu_done = nullptr);
// Upload a planned image; the caller holds c->mu. The handle holds a context
// reference, as one made by qi_hip_weights_create.
qi_hip_status create_weights_locked(qi_hip_ctx* c, const qi::Image& im, const void* blocks,
                                    qi_hip_weights** out);
// Free a handle made by create_weights_locked while holding c->mu (the caller
// keeps its own context reference, so the context cannot go away here).
void free_weights_locked(qi_hip_weights* w);
void ctx_release(qi_hip_ctx* c);
// Number of workspace reallocations so far (any context): a captured graph
// that reads a workspace is stale once this changes.
uint64_t workspace_version();
// Before enqueueing work that uses a context workspace on `st`: make st wait
// for the previous workspace user (another stream). After enqueueing it:
// record it as the last user. No-ops while st is under graph capture.
qi_hip_status ws_before(qi_hip_ctx* c, hipStream_t st);
qi_hip_status ws_after(qi_hip_ctx* c, hipStream_t st);

}  // namespace qi_abi

#define QI_HIP_TRY(expr, what)                                   \
  do {                                                           \
    hipError_t e_ = (expr);                                      \
    if (e_ != hipSuccess) return qi_abi::hip_fail(e_, what);     \
  } while (0)
