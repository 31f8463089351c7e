/*
 * qi_hip: MI355X (gfx950) quantized-linear backend for QuantInfer, C ABI.
 *
 * This is the drop-in boundary a `backends/hip` crate binds. It replaces the
 * quantized-matmul methods of the reference's operator contract
 *   trait KernelBackend            crates/quantinfer-kernel/src/lib.rs:83-154
 * for the GGML block formats Q8_0, Q4_0, Q4_K, Q5_K, Q6_K (and F32), in both
 * the row-major (QuantInfer) and output-rows (GGML) layouts.
 *
 * Conventions follow the reference's own C ABI (bindings/c/include/quantinfer.h:
 * 12-19 status codes, :36-37 thread-local last error):
 *  - every call returns a qi_hip_status; on failure qi_hip_last_error() holds a
 *    message for the calling thread;
 *  - plain pointers and sizes only; the caller owns host buffers; a weights
 *    handle owns its device memory; a context owns its stream, its scratch
 *    workspace and a mutex (calls on one context are serialized, handles may
 *    cross threads);
 *  - status -> reference error: QI_HIP_INVALID_INPUT -> KernelError::InvalidInput,
 *    QI_HIP_UNSUPPORTED and QI_HIP_RUNTIME_ERROR -> KernelError::Unsupported
 *    (crates/quantinfer-kernel/src/lib.rs:14-19; the device-failure mapping is
 *    the one backends/cuda/src/native.rs:238-244 uses).
 */
#ifndef QI_HIP_H
#define QI_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define QI_HIP_ABI_VERSION 1

typedef int32_t qi_hip_status;
#define QI_HIP_OK 0
#define QI_HIP_INVALID_INPUT 1
#define QI_HIP_UNSUPPORTED 2
#define QI_HIP_RUNTIME_ERROR 3

/* Weight element types (core DType / runtime LinearWeight variants,
 * crates/quantinfer-runtime/src/linear.rs:14-30). */
#define QI_HIP_F32 0
#define QI_HIP_Q8_0 1
#define QI_HIP_Q4_0 2
#define QI_HIP_Q4_K 3
#define QI_HIP_Q5_K 4
#define QI_HIP_Q6_K 5

/* Layouts of the logical RHS [K, N] (core quantized/mod.rs:10 names the second):
 * ROW_MAJOR   element (k, n) at flat index k*N + n; blocks run along N
 *             (backends/cpu/src/matmul.rs:162-168).
 * OUTPUT_ROWS blocks ordered output-major: output n owns K/bs consecutive
 *             blocks (crates/quantinfer-kernel/src/lib.rs:101, matmul.rs:141-158). */
#define QI_HIP_LAYOUT_ROW_MAJOR 0
#define QI_HIP_LAYOUT_OUTPUT_ROWS 1

/* Arithmetic modes of a linear call.
 * AUTO  F32 below 128 activation rows, MFMA at 128 and above (the decode /
 *       prefill split of the kernels).
 * F32   f32-accurate for any M, judged by tolerance (1e-5) against the CPU
 *       reference: f32 GEMV kernels, and for output rows (K a multiple of
 *       256) from 33 rows a matrix-core GEMM of exact products (activations
 *       split into two f16 halves, weights as exact f16 codes or two f16
 *       halves) accumulated in f32.
 * EXACT bit-identical to CpuScalar: per output, acc = acc + x[k]*w[k] in f32,
 *       k ascending, no FMA (backends/cpu/src/matmul.rs:146-157, 319-330).
 * MFMA  f16 operands into f32 matrix-core accumulation (prefill GEMM). */
#define QI_HIP_MODE_AUTO 0
#define QI_HIP_MODE_F32 1
#define QI_HIP_MODE_EXACT 2
#define QI_HIP_MODE_MFMA 3

/* Logical blocks: field-for-field the reference core structs, which are not
 * repr(C); the Rust glue copies fields into these. No padding. */
typedef struct { float scale; int8_t values[32]; } qi_hip_q8_0_block;     /* core quantized/q8.rs:7-11  */
typedef struct { float scale; uint8_t values[32]; } qi_hip_q4_0_block;    /* core quantized/q4.rs:7-13  */
typedef struct {
  float scale, min_scale;
  uint8_t scales[12];
  uint8_t values[128];
} qi_hip_q4_k_block;                                                      /* core quantized/q4.rs:72-78 */
typedef struct {
  float scale, min_scale;
  uint8_t scales[12];
  uint8_t high_bits[32];
  uint8_t values[128];
} qi_hip_q5_k_block;                                                      /* core quantized/k.rs:7-14   */
typedef struct {
  float scale;
  int8_t scales[16];
  uint8_t low_bits[128];
  uint8_t high_bits[64];
} qi_hip_q6_k_block;                                                      /* core quantized/k.rs:55-61  */

typedef struct qi_hip_ctx qi_hip_ctx;
typedef struct qi_hip_weights qi_hip_weights;

typedef struct {
  int32_t qtype, layout;
  uint64_t k, n;
  uint64_t device_bytes;   /* bytes of the resident device image */
  int32_t f16_scales;      /* 1: every scale is f16-exact, so the image has GGUF wire size */
} qi_hip_weights_info;

/* ABI version; the glue refuses a library whose version differs. */
int32_t qi_hip_abi_version(void);

/* Message of the calling thread's last failure ("" if none). */
const char *qi_hip_last_error(void);

/* Open device `device` (HIP ordinal). QI_HIP_UNSUPPORTED when no gfx950 device
 * is visible or the HIP runtime is unavailable.
 * Replaces: CudaBackend::open (backends/cuda/src/native.rs:29-57). */
qi_hip_status qi_hip_open(int32_t device, qi_hip_ctx **out);
void qi_hip_close(qi_hip_ctx *ctx);

/* Device marketing name, NUL-terminated into buf.
 * Replaces: CudaBackend::device_name (backends/cuda/src/native.rs:59-61). */
qi_hip_status qi_hip_device_name(qi_hip_ctx *ctx, char *buf, size_t len);

/* Upload logical blocks as a resident weight of logical shape [K, N].
 * `blocks` holds `count` qi_hip_*_block structs of `qtype` in the reference's
 * block order for `layout`, or K*N f32 values (row-major [K, N]) for QI_HIP_F32.
 * Validation is the reference's: QuantizedTensor*::from_blocks
 * (core quantized/q8.rs:20-40, q4.rs:22-51, q4.rs:87-120, k.rs:23-41, k.rs:70-85)
 * plus the matmul shape checks (backends/cpu/src/matmul.rs:131-140, 293-314).
 * Replaces: the per-call weight upload of CudaBackend::multiply
 * (backends/cuda/src/native.rs:99-104) with a resident handle. */
qi_hip_status qi_hip_weights_create(qi_hip_ctx *ctx, int32_t qtype, int32_t layout, uint64_t k,
                                    uint64_t n, const void *blocks, uint64_t count,
                                    qi_hip_weights **out);
void qi_hip_weights_free(qi_hip_weights *w);
qi_hip_status qi_hip_weights_info_get(const qi_hip_weights *w, qi_hip_weights_info *out);

/* y[M, N] = x[M, K] * W, host buffers, synchronous.
 * Replaces: KernelBackend::matmul (lib.rs:95), matmul_q8_0 / matmul_q4_0
 * (lib.rs:97-99), matmul_q8_0_output_rows / matmul_q4_0_output_rows
 * (lib.rs:102-113), matmul_q4_k / q5_k / q6_k (lib.rs:115-119) and
 * matmul_q{4,5,6}_k_output_rows (lib.rs:122-140): the variant is selected by the
 * handle's qtype and layout. x and y pass through pinned host buffers the
 * context keeps (grown to the largest call up to 64 MiB each way, freed at
 * close); larger ones are copied from and to the caller's memory directly. */
qi_hip_status qi_hip_linear(qi_hip_ctx *ctx, const qi_hip_weights *w, const float *x_host,
                            uint64_t m, float *y_host, int32_t mode);

/* Same on device buffers, enqueued on `stream` (a hipStream_t; NULL = the
 * context's stream). Returns after the launch; no host synchronisation.
 * x_dev and y_dev must be 16-byte aligned (QI_HIP_INVALID_INPUT otherwise). */
qi_hip_status qi_hip_linear_device(qi_hip_ctx *ctx, const qi_hip_weights *w, const float *x_dev,
                                   uint64_t m, float *y_dev, int32_t mode, void *stream);

/* qi_hip_linear_device for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc). No counterpart in the reference. Same kernels and results as
 * qi_hip_linear_device, but every workspace (the GEMM's f16 activations and
 * split-K partials, the activation records of the multi-row GEMV and of F32
 * mode's split-half GEMM, the K-part sums of row-major calls of 3 rows or
 * more, at most 32 MB) is carved out of a fixed 64 MiB scratch array the
 * library holds on each GPU until the process ends; no call allocates or
 * frees. A call whose workspaces exceed 64 MiB is refused with
 * QI_HIP_INVALID_INPUT (the f16 GEMM takes 2*M*K bytes of f16 activations, M
 * rounded up to 128, plus split-K partials when fewer than 256 row x column
 * blocks: every BASELINE GEMM shape fits; the split-half GEMM about 4.1*M*K
 * bytes, M rounded up to 64 and at most 4096 per launch). Every call on one GPU
 * shares that GPU's array: calls that overlap on one GPU (other streams, other
 * threads, other contexts on the same device) race, and the caller must order
 * them. Nothing in the array needs clearing between calls. */
qi_hip_status qi_hip_linear_device_noalloc(qi_hip_ctx *ctx, const qi_hip_weights *w, const float *x_dev,
                                           uint64_t m, float *y_dev, int32_t mode, void *stream);

/* Bit-exact f32 dequantization in block order (K*N floats).
 * Replaces: dequantize_q8_0 / q4_0 / q4_k / q5_k / q6_k
 * (crates/quantinfer-quant/src/schemes/q8.rs:33-45, q4.rs:35-47, q4_k.rs:90-121,
 * q5_k.rs:96-135, q6_k.rs:74-103). */
qi_hip_status qi_hip_dequantize(qi_hip_ctx *ctx, const qi_hip_weights *w, float *out_host);
qi_hip_status qi_hip_dequantize_device(qi_hip_ctx *ctx, const qi_hip_weights *w, float *out_dev,
                                       void *stream);

/* Host-only: build the device image of a weight without a device (validation
 * and packing exactly as qi_hip_weights_create). With out == NULL only the
 * size is returned in *bytes. Replaces the GGUF block writers' role
 * (crates/quantinfer-format/src/gguf/writer.rs:183-261) for the device layout. */
qi_hip_status qi_hip_pack_weights(int32_t qtype, int32_t layout, uint64_t k, uint64_t n,
                                  const void *blocks, uint64_t count, void *out, uint64_t *bytes,
                                  int32_t *f16_scales);

/* Upload a GGUF tensor's block bytes directly: `wire` holds `wire_bytes` bytes
 * of GGUF wire blocks of `qtype` (Q8_0 34 B, Q4_0 18 B, Q4_K 144 B, Q5_K 176 B,
 * Q6_K 210 B per block; QI_HIP_F32: little-endian f32 values) in the block
 * order of `layout`. legacy = 1 reads the files' old layout (Q4_0 nibble pairs
 * (2j, 2j+1); Q6_K d, scales, ql, qh), which the reader selects by file
 * version (format/src/gguf/decode.rs:168-172, 288-290); the other types ignore
 * it. Decoding and validation are the reference's GGUF block readers
 * (format/src/gguf/decode.rs:90-312: byte length a multiple of the block
 * size, finite f16 scales), then as qi_hip_weights_create.
 * Replaces: GgufFile::tensor_q8_0 / tensor_q4_0 / tensor_q4_k / tensor_q5_k /
 * tensor_q6_k (format/src/gguf/decode.rs:90-312) followed by the upload. */
qi_hip_status qi_hip_weights_create_gguf(qi_hip_ctx *ctx, int32_t qtype, int32_t layout, uint64_t k,
                                         uint64_t n, const void *wire, uint64_t wire_bytes,
                                         int32_t legacy, qi_hip_weights **out);
/* Host-only: the device image of a GGUF tensor, as qi_hip_pack_weights. */
qi_hip_status qi_hip_pack_gguf(int32_t qtype, int32_t layout, uint64_t k, uint64_t n,
                               const void *wire, uint64_t wire_bytes, int32_t legacy, void *out,
                               uint64_t *bytes, int32_t *f16_scales);

/* Host-only: quantize n f32 values (a multiple of 32 for Q8_0/Q4_0, of 256
 * for the K-quants) into out_count = n / block-size logical blocks of `qtype`,
 * bit for bit as the reference's quantizers: quantize_q8_0 / q4_0 / q4_k /
 * q5_k / q6_k (crates/quantinfer-quant/src/schemes/q8.rs:8-31, q4.rs:8-33,
 * q4_k.rs:8-88, q5_k.rs:8-94, q6_k.rs:8-72). storage_f16 = 1 then rounds every
 * scale to its f16 storage value as QuantizedData::with_storage_precision
 * (quant/src/providers/storage.rs:28-87; the K-quant scales already are).
 * Blocks are split over `threads` host threads (<= 0: one per hardware
 * thread); the result does not depend on the count. QI_HIP_INVALID_INPUT for a
 * non-finite value, a bad count or a scale f16 cannot hold finitely (the
 * reference's QuantizationError::InvalidInput); `out` is then unspecified. */
qi_hip_status qi_hip_quantize(int32_t qtype, const float *values, uint64_t n, int32_t storage_f16,
                              void *out, uint64_t out_count, int32_t threads);

/* Host-only synthetic inputs (no counterpart in the reference; used to build
 * benchmark weights and activations of a stated distribution): out[i] =
 * z_i * s_i for n elements, z_i standard normal by Box-Muller from
 * counter-based SplitMix64 draws 3i and 3i+1 of `seed`, s_i = outlier_std when
 * draw 3i+2 (uniform on (0, 1]) is <= outlier_rate, else std. Independent of
 * the thread count (<= 0: one per hardware thread). */
qi_hip_status qi_hip_synth_normal(uint64_t seed, uint64_t n, double std, double outlier_rate,
                                  double outlier_std, float *out, int32_t threads);

/* ------------------------------------------------------------------------
 * GPU-resident Qwen3 dense decoder.
 *
 * Replaces, for a model whose tensors live on the device: Qwen3Model::new /
 * forward / forward_batch (crates/quantinfer-runtime/src/qwen3/mod.rs:211-378),
 * KvCache (runtime/src/cache.rs:14-125) and generate_qwen3_stream with greedy
 * selection (runtime/src/generation.rs:58-76, 160-201). The layer arithmetic is
 * qwen3/mod.rs:117-208, attention.rs:7-141 and batch.rs:21-67; the element-wise
 * operators are the KernelBackend methods rms_norm, rms_norm_heads, silu_mul,
 * apply_rope and embedding (kernel lib.rs:142-153, cpu backend.rs:172-298).
 * Weights, activations and the KV cache stay in device memory; a call moves
 * only token ids (and, on request, the last row's logits) across PCIe.
 * ------------------------------------------------------------------------ */

/* The Qwen3Config fields the forward pass reads (crates/quantinfer-model/src/
 * qwen3.rs:11-37; head_dim is effective_head_dim()). */
typedef struct {
  uint32_t vocab_size;
  uint32_t hidden_size;
  uint32_t intermediate_size;
  uint32_t num_hidden_layers;
  uint32_t num_attention_heads;
  uint32_t num_key_value_heads;
  uint32_t head_dim;
  uint32_t max_position_embeddings;
  float rms_norm_eps;
  float rope_theta;
} qi_hip_qwen3_config;

/* One linear weight as the runtime holds it (LinearWeight, runtime/src/
 * linear.rs:14-30): qtype/layout as for qi_hip_weights_create, `data` the
 * logical blocks (or row-major f32 values for QI_HIP_F32), `count` the number
 * of blocks (of floats for QI_HIP_F32). Logical shape [K, N] = [in, out]. */
typedef struct {
  int32_t qtype;
  int32_t layout;
  const void *data;
  uint64_t count;
} qi_hip_linear_weight;

/* Qwen3LayerWeights (qwen3/mod.rs:10-22); norms are f32 host vectors. */
typedef struct {
  const float *input_layernorm;          /* [hidden] */
  const float *q_norm;                   /* [head_dim] */
  const float *k_norm;                   /* [head_dim] */
  const float *post_attention_layernorm; /* [hidden] */
  qi_hip_linear_weight q_proj;           /* [hidden, heads*head_dim] */
  qi_hip_linear_weight k_proj;           /* [hidden, kv_heads*head_dim] */
  qi_hip_linear_weight v_proj;           /* [hidden, kv_heads*head_dim] */
  qi_hip_linear_weight o_proj;           /* [heads*head_dim, hidden] */
  qi_hip_linear_weight gate_proj;        /* [hidden, intermediate] */
  qi_hip_linear_weight up_proj;          /* [hidden, intermediate] */
  qi_hip_linear_weight down_proj;        /* [intermediate, hidden] */
} qi_hip_qwen3_layer;

typedef struct qi_hip_qwen3 qi_hip_qwen3;
typedef struct qi_hip_kv_cache qi_hip_kv_cache;

/* Create an empty model on the context's device (Qwen3Model::new validation,
 * qwen3/mod.rs:220-258 and Qwen3Config::validate). head_dim must be 64 or 128,
 * hidden_size a multiple of 256. Every set_* call below must be made once
 * before the first forward. */
qi_hip_status qi_hip_qwen3_create(qi_hip_ctx *ctx, const qi_hip_qwen3_config *config,
                                  qi_hip_qwen3 **out);
/* embedding: f32 [vocab_size, hidden_size] row-major (the runtime's embedding
 * Tensor). */
qi_hip_status qi_hip_qwen3_set_embedding(qi_hip_qwen3 *model, const float *embedding);
/* Layer `index`: q/k/v and gate/up are fused into one device image each, so
 * each pair/triple must share qtype and layout. */
qi_hip_status qi_hip_qwen3_set_layer(qi_hip_qwen3 *model, uint32_t index,
                                     const qi_hip_qwen3_layer *layer);
/* final_norm: f32 [hidden]; lm_head: [hidden, vocab] (a Q6_K output-rows head
 * stays quantized on the device instead of being dequantized at load as
 * runtime/src/qwen3/loader.rs:47-61 does). */
qi_hip_status qi_hip_qwen3_set_output(qi_hip_qwen3 *model, const float *final_norm,
                                      const qi_hip_linear_weight *lm_head);
/* Arithmetic mode of every linear layer (QI_HIP_MODE_*). Default F32, whose
 * greedy ids equal the CPU run's (runtime/src/generation.rs:58-76); AUTO
 * prefills prompt chunks of 128+ tokens on the f16-operand GEMM instead. */
qi_hip_status qi_hip_qwen3_set_mode(qi_hip_qwen3 *model, int32_t mode);
void qi_hip_qwen3_free(qi_hip_qwen3 *model);

/* KvCache::new(num_layers, max_sequence_length, num_key_value_heads, head_dim)
 * (cache.rs:25-60), in device memory. */
qi_hip_status qi_hip_kv_cache_create(qi_hip_ctx *ctx, uint32_t num_layers,
                                     uint32_t max_sequence_length, uint32_t num_key_value_heads,
                                     uint32_t head_dim, qi_hip_kv_cache **out);
qi_hip_status qi_hip_kv_cache_length(const qi_hip_kv_cache *cache, uint64_t *out);
/* Forget every cached position (a fresh KvCache of the same shape). */
qi_hip_status qi_hip_kv_cache_reset(qi_hip_kv_cache *cache);
void qi_hip_kv_cache_free(qi_hip_kv_cache *cache);

/* Qwen3Model::forward(token_ids, cache) (qwen3/mod.rs:260-263, 297-335): runs
 * the tokens at the next cache positions and appends their keys/values.
 * Writes the LAST token's logits to `last_logits` ([vocab], host, may be NULL)
 * and their argmax (generation.rs:58-76) to `next_token` (may be NULL); the
 * rows before the last are not projected to logits. */
qi_hip_status qi_hip_qwen3_forward(qi_hip_qwen3 *model, qi_hip_kv_cache *cache,
                                   const int32_t *tokens, uint64_t count, float *last_logits,
                                   int32_t *next_token);

/* generate_qwen3_stream with temperature 0 (generation.rs:160-201): forward the
 * prompt, then repeatedly select the argmax and forward it, up to
 * max_new_tokens or until eos_token_id (< 0: none) is selected. Writes the
 * selected ids to out_tokens and their number to *out_count. Decode steps run
 * as one replayed HIP graph per token. */
qi_hip_status qi_hip_qwen3_generate(qi_hip_qwen3 *model, qi_hip_kv_cache *cache,
                                    const int32_t *prompt, uint64_t prompt_count,
                                    uint64_t max_new_tokens, int32_t eos_token_id,
                                    int32_t *out_tokens, uint64_t *out_count);

/* Device time of the last qi_hip_qwen3_generate on this model, from HIP events
 * on the context stream: the prompt forward and the decode steps. */
typedef struct {
  double prefill_ms;
  double decode_ms;
  uint64_t prompt_tokens;
  uint64_t decode_steps;
} qi_hip_qwen3_timing;
qi_hip_status qi_hip_qwen3_last_timing(const qi_hip_qwen3 *model, qi_hip_qwen3_timing *out);

#ifdef __cplusplus
}
#endif
#endif
