/*
 * CPU oracle for the quantized-linear hot path of aiqubits/quantinfer.
 *
 * TEST INFRASTRUCTURE ONLY. This library restates, in plain C, the reference
 * algorithms that define the numerics of the path (quantizers, dequantizers,
 * the CpuScalar output-row / row-major matmuls, the cpu-simd block dots, the
 * GGUF block wire codecs and the f16 storage rules). It is the checker for the
 * HIP product path and the CPU baseline timed by bench.py. Only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it; the
 * product library (quantinfer_amd/libqi_hip.so) never links or calls it.
 *
 * Every function cites the reference file:line it follows (paths relative to
 * the aiqubits/quantinfer source tree). Arithmetic is IEEE-754 binary32 with
 * no contraction (compiled with -ffp-contract=off, no fast-math), which is
 * what the reference's Rust code does (Rust never fuses a*b+c implicitly).
 *
 * Parity status of each part (how it is pinned) is listed in oracle.c's
 * header comment.
 */
#ifndef QI_ORACLE_H
#define QI_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes shared with the product ABI: 0 ok, 1 invalid input. */
#define QO_OK 0
#define QO_INVALID 1

/* Logical blocks, field-for-field the reference core structs. All have
 * natural alignment 4 and no padding. */
typedef struct { float scale; int8_t values[32]; } qo_q8_0_block;          /* core quantized/q8.rs:7-11  */
typedef struct { float scale; uint8_t values[32]; } qo_q4_0_block;         /* core quantized/q4.rs:7-13  */
typedef struct { float scale; float min_scale; uint8_t scales[12];
                 uint8_t values[128]; } qo_q4_k_block;                     /* core quantized/q4.rs:72-78 */
typedef struct { float scale; float min_scale; uint8_t scales[12];
                 uint8_t high_bits[32]; uint8_t values[128]; } qo_q5_k_block; /* core quantized/k.rs:7-14 */
typedef struct { float scale; int8_t scales[16]; uint8_t low_bits[128];
                 uint8_t high_bits[64]; } qo_q6_k_block;                   /* core quantized/k.rs:55-61  */

size_t qo_block_bytes(int qtype);   /* logical block size in bytes, 0 for an unknown type */
size_t qo_wire_bytes(int qtype);    /* GGUF wire block size in bytes */
size_t qo_block_elems(int qtype);   /* 32 or 256 */

/* qtype numbering (same as the product ABI) */
#define QO_F32 0
#define QO_Q8_0 1
#define QO_Q4_0 2
#define QO_Q4_K 3
#define QO_Q5_K 4
#define QO_Q6_K 5

/* ---- half-precision conversions (IEEE-754 binary16, round to nearest even) ---- */
uint16_t qo_f32_to_f16(float value);
float qo_f16_to_f32(uint16_t bits);
void qo_f32_to_f16_array(const float *in, size_t n, uint16_t *out);
void qo_f16_to_f32_array(const uint16_t *in, size_t n, float *out);
int qo_stored_f16_scale(float value, float *out);

/* ---- quantizers (reference quant/src/schemes) ---- */
int qo_quantize_q8_0(const float *values, size_t n, qo_q8_0_block *out);
int qo_quantize_q4_0(const float *values, size_t n, qo_q4_0_block *out);
int qo_quantize_q4_k(const float *values, size_t n, qo_q4_k_block *out);
int qo_quantize_q5_k(const float *values, size_t n, qo_q5_k_block *out);
int qo_quantize_q6_k(const float *values, size_t n, qo_q6_k_block *out);
/* with_storage_precision (quant/src/providers/storage.rs:28-87), in place */
int qo_storage_precision(int qtype, void *blocks, size_t count);
/* QuantizedTensor*::from_blocks validation (core quantized/{q8,q4,k}.rs) */
int qo_validate_blocks(int qtype, const void *blocks, size_t count, size_t elements);

/* ---- dequantizers (bit-exact targets) ---- */
int qo_dequantize(int qtype, const void *blocks, size_t count, float *out);
/* the per-element value of backends/cpu/src/matmul.rs:162-280 */
float qo_value(int qtype, const void *blocks, size_t index);

/* ---- CpuScalar matmuls ----
 * output rows: rhs logical [K, N], blocks ordered output-major (row n holds
 *   K/bs consecutive blocks); y[M, N] (matmul.rs:119-160, 282-332).
 * row major: rhs logical [K, N], element (k, n) at flat index k*N+n
 *   (matmul.rs:14-32 with quantized_value*).
 * f32: rhs [K, N] row-major f32 (matmul.rs:92-117).
 * Returns QO_INVALID on the shape errors the reference rejects. */
int qo_matmul_output_rows(int qtype, const float *x, size_t m, size_t k,
                          const void *blocks, size_t nblocks, size_t n, float *y);
int qo_matmul_row_major(int qtype, const float *x, size_t m, size_t k,
                        const void *blocks, size_t nblocks, size_t n, float *y);
int qo_matmul_f32(const float *x, size_t m, size_t k, const float *w, size_t n, float *y);
/* Row-parallel restatement (rows split across `threads` workers; per-output
 * arithmetic unchanged, so it is bit-identical to the scalar call). */
int qo_matmul_output_rows_threaded(int qtype, const float *x, size_t m, size_t k,
                                   const void *blocks, size_t nblocks, size_t n,
                                   float *y, int threads);

/* ---- cpu-simd Q8_0 / Q4_0 output-row variants (backends/cpu/src/matmul.rs:334-412,
 * backends/cpu-simd/src/lib.rs:100-129, 179-204). isa: 1 = AVX2, 2 = AVX-512.
 * Returns QO_INVALID if the host lacks the ISA. ---- */
int qo_simd_isa_available(int isa);
int qo_matmul_output_rows_simd(int qtype, int isa, const float *x, size_t m, size_t k,
                               const void *blocks, size_t nblocks, size_t n, float *y);

/* ---- GGUF block wire codecs (format/src/gguf/writer.rs:183-261, decode.rs:90-312) ---- */
int qo_wire_pack(int qtype, const void *blocks, size_t count, uint8_t *out);
int qo_wire_unpack(int qtype, const uint8_t *bytes, size_t count, int legacy, void *blocks);

/* ---- deterministic synthetic inputs ----
 * SplitMix64 stream -> Box-Muller (double) -> f32 * std. With outlier_rate > 0,
 * each element is independently replaced by N(0, outlier_std^2) with that
 * probability (the K-quant configs use 0.005 and 0.2). */
void qo_fill_normal(uint64_t seed, size_t n, double std, double outlier_rate,
                    double outlier_std, float *out);

/* ---- Qwen3 dense decoder (oracle/qwen3.c; runtime/src/qwen3/mod.rs,
 * attention.rs, batch.rs, cache.rs, generation.rs, cpu backend.rs:172-298) ---- */
int qo_rms_norm(const float *x, size_t rows, size_t dim, const float *w, float eps, float *out);
int qo_softmax(const float *x, size_t rows, size_t dim, float *out);
int qo_silu_mul(const float *gate, const float *up, size_t n, float *out);
int qo_rope_tables(float theta, size_t head_dim, size_t start, size_t length, float *cos_out,
                   float *sin_out);
int qo_apply_rope(const float *x, size_t tokens, size_t heads, size_t head_dim,
                  const float *cos_t, const float *sin_t, size_t table_rows, float *out);
int qo_embedding(const float *table, size_t vocab, size_t hidden, const int32_t *tokens, size_t n,
                 float *out);
int qo_gqa_attention(const float *q, size_t q_tokens, size_t q_heads, size_t kv_heads,
                     size_t head_dim, const float *keys, const float *values, size_t key_tokens,
                     size_t start, float *out);
int qo_argmax(const float *logits, size_t n, int32_t *out);
/* y[m][n] = sum_k x[m][k] w[n][k], the CpuScalar per-output sequence, outputs
 * split over `threads` OpenMP threads (bit-identical to one thread). */
int qo_linear_rows(const float *x, size_t m, size_t k, const float *w, size_t n, float *y,
                   int threads);

/* One projection of logical shape [k, n] as the runtime holds it: QO_F32 with
 * `data` f32 output rows w[n][k], or the logical blocks of a quantized type in
 * output-rows order (output n owns blocks n*(k/bs) .. +k/bs). */
typedef struct {
  int qtype;
  const void *data;
} qo_weight;
/* qo_linear_rows on a qo_weight. For blocks, each output's weights w(k) are
 * the dequantized values (bit-identical to the per-element value()), so this is
 * the CpuScalar output-row matmul (backends/cpu/src/matmul.rs:282-332,
 * 119-160) with its per-output operation sequence. */
int qo_linear(const float *x, size_t m, size_t k, qo_weight w, size_t n, float *y, int threads);

typedef struct {
  uint32_t vocab, hidden, intermediate, layers, heads, kv_heads, head_dim, max_positions;
  float eps, theta;
} qo_qwen3_config;

/* Projections (qo_weight: f32 output rows or output-rows blocks) of logical
 * shape [in, out]: q [hidden, heads*hd], k and v [hidden, kv_heads*hd],
 * o [heads*hd, hidden], gate and up [hidden, intermediate], down
 * [intermediate, hidden]. Norms are f32 vectors. The model borrows every
 * pointer. */
typedef struct {
  const float *input_norm, *q_norm, *k_norm, *post_norm;
  qo_weight q, k, v, o, gate, up, down;
} qo_qwen3_layer;

typedef struct qo_qwen3 qo_qwen3;
/* embedding [vocab][hidden]; head [hidden, vocab] (output rows); capacity =
 * KV cache positions. */
qo_qwen3 *qo_qwen3_new(const qo_qwen3_config *cfg, const float *embedding,
                       const qo_qwen3_layer *layers, const float *final_norm, qo_weight head,
                       size_t capacity, int threads);
void qo_qwen3_free(qo_qwen3 *m);
size_t qo_qwen3_length(const qo_qwen3 *m);
void qo_qwen3_reset(qo_qwen3 *m);
int qo_qwen3_forward(qo_qwen3 *m, const int32_t *tokens, size_t n, int last_only, float *logits);
int qo_qwen3_generate(qo_qwen3 *m, const int32_t *prompt, size_t n, size_t max_new, int32_t eos,
                      int32_t *out, size_t *count);

#ifdef __cplusplus
}
#endif
#endif
