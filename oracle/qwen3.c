/*
 * CPU oracle, second part: the Qwen3 dense decoder forward pass and greedy
 * generation of the reference runtime, restated in plain C. TEST
 * INFRASTRUCTURE ONLY (see oracle.h): it is the checker for the HIP decoder
 * (quantinfer_amd/csrc/qi_qwen3.hip) and nothing in the product links it.
 *
 * Followed step by step (paths relative to the aiqubits/quantinfer tree):
 *  - layer forward: crates/quantinfer-runtime/src/qwen3/mod.rs:117-208
 *  - model forward, logits: qwen3/mod.rs:334-378
 *  - RoPE tables: runtime/src/attention.rs:7-35
 *  - GQA attention over the KV cache: attention.rs:37-141
 *  - RoPE before the cache append: runtime/src/batch.rs:21-67
 *  - KV cache append: runtime/src/cache.rs:96-125
 *  - rms_norm, rms_norm_heads, softmax, silu_mul, apply_rope, embedding:
 *    backends/cpu/src/backend.rs:172-298
 *  - residual add: runtime/src/linear.rs:129-142
 *  - argmax and the generation loop: runtime/src/generation.rs:58-76, 174-201
 *
 * The linear layers are the CpuScalar matmuls: for every output, acc = 0 and
 * acc = acc + x[k] * w(k) in ascending k (backends/cpu/src/matmul.rs:146-157,
 * 319-330 for output rows; :92-117 for the f32 LM head). The per-element
 * weight w(k) equals the dequantized value bit for bit (matmul.rs:162-280 vs
 * quant/src/schemes), so a projection is given either as f32 output rows
 * w[n][k] or as its quantized blocks, whose rows are dequantized a few at a
 * time just before use (the 8B shape then needs its 4.6 GB of blocks, not
 * 30 GB of f32); either way the per-output operation sequence is the same.
 * Several rows (or outputs) are computed side by side in vector registers,
 * and outputs (and attention's (token, head) pairs) are split over OpenMP
 * threads; neither changes any output's operation sequence, so the result is
 * bit-identical to the scalar loop (the threading is this oracle's, not the
 * reference's).
 *
 * f32 functions expf, powf, cosf, sinf, sqrtf are the C library's; Rust's
 * f32::exp/powf/cos/sin lower to the same libm calls. Sums start from 0.0 and
 * run in index order, as Rust's Iterator::sum over f32 does (a start value of
 * -0.0 would only change the sign of an all-zero sum).
 *
 * Pinned by tests/test_oracle_qwen3.py: closed forms of RMSNorm and softmax,
 * RoPE against the rotation it defines (norm preservation, composition of
 * angles, the table formula in float64), attention against a float64 softmax
 * brute force, the decoder against an independent float64 numpy restatement
 * of the same forward pass, prefill-then-decode == one-shot prefill (the KV
 * cache invariant), and the reference's own qwen3 test shapes
 * (runtime/src/qwen3/tests.rs:22-99). The exact libm bits of expf/powf/cosf/
 * sinf as the reference's Rust build links them are parity unpinned (only
 * greedy token ids are compared end to end).
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------ ops */

/* backends/cpu/src/backend.rs:172-190 */
int qo_rms_norm(const float *x, size_t rows, size_t dim, const float *w, float eps, float *out) {
  if (dim == 0) return QO_INVALID;
  for (size_t r = 0; r < rows; ++r) {
    const float *v = x + r * dim;
    float ms = 0.0f;
    for (size_t c = 0; c < dim; ++c) ms += v[c] * v[c];
    ms = ms / (float)dim;
    float inv = 1.0f / sqrtf(ms + eps);
    for (size_t c = 0; c < dim; ++c) out[r * dim + c] = v[c] * inv * w[c];
  }
  return QO_OK;
}

/* backends/cpu/src/backend.rs:200-222 */
int qo_softmax(const float *x, size_t rows, size_t dim, float *out) {
  if (dim == 0) return QO_INVALID;
  for (size_t r = 0; r < rows; ++r) {
    const float *v = x + r * dim;
    float mx = -INFINITY;
    for (size_t c = 0; c < dim; ++c) mx = fmaxf(mx, v[c]);
    float sum = 0.0f;
    for (size_t c = 0; c < dim; ++c) sum += expf(v[c] - mx);
    for (size_t c = 0; c < dim; ++c) out[r * dim + c] = expf(v[c] - mx) / sum;
  }
  return QO_OK;
}

/* backends/cpu/src/backend.rs:224-237: gate / (1 + exp(-gate)) * up */
int qo_silu_mul(const float *gate, const float *up, size_t n, float *out) {
  for (size_t i = 0; i < n; ++i) {
    float g = gate[i];
    out[i] = g / (1.0f + expf(-g)) * up[i];
  }
  return QO_OK;
}

/* runtime/src/attention.rs:7-35: rows position start..start+length, pair p:
 * angle = position * theta^(-(2p)/head_dim) in f32. */
int qo_rope_tables(float theta, size_t head_dim, size_t start, size_t length, float *cos_out,
                   float *sin_out) {
  if (head_dim == 0 || head_dim % 2 != 0 || !isfinite(theta) || theta <= 0.0f) return QO_INVALID;
  size_t pairs = head_dim / 2;
  for (size_t i = 0; i < length; ++i) {
    float position = (float)(start + i);
    for (size_t p = 0; p < pairs; ++p) {
      float exponent = (2.0f * (float)p) / (float)head_dim;
      float angle = position * powf(theta, -exponent);
      cos_out[i * pairs + p] = cosf(angle);
      sin_out[i * pairs + p] = sinf(angle);
    }
  }
  return QO_OK;
}

/* backends/cpu/src/backend.rs:239-279: pairs (p, p + head_dim/2); tables hold
 * one row (table_rows == 1) or one row per token. */
int qo_apply_rope(const float *x, size_t tokens, size_t heads, size_t head_dim,
                  const float *cos_t, const float *sin_t, size_t table_rows, float *out) {
  if (head_dim == 0 || head_dim % 2 != 0) return QO_INVALID;
  if (table_rows != 1 && table_rows != tokens) return QO_INVALID;
  size_t pairs = head_dim / 2;
  if (out != x) memcpy(out, x, tokens * heads * head_dim * sizeof(float));
  for (size_t t = 0; t < tokens; ++t) {
    size_t toff = table_rows == 1 ? 0 : t * pairs;
    for (size_t h = 0; h < heads; ++h) {
      const float *in = x + (t * heads + h) * head_dim;
      float *o = out + (t * heads + h) * head_dim;
      for (size_t p = 0; p < pairs; ++p) {
        float first = in[p], second = in[pairs + p];
        float c = cos_t[toff + p], s = sin_t[toff + p];
        o[p] = first * c - second * s;
        o[pairs + p] = first * s + second * c;
      }
    }
  }
  return QO_OK;
}

/* backends/cpu/src/backend.rs:281-298 */
int qo_embedding(const float *table, size_t vocab, size_t hidden, const int32_t *tokens, size_t n,
                 float *out) {
  for (size_t i = 0; i < n; ++i) {
    if (tokens[i] < 0 || (size_t)tokens[i] >= vocab) return QO_INVALID;
    memcpy(out + i * hidden, table + (size_t)tokens[i] * hidden, hidden * sizeof(float));
  }
  return QO_OK;
}

/* runtime/src/attention.rs:37-141. q [q_tokens][q_heads][head_dim]; keys and
 * values [key_tokens][kv_heads][head_dim]; query token t sees keys
 * 0..=start+t. Every (token, head) pair is independent; they are split over
 * `threads` OpenMP threads (bit-identical to one thread). */
static int gqa_attention(const float *q, size_t q_tokens, size_t q_heads, size_t kv_heads,
                         size_t head_dim, const float *keys, const float *values, size_t key_tokens,
                         size_t start, float *out, int threads) {
  if (kv_heads == 0 || key_tokens == 0 || q_heads % kv_heads != 0) return QO_INVALID;
  if (key_tokens < start + q_tokens) return QO_INVALID;
  size_t group = q_heads / kv_heads;
  float scale = 1.0f / sqrtf((float)head_dim);
  int status = QO_OK;
  memset(out, 0, q_tokens * q_heads * head_dim * sizeof(float));
#pragma omp parallel num_threads(threads < 1 ? 1 : threads)
  {
    float *scores = (float *)malloc(key_tokens * sizeof(float));
    if (scores == NULL) {
#pragma omp atomic write
      status = QO_INVALID;
    }
#pragma omp for schedule(dynamic, 4)
    for (size_t th = 0; th < q_tokens * q_heads; ++th) {
      if (scores == NULL) continue;
      size_t t = th / q_heads, h = th % q_heads;
      size_t last = start + t;
      size_t g = h / group;
      const float *qv = q + (t * q_heads + h) * head_dim;
      for (size_t j = 0; j <= last; ++j) {
        const float *kv = keys + (j * kv_heads + g) * head_dim;
        float dot = 0.0f;
        for (size_t d = 0; d < head_dim; ++d) dot += qv[d] * kv[d];
        scores[j] = dot * scale;
      }
      float mx = -INFINITY;
      for (size_t j = 0; j <= last; ++j) mx = fmaxf(mx, scores[j]);
      float denom = 0.0f;
      for (size_t j = 0; j <= last; ++j) denom += expf(scores[j] - mx);
      float *o = out + (t * q_heads + h) * head_dim;
      for (size_t j = 0; j <= last; ++j) {
        float weight = expf(scores[j] - mx) / denom;
        const float *vv = values + (j * kv_heads + g) * head_dim;
        for (size_t d = 0; d < head_dim; ++d) o[d] += weight * vv[d];
      }
    }
    free(scores);
  }
  return status;
}

int qo_gqa_attention(const float *q, size_t q_tokens, size_t q_heads, size_t kv_heads,
                     size_t head_dim, const float *keys, const float *values, size_t key_tokens,
                     size_t start, float *out) {
  return gqa_attention(q, q_tokens, q_heads, kv_heads, head_dim, keys, values, key_tokens, start,
                       out, 1);
}

/* generation.rs:58-76: the first index of the maximum; non-finite logits are
 * rejected. */
int qo_argmax(const float *logits, size_t n, int32_t *out) {
  if (n == 0) return QO_INVALID;
  for (size_t i = 0; i < n; ++i)
    if (!isfinite(logits[i])) return QO_INVALID;
  size_t best = 0;
  for (size_t i = 1; i < n; ++i)
    if (logits[i] > logits[best]) best = i;
  *out = (int32_t)best;
  return QO_OK;
}

/* --------------------------------------------------------------- linear */

/* y[m][n] = sum_k x[m][k] * w[n][k], per output acc = acc + x*w ascending k. */
#define ROWS 8
__attribute__((target_clones("avx512f", "avx2", "default")))
static void lin_rows8(const float *xt, size_t mp, size_t k, const float *w0, const float *w1,
                      const float *w2, const float *w3, float acc[4][ROWS]) {
  float a0[ROWS] = {0}, a1[ROWS] = {0}, a2[ROWS] = {0}, a3[ROWS] = {0};
  for (size_t i = 0; i < k; ++i) {
    const float *xr = xt + i * mp;
    float b0 = w0[i], b1 = w1[i], b2 = w2[i], b3 = w3[i];
    for (int r = 0; r < ROWS; ++r) {
      a0[r] = a0[r] + xr[r] * b0;
      a1[r] = a1[r] + xr[r] * b1;
      a2[r] = a2[r] + xr[r] * b2;
      a3[r] = a3[r] + xr[r] * b3;
    }
  }
  for (int r = 0; r < ROWS; ++r) {
    acc[0][r] = a0[r];
    acc[1][r] = a1[r];
    acc[2][r] = a2[r];
    acc[3][r] = a3[r];
  }
}

/* Source of output n's weights: f32 rows are used in place; quantized rows
 * are dequantized into `buf` (k floats) by the bit-exact dequantizer. */
static const float *weight_row(qo_weight w, size_t k, size_t n, float *buf) {
  if (w.qtype == QO_F32) return (const float *)w.data + n * k;
  size_t bs = qo_block_elems(w.qtype), bb = qo_block_bytes(w.qtype);
  qo_dequantize(w.qtype, (const uint8_t *)w.data + n * (k / bs) * bb, k / bs, buf);
  return buf;
}

static void lin_row1(const float *x, size_t k, qo_weight w, size_t n0, size_t n1, float *buf,
                     float *y) {
  size_t n = n0;
  for (; n + 4 <= n1; n += 4) {
    const float *w0 = weight_row(w, k, n, buf), *w1 = weight_row(w, k, n + 1, buf + k);
    const float *w2 = weight_row(w, k, n + 2, buf + 2 * k), *w3 = weight_row(w, k, n + 3, buf + 3 * k);
    float a0 = 0.0f, a1 = 0.0f, a2 = 0.0f, a3 = 0.0f;
    for (size_t i = 0; i < k; ++i) {
      a0 = a0 + x[i] * w0[i];
      a1 = a1 + x[i] * w1[i];
      a2 = a2 + x[i] * w2[i];
      a3 = a3 + x[i] * w3[i];
    }
    y[n] = a0;
    y[n + 1] = a1;
    y[n + 2] = a2;
    y[n + 3] = a3;
  }
  for (; n < n1; ++n) {
    const float *wr = weight_row(w, k, n, buf);
    float a = 0.0f;
    for (size_t i = 0; i < k; ++i) a = a + x[i] * wr[i];
    y[n] = a;
  }
}

int qo_linear(const float *x, size_t m, size_t k, qo_weight w, size_t n, float *y, int threads) {
  if (m == 0 || k == 0 || n == 0 || w.data == NULL) return QO_INVALID;
  if (w.qtype != QO_F32) {
    size_t bs = qo_block_elems(w.qtype);
    if (bs == 0 || k % bs != 0) return QO_INVALID;
  }
  int nt = threads < 1 ? 1 : threads;
  int status = QO_OK;
  if (m == 1) {
    size_t chunk = (n + (size_t)nt * 64 - 1) / ((size_t)nt * 64) * 4;
    size_t chunks = (n + chunk - 1) / chunk;
#pragma omp parallel num_threads(nt)
    {
      float *buf = (float *)malloc(4 * k * sizeof(float));
      if (buf == NULL) {
#pragma omp atomic write
        status = QO_INVALID;
      }
#pragma omp for schedule(dynamic, 1)
      for (size_t c = 0; c < chunks; ++c) {
        if (buf == NULL) continue;
        size_t n0 = c * chunk, n1 = n0 + chunk < n ? n0 + chunk : n;
        lin_row1(x, k, w, n0, n1, buf, y);
      }
      free(buf);
    }
    return status;
  }
  size_t mp = (m + ROWS - 1) / ROWS * ROWS;
  float *xt = (float *)calloc(mp * k, sizeof(float));
  if (xt == NULL) return QO_INVALID;
  for (size_t r = 0; r < m; ++r)
    for (size_t i = 0; i < k; ++i) xt[i * mp + r] = x[r * k + i];
  size_t groups = (n + 3) / 4;
#pragma omp parallel num_threads(nt)
  {
    float *buf = (float *)malloc(4 * k * sizeof(float));
    if (buf == NULL) {
#pragma omp atomic write
      status = QO_INVALID;
    }
#pragma omp for schedule(dynamic, 8)
    for (size_t g = 0; g < groups; ++g) {
      if (buf == NULL) continue;
      size_t nb = g * 4;
      const float *wr[4];
      for (int j = 0; j < 4; ++j) wr[j] = weight_row(w, k, nb + j < n ? nb + j : n - 1, buf + j * k);
      float acc[4][ROWS];
      for (size_t r0 = 0; r0 < m; r0 += ROWS) {
        lin_rows8(xt + r0, mp, k, wr[0], wr[1], wr[2], wr[3], acc);
        for (int j = 0; j < 4; ++j) {
          if (nb + j >= n) break;
          for (int r = 0; r < ROWS && r0 + r < m; ++r) y[(r0 + r) * n + nb + j] = acc[j][r];
        }
      }
    }
    free(buf);
  }
  free(xt);
  return status;
}

int qo_linear_rows(const float *x, size_t m, size_t k, const float *w, size_t n, float *y,
                   int threads) {
  qo_weight f = {QO_F32, w};
  return qo_linear(x, m, k, f, n, y, threads);
}

/* ---------------------------------------------------------------- model */

struct qo_qwen3 {
  qo_qwen3_config cfg;
  const float *embedding;
  qo_qwen3_layer *layers;
  const float *final_norm;
  qo_weight head;
  int threads;
  size_t capacity;
  size_t length;
  float **keys;   /* per layer [capacity][kv_heads][head_dim] */
  float **values;
};

qo_qwen3 *qo_qwen3_new(const qo_qwen3_config *cfg, const float *embedding,
                       const qo_qwen3_layer *layers, const float *final_norm, qo_weight head,
                       size_t capacity, int threads) {
  if (cfg == NULL || cfg->layers == 0 || cfg->heads == 0 || cfg->kv_heads == 0 ||
      cfg->heads % cfg->kv_heads != 0 || cfg->head_dim == 0 || cfg->head_dim % 2 != 0 ||
      capacity == 0 || capacity > cfg->max_positions)
    return NULL;
  qo_qwen3 *m = (qo_qwen3 *)calloc(1, sizeof(qo_qwen3));
  if (m == NULL) return NULL;
  m->cfg = *cfg;
  m->embedding = embedding;
  m->final_norm = final_norm;
  m->head = head;
  m->threads = threads < 1 ? 1 : threads;
  m->capacity = capacity;
  m->layers = (qo_qwen3_layer *)malloc(cfg->layers * sizeof(qo_qwen3_layer));
  m->keys = (float **)calloc(cfg->layers, sizeof(float *));
  m->values = (float **)calloc(cfg->layers, sizeof(float *));
  int ok = m->layers && m->keys && m->values;
  size_t per = capacity * cfg->kv_heads * cfg->head_dim;
  for (uint32_t l = 0; ok && l < cfg->layers; ++l) {
    m->layers[l] = layers[l];
    m->keys[l] = (float *)malloc(per * sizeof(float));
    m->values[l] = (float *)malloc(per * sizeof(float));
    ok = m->keys[l] && m->values[l];
  }
  if (!ok) {
    qo_qwen3_free(m);
    return NULL;
  }
  return m;
}

void qo_qwen3_free(qo_qwen3 *m) {
  if (m == NULL) return;
  for (uint32_t l = 0; m->keys && l < m->cfg.layers; ++l) {
    free(m->keys[l]);
    free(m->values[l]);
  }
  free(m->keys);
  free(m->values);
  free(m->layers);
  free(m);
}

size_t qo_qwen3_length(const qo_qwen3 *m) { return m->length; }
void qo_qwen3_reset(qo_qwen3 *m) { m->length = 0; }

static void add_into(float *acc, const float *b, size_t n) {
  for (size_t i = 0; i < n; ++i) acc[i] = acc[i] + b[i];
}

/* qwen3/mod.rs:334-378 with the layer forward of :117-208. Writes the logits
 * of every token ([n][vocab]) or, with last_only, of the last token. */
int qo_qwen3_forward(qo_qwen3 *m, const int32_t *tokens, size_t n, int last_only,
                     float *logits) {
  const qo_qwen3_config *c = &m->cfg;
  if (n == 0) return QO_INVALID;
  if (m->length + n > m->capacity) return QO_INVALID;
  const size_t H = c->hidden, I = c->intermediate, hd = c->head_dim;
  const size_t QS = (size_t)c->heads * hd, KS = (size_t)c->kv_heads * hd;
  const size_t start = m->length, pairs = hd / 2;
  int status = QO_INVALID;
  float *hidden = malloc(n * H * sizeof(float));
  float *norm = malloc(n * H * sizeof(float));
  float *q = malloc(n * QS * sizeof(float));
  float *k = malloc(n * KS * sizeof(float));
  float *v = malloc(n * KS * sizeof(float));
  float *att = malloc(n * QS * sizeof(float));
  float *proj = malloc(n * H * sizeof(float));
  float *gate = malloc(n * I * sizeof(float));
  float *up = malloc(n * I * sizeof(float));
  float *cs = malloc(n * pairs * sizeof(float));
  float *sn = malloc(n * pairs * sizeof(float));
  if (!hidden || !norm || !q || !k || !v || !att || !proj || !gate || !up || !cs || !sn) goto done;
  if (qo_embedding(m->embedding, c->vocab, H, tokens, n, hidden) != QO_OK) goto done;
  if (qo_rope_tables(c->theta, hd, start, n, cs, sn) != QO_OK) goto done;
  for (uint32_t l = 0; l < c->layers; ++l) {
    const qo_qwen3_layer *L = &m->layers[l];
    qo_rms_norm(hidden, n, H, L->input_norm, c->eps, norm);
    if (qo_linear(norm, n, H, L->q, QS, q, m->threads) != QO_OK) goto done;
    if (qo_linear(norm, n, H, L->k, KS, k, m->threads) != QO_OK) goto done;
    if (qo_linear(norm, n, H, L->v, KS, v, m->threads) != QO_OK) goto done;
    qo_rms_norm(q, n * c->heads, hd, L->q_norm, c->eps, q);
    qo_rms_norm(k, n * c->kv_heads, hd, L->k_norm, c->eps, k);
    qo_apply_rope(q, n, c->heads, hd, cs, sn, n, q);
    qo_apply_rope(k, n, c->kv_heads, hd, cs, sn, n, k);
    memcpy(m->keys[l] + start * KS, k, n * KS * sizeof(float));
    memcpy(m->values[l] + start * KS, v, n * KS * sizeof(float));
    if (gqa_attention(q, n, c->heads, c->kv_heads, hd, m->keys[l], m->values[l], start + n,
                      start, att, m->threads) != QO_OK)
      goto done;
    if (qo_linear(att, n, QS, L->o, H, proj, m->threads) != QO_OK) goto done;
    add_into(hidden, proj, n * H);
    qo_rms_norm(hidden, n, H, L->post_norm, c->eps, norm);
    if (qo_linear(norm, n, H, L->gate, I, gate, m->threads) != QO_OK) goto done;
    if (qo_linear(norm, n, H, L->up, I, up, m->threads) != QO_OK) goto done;
    qo_silu_mul(gate, up, n * I, gate);
    if (qo_linear(gate, n, I, L->down, H, proj, m->threads) != QO_OK) goto done;
    add_into(hidden, proj, n * H);
  }
  m->length = start + n;
  {
    size_t first = last_only ? n - 1 : 0, rows = n - first;
    qo_rms_norm(hidden + first * H, rows, H, m->final_norm, c->eps, norm);
    if (qo_linear(norm, rows, H, m->head, c->vocab, logits, m->threads) != QO_OK) goto done;
  }
  status = QO_OK;
done:
  free(hidden);
  free(norm);
  free(q);
  free(k);
  free(v);
  free(att);
  free(proj);
  free(gate);
  free(up);
  free(cs);
  free(sn);
  return status;
}

/* generation.rs:174-201 with temperature 0 (argmax), no sink stop. */
int qo_qwen3_generate(qo_qwen3 *m, const int32_t *prompt, size_t n, size_t max_new,
                      int32_t eos, int32_t *out, size_t *count) {
  *count = 0;
  float *logits = malloc(m->cfg.vocab * sizeof(float));
  if (logits == NULL) return QO_INVALID;
  int status = qo_qwen3_forward(m, prompt, n, 1, logits);
  for (size_t i = 0; status == QO_OK && i < max_new; ++i) {
    int32_t next;
    status = qo_argmax(logits, m->cfg.vocab, &next);
    if (status != QO_OK) break;
    out[(*count)++] = next;
    if (eos >= 0 && next == eos) break;
    status = qo_qwen3_forward(m, &next, 1, 1, logits);
  }
  free(logits);
  return status;
}
