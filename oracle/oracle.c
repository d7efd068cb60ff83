/*
 * CPU oracle for the Qwen3.5 attention / gated-delta hot path.
 * TEST INFRASTRUCTURE ONLY -- see oracle.h.  Restates, in plain C, the
 * reference CPU truth in cpp/reference/qwen35.cpp (double accumulation where
 * the reference accumulates in double, float elsewhere, same loop order) and
 * the integer bookkeeping of cpp/kernels/qwen35_online_attention.cu.
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------ bf16 */
/* cpp/reference/bf16.hpp:12-32: RNE with NaN payload kept quiet. */
uint16_t orc_f32_to_bf16(float value) {
  uint32_t bits;
  memcpy(&bits, &value, sizeof bits);
  if ((bits & 0x7F800000u) == 0x7F800000u) {
    const uint16_t sign_and_exp = (uint16_t)((bits >> 16) & 0xFF80u);
    if ((bits & 0x007FFFFFu) == 0) return sign_and_exp;
    uint16_t payload = (uint16_t)((bits >> 16) & 0x007Fu);
    if (payload == 0) payload = 1;
    return (uint16_t)(sign_and_exp | payload);
  }
  const uint32_t lsb = (bits >> 16) & 1u;
  const uint32_t rounded = bits + 0x7FFFu + lsb;
  return (uint16_t)(rounded >> 16);
}

float orc_bf16_to_f32(uint16_t b) {
  const uint32_t bits = (uint32_t)b << 16;
  float f;
  memcpy(&f, &bits, sizeof f);
  return f;
}

void orc_bf16_round_array(const float *in, float *out, size_t n) {
  for (size_t i = 0; i < n; ++i) out[i] = orc_bf16_to_f32(orc_f32_to_bf16(in[i]));
}

/* ------------------------------------------------------ plan and layout */
static int model_signature(size_t tokens, size_t hq, size_t hkv, size_t d,
                           size_t max_ctx) {
  /* qwen35_online_attention.cu:141-145 */
  return tokens == 1 && hq == 16 && hkv == 4 && d == 256 && max_ctx != 0;
}

/* qwen35_online_attention.cu:171-183; -1 = unsupported mode. */
static long partition_for_mode(int mode) {
  switch (mode) {
  case ORC_MODE_SPLIT_K_256: return 256;
  case ORC_MODE_SPLIT_K_512: return 512;
  case ORC_MODE_SINGLE_BLOCK:
  case ORC_MODE_AUTO: return 0;
  default: return -1;
  }
}

/* qwen35_online_attention.cu:185-196 */
static size_t context_bucket(size_t max_ctx, size_t ctx) {
  size_t bucket = 512;
  while (bucket < ctx && bucket < max_ctx) {
    if (bucket > ((size_t)-1) / 2) {
      bucket = max_ctx;
      break;
    }
    bucket *= 2;
  }
  return bucket < max_ctx ? bucket : max_ctx;
}

static size_t ceil_div(size_t n, size_t d) { return n / d + (n % d ? 1 : 0); }

/* qwen35_online_attention.cu:1071-1109 */
int orc_decode_plan(size_t tokens, size_t hq, size_t hkv, size_t d,
                    size_t max_ctx, int requested, size_t ctx,
                    orc_decode_plan_t *out) {
  if (max_ctx == 0 || ctx == 0 || ctx > max_ctx) return -1;
  const int resolved = requested == ORC_MODE_AUTO ? ORC_MODE_SPLIT_K_256 : requested;
  const long p = partition_for_mode(resolved);
  if (p < 0) return -1;
  if (p != 0 && !model_signature(tokens, hq, hkv, d, max_ctx)) return -1;
  const size_t bucket = context_bucket(max_ctx, ctx);
  out->resolved_mode = resolved;
  out->context_bucket_tokens = bucket;
  if (p == 0) {
    out->partition_tokens = 0;
    out->split_k_threshold_tokens = 0;
    out->active_partition_capacity = 1;
    return 0;
  }
  out->partition_tokens = (size_t)p;
  out->split_k_threshold_tokens = (size_t)p;
  out->active_partition_capacity = ceil_div(bucket, (size_t)p);
  return 0;
}

/* qwen35_online_attention.cu:1111-1143 */
int orc_decode_workspace_layout(size_t tokens, size_t hq, size_t hkv, size_t d,
                                size_t max_ctx, int resolved,
                                orc_decode_layout_t *out) {
  memset(out, 0, sizeof *out);
  if (resolved == ORC_MODE_AUTO) return -1;
  const long p = partition_for_mode(resolved);
  if (p < 0) return -1;
  if (p == 0) return 0;
  if (!model_signature(tokens, hq, hkv, d, max_ctx)) return -1;
  const size_t max_partitions = ceil_div(max_ctx, (size_t)p);
  const size_t pc = hq * max_partitions;
  const size_t partial_bytes = pc * sizeof(float);
  out->partial_count = pc;
  out->max_offset_bytes = 0;
  out->sum_offset_bytes = partial_bytes;
  out->value_offset_bytes = 2 * partial_bytes;
  out->bytes = 2 * partial_bytes + pc * d * sizeof(float);
  return 0;
}

/* ------------------------------------------------------- float helpers */
/* cpp/reference/qwen35.cpp:35-48 (float overloads of std::exp/log1p). */
static float sigmoidf_(float v) { return 1.0f / (1.0f + expf(-v)); }
static float siluf_(float v) { return v / (1.0f + expf(-v)); }
static float softplusf_(float v) {
  if (v > 20.0f) return v;
  if (v < -20.0f) return expf(v);
  return log1pf(expf(v));
}

/* qwen35.cpp:124-154 (weight_base 0): double square sum, float scale. */
static void rms_norm_rows(const float *in, const float *w, float *out,
                          size_t rows, size_t cols, float eps) {
  for (size_t r = 0; r < rows; ++r) {
    double ss = 0.0;
    for (size_t c = 0; c < cols; ++c) {
      const double v = in[r * cols + c];
      ss += v * v;
    }
    const float scale = 1.0f / sqrtf((float)(ss / (double)cols) + eps);
    for (size_t c = 0; c < cols; ++c)
      out[r * cols + c] = in[r * cols + c] * scale * (0.0f + w[c]);
  }
}

/* qwen35.cpp:156-166 */
static void l2_normalize(float *v, size_t n, float eps) {
  double ss = 0.0;
  for (size_t i = 0; i < n; ++i) ss += (double)v[i] * (double)v[i];
  const float scale = 1.0f / sqrtf((float)ss + eps);
  for (size_t i = 0; i < n; ++i) v[i] *= scale;
}

/* qwen35.cpp:168-186: NeoX half-split partial rotary. */
static void partial_rope(float *v, size_t rotary_dim, size_t position,
                         float base) {
  const size_t pairs = rotary_dim / 2;
  for (size_t p = 0; p < pairs; ++p) {
    const double exponent = (double)(2 * p) / (double)rotary_dim;
    const double theta = (double)position / pow((double)base, exponent);
    const float c = (float)cos(theta);
    const float s = (float)sin(theta);
    const float x0 = v[p], x1 = v[p + pairs];
    v[p] = x0 * c - x1 * s;
    v[p + pairs] = x0 * s + x1 * c;
  }
}

/* -------------------------------------------------- attention core */
/* qwen35.cpp:316-364 generalised to a past prefix: query row t sees keys
 * 0..past+t, i.e. exactly what the cache-based kernels see. */
void orc_attention_core(const float *q, const float *keys, const float *values,
                        const float *gate, float *out, size_t tokens,
                        size_t hq, size_t hkv, size_t d, size_t past) {
  const size_t ctx = past + tokens;
  float *logits = (float *)malloc(ctx * sizeof(float));
  float *probs = (float *)malloc(ctx * sizeof(float));
  const size_t group = hq / hkv;
  const double root = sqrt((double)d);
  for (size_t t = 0; t < tokens; ++t) {
    const size_t visible = past + t + 1;
    for (size_t h = 0; h < hq; ++h) {
      const size_t kvh = h / group;
      const float *qv = q + (t * hq + h) * d;
      float max_logit = -INFINITY;
      for (size_t j = 0; j < visible; ++j) {
        const float *kv = keys + (j * hkv + kvh) * d;
        double dot = 0.0;
        for (size_t x = 0; x < d; ++x) dot += (double)qv[x] * (double)kv[x];
        const float logit = (float)(dot / root);
        logits[j] = logit;
        if (logit > max_logit) max_logit = logit;
      }
      double psum = 0.0;
      for (size_t j = 0; j < visible; ++j) {
        probs[j] = (float)exp((double)logits[j] - (double)max_logit);
        psum += probs[j];
      }
      for (size_t j = 0; j < visible; ++j)
        probs[j] = (float)((double)probs[j] / psum);
      float *o = out + (t * hq + h) * d;
      for (size_t x = 0; x < d; ++x) o[x] = 0.0f;
      for (size_t j = 0; j < visible; ++j) {
        const float *vv = values + (j * hkv + kvh) * d;
        for (size_t x = 0; x < d; ++x) o[x] += probs[j] * vv[x];
      }
      /* qwen35.cpp:366-370 */
      const float *g = gate + (t * hq + h) * d;
      for (size_t x = 0; x < d; ++x) o[x] *= sigmoidf_(g[x]);
    }
  }
  free(logits);
  free(probs);
}

/* qwen35.cpp:254-382 */
void orc_gated_full_attention(const float *input, const float *qnw,
                              const float *knw, const float *ow, float *output,
                              size_t tokens, size_t hidden, size_t hq,
                              size_t hkv, size_t d, size_t rotary_dim,
                              size_t position_offset, float rope_base,
                              float eps) {
  const size_t qs = hq * d, kvs = hkv * d;
  const size_t stride = qs + 2 * kvs + hidden;
  float *queries = (float *)malloc(tokens * qs * sizeof(float));
  float *keys = (float *)malloc(tokens * kvs * sizeof(float));
  float *values = (float *)malloc(tokens * kvs * sizeof(float));
  float *gate = (float *)malloc(tokens * qs * sizeof(float));
  float *attn = (float *)malloc(tokens * qs * sizeof(float));
  for (size_t t = 0; t < tokens; ++t) {
    const float *in = input + t * stride;
    memcpy(queries + t * qs, in, qs * sizeof(float));
    memcpy(keys + t * kvs, in + qs, kvs * sizeof(float));
    memcpy(values + t * kvs, in + qs + kvs, kvs * sizeof(float));
    memcpy(gate + t * qs, in + qs + 2 * kvs, qs * sizeof(float));
    for (size_t h = 0; h < hq; ++h) {
      float *v = queries + t * qs + h * d;
      rms_norm_rows(v, qnw, v, 1, d, eps);
      partial_rope(v, rotary_dim, position_offset + t, rope_base);
    }
    for (size_t h = 0; h < hkv; ++h) {
      float *v = keys + t * kvs + h * d;
      rms_norm_rows(v, knw, v, 1, d, eps);
      partial_rope(v, rotary_dim, position_offset + t, rope_base);
    }
  }
  orc_attention_core(queries, keys, values, gate, attn, tokens, hq, hkv, d, 0);
  for (size_t t = 0; t < tokens; ++t) {
    const float *a = attn + t * qs;
    for (size_t oc = 0; oc < hidden; ++oc) {
      double s = 0.0;
      for (size_t ic = 0; ic < hidden; ++ic)
        s += (double)a[ic] * (double)ow[ic * hidden + oc];
      output[t * hidden + oc] = (float)s;
    }
  }
  free(queries); free(keys); free(values); free(gate); free(attn);
}

/* ------------------------------------------- split-K partials / merge */
/* Per-token online recurrence of scan_online_decode_range
 * (qwen35_online_attention.cu:354-405) over [p*P, min(ctx,(p+1)P)), written
 * at index qh*max_partitions+p (:681-690); the same recomputation the
 * reference test performs (qwen35_cuda_attention_test.cu:883-957). */
void orc_decode_partials(const float *q, const float *keys, const float *values,
                         size_t ctx, size_t hq, size_t hkv, size_t d,
                         size_t P, size_t max_partitions, float *pmax,
                         float *psum, float *pval) {
  const size_t group = hq / hkv;
  const size_t active = ceil_div(ctx, P);
  const float inv_root = 1.0f / sqrtf((float)d);
  float *acc = (float *)malloc(d * sizeof(float));
  for (size_t h = 0; h < hq; ++h) {
    const size_t kvh = h / group;
    for (size_t p = 0; p < active; ++p) {
      const size_t begin = p * P;
      const size_t end = ctx < begin + P ? ctx : begin + P;
      float m = -INFINITY, s = 0.0f;
      for (size_t x = 0; x < d; ++x) acc[x] = 0.0f;
      for (size_t j = begin; j < end; ++j) {
        const float *kv = keys + (j * hkv + kvh) * d;
        float score = 0.0f;
        for (size_t x = 0; x < d; ++x) score += q[h * d + x] * kv[x];
        score *= inv_root;
        const float next = m > score ? m : score;
        const float left = isinf(m) ? 0.0f : expf(m - next);
        const float right = expf(score - next);
        s = s * left + right;
        const float *vv = values + (j * hkv + kvh) * d;
        for (size_t x = 0; x < d; ++x) acc[x] = acc[x] * left + vv[x] * right;
        m = next;
      }
      const size_t idx = h * max_partitions + p;
      pmax[idx] = m;
      psum[idx] = s;
      memcpy(pval + idx * d, acc, d * sizeof(float));
    }
  }
  free(acc);
}

/* online_decode_merge_kernel (qwen35_online_attention.cu:693-756) */
void orc_decode_merge(const float *gate, const float *pmax, const float *psum,
                      const float *pval, size_t ctx, size_t hq, size_t d,
                      size_t P, size_t max_partitions, float *out) {
  const size_t active = ceil_div(ctx, P);
  float *acc = (float *)malloc(d * sizeof(float));
  for (size_t h = 0; h < hq; ++h) {
    const size_t first = h * max_partitions;
    float m = pmax[first], s = psum[first];
    memcpy(acc, pval + first * d, d * sizeof(float));
    for (size_t p = 1; p < active; ++p) {
      const size_t i = first + p;
      const float next = m > pmax[i] ? m : pmax[i];
      const float left = expf(m - next);
      const float right = expf(pmax[i] - next);
      s = s * left + psum[i] * right;
      for (size_t x = 0; x < d; ++x)
        acc[x] = acc[x] * left + pval[i * d + x] * right;
      m = next;
    }
    for (size_t x = 0; x < d; ++x)
      out[h * d + x] = (acc[x] / s) / (1.0f + expf(-gate[h * d + x]));
  }
  free(acc);
}

/* ----------------------------------------------------- gated delta */
/* Recurrence for one token, qwen35.cpp:459-518.  q, k already normalised
 * and q already scaled; state [Hv][dk][dv]. */
static void delta_recurrence_token(const float *q, const float *k,
                                   const float *v, const float *beta,
                                   const float *decay, float *state,
                                   float *raw, size_t hk, size_t hv,
                                   size_t dk, size_t dv, float *delta) {
  for (size_t h = 0; h < hv; ++h) {
    const size_t kh = h % hk; /* qwen35.cpp:462 */
    const float *qh = q + kh * dk;
    const float *kh_ = k + kh * dk;
    const float *vh = v + h * dv;
    float *S = state + h * dk * dv;
    for (size_t i = 0; i < dk * dv; ++i) S[i] *= decay[h];
    for (size_t c = 0; c < dv; ++c) {
      double mem = 0.0;
      for (size_t r = 0; r < dk; ++r) mem += (double)S[r * dv + c] * (double)kh_[r];
      delta[c] = (vh[c] - (float)mem) * beta[h];
    }
    for (size_t r = 0; r < dk; ++r)
      for (size_t c = 0; c < dv; ++c) S[r * dv + c] += kh_[r] * delta[c];
    for (size_t c = 0; c < dv; ++c) {
      double s = 0.0;
      for (size_t r = 0; r < dk; ++r) s += (double)S[r * dv + c] * (double)qh[r];
      raw[h * dv + c] = (float)s;
    }
  }
}

/* qwen35.cpp:384-526 */
void orc_gated_delta_step(const float *input, const float *conv_weight,
                          const float *recurrent_a, const float *dt_bias,
                          const float *norm_w, float *output, float *conv_state,
                          float *rec_state, size_t hidden, size_t hk,
                          size_t hv, size_t dk, size_t dv, size_t W,
                          float eps) {
  const size_t ks = hk * dk, vs = hv * dv;
  const size_t conv_dim = 2 * ks + vs;
  float *conv = (float *)malloc(conv_dim * sizeof(float));
  /* :417-427 causal depthwise conv + SiLU */
  for (size_t ch = 0; ch < conv_dim; ++ch) {
    float sum = input[ch] * conv_weight[ch * W + W - 1];
    for (size_t hst = 0; hst + 1 < W; ++hst)
      sum += conv_state[ch * (W - 1) + hst] * conv_weight[ch * W + hst];
    conv[ch] = siluf_(sum);
  }
  /* :429-438 history shift */
  if (W > 1) {
    for (size_t ch = 0; ch < conv_dim; ++ch) {
      const size_t base = ch * (W - 1);
      for (size_t hst = 0; hst + 2 < W; ++hst)
        conv_state[base + hst] = conv_state[base + hst + 1];
      conv_state[base + W - 2] = input[ch];
    }
  }
  float *q = conv, *k = conv + ks, *v = conv + 2 * ks;
  const float *b = input + conv_dim;
  const float *a = input + conv_dim + hv;
  const float *z = input + 2 * ks + vs + 2 * hv;
  /* :448-457 */
  const float qscale = 1.0f / sqrtf((float)dk);
  for (size_t h = 0; h < hk; ++h) {
    l2_normalize(q + h * dk, dk, 1.0e-6f);
    l2_normalize(k + h * dk, dk, 1.0e-6f);
    for (size_t i = 0; i < dk; ++i) q[h * dk + i] *= qscale;
  }
  float *beta = (float *)malloc(hv * sizeof(float));
  float *decay = (float *)malloc(hv * sizeof(float));
  for (size_t h = 0; h < hv; ++h) {
    beta[h] = sigmoidf_(b[h]);
    decay[h] = expf(recurrent_a[h] * softplusf_(a[h] + dt_bias[h]));
  }
  float *raw = (float *)malloc(vs * sizeof(float));
  float *delta = (float *)malloc(dv * sizeof(float));
  delta_recurrence_token(q, k, v, beta, decay, rec_state, raw, hk, hv, dk, dv,
                         delta);
  /* :520-525 */
  rms_norm_rows(raw, norm_w, output, hv, dv, eps);
  for (size_t i = 0; i < hidden; ++i) output[i] *= siluf_(z[i]);
  free(conv); free(beta); free(decay); free(raw); free(delta);
}

/* qwen35.cpp:528-549 */
void orc_gated_delta_prefill(const float *input, const float *conv_weight,
                             const float *recurrent_a, const float *dt_bias,
                             const float *norm_w, float *output,
                             float *conv_state, float *rec_state,
                             size_t tokens, size_t hidden, size_t hk,
                             size_t hv, size_t dk, size_t dv, size_t W,
                             float eps) {
  const size_t stride = 2 * hk * dk + hv * dv + 2 * hv + hidden;
  for (size_t t = 0; t < tokens; ++t)
    orc_gated_delta_step(input + t * stride, conv_weight, recurrent_a, dt_bias,
                         norm_w, output + t * hidden, conv_state, rec_state,
                         hidden, hk, hv, dk, dv, W, eps);
}

void orc_delta_core(const float *q, const float *k, const float *v,
                    const float *beta, const float *log_decay, float q_scale,
                    float *state, float *raw_out, size_t tokens, size_t hk,
                    size_t hv, size_t dk, size_t dv) {
  float *qs = (float *)malloc(hk * dk * sizeof(float));
  float *decay = (float *)malloc(hv * sizeof(float));
  float *delta = (float *)malloc(dv * sizeof(float));
  for (size_t t = 0; t < tokens; ++t) {
    for (size_t i = 0; i < hk * dk; ++i) qs[i] = q[t * hk * dk + i] * q_scale;
    for (size_t h = 0; h < hv; ++h) decay[h] = expf(log_decay[t * hv + h]);
    delta_recurrence_token(qs, k + t * hk * dk, v + t * hv * dv, beta + t * hv,
                           decay, state, raw_out + t * hv * dv, hk, hv, dk, dv,
                           delta);
  }
  free(qs); free(decay); free(delta);
}

/* ------------------------------------------------ attention producers */
void orc_qk_norm_rope(const float *input, const float *weight, float *output,
                      size_t tokens, size_t heads, size_t head_dim,
                      size_t rotary_dim, size_t position_offset,
                      float rope_base, float epsilon) {
  for (size_t t = 0; t < tokens; ++t)
    for (size_t h = 0; h < heads; ++h) {
      const size_t base = (t * heads + h) * head_dim;
      rms_norm_rows(input + base, weight, output + base, 1, head_dim, epsilon);
      partial_rope(output + base, rotary_dim, position_offset + t, rope_base);
    }
}

void orc_split_full_query_gate(const float *query_gate, float *query,
                               float *gate, size_t tokens, size_t heads,
                               size_t head_dim) {
  for (size_t t = 0; t < tokens; ++t)
    for (size_t h = 0; h < heads; ++h)
      for (size_t d = 0; d < head_dim; ++d) {
        const size_t src = (t * heads + h) * 2 * head_dim + d;
        const size_t dst = (t * heads + h) * head_dim + d;
        query[dst] = query_gate[src];
        gate[dst] = query_gate[src + head_dim];
      }
}

void orc_pack_linear_delta_input(const float *qkv, const float *beta,
                                 const float *alpha, const float *gate,
                                 float *packed, size_t tokens, size_t qkv_width,
                                 size_t beta_width, size_t alpha_width,
                                 size_t gate_width) {
  const size_t width = qkv_width + beta_width + alpha_width + gate_width;
  for (size_t t = 0; t < tokens; ++t) {
    float *row = packed + t * width;
    memcpy(row, qkv + t * qkv_width, qkv_width * sizeof(float));
    memcpy(row + qkv_width, beta + t * beta_width, beta_width * sizeof(float));
    memcpy(row + qkv_width + beta_width, alpha + t * alpha_width, alpha_width * sizeof(float));
    memcpy(row + qkv_width + beta_width + alpha_width, gate + t * gate_width,
           gate_width * sizeof(float));
  }
}

/* ------------------------------------------------------------ metrics */
void orc_compare(const float *c, const float *r, size_t n, double floor_,
                 double *out) {
  double max_abs = 0.0, max_rel = 0.0, dot = 0.0, cn = 0.0, rn = 0.0, dn = 0.0;
  double nonfinite = 0.0;
  for (size_t i = 0; i < n; ++i) {
    const float cv = c[i], rv = r[i];
    if (!isfinite(cv) || !isfinite(rv)) {
      if (!(isinf(cv) && isinf(rv) && signbit(cv) == signbit(rv))) nonfinite += 1.0;
      continue;
    }
    const double a = fabs((double)cv - (double)rv);
    const double den = fabs((double)rv) > floor_ ? fabs((double)rv) : floor_;
    if (a > max_abs) max_abs = a;
    if (a / den > max_rel) max_rel = a / den;
    dot += (double)cv * rv;
    cn += (double)cv * cv;
    rn += (double)rv * rv;
    dn += a * a;
  }
  double cosine = 1.0;
  if (cn == 0.0 && rn == 0.0) cosine = 1.0;
  else if (cn == 0.0 || rn == 0.0) cosine = 0.0;
  else {
    cosine = dot / (sqrt(cn) * sqrt(rn));
    if (cosine > 1.0) cosine = 1.0;
    if (cosine < -1.0) cosine = -1.0;
  }
  out[0] = max_abs;
  out[1] = max_rel;
  out[2] = cosine;
  out[3] = nonfinite;
  out[4] = rn > 0.0 ? sqrt(dn) / sqrt(rn) : sqrt(dn);
}
