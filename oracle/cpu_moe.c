/*
 * CPU oracle for the quantized sparse-MoE block.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the shipped path (runnel_amd/) may
 * load, link or call this file; only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py use it, always as the checker or as the timed
 * CPU baseline, never as the thing measured on the GPU.
 *
 * Two groups of functions live here.
 *
 * 1. Restatements of the reference's native CPU oracles and synthetic data
 *    generators, so that the reference's recorded checksums can be
 *    reproduced (they are the only golden vectors the reference holds):
 *      - xorshift64 generator     native/src/fused_moe_probe.mm:69-87
 *                                 native/src/quantized_qmv_probe.mm:64-82
 *      - float_to_bf16 (RNE, NaN/Inf truncated)
 *                                 native/src/fused_moe_probe.mm:89-104
 *      - QMV dataset + reference  native/src/quantized_qmv_probe.mm:355-433
 *      - fused two-stage dataset  native/src/fused_moe_probe.mm:449-537,600-695
 *      - QMM dataset + reference  native/src/quantized_qmm_probe.mm:243-307
 *    Accumulation orders and the q4 "low nibble of every byte" quirk follow
 *    those files exactly.
 *
 * 2. The block contract that the HIP kernels implement (router, top-k,
 *    softmax + renormalisation, packed [up; gate] gate/up projection with
 *    SwiGLU, down projection, weighted combine, sigmoid-gated shared expert,
 *    optional residual), computed in fp32 with OpenMP.  It is the timed CPU
 *    baseline ("port") and a second, independent implementation of the same
 *    contract as oracle/moe_ref.py.  The semantics follow the mlx-lm
 *    SparseMoeBlock that calls src/runnel/mlx.py:57-82; the bf16 rounding
 *    points and the top-k tie rule are this library's own definition, because
 *    mlx/mlx-lm are third-party code that is not available here.
 *
 * Build: oracle/Makefile (gcc -O2 -fopenmp -ffp-contract=off).
 */
#include <math.h>
#include <stddef.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define ORC_OK 0
#define ORC_EINVAL (-1)

/* ------------------------------------------------------------------------ */
/* Scalars                                                                   */
/* ------------------------------------------------------------------------ */

/* xorshift64 with the (13, 7, 17) triple, high 32 bits returned.
 * native/src/fused_moe_probe.mm:69-76 */
typedef struct {
  uint64_t state;
} orc_random;

static uint32_t rnd_next(orc_random* r) {
  r->state ^= r->state << 13;
  r->state ^= r->state >> 7;
  r->state ^= r->state << 17;
  return (uint32_t)(r->state >> 32);
}

/* native/src/fused_moe_probe.mm:78-81: the unit value is a double, the
 * affine map is evaluated in float.  The reference's compiler contracts
 * `low + unit * (high - low)` into one fused multiply-add: only the fused
 * form reproduces the SHA-256 of the reference's recorded q4 dataset
 * (bench/results/m0/mlx-current-ornith-shape-qmv-q4.json, dataset_sha256);
 * the q8 dataset hashes the same either way. */
static float rnd_uniform(orc_random* r, float low, float high) {
  const double unit = (double)rnd_next(r) / 4294967295.0;
  return fmaf((float)unit, high - low, low);
}

uint16_t orc_f32_to_bf16(float value) {
  uint32_t bits;
  memcpy(&bits, &value, sizeof(bits));
  if (((bits >> 23) & 0xFFu) == 0xFFu) {
    return (uint16_t)(bits >> 16); /* NaN / Inf: truncate */
  }
  const uint32_t rounding = 0x7FFFu + ((bits >> 16) & 1u);
  return (uint16_t)((bits + rounding) >> 16);
}

float orc_bf16_to_f32(uint16_t value) {
  const uint32_t bits = (uint32_t)value << 16;
  float out;
  memcpy(&out, &bits, sizeof(out));
  return out;
}

static float round_bf16(float v) { return orc_bf16_to_f32(orc_f32_to_bf16(v)); }

uint32_t orc_random_sequence(uint64_t seed, size_t n, uint32_t* out) {
  orc_random r = {seed};
  for (size_t i = 0; i < n; ++i) out[i] = rnd_next(&r);
  return n ? out[n - 1] : 0;
}

static unsigned values_per_word(int bits) { return 32u / (unsigned)bits; }

static uint32_t unpack_q(const uint32_t* row_words, size_t k, int bits) {
  const unsigned vpp = values_per_word(bits);
  const uint32_t mask = (1u << bits) - 1u;
  return (row_words[k / vpp] >> ((unsigned)bits * (k % vpp))) & mask;
}

/* ------------------------------------------------------------------------ */
/* 1. Reference generators and reference CPU oracles (restated)              */
/* ------------------------------------------------------------------------ */

/* Packed words of four masked draws at byte offsets (the q4 quirk: only the
 * low nibble of every byte is ever non-zero).
 * native/src/fused_moe_probe.mm:620-627, quantized_qmv_probe.mm:394-404 */
static uint32_t draw_word(orc_random* r, uint32_t maximum) {
  uint32_t value = 0;
  for (unsigned byte = 0; byte < 4; ++byte) {
    value |= (rnd_next(r) & maximum) << (byte * 8u);
  }
  return value;
}

/*
 * QMV probe dataset and reference output.
 * native/src/quantized_qmv_probe.mm:114-124 (defaults), :344-352 (row map),
 * :355-433 (data + expected).  The expected value of an output row is
 *   sum_g ( sum_{k in g} (q_k * scale) * x_k  +  (sum_{k in g} x_k) * bias ).
 * `selected` may be NULL when n_selected == 0, which the reference turns
 * into the single expert {0}.
 */
int orc_qmv_build(int bits, size_t output_size, size_t reduction_size,
                  size_t group, size_t bank_rows, size_t rows_per_expert,
                  const uint32_t* selected, size_t n_selected,
                  uint32_t* weights, uint16_t* scales, uint16_t* biases,
                  uint16_t* x, float* expected) {
  if (bits != 4 && bits != 8) return ORC_EINVAL;
  const unsigned vpp = values_per_word(bits);
  if (bank_rows == 0) bank_rows = output_size;
  if (rows_per_expert == 0) rows_per_expert = output_size;
  uint32_t zero = 0;
  if (n_selected == 0) {
    selected = &zero;
    n_selected = 1;
  }
  if (reduction_size % vpp || reduction_size % group ||
      bank_rows % rows_per_expert || output_size != n_selected * rows_per_expert)
    return ORC_EINVAL;
  const size_t packed_stride = reduction_size / vpp;
  const size_t groups = reduction_size / group;
  const size_t params = bank_rows * groups;
  float* xv = (float*)malloc(reduction_size * sizeof(float));
  if (!xv) return ORC_EINVAL;

  orc_random r = {bits == 4 ? 0x4A17C0DEull : 0x8A17C0DEull};
  for (size_t i = 0; i < reduction_size; ++i) {
    x[i] = orc_f32_to_bf16(rnd_uniform(&r, -1.0f, 1.0f));
    xv[i] = orc_bf16_to_f32(x[i]);
  }
  const float scale_low = bits == 4 ? 0.002f : 0.00005f;
  const float scale_high = bits == 4 ? 0.008f : 0.00015f;
  for (size_t p = 0; p < params; ++p) {
    scales[p] = orc_f32_to_bf16(rnd_uniform(&r, scale_low, scale_high));
    biases[p] = orc_f32_to_bf16(rnd_uniform(&r, -0.0005f, 0.0005f));
  }
  const uint32_t maximum = bits == 4 ? 0x0Fu : 0xFFu;
  for (size_t row = 0; row < bank_rows; ++row)
    for (size_t w = 0; w < packed_stride; ++w)
      weights[row * packed_stride + w] = draw_word(&r, maximum);

  for (size_t row = 0; row < output_size; ++row) {
    size_t wrow = row;
    if (!(bank_rows == output_size && n_selected == 1)) {
      wrow = (size_t)selected[row / rows_per_expert] * rows_per_expert +
             row % rows_per_expert;
    }
    float result = 0.0f;
    for (size_t g = 0; g < groups; ++g) {
      const float scale = orc_bf16_to_f32(scales[wrow * groups + g]);
      const float bias = orc_bf16_to_f32(biases[wrow * groups + g]);
      float weighted = 0.0f, xsum = 0.0f;
      for (size_t i = 0; i < group; ++i) {
        const size_t k = g * group + i;
        const float q = (float)unpack_q(weights + wrow * packed_stride, k, bits);
        weighted += q * scale * xv[k];
        xsum += xv[k];
      }
      result += weighted + xsum * bias;
    }
    expected[row] = result;
  }
  free(xv);
  return ORC_OK;
}

/* Shapes of the reference's fused probe: native/src/fused_moe_probe.mm:27-32 */
#define FUSED_H 2048
#define FUSED_I 512
#define FUSED_K 8
#define FUSED_G 64

/* Per row: all (scale, bias) draws of the row, then the row's packed words.
 * native/src/fused_moe_probe.mm:600-628 */
static void fill_bank(orc_random* r, int bits, size_t rows, size_t reduction,
                      uint32_t* weights, uint16_t* scales, uint16_t* biases) {
  const size_t stride = reduction / values_per_word(bits);
  const size_t groups = reduction / FUSED_G;
  const float scale_low = bits == 4 ? 0.002f : 0.00005f;
  const float scale_high = bits == 4 ? 0.008f : 0.00015f;
  const uint32_t maximum = bits == 4 ? 0x0Fu : 0xFFu;
  for (size_t row = 0; row < rows; ++row) {
    for (size_t g = 0; g < groups; ++g) {
      scales[row * groups + g] =
          orc_f32_to_bf16(rnd_uniform(r, scale_low, scale_high));
      biases[row * groups + g] =
          orc_f32_to_bf16(rnd_uniform(r, -0.0005f, 0.0005f));
    }
    for (size_t w = 0; w < stride; ++w)
      weights[row * stride + w] = draw_word(r, maximum);
  }
}

/* native/src/fused_moe_probe.mm:449-492 */
int orc_fused_build(int bits, size_t total_experts, uint32_t* gu_w,
                    uint16_t* gu_s, uint16_t* gu_b, uint32_t* dn_w,
                    uint16_t* dn_s, uint16_t* dn_b, uint16_t* x,
                    float* router) {
  if (bits != 4 && bits != 8) return ORC_EINVAL;
  orc_random r = {bits == 4 ? 0xF05EEDB1ull : 0xF05EEDB2ull};
  for (size_t i = 0; i < FUSED_H; ++i)
    x[i] = orc_f32_to_bf16(rnd_uniform(&r, -1.0f, 1.0f));
  fill_bank(&r, bits, total_experts * 2 * FUSED_I, FUSED_H, gu_w, gu_s, gu_b);
  fill_bank(&r, bits, total_experts * FUSED_H, FUSED_I, dn_w, dn_s, dn_b);
  float sum = 0.0f;
  for (size_t j = 0; j < FUSED_K; ++j) {
    router[j] = rnd_uniform(&r, 0.5f, 1.5f);
    sum += router[j];
  }
  for (size_t j = 0; j < FUSED_K; ++j) router[j] /= sum;
  return ORC_OK;
}

/* Reference row dot: per group `weighted * scale + input_sum * bias`.
 * native/src/fused_moe_probe.mm:630-695, quantized_qmm_probe.mm:286-302 */
static float ref_row_dot(const uint32_t* weights, const uint16_t* scales,
                         const uint16_t* biases, size_t row, size_t reduction,
                         int bits, const float* values) {
  const size_t stride = reduction / values_per_word(bits);
  const size_t groups = reduction / FUSED_G;
  float result = 0.0f;
  for (size_t g = 0; g < groups; ++g) {
    const float scale = orc_bf16_to_f32(scales[row * groups + g]);
    const float bias = orc_bf16_to_f32(biases[row * groups + g]);
    float weighted = 0.0f, input_sum = 0.0f;
    for (size_t i = 0; i < FUSED_G; ++i) {
      const size_t k = g * FUSED_G + i;
      weighted += (float)unpack_q(weights + row * stride, k, bits) * values[k];
      input_sum += values[k];
    }
    result += weighted * scale + input_sum * bias;
  }
  return result;
}

/* expected_direct_ of native/src/fused_moe_probe.mm:494-537: per selected
 * slot, SwiGLU over [up; gate] rows, then the router-weighted sum of the
 * expert's down rows.  `intermediate` ([8, 512]) may be NULL. */
int orc_fused_reference(int bits, const uint32_t* selected,
                        const uint32_t* gu_w, const uint16_t* gu_s,
                        const uint16_t* gu_b, const uint32_t* dn_w,
                        const uint16_t* dn_s, const uint16_t* dn_b,
                        const uint16_t* x, const float* router,
                        float* expected_direct, float* intermediate) {
  if (bits != 4 && bits != 8) return ORC_EINVAL;
  float xv[FUSED_H];
  for (size_t i = 0; i < FUSED_H; ++i) xv[i] = orc_bf16_to_f32(x[i]);
  for (size_t h = 0; h < FUSED_H; ++h) expected_direct[h] = 0.0f;
  float inter[FUSED_I];
  for (size_t slot = 0; slot < FUSED_K; ++slot) {
    const size_t e = selected[slot];
    for (size_t c = 0; c < FUSED_I; ++c) {
      const size_t up_row = e * 2 * FUSED_I + c;
      const float up = ref_row_dot(gu_w, gu_s, gu_b, up_row, FUSED_H, bits, xv);
      const float gate =
          ref_row_dot(gu_w, gu_s, gu_b, up_row + FUSED_I, FUSED_H, bits, xv);
      inter[c] = (gate / (1.0f + expf(-gate))) * up;
      if (intermediate) intermediate[slot * FUSED_I + c] = inter[c];
    }
    for (size_t h = 0; h < FUSED_H; ++h) {
      const float v = ref_row_dot(dn_w, dn_s, dn_b, e * FUSED_H + h, FUSED_I,
                                  bits, inter);
      expected_direct[h] += router[slot] * v;
    }
  }
  return ORC_OK;
}

/* native/src/quantized_qmm_probe.mm:243-307 (group fixed at 64). */
int orc_qmm_build(int bits, size_t tokens, size_t outputs, size_t reduction,
                  uint32_t* weights, uint16_t* scales, uint16_t* biases,
                  uint16_t* x, float* expected) {
  if (bits != 4 && bits != 8) return ORC_EINVAL;
  if (reduction % FUSED_G) return ORC_EINVAL;
  const size_t total_x = tokens * reduction;
  float* xv = (float*)malloc(total_x * sizeof(float));
  if (!xv) return ORC_EINVAL;
  orc_random r = {bits == 4 ? 0x4D4D4D01ull : 0x4D4D4D02ull};
  for (size_t i = 0; i < total_x; ++i) {
    x[i] = orc_f32_to_bf16(rnd_uniform(&r, -1.0f, 1.0f));
    xv[i] = orc_bf16_to_f32(x[i]);
  }
  fill_bank(&r, bits, outputs, reduction, weights, scales, biases);
#pragma omp parallel for schedule(static)
  for (long long t = 0; t < (long long)tokens; ++t)
    for (size_t n = 0; n < outputs; ++n)
      expected[(size_t)t * outputs + n] = ref_row_dot(
          weights, scales, biases, n, reduction, bits, xv + (size_t)t * reduction);
  free(xv);
  return ORC_OK;
}

/* ------------------------------------------------------------------------ */
/* 2. The block contract (fp32, OpenMP)                                      */
/* ------------------------------------------------------------------------ */

typedef struct {
  const uint32_t* w;      /* [experts, rows, cols / (32/bits)] */
  const uint16_t* scales; /* bf16 [experts, rows, cols / group] */
  const uint16_t* biases; /* bf16 [experts, rows, cols / group] */
  int32_t experts, rows, cols, bits, group;
} orc_qweight;

typedef struct {
  int32_t hidden, inter, shared_inter, experts, top_k, norm_topk_prob;
  const uint16_t* router_w;      /* bf16 [experts, hidden] */
  const uint16_t* shared_gate_w; /* bf16 [hidden] or NULL */
  orc_qweight gate_up;           /* [experts, 2*inter, hidden], rows [up; gate] */
  orc_qweight down;              /* [experts, hidden, inter] */
  orc_qweight shared_gate_up;    /* [1, 2*shared_inter, hidden] or w == NULL */
  orc_qweight shared_down;       /* [1, hidden, shared_inter] */
  orc_qweight router_q;          /* quantized gate [1, experts, hidden], used
                                    when router_w is NULL */
  orc_qweight shared_gate_q;     /* quantized shared gate [1, 1, hidden], used
                                    when shared_gate_w is NULL and w != NULL */
  const uint16_t* post_norm_w;   /* bf16 [hidden]: RMSNorm of x before the
                                    block, or NULL */
  float norm_eps;
} orc_layer;

/*
 * Router dot product in the fixed order the GPU router kernel uses, so that
 * the bf16 logits (and therefore the selected experts) are bit-identical.
 * The reduction axis is cut into 8-element chunks; lane l of a 64-lane
 * wavefront sums chunks l, l+64, l+128, ... in order, element by element,
 * starting from +0.0f; the 64 lane sums are then combined by a butterfly
 * p_l <- p_l + p_{l xor d} for d = 1, 2, 4, 8, 16, 32.  Products of two bf16
 * values are exact in fp32, so fused and unfused multiply-add agree.
 */
float orc_router_dot(const uint16_t* x, const uint16_t* w, int hidden) {
  float p[64];
  const int chunks = hidden / 8;
  for (int l = 0; l < 64; ++l) {
    float acc = 0.0f;
    for (int c = l; c < chunks; c += 64)
      for (int j = 0; j < 8; ++j)
        acc += orc_bf16_to_f32(x[c * 8 + j]) * orc_bf16_to_f32(w[c * 8 + j]);
    p[l] = acc;
  }
  for (int d = 1; d <= 32; d <<= 1) {
    float q[64];
    for (int l = 0; l < 64; ++l) q[l] = p[l] + p[l ^ d];
    memcpy(p, q, sizeof(p));
  }
  return p[0];
}

/*
 * Quantized gate (MLX affine, group 64) row dot in the GPU router's fixed
 * order.  The codes are cut into 16-byte chunks of V = 128 / bits values;
 * lane l of 64 takes chunks l, l+64, ... from acc = +0: per chunk
 * qa = sum q_i x_i and xs = sum x_i, each sequential from +0 (the products
 * are exact in fp32), then acc = fmaf(qa, s, acc), acc = fmaf(xs, b, acc)
 * with the chunk's group scale and bias; the lane sums are combined by the
 * butterfly of orc_router_dot.
 */
float orc_qrouter_dot(const orc_qweight* qw, int row, const uint16_t* x) {
  const int H = qw->cols, bits = qw->bits, V = 128 / bits;
  const size_t stride = (size_t)H / values_per_word(bits);
  const size_t groups = (size_t)H / (size_t)qw->group;
  const uint32_t* words = qw->w + (size_t)row * stride;
  const int chunks = H / V;
  float p[64];
  for (int l = 0; l < 64; ++l) {
    float acc = 0.0f;
    for (int c = l; c < chunks; c += 64) {
      float qa = 0.0f, xs = 0.0f;
      for (int i = 0; i < V; ++i) {
        const size_t k = (size_t)c * V + (size_t)i;
        const float xv = orc_bf16_to_f32(x[k]);
        qa += (float)unpack_q(words, k, bits) * xv;
        xs += xv;
      }
      const size_t g = (size_t)row * groups + (size_t)c * V / (size_t)qw->group;
      acc = fmaf(qa, orc_bf16_to_f32(qw->scales[g]), acc);
      acc = fmaf(xs, orc_bf16_to_f32(qw->biases[g]), acc);
    }
    p[l] = acc;
  }
  for (int d = 1; d <= 32; d <<= 1) {
    float q[64];
    for (int l = 0; l < 64; ++l) q[l] = p[l] + p[l ^ d];
    memcpy(p, q, sizeof(p));
  }
  return p[0];
}

/*
 * RMSNorm of one bf16 row in front of the block: s = sum x^2 in the router
 * dot's order (orc_router_dot of x with itself; squares of bf16 values are
 * exact), ms = s / H, v = ms + eps, r = 1 / sqrt(v) (each correctly rounded
 * in fp32), out = bf16(bf16(x r) w).
 */
void orc_rms_norm(const uint16_t* x, const uint16_t* w, int hidden, float eps,
                  uint16_t* out) {
  const float s = orc_router_dot(x, x, hidden);
  const float ms = s / (float)hidden;
  const float v = ms + eps;
  const float r = 1.0f / sqrtf(v);
  for (int k = 0; k < hidden; ++k) {
    const float n = round_bf16(orc_bf16_to_f32(x[k]) * r);
    out[k] = orc_f32_to_bf16(n * orc_bf16_to_f32(w[k]));
  }
}

/* Elementwise fmaf, exported so the numpy oracle's float32 FMA can be
 * checked against the C library's. */
void orc_fmaf_array(const float* a, const float* b, const float* c, float* out, size_t n) {
  for (size_t i = 0; i < n; ++i) out[i] = fmaf(a[i], b[i], c[i]);
}

/* Group-affine row dot: sum_g ( s_g * sum_{k in g} q_k v_k + b_g * vsum_g ). */
static float qdot(const orc_qweight* qw, size_t expert, size_t row,
                  const float* v, const float* vsum) {
  const size_t stride = (size_t)qw->cols / values_per_word(qw->bits);
  const size_t groups = (size_t)qw->cols / (size_t)qw->group;
  const size_t grow = expert * (size_t)qw->rows + row;
  const uint32_t* words = qw->w + grow * stride;
  float result = 0.0f;
  for (size_t g = 0; g < groups; ++g) {
    float acc = 0.0f;
    for (size_t i = 0; i < (size_t)qw->group; ++i) {
      const size_t k = g * (size_t)qw->group + i;
      acc += (float)unpack_q(words, k, qw->bits) * v[k];
    }
    const float s = orc_bf16_to_f32(qw->scales[grow * groups + g]);
    const float b = orc_bf16_to_f32(qw->biases[grow * groups + g]);
    result += s * acc + b * vsum[g];
  }
  return result;
}

static void group_sums(const float* v, int n, int group, float* out) {
  for (int g = 0; g < n / group; ++g) {
    float s = 0.0f;
    for (int i = 0; i < group; ++i) s += v[g * group + i];
    out[g] = s;
  }
}

static float silu(float g) { return g / (1.0f + expf(-g)); }

/* act[c] = bf16(silu(bf16(gate_c)) * bf16(up_c)) for one expert row pair. */
static float expert_act(const orc_qweight* gu, size_t expert, int inter, int c,
                        const float* xv, const float* xsum) {
  const float up = round_bf16(qdot(gu, expert, (size_t)c, xv, xsum));
  const float gate = round_bf16(qdot(gu, expert, (size_t)(inter + c), xv, xsum));
  return round_bf16(silu(gate) * up);
}

/*
 * Router for one token: bf16 logits in the canonical order, top-k by
 * (logit desc, expert index asc), softmax over all experts in fp32,
 * probabilities rounded to bf16, renormalised over the selection and
 * rounded to bf16.  Writes idx[top_k] (rank order) and scores[top_k].
 */
void orc_route_token(const orc_layer* L, const uint16_t* x, int32_t* idx,
                     float* scores, float* logits_out) {
  const int E = L->experts, K = L->top_k;
  float logit[1024];
  for (int e = 0; e < E; ++e)
    logit[e] = round_bf16(L->router_w ? orc_router_dot(x, L->router_w + (size_t)e * L->hidden,
                                                       L->hidden)
                                      : orc_qrouter_dot(&L->router_q, e, x));
  if (logits_out) memcpy(logits_out, logit, (size_t)E * sizeof(float));
  unsigned char taken[1024];
  memset(taken, 0, sizeof(taken));
  for (int j = 0; j < K; ++j) {
    int best = -1;
    for (int e = 0; e < E; ++e) {
      if (taken[e]) continue;
      if (best < 0 || logit[e] > logit[best]) best = e;
    }
    taken[best] = 1;
    idx[j] = best;
  }
  float m = logit[0];
  for (int e = 1; e < E; ++e) m = logit[e] > m ? logit[e] : m;
  float z = 0.0f;
  for (int e = 0; e < E; ++e) z += expf(logit[e] - m);
  float pb[64], total = 0.0f;
  for (int j = 0; j < K; ++j) {
    pb[j] = round_bf16(expf(logit[idx[j]] - m) / z);
    total += pb[j];
  }
  /* mlx-lm divides by scores.sum(-1), a bf16 value */
  total = round_bf16(total);
  for (int j = 0; j < K; ++j)
    scores[j] = L->norm_topk_prob ? round_bf16(pb[j] / total) : pb[j];
}

/*
 * Whole block for T tokens: out[t] = bf16( sum_j score_j * y_j
 *     + bf16(sigmoid(bf16(x . w_sg))) * y_shared ), then, if residual is
 * given, out[t] = bf16(residual[t] + out[t]).
 * idx / scores may be NULL.  nthreads <= 0 uses the OpenMP default.
 */
int orc_moe_block(const orc_layer* L, const uint16_t* x, int T,
                  const uint16_t* residual, uint16_t* out, int32_t* idx_out,
                  float* scores_out, int nthreads) {
  if (!L || !x || !out || T < 0) return ORC_EINVAL;
  if (L->top_k > 64 || L->experts > 1024 || L->top_k > L->experts) return ORC_EINVAL;
  if (!L->router_w && (!L->router_q.w || L->router_q.rows != L->experts ||
                       L->router_q.cols != L->hidden || L->router_q.group != 64))
    return ORC_EINVAL;
  const int H = L->hidden, I = L->inter, K = L->top_k;
  const int has_shared = L->shared_gate_up.w != NULL;
  const int Is = has_shared ? L->shared_inter : 0;
  const int maxI = I > Is ? I : Is;
#ifdef _OPENMP
  if (nthreads > 0) omp_set_num_threads(nthreads);
#else
  (void)nthreads;
#endif
  uint16_t* xnorm = L->post_norm_w ? (uint16_t*)malloc((size_t)H * sizeof(uint16_t)) : NULL;
  if (L->post_norm_w && !xnorm) return ORC_EINVAL;
  for (int t = 0; t < T; ++t) {
    const uint16_t* xt = x + (size_t)t * H;
    if (xnorm) {
      orc_rms_norm(xt, L->post_norm_w, H, L->norm_eps, xnorm);
      xt = xnorm;
    }
    int32_t idx[64];
    float scores[64];
    orc_route_token(L, xt, idx, scores, NULL);
    if (idx_out) memcpy(idx_out + (size_t)t * K, idx, (size_t)K * sizeof(int32_t));
    if (scores_out) memcpy(scores_out + (size_t)t * K, scores, (size_t)K * sizeof(float));
    float sgate = 0.0f;
    if (has_shared) {
      const int gated = L->shared_gate_w != NULL || L->shared_gate_q.w != NULL;
      const float sl = L->shared_gate_w ? round_bf16(orc_router_dot(xt, L->shared_gate_w, H))
                       : L->shared_gate_q.w ? round_bf16(orc_qrouter_dot(&L->shared_gate_q, 0, xt))
                                            : 0.0f;
      sgate = gated ? round_bf16(1.0f / (1.0f + expf(-sl))) : 1.0f;
    }
    float* xv = (float*)malloc((size_t)H * sizeof(float));
    float* xsum = (float*)malloc((size_t)H * sizeof(float));
    const int n_units = K + has_shared;
    float* act = (float*)malloc((size_t)n_units * maxI * sizeof(float));
    float* asum = (float*)malloc((size_t)n_units * maxI * sizeof(float));
    if (!xv || !xsum || !act || !asum) {
      free(xv); free(xsum); free(act); free(asum); free(xnorm);
      return ORC_EINVAL;
    }
    for (int h = 0; h < H; ++h) xv[h] = orc_bf16_to_f32(xt[h]);
    group_sums(xv, H, L->gate_up.group, xsum);
    /* Gate/up rows of every unit, then the down rows; each output value is
     * computed by one thread in the same order whatever the thread count. */
#pragma omp parallel for schedule(static)
    for (int uc = 0; uc < n_units * maxI; ++uc) {
      const int u = uc / maxI, c = uc % maxI;
      if (u < K) {
        if (c < I) act[(size_t)u * maxI + c] = expert_act(&L->gate_up, (size_t)idx[u], I, c, xv, xsum);
      } else if (c < Is) {
        act[(size_t)u * maxI + c] = expert_act(&L->shared_gate_up, 0, Is, c, xv, xsum);
      }
    }
    for (int u = 0; u < n_units; ++u) {
      const int Iu = u < K ? I : Is;
      group_sums(act + (size_t)u * maxI, Iu, L->down.group, asum + (size_t)u * maxI);
    }
#pragma omp parallel for schedule(static)
    for (int h = 0; h < H; ++h) {
      float acc = 0.0f;
      for (int j = 0; j < K; ++j) {
        const float y = round_bf16(qdot(&L->down, (size_t)idx[j], (size_t)h,
                                        act + (size_t)j * maxI, asum + (size_t)j * maxI));
        acc += scores[j] * y;
      }
      if (has_shared) {
        const float y = round_bf16(qdot(&L->shared_down, 0, (size_t)h,
                                        act + (size_t)K * maxI, asum + (size_t)K * maxI));
        acc += sgate * y;
      }
      float o = round_bf16(acc);
      if (residual) o = round_bf16(orc_bf16_to_f32(residual[(size_t)t * H + h]) + o);
      out[(size_t)t * H + h] = orc_f32_to_bf16(o);
    }
    free(xv);
    free(xsum);
    free(act);
    free(asum);
  }
  free(xnorm);
  return ORC_OK;
}

int orc_max_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}
