/*
 * oracle_model.c -- CPU restatement of the verify forward (decoder over MLX
 * 4-bit affine g64 weights, per-row KV with O(1) rollback by length).
 *
 * TEST INFRASTRUCTURE ONLY (parity checker and CPU baseline); the product
 * never links this file.  Layer wiring follows the public mlx-lm Qwen3 /
 * Llama / Qwen3-MoE definitions (EXTERNAL to the reference tree, so its
 * rounding is parity-unpinned and compared within bf16 tolerance).
 */
#include "oracle.h"
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

static inline float bf(uint16_t h) { return or_bf16_to_f32(h); }
static inline uint16_t tobf(float f) { return or_f32_to_bf16(f); }

/* ------------------------------------------------------------------ */
/* model                                                                */
/* ------------------------------------------------------------------ */
typedef struct or_linear { int N, K; uint32_t* wq; uint16_t* s; uint16_t* b; } or_linear;
typedef struct or_layer {
  or_linear q, k, v, o, gate, up, down, router;
  or_linear* experts; /* [n_experts * 3]: gate, up, down */
  uint16_t *in_norm, *post_norm, *q_norm, *k_norm;
  uint16_t *kc, *vc;  /* [max_rows][n_kv][max_ctx][d] */
} or_layer;

struct or_model {
  or_config cfg;
  uint64_t seed;
  int max_ctx, max_rows;
  or_linear embed, lm_head;
  uint16_t* final_norm;
  or_layer* layers;
  float *rope_cos, *rope_sin;
  int* kv_len;
  int fake;
};

static int g_threads = 0;
/* 1: every fp32 reduction runs in another order -- the linears sum their 64-wide groups
 * last to first, RMSNorm and the attention dot products sum sequentially from the last
 * element, softmax sums run over the keys last to first.  Mathematically the same forward;
 * its distance from the default order is the rounding noise floor of a correct
 * implementation that sums in another order. */
static int g_reversed = 0;
void or_set_reduction_order(int reversed) { g_reversed = reversed != 0; }

void or_set_threads(int n) {
  g_threads = n;
#ifdef _OPENMP
  if (n > 0) omp_set_num_threads(n);
#endif
}

static void lin_alloc(or_linear* L, int N, int K) {
  L->N = N; L->K = K;
  L->wq = (uint32_t*)malloc(sizeof(uint32_t) * (size_t)N * (size_t)(K / 8));
  L->s = (uint16_t*)malloc(sizeof(uint16_t) * (size_t)N * (size_t)(K / 64));
  L->b = (uint16_t*)malloc(sizeof(uint16_t) * (size_t)N * (size_t)(K / 64));
}
static void lin_gen(or_linear* L, uint64_t seed, uint64_t tid, int N, int K, int scale_exp) {
  lin_alloc(L, N, K);
  or_gen_linear(seed, tid, N, K, scale_exp, L->wq, L->s, L->b);
}
static void lin_free(or_linear* L) { free(L->wq); free(L->s); free(L->b); }

or_model* or_model_create(const or_config* cfg, uint64_t seed, int max_ctx, int max_rows) {
  or_model* m = (or_model*)calloc(1, sizeof(or_model));
  m->cfg = *cfg;
  m->seed = seed;
  m->max_ctx = max_ctx;
  m->max_rows = max_rows;
  m->kv_len = (int*)calloc((size_t)max_rows, sizeof(int));
  if (cfg->arch >= 100) { m->fake = 1; return m; }
  const int H = cfg->hidden, d = cfg->head_dim, nq = cfg->n_q_heads, nkv = cfg->n_kv_heads;
  const int I = cfg->intermediate, V = cfg->vocab, L = cfg->n_layers;
  lin_gen(&m->embed, seed, OR_TID_EMBED, V, H, -7);
  if (!cfg->tied_embeddings) lin_gen(&m->lm_head, seed, OR_TID_LM_HEAD, V, H, -7);
  m->final_norm = (uint16_t*)malloc(2 * (size_t)H);
  or_gen_norm(seed, OR_TID_FINAL_NORM, H, m->final_norm);
  m->layers = (or_layer*)calloc((size_t)L, sizeof(or_layer));
  for (int l = 0; l < L; ++l) {
    or_layer* y = &m->layers[l];
    lin_gen(&y->q, seed, or_tensor_id(l, OR_T_Q), nq * d, H, -7);
    lin_gen(&y->k, seed, or_tensor_id(l, OR_T_K), nkv * d, H, -7);
    lin_gen(&y->v, seed, or_tensor_id(l, OR_T_V), nkv * d, H, -7);
    lin_gen(&y->o, seed, or_tensor_id(l, OR_T_O), H, nq * d, -7);
    if (cfg->arch == OR_ARCH_QWEN3_MOE) {
      const int E = cfg->n_experts, MI = cfg->moe_intermediate;
      lin_gen(&y->router, seed, or_tensor_id(l, OR_T_ROUTER), E, H, -7);
      y->experts = (or_linear*)calloc((size_t)E * 3, sizeof(or_linear));
      for (int e = 0; e < E; ++e) {
        lin_gen(&y->experts[e * 3 + 0], seed, or_expert_tensor_id(l, e, OR_T_GATE), MI, H, -7);
        lin_gen(&y->experts[e * 3 + 1], seed, or_expert_tensor_id(l, e, OR_T_UP), MI, H, -7);
        lin_gen(&y->experts[e * 3 + 2], seed, or_expert_tensor_id(l, e, OR_T_DOWN), H, MI, -7);
      }
    } else {
      lin_gen(&y->gate, seed, or_tensor_id(l, OR_T_GATE), I, H, -7);
      lin_gen(&y->up, seed, or_tensor_id(l, OR_T_UP), I, H, -7);
      lin_gen(&y->down, seed, or_tensor_id(l, OR_T_DOWN), H, I, -7);
    }
    y->in_norm = (uint16_t*)malloc(2 * (size_t)H);
    y->post_norm = (uint16_t*)malloc(2 * (size_t)H);
    or_gen_norm(seed, or_tensor_id(l, OR_T_IN_NORM), H, y->in_norm);
    or_gen_norm(seed, or_tensor_id(l, OR_T_POST_NORM), H, y->post_norm);
    if (cfg->arch != OR_ARCH_LLAMA) {
      y->q_norm = (uint16_t*)malloc(2 * (size_t)d);
      y->k_norm = (uint16_t*)malloc(2 * (size_t)d);
      or_gen_norm(seed, or_tensor_id(l, OR_T_Q_NORM), d, y->q_norm);
      or_gen_norm(seed, or_tensor_id(l, OR_T_K_NORM), d, y->k_norm);
    }
    size_t kvn = (size_t)max_rows * nkv * (size_t)max_ctx * d;
    y->kc = (uint16_t*)calloc(kvn, 2);
    y->vc = (uint16_t*)calloc(kvn, 2);
  }
  /* RoPE table (non-traditional / rotate-half): angle = pos * theta^(-2i/d), in double */
  const int hd = d / 2;
  m->rope_cos = (float*)malloc(sizeof(float) * (size_t)max_ctx * hd);
  m->rope_sin = (float*)malloc(sizeof(float) * (size_t)max_ctx * hd);
  for (int p = 0; p < max_ctx; ++p)
    for (int i = 0; i < hd; ++i) {
      double inv = pow((double)cfg->rope_theta, -2.0 * (double)i / (double)d);
      double a = (double)p * inv;
      m->rope_cos[(size_t)p * hd + i] = (float)cos(a);
      m->rope_sin[(size_t)p * hd + i] = (float)sin(a);
    }
  return m;
}

void or_model_destroy(or_model* m) {
  if (!m) return;
  if (!m->fake) {
    lin_free(&m->embed);
    if (!m->cfg.tied_embeddings) lin_free(&m->lm_head);
    free(m->final_norm);
    for (int l = 0; l < m->cfg.n_layers; ++l) {
      or_layer* y = &m->layers[l];
      lin_free(&y->q); lin_free(&y->k); lin_free(&y->v); lin_free(&y->o);
      if (y->experts) {
        lin_free(&y->router);
        for (int e = 0; e < m->cfg.n_experts * 3; ++e) lin_free(&y->experts[e]);
        free(y->experts);
      } else {
        lin_free(&y->gate); lin_free(&y->up); lin_free(&y->down);
      }
      free(y->in_norm); free(y->post_norm); free(y->q_norm); free(y->k_norm);
      free(y->kc); free(y->vc);
    }
    free(m->layers);
    free(m->rope_cos); free(m->rope_sin);
  }
  free(m->kv_len);
  free(m);
}

int or_model_linear(or_model* m, int layer, int which, int expert, const uint32_t** wq,
                    const uint16_t** s, const uint16_t** b, int* N, int* K) {
  if (m->fake) return -1;
  or_linear* L = NULL;
  if (layer < 0) {
    L = which == 0 ? &m->embed : (m->cfg.tied_embeddings ? &m->embed : &m->lm_head);
  } else {
    if (layer >= m->cfg.n_layers) return -1;
    or_layer* y = &m->layers[layer];
    if (expert >= 0) {
      if (!y->experts || expert >= m->cfg.n_experts) return -1;
      int slot = which == OR_T_GATE ? 0 : which == OR_T_UP ? 1 : which == OR_T_DOWN ? 2 : -1;
      if (slot < 0) return -1;
      L = &y->experts[expert * 3 + slot];
    } else {
      switch (which) {
        case OR_T_Q: L = &y->q; break;
        case OR_T_K: L = &y->k; break;
        case OR_T_V: L = &y->v; break;
        case OR_T_O: L = &y->o; break;
        case OR_T_GATE: L = y->experts ? NULL : &y->gate; break;
        case OR_T_UP: L = y->experts ? NULL : &y->up; break;
        case OR_T_DOWN: L = y->experts ? NULL : &y->down; break;
        case OR_T_ROUTER: L = y->experts ? &y->router : NULL; break;
        default: L = NULL;
      }
    }
  }
  if (!L) return -1;
  *wq = L->wq; *s = L->s; *b = L->b; *N = L->N; *K = L->K;
  return 0;
}

const or_config* or_model_cfg(or_model* m) { return &m->cfg; }
const float* or_model_rope_cos(or_model* m) { return m->rope_cos; }
const float* or_model_rope_sin(or_model* m) { return m->rope_sin; }
int or_kv_len(or_model* m, int row) { return m->kv_len[row]; }
void or_kv_set_len(or_model* m, int row, int len) { m->kv_len[row] = len; }

static inline size_t kv_index(const or_model* m, int row, int h, int pos) {
  return (((size_t)row * m->cfg.n_kv_heads + h) * (size_t)m->max_ctx + pos) * m->cfg.head_dim;
}

void or_kv_fill_synthetic(or_model* m, int row, int n, uint64_t seed) {
  if (m->fake) { m->kv_len[row] = n; return; }
  const int d = m->cfg.head_dim, nkv = m->cfg.n_kv_heads;
  for (int l = 0; l < m->cfg.n_layers; ++l)
    for (int w = 0; w < 2; ++w) {
      uint16_t* c = w ? m->layers[l].vc : m->layers[l].kc;
#pragma omp parallel for schedule(static)
      for (int h = 0; h < nkv; ++h)
        for (int p = 0; p < n; ++p)
          for (int i = 0; i < d; ++i) {
            uint64_t hh = or_mix64(seed ^ or_mix64((((uint64_t)l * 2 + w) << 40) ^ ((uint64_t)row << 32) ^
                                                    ((uint64_t)h << 24) ^ ((uint64_t)p << 8)) ^ (uint64_t)i);
            /* bf16 in [-1, 1): sign, exponent 2^-1..2^-4, 7 random mantissa bits */
            uint32_t sign = (uint32_t)(hh & 1u), e = 126u - (uint32_t)((hh >> 1) & 3u), mant = (uint32_t)((hh >> 3) & 0x7Fu);
            c[kv_index(m, row, h, p) + i] = (uint16_t)((sign << 15) | (e << 7) | mant);
          }
    }
  m->kv_len[row] = n;
}

void or_kv_read(or_model* m, int layer, int row, int which_v, uint16_t* out) {
  const int d = m->cfg.head_dim, nkv = m->cfg.n_kv_heads, len = m->kv_len[row];
  uint16_t* c = which_v ? m->layers[layer].vc : m->layers[layer].kc;
  for (int h = 0; h < nkv; ++h)
    memcpy(out + (size_t)h * len * d, c + kv_index(m, row, h, 0), (size_t)len * d * 2);
}

/* y[m][n] = sum_g ( s_ng * sum_{k in g} x_mk q_nk + b_ng * sum_{k in g} x_mk ), fp32.
 * Each output is one thread's fixed-order sum, independent of M. */
static void qlinear(const or_linear* L, const float* x, int M, float* y) {
  const int K = L->K, N = L->N, G = K / 64, KW = K / 8;
  float* xs = (float*)malloc(sizeof(float) * (size_t)M * G);
  for (int m = 0; m < M; ++m)
    for (int g = 0; g < G; ++g) {
      const float* xp = x + (size_t)m * K + g * 64;
      float a[8] = {0, 0, 0, 0, 0, 0, 0, 0};
      for (int k = 0; k < 64; k += 8)
        for (int j = 0; j < 8; ++j) a[j] += xp[k + j];
      xs[(size_t)m * G + g] = ((a[0] + a[1]) + (a[2] + a[3])) + ((a[4] + a[5]) + (a[6] + a[7]));
    }
#pragma omp parallel
  {
    float* accm = (float*)malloc(sizeof(float) * (size_t)M);
    float q[64];
#pragma omp for schedule(static)
    for (int n = 0; n < N; ++n) {
      for (int m = 0; m < M; ++m) accm[m] = 0.0f;
      for (int gi = 0; gi < G; ++gi) {
        const int g = g_reversed ? G - 1 - gi : gi;
        for (int w = 0; w < 8; ++w) {
          uint32_t word = L->wq[(size_t)n * KW + g * 8 + w];
          for (int j = 0; j < 8; ++j) q[w * 8 + j] = (float)((word >> (4 * j)) & 0xFu);
        }
        float s = bf(L->s[(size_t)n * G + g]), b = bf(L->b[(size_t)n * G + g]);
        for (int m = 0; m < M; ++m) {
          const float* xp = x + (size_t)m * K + g * 64;
          float a[8] = {0, 0, 0, 0, 0, 0, 0, 0};
          for (int k = 0; k < 64; k += 8)
            for (int j = 0; j < 8; ++j) a[j] += xp[k + j] * q[k + j];
          float dot = ((a[0] + a[1]) + (a[2] + a[3])) + ((a[4] + a[5]) + (a[6] + a[7]));
          accm[m] += s * dot + b * xs[(size_t)m * G + g];
        }
      }
      for (int m = 0; m < M; ++m) y[(size_t)m * N + n] = accm[m];
    }
    free(accm);
  }
  free(xs);
}

void or_qmatmul(const uint32_t* wq, const uint16_t* scales, const uint16_t* biases, int N, int K,
                const float* x, int M, float* y) {
  or_linear L;
  L.N = N; L.K = K;
  L.wq = (uint32_t*)wq; L.s = (uint16_t*)scales; L.b = (uint16_t*)biases;
  qlinear(&L, x, M, y);
}

/* rmsnorm over n values: y = bf16((x * r) * w), r = 1/sqrt(mean(x^2) + eps) */
static void rmsnorm(const float* x, const uint16_t* w, int n, float eps, float* out) {
  float a[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  int i = 0;
  for (; i + 8 <= n; i += 8)
    for (int j = 0; j < 8; ++j) a[j] += x[i + j] * x[i + j];
  for (; i < n; ++i) a[0] += x[i] * x[i];
  float ss = ((a[0] + a[1]) + (a[2] + a[3])) + ((a[4] + a[5]) + (a[6] + a[7]));
  if (g_reversed) {
    ss = 0.0f;
    for (int k = n - 1; k >= 0; --k) ss += x[k] * x[k];
  }
  float r = 1.0f / sqrtf(ss / (float)n + eps);
  for (int k = 0; k < n; ++k) out[k] = bf(tobf((x[k] * r) * bf(w[k])));
}

static void rope(float* v, int d, const float* cs, const float* sn) {
  const int h = d / 2;
  for (int i = 0; i < h; ++i) {
    float x1 = v[i], x2 = v[i + h];
    float o1 = x1 * cs[i] - x2 * sn[i];
    float o2 = x1 * sn[i] + x2 * cs[i];
    v[i] = bf(tobf(o1));
    v[i + h] = bf(tobf(o2));
  }
}

static float silu(float z) { return z / (1.0f + expf(-z)); }

typedef struct { int row, pos; } tokpos_t;

static void fake_logits(const or_model* m, const int32_t* tokens, int M, uint16_t* logits) {
  const int V = m->cfg.vocab;
  for (int t = 0; t < M; ++t) {
    int tok = tokens[t];
    int nx = tok == 1 ? 2 : tok == 2 ? 3 : 1;            /* SchedulerSpeculativeDecodingTests.swift:225-234 */
    if (m->cfg.arch == OR_ARCH_FAKE_MISMATCHING && tok == 3) nx = 4;  /* :257-261 */
    for (int v = 0; v < V; ++v) logits[(size_t)t * V + v] = tobf(v == nx ? 20.0f : -20.0f); /* :236-248 */
  }
}

int or_forward_trace(or_model* m, int nrows, const int32_t* rows, const int32_t* counts,
                     const int32_t* tokens, uint16_t* logits, uint16_t* hidden) {
  return or_forward_attn(m, nrows, rows, counts, tokens, logits, hidden, NULL);
}

static uint16_t* g_router_out = NULL;
void or_capture_router(uint16_t* out) { g_router_out = out; }

int or_forward_attn(or_model* m, int nrows, const int32_t* rows, const int32_t* counts,
                    const int32_t* tokens, uint16_t* logits, uint16_t* hidden, uint16_t* attn) {
  const or_config* c = &m->cfg;
  int M = 0;
  for (int i = 0; i < nrows; ++i) {
    if (rows[i] < 0 || rows[i] >= m->max_rows) return -1;
    if (m->kv_len[rows[i]] + counts[i] > m->max_ctx) return -2;
    M += counts[i];
  }
  if (M == 0) return 0;
  tokpos_t* tp = (tokpos_t*)malloc(sizeof(tokpos_t) * (size_t)M);
  for (int i = 0, t = 0; i < nrows; ++i)
    for (int j = 0; j < counts[i]; ++j, ++t) { tp[t].row = rows[i]; tp[t].pos = m->kv_len[rows[i]] + j; }
  if (m->fake) {
    if (logits) fake_logits(m, tokens, M, logits);
    for (int i = 0; i < nrows; ++i) m->kv_len[rows[i]] += counts[i];
    free(tp);
    return 0;
  }
  const int H = c->hidden, d = c->head_dim, nq = c->n_q_heads, nkv = c->n_kv_heads, V = c->vocab;
  const int I = c->arch == OR_ARCH_QWEN3_MOE ? c->moe_intermediate : c->intermediate;
  const int hd = d / 2, grp = nq / nkv;
  const float scale = 1.0f / sqrtf((float)d);
  float* x = (float*)malloc(sizeof(float) * (size_t)M * H);
  float* xn = (float*)malloc(sizeof(float) * (size_t)M * H);
  float* q = (float*)malloc(sizeof(float) * (size_t)M * nq * d);
  float* k = (float*)malloc(sizeof(float) * (size_t)M * nkv * d);
  float* v = (float*)malloc(sizeof(float) * (size_t)M * nkv * d);
  float* att = (float*)malloc(sizeof(float) * (size_t)M * nq * d);
  float* o = (float*)malloc(sizeof(float) * (size_t)M * H);
  float* g = (float*)malloc(sizeof(float) * (size_t)M * I);
  float* u = (float*)malloc(sizeof(float) * (size_t)M * I);
  float* act = (float*)malloc(sizeof(float) * (size_t)M * I);
  /* embedding: dequantized row, bf16(s*q + b) */
  {
    const or_linear* E = &m->embed;
    const int G = H / 64, KW = H / 8;
    for (int t = 0; t < M; ++t) {
      int tok = tokens[t];
      if (tok < 0 || tok >= V) tok = 0;
      for (int kk = 0; kk < H; ++kk) {
        uint32_t word = E->wq[(size_t)tok * KW + kk / 8];
        float qv = (float)((word >> (4 * (kk % 8))) & 0xFu);
        float s = bf(E->s[(size_t)tok * G + kk / 64]), b = bf(E->b[(size_t)tok * G + kk / 64]);
        x[(size_t)t * H + kk] = bf(tobf(fmaf(s, qv, b)));
      }
    }
  }
  if (hidden)
    for (size_t i = 0; i < (size_t)M * H; ++i) hidden[i] = tobf(x[i]);
  for (int l = 0; l < c->n_layers; ++l) {
    or_layer* y = &m->layers[l];
    for (int t = 0; t < M; ++t) rmsnorm(x + (size_t)t * H, y->in_norm, H, c->rms_eps, xn + (size_t)t * H);
    qlinear(&y->q, xn, M, q);
    qlinear(&y->k, xn, M, k);
    qlinear(&y->v, xn, M, v);
    for (size_t i = 0; i < (size_t)M * nq * d; ++i) q[i] = bf(tobf(q[i]));
    for (size_t i = 0; i < (size_t)M * nkv * d; ++i) { k[i] = bf(tobf(k[i])); v[i] = bf(tobf(v[i])); }
    for (int t = 0; t < M; ++t) {
      const float* cs = m->rope_cos + (size_t)tp[t].pos * hd;
      const float* sn = m->rope_sin + (size_t)tp[t].pos * hd;
      for (int h = 0; h < nq; ++h) {
        float* qv = q + ((size_t)t * nq + h) * d;
        if (y->q_norm) { float tmp[512]; rmsnorm(qv, y->q_norm, d, c->rms_eps, tmp); memcpy(qv, tmp, sizeof(float) * d); }
        rope(qv, d, cs, sn);
      }
      for (int h = 0; h < nkv; ++h) {
        float* kv = k + ((size_t)t * nkv + h) * d;
        if (y->k_norm) { float tmp[512]; rmsnorm(kv, y->k_norm, d, c->rms_eps, tmp); memcpy(kv, tmp, sizeof(float) * d); }
        rope(kv, d, cs, sn);
        size_t base = kv_index(m, tp[t].row, h, tp[t].pos);
        for (int i = 0; i < d; ++i) {
          y->kc[base + i] = tobf(kv[i]);
          y->vc[base + i] = tobf(v[((size_t)t * nkv + h) * d + i]);
        }
      }
    }
    /* attention: query at pos p sees keys [0, p] of its row (CausalMask.swift:4-28) */
#pragma omp parallel for collapse(2) schedule(static)
    for (int t = 0; t < M; ++t)
      for (int h = 0; h < nq; ++h) {
        const int kh = h / grp, row = tp[t].row, P = tp[t].pos;
        const float* qv = q + ((size_t)t * nq + h) * d;
        float* sc = (float*)malloc(sizeof(float) * (size_t)(P + 1));
        float mx = -INFINITY;
        for (int j = 0; j <= P; ++j) {
          const uint16_t* kk = y->kc + kv_index(m, row, kh, j);
          float a[8] = {0, 0, 0, 0, 0, 0, 0, 0};
          for (int i = 0; i < d; i += 8)
            for (int z = 0; z < 8; ++z) a[z] += qv[i + z] * bf(kk[i + z]);
          float dsum = ((a[0] + a[1]) + (a[2] + a[3])) + ((a[4] + a[5]) + (a[6] + a[7]));
          if (g_reversed) {
            dsum = 0.0f;
            for (int i = d - 1; i >= 0; --i) dsum += qv[i] * bf(kk[i]);
          }
          float s = dsum * scale;
          sc[j] = s;
          if (s > mx) mx = s;
        }
        float den = 0.0f;
        float acc[512];
        for (int i = 0; i < d; ++i) acc[i] = 0.0f;
        for (int jj = 0; jj <= P; ++jj) {
          const int j = g_reversed ? P - jj : jj;
          float p = expf(sc[j] - mx);
          den += p;
          const uint16_t* vv = y->vc + kv_index(m, row, kh, j);
          for (int i = 0; i < d; ++i) acc[i] += p * bf(vv[i]);
        }
        float inv = 1.0f / den;
        for (int i = 0; i < d; ++i) att[((size_t)t * nq + h) * d + i] = bf(tobf(acc[i] * inv));
        free(sc);
      }
    if (attn)
      for (size_t i = 0; i < (size_t)M * nq * d; ++i) attn[(size_t)l * M * nq * d + i] = tobf(att[i]);
    qlinear(&y->o, att, M, o);
    for (size_t i = 0; i < (size_t)M * H; ++i) x[i] = bf(tobf(x[i] + o[i]));
    for (int t = 0; t < M; ++t) rmsnorm(x + (size_t)t * H, y->post_norm, H, c->rms_eps, xn + (size_t)t * H);
    if (c->arch == OR_ARCH_QWEN3_MOE) {
      const int E = c->n_experts, TK = c->n_experts_per_tok;
      float* rl = (float*)malloc(sizeof(float) * (size_t)M * E);
      qlinear(&y->router, xn, M, rl);
      float* mo = (float*)calloc((size_t)M * H, sizeof(float));
      for (int t = 0; t < M; ++t) {
        /* router: softmax in fp32 over bf16 logits, top-k (ties -> lower index), renormalise */
        float* r = rl + (size_t)t * E;
        float mxr = -INFINITY;
        for (int e = 0; e < E; ++e) { r[e] = bf(tobf(r[e])); if (r[e] > mxr) mxr = r[e]; }
        if (g_router_out)
          for (int e = 0; e < E; ++e) g_router_out[((size_t)l * M + t) * E + e] = tobf(r[e]);
        float den = 0.0f;
        for (int e = 0; e < E; ++e) { r[e] = expf(r[e] - mxr); den += r[e]; }
        for (int e = 0; e < E; ++e) r[e] /= den;
        int sel[64];
        float wsel[64], wsum = 0.0f;
        for (int kk = 0; kk < TK; ++kk) {
          int best = -1;
          for (int e = 0; e < E; ++e) {
            int used = 0;
            for (int z = 0; z < kk; ++z) used |= sel[z] == e;
            if (used) continue;
            if (best < 0 || r[e] > r[best]) best = e;
          }
          sel[kk] = best; wsel[kk] = r[best]; wsum += r[best];
        }
        for (int kk = 0; kk < TK; ++kk) {
          const int e = sel[kk];
          const float w = wsel[kk] / wsum;
          float* gg = (float*)malloc(sizeof(float) * I);
          float* uu = (float*)malloc(sizeof(float) * I);
          float* aa = (float*)malloc(sizeof(float) * I);
          float* dd = (float*)malloc(sizeof(float) * H);
          qlinear(&y->experts[e * 3 + 0], xn + (size_t)t * H, 1, gg);
          qlinear(&y->experts[e * 3 + 1], xn + (size_t)t * H, 1, uu);
          for (int i = 0; i < I; ++i) aa[i] = bf(tobf(silu(gg[i]) * uu[i]));
          qlinear(&y->experts[e * 3 + 2], aa, 1, dd);
          for (int i = 0; i < H; ++i) mo[(size_t)t * H + i] += w * dd[i];
          free(gg); free(uu); free(aa); free(dd);
        }
      }
      for (size_t i = 0; i < (size_t)M * H; ++i) x[i] = bf(tobf(x[i] + mo[i]));
      free(mo);
      free(rl);
    } else {
      qlinear(&y->gate, xn, M, g);
      qlinear(&y->up, xn, M, u);
      for (size_t i = 0; i < (size_t)M * I; ++i) act[i] = bf(tobf(silu(g[i]) * u[i]));
      qlinear(&y->down, act, M, o);
      for (size_t i = 0; i < (size_t)M * H; ++i) x[i] = bf(tobf(x[i] + o[i]));
    }
    if (hidden)
      for (size_t i = 0; i < (size_t)M * H; ++i) hidden[(size_t)(l + 1) * M * H + i] = tobf(x[i]);
  }
  if (logits) {
    for (int t = 0; t < M; ++t) rmsnorm(x + (size_t)t * H, m->final_norm, H, c->rms_eps, xn + (size_t)t * H);
    const or_linear* LM = c->tied_embeddings ? &m->embed : &m->lm_head;
    float* lg = (float*)malloc(sizeof(float) * (size_t)M * V);
    qlinear(LM, xn, M, lg);
    for (size_t i = 0; i < (size_t)M * V; ++i) logits[i] = tobf(lg[i]);
    free(lg);
  }
  for (int i = 0; i < nrows; ++i) m->kv_len[rows[i]] += counts[i];
  free(x); free(xn); free(q); free(k); free(v); free(att); free(o); free(g); free(u); free(act);
  free(tp);
  return 0;
}

int or_forward(or_model* m, int nrows, const int32_t* rows, const int32_t* counts,
               const int32_t* tokens, uint16_t* logits) {
  return or_forward_trace(m, nrows, rows, counts, tokens, logits, NULL);
}

