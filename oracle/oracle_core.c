/*
 * oracle.c -- CPU restatement of mlxcat's n-gram speculative-decode step.
 *
 * TEST INFRASTRUCTURE ONLY: the parity checker and CPU baseline for the HIP
 * product.  The product never links or calls this file.  Reference citations
 * are to local-ai-cat/mlxcat (paths relative to its root); see oracle.h.
 *
 * Built with -ffp-contract=off so that the integer-mass acceptance helpers
 * (or_exp_neg and the top-p / sampling arithmetic) evaluate exactly the
 * operation sequence the GPU evaluates.
 */
#include "oracle.h"
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ------------------------------------------------------------------ */
/* integer generators                                                   */
/* ------------------------------------------------------------------ */
uint64_t or_mix64(uint64_t z) {
  /* splitmix64 finalizer (Steele, Lea, Flood 2014) */
  z += 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

uint32_t or_uniform_u32(uint64_t seed, uint64_t counter, uint32_t pos, uint32_t kind) {
  uint64_t h = or_mix64(seed ^ 0x5851F42D4C957F2Dull);
  h = or_mix64(h ^ counter);
  h = or_mix64(h ^ (((uint64_t)pos << 8) | kind));
  return (uint32_t)(h >> 32);
}

uint16_t or_f32_to_bf16(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  if ((u & 0x7F800000u) == 0x7F800000u && (u & 0x007FFFFFu)) return (uint16_t)((u >> 16) | 0x40);
  uint32_t r = u + 0x7FFFu + ((u >> 16) & 1u);
  return (uint16_t)(r >> 16);
}

float or_bf16_to_f32(uint16_t h) {
  uint32_t u = (uint32_t)h << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

static inline float bf(uint16_t h) { return or_bf16_to_f32(h); }
static inline uint16_t tobf(float f) { return or_f32_to_bf16(f); }

uint64_t or_tensor_id(int layer, int which) { return ((uint64_t)(layer + 1) << 8) | (uint64_t)which; }
uint64_t or_expert_tensor_id(int layer, int expert, int which) {
  return 0x100000000ull | ((uint64_t)layer << 20) | ((uint64_t)expert << 4) | (uint64_t)which;
}

void or_gen_linear(uint64_t seed, uint64_t tid, int N, int K, int scale_exp, uint32_t* wq,
                   uint16_t* scales, uint16_t* biases) {
  const int KW = K / 8, G = K / 64;
  const uint64_t base = or_mix64(seed ^ or_mix64(tid));
#pragma omp parallel for schedule(static)
  for (int n = 0; n < N; ++n) {
    for (int kw = 0; kw < KW; ++kw) {
      uint64_t idx = ((uint64_t)n * (uint64_t)KW + (uint64_t)kw) * 2u;
      uint64_t h0 = or_mix64(base ^ idx), h1 = or_mix64(base ^ (idx + 1));
      uint32_t w = 0;
      for (int j = 0; j < 8; ++j) {
        uint64_t h = j < 4 ? h0 : h1;
        uint32_t q = (uint32_t)__builtin_popcountll((h >> (15 * (j & 3))) & 0x7FFFull);
        w |= q << (4 * j);
      }
      wq[(size_t)n * KW + kw] = w;
    }
    for (int g = 0; g < G; ++g) {
      uint64_t h = or_mix64(base ^ 0xA5A5A5A500000000ull ^ ((uint64_t)n * (uint64_t)G + (uint64_t)g));
      uint16_t sb = (uint16_t)(((uint32_t)(127 + scale_exp) << 7) | (0x28u + (uint32_t)(h & 0xFu)));
      float s = bf(sb);
      scales[(size_t)n * G + g] = sb;
      biases[(size_t)n * G + g] = tobf(-7.5f * s);
    }
  }
}

void or_gen_norm(uint64_t seed, uint64_t tid, int n, uint16_t* w) {
  const uint64_t base = or_mix64(seed ^ or_mix64(tid ^ 0x4E4F524Dull));
  for (int i = 0; i < n; ++i) {
    uint64_t h = or_mix64(base ^ (uint64_t)i);
    int k = (int)(h % 32u) - 16;
    w[i] = tobf(1.0f + (float)k / 128.0f);
  }
}

/* ------------------------------------------------------------------ */
/* exp for the acceptance masses                                        */
/* ------------------------------------------------------------------ */
float or_exp_neg(float x) {
  /* x <= 0.  2^y with y = x*log2(e); y = n + f, n = rint(y), |f| <= 1/2;
   * 2^f = sum_k (f ln2)^k / k!, k <= 7, coefficients (ln 2)^k / k! rounded to float. */
  if (!(x > -87.0f)) return 0.0f;
  const float LOG2E = 1.44269504088896341f;
  float y = x * LOG2E;
  float n = rintf(y);
  float f = y - n;
  if (n < -40.0f) return 0.0f;
  const float c7 = 1.52527338e-05f, c6 = 1.54035304e-04f, c5 = 1.33335581e-03f,
              c4 = 9.61812911e-03f, c3 = 5.55041087e-02f, c2 = 2.40226507e-01f,
              c1 = 6.93147181e-01f, c0 = 1.0f;
  float p = c7;
  p = fmaf(p, f, c6);
  p = fmaf(p, f, c5);
  p = fmaf(p, f, c4);
  p = fmaf(p, f, c3);
  p = fmaf(p, f, c2);
  p = fmaf(p, f, c1);
  p = fmaf(p, f, c0);
  return ldexpf(p, (int)n);
}

static inline uint64_t mass_of(float e) { return (uint64_t)rintf(e * 4294967296.0f); }

/* ------------------------------------------------------------------ */
/* n-gram proposer: restates BatchGenerator.swift:982-1010              */
/* ------------------------------------------------------------------ */
int or_ngram_propose(const int32_t* ctx, int n, int max_suffix, int min_context, int limit,
                     int32_t* out) {
  if (n < min_context || limit <= 0) return 0;                 /* :983 */
  int max_len = max_suffix < n - 1 ? max_suffix : n - 1;       /* :987-990 */
  if (max_len <= 0) return 0;                                  /* :991 */
  for (int L = max_len; L >= 1; --L) {                         /* :993 */
    int suffix_start = n - L;                                  /* :994 */
    if (suffix_start <= 0) continue;                           /* :996 */
    for (int c = suffix_start - 1; c >= 0; --c) {              /* :998 */
      int cend = c + L;                                        /* :999 */
      if (cend > suffix_start) continue;                       /* :1000 */
      if (memcmp(ctx + c, ctx + suffix_start, (size_t)L * sizeof(int32_t)) == 0) {  /* :1001 */
        int ps = cend;                                         /* :1002 */
        int pe = n < ps + limit ? n : ps + limit;              /* :1003 */
        if (ps >= pe) continue;                                /* :1004 */
        for (int i = ps; i < pe; ++i) out[i - ps] = ctx[i];
        return pe - ps;                                        /* :1005 */
      }
    }
  }
  return 0;                                                    /* :1009 */
}

/* ------------------------------------------------------------------ */
/* acceptance building blocks                                           */
/* ------------------------------------------------------------------ */
int or_argmax_bf16(const uint16_t* logits, int V) {
  int best = 0;
  float bv = bf(logits[0]);
  for (int i = 1; i < V; ++i) {
    float v = bf(logits[i]);
    if (v > bv) { bv = v; best = i; }
  }
  return best;
}

static inline float canon(uint16_t h) {  /* -0 -> +0 */
  float v = bf(h);
  return v == 0.0f ? 0.0f : v;
}

static int is_eos_tok(const or_sampling* sp, int tok) {
  for (int i = 0; i < sp->n_eos; ++i)
    if (sp->eos[i] == tok) return 1;
  return 0;
}

static int penalties_on(const or_sampling* sp) {
  const float rp = sp->repetition_penalty == 0.0f ? 1.0f : sp->repetition_penalty;
  return rp != 1.0f || sp->presence_penalty != 0.0f || sp->frequency_penalty != 0.0f;
}

int or_process_logits(const uint16_t* lg, int V, const or_sampling* sp, const int32_t* gen, int n_gen,
                      float* out) {
  for (int i = 0; i < V; ++i) out[i] = canon(lg[i]);
  int applied = 0;
  /* applyLogitBias, Sampling.swift:695-704: ids outside [0, V) are ignored */
  for (int k = 0; k < sp->n_bias; ++k) {
    const int t = sp->bias_token[k];
    if (t >= 0 && t < V) { out[t] = out[t] + sp->bias_value[k]; applied = 1; }
  }
  /* shouldApplyMinTokens + maskTokens, :677-684 and :648-650 */
  if (sp->min_tokens > 0 && n_gen < sp->min_tokens && sp->n_eos > 0) {
    for (int k = 0; k < sp->n_eos; ++k)
      if (sp->eos[k] >= 0 && sp->eos[k] < V) out[sp->eos[k]] = -INFINITY;
    applied = 1;
  }
  /* applyPenalties, :592-636 (nothing to do without generated tokens, :597) */
  if (penalties_on(sp) && n_gen > 0) {
    const float rp = sp->repetition_penalty == 0.0f ? 1.0f : sp->repetition_penalty;
    int32_t* cnt = (int32_t*)calloc((size_t)V, sizeof(int32_t));
    for (int i = 0; i < n_gen; ++i)
      if (gen[i] >= 0 && gen[i] < V) cnt[gen[i]]++;
    for (int t = 0; t < V; ++t) {
      if (!cnt[t]) continue;
      float v = out[t];
      if (rp != 1.0f) v = v < 0.0f ? v * rp : v / rp;
      if (sp->presence_penalty != 0.0f) v = v - sp->presence_penalty;
      if (sp->frequency_penalty != 0.0f) v = v - (float)cnt[t] * sp->frequency_penalty;
      out[t] = v;
    }
    free(cnt);
    applied = 1;
  }
  for (int i = 0; i < V; ++i)
    if (out[i] == 0.0f) out[i] = 0.0f; /* -0 -> +0 */
  return applied;
}

float or_min_p_log(float min_p) { return min_p > 0.0f ? logf(min_p) : -INFINITY; }

static int argmax_f(const float* v, int V) {
  int best = 0;
  for (int i = 1; i < V; ++i)
    if (v[i] > v[best]) best = i;
  return best;
}

typedef struct { float v; uint64_t w; int i; } vw_t;
static int cmp_desc(const void* a, const void* b) {  /* value descending, index ascending */
  const vw_t* x = (const vw_t*)a;
  const vw_t* y = (const vw_t*)b;
  if (x->v != y->v) return x->v < y->v ? 1 : -1;
  return x->i < y->i ? -1 : (x->i > y->i ? 1 : 0);
}

static inline int kept(const or_dist* d, float v, int i) {
  if (d->filtered && v < d->tau) return 0;
  if (!(v - d->max_logit >= d->min_p_log)) return 0;
  if (v < d->topk_value || (v == d->topk_value && i > d->topk_index)) return 0;
  return 1;
}

void or_dist_build_f(const float* v, int V, float temperature, float top_p, int top_k, float min_p_log,
                     or_dist* d) {
  float m = -INFINITY;
  for (int i = 0; i < V; ++i) if (v[i] > m) m = v[i];
  d->max_logit = m;
  d->filtered = (top_p > 0.0f && top_p < 1.0f);
  d->tau = -INFINITY;
  d->min_p_log = min_p_log;
  d->topk_value = -INFINITY;
  d->topk_index = 0x7FFFFFFF;
  const int use_k = top_k > 0 && top_k < V;
  if (d->filtered || use_k) {
    vw_t* a = (vw_t*)malloc(sizeof(vw_t) * (size_t)V);
    uint64_t total1 = 0;
    for (int i = 0; i < V; ++i) {
      a[i].v = v[i];
      a[i].i = i;
      a[i].w = mass_of(or_exp_neg(v[i] - m));
      total1 += a[i].w;
    }
    qsort(a, (size_t)V, sizeof(vw_t), cmp_desc);
    if (d->filtered) {
      /* Sampling.swift:847-858: drop sorted positions whose mass strictly above is
       * >= topP * total; keep every token whose value is >= the first kept value. */
      double X = (double)top_p * (double)total1;
      uint64_t above = 0;
      int i = 0;
      while (i < V) {
        float x = a[i].v;
        if (!((double)above < X)) break;
        d->tau = x;
        while (i < V && a[i].v == x) { above += a[i].w; ++i; }
      }
    }
    if (use_k) {  /* Sampling.swift:893-906 */
      d->topk_value = a[top_k - 1].v;
      d->topk_index = a[top_k - 1].i;
    }
    free(a);
  }
  float inv_t = 1.0f / temperature;
  uint64_t tot = 0;
  for (int i = 0; i < V; ++i)
    if (kept(d, v[i], i)) tot += mass_of(or_exp_neg((v[i] - m) * inv_t));
  d->total = tot;
}

uint64_t or_dist_mass_f(const or_dist* d, const float* v, float inv_temp, int token) {
  if (!kept(d, v[token], token)) return 0;
  return mass_of(or_exp_neg((v[token] - d->max_logit) * inv_temp));
}

int or_dist_sample_f(const or_dist* d, const float* v, int V, float inv_temp, uint32_t u, int exclude) {
  uint64_t total = d->total;
  if (exclude >= 0) total -= or_dist_mass_f(d, v, inv_temp, exclude);
  unsigned __int128 prod = (unsigned __int128)u * (unsigned __int128)total;
  uint64_t R = (uint64_t)(prod >> 32);
  uint64_t c = 0;
  int last = -1;
  for (int i = 0; i < V; ++i) {
    if (i == exclude) continue;
    uint64_t w = or_dist_mass_f(d, v, inv_temp, i);
    if (w == 0) continue;
    last = i;
    if (c + w > R) return i;
    c += w;
  }
  return last < 0 ? 0 : last; /* last < 0 only when nothing has mass */
}

static float* canon_row(const uint16_t* logits, int V) {
  float* v = (float*)malloc(sizeof(float) * (size_t)V);
  for (int i = 0; i < V; ++i) v[i] = canon(logits[i]);
  return v;
}

void or_dist_build(const uint16_t* logits, int V, float temperature, float top_p, or_dist* d) {
  float* v = canon_row(logits, V);
  or_dist_build_f(v, V, temperature, top_p, 0, -INFINITY, d);
  free(v);
}

uint64_t or_dist_mass(const or_dist* d, const uint16_t* logits, float inv_temp, int token) {
  const float x = canon(logits[token]);
  if (!kept(d, x, token)) return 0;
  return mass_of(or_exp_neg((x - d->max_logit) * inv_temp));
}

int or_dist_sample(const or_dist* d, const uint16_t* logits, int V, float inv_temp, uint32_t u, int exclude) {
  float* v = canon_row(logits, V);
  const int t = or_dist_sample_f(d, v, V, inv_temp, u, exclude);
  free(v);
  return t;
}

static int accept_draft(const or_dist* d, const float* v, float inv_temp, int x, uint32_t u) {
  uint64_t w = or_dist_mass_f(d, v, inv_temp, x);
  unsigned __int128 lhs = (unsigned __int128)u * (unsigned __int128)d->total;
  unsigned __int128 rhs = (unsigned __int128)w << 32;
  return lhs < rhs;
}

/* ------------------------------------------------------------------ */
/* acceptance of one row's verify block                                 */
/* ------------------------------------------------------------------ */
/* the values position j samples from: generated tokens so far = gen + dr[0 .. j) */
static void position_values(const uint16_t* lg, int V, const or_sampling* sp, const int32_t* gen, int n_gen,
                            const int32_t* dr, int j, int32_t* scratch, float* out) {
  if (n_gen > 0) memcpy(scratch, gen, sizeof(int32_t) * (size_t)n_gen);
  if (j > 0) memcpy(scratch + n_gen, dr, sizeof(int32_t) * (size_t)j);
  or_process_logits(lg, V, sp, scratch, n_gen + j, out);
}

static uint32_t draw(const uint32_t* uniforms, uint64_t seed, uint64_t counter, int pos, int kind) {
  return uniforms ? uniforms[2 * pos + kind] : or_uniform_u32(seed, counter, (uint32_t)pos, (uint32_t)kind);
}

int or_accept_row(const uint16_t* lg, int V, const int32_t* dr, int P, const or_sampling* sp,
                  const int32_t* gen, int n_gen, uint64_t seed, uint64_t counter, const uint32_t* uniforms,
                  int acceptance, int forced_cap, int has_ext, int32_t* out, int* kv_keep, int* n_acc,
                  int* rejected) {
  const int sampled = sp->temperature != 0.0f;
  const float inv_t = sampled ? 1.0f / sp->temperature : 0.0f;
  const float lmp = or_min_p_log(sp->min_p);
  float* v = (float*)malloc(sizeof(float) * (size_t)V);
  int32_t* gbuf = (int32_t*)malloc(sizeof(int32_t) * (size_t)(n_gen + P + 1));
  int n_emit = 0;
  *kv_keep = 1;
  *n_acc = 0;
  *rejected = 0;
#define VALUES(pos) position_values(lg + (size_t)(pos) * V, V, sp, gen, n_gen, dr, (pos), gbuf, v)
  if (!sampled && acceptance == OR_ACCEPT_ALL_OR_NOTHING) {
    /* BatchGenerator.swift:906-947 */
    if (P == 0) {                                                  /* plain decodeOneToken */
      VALUES(0);
      out[0] = argmax_f(v, V);
      free(v); free(gbuf);
      return 1;
    }
    int all = 1, na = 0;
    for (int pos = 0; pos <= P; ++pos) {
      VALUES(pos);   /* generatedHistory grows by the accepted tokens, :930; they equal the drafts */
      const int s = argmax_f(v, V);
      if (sp->reject_token >= 0 && s == sp->reject_token) { all = 0; break; }  /* :920-923 */
      if (pos < P && s != dr[pos]) { all = 0; break; }                         /* :925-928 */
      out[na++] = s;
      if (is_eos_tok(sp, s)) break;                                            /* :932-934 */
    }
    if (!all) {
      *rejected = 1;                                               /* :938 */
      /* :939 decodeOneToken on the original cache: the same logits as position 0 */
      VALUES(0);
      out[0] = argmax_f(v, V);
      free(v); free(gbuf);
      return 1;
    }
    *kv_keep = P + 1;                                              /* :942 adopt the working cache */
    *n_acc = na > 1 ? na - 1 : 0;                                  /* :952 */
    free(v); free(gbuf);
    return na;
  }
  if (forced_cap >= 0) {
    /* forced accept-length schedule (stress workloads): exactly min(forced_cap, P) drafts
     * count as accepted whatever the model says (up to an EOS or reject token among them),
     * then the history's continuation token after them (dr[a]: the next draft, or when all
     * P were accepted the extension dr[P] if has_ext), else the model's token at the next
     * position, drawn without exclusion */
    int a = forced_cap < P ? forced_cap : P, stop = 0;
    for (int pos = 0; pos < a; ++pos) {
      out[n_emit++] = dr[pos];
      if (dr[pos] == sp->reject_token || is_eos_tok(sp, dr[pos])) { a = pos + 1; stop = 1; break; }
    }
    if (!stop && (a < P || (P > 0 && has_ext))) {
      out[n_emit++] = dr[a];
      stop = 1;
    }
    if (!stop) {
      VALUES(a);
      if (sampled) {
        or_dist d;
        or_dist_build_f(v, V, sp->temperature, sp->top_p, sp->top_k, lmp, &d);
        out[n_emit++] = or_dist_sample_f(&d, v, V, inv_t, draw(uniforms, seed, counter, a, 1), -1);
      } else {
        out[n_emit++] = argmax_f(v, V);
      }
    }
    *kv_keep = a + 1;
    *n_acc = a;
    *rejected = (P > 0 && a < P) ? 1 : 0;
    free(v);
    free(gbuf);
    return n_emit;
  }
  /* prefix acceptance (greedy) and speculative sampling (temperature > 0): accept drafts
   * while they agree, emit the correction (or the bonus token after a full accept), keep
   * the current token + accepted drafts in the KV. */
  int a = 0, stop = 0;
  for (int pos = 0; pos < P; ++pos) {
    VALUES(pos);
    int tok;
    if (!sampled) {
      tok = argmax_f(v, V);
      if (tok != dr[pos] || tok == sp->reject_token) {
        out[n_emit++] = tok;
        stop = 1;
        break;
      }
    } else {
      or_dist d;
      or_dist_build_f(v, V, sp->temperature, sp->top_p, sp->top_k, lmp, &d);
      const int ok = accept_draft(&d, v, inv_t, dr[pos], draw(uniforms, seed, counter, pos, 0));
      if (!ok) {
        out[n_emit++] = or_dist_sample_f(&d, v, V, inv_t, draw(uniforms, seed, counter, pos, 1), dr[pos]);
        stop = 1;
        break;
      }
      tok = dr[pos];
    }
    out[n_emit++] = tok;
    a++;
    if (tok == sp->reject_token || is_eos_tok(sp, tok)) { stop = 1; break; }
  }
  if (!stop) {
    VALUES(P);
    if (sampled) {
      or_dist d;
      or_dist_build_f(v, V, sp->temperature, sp->top_p, sp->top_k, lmp, &d);
      out[n_emit++] = or_dist_sample_f(&d, v, V, inv_t, draw(uniforms, seed, counter, P, 1), -1);
    } else {
      out[n_emit++] = argmax_f(v, V);
    }
  }
#undef VALUES
  *kv_keep = a + 1;
  *n_acc = a;
  *rejected = (P > 0 && a < P) ? 1 : 0;
  free(v);
  free(gbuf);
  return n_emit;
}

/* ------------------------------------------------------------------ */
/* KV trim known answer: BatchCache.swift:403-424                       */
/* ------------------------------------------------------------------ */
int or_batch_trim(int* idx, int B, int32_t* lp, int32_t* off, int n) {
  int trimmed = *idx < n ? *idx : n;                                       /* :406 */
  if (trimmed <= 0) return 0;                                              /* :407 */
  int cur = *idx;
  int* row_tr = (int*)malloc(sizeof(int) * (size_t)(B > 0 ? B : 1));
  for (int r = 0; r < B; ++r) {                                            /* :412-414 */
    int avail = cur - lp[r];
    if (avail < 0) avail = 0;
    row_tr[r] = trimmed < avail ? trimmed : avail;
  }
  *idx -= trimmed;                                                         /* :416 */
  for (int r = 0; r < B; ++r) {
    int rem = cur - lp[r] - row_tr[r];                                     /* :418 */
    if (rem < 0) rem = 0;
    lp[r] = *idx - rem;                                                    /* :419 */
    off[r] -= row_tr[r];                                                   /* :422 */
  }
  free(row_tr);
  return trimmed;
}

/* ------------------------------------------------------------------ */
/* generator + scheduler restatement                                    */
/* ------------------------------------------------------------------ */
typedef struct or_row {
  int active;
  int32_t* hist;      /* speculativeTokenHistory: prompt + generated (incl. pending current) */
  int hist_len;
  int generated;      /* generatedTokenHistory.count */
  int max_tokens;
  int cur;            /* currentTokens[row], not yet in the KV */
  or_sampling sp;
  uint64_t seed;
  uint64_t counter;   /* per-row draw counter */
} or_row;

struct or_generator {
  or_model* m;
  or_spec_config cfg;
  int max_rows, max_hist;
  or_row* rows;
  or_stats stats;
  uint64_t global_seed;
  uint64_t unseeded_count;
  int32_t* widths;
  int n_widths, cap_widths;
};

or_generator* or_generator_create(or_model* m, const or_spec_config* cfg, int max_rows,
                                  int max_hist, uint64_t global_seed) {
  or_generator* g = (or_generator*)calloc(1, sizeof(or_generator));
  g->m = m;
  g->cfg = *cfg;
  /* SpeculativeDecodingConfiguration clamps, BatchGenerator.swift:23-25 */
  if (g->cfg.max_proposal_tokens < 0) g->cfg.max_proposal_tokens = 0;
  if (g->cfg.max_suffix_tokens < 1) g->cfg.max_suffix_tokens = 1;
  if (g->cfg.min_context_tokens < 2) g->cfg.min_context_tokens = 2;
  g->max_rows = max_rows;
  g->max_hist = max_hist;
  g->global_seed = global_seed;
  g->rows = (or_row*)calloc((size_t)max_rows, sizeof(or_row));
  for (int r = 0; r < max_rows; ++r) g->rows[r].hist = (int32_t*)malloc(sizeof(int32_t) * (size_t)max_hist);
  g->cap_widths = 4096;
  g->widths = (int32_t*)malloc(sizeof(int32_t) * (size_t)g->cap_widths);
  return g;
}

void or_generator_destroy(or_generator* g) {
  if (!g) return;
  for (int r = 0; r < g->max_rows; ++r) free(g->rows[r].hist);
  free(g->rows);
  free(g->widths);
  free(g);
}

static void record_width(or_generator* g, int w) {
  if (g->n_widths < g->cap_widths) g->widths[g->n_widths++] = w;
}

static int is_eos(const or_sampling* sp, int tok) {
  for (int i = 0; i < sp->n_eos; ++i)
    if (sp->eos[i] == tok) return 1;
  return 0;
}

/* the generated tokens of a row (generatedTokenHistory): the last `generated` entries of
 * its history */
static const int32_t* generated_of(const or_row* rw, int* n) {
  *n = rw->generated < rw->hist_len ? rw->generated : rw->hist_len;
  return rw->hist + (rw->hist_len - *n);
}

static int finish_of(const or_row* rw, int tok) {   /* Scheduler.swift:1215-1227 */
  if (is_eos(&rw->sp, tok)) return 1;
  if (rw->generated >= rw->max_tokens) return 2;
  return 0;
}

int or_generator_insert(or_generator* g, int row, const int32_t* prompt, int n_prompt,
                        int max_tokens, const or_sampling* sp, int* finished) {
  if (row < 0 || row >= g->max_rows || n_prompt < 1 || n_prompt + 2 > g->max_hist) return -1;
  or_row* rw = &g->rows[row];
  const int V = or_model_cfg(g->m)->vocab;
  or_kv_set_len(g->m, row, 0);
  /* prefill all but the last prompt token, then the last one alone (Scheduler.swift:722-739) */
  if (n_prompt > 1) {
    int cnt = n_prompt - 1;
    if (or_forward(g->m, 1, &row, &cnt, prompt, NULL)) return -2;
  }
  uint16_t* lg = (uint16_t*)malloc(2 * (size_t)V);
  int one = 1;
  if (or_kv_len(g->m, row) > 0) record_width(g, 1);
  if (or_forward(g->m, 1, &row, &one, prompt + n_prompt - 1, lg)) { free(lg); return -2; }
  rw->sp = *sp;
  rw->seed = sp->has_seed ? sp->seed : or_mix64(g->global_seed ^ or_mix64(++g->unseeded_count));
  rw->counter = 0;
  int tok, keep, nacc, rej;
  or_accept_row(lg, V, NULL, 0, sp, NULL, 0, rw->seed, rw->counter, NULL, g->cfg.acceptance, -1, 0, &tok, &keep, &nacc,
                &rej);
  rw->counter++;
  free(lg);
  rw->generated = 1;
  rw->max_tokens = max_tokens;
  memcpy(rw->hist, prompt, sizeof(int32_t) * (size_t)n_prompt);
  rw->hist[n_prompt] = tok;
  rw->hist_len = n_prompt + 1;
  rw->cur = tok;
  int fin = finish_of(rw, tok);
  if (finished) *finished = fin;
  rw->active = fin == 0;
  return tok;
}

int or_generator_insert_prefilled(or_generator* g, int row, const int32_t* ctx, int n_ctx,
                                  int max_tokens, const or_sampling* sp) {
  if (row < 0 || row >= g->max_rows || n_ctx < 1 || n_ctx > g->max_hist) return -1;
  if (or_kv_len(g->m, row) != n_ctx - 1) return -3;
  or_row* rw = &g->rows[row];
  rw->sp = *sp;
  rw->seed = sp->has_seed ? sp->seed : or_mix64(g->global_seed ^ or_mix64(++g->unseeded_count));
  rw->counter = 0;
  rw->generated = 1;
  rw->max_tokens = max_tokens;
  memcpy(rw->hist, ctx, sizeof(int32_t) * (size_t)n_ctx);
  rw->hist_len = n_ctx;
  rw->cur = ctx[n_ctx - 1];
  rw->active = 1;
  return 0;
}

void or_generator_remove(or_generator* g, int row) {
  if (row >= 0 && row < g->max_rows) g->rows[row].active = 0;
}

/* canSpeculate, BatchGenerator.swift:957-975, generalised to many rows */
static int can_speculate(const or_generator* g, const or_row* rw, int n_active) {
  if (!g->cfg.enabled || g->cfg.max_proposal_tokens <= 0) return 0;
  if (g->cfg.single_row_only && n_active != 1) return 0;
  if (rw->hist_len < g->cfg.min_context_tokens) return 0;
  if (g->cfg.greedy_only && (rw->sp.temperature != 0.0f || rw->sp.has_seed)) return 0;
  return 1;
}

int or_generator_step(or_generator* g, int32_t* out_tokens, int32_t* out_counts,
                      int32_t* out_finish, const int32_t* forced_accept) {
  const int K = g->cfg.max_proposal_tokens, V = or_model_cfg(g->m)->vocab, R = g->max_rows;
  int n_active = 0;
  for (int r = 0; r < R; ++r) n_active += g->rows[r].active;
  for (int r = 0; r < R; ++r) { out_counts[r] = 0; out_finish[r] = 0; }
  if (n_active == 0) return 0;
  int32_t* rows = (int32_t*)malloc(sizeof(int32_t) * (size_t)R);
  int32_t* counts = (int32_t*)malloc(sizeof(int32_t) * (size_t)R);
  int32_t* drafts = (int32_t*)malloc(sizeof(int32_t) * (size_t)R * (size_t)(K + 2));
  int32_t* nprop = (int32_t*)calloc((size_t)R, sizeof(int32_t));
  int* ext = (int*)calloc((size_t)R, sizeof(int));
  int32_t* toks = (int32_t*)malloc(sizeof(int32_t) * (size_t)R * (size_t)(K + 1));
  int nr = 0, M = 0;
  for (int r = 0; r < R; ++r) {
    or_row* rw = &g->rows[r];
    if (!rw->active) continue;
    int P = 0;
    if (can_speculate(g, rw, n_active)) {
      int remaining = rw->max_tokens - rw->generated;                        /* :977-980 */
      if (remaining < 0) remaining = 0;
      if (remaining > 1) {                                                   /* :878 */
        int limit = K < remaining - 1 ? K : remaining - 1;                   /* :883 */
        if (limit > 0) {  /* one more token: the continuation after the drafts (forced schedule) */
          P = or_ngram_propose(rw->hist, rw->hist_len, g->cfg.max_suffix_tokens,
                               g->cfg.min_context_tokens, limit + 1, drafts + (size_t)r * (K + 2));
          ext[r] = P > limit;
          if (P > limit) P = limit;
        }
      }
    }
    nprop[r] = P;
    if (P > 0) { g->stats.proposal_batches++; g->stats.proposed += P; }     /* :894-895 */
    rows[nr] = r;
    counts[nr] = P + 1;
    toks[M] = rw->cur;                                                       /* :897 */
    for (int j = 0; j < P; ++j) toks[M + 1 + j] = drafts[(size_t)r * (K + 2) + j];
    if (or_kv_len(g->m, r) > 0) record_width(g, P + 1);
    M += P + 1;
    nr++;
  }
  uint16_t* lg = (uint16_t*)malloc(2 * (size_t)M * (size_t)V);
  if (or_forward(g->m, nr, rows, counts, toks, lg)) {
    free(rows); free(counts); free(drafts); free(nprop); free(ext); free(toks); free(lg);
    return -1;
  }
  int produced = 0;
  for (int i = 0, t0 = 0; i < nr; t0 += counts[i], ++i) {
    const int r = rows[i], P = nprop[r];
    or_row* rw = &g->rows[r];
    int32_t* out = out_tokens + (size_t)r * (K + 1);
    int kv_keep = 1, n_acc = 0, rejected = 0, n_gen = 0;
    const int32_t* gen = generated_of(rw, &n_gen);
    const int n_emit = or_accept_row(lg + (size_t)t0 * V, V, drafts + (size_t)r * (K + 2), P, &rw->sp, gen, n_gen,
                                     rw->seed, rw->counter, NULL, g->cfg.acceptance,
                                     forced_accept ? forced_accept[r] : -1, ext[r], out, &kv_keep, &n_acc,
                                     &rejected);
    if (P > 0) {
      g->stats.accepted += n_acc;                                     /* :952 */
      g->stats.rejected_batches += rejected;                          /* :938 */
    }
    rw->counter++;
    /* rollback: drop verified positions beyond what is kept (O(1): length only) */
    or_kv_set_len(g->m, r, or_kv_len(g->m, r) - (P + 1 - kv_keep));
    int fin = 0, emitted = 0;
    for (int z = 0; z < n_emit; ++z) {
      const int tok = out[z];
      if (rw->hist_len < g->max_hist) rw->hist[rw->hist_len++] = tok;    /* :1012-1014 */
      rw->generated++;
      emitted++;
      fin = finish_of(rw, tok);                                           /* Scheduler.swift:381-387 */
      if (fin) break;
    }
    rw->cur = out[n_emit - 1];
    out_counts[r] = emitted;
    out_finish[r] = fin;
    if (fin) rw->active = 0;                                              /* Scheduler.swift:413-427 */
    produced++;
  }
  free(rows); free(counts); free(drafts); free(nprop); free(ext); free(toks); free(lg);
  return produced;
}

void or_generator_stats(or_generator* g, or_stats* out) { *out = g->stats; }

int or_generator_call_widths(or_generator* g, int32_t* out, int cap) {
  int n = g->n_widths < cap ? g->n_widths : cap;
  memcpy(out, g->widths, sizeof(int32_t) * (size_t)n);
  return g->n_widths;
}

int or_generator_active(or_generator* g, int row) { return g->rows[row].active; }

int or_generator_history(or_generator* g, int row, int32_t* out, int cap) {
  const or_row* rw = &g->rows[row];
  int n = rw->hist_len < cap ? rw->hist_len : cap;
  memcpy(out, rw->hist, sizeof(int32_t) * (size_t)n);
  return rw->hist_len;
}
