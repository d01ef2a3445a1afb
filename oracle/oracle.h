/*
 * oracle.h -- CPU restatement of mlxcat's n-gram speculative-decode step.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the parity checker for the HIP
 * product in mlxcat_amd/ and the CPU baseline timed beside it.  Only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it; the
 * product path never links, imports or falls back to it.
 *
 * What it restates (reference = local-ai-cat/mlxcat, paths relative to its root):
 *   - n-gram proposer      Sources/MLXCat/TrackB/BatchGenerator.swift:982-1010
 *   - speculative step     Sources/MLXCat/TrackB/BatchGenerator.swift:875-955
 *     (all-or-nothing acceptance, reject -> one-token decode, EOS break,
 *      tool-trigger reject, stats at :894-895,938,952)
 *   - step gate            BatchGenerator.swift:957-980
 *   - finish reasons       Sources/MLXCat/TrackB/Scheduler.swift:372-401,1215-1227
 *   - sampler              Sources/MLXCat/TrackB/Sampling.swift:483-528,592-652,847-906
 *     (logit bias, minTokens EOS mask, repetition / presence / frequency penalties,
 *      top-p, min-p, top-k, temperature)
 *   - KV trim              Sources/MLXCat/TrackB/BatchCache.swift:403-424
 *   - 4-bit affine g64 group cost  Sources/MLXCat/TrackB/KVQuantizationPolicy.swift:12-14
 * Beyond the reference (it speculates only at width 1, greedy): batched
 * prefix acceptance with per-row KV rollback, and textbook speculative
 * sampling (Leviathan et al. 2023, arXiv:2211.17192) with a one-hot n-gram
 * draft, evaluated with integer probability masses so that the CPU and GPU
 * decisions are bit-identical given the same logits and uniforms.
 *
 * The decoder forward (Qwen3 / Llama / Qwen3-MoE wiring) follows the public
 * mlx-lm model definitions, which live outside the reference tree
 * (mlx-swift-lm @ dcfa3aa1, Package.swift:61-78): its rounding is "parity
 * unpinned" and is checked against the HIP path only within the bf16
 * tolerance 2e-2 abs / 1e-2 rel.
 */
#ifndef MLXCAT_ORACLE_H
#define MLXCAT_ORACLE_H
#include <stdint.h>
#include <stddef.h>
#ifdef __cplusplus
extern "C" {
#endif

/* ---- deterministic integer generators (shared definition with the HIP side) ---- */
uint64_t or_mix64(uint64_t z);
/* 32-bit uniform for (seed, step counter, position, kind): kind 0 = accept test, 1 = sample draw */
uint32_t or_uniform_u32(uint64_t seed, uint64_t counter, uint32_t pos, uint32_t kind);

/* bf16 helpers (round to nearest even) */
uint16_t or_f32_to_bf16(float f);
float or_bf16_to_f32(uint16_t h);

/* Synthetic MLX-format 4-bit affine g64 tensor: wq[N][K/8] u32 (element j of a
 * word at bits 4j), scales/biases [N][K/64] bf16.  The nibble is Binomial(15,1/2)
 * (popcount of 15 hash bits) and the scale is ~0.0107, so w = s*q + b has mean ~0
 * and std ~0.02.  `scale_exp` selects the scale's binade: 2^scale_exp (default -7). */
void or_gen_linear(uint64_t seed, uint64_t tensor_id, int N, int K, int scale_exp,
                   uint32_t* wq, uint16_t* scales, uint16_t* biases);
/* RMSNorm weights: bf16 1 + (h%32 - 16)/128, exact in bf16 */
void or_gen_norm(uint64_t seed, uint64_t tensor_id, int n, uint16_t* w);

/* tensor ids used by the synthetic generator */
enum {
  OR_T_Q = 0, OR_T_K = 1, OR_T_V = 2, OR_T_O = 3, OR_T_GATE = 4, OR_T_UP = 5, OR_T_DOWN = 6,
  OR_T_IN_NORM = 7, OR_T_POST_NORM = 8, OR_T_Q_NORM = 9, OR_T_K_NORM = 10, OR_T_ROUTER = 11,
};
uint64_t or_tensor_id(int layer, int which);          /* layer >= 0 */
uint64_t or_expert_tensor_id(int layer, int expert, int which); /* which in GATE/UP/DOWN */
#define OR_TID_EMBED 0xE0000001ull
#define OR_TID_LM_HEAD 0xE0000002ull
#define OR_TID_FINAL_NORM 0xE0000003ull

/* exp(x) for x <= 0 with a fixed operation sequence (rint range reduction to
 * 2^f, f in [-1/2,1/2], degree-7 Taylor polynomial of 2^f in Horner form with
 * fused multiply-adds, exact ldexp).  Identical bits on CPU and GPU. */
float or_exp_neg(float x);

/* ---- n-gram proposer: BatchGenerator.swift:982-1010 ---- */
/* Returns the proposal length (0 = nil) and writes up to `limit` tokens. */
int or_ngram_propose(const int32_t* ctx, int n, int max_suffix, int min_context, int limit,
                     int32_t* out);

/* ---- acceptance building blocks ---- */
/* argmax over bf16 logits, lowest index wins ties (MLX argMax convention) */
int or_argmax_bf16(const uint16_t* logits, int V);
/* Integer-mass sampling state of one position's values (the fp32 logits after the
 * processors and penalties of or_process_logits).  Filters, in the order of
 * Sampling.swift:500-522: top-p in (0,1) with :847-858 semantics on T=1 masses, min-p
 * (:860-863: keep v - max >= log(min_p)), top-k (:893-906: the k largest values, the
 * lowest indices first among equal values); the temperature then scales the kept values.
 * Masses are round(exp(.) * 2^32) as uint64. */
typedef struct or_dist {
  uint64_t total;     /* sum of kept temperature masses */
  float max_logit;
  float tau;          /* smallest kept value under top-p */
  int filtered;       /* 1 if top-p was applied */
  float min_p_log;    /* log(min_p); -inf when min-p is off */
  float topk_value;   /* the k-th largest value; -inf when top-k is off */
  int32_t topk_index; /* among values equal to topk_value, larger indices are dropped */
} or_dist;
struct or_sampling;
void or_dist_build_f(const float* v, int V, float temperature, float top_p, int top_k, float min_p_log,
                     or_dist* d);
uint64_t or_dist_mass_f(const or_dist* d, const float* v, float inv_temp, int token);
/* sample with 32-bit uniform u from the kept distribution, excluding `exclude` (-1: none) */
int or_dist_sample_f(const or_dist* d, const float* v, int V, float inv_temp, uint32_t u, int exclude);
/* the same over bf16 logits with top-p only */
void or_dist_build(const uint16_t* logits, int V, float temperature, float top_p, or_dist* d);
uint64_t or_dist_mass(const or_dist* d, const uint16_t* logits, float inv_temp, int token);
int or_dist_sample(const or_dist* d, const uint16_t* logits, int V, float inv_temp, uint32_t u,
                   int exclude);
/* log(min_p) as the sampler uses it (-inf for min_p <= 0); computed once per request */
float or_min_p_log(float min_p);

/* Values one position samples from: the bf16 logits in fp32 after the logits processors
 * (Sampling.swift:638-652: logit bias added in fp32 at its valid token ids, EOS ids set to
 * -inf while fewer than min_tokens tokens were generated) and the penalties over the
 * generated tokens (:592-636: repetition v < 0 ? v * rp : v / rp, then presence - pp, then
 * frequency - count * fp, at each distinct generated token).  gen holds the n_gen generated
 * tokens so far (the request's, then the drafts accepted before this position).  Returns 1
 * when any processor or penalty applied, 0 when out[] is the plain logits. */
int or_process_logits(const uint16_t* lg, int V, const struct or_sampling* sp, const int32_t* gen, int n_gen,
                      float* out);

/* Acceptance of one row's verify block: lg holds P+1 logits rows (position j scores
 * the token after verify token j), dr the P drafts, gen the n_gen tokens the request has
 * generated so far (penalties, min_tokens).  Greedy rows (temperature 0) use
 * `acceptance` (OR_ACCEPT_ALL_OR_NOTHING restates BatchGenerator.swift:906-947, where a
 * rejection falls back to a one-token decode whose logits are position 0); rows with
 * temperature > 0 use speculative sampling with the uniforms of (seed, counter), or the
 * caller's: uniforms[j][0] the accept test and uniforms[j][1] the sample draw of position
 * j (NULL = derived).  forced_cap >= 0 (a forced accept-length schedule, stress workloads)
 * accepts exactly min(forced_cap, P) drafts whatever the model says, up to an EOS or reject
 * token among them, then emits the history's continuation token after them: the next draft,
 * or dr[P] when all were accepted and has_ext says the history holds one, else the model's
 * token at that position (sampled rows draw it without exclusion); -1 = none.  A row that
 * keeps copying its history keeps proposing, so the schedule sets the accepted lengths
 * whatever the weights.  Writes the emitted tokens to out and returns their count;
 * *kv_keep = verified positions kept in the KV, *n_acc = drafts accepted (the
 * SpeculativeDecodingStats increment, :952), *rejected = 1 when a proposal was (partly)
 * rejected (:938). */
int or_accept_row(const uint16_t* lg, int V, const int32_t* dr, int P, const struct or_sampling* sp,
                  const int32_t* gen, int n_gen, uint64_t seed, uint64_t counter, const uint32_t* uniforms,
                  int acceptance, int forced_cap, int has_ext, int32_t* out, int* kv_keep, int* n_acc,
                  int* rejected);

/* ---- KV trim known answer: BatchCache.swift:403-424 ---- */
/* Uniform trim of a left-padded batch: returns trimmed count, updates idx,
 * left_padding[] and offsets[] in place. */
int or_batch_trim(int* idx, int B, int32_t* left_padding, int32_t* offsets, int n);

/* ---- decoder model ---- */
enum { OR_ARCH_QWEN3 = 0, OR_ARCH_LLAMA = 1, OR_ARCH_QWEN3_MOE = 2,
       OR_ARCH_FAKE_REPEATING = 100, OR_ARCH_FAKE_MISMATCHING = 101 };

typedef struct or_config {
  int arch;
  int n_layers, hidden, n_q_heads, n_kv_heads, head_dim, intermediate, vocab;
  int tied_embeddings;
  float rms_eps, rope_theta;
  int n_experts, n_experts_per_tok, moe_intermediate;
} or_config;

typedef struct or_model or_model;
or_model* or_model_create(const or_config* cfg, uint64_t seed, int max_ctx, int max_rows);
void or_model_destroy(or_model* m);
/* direct tensor access for parity checks: which = OR_T_* (layer >= 0), or layer = -1 with
 * which = 0 embed, 1 lm_head; expert >= 0 selects a MoE expert tensor */
int or_model_linear(or_model* m, int layer, int which, int expert, const uint32_t** wq,
                    const uint16_t** scales, const uint16_t** biases, int* N, int* K);
const or_config* or_model_cfg(or_model* m);
const float* or_model_rope_cos(or_model* m);
const float* or_model_rope_sin(or_model* m);

/* KV state per row */
int or_kv_len(or_model* m, int row);
void or_kv_set_len(or_model* m, int row, int len);
/* fill positions [0,n) of a row with seeded synthetic bf16 K/V (stress workloads) */
void or_kv_fill_synthetic(or_model* m, int row, int n, uint64_t seed);
/* copy one row's K or V for a layer: out[n_kv][len][d] bf16 */
void or_kv_read(or_model* m, int layer, int row, int which_v, uint16_t* out);

/* Forward over `counts[r]` new tokens per row (rows listed in `rows`), positions
 * kv_len[row] + j; appends K/V and advances kv_len.  logits [sum counts][V] as
 * bf16-rounded values stored in uint16 (NULL to skip). */
int or_forward(or_model* m, int nrows, const int32_t* rows, const int32_t* counts,
               const int32_t* tokens, uint16_t* logits);
/* Same forward but returning each layer's hidden state after the layer (debug/parity),
 * hidden[(layer+1)][M][H] bf16 with hidden[0] = embeddings; NULL to skip. */
int or_forward_trace(or_model* m, int nrows, const int32_t* rows, const int32_t* counts,
                     const int32_t* tokens, uint16_t* logits, uint16_t* hidden);
/* ... and each layer's attention output (before o_proj), attn[layer][M][n_q_heads * head_dim]
 * bf16; NULL to skip. */
int or_forward_attn(or_model* m, int nrows, const int32_t* rows, const int32_t* counts,
                    const int32_t* tokens, uint16_t* logits, uint16_t* hidden, uint16_t* attn);

void or_set_threads(int n);
/* While out != NULL, every Qwen3-MoE forward writes each layer's bf16 router logits there,
 * out[layer][M][n_experts] (the values the top-k selection reads); NULL to stop. */
void or_capture_router(uint16_t* out);
/* reversed != 0: every fp32 reduction of the forward (linears, RMSNorm, attention) runs in
 * another order (test aid: the rounding noise floor between two exact summation orders) */
void or_set_reduction_order(int reversed);

/* y[M][N] = x[M][K] . dequant(W)^T for one MLX 4-bit affine g64 tensor (fp32 in/out);
 * the same per-output fixed-order reduction the forward uses. */
void or_qmatmul(const uint32_t* wq, const uint16_t* scales, const uint16_t* biases, int N, int K,
                const float* x, int M, float* y);

/* ---- generator + scheduler restatement ---- */
enum { OR_ACCEPT_ALL_OR_NOTHING = 0, OR_ACCEPT_PREFIX = 1 };

typedef struct or_spec_config {   /* SpeculativeDecodingConfiguration, BatchGenerator.swift:10-29 */
  int enabled, max_proposal_tokens, max_suffix_tokens, min_context_tokens;
  int acceptance;        /* OR_ACCEPT_* */
  int single_row_only;   /* reference gate rowUIDs.count == 1 (:959) */
  int greedy_only;       /* reference gate temperature == 0 && no RNG (:963,970) */
} or_spec_config;

typedef struct or_sampling {      /* subset of SamplingParameters, Sampling.swift:139-217 */
  float temperature, top_p;
  int has_seed;
  uint64_t seed;
  int n_eos;
  int32_t eos[8];
  int32_t reject_token;          /* QwenXMLToolGrammar toolCallStartTokenID; -1 = none */
  int32_t top_k;                 /* 0 = off */
  float min_p;                   /* 0 = off */
  float repetition_penalty;      /* 1 = off (0 is read as 1) */
  float presence_penalty, frequency_penalty;
  int32_t min_tokens;
  int32_t n_bias;                /* logit bias entries, at most 16 */
  int32_t bias_token[16];
  float bias_value[16];
} or_sampling;

typedef struct or_stats {         /* SpeculativeDecodingStats, BatchGenerator.swift:31-38 */
  int64_t proposed, accepted, proposal_batches, rejected_batches;
} or_stats;

typedef struct or_generator or_generator;
or_generator* or_generator_create(or_model* m, const or_spec_config* cfg, int max_rows,
                                  int max_hist, uint64_t global_seed);
void or_generator_destroy(or_generator* g);
/* Admit a request into slot `row`: prefill the prompt (all but the last token, then the
 * last token alone, Scheduler.swift:722-739), sample the first token, seed the token
 * history with prompt + first token (Scheduler.swift:630).  Returns the first token,
 * and sets *finished (1 stop, 2 length) when the request ends at admission. */
int or_generator_insert(or_generator* g, int row, const int32_t* prompt, int n_prompt,
                        int max_tokens, const or_sampling* sp, int* finished);
/* Admit with a pre-filled KV (stress workloads): history = ctx, cur token = last of ctx,
 * kv_len = n_ctx - 1 must already hold. */
int or_generator_insert_prefilled(or_generator* g, int row, const int32_t* ctx, int n_ctx,
                                  int max_tokens, const or_sampling* sp);
void or_generator_remove(or_generator* g, int row);
/* One Scheduler.step of decode: out_tokens[row][K+1], out_counts[row], out_finish[row]
 * (0 running, 1 stop, 2 length); finished rows are removed.  Returns number of rows
 * that produced tokens.  `forced_accept` (NULL = none) caps each row's accepted drafts
 * (stress workloads: forced accept-length schedule). */
int or_generator_step(or_generator* g, int32_t* out_tokens, int32_t* out_counts,
                      int32_t* out_finish, const int32_t* forced_accept);
void or_generator_stats(or_generator* g, or_stats* out);
/* width of each warm-cache forward per row, for the reference's decode-call accounting */
int or_generator_call_widths(or_generator* g, int32_t* out, int cap);
int or_generator_active(or_generator* g, int row);
int or_generator_history(or_generator* g, int row, int32_t* out, int cap);

#ifdef __cplusplus
}
#endif
#endif
