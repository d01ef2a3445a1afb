/*
 * mlxcat_hip.h -- C ABI of the MI355X (gfx950) n-gram speculative-decode step.
 *
 * This is the drop-in boundary a Swift C target (`CMLXCatHIP`) binds in place
 * of the Metal path behind mlxcat's ContinuousBatchGenerator.  Every entry
 * point names the reference interface it replaces (local-ai-cat/mlxcat, paths
 * relative to its root; MLX / mlx-swift-lm symbols are external SwiftPM
 * dependencies pinned at Package.swift:61-95).
 *
 * Conventions
 *   - Every function returns 0 on success and a negative MC_E_* code on
 *     failure; mc_last_error() returns a thread-local message.  In Swift these
 *     map to `throws` (BatchGeneratorError / BatchKVCacheError) and at the
 *     scheduler to Response(token: -1, finishReason: .failed(msg))
 *     (Sources/MLXCat/TrackB/Scheduler.swift:532-541).
 *   - Host buffers are caller-owned; device memory is owned by the handles.
 *   - Handles are not thread-safe.  Each batch handle owns one HIP stream, which
 *     matches the reference's actor serialisation (Scheduler.swift:13).
 *   - Tokens are int32, logits bf16 stored as uint16.
 *   - Weights use MLX's 4-bit affine format with group size 64: wq[N][K/8]
 *     uint32 with element j of a word at bits 4j, scales/biases [N][K/64] bf16
 *     (group cost 64*bits/8 + 4 bytes: Sources/MLXCat/TrackB/KVQuantizationPolicy.swift:12-14).
 *     The library repacks them once, losslessly, into its MFMA tile layout.
 */
#ifndef MLXCAT_HIP_H
#define MLXCAT_HIP_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes ---- */
#define MC_OK 0
#define MC_E_INVALID (-1)  /* bad argument or shape */
#define MC_E_HIP (-2)      /* HIP runtime error */
#define MC_E_NOMEM (-3)    /* device allocation failed */
#define MC_E_STATE (-4)    /* call not valid in the handle's current state */
#define MC_E_CAPACITY (-5) /* row, context or history capacity exceeded */

/* ---- architectures ---- */
#define MC_ARCH_QWEN3 0
#define MC_ARCH_LLAMA 1
#define MC_ARCH_QWEN3_MOE 2
/* The reference's scheduler test doubles, SchedulerSpeculativeDecodingTests.swift:174-261:
 * logits +20 at next(token) and -20 elsewhere, next(1)=2, next(2)=3, else 1;
 * the mismatching variant maps 3 -> 4. */
#define MC_ARCH_FAKE_REPEATING 100
#define MC_ARCH_FAKE_MISMATCHING 101

/* linear tensor slots (mc_model_set_linear / mc_model_get_linear) */
#define MC_W_Q 0
#define MC_W_K 1
#define MC_W_V 2
#define MC_W_O 3
#define MC_W_GATE 4
#define MC_W_UP 5
#define MC_W_DOWN 6
#define MC_W_ROUTER 11
#define MC_W_EMBED 100   /* layer ignored; tied models use it as the LM head */
#define MC_W_LM_HEAD 101 /* untied models only */
/* norm slots (mc_model_set_norm) */
#define MC_N_INPUT 7
#define MC_N_POST 8
#define MC_N_Q 9
#define MC_N_K 10
#define MC_N_FINAL 102

/* acceptance rules */
#define MC_ACCEPT_ALL_OR_NOTHING 0 /* the reference rule, BatchGenerator.swift:906-947 */
#define MC_ACCEPT_PREFIX 1         /* longest agreeing prefix + correction, per-row rollback */

typedef struct mc_model mc_model;
typedef struct mc_batch mc_batch;

/* Model shape.  Mirrors the config.json keys an MLX checkpoint carries
 * (Sources/MLXCatNative/NativeModelEngine.swift:1147-1231).  Supported: head_dim 64 or 128,
 * hidden a multiple of 64 up to 4096; Qwen3-MoE up to 256 experts, top-k <= 8, hidden and
 * moe_intermediate up to 2560. */
typedef struct mc_model_config {
  int32_t arch;
  int32_t n_layers, hidden, n_q_heads, n_kv_heads, head_dim, intermediate, vocab;
  int32_t tied_embeddings;
  float rms_eps, rope_theta;
  int32_t n_experts, n_experts_per_tok, moe_intermediate;
} mc_model_config;

/* SpeculativeDecodingConfiguration, Sources/MLXCat/TrackB/BatchGenerator.swift:10-29.
 * Clamped like the Swift initialiser: K >= 0, max_suffix >= 1, min_context >= 2. */
typedef struct mc_spec_config {
  int32_t enabled;
  int32_t max_proposal_tokens; /* K */
  int32_t max_suffix_tokens;   /* default 16 */
  int32_t min_context_tokens;  /* default 8 */
  int32_t acceptance;          /* MC_ACCEPT_* for greedy rows */
  int32_t single_row_only;     /* reference gate rowUIDs.count == 1 (BatchGenerator.swift:959) */
  int32_t greedy_only;         /* reference gate temperature == 0 && no RNG (:963,970) */
} mc_spec_config;

/* Subset of SamplingParameters (Sources/MLXCat/TrackB/Sampling.swift:139-217) used by the step.
 * Per position the sampler sees the bf16 logits in fp32 after the logit bias and the
 * min_tokens EOS mask (Sampling.swift:638-652) and the penalties over the generated tokens
 * (:592-636); greedy rows take the argmax of those values, sampled rows filter them with
 * top-p, min-p and top-k in that order (:500-522) and scale by 1 / temperature.  A
 * zero-filled struct is plain greedy decoding. */
typedef struct mc_sampling {
  float temperature;   /* 0 = greedy argmax, lowest index on ties */
  float top_p;         /* applied when 0 < top_p < 1, Sampling.swift:847-858 */
  int32_t has_seed;
  uint64_t seed;       /* per-request RNG (BatchGenerator.swift:1089-1091) */
  int32_t n_eos;
  int32_t eos[8];
  int32_t reject_token; /* tool-call trigger (BatchGenerator.swift:920-923); -1 = none */
  int32_t top_k;        /* 0 = off; ties at the k-th value keep the lowest token ids */
  float min_p;          /* 0 = off; keeps values v with v - max >= log(min_p) */
  float repetition_penalty; /* 1 = off; 0 is read as 1 */
  float presence_penalty;   /* 0 = off */
  float frequency_penalty;  /* 0 = off */
  int32_t min_tokens;   /* EOS ids masked while fewer tokens were generated */
  int32_t n_bias;       /* logit bias entries (at most 16; ids outside the vocabulary ignored) */
  int32_t bias_token[16];
  float bias_value[16];
} mc_sampling;

/* SpeculativeDecodingStats, BatchGenerator.swift:31-38 */
typedef struct mc_spec_stats {
  int64_t proposed, accepted, proposal_batches, rejected_batches;
} mc_spec_stats;

/* ---- errors / device ---- */
const char* mc_last_error(void);
/* Selects the HIP device for subsequent handle creation. */
int mc_set_device(int device);

/* ---- model: replaces the mlx-swift-lm LanguageModel (Qwen3 / Llama / Qwen3-MoE modules),
 * protocol shape at Tests/MLXCatTests/SchedulerSpeculativeDecodingTests.swift:174-223 ---- */
int mc_model_create(const mc_model_config* cfg, mc_model** out);
void mc_model_destroy(mc_model* m);
/* Fill every tensor with the seeded synthetic generator (random-init workloads). */
int mc_model_init_synthetic(mc_model* m, uint64_t seed);
/* Load one quantized linear from host MLX tensors (a .weight/.scales/.biases triplet);
 * expert >= 0 selects a MoE expert's gate/up/down. */
int mc_model_set_linear(mc_model* m, int32_t layer, int32_t which, int32_t expert,
                        const uint32_t* wq, const uint16_t* scales, const uint16_t* biases);
/* Export a linear back to MLX format (host buffers of the MLX shapes). */
int mc_model_get_linear(mc_model* m, int32_t layer, int32_t which, int32_t expert, uint32_t* wq,
                        uint16_t* scales, uint16_t* biases);
int mc_model_set_norm(mc_model* m, int32_t layer, int32_t which, const uint16_t* w);

/* ---- batch state: replaces BatchKVCache (Sources/MLXCat/TrackB/BatchCache.swift:37-433),
 * the per-row token histories and currentTokens of ContinuousBatchGenerator
 * (BatchGenerator.swift:144-215).  Per-row contiguous bf16 K/V with a length; fork,
 * commit and rollback are O(1) length updates instead of copy() (BatchCache.swift:426-433)
 * plus trim (:403-424). ---- */
int mc_batch_create(mc_model* m, int32_t max_rows, int32_t max_ctx, int32_t max_draft,
                    const mc_spec_config* spec, mc_batch** out);
void mc_batch_destroy(mc_batch* b);
/* ContinuousBatchGenerator.insert after admission (BatchGenerator.swift:344-474,
 * Scheduler.swift:599-668): prefill the prompt into `row`, sample the first token,
 * seed the speculative history with prompt + first token.  *finished = 1 (EOS) or
 * 2 (length) when the request ends at admission. */
int mc_batch_insert(mc_batch* b, int32_t row, const int32_t* prompt, int32_t n_prompt,
                    int32_t max_tokens, const mc_sampling* sp, int32_t* first_token,
                    int32_t* finished);
/* mc_batch_insert after a prefix-cache hit (Scheduler.swift:960-990 prepareHitRow): the
 * row's K/V already holds prompt positions [0, n_cached) (mc_batch_import_kv_block), and
 * prefill resumes at n_cached (0 <= n_cached < n_prompt; MC_E_STATE unless the row's K/V
 * length is n_cached). */
int mc_batch_insert_cached(mc_batch* b, int32_t row, const int32_t* prompt, int32_t n_prompt, int32_t n_cached,
                           int32_t max_tokens, const mc_sampling* sp, int32_t* first_token, int32_t* finished);
/* Admit a row whose first n_ctx-1 positions of K/V were filled by
 * mc_batch_fill_synthetic_kv; the last token of ctx is the pending current token. */
int mc_batch_insert_prefilled(mc_batch* b, int32_t row, const int32_t* ctx, int32_t n_ctx,
                              int32_t max_tokens, const mc_sampling* sp);
/* Seeded synthetic bf16 K/V for positions [0, n) of a row (stress workloads). */
int mc_batch_fill_synthetic_kv(mc_batch* b, int32_t row, int32_t n, uint64_t seed);
/* ContinuousBatchGenerator.remove (BatchGenerator.swift:476-480). */
int mc_batch_remove(mc_batch* b, int32_t row);
/* BatchKVCache.trim (BatchCache.swift:403-424): drop min(n, len) trailing positions of
 * every active row; returns the trimmed count (>= 0) or an error. */
int mc_batch_trim(mc_batch* b, int32_t n);
/* Per-row ragged rollback (no reference counterpart: the reference drops the forked
 * cache wholesale).  Drops min(n, len) trailing positions of one row. */
int mc_batch_rollback(mc_batch* b, int32_t row, int32_t n);
/* BatchKVCache.filter(keeping:) (BatchCache.swift:217-246): rows[0..n) of the batch, in that
 * order, become rows 0..n-1 with their K/V, lengths, token histories and sampler state
 * (a row may be listed more than once, as the reference's take() allows); the remaining
 * rows are left empty (inactive, no K/V).  Rows have no left padding to drop. */
int mc_batch_filter(mc_batch* b, const int32_t* rows, int32_t n);
/* BatchKVCache.extract(_:) (BatchCache.swift:196-215): one row's K/V, positions
 * [0, kv_len), copied into row dst_row of dst (a batch of a model with the same K/V shape,
 * on the same device, or the same batch); that row becomes inactive with this K/V and
 * length, ready for mc_batch_insert_prefilled.  MC_E_CAPACITY if the K/V does not fit. */
int mc_batch_extract_kv(mc_batch* b, int32_t row, mc_batch* dst, int32_t dst_row);
/* Prefix blocks (TrackA/BlockAwarePrefixCache.swift:140-162 payloadForBlock): positions
 * [t0, t0 + n) of one row's K/V in the reference's per-layer cache-state layout, keys and
 * values each [n_layers][n_kv][n][d] bf16 host arrays (layer l's state[0|1][0, :, t0..<t0+n, :],
 * the tensors that TrackA/SafetensorsBlockIO.swift:40-50 writes as layer.l.keys / .values).
 * t0 + n <= the row's K/V length. */
int mc_batch_export_kv_block(mc_batch* b, int32_t row, int32_t t0, int32_t n, uint16_t* keys, uint16_t* values);
/* The reverse (reconstructCache, TrackA/BlockAwarePrefixCache.swift:57-85, which concatenates
 * a hit's blocks in order): writes positions [t0, t0 + n) of the row, t0 <= its K/V length;
 * the row becomes inactive with K/V length t0 + n, ready for mc_batch_insert_cached. */
int mc_batch_import_kv_block(mc_batch* b, int32_t row, int32_t t0, int32_t n, const uint16_t* keys,
                             const uint16_t* values);
int mc_batch_kv_len(mc_batch* b, int32_t row, int32_t* len);
/* Copy one row's K (which_v = 0) or V (1) of one layer to host: [n_kv][len][d] bf16. */
int mc_batch_read_kv(mc_batch* b, int32_t layer, int32_t row, int32_t which_v, uint16_t* out);
int mc_batch_history(mc_batch* b, int32_t row, int32_t* out, int32_t cap, int32_t* len);
/* The last layer's attention output (before o_proj) of the last forward, the first M of
 * its token slots: out[M][n_q_heads * head_dim] bf16 (parity inspection, like
 * mc_batch_read_kv; the slots of mc_forward are its rows' tokens in call order). */
int mc_batch_read_attention(mc_batch* b, int32_t M, uint16_t* out);
/* Logits of token slots [slot0, slot0 + n) of the last forward: out[n][vocab] bf16.  After
 * mc_step, row r's verify position j is slot r * (K + 1) + j. */
int mc_batch_read_logits(mc_batch* b, int32_t slot0, int32_t n, uint16_t* out);
/* Qwen3-MoE: the last layer's bf16 router logits of the last forward's token slots,
 * out[M][n_experts], for forwards of at most 64 slots (parity inspection of the top-k
 * routing, like mc_batch_read_attention). */
int mc_batch_read_router(mc_batch* b, int32_t M, uint16_t* out);

/* ---- forward: LanguageModel.callAsFunction(LMInput.Text, cache:, state:)
 * (BatchGenerator.swift:900-904).  counts[r] new tokens for each listed row, positions
 * kv_len[row] + j; K/V appended and kv_len advanced.  logits_host [sum counts][vocab]
 * bf16 (NULL to skip). ---- */
int mc_forward(mc_batch* b, int32_t nrows, const int32_t* rows, const int32_t* counts,
               const int32_t* tokens, uint16_t* logits_host);

/* ---- n-gram proposer: ContinuousBatchGenerator.proposeSuffixTokens
 * (BatchGenerator.swift:982-1010), run on the GPU over host-supplied histories.
 * hist_off[B+1] are offsets into hist; limit[B] per row; out[B][max(limit)] and
 * out_len[B] (0 = nil). ---- */
int mc_ngram_propose(const int32_t* hist, const int64_t* hist_off, int32_t B,
                     int32_t max_suffix, int32_t min_context, const int32_t* limit,
                     int32_t out_stride, int32_t* out, int32_t* out_len);

/* ---- acceptance: the loop over TokenSampler.sample at BatchGenerator.swift:906-935,
 * run on the GPU over host logits.  Per row r: logits rows [row_off[r], row_off[r] +
 * n_draft[r] + 1), drafts[r][0..n_draft[r]), generated tokens so far
 * generated[gen_off[r] .. gen_off[r+1]) (the penalties' and min_tokens' history; NULL =
 * none).  Greedy rows use `acceptance`; rows with temperature > 0 use speculative sampling
 * with 32-bit uniforms: uniforms[r][j][0] the accept test and [r][j][1] the sample draw of
 * position j (row stride 2 * (draft_stride + 1)), or, when uniforms is NULL, the ones
 * derived from (seed, counter[r]).  Outputs: n_emit[r] tokens in out_tokens[r][0 ..
 * draft_stride] (row stride draft_stride + 1), kv_keep[r] positions of the verified block
 * to keep, n_accepted[r] drafts accepted. ---- */
int mc_accept(const uint16_t* logits, int32_t vocab, int32_t B, const int64_t* row_off,
              const int32_t* drafts, int32_t draft_stride, const int32_t* n_draft,
              const mc_sampling* sp, const int32_t* generated, const int64_t* gen_off,
              const uint64_t* counter, const uint32_t* uniforms, int32_t acceptance,
              int32_t* out_tokens, int32_t* n_emit, int32_t* kv_keep, int32_t* n_accepted);

/* ---- acceptance that allocates nothing.  No counterpart in the reference: for callers that
 * cannot allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  The same acceptance as mc_accept with no generated
 * history, over caller DEVICE buffers: logits [B][K+1][vocab] bf16 (row r's position j at
 * r*(K+1)+j), drafts [B][K], n_draft [B], uniforms [B][K+1][2] or NULL (derived from seed
 * and counter), outputs out_tokens [B][K+1], n_emit, kv_keep, n_accepted [B].  sp and
 * counter are host arrays of B entries.  At most 64 rows and K <= 16 (MC_E_CAPACITY
 * beyond).  Its state is a 64 KiB device array per GPU, held until the process ends and
 * shared by all calls on that GPU: calls that overlap on one GPU race.  Runs on the null
 * stream of the device mc_set_device selected and returns after the results are written;
 * MC_E_INVALID if an n_draft or draft id is out of range. ---- */
int mc_accept_noalloc(const uint16_t* logits, int32_t vocab, int32_t B, int32_t K, const int32_t* drafts,
                      const int32_t* n_draft, const mc_sampling* sp, const uint64_t* counter,
                      const uint32_t* uniforms, int32_t acceptance, int32_t* out_tokens, int32_t* n_emit,
                      int32_t* kv_keep, int32_t* n_accepted);

/* ---- fused step: ContinuousBatchGenerator.next() -> speculativeNext()
 * (BatchGenerator.swift:593-600, 875-955) plus Scheduler.step's finish handling
 * (Scheduler.swift:361-427), for every active row at once: propose, verify forward,
 * accept, roll back, append history; one host synchronisation.  out_tokens[row][K+1],
 * out_counts[row] tokens emitted, out_finish[row] 0 running / 1 stop (EOS) / 2 length;
 * finished rows are removed.  forced_accept (NULL = none) caps each row's accepted drafts
 * (stress workloads with a forced accept-length schedule).  uniforms (NULL = derived from
 * each row's seed and step counter) supplies the draws of sampled rows as in mc_accept,
 * uniforms[row][j][kind] with row stride 2 * (K + 1). ---- */
int mc_step(mc_batch* b, const int32_t* forced_accept, const uint32_t* uniforms, int32_t* out_tokens,
            int32_t* out_counts, int32_t* out_finish);
/* SpeculativeDecodingStats accumulated by mc_step (Scheduler.swift:474-476). */
int mc_batch_stats(mc_batch* b, mc_spec_stats* out);
/* Widths of the warm-cache forwards issued so far (the reference tests' decode-call
 * accounting, SchedulerSpeculativeDecodingTests.swift:202-208); returns the count. */
int mc_batch_call_widths(mc_batch* b, int32_t* out, int32_t cap);

/* ---- timing support ---- */
/* Average device time (ms) of each kernel class over the last mc_step when profiling is
 * enabled; used by bench.py for the live roofline.  kind: 0 = dequant GEMV (all),
 * 1 = attention, 2 = whole verify step. */
int mc_batch_set_profiling(mc_batch* b, int32_t enabled);
int mc_batch_profile(mc_batch* b, int32_t kind, double* ms, double* bytes, int32_t* launches);

/* ---- measurement ---- */
/* No counterpart in the reference: the HBM read ceiling for the roofline fractions.  Reads
 * `bytes` per launch, `launches` launches back to back on a new stream of the current
 * device, each from its own slice of a pool of at least 1 GiB and 2 x bytes (larger than the
 * 256 MB Infinity Cache, so no launch hits a cache), for grids of 1.5, 3 and 6 blocks per CU;
 * returns the fastest grid's average time per launch (event-timed, launch gaps included)
 * and bytes / that time.  Allocates and frees the pool. */
int mc_probe_hbm_read(int64_t bytes, int32_t launches, double* us_per_launch, double* gb_per_s);

#ifdef __cplusplus
}
#endif
#endif
