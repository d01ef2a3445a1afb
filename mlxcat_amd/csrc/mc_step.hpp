// mc_step.hpp -- device state and kernels of the speculative step (n-gram proposer,
// acceptance scan, commit with per-row KV rollback).
#pragma once
#include "mc_common.hpp"

namespace mc {

// Device-resident state of every row.  All arrays are indexed by row r < R; the
// per-position ones by r * K1 + j with K1 = K + 1.
struct StepState {
  int R = 0, K = 0, K1 = 1, hcap = 0, V = 0;
  // SpeculativeDecodingConfiguration (BatchGenerator.swift:10-29)
  int enabled = 0, max_suffix = 16, min_ctx = 8, acceptance = 0, single_row_only = 0, greedy_only = 0;
  // rows
  int32_t* active = nullptr;
  int32_t* hist = nullptr;      // [R][hcap] speculativeTokenHistory
  int32_t* hist_len = nullptr;
  int32_t* gen = nullptr;       // generatedTokenHistory.count
  int32_t* max_gen = nullptr;
  int32_t* cur = nullptr;       // currentTokens (pending, not in the KV)
  int32_t* kv_len = nullptr;    // committed KV positions
  // sampling
  float* temp = nullptr;
  float* top_p = nullptr;
  float* inv_temp = nullptr;
  int32_t* has_seed = nullptr;
  uint64_t* seed = nullptr;
  uint64_t* counter = nullptr;
  int32_t* eos = nullptr;       // [R][8]
  int32_t* n_eos = nullptr;
  int32_t* reject = nullptr;
  // sampler options beyond temperature / top-p (Sampling.swift:139-217)
  int32_t* top_k = nullptr;     // 0 = off
  float* min_p_log = nullptr;   // log(min_p), -inf = off
  float* rep_pen = nullptr;     // 1 = off
  float* pres_pen = nullptr;
  float* freq_pen = nullptr;
  int32_t* min_tokens = nullptr;
  int32_t* n_bias = nullptr;
  int32_t* bias_tok = nullptr;  // [R][16]
  float* bias_val = nullptr;    // [R][16]
  int32_t* proc = nullptr;      // bit 0: bias, bit 1: min_tokens mask possible, bit 2: penalties
  int32_t* gen_cnt = nullptr;   // [R][V] occurrences of each token among the generated ones
                                // (maintained for rows with penalties only)
  // caller-supplied uniforms [R][K1][2] (accept test, sample draw), used when *use_uniforms
  const uint32_t* uniforms = nullptr;
  const int32_t* use_uniforms = nullptr;
  // step scratch
  int32_t* drafts = nullptr;    // [R][K1]
  int32_t* nprop = nullptr;     // [R]
  int32_t* dext = nullptr;      // [R] 1: drafts[r][nprop] holds the history's next token (forced schedule)
  int32_t* slot_tok = nullptr;  // [R * K1] (or larger for prefill)
  int32_t* slot_row = nullptr;
  int32_t* slot_pos = nullptr;
  int32_t* row_slot0 = nullptr; // [R]
  int32_t* n_valid = nullptr;   // [R]
  int32_t* qbase = nullptr;     // [R]
  int32_t* scan_tok = nullptr;  // [R][K1]
  int32_t* scan_acc = nullptr;  // [R][K1]
  int32_t* scan_res = nullptr;  // [R][K1]
  int32_t* forced = nullptr;    // [R], -1 = none
  // outputs
  int32_t* out_tok = nullptr;   // [R][K1]
  int32_t* out_cnt = nullptr;   // [R]
  int32_t* out_fin = nullptr;   // [R]
  unsigned long long* stats = nullptr;  // proposed, accepted, proposal_batches, rejected_batches
  // greedy argmax partials of the verify logits written by the head (NULL: scan the logits)
  const unsigned long long* amax = nullptr;  // [slot][amax_nt]
  int amax_nt = 0;
};

int launch_propose(const StepState& s, hipStream_t st);
// row_filter -1: every active row; r >= 0: only row r (first-token sampling at admission)
int launch_accept_scan(const StepState& s, const uint16_t* logits, int row_filter, hipStream_t st);
int launch_commit(const StepState& s, int row_filter, hipStream_t st);
int launch_decide(const StepState& s, int32_t* n_emit, int32_t* keep_out, int32_t* nacc_out, hipStream_t st);
// drafts [R][K] and n_draft [R] of caller device buffers into s (bad rows counted in *err)
int launch_accept_prep(const StepState& s, const int32_t* drafts, const int32_t* n_draft, int K, int32_t* err,
                       hipStream_t st);

// standalone entry points over caller data (mc_ngram_propose / mc_accept)
int launch_ngram_standalone(const int32_t* hist, const int64_t* off, int B, int max_suffix, int min_ctx,
                            const int32_t* limit, int out_stride, int32_t* out, int32_t* out_len, hipStream_t st);

}  // namespace mc
