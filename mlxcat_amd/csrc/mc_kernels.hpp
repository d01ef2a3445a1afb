// mc_kernels.hpp -- launch interface of the per-token kernels of the verify forward
// (embedding, q/k-norm + RoPE + KV append, split-KV GQA attention) and the
// step kernels (n-gram proposer, acceptance, commit).
#pragma once
#include "mc_common.hpp"

namespace mc {

// Verify-forward token slots.  Slot m carries token slot_tok[m] of row slot_row[m]
// (-1 = padding) at absolute position slot_pos[m].  Per row, the queries occupy
// slots [row_slot0[r], row_slot0[r] + n_valid[r]) at positions qbase[r] + j.
struct SlotView {
  const int32_t* slot_tok;
  const int32_t* slot_row;
  const int32_t* slot_pos;
  const int32_t* row_slot0;
  const int32_t* n_valid;
  const int32_t* qbase;
};

struct KVLayer {
  uint16_t* k;  // [R][n_kv][cap][d]
  uint16_t* v;  // transposed: [R][n_kv][d][cap], so 8 consecutive positions of one
                // dimension are one 16-byte load (the k operand of the P V product)
  int cap;      // position stride, a multiple of 64
};

// x[m][:] = embedding row of slot_tok[m]; ssq[m * ss_ld + t] = sum of squares of x[m][16t : 16t + 16]
int launch_embed(const QLinear& E, const int32_t* slot_tok, int M, int H, uint16_t* x, float* ssq, int ss_ld,
                 hipStream_t st);
// qkv [M][(nq + 2 nkv) d] -> q [M][nq d] (normed + rotated), K/V cache append for valid slots
int launch_qk_rope_append(const uint16_t* qkv, const uint16_t* q_norm, const uint16_t* k_norm, const float* rope_cos,
                          const float* rope_sin, int M, int nq, int nkv, int d, float eps, const int32_t* slot_row,
                          const int32_t* slot_pos, KVLayer kv, uint16_t* q_out, hipStream_t st);
// split-KV attention (head_dim 64 or 128): per-split partials, then their merge into att [M][nq d]
struct AttnWork {
  float* part_o;   // [M][nq][nchunk][d]
  float* part_ml;  // [M][nq][nchunk][2]
  int nchunk;      // ceil(cap / ATTN_CHUNK)
};
constexpr int ATTN_CHUNK = 64;
// The fused path (fuse != NULL): the attention blocks also do the q/k-norm + RoPE of their
// queries and append the new keys (no launch_qk_rope_append), and the last block of each
// (row, kv head) merges the splits (no merge launch).  At most 64 queries per (row, kv head).
constexpr int FUSE_QMAX = 64;
struct AttnFuse {
  const uint16_t* qkv = nullptr;     // [M][(nq + 2 nkv) d] projections of the slots
  const uint16_t* q_norm = nullptr;  // [d] (NULL: no q/k norm, Llama)
  const uint16_t* k_norm = nullptr;
  const float* rope_cos = nullptr;   // [pos][d / 2]
  const float* rope_sin = nullptr;
  float eps = 0.f;
  unsigned* counters = nullptr;      // [R * nkv] split arrivals, zero at rest
  uint16_t* att = nullptr;           // [M][nq d]
};
// 64-key sub-chunks per attention block; whether the fused path serves a call
int attn_split(int R, int nkv, int nchunk, bool fused);
bool attn_fuse_ok(int R, int nkv, int nchunk, int max_q, int nq, int d);
int launch_attention(const uint16_t* q, KVLayer kv, const SlotView& sv, int R, int max_q, int nq, int nkv, int d,
                     int M, const AttnWork& w, const AttnFuse* fuse, uint16_t* att, hipStream_t st);

int launch_fake_logits(int arch, const int32_t* slot_tok, int M, int V, uint16_t* logits, hipStream_t st);

// Fill positions [0, n) of a row with seeded synthetic bf16 K/V (matches the oracle).
int launch_kv_synth(KVLayer kv, int layer, int row, int nkv, int d, int n, uint64_t seed, hipStream_t st);
// Positions [t0, t0 + n) of one row's V (v_row: that row's [nkv][d][cap]) to or from a prefix
// block's [nkv][n][d] (blk, device memory).
int launch_kv_block_v(uint16_t* v_row, int cap, uint16_t* blk, int nkv, int n, int d, int t0, bool to_block,
                      hipStream_t st);

}  // namespace mc
