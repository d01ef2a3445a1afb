// mc_fused.hpp -- the verify forward as one persistent kernel for small token counts
// (kernels in mc_fused.hip).
//
// One block per CU; every block stays resident for the whole forward.  Waves 0..2 of a
// block stream weights / KV into registers and run the matrix-core work units; wave 3
// (the control wave) runs the split-K reductions, the attention combine and the
// embedding.  Phases hand data to each other through "LL" words: 8-byte
// device-coherent stores of (32-bit payload, 32-bit tag), where the tag names the
// forward call and the producing phase.  A consumer polls the words it needs until every
// tag matches, so there is no grid barrier and a unit's weights are loaded before its
// inputs exist.
#pragma once
#include "mc_common.hpp"
#include "mc_kernels.hpp"

namespace mc {

constexpr int FW_THREADS = 256;
constexpr int FW_CW = 3;       // compute waves per block; wave FW_CW is the control wave
constexpr int FW_MMAX = 8;     // tokens per launch, at most
constexpr int FW_UGP = 20;     // group pairs (128 inputs) per GEMV work unit, at most
constexpr int FW_QROWS = 32;   // query rows per (row, kv head): GQA group (<= 4) x 8 tokens
constexpr int FW_AKEYS = 64;   // cached keys per attention work unit

// One linear in the tile layout of mc_gemv (qw [NT][GP][64][4], sb [NT][16][GP][2]),
// split into ks K-ranges of ugp group pairs (the last one may be shorter).
struct FwLin {
  const uint32_t* qw = nullptr;
  const uint32_t* sb = nullptr;
  int N = 0, K = 0, NT = 0, GP = 0;
  int ks = 1, ugp = 0;
};

struct FwLayer {
  FwLin qkv, o, gu, dn;
  const uint16_t* in_norm = nullptr;
  const uint16_t* post_norm = nullptr;
  const uint16_t* q_norm = nullptr;   // NULL: no q/k norm (Llama)
  const uint16_t* k_norm = nullptr;
  uint16_t* k = nullptr;              // cache K [R][nkv][cap][d]
  uint16_t* v = nullptr;              // cache V^T [R][nkv][d][cap]
};

struct FwArgs {
  const FwLayer* layers = nullptr;    // device array [L]
  int L = 0;
  QLinear embed;                      // tile layout [V][H]
  FwLin head;
  const uint16_t* final_norm = nullptr;
  int H = 0, nq = 0, nkv = 0, d = 0, I = 0, V = 0;
  float eps = 0.f, scale = 0.f;
  const float* rope_cos = nullptr;    // [ctx][d / 2]
  const float* rope_sin = nullptr;
  int cap = 0;                        // cache position stride
  int R = 0, M = 0;                   // rows with slots, slots (tokens)
  // slots: slot m belongs to row slot_row[m] (< 0: padding) at position slot_pos[m];
  // row r owns slots row_slot0[r] .. + n_valid[r] - 1 and has qbase[r] cached keys
  const int32_t* slot_tok = nullptr;
  const int32_t* slot_row = nullptr;
  const int32_t* row_slot0 = nullptr;
  const int32_t* n_valid = nullptr;
  const int32_t* qbase = nullptr;
  // LL words (payload | tag << 32)
  unsigned long long* x = nullptr;      // [FW_MMAX][H / 2]   residual stream, bf16 pairs
  unsigned long long* xss = nullptr;    // [FW_MMAX][H / 16]  sum of squares per 16 columns
  unsigned long long* qkv = nullptr;    // [FW_MMAX][Nqkv / 2]
  unsigned long long* att = nullptr;    // [FW_MMAX][nq d / 2]
  unsigned long long* act = nullptr;    // [FW_MMAX][I / 2]
  unsigned long long* opart = nullptr;  // [o.ks][FW_MMAX][H]   f32 split-K partials
  unsigned long long* dpart = nullptr;  // [dn.ks][FW_MMAX][H]
  unsigned long long* ao = nullptr;     // [R][nkv][npb_cap][FW_QROWS][d]  attention block partials
  unsigned long long* aml = nullptr;    // [R][nkv][npb_cap][FW_QROWS][2]  (max, sum)
  int npb_cap = 0;
  int with_head = 1;                    // 0: stop after the last layer (no logits)
  uint16_t* logits = nullptr;           // [M][V]
  unsigned long long* amax = nullptr;   // [M][head.NT] tile argmax keys (mc_gemv's encoding)
  const unsigned* epoch = nullptr;      // forward-call counter (bumped after each launch)
  unsigned* err = nullptr;              // sticky: nonzero after a wait timed out
};

// The kernel (grid: fused_grid() blocks of FW_THREADS, fused_lds_bytes() of dynamic LDS).
__global__ void fused_forward_kernel(FwArgs a);

// Plan of one linear: K-ranges of at most FW_UGP group pairs, an even count each.
FwLin fused_lin(const QLinear& L, int max_ks);
// Whether the persistent forward serves this shape (M tokens over R rows).
bool fused_supported(const mc_model_config& c, int M, int cap, const char** why);
int fused_npb_cap(int cap);
size_t fused_lds_bytes();
int launch_fused_forward(const FwArgs& a, int grid, hipStream_t st);
int launch_epoch_bump(unsigned* epoch, hipStream_t st);
int fused_grid(int device);

}  // namespace mc
