// mc_xfwd.hpp -- the verify forward of at most 8 tokens as one persistent kernel laid out
// over the XCDs of the chip (kernels in mc_xfwd.hip).
//
// MI355X has 8 XCDs of 32 CUs, each XCD with its own L2.  The kernel runs one block per CU
// and gives XCD i one kv head (and its GQA group of q heads), 1/8 of the MLP intermediate
// and 1/8 of the K range of the o and down projections, so that every exchange inside a
// layer stays in the XCD's L2 except two: the o and down partial sums, which every XCD
// reduces redundantly from all eight (tensor-parallel style, with the all-reduce done by
// readers).  Blocks exchange data through tagged 8-byte words (32-bit payload | 32-bit
// tag naming the forward call, layer and phase); a consumer polls exactly the words it
// needs until every tag matches.
//
// A block has 8 waves: waves 0..3 compute, waves 4..7 are loaders.  Loader 4 + i streams
// the weights (and cached K/V) that compute wave i will consume, in consumption order,
// into its LDS ring with direct-to-LDS buffer loads, as far ahead as the ring allows.  So
// the HBM stream never waits for a phase's inputs, and a compute wave's own vector-memory
// counter holds only its polls (never a prefetch it would have to drain first).
#pragma once
#include "mc_common.hpp"

namespace mc {

constexpr int XF_XCD = 8;        // XCDs; XCD i owns kv head i
constexpr int XF_NCW = 4;        // compute waves per block (one per SIMD)
constexpr int XF_NLW = 4;        // loader waves per block; loader i feeds compute wave i
constexpr int XF_G = 4;          // GQA group size: compute waves 0..3 take one q head each in attention
constexpr int XF_CT = XF_NCW * 64;                 // compute threads
constexpr int XF_THREADS = (XF_NCW + XF_NLW) * 64;  // 512
constexpr int XF_MMAX = 8;       // tokens per launch, at most
constexpr int XF_TG = 5;         // output tiles per compute group
constexpr int XF_SLOT = 1152;    // ring slot: 1 KiB of weights or K/V + 128 B of scales/biases
constexpr int XF_NF = 14;        // ring chunks in flight per loader wave
constexpr int XF_QS = 136;       // q / new-k row stride in LDS (bf16)
constexpr int XF_REC = 132;      // words per attention record: o[128], max, sum, pad

// One linear in the tile layout of mc_gemv: qw [NT][GP][64 lanes][4 words],
// sb [NT][16 rows][GP][2 groups].
struct XLin {
  const uint32_t* qw = nullptr;
  const uint32_t* sb = nullptr;
  int N = 0, K = 0, NT = 0, GP = 0;
};

struct XLayer {
  XLin qkv, o, gu, dn;
  const uint16_t* in_norm = nullptr;
  const uint16_t* post_norm = nullptr;
  const uint16_t* q_norm = nullptr;  // NULL: no q/k norm (Llama)
  const uint16_t* k_norm = nullptr;
  uint16_t* k = nullptr;             // cache K [R][nkv][cap][d]
  uint16_t* v = nullptr;             // cache V^T [R][nkv][d][cap]
};

struct XArgs {
  const XLayer* layers = nullptr;  // device [L]
  int L = 0;
  XLin embed;                      // tile layout [V][H] (also the tied head)
  XLin head;
  const uint16_t* final_norm = nullptr;
  int H = 0, nq = 0, nkv = 0, d = 0, I = 0, V = 0;
  float eps = 0.f, scale = 0.f;
  const float* rope_cos = nullptr;  // [ctx][d / 2]
  const float* rope_sin = nullptr;
  int cap = 0;                      // cache position stride
  int R = 0;
  int bpx = 32;                     // blocks per XCD (grid = 8 bpx)
  int pdn[XF_XCD + 1] = {0};        // down-projection group-pair split over the XCDs
  int act_w = 0;                    // words per token row of the local activation slice
  int nch_cap = 0;                  // attention chunks (64 keys) per row, at most
  // slots: slot m belongs to row slot_row[m]; row r owns slots row_slot0[r] .. + n_valid[r] - 1
  // and has qbase[r] cached keys
  const int32_t* slot_tok = nullptr;
  const int32_t* slot_row = nullptr;
  const int32_t* row_slot0 = nullptr;
  const int32_t* n_valid = nullptr;
  const int32_t* qbase = nullptr;
  // tagged words (payload | tag << 32)
  unsigned long long* xl = nullptr;     // [8][MMAX][H / 2]       residual stream before attention (XCD-local)
  unsigned long long* xss = nullptr;    // [8][bpx][MMAX]         its sums of squares, per block's columns
  unsigned long long* x1l = nullptr;    // [8][MMAX][H / 2]       after attention
  unsigned long long* x1ss = nullptr;   // [8][bpx][MMAX]
  unsigned long long* qkvl = nullptr;   // [8][MMAX][(g + 2) d / 2]
  unsigned long long* rec = nullptr;    // [8][R][nch_cap][32][XF_REC] attention records (f32)
  unsigned long long* attl = nullptr;   // [8][MMAX][g d / 2]
  unsigned long long* opart = nullptr;  // [8][MMAX][H] o-projection partials (f32, read by every XCD)
  unsigned long long* actl = nullptr;   // [8][MMAX][act_w]
  unsigned long long* dpart = nullptr;  // [8][MMAX][H] down-projection partials
  uint16_t* logits = nullptr;           // [M][V]
  unsigned long long* amax = nullptr;   // [M][head.NT] tile argmax keys (mc_gemv's encoding)
  const unsigned* epoch = nullptr;      // forward-call counter (bumped after each launch)
  unsigned* err = nullptr;              // sticky: nonzero after a wait timed out
  unsigned* xcd_ctr = nullptr;          // [8] arrivals per XCD (reset after each launch)
  // LDS layout (bytes)
  int o_xprev = 0, o_red = 0, o_exch = 0, o_cm = 0, o_xsum = 0, o_x = 0, o_ring = 0, xst = 0, ring_slots = 0;
  int lds_bytes = 0;
};

// The fixed arguments live in device memory (scalar loads; a by-value argument struct whose
// address is taken is copied to scratch); the token count and the head flag vary per launch.
__global__ void xfwd_kernel(const XArgs* __restrict__ args, int M, int with_head);

// Whether the XCD-partitioned forward serves this model and batch (why: the reason if not).
bool xfwd_supported(const mc_model_config& c, int R, int cap, int cus, const char** why);
// Fill the LDS layout and the down-projection split of a; false if the shape does not fit.
bool xfwd_plan(XArgs& a);
int launch_xfwd(const XArgs* dev_args, int lds_bytes, int M, int with_head, int grid, hipStream_t st);
// epoch += 1 and the per-XCD arrival counters back to zero
int launch_xfwd_epoch(unsigned* epoch, unsigned* xcd_ctr, hipStream_t st);

}  // namespace mc
