// mc_gemv.hpp -- dequant GEMV launch interface (kernels in mc_gemv.hip).
#pragma once
#include "mc_common.hpp"

namespace mc {

enum Epi { EPI_STORE = 0, EPI_RESIDUAL = 1, EPI_SWIGLU = 2 };

struct GemvArgs {
  const uint32_t* qw = nullptr;      // tile-layout nibbles
  const uint32_t* sb = nullptr;      // tile-layout scale|bias
  const uint16_t* x = nullptr;       // [M][ldx] bf16
  int ldx = 0;
  // RMSNorm fused into the consumer: with norm_w set the input rows are the raw residual
  // stream x and each block stages bf16((x[m][k] * r[m]) * norm_w[k]) for its K-range, with
  // r[m] = 1 / sqrt(sum_t ss_in[m * ss_ld + t] / K + eps) from the producer's per-tile sums of
  // squares -- the rounding point of a standalone RMSNorm followed by the linear
  const uint16_t* norm_w = nullptr;  // [K] bf16 (NULL: no norm)
  const float* ss_in = nullptr;
  int ss_nt = 0, ss_ld = 0;
  float eps = 0.f;
  float* ss_out = nullptr;           // EPI_RESIDUAL: ss_out[m * ss_ld_out + t] of the new rows (NULL = skip)
  int ss_ld_out = 0;
  uint16_t* y = nullptr;             // [M][ldy] bf16 (EPI_RESIDUAL: read-modify-write)
  int ldy = 0;
  int M = 0, N = 0, K = 0, NT = 0, GP = 0;
  int kr = 0, ksplit = 1;            // group pairs per K-range, K-ranges
  float* part = nullptr;             // split-K partials [ksplit][NT][MT][64][4]
  size_t part_floats = 0;            // capacity of part (checked at launch)
  unsigned* counters = nullptr;      // [NT], zero at rest
  int counters_n = 0;                // capacity of counters (checked at launch)
  int epi = EPI_STORE;
  uint32_t dq_mask = DQ_MASK, dq_magic = DQ_MAGIC;  // nibble pair -> bf16 (1 + q / 16) constants
  // EPI_STORE only, non-null: amax[m * NT + t] = max over the tile's 16 rows of
  // (order-preserving key of the stored bf16 value) << 32 | (0xFFFFFFFF - row): the tile's
  // greedy argmax, lowest row on ties
  unsigned long long* amax = nullptr;
};

// Grouped GEMV over the experts a verify block touches (Qwen3-MoE SwitchGLU).  Every
// touched expert's tiles are streamed once for all the (token, slot) pairs routed to it.
// Pairs are numbered t * TK + kk (token t, k-th selected expert); the routing kernel lists
// them per touched expert in ascending order.
struct MoeRoute {
  int32_t* n_active = nullptr;  // [1] touched experts
  int32_t* act_e = nullptr;     // [E] touched experts, ascending
  int32_t* off = nullptr;       // [E + 1] offsets into pairs per touched expert
  int32_t* pairs = nullptr;     // [M * TK] pair numbers grouped by expert
  int32_t* sel = nullptr;       // [M * TK] selected expert of each pair
  int32_t* slot_pairs = nullptr; // [E][64] pair numbers of touched slot s, ascending (M <= 64)
  float* wts = nullptr;         // [M * TK] renormalised routing weight of each pair
};

struct MoeGemvArgs {
  const uint32_t* qw = nullptr;  // expert 0 (tile layout); expert e at + e * qw_es words
  const uint32_t* sb = nullptr;
  size_t qw_es = 0, sb_es = 0;
  int N = 0, K = 0, NT = 0, GP = 0;
  const uint16_t* x = nullptr;   // input row of pair p: x + (p / x_div) * ldx
  int ldx = 0, x_div = 1;
  MoeRoute rt;
  int epi = EPI_SWIGLU;          // EPI_SWIGLU: y[p][N / 2] bf16; EPI_STORE: yf[p][N] f32
  uint16_t* y = nullptr;
  float* yf = nullptr;
  int ldy = 0;
  int max_active = 0;            // touched experts, at most (grid rows)
  int nb = 1;                    // blocks per touched expert
  uint32_t dq_mask = DQ_MASK, dq_magic = DQ_MAGIC;
};

int moe_gemv_launch(const MoeGemvArgs& a, hipStream_t st);
// xn[t] = RMSNorm(x[t]) * w for t < M (bf16 rows of width H)
int launch_rows_rmsnorm(const uint16_t* x, const uint16_t* w, int M, int H, float eps, uint16_t* xn, hipStream_t st);
// softmax over the bf16 router logits, top-k (ties -> lower index), renormalised weights,
// and the per-expert pair lists
int launch_moe_route(const uint16_t* logits, int M, int E, int TK, const MoeRoute& rt, hipStream_t st);
// x[t] = bf16(x[t] + sum_kk wts[t TK + kk] * yd[t TK + kk]) in kk order; ss[t * (H / 16) + j]
// = sum of squares of the new row's 16-column tile j
int launch_moe_combine(uint16_t* x, const float* yd, const float* wts, int M, int TK, int H, float* ss, hipStream_t st);

size_t gemv_lds_bytes(int Mr, int kr, int MT);
void gemv_plan(const QLinear& L, int MT, int* kr, int* ksplit);
int gemv_launch(const GemvArgs& a, int MT, hipStream_t st);
// M > 64 tokens: every token tile of a block against each dequantised K-step (input rows
// already normalised: norm_w must be NULL)
int qgemm_launch(const GemvArgs& a, hipStream_t st);
// The next GEMV / GEMM kernel launched on this thread records its own start and end in
// these events (hipExtLaunchKernel: the kernel's execution, without the dispatch gap
// before it); consumed by that launch.  Profiled steps only.
void gemv_time_next_launch(hipEvent_t start, hipEvent_t stop);
// Its split-K plan (group pairs per K-range, K-ranges) for M tokens on `cus` CUs, and the
// workspace every M up to Mmax needs on the current device: partial floats and counters
// (zero when no plan splits).
void qgemm_plan(int NT, int GP, int M, int cus, int* kr, int* ksplit);
void qgemm_workspace(int NT, int GP, int Mmax, size_t* part_floats, int* counters);
int gemv_setup_lds();

int qlinear_repack(const QLinear& L, int row_off, int row_stride, int Nsrc, const uint32_t* wq_dev,
                   const uint16_t* s_dev, const uint16_t* b_dev, hipStream_t st);
int qlinear_export(const QLinear& L, int row_off, int row_stride, int Nsrc, uint32_t* wq_dev, uint16_t* s_dev,
                   uint16_t* b_dev, hipStream_t st);
int qlinear_synth(const QLinear& L, int row_off, int row_stride, int Nsrc, uint64_t base, int scale_exp,
                  hipStream_t st);

}  // namespace mc
