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
  const uint16_t* norm_w = nullptr;  // non-null: the input is RMSNorm(x) * norm_w over the full row,
  float eps = 0.f;                   //   whose sum of squares is sum_t ss_in[t * ss_ld + m], t < ss_nt
  const float* ss_in = nullptr;
  int ss_nt = 0, ss_ld = 0;
  float* ss_out = nullptr;           // EPI_RESIDUAL: per-tile sums of squares of the new rows,
  int ss_ld_out = 0;                 //   ss_out[t * ss_ld_out + m] (NULL = skip)
  uint16_t* y = nullptr;             // [M][ldy] bf16 (EPI_RESIDUAL: read-modify-write)
  int ldy = 0;
  int M = 0, N = 0, K = 0, NT = 0, GP = 0;
  int kr = 0, ksplit = 1;            // group pairs per K-range, K-ranges
  float* part = nullptr;             // split-K partials [ksplit][NT][MT][64][4]
  unsigned* counters = nullptr;      // [NT], zero at rest
  int epi = EPI_STORE;
  uint32_t dq_mask = 0x000F000Fu, dq_magic = 0x43004300u;  // nibble-pair -> bf16 (128 + q) constants
};

size_t gemv_lds_bytes(int Mr, int kr, int MT);
void gemv_plan(const QLinear& L, int MT, int* kr, int* ksplit);
int gemv_launch(const GemvArgs& a, int MT, hipStream_t st);
int gemv_setup_lds();

int qlinear_repack(const QLinear& L, int row_off, int row_stride, int Nsrc, const uint32_t* wq_dev,
                   const uint16_t* s_dev, const uint16_t* b_dev, hipStream_t st);
int qlinear_export(const QLinear& L, int row_off, int row_stride, int Nsrc, uint32_t* wq_dev, uint16_t* s_dev,
                   uint16_t* b_dev, hipStream_t st);
int qlinear_synth(const QLinear& L, int row_off, int row_stride, int Nsrc, uint64_t base, int scale_exp,
                  hipStream_t st);

}  // namespace mc
