// mc_gemv.hpp -- dequant GEMV launch interface (kernels in mc_gemv.hip).
#pragma once
#include "mc_common.hpp"

namespace mc {

enum Epi { EPI_STORE = 0, EPI_RESIDUAL = 1, EPI_SWIGLU = 2 };

struct GemvArgs {
  const uint32_t* qw = nullptr;  // tile-layout nibbles
  const uint32_t* sb = nullptr;  // tile-layout scale|bias
  const uint16_t* x = nullptr;   // [M][ldx] bf16
  int ldx = 0;
  uint16_t* y = nullptr;         // [M][ldy] bf16 (EPI_RESIDUAL: read-modify-write)
  int ldy = 0;
  int M = 0, N = 0, K = 0, NT = 0, GP = 0;
  int gpr = 0, ksplit = 1;
  float* part = nullptr;         // split-K partials [ksplit][NT][MT][64][4]
  unsigned* counters = nullptr;  // [NT], zero at rest
  int epi = EPI_STORE;
};

size_t gemv_lds_bytes(int MT, int gpr);
void gemv_plan(const QLinear& L, int MT, int* gpr, int* ksplit);
int gemv_launch(const GemvArgs& a, int MT, hipStream_t st);
int gemv_setup_lds();

int qlinear_repack(const QLinear& L, int row_off, int row_stride, int Nsrc, const uint32_t* wq_dev,
                   const uint16_t* s_dev, const uint16_t* b_dev, hipStream_t st);
int qlinear_export(const QLinear& L, int row_off, int row_stride, int Nsrc, uint32_t* wq_dev, uint16_t* s_dev,
                   uint16_t* b_dev, hipStream_t st);
int qlinear_synth(const QLinear& L, int row_off, int row_stride, int Nsrc, uint64_t base, int scale_exp,
                  hipStream_t st);

}  // namespace mc
