// mc_gemv.hip -- 4-bit affine (g64) dequant skinny GEMM for gfx950, plus the
// weight repack / synthetic-generation kernels for its tile layout.
//
// Y[M, N] = X[M, K] . W^T with W = s*q + b per group of 64 inputs (MLX affine
// quantisation, the `quantizedMatmul` every QuantizedLinear runs in the verify
// forward).  Bandwidth-bound at small M, so the design streams the packed weights
// once with 16-byte lane loads (1 KiB per wave per group pair), keeps X in LDS,
// and multiplies on the matrix cores:
//   * the nibbles become exact bf16 values 128 + q with one shift and one and-or
//     per pair (no int->float conversion),
//   * v_mfma_f32_16x16x32_bf16 computes sum_k x_k (128 + q_k) per group exactly
//     (bf16 products are exact in fp32),
//   * y += s * acc_g + (b - 128 s) * xsum_g folds the affine scale/bias per group,
//     with xsum_g = sum_k x_k precomputed once per block in LDS.
// Each output's reduction order depends only on (N, K) -- never on M -- so a
// token's result is bit-identical whether it is verified alone or with drafts.
#include "mc_gemv.hpp"

namespace mc {

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4;
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

__device__ inline bf16x8 dequant_word(uint32_t w) {
  u32x4 p;
  p.x = (w & 0x000F000Fu) | 0x43004300u;
  p.y = ((w >> 4) & 0x000F000Fu) | 0x43004300u;
  p.z = ((w >> 8) & 0x000F000Fu) | 0x43004300u;
  p.w = ((w >> 12) & 0x000F000Fu) | 0x43004300u;
  return __builtin_bit_cast(bf16x8, p);
}

__device__ inline float silu_f(float z) { return z / (1.0f + __expf(-z)); }

// LDS row stride (bf16 elements) of the X tile: +8 elements (16 B) of padding so
// the 16 lanes that read one k-slot block from 16 different rows spread over banks.
__host__ __device__ constexpr int xrow_stride(int gpr) { return gpr * 128 + 8; }

constexpr int GEMV_WAVES = 4;
constexpr int GEMV_LDS_LIMIT = 64 * 1024;

// One block = one 16-row tile x one K-range of `gpr` group pairs; its 4 waves take
// the range's group pairs round-robin (so the block streams one contiguous run of
// 1 KiB blocks), then reduce through LDS in wave order.  With ksplit > 1 the K-range
// partials go to a workspace and the last block of a tile sums them in kr order.
// X rows m < M are staged in LDS; lanes of columns m >= M read a zero row.
template <int MT>
__global__ void __launch_bounds__(256) qgemv_kernel(GemvArgs a) {
  extern __shared__ __align__(16) unsigned char smem[];
  const int gpr = a.gpr;
  const int XS = xrow_stride(gpr);
  const int Mr = a.M < 16 * MT ? a.M : 16 * MT;                           // staged rows
  uint16_t* xl = reinterpret_cast<uint16_t*>(smem);                        // [Mr + 1][XS]
  float* xsum = reinterpret_cast<float*>(smem + (size_t)(16 * MT + 1) * XS * 2);  // [16*MT + 1][2*gpr]
  float* red = xsum + (16 * MT + 1) * 2 * gpr;                             // [4 waves][MT][64][4]

  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int t = blockIdx.x, kr = blockIdx.y;
  const int gp0 = kr * gpr;
  const int gp1 = min(a.GP, gp0 + gpr);
  const int ngp = gp1 - gp0;
  const int k0 = gp0 * 128;
  const int ng = ngp * 2;

  // ---- stage X[0:Mr][k0 : k0 + ngp*128] and a zero row into LDS ----
  {
    const int cpr = ngp * 16;  // 16-byte chunks per row
    const int total = (Mr + 1) * cpr;
    for (int i = tid; i < total; i += 256) {
      const int m = i / cpr, ch = i - m * cpr;
      const int k = k0 + ch * 8;
      u32x4 v = {0u, 0u, 0u, 0u};
      if (m < Mr && k < a.K) v = *reinterpret_cast<const u32x4*>(a.x + (size_t)m * a.ldx + k);
      *reinterpret_cast<u32x4*>(xl + m * XS + ch * 8) = v;
    }
  }
  __syncthreads();
  for (int i = tid; i < (Mr + 1) * ng; i += 256) {
    const int m = i / ng, gl = i - m * ng;
    const uint16_t* p = xl + m * XS + gl * 64;
    float s0 = 0.f, s1 = 0.f, s2 = 0.f, s3 = 0.f;
#pragma unroll
    for (int k = 0; k < 64; k += 4) {
      s0 += bf16_to_f32(p[k]);
      s1 += bf16_to_f32(p[k + 1]);
      s2 += bf16_to_f32(p[k + 2]);
      s3 += bf16_to_f32(p[k + 3]);
    }
    xsum[m * ng + gl] = (s0 + s1) + (s2 + s3);
  }
  __syncthreads();

  const int c = lane >> 4, r16 = lane & 15;
  f32x4 acc[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) acc[mt] = (f32x4){0.f, 0.f, 0.f, 0.f};

  // column of this lane per m-tile: its staged row, or the zero row
  int xr[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) xr[mt] = (mt * 16 + r16 < Mr) ? (mt * 16 + r16) : Mr;

  const u32x4* qbase = reinterpret_cast<const u32x4*>(a.qw) + ((size_t)t * a.GP + gp0) * 64 + lane;
  const u32x4* sbase = reinterpret_cast<const u32x4*>(a.sb) + (((size_t)t * a.GP + gp0) * 4 + c) * 2;

  auto compute = [&](int j, const u32x4& nib, const u32x4& sc0, const u32x4& sc1) {
#pragma unroll
    for (int gi = 0; gi < 2; ++gi) {
      const bf16x8 wv0 = dequant_word(gi ? nib.z : nib.x);
      const bf16x8 wv1 = dequant_word(gi ? nib.w : nib.y);
      const u32x4 scv = gi ? sc1 : sc0;
      const int kl = j * 128 + gi * 64;
      const int gl = j * 2 + gi;
      float sv[4], bv[4];
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        sv[v] = bf16_to_f32((uint16_t)(scv[v] & 0xFFFFu));
        bv[v] = bf16_to_f32((uint16_t)(scv[v] >> 16)) - 128.0f * sv[v];
      }
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        const uint16_t* xrow = xl + xr[mt] * XS + kl + 8 * c;
        const bf16x8 xv0 = *reinterpret_cast<const bf16x8*>(xrow);
        const bf16x8 xv1 = *reinterpret_cast<const bf16x8*>(xrow + 32);
        f32x4 g = {0.f, 0.f, 0.f, 0.f};
        g = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wv0, xv0, g, 0, 0, 0);
        g = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wv1, xv1, g, 0, 0, 0);
        const float xs = xsum[xr[mt] * ng + gl];
#pragma unroll
        for (int v = 0; v < 4; ++v) acc[mt][v] += sv[v] * g[v] + bv[v] * xs;
      }
    }
  };

  // wave takes local group pairs j = wave, wave + 4, ...; two in flight
  {
    int j = wave;
    u32x4 nA = {0u, 0u, 0u, 0u}, sA0 = nA, sA1 = nA, nB = nA, sB0 = nA, sB1 = nA;
    if (j < ngp) {
      nA = __builtin_nontemporal_load(qbase + (size_t)j * 64);
      sA0 = sbase[(size_t)j * 8];
      sA1 = sbase[(size_t)j * 8 + 1];
    }
    while (j < ngp) {
      const int jn = j + GEMV_WAVES;
      if (jn < ngp) {
        nB = __builtin_nontemporal_load(qbase + (size_t)jn * 64);
        sB0 = sbase[(size_t)jn * 8];
        sB1 = sbase[(size_t)jn * 8 + 1];
      }
      compute(j, nA, sA0, sA1);
      j = jn;
      if (j >= ngp) break;
      const int jn2 = j + GEMV_WAVES;
      if (jn2 < ngp) {
        nA = __builtin_nontemporal_load(qbase + (size_t)jn2 * 64);
        sA0 = sbase[(size_t)jn2 * 8];
        sA1 = sbase[(size_t)jn2 * 8 + 1];
      }
      compute(j, nB, sB0, sB1);
      j = jn2;
    }
  }

  // ---- in-block reduction over the 4 waves, in wave order ----
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
    *reinterpret_cast<f32x4*>(red + ((wave * MT + mt) * 64 + lane) * 4) = acc[mt];
  __syncthreads();
  if (wave != 0) return;
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    f32x4 s = *reinterpret_cast<const f32x4*>(red + ((0 * MT + mt) * 64 + lane) * 4);
#pragma unroll
    for (int w = 1; w < GEMV_WAVES; ++w) s += *reinterpret_cast<const f32x4*>(red + ((w * MT + mt) * 64 + lane) * 4);
    acc[mt] = s;
  }

  // ---- cross-block split-K reduction (fixed order kr = 0..ksplit-1) ----
  if (a.ksplit > 1) {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      float* dst = a.part + ((((size_t)kr * a.NT + t) * MT + mt) * 64 + lane) * 4;
      *reinterpret_cast<f32x4*>(dst) = acc[mt];
    }
    __threadfence();
    unsigned arrived = 0u;
    if (lane == 0) arrived = atomicAdd(a.counters + t, 1u);
    arrived = __shfl(arrived, 0);
    if (arrived != (unsigned)(a.ksplit - 1)) return;
    __threadfence();
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[mt] = (f32x4){0.f, 0.f, 0.f, 0.f};
    for (int k2 = 0; k2 < a.ksplit; ++k2) {
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        const float* src = a.part + ((((size_t)k2 * a.NT + t) * MT + mt) * 64 + lane) * 4;
        acc[mt] += *reinterpret_cast<const f32x4*>(src);
      }
    }
    if (lane == 0) a.counters[t] = 0u;
  }

  // ---- epilogue: lane holds rows n = 16t + 4c + v (v = 0..3) of column m ----
  const int n0 = t * 16 + c * 4;
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int m = mt * 16 + r16;
    if (m >= a.M) continue;
    if (a.epi == EPI_SWIGLU) {
      // rows interleave (gate_i, up_i): outputs n0/2 and n0/2 + 1
      const int i0 = n0 >> 1;
      if (n0 + 1 < a.N) a.y[(size_t)m * a.ldy + i0] = f32_to_bf16(silu_f(acc[mt][0]) * acc[mt][1]);
      if (n0 + 3 < a.N) a.y[(size_t)m * a.ldy + i0 + 1] = f32_to_bf16(silu_f(acc[mt][2]) * acc[mt][3]);
    } else if (n0 + 3 < a.N) {
      uint16_t* yp = a.y + (size_t)m * a.ldy + n0;
      float o[4] = {acc[mt][0], acc[mt][1], acc[mt][2], acc[mt][3]};
      if (a.epi == EPI_RESIDUAL) {
        const uint2 old = *reinterpret_cast<const uint2*>(yp);
        o[0] += bf16_to_f32((uint16_t)(old.x & 0xFFFFu));
        o[1] += bf16_to_f32((uint16_t)(old.x >> 16));
        o[2] += bf16_to_f32((uint16_t)(old.y & 0xFFFFu));
        o[3] += bf16_to_f32((uint16_t)(old.y >> 16));
      }
      uint2 pk;
      pk.x = (uint32_t)f32_to_bf16(o[0]) | ((uint32_t)f32_to_bf16(o[1]) << 16);
      pk.y = (uint32_t)f32_to_bf16(o[2]) | ((uint32_t)f32_to_bf16(o[3]) << 16);
      *reinterpret_cast<uint2*>(yp) = pk;
    } else {
      for (int v = 0; v < 4; ++v) {
        const int n = n0 + v;
        if (n >= a.N) break;
        float o = acc[mt][v];
        if (a.epi == EPI_RESIDUAL) o += bf16_to_f32(a.y[(size_t)m * a.ldy + n]);
        a.y[(size_t)m * a.ldy + n] = f32_to_bf16(o);
      }
    }
  }
}

size_t gemv_lds_bytes(int MT, int gpr) {
  return (size_t)(16 * MT + 1) * xrow_stride(gpr) * 2 + (size_t)(16 * MT + 1) * gpr * 2 * 4 +
         (size_t)GEMV_WAVES * MT * 64 * 4 * 4;
}

// K-range plan for a shape.  Depends only on (N, K, MT): a token's reduction order
// never changes with the number of tokens in the same m-tile class.
void gemv_plan(const QLinear& L, int MT, int* gpr, int* ksplit) {
  int s = 1;
  // LDS must hold the K-range for the class's largest M
  while (gemv_lds_bytes(MT, (L.GP + s - 1) / s) > (size_t)GEMV_LDS_LIMIT) ++s;
  // at least ~640 blocks (2.5 per CU) and at least 4 group pairs per block
  while ((long)L.NT * s < 640 && (L.GP + s) / (s + 1) >= 4) ++s;
  *gpr = (L.GP + s - 1) / s;
  *ksplit = (L.GP + *gpr - 1) / *gpr;
}

int gemv_launch(const GemvArgs& a, int MT, hipStream_t st) {
  dim3 grid(a.NT, a.ksplit), block(256);
  const size_t lds = gemv_lds_bytes(MT, a.gpr);
  if (lds > (size_t)GEMV_LDS_LIMIT) return fail(MC_E_INVALID, "gemv: K-range exceeds LDS");
  if (a.M < 1 || a.M > 16 * MT) return fail(MC_E_INVALID, "gemv: M outside the m-tile class");
  switch (MT) {
    case 1: hipLaunchKernelGGL(qgemv_kernel<1>, grid, block, lds, st, a); break;
    case 2: hipLaunchKernelGGL(qgemv_kernel<2>, grid, block, lds, st, a); break;
    case 3: hipLaunchKernelGGL(qgemv_kernel<3>, grid, block, lds, st, a); break;
    case 4: hipLaunchKernelGGL(qgemv_kernel<4>, grid, block, lds, st, a); break;
    default: return fail(MC_E_INVALID, "gemv: unsupported m-tile count");
  }
  MC_HIP(hipGetLastError());
  return MC_OK;
}

int gemv_setup_lds() {
  MC_HIP(hipFuncSetAttribute((const void*)qgemv_kernel<1>, hipFuncAttributeMaxDynamicSharedMemorySize, GEMV_LDS_LIMIT));
  MC_HIP(hipFuncSetAttribute((const void*)qgemv_kernel<2>, hipFuncAttributeMaxDynamicSharedMemorySize, GEMV_LDS_LIMIT));
  MC_HIP(hipFuncSetAttribute((const void*)qgemv_kernel<3>, hipFuncAttributeMaxDynamicSharedMemorySize, GEMV_LDS_LIMIT));
  MC_HIP(hipFuncSetAttribute((const void*)qgemv_kernel<4>, hipFuncAttributeMaxDynamicSharedMemorySize, GEMV_LDS_LIMIT));
  return MC_OK;
}

// ---------------------------------------------------------------------------
// repack / export / synthetic generation
// ---------------------------------------------------------------------------
__device__ inline size_t tile_word_index(const QLinear& L, int nd, int kw) {
  const int t = nd >> 4, r = nd & 15;
  const int g = kw >> 3, w8 = kw & 7, am = w8 >> 2, c = w8 & 3;
  const int gp = g >> 1, gi = g & 1;
  const int lane = c * 16 + r;
  return (((size_t)t * L.GP + gp) * 64 + lane) * 4 + gi * 2 + am;
}
__device__ inline size_t tile_sb_index(const QLinear& L, int nd, int g) {
  const int t = nd >> 4, r = nd & 15, c = r >> 2, v = r & 3;
  const int gp = g >> 1, gi = g & 1;
  return (((size_t)t * L.GP + gp) * 4 + c) * 8 + gi * 4 + v;
}

__global__ void repack_kernel(QLinear L, int row_off, int row_stride, int Nsrc, const uint32_t* wq,
                              const uint16_t* s, const uint16_t* b) {
  const int KW = L.K / 8, G = L.K / 64;
  const size_t total = (size_t)Nsrc * KW;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (size_t)gridDim.x * blockDim.x) {
    const int n = (int)(i / KW), kw = (int)(i % KW);
    const int nd = row_off + n * row_stride;
    L.qw[tile_word_index(L, nd, kw)] = permute_mlx_word(wq[i]);
    if (kw < G) {
      const size_t si = (size_t)n * G + kw;
      L.sb[tile_sb_index(L, nd, kw)] = (uint32_t)s[si] | ((uint32_t)b[si] << 16);
    }
  }
}

__global__ void export_kernel(QLinear L, int row_off, int row_stride, int Nsrc, uint32_t* wq, uint16_t* s,
                              uint16_t* b) {
  const int KW = L.K / 8, G = L.K / 64;
  const size_t total = (size_t)Nsrc * KW;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (size_t)gridDim.x * blockDim.x) {
    const int n = (int)(i / KW), kw = (int)(i % KW);
    const int nd = row_off + n * row_stride;
    wq[i] = unpermute_tile_word(L.qw[tile_word_index(L, nd, kw)]);
    if (kw < G) {
      const uint32_t v = L.sb[tile_sb_index(L, nd, kw)];
      s[(size_t)n * G + kw] = (uint16_t)(v & 0xFFFFu);
      b[(size_t)n * G + kw] = (uint16_t)(v >> 16);
    }
  }
}

__global__ void synth_kernel(QLinear L, int row_off, int row_stride, int Nsrc, uint64_t base, int scale_exp) {
  const int KW = L.K / 8, G = L.K / 64;
  const size_t total = (size_t)Nsrc * KW;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (size_t)gridDim.x * blockDim.x) {
    const int n = (int)(i / KW), kw = (int)(i % KW);
    const int nd = row_off + n * row_stride;
    L.qw[tile_word_index(L, nd, kw)] = permute_mlx_word(synth_mlx_word(base, n, KW, kw));
    if (kw < G) L.sb[tile_sb_index(L, nd, kw)] = synth_scale_bias(base, n, G, kw, scale_exp);
  }
}

static dim3 grid_for(size_t total) {
  size_t b = (total + 255) / 256;
  if (b > 65535 * 4) b = 65535 * 4;
  if (b < 1) b = 1;
  return dim3((unsigned)b);
}

int qlinear_repack(const QLinear& L, int row_off, int row_stride, int Nsrc, const uint32_t* wq_dev,
                   const uint16_t* s_dev, const uint16_t* b_dev, hipStream_t st) {
  hipLaunchKernelGGL(repack_kernel, grid_for((size_t)Nsrc * (L.K / 8)), dim3(256), 0, st, L, row_off, row_stride,
                     Nsrc, wq_dev, s_dev, b_dev);
  MC_HIP(hipGetLastError());
  return MC_OK;
}

int qlinear_export(const QLinear& L, int row_off, int row_stride, int Nsrc, uint32_t* wq_dev, uint16_t* s_dev,
                   uint16_t* b_dev, hipStream_t st) {
  hipLaunchKernelGGL(export_kernel, grid_for((size_t)Nsrc * (L.K / 8)), dim3(256), 0, st, L, row_off, row_stride,
                     Nsrc, wq_dev, s_dev, b_dev);
  MC_HIP(hipGetLastError());
  return MC_OK;
}

int qlinear_synth(const QLinear& L, int row_off, int row_stride, int Nsrc, uint64_t base, int scale_exp,
                  hipStream_t st) {
  hipLaunchKernelGGL(synth_kernel, grid_for((size_t)Nsrc * (L.K / 8)), dim3(256), 0, st, L, row_off, row_stride,
                     Nsrc, base, scale_exp);
  MC_HIP(hipGetLastError());
  return MC_OK;
}

}  // namespace mc
