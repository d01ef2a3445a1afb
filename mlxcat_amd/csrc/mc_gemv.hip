// mc_gemv.hip -- 4-bit affine (g64) dequant skinny GEMM for gfx950, plus the
// weight repack / synthetic-generation kernels for its tile layout.
//
// Y[M, N] = X[M, K] . W^T with W = s*q + b per group of 64 inputs (MLX affine
// quantisation, the `quantizedMatmul` every QuantizedLinear runs in the verify
// forward).  At verify sizes (M = rows x (K+1) <= 64) the op is bound by streaming
// the packed weights from HBM, so the kernel is built around memory-level
// parallelism:
//   * one block = one 16-row tile x one K-range; each wave issues every 16-byte
//     weight load it will need (up to 5 group pairs = 5 KiB per wave) before it
//     touches anything else, so a CU keeps tens of KiB in flight;
//   * the activations of the K-range are staged in LDS while the weights are in
//     flight; an optional RMSNorm over the full input row is fused into that staging;
//   * nibbles become exact bf16 values 128 + q with one shift and one and-or per
//     pair, and v_mfma_f32_16x16x32_bf16 forms sum_k x_k (128 + q_k) per group;
//     y += s * acc + (b - 128 s) * sum_k x_k folds in the affine scale/bias;
//   * split-K partials travel through device-coherent (sc1) stores and loads with
//     an arrival counter per tile, so no L2 writeback/invalidate fence is needed;
//     the last-arriving block reduces them in K-range order and runs the epilogue
//     (store, residual add, or SwiGLU of interleaved gate/up rows).
// For M <= 64 the K-range plan depends only on (N, K) and the M class (M <= 16 or
// M <= 64), and every reduction runs in a fixed order, so a token's result is
// bit-identical whatever the number of tokens in the launch within its class.  The
// M > 64 GEMM's split-K plan depends on M (and the CU count), and the attention's split
// on the batch's rows and capacity, so across batch shapes results agree to rounding,
// not bit for bit.
#include "mc_gemv.hpp"

#ifndef MC_EMULATE
#include <hip/hip_ext.h>
#endif

#include <algorithm>

namespace mc {

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4;
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

// mask = DQ_MASK, magic = DQ_MAGIC, passed in registers so that each pair becomes a shift
// and one v_and_or_b32 (VOP3 takes no literal operands on this architecture)
__device__ inline bf16x8 dequant_word(uint32_t w, uint32_t mask, uint32_t magic) {
  u32x4 p;
  p.x = ((w << 3) & mask) | magic;
  p.y = ((w >> 1) & mask) | magic;
  p.z = ((w >> 5) & mask) | magic;
  p.w = ((w >> 9) & mask) | magic;
  return __builtin_bit_cast(bf16x8, p);
}

__device__ inline float silu_f(float z) { return z / (1.0f + __expf(-z)); }

// Workgroup barrier for LDS traffic only: waits for this wave's LDS operations, not for
// its outstanding global loads (__syncthreads would also drain the prefetched weights).
__device__ inline void lds_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0), vmcnt/expcnt unconstrained
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// LDS row stride (bf16 elements) of the X tile: +8 elements (16 B) of padding so the
// 16 lanes that read one k-slot block from 16 different rows spread over banks.
__host__ __device__ constexpr int xrow_stride(int kr) { return kr * 128 + 8; }

// A raw buffer over n bytes at p: a load at an offset past n returns zero (the hardware's
// range check), so a masked-off load needs no branch and no wait of its own.
__device__ inline __amdgpu_buffer_rsrc_t buf_rsrc(const void* p, int n) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, n, 0x00020000);
}
constexpr unsigned NOWHERE = 0x80000000u;  // a buffer offset past every range used here

constexpr int GEMV_WAVES = 4;
constexpr int GEMV_LDS_LIMIT = 160 * 1024;

size_t gemv_lds_bytes(int Mr, int kr, int MT) {
  return (size_t)Mr * xrow_stride(kr) * 2 + (size_t)16 * MT * 2 * kr * 4 + (size_t)2 * GEMV_WAVES * MT * 64 * 16 +
         64 * 4 + (size_t)kr * 128 * 2;
}

// Weight registers of one work unit (tile x K-range) for one wave: D group pairs.
template <int D>
struct WBuf {
  u32x4 nib[D];
  uint2 sb[D];  // (scale | bias << 16) of this lane's weight row, groups 2gp and 2gp + 1
};

// Pairs wave + WS i of the unit (WS = 1: all of them, for a wave that owns the unit).
template <int D, int WS = GEMV_WAVES>
__device__ inline void load_unit(WBuf<D>& w, const GemvArgs& a, int t, int gp0, int ngp, int wave, int lane, int r16) {
  const u32x4* qbase = reinterpret_cast<const u32x4*>(a.qw) + ((size_t)t * a.GP + gp0) * 64 + lane;
  const uint2* sbase = reinterpret_cast<const uint2*>(a.sb) + tile_sb_word(t, r16, gp0, 0, a.GP) / 2;
#pragma unroll
  for (int i = 0; i < D; ++i) {
    const int j = min(wave + WS * i, ngp - 1);  // a short K-range re-reads its last pair
    w.nib[i] = __builtin_nontemporal_load(qbase + (size_t)j * 64);
    w.sb[i] = sbase[j];
  }
}

// Sum over this wave's group pairs of one unit.  The activations are the MFMA's A
// operand (rows = tokens) and the weights its B operand (columns = weight rows), so lane
// (c, r16) ends with tokens mt*16 + 4c + v (v = 0..3) of weight row 16t + r16 and applies
// one row's scale and bias.  xsum is laid out [group][16 * MT tokens].
template <int MT, int D, int WS = GEMV_WAVES>
__device__ inline void compute_unit(f32x4 (&acc)[MT], const WBuf<D>& w, const uint16_t* xl, const float* xsum, int XS,
                                    int Mr, int ngp, int wave, int c, int r16, uint32_t mask, uint32_t magic) {
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) acc[mt] = (f32x4){0.f, 0.f, 0.f, 0.f};
  // per group pair: every LDS read of its groups and MT token tiles first, then all their
  // MFMAs (independent chains back to back), then the scalings in the order of one
  // element's sum (group 2j, then 2j + 1), so a tile's FMAs do not wait on its own fresh
  // MFMA result while the other tiles' reads are still to go.  At MT = 4 (registers) one
  // group and token tile at a time, in the same order.
  constexpr int GB = MT >= 4 ? 1 : 2;
  constexpr int TB = MT >= 4 ? 1 : MT;  // token tiles per batch
#pragma unroll
  for (int i = 0; i < D; ++i) {
    const int j = wave + WS * i;
    if (j >= ngp) break;
#pragma unroll
    for (int g0 = 0; g0 < 2; g0 += GB)
#pragma unroll
    for (int t0 = 0; t0 < MT; t0 += TB) {
      bf16x8 xv[GB][TB][2];
      f32x4 xs[GB][TB];
#pragma unroll
      for (int b = 0; b < GB; ++b) {
        const int gi = g0 + b;
        const int kl = j * 128 + gi * 64;
        const int gl = j * 2 + gi;
#pragma unroll
        for (int tb = 0; tb < TB; ++tb) {
          const int mt = t0 + tb;
          // token rows >= M read row Mr - 1: finite values whose results are never stored
          const int m = min(mt * 16 + r16, Mr - 1);
          const uint16_t* xrow = xl + m * XS + kl + 8 * c;
          xv[b][tb][0] = *reinterpret_cast<const bf16x8*>(xrow);
          xv[b][tb][1] = *reinterpret_cast<const bf16x8*>(xrow + 32);
          xs[b][tb] = *reinterpret_cast<const f32x4*>(xsum + gl * 16 * MT + mt * 16 + 4 * c);
        }
      }
      f32x4 g[GB][TB];
      float sv[GB], bv[GB];
#pragma unroll
      for (int b = 0; b < GB; ++b) {
        const int gi = g0 + b;
        const bf16x8 wv0 = dequant_word(gi ? w.nib[i].z : w.nib[i].x, mask, magic);
        const bf16x8 wv1 = dequant_word(gi ? w.nib[i].w : w.nib[i].y, mask, magic);
        const uint32_t sbv = gi ? w.sb[i].y : w.sb[i].x;
        sv[b] = DQ_STEP * __uint_as_float(sbv << 16);
        bv[b] = __uint_as_float(sbv & 0xFFFF0000u) - sv[b];
#pragma unroll
        for (int tb = 0; tb < TB; ++tb) {
          g[b][tb] = (f32x4){0.f, 0.f, 0.f, 0.f};
          g[b][tb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xv[b][tb][0], wv0, g[b][tb], 0, 0, 0);
          g[b][tb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xv[b][tb][1], wv1, g[b][tb], 0, 0, 0);
        }
      }
#pragma unroll
      for (int b = 0; b < GB; ++b)
#pragma unroll
        for (int tb = 0; tb < TB; ++tb)
#pragma unroll
          for (int v = 0; v < 4; ++v) {
            acc[t0 + tb][v] = __builtin_fmaf(sv[b], g[b][tb][v], acc[t0 + tb][v]);
            acc[t0 + tb][v] = __builtin_fmaf(bv[b], xs[b][tb][v], acc[t0 + tb][v]);
          }
    }
  }
}

// Sum of the 4 waves' unit results, in wave order.
template <int MT>
__device__ inline void reduce_waves(f32x4 (&acc)[MT], const float* red, int lane) {
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    f32x4 sacc = *reinterpret_cast<const f32x4*>(red + ((0 * MT + mt) * 64 + lane) * 4);
#pragma unroll
    for (int w = 1; w < GEMV_WAVES; ++w) sacc += *reinterpret_cast<const f32x4*>(red + ((w * MT + mt) * 64 + lane) * 4);
    acc[mt] = sacc;
  }
}

// The epilogue of one tile: lane holds tokens m = mt*16 + 4c + v of weight row n = 16t + r16.
// Loads and cross-lane sums of the tile's tokens are issued all together (a token past M
// reads row 0 and drops it): a load or a reduction under a per-token condition becomes a
// branch with its own wait, and the tokens would take one round trip after another.
// The residual rows a tile's EPI_RESIDUAL epilogue adds to (row 0 for a token past M).
template <int MT>
__device__ inline void load_residual(const GemvArgs& a, int t, int c, int r16, uint16_t (&old)[MT][4]) {
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int m = mt * 16 + 4 * c + v;
      old[mt][v] = a.y[(size_t)(m < a.M ? m : 0) * a.ldy + t * 16 + r16];
    }
}

// old: the tile's residual rows (load_residual) when EPI_RESIDUAL, else unused.
template <int MT>
__device__ inline void epilogue_with(const GemvArgs& a, const f32x4 (&acc)[MT], int t, int c, int r16,
                                     const uint16_t (&old)[MT][4]) {
  const int n = t * 16 + r16;
  if (a.epi == EPI_SWIGLU) {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int m = mt * 16 + 4 * c + v;
        // rows interleave (gate_i, up_i): the even lane takes up_i from its odd neighbour
        const float up = __shfl_xor(acc[mt][v], 1);
        if (m < a.M && !(r16 & 1) && n + 1 < a.N) a.y[(size_t)m * a.ldy + (n >> 1)] = f32_to_bf16(silu_f(acc[mt][v]) * up);
      }
  } else if (a.epi == EPI_RESIDUAL) {
    // residual add, and this tile's sum of squares of the new rows for the next RMSNorm
    // (N % 16 == 0 here: the hidden size)
    float q[MT][4];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int m = mt * 16 + 4 * c + v;
        const uint16_t h = f32_to_bf16(acc[mt][v] + bf16_to_f32(old[mt][v]));
        const float rr = bf16_to_f32(h);
        q[mt][v] = m < a.M ? rr * rr : 0.f;
        if (m < a.M) a.y[(size_t)m * a.ldy + n] = h;
      }
#pragma unroll
    for (int o = 1; o < 16; o <<= 1)
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int v = 0; v < 4; ++v) q[mt][v] += __shfl_xor(q[mt][v], o);
    if (a.ss_out && r16 == 0)
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const int m = mt * 16 + 4 * c + v;
          if (m < a.M) a.ss_out[(size_t)m * a.ss_ld_out + t] = q[mt][v];
        }
  } else {
    unsigned key[MT][4];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int m = mt * 16 + 4 * c + v;
        const bool live = m < a.M && n < a.N;
        const uint16_t h = f32_to_bf16(acc[mt][v]);
        if (live) a.y[(size_t)m * a.ldy + n] = h;
        // tile argmax over 16 rows: 32-bit key (value key << 16 | 15 - row), lowest row on ties
        key[mt][v] = live ? (bf16_order_key(h) << 16) | (unsigned)(15 - r16) : 0u;
      }
    if (a.amax) {
#pragma unroll
      for (int o = 1; o < 16; o <<= 1)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
          for (int v = 0; v < 4; ++v) key[mt][v] = max(key[mt][v], (unsigned)__shfl_xor((int)key[mt][v], o));
      if (r16 == 0)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
          for (int v = 0; v < 4; ++v) {
            const int m = mt * 16 + 4 * c + v;
            const unsigned k = key[mt][v];
            if (m < a.M && k)
              a.amax[(size_t)m * a.NT + t] =
                  ((unsigned long long)(k >> 16) << 32) | (0xFFFFFFFFull - (unsigned)(t * 16 + 15 - (int)(k & 15u)));
          }
    }
  }
}

template <int MT>
__device__ inline void epilogue(const GemvArgs& a, const f32x4 (&acc)[MT], int t, int c, int r16) {
  uint16_t old[MT][4] = {};
  if (a.epi == EPI_RESIDUAL) load_residual<MT>(a, t, c, r16, old);
  epilogue_with<MT>(a, acc, t, c, r16, old);
}

// Device-coherent partial of unit (t, kr); no wait here (the arrival is counted later).
template <int MT>
__device__ inline void store_partial(const GemvArgs& a, const f32x4 (&acc)[MT], int t, int kr, int lane) {
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    float* dst = a.part + ((((size_t)kr * a.NT + t) * MT + mt) * 64 + lane) * 4;
    st_coherent(dst, acc[mt][0], acc[mt][1]);
    st_coherent(dst + 2, acc[mt][2], acc[mt][3]);
  }
}

// Count this wave's arrival for tile t (its partial stores are complete); the last of the
// ksplit arrivals sums the partials in K-range order and runs the epilogue.
// The last arrival of tile t: sum its partials in K-range order, rearm the counter, epilogue.
template <int MT>
__device__ inline void finish_tile(const GemvArgs& a, int t, int lane, int c, int r16) {
  f32x4 acc[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) acc[mt] = (f32x4){0.f, 0.f, 0.f, 0.f};
  // the residual rows go out with the first partials (one round trip for both; at MT = 4
  // after them, for registers)
  uint16_t old[MT][4] = {};
  if constexpr (MT <= 3)
    if (a.epi == EPI_RESIDUAL) load_residual<MT>(a, t, c, r16, old);
  // the partials of KB K-ranges are loaded together (one memory round trip per KB ranges,
  // not per range: the tail of a launch is its last tile's reduction), then summed in
  // K-range order; ranges past the last are neither loaded nor summed
  constexpr int KB = MT == 1 ? 8 : 4;
  for (int k0 = 0; k0 < a.ksplit; k0 += KB) {
    float2 p[KB][MT][2];
#pragma unroll
    for (int j = 0; j < KB; ++j) {
      const int k2 = k0 + j;
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        const float* src = a.part + ((((size_t)k2 * a.NT + t) * MT + mt) * 64 + lane) * 4;
        p[j][mt][0] = p[j][mt][1] = make_float2(0.f, 0.f);
        if (k2 < a.ksplit) {
          p[j][mt][0] = ld_coherent(src);
          p[j][mt][1] = ld_coherent(src + 2);
        }
      }
    }
#pragma unroll
    for (int j = 0; j < KB; ++j) {
      if (k0 + j >= a.ksplit) break;
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        acc[mt][0] += p[j][mt][0].x;
        acc[mt][1] += p[j][mt][0].y;
        acc[mt][2] += p[j][mt][1].x;
        acc[mt][3] += p[j][mt][1].y;
      }
    }
  }
  if (lane == 0) __hip_atomic_store(a.counters + t, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  if constexpr (MT > 3)
    if (a.epi == EPI_RESIDUAL) load_residual<MT>(a, t, c, r16, old);
  epilogue_with<MT>(a, acc, t, c, r16, old);
}

// Ordering of the split-K hand-over.  A K-range's partials are agent-scope (sc1) stores,
// which gfx950 writes through to memory; the writer waits for them (s_waitcnt vmcnt(0)
// after a workgroup release fence) before its relaxed agent-scope atomicAdd on the tile's
// counter, so the partials are in memory when the counter moves.  The last arriver learns
// it is last from the atomic's returned value (the wave waits for it before the branch),
// and only then loads the partials, again with agent-scope (sc1) loads, which read memory
// rather than a possibly stale L2 line, so no cache invalidation is needed on that path.
// What the relaxed atomics alone do not promise is the compiler's order: the memory
// clobber after the branch keeps the partial loads below the atomic.  (An agent-scope
// acquire fence there would say the same in the memory model's terms, but it also emits an
// L2 invalidate per finished tile, measured at +6% on the batch-1 verify step.)
template <int MT>
__device__ inline void arrive(const GemvArgs& a, int t, int lane, int c, int r16) {
  unsigned arrived = 0u;
  if (lane == 0) arrived = atomicAdd(a.counters + t, 1u);
  arrived = __shfl(arrived, 0);
  if (arrived != (unsigned)(a.ksplit - 1)) return;
  MC_FENCE();
  finish_tile<MT>(a, t, lane, c, r16);
}

// Arrivals of a wave's units t0, t0 + ts, ... < NT, 64 at a time: lane i counts unit i (the
// atomics of all units are in flight together), then the wave finishes the tiles whose
// last arrival it was.
template <int MT>
__device__ inline void arrive_units(const GemvArgs& a, int t0, int ts, int lane, int c, int r16) {
  for (int b = t0; b < a.NT; b += 64 * ts) {
    const int t = b + lane * ts;
    unsigned arrived = 0u;
    if (t < a.NT) arrived = atomicAdd(a.counters + t, 1u);
    unsigned long long last = __ballot(t < a.NT && arrived == (unsigned)(a.ksplit - 1));
    MC_FENCE();  // the partial loads stay below the atomics, as in arrive()
    while (last) {
      const int i = __ffsll((long long)last) - 1;
      last &= last - 1;
      finish_tile<MT>(a, b + i * ts, lane, c, r16);
    }
  }
}

// U work units per block: unit u = tile (u / ksplit) x K-range (u % ksplit); block b takes
// u = b, b + G, ..., b + (U-1) G with G % ksplit == 0, so its K-range -- and the
// activations it stages in LDS -- never change.  The next unit's weights are in flight
// while the current one is computed; the steps are unrolled (straight-line code) and
// every prefetch is unconditional (a block past the end re-reads the last unit), so the
// compiler's load counters keep the prefetch outstanding during the compute.
template <int MT, int D, int U>
__global__ void __launch_bounds__(256) qgemv_kernel(GemvArgs a) {
  MC_DYN_LDS(smem);
  const int kr_gp = a.kr;
  const int XS = xrow_stride(kr_gp);
  const int Mr = min(a.M, 16 * MT);
  uint16_t* xl = reinterpret_cast<uint16_t*>(smem);                                   // [Mr][XS]
  float* xsum = reinterpret_cast<float*>(smem + (size_t)Mr * XS * 2);                 // [2 kr][16 MT]
  float* red = xsum + 16 * MT * 2 * kr_gp;                                            // [2][4][MT][64][4]
  float* rs = red + 2 * GEMV_WAVES * MT * 64 * 4;                                      // [64] row scales
  uint16_t* wl = reinterpret_cast<uint16_t*>(rs + 64);                                 // [kr * 128] norm weights

  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int G = gridDim.x, ks = a.ksplit, nunits = a.NT * ks;
  const int kr = blockIdx.x % ks;
  const int gp0 = kr * kr_gp;
  const int ngp = min(a.GP, gp0 + kr_gp) - gp0;
  const int k0 = gp0 * 128;
  const int ng = ngp * 2;
  const int c = lane >> 4, r16 = lane & 15;

  // ---- 1. small loads first (vmcnt retires in order): norm partials and weights, X ----
  // row scale of the fused RMSNorm, r[m] = 1 / sqrt(mean(x^2) + eps): wave w reduces rows
  // w, w + 4, ... over the producer's per-tile sums of squares, lane l taking tiles
  // l, l + 64, ... (fixed order)
  // Every load of this section is issued unconditionally through a range-checked buffer (a
  // masked-off element reads offset NOWHERE, i.e. zero): no branch around a load, so the
  // activations and the first weights are in flight within a few hundred cycles of the
  // block's start.
  constexpr int RW = MT * 4;         // rows per wave, at most
  constexpr int SL = 4;              // producer tiles per lane, at most (ss_nt <= 256)
  const bool has_norm = a.norm_w != nullptr;
  const __amdgpu_buffer_rsrc_t rss = buf_rsrc(a.ss_in, has_norm ? Mr * a.ss_ld * 4 : 0);
  float ssv[RW][SL];
#pragma unroll
  for (int r = 0; r < RW; ++r)
#pragma unroll
    for (int q = 0; q < SL; ++q) {
      const int m = wave + GEMV_WAVES * r, tt = lane + 64 * q;
      const unsigned off = (has_norm && m < Mr && tt < a.ss_nt) ? (unsigned)((m * a.ss_ld + tt) * 4) : NOWHERE;
      ssv[r][q] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rss, off, 0, 0));
    }
  constexpr int XCH = 8;             // 16-byte X chunks per thread per pass
  const int cpr = ngp * 16;          // chunks per row in this K-range
  u32x4 nw[2];                       // norm weights of the K-range (cpr <= 320 chunks)
  const __amdgpu_buffer_rsrc_t rnw = buf_rsrc(a.norm_w, has_norm ? a.K * 2 : 0);
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    const int k = k0 + (tid + 256 * q) * 8;
    const unsigned off = (has_norm && tid + 256 * q < cpr && k < a.K) ? (unsigned)(k * 2) : NOWHERE;
    nw[q] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rnw, off, 0, 0));
  }
  const int xtotal = Mr * cpr;
  // chunk i of the K-range's activations is row i / cpr, chunk i % cpr: the quotient by a
  // multiply-high with ceil(2^32 / cpr), exact for i * cpr < 2^32 (i < 16 MT cpr <= 20480)
  const unsigned cpr_magic = 0xFFFFFFFFu / (unsigned)cpr + 1u;
  auto row_of = [&](int i) { return (int)__umulhi((unsigned)i, cpr_magic); };
  const __amdgpu_buffer_rsrc_t rx = buf_rsrc(a.x, Mr * a.ldx * 2);
  u32x4 xv[XCH];
#pragma unroll
  for (int q = 0; q < XCH; ++q) {
    const int i = tid + 256 * q;
    const int m = row_of(i), ch = i - m * cpr;
    const unsigned off = (i < xtotal && k0 + ch * 8 < a.K) ? (unsigned)((m * a.ldx + k0 + ch * 8) * 2) : NOWHERE;
    xv[q] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rx, off, 0, 0));
  }

  // ---- 2. the first unit's weights ----
  int u = blockIdx.x;
  WBuf<D> wa, wb;
  load_unit<D>(wa, a, min(u, nunits - 1) / ks, gp0, ngp, wave, lane, r16);

  // ---- 3. row scales and norm weights, then X (normalised) into LDS while the weights are
  // in flight ----
  if (has_norm) {
#pragma unroll
    for (int q = 0; q < 2; ++q)
      if (tid + 256 * q < cpr) *reinterpret_cast<u32x4*>(wl + (tid + 256 * q) * 8) = nw[q];
    // the RW rows' butterflies interleaved, each in its fixed order (a branch between them
    // would serialise their LDS round trips)
    float q[RW];
#pragma unroll
    for (int r = 0; r < RW; ++r) {
      q[r] = 0.f;
#pragma unroll
      for (int v = 0; v < SL; ++v) q[r] += ssv[r][v];
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1)
#pragma unroll
      for (int r = 0; r < RW; ++r) q[r] += __shfl_xor(q[r], o);
    if (lane == 0)
#pragma unroll
      for (int r = 0; r < RW; ++r) {
        const int m = wave + GEMV_WAVES * r;
        if (m < Mr) rs[m] = 1.0f / sqrtf(q[r] / (float)a.K + a.eps);
      }
    lds_barrier();
  }
  // Staging in phases over SB chunks at a time (LDS reads, normalise, LDS stores, group sums,
  // cross-lane sums, xsum stores) so that the LDS latencies of the chunks overlap.
  constexpr int SB = 4;
  auto stage = [&](int base) {
#pragma unroll
    for (int q0 = 0; q0 < XCH; q0 += SB) {
      int mm[SB], cc[SB];
      bool in[SB];
#pragma unroll
      for (int j = 0; j < SB; ++j) {
        const int i = base + tid + 256 * (q0 + j);
        in[j] = i < xtotal;
        mm[j] = row_of(i);
        cc[j] = i - mm[j] * cpr;
      }
      if (a.norm_w) {
        float rr[SB];
        u32x4 ww[SB];
#pragma unroll
        for (int j = 0; j < SB; ++j) {
          rr[j] = in[j] ? rs[mm[j]] : 0.f;
          ww[j] = in[j] ? *reinterpret_cast<const u32x4*>(wl + cc[j] * 8) : (u32x4){0u, 0u, 0u, 0u};
        }
        // bf16((x * r) * w): the rounding of a standalone RMSNorm
#pragma unroll
        for (int j = 0; j < SB; ++j)
#pragma unroll
          for (int h = 0; h < 4; ++h) {
            u32x4& v = xv[q0 + j];
            const float lo = (__uint_as_float(v[h] << 16) * rr[j]) * __uint_as_float(ww[j][h] << 16);
            const float hi = (__uint_as_float(v[h] & 0xFFFF0000u) * rr[j]) * __uint_as_float(ww[j][h] & 0xFFFF0000u);
            v[h] = (uint32_t)f32_to_bf16(lo) | ((uint32_t)f32_to_bf16(hi) << 16);
          }
      }
#pragma unroll
      for (int j = 0; j < SB; ++j)
        if (in[j]) *reinterpret_cast<u32x4*>(xl + mm[j] * XS + cc[j] * 8) = xv[q0 + j];
      // group sum of X: the 8 chunks of a 64-wide group sit in 8 consecutive lanes (cpr is
      // a multiple of 16), reduced in a fixed order
      float gs[SB];
#pragma unroll
      for (int j = 0; j < SB; ++j) {
        float s0 = 0.f, s1 = 0.f;
#pragma unroll
        for (int h = 0; h < 4; ++h) {
          s0 += __uint_as_float(xv[q0 + j][h] << 16);
          s1 += __uint_as_float(xv[q0 + j][h] & 0xFFFF0000u);
        }
        gs[j] = in[j] ? s0 + s1 : 0.f;
      }
#pragma unroll
      for (int j = 0; j < SB; ++j) gs[j] = sum8_lanes(gs[j]);
#pragma unroll
      for (int j = 0; j < SB; ++j)
        if (in[j] && (cc[j] & 7) == 0) xsum[(cc[j] >> 3) * 16 * MT + mm[j]] = gs[j];
    }
  };
  stage(0);
  if (xtotal > 256 * XCH) {  // rare (large M x K-range): further passes, which also wait for the weights
    for (int base = 256 * XCH; base < xtotal; base += 256 * XCH) {
#pragma unroll
      for (int q = 0; q < XCH; ++q) {
        const int i = base + tid + 256 * q;
        xv[q] = (u32x4){0u, 0u, 0u, 0u};
        if (i < xtotal) {
          const int m = row_of(i), ch = i - m * cpr;
          if (k0 + ch * 8 < a.K) xv[q] = *reinterpret_cast<const u32x4*>(a.x + (size_t)m * a.ldx + k0 + ch * 8);
        }
      }
      stage(base);
    }
    __builtin_amdgcn_s_waitcnt(0);  // leave no load of this branch pending at the merge
  }
  // token rows Mr .. 16 MT - 1 of xsum: zero (their MFMA columns are finite and never stored)
  if (lane < 16 * MT - Mr)
    for (int gl = wave; gl < ng; gl += GEMV_WAVES) xsum[gl * 16 * MT + Mr + lane] = 0.f;
  lds_barrier();

  // ---- 4. units: prefetch the next, compute this one, reduce (waves take turns) ----
  // A unit whose epilogue needs no load (ksplit == 1, store / SwiGLU) finishes in the loop;
  // the others leave a coherent partial and are counted after the loop, when no prefetch
  // is outstanding any more (vmcnt retires in order, so a wait inside the loop would
  // also wait for the next unit's weights).
  // one dequant constant in an SGPR, the other in a VGPR: v_and_or_b32 may read one SGPR
  const uint32_t mask = a.dq_mask;
  uint32_t magic;
  MC_TO_VGPR(magic, a.dq_magic);
  const bool deferred = ks > 1 || a.epi == EPI_RESIDUAL;
  f32x4 acc[MT];
  const int u0 = u;
#pragma unroll
  for (int step = 0; step < U; ++step) {
    WBuf<D>& cur = (step & 1) ? wb : wa;
    WBuf<D>& nxt = (step & 1) ? wa : wb;
    if (step + 1 < U) load_unit<D>(nxt, a, min(u + G, nunits - 1) / ks, gp0, ngp, wave, lane, r16);
    if (u < nunits) {  // uniform: the whole block
      compute_unit<MT, D>(acc, cur, xl, xsum, XS, Mr, ngp, wave, c, r16, mask, magic);
      float* rb = red + (size_t)(step & 1) * GEMV_WAVES * MT * 64 * 4;
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) *reinterpret_cast<f32x4*>(rb + ((wave * MT + mt) * 64 + lane) * 4) = acc[mt];
      lds_barrier();
      if (wave == (step & 3)) {
        reduce_waves<MT>(acc, rb, lane);
        if (deferred) store_partial<MT>(a, acc, u / ks, kr, lane);
        else epilogue<MT>(a, acc, u / ks, c, r16);
      }
    }
    u += G;
  }
  if (deferred) {
    // this wave's partial stores are complete (device-visible) before its arrivals count
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    __builtin_amdgcn_s_waitcnt(0);
#pragma unroll
    for (int step = 0; step < U; ++step) {
      const int uu = u0 + step * G;
      if (wave == (step & 3) && uu < nunits) arrive<MT>(a, uu / ks, lane, c, r16);
    }
  }
}

// ---------------------------------------------------------------------------------------
// multi-row GEMV (16 < M <= 64): 8 waves per block, each wave owning whole units
// ---------------------------------------------------------------------------------------
// The activations of a K-range take Mr x kr x 256 bytes of LDS (up to 64 x 8 x 256), so
// one or two blocks fit a CU; with 8 waves per block and a wave computing a unit's whole
// K-range (no cross-wave reduction), every wave keeps the next unit's weights (up to 8
// KiB) in flight while it computes the current one.
constexpr int MID_WAVES = 8;
constexpr int MID_THREADS = MID_WAVES * 64;
constexpr int MID_KMAX = 8;  // the unit buffers of larger K-ranges are not kept in registers
constexpr int MID_LDS_CAP = 150 * 1024;

size_t mid_lds_bytes(int Mr, int kr, int MT) {
  return (size_t)Mr * xrow_stride(kr) * 2 + (size_t)16 * MT * 2 * kr * 4 + 64 * 4 + (size_t)kr * 128 * 2;
}

template <int MT, int D>
__global__ void __launch_bounds__(MID_THREADS) qgemv_mid_kernel(GemvArgs a) {
  MC_DYN_LDS(smem);
  const int kr_gp = a.kr, ks = a.ksplit;
  const int XS = xrow_stride(kr_gp);
  const int Mr = min(a.M, 16 * MT);
  uint16_t* xl = reinterpret_cast<uint16_t*>(smem);                     // [Mr][XS]
  float* xsum = reinterpret_cast<float*>(smem + (size_t)Mr * XS * 2);   // [2 kr][16 MT]
  float* rs = xsum + 16 * MT * 2 * kr_gp;                               // [64] row scales
  uint16_t* wl = reinterpret_cast<uint16_t*>(rs + 64);                  // [kr * 128] norm weights
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, c = lane >> 4, r16 = lane & 15;
  const int kq = blockIdx.x % ks;
  const int gp0 = kq * kr_gp, ngp = min(a.GP, gp0 + kr_gp) - gp0, k0 = gp0 * 128, ng = 2 * ngp;
  const int tstride = (int)(gridDim.x / ks) * MID_WAVES;
  const int t0 = (int)(blockIdx.x / ks) * MID_WAVES + wave;
  const int cpr = ngp * 16, xtotal = Mr * cpr;
  const unsigned cpr_magic = 0xFFFFFFFFu / (unsigned)cpr + 1u;

  // ---- small loads first (vmcnt retires in order): norm partials, norm weights, the first
  // pass of X; then the first unit's weights ----
  constexpr int XCH = 4;                 // chunks per thread and staging batch
  constexpr int XALL = 4 * XCH;          // every chunk of X: Mr x kr x 16 <= 64 x 8 x 16 = 16 x 512
  // norm partials: rows wave + 8 j (j < 8 covers Mr <= 64), producer tiles lane + 64 q (ss_nt <= 256)
  float ssq[8][4];
  if (a.norm_w) {
#pragma unroll
    for (int j = 0; j < 8; ++j)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int m = wave + MID_WAVES * j, tt = lane + 64 * q;
        ssq[j][q] = (m < Mr && tt < a.ss_nt) ? a.ss_in[(size_t)m * a.ss_ld + tt] : 0.f;
      }
  }
  u32x4 nw = {0u, 0u, 0u, 0u};
  if (a.norm_w && tid < cpr && k0 + tid * 8 < a.K) nw = *reinterpret_cast<const u32x4*>(a.norm_w + k0 + tid * 8);
  // all of X before the weights (vmcnt retires in order: the staging below then waits for X only)
  u32x4 xv[XALL];
#pragma unroll
  for (int q = 0; q < XALL; ++q) {
    const int i = tid + MID_THREADS * q;
    xv[q] = (u32x4){0u, 0u, 0u, 0u};
    if (i < xtotal) {
      const int m = (int)__umulhi((unsigned)i, cpr_magic), ch = i - m * cpr;
      if (k0 + ch * 8 < a.K) xv[q] = *reinterpret_cast<const u32x4*>(a.x + (size_t)m * a.ldx + k0 + ch * 8);
    }
  }
  WBuf<D> wa, wb;
  load_unit<D, 1>(wa, a, min(t0, a.NT - 1), gp0, ngp, 0, lane, r16);

  // ---- row scales of the fused RMSNorm, r[m] = 1 / sqrt(mean(x^2) + eps), fixed order ----
  if (a.norm_w) {
    if (tid < cpr) *reinterpret_cast<u32x4*>(wl + tid * 8) = nw;
    // the eight rows' butterflies interleaved, each in its fixed order
    float q[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) q[j] = (ssq[j][0] + ssq[j][1]) + (ssq[j][2] + ssq[j][3]);
#pragma unroll
    for (int o = 32; o > 0; o >>= 1)
#pragma unroll
      for (int j = 0; j < 8; ++j) q[j] += __shfl_xor(q[j], o);
    if (lane == 0)
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int m = wave + MID_WAVES * j;
        if (m < Mr) rs[m] = 1.0f / sqrtf(q[j] / (float)a.K + a.eps);
      }
    lds_barrier();
  }

  // ---- X (normalised) into LDS with its group sums ----
#pragma unroll
  for (int bq = 0; bq < XALL / XCH; ++bq) {
    const int base = bq * MID_THREADS * XCH;
    if (base >= xtotal) break;
    u32x4* xb = xv + bq * XCH;
    int mm[XCH], cc[XCH];
    bool in[XCH];
#pragma unroll
    for (int q = 0; q < XCH; ++q) {
      const int i = base + tid + MID_THREADS * q;
      in[q] = i < xtotal;
      mm[q] = (int)__umulhi((unsigned)i, cpr_magic);
      cc[q] = i - mm[q] * cpr;
    }
    if (a.norm_w) {
      float rr[XCH];
      u32x4 ww[XCH];
#pragma unroll
      for (int q = 0; q < XCH; ++q) {
        rr[q] = in[q] ? rs[mm[q]] : 0.f;
        ww[q] = in[q] ? *reinterpret_cast<const u32x4*>(wl + cc[q] * 8) : (u32x4){0u, 0u, 0u, 0u};
      }
#pragma unroll
      for (int q = 0; q < XCH; ++q)
#pragma unroll
        for (int h = 0; h < 4; ++h) {
          const float lo = (__uint_as_float(xb[q][h] << 16) * rr[q]) * __uint_as_float(ww[q][h] << 16);
          const float hi = (__uint_as_float(xb[q][h] & 0xFFFF0000u) * rr[q]) * __uint_as_float(ww[q][h] & 0xFFFF0000u);
          xb[q][h] = (uint32_t)f32_to_bf16(lo) | ((uint32_t)f32_to_bf16(hi) << 16);
        }
    }
    float gs[XCH];
#pragma unroll
    for (int q = 0; q < XCH; ++q) {
      if (in[q]) *reinterpret_cast<u32x4*>(xl + mm[q] * XS + cc[q] * 8) = xb[q];
      float s0 = 0.f, s1 = 0.f;
#pragma unroll
      for (int h = 0; h < 4; ++h) {
        s0 += __uint_as_float(xb[q][h] << 16);
        s1 += __uint_as_float(xb[q][h] & 0xFFFF0000u);
      }
      gs[q] = in[q] ? s0 + s1 : 0.f;
    }
#pragma unroll
    for (int q = 0; q < XCH; ++q) gs[q] = sum8_lanes(gs[q]);
#pragma unroll
    for (int q = 0; q < XCH; ++q)
      if (in[q] && (cc[q] & 7) == 0) xsum[(cc[q] >> 3) * 16 * MT + mm[q]] = gs[q];
  }
  if (lane < 16 * MT - Mr)
    for (int gl = wave; gl < ng; gl += MID_WAVES) xsum[gl * 16 * MT + Mr + lane] = 0.f;
  lds_barrier();

  // ---- units: the next one's weights in flight while this one is computed ----
  const uint32_t mask = a.dq_mask;
  uint32_t magic;
  MC_TO_VGPR(magic, a.dq_magic);
  const bool deferred = ks > 1 || a.epi == EPI_RESIDUAL;
  int t = t0;
  while (t < a.NT) {
    {
      const int tn = t + tstride < a.NT ? t + tstride : t;
      load_unit<D, 1>(wb, a, tn, gp0, ngp, 0, lane, r16);
      f32x4 acc[MT];
      compute_unit<MT, D, 1>(acc, wa, xl, xsum, XS, Mr, ngp, 0, c, r16, mask, magic);
      if (deferred) store_partial<MT>(a, acc, t, kq, lane);
      else epilogue<MT>(a, acc, t, c, r16);
      t += tstride;
    }
    if (t >= a.NT) break;
    {
      const int tn = t + tstride < a.NT ? t + tstride : t;
      load_unit<D, 1>(wa, a, tn, gp0, ngp, 0, lane, r16);
      f32x4 acc[MT];
      compute_unit<MT, D, 1>(acc, wb, xl, xsum, XS, Mr, ngp, 0, c, r16, mask, magic);
      if (deferred) store_partial<MT>(a, acc, t, kq, lane);
      else epilogue<MT>(a, acc, t, c, r16);
      t += tstride;
    }
  }
  if (deferred) {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    __builtin_amdgcn_s_waitcnt(0);
    arrive_units<MT>(a, t0, tstride, lane, c, r16);
  }
}

// ---------------------------------------------------------------------------------------
// GEMM for M > 64 (verify blocks of many rows): the weights are dequantised once per K-step
// and used against every token tile of the block
// ---------------------------------------------------------------------------------------
// Block (n-block, m-block): 128 weight rows (wave w owns tiles 8 nb + 2 w, + 1) x 16 MB
// tokens, accumulators resident over the whole K; two blocks per CU (64-token blocks keep
// the kernel within 256 registers, so one block's waits overlap the other's MFMAs).  The activations go through LDS one
// 128-wide K-step (group pair) at a time, double-buffered: the next step's loads are in
// flight while the current step is computed, and its group sums are formed as it is
// written.  The input rows are already normalised (no fused RMSNorm here).  When the
// (weight-block, token-block) grid would leave CUs idle, K is split over blockIdx.z: each
// K-range leaves device-coherent fp32 partials and the last arrival per tile sums them in
// K-range order and runs the epilogue (the same protocol as the 17-64-token kernel).
constexpr int QG_MB = 4;                 // token tiles per block (64 tokens)
constexpr int QG_NTW = 2;                // weight tiles per wave
constexpr int QG_RD = 4;                 // K-steps of weights held in registers (prefetch distance QG_RD - 1)
constexpr int QG_XS = 128 + 8;           // LDS row stride (bf16) of one K-step of X
constexpr int QG_XCH = QG_MB * 16 * 16 / 256;  // 16-byte X chunks per thread per K-step
constexpr int QG_KSPLIT_MAX = 8;
constexpr int QG_OCC = 2;                // resident blocks per CU (the kernel's launch bounds)

size_t qgemm_lds_bytes() { return (size_t)2 * 16 * QG_MB * QG_XS * 2 + (size_t)2 * 2 * 16 * QG_MB * 4; }

__global__ void __launch_bounds__(256, 2) qgemm_kernel(GemvArgs a) {
  MC_DYN_LDS(smem);
  constexpr int MR = 16 * QG_MB;
  uint16_t* xl = reinterpret_cast<uint16_t*>(smem);                          // [2][MR][QG_XS]
  float* xsum = reinterpret_cast<float*>(smem + (size_t)2 * MR * QG_XS * 2);  // [2][2 groups][MR]
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, c = lane >> 4, r16 = lane & 15;
  const int m0 = blockIdx.y * MR;
  const int Mb = min(MR, a.M - m0);  // live tokens of this block
  const int tw = blockIdx.x * 4 * QG_NTW + wave * QG_NTW;  // this wave's first weight tile
  const int GP = a.GP;
  const int kq = blockIdx.z;                                 // K-range: group pairs gq0 .. gq0 + NS - 1
  const int gq0 = kq * a.kr;
  const int NS = min(a.GP, gq0 + a.kr) - gq0;                // >= 1 (the plan leaves no empty range)

  // X chunk q of a K-step: token row (tid + 256 q) / 16, 16-byte chunk (tid + 256 q) % 16
  auto load_x = [&](int gp, u32x4 (&xv)[QG_XCH]) {
#pragma unroll
    for (int q = 0; q < QG_XCH; ++q) {
      const int i = tid + 256 * q, m = i >> 4, ch = i & 15;
      xv[q] = (u32x4){0u, 0u, 0u, 0u};
      if (m < Mb && gp * 128 + ch * 8 < a.K)
        xv[q] = *reinterpret_cast<const u32x4*>(a.x + (size_t)(m0 + m) * a.ldx + gp * 128 + ch * 8);
    }
  };
  auto store_x = [&](int buf, const u32x4 (&xv)[QG_XCH]) {
    uint16_t* xb = xl + (size_t)buf * MR * QG_XS;
    float* sb = xsum + (size_t)buf * 2 * MR;
    float gs[QG_XCH];
#pragma unroll
    for (int q = 0; q < QG_XCH; ++q) {
      const int i = tid + 256 * q, m = i >> 4, ch = i & 15;
      *reinterpret_cast<u32x4*>(xb + m * QG_XS + ch * 8) = xv[q];
      float s0 = 0.f, s1 = 0.f;
#pragma unroll
      for (int h = 0; h < 4; ++h) {
        s0 += __uint_as_float(xv[q][h] << 16);
        s1 += __uint_as_float(xv[q][h] & 0xFFFF0000u);
      }
      gs[q] = s0 + s1;
    }
#pragma unroll
    for (int q = 0; q < QG_XCH; ++q) gs[q] = sum8_lanes(gs[q]);
#pragma unroll
    for (int q = 0; q < QG_XCH; ++q) {
      const int i = tid + 256 * q, m = i >> 4, ch = i & 15;
      if ((ch & 7) == 0) sb[(ch >> 3) * MR + m] = gs[q];
    }
  };
  // weights of K-step gp for the wave's tiles (a tile past the end re-reads the last one)
  auto load_w = [&](int gp, u32x4 (&wq)[QG_NTW], uint2 (&wsb)[QG_NTW]) {
#pragma unroll
    for (int n = 0; n < QG_NTW; ++n) {
      const int t = min(tw + n, a.NT - 1);
      wq[n] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(a.qw) + ((size_t)t * GP + gp) * 64 + lane);
      wsb[n] = reinterpret_cast<const uint2*>(a.sb)[tile_sb_word(t, r16, gp, 0, GP) / 2];
    }
  };

  f32x4 acc[QG_NTW][QG_MB];
#pragma unroll
  for (int n = 0; n < QG_NTW; ++n)
#pragma unroll
    for (int mt = 0; mt < QG_MB; ++mt) acc[n][mt] = (f32x4){0.f, 0.f, 0.f, 0.f};
  const uint32_t mask = a.dq_mask;
  uint32_t magic;
  MC_TO_VGPR(magic, a.dq_magic);

  // weights of K-steps s .. s + QG_RD - 1 in a ring of registers (slot s % QG_RD, static
  // after the unroll)
  u32x4 wr[QG_RD][QG_NTW];
  uint2 sr[QG_RD][QG_NTW];
  u32x4 xv[QG_XCH];
  load_x(gq0, xv);
#pragma unroll
  for (int r = 0; r < QG_RD - 1; ++r) load_w(gq0 + min(r, NS - 1), wr[r], sr[r]);
  store_x(0, xv);
  lds_barrier();
  for (int g0 = 0; g0 < NS; g0 += QG_RD) {
#pragma unroll
    for (int u = 0; u < QG_RD; ++u) {
      const int gs = g0 + u;  // K-step of this range
      if (gs >= NS) break;    // uniform
      const int buf = gs & 1;
      // every load unconditional (the last steps re-read themselves), X first: the wait for
      // X below then leaves the weights of step gp + QG_RD - 1 in flight
      load_x(gq0 + min(gs + 1, NS - 1), xv);
      load_w(gq0 + min(gs + QG_RD - 1, NS - 1), wr[(u + QG_RD - 1) % QG_RD], sr[(u + QG_RD - 1) % QG_RD]);
      const u32x4 (&wq0)[QG_NTW] = wr[u];
      const uint2 (&ws0)[QG_NTW] = sr[u];
      // ---- compute K-step gs ----
      const uint16_t* xb = xl + (size_t)buf * MR * QG_XS;
      const float* sbuf = xsum + (size_t)buf * 2 * MR;
#pragma unroll
      for (int gi = 0; gi < 2; ++gi) {
        bf16x8 wv[QG_NTW][2];
        float sv[QG_NTW], bv[QG_NTW];
#pragma unroll
        for (int n = 0; n < QG_NTW; ++n) {
          wv[n][0] = dequant_word(gi ? wq0[n].z : wq0[n].x, mask, magic);
          wv[n][1] = dequant_word(gi ? wq0[n].w : wq0[n].y, mask, magic);
          const uint32_t sbv = gi ? ws0[n].y : ws0[n].x;
          sv[n] = DQ_STEP * __uint_as_float(sbv << 16);
          bv[n] = __uint_as_float(sbv & 0xFFFF0000u) - sv[n];
        }
#pragma unroll
        for (int mt = 0; mt < QG_MB; ++mt) {
          const uint16_t* xrow = xb + (mt * 16 + r16) * QG_XS + gi * 64 + 8 * c;
          const bf16x8 xa0 = *reinterpret_cast<const bf16x8*>(xrow);
          const bf16x8 xa1 = *reinterpret_cast<const bf16x8*>(xrow + 32);
          const f32x4 xs = *reinterpret_cast<const f32x4*>(sbuf + gi * MR + mt * 16 + 4 * c);
#pragma unroll
          for (int n = 0; n < QG_NTW; ++n) {
            f32x4 g = {0.f, 0.f, 0.f, 0.f};
            g = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xa0, wv[n][0], g, 0, 0, 0);
            g = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xa1, wv[n][1], g, 0, 0, 0);
#pragma unroll
            for (int v = 0; v < 4; ++v) {
              acc[n][mt][v] = __builtin_fmaf(sv[n], g[v], acc[n][mt][v]);
              acc[n][mt][v] = __builtin_fmaf(bv[n], xs[v], acc[n][mt][v]);
            }
          }
        }
      }
      if (gs + 1 < NS) store_x(buf ^ 1, xv);  // uniform
      lds_barrier();  // step gs + 1 is in LDS; step gs's buffer is free for step gs + 2
    }
  }
  // ---- epilogues: this block's tokens m0 .. m0 + Mb - 1 ----
  GemvArgs e = a;
  e.M = Mb;
  e.y = a.y + (size_t)m0 * a.ldy;
  if (a.amax) e.amax = a.amax + (size_t)m0 * a.NT;
  if (a.ss_out) e.ss_out = a.ss_out + (size_t)m0 * a.ss_ld_out;
  if (a.ksplit == 1) {
#pragma unroll
    for (int n = 0; n < QG_NTW; ++n)
      if (tw + n < a.NT) epilogue<QG_MB>(e, acc[n], tw + n, c, r16);
    return;
  }
  // split K: this token block's partials [ksplit][NT][MB][64][4] and counters [NT]
  e.part = a.part + (size_t)blockIdx.y * a.ksplit * a.NT * QG_MB * 256;
  e.counters = a.counters + (size_t)blockIdx.y * a.NT;
#pragma unroll
  for (int n = 0; n < QG_NTW; ++n)
    if (tw + n < a.NT) store_partial<QG_MB>(e, acc[n], tw + n, kq, lane);
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
  __builtin_amdgcn_s_waitcnt(0);
#pragma unroll
  for (int n = 0; n < QG_NTW; ++n)
    if (tw + n < a.NT) arrive<QG_MB>(e, tw + n, lane, c, r16);
}

static thread_local hipEvent_t t_launch_ev[2] = {nullptr, nullptr};
void gemv_time_next_launch(hipEvent_t start, hipEvent_t stop) {
  t_launch_ev[0] = start;
  t_launch_ev[1] = stop;
}

// hipLaunchKernelGGL, or hipExtLaunchKernelGGL with the events of gemv_time_next_launch
template <typename F, typename... Args>
static void launch_gemv_kernel(F kernel, dim3 grid, dim3 block, size_t lds, hipStream_t st, Args... args) {
  if (t_launch_ev[0]) {
    hipExtLaunchKernelGGL(kernel, grid, block, (std::uint32_t)lds, st, t_launch_ev[0], t_launch_ev[1], 0u, args...);
    t_launch_ev[0] = t_launch_ev[1] = nullptr;
  } else {
    hipLaunchKernelGGL(kernel, grid, block, lds, st, args...);
  }
}

static int device_cus();

// Split-K plan of the large-M GEMM: the K-range length (group pairs) and the number of
// ranges that minimise the modelled time -- rounds of one block per CU times the steps per
// block (plus about 1.5 steps of pipeline fill), plus the partials' HBM round trip priced
// at 4 TB/s against a measured ~2.2 us per K-step of a block.  Depends on (NT, GP, the
// token-block count, the CU count) only.
void qgemm_plan(int NT, int GP, int M, int cus, int* kr, int* ksplit) {
  const long tiles = (long)((NT + 4 * QG_NTW - 1) / (4 * QG_NTW)) * ((M + 16 * QG_MB - 1) / (16 * QG_MB));
  double best = 0.0;
  *kr = GP;
  *ksplit = 1;
  for (int ks = 1; ks <= QG_KSPLIT_MAX && ks <= GP; ++ks) {
    const int r = (GP + ks - 1) / ks, kse = (GP + r - 1) / r;
    if (kse != ks) continue;  // the same split as a smaller ks
    const long blocks = tiles * kse;
    const double rounds = (double)((blocks + QG_OCC * cus - 1) / (QG_OCC * cus));
    double us = rounds * (r + 1.5) * 2.2;
    if (kse > 1) us += (double)blocks * 4 * QG_NTW * 16 * 16 * QG_MB * 4 * 2 / 4e6;
    if (ks == 1 || us < best) {
      best = us;
      *kr = r;
      *ksplit = kse;
    }
  }
}

void qgemm_workspace(int NT, int GP, int Mmax, size_t* part_floats, int* counters) {
  const int cus = device_cus();
  *part_floats = 0;
  *counters = 0;
  for (int mb = 1; mb <= (Mmax + 16 * QG_MB - 1) / (16 * QG_MB); ++mb) {
    int kr, ks;
    qgemm_plan(NT, GP, mb * 16 * QG_MB, cus, &kr, &ks);
    if (ks > 1) {
      *part_floats = std::max(*part_floats, (size_t)mb * ks * NT * QG_MB * 256);
      *counters = std::max(*counters, mb * NT);
    }
  }
}

int qgemm_launch(const GemvArgs& a, hipStream_t st) {
  if (a.M <= 64) return fail(MC_E_INVALID, "qgemm: for more than 64 tokens");
  if (a.K % 64 || a.GP != (a.K + 127) / 128 || a.NT != (a.N + 15) / 16) return fail(MC_E_INVALID, "qgemm: bad shape");
  if (a.norm_w) return fail(MC_E_INVALID, "qgemm: normalise the input rows first");
  if (a.amax && a.epi != EPI_STORE) return fail(MC_E_INVALID, "qgemm: argmax partials need the store epilogue");
  if (a.epi == EPI_RESIDUAL && a.N % 16) return fail(MC_E_INVALID, "qgemm: residual epilogue needs N % 16 == 0");
  GemvArgs p = a;
  qgemm_plan(a.NT, a.GP, a.M, device_cus(), &p.kr, &p.ksplit);
  const unsigned mblocks = (unsigned)((a.M + 16 * QG_MB - 1) / (16 * QG_MB));
  if (p.ksplit > 1 && (!a.part || a.part_floats < (size_t)mblocks * p.ksplit * a.NT * QG_MB * 256 || !a.counters ||
                       (size_t)a.counters_n < (size_t)mblocks * a.NT))
    return fail(MC_E_INVALID, "qgemm: split-K workspace too small");
  const dim3 grid((unsigned)((a.NT + 4 * QG_NTW - 1) / (4 * QG_NTW)), mblocks, (unsigned)p.ksplit);
  launch_gemv_kernel(qgemm_kernel, grid, dim3(256), qgemm_lds_bytes(), st, p);
  MC_HIP(hipGetLastError());
  return MC_OK;
}

// K-range plan of the multi-row classes: the largest K-range whose activations fit the LDS
// cap (at most 8 group pairs), split further (down to 4 pairs) while there are fewer than
// 4 units per CU.  Splitting until every wave of the device had a unit (8 per CU) cost
// more in activation staging and partial sums than it gained in parallelism (batch-8
// Qwen3-4B-shape step 5.50 -> 5.08 ms at 4 per CU).  Depends only on (N, K, MT) and the CU
// count.
constexpr int MID_UNITS_PER_CU = 4;
void mid_plan(const QLinear& L, int MT, int cus, int* kr, int* ksplit) {
  int kmax = MID_KMAX;
  while (kmax > 1 && mid_lds_bytes(16 * MT, kmax, MT) > (size_t)MID_LDS_CAP) --kmax;
  int ks = (L.GP + kmax - 1) / kmax;
  while ((size_t)L.NT * ks < (size_t)MID_UNITS_PER_CU * cus && (L.GP + ks) / (ks + 1) >= 4) ++ks;
  *kr = (L.GP + ks - 1) / ks;
  *ksplit = (L.GP + *kr - 1) / *kr;
}

// K-range plan of a shape for an M class (MT = 1: M <= 16; MT > 1: M <= 64).  Depends
// only on (N, K, class): a token's reduction order never changes with the number of
// tokens in its class, nor with the grid the launch gets.
static int g_cus = 0;

static int device_cus() {
  if (g_cus == 0) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&g_cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || g_cus < 1)
      g_cus = 1;
  }
  return g_cus;
}

void gemv_plan(const QLinear& L, int MT, int* kr, int* ksplit) {
  if (MT > 1) {
    mid_plan(L, MT, device_cus(), kr, ksplit);
    return;
  }
  const int Mr = 16;
  // one K-range when it fits 5 group pairs per wave (no split-K tail), else 4 per wave
  // (K = 4096: two K-ranges, K = 9728: five; 4 per wave measured faster than 3 and 5)
  int d = (MT == 1 && L.GP <= GEMV_WAVES * 5) ? 5 : 4;
  while (d > 1 && gemv_lds_bytes(Mr, GEMV_WAVES * d, MT) > (size_t)GEMV_LDS_LIMIT) --d;
  *kr = std::min(L.GP, GEMV_WAVES * d);
  *ksplit = (L.GP + *kr - 1) / *kr;
}

// resident blocks per CU of one kernel instance at one LDS size (cached)
template <int MT, int D, int U>
static int occupancy(size_t lds) {
  static int cache_lds[8] = {-1, -1, -1, -1, -1, -1, -1, -1}, cache_n[8];
  for (int i = 0; i < 8; ++i)
    if (cache_lds[i] == (int)lds) return cache_n[i];
  int n = 1;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, (const void*)qgemv_kernel<MT, D, U>, 256, lds) != hipSuccess || n < 1)
    n = 1;
  for (int i = 0; i < 8; ++i)
    if (cache_lds[i] < 0) { cache_lds[i] = (int)lds; cache_n[i] = n; break; }
  return n;
}

template <int MT, int D, int U>
static void launch_mdu(const GemvArgs& a, size_t lds, int G, hipStream_t st) {
  G += (a.ksplit - G % a.ksplit) % a.ksplit;  // a block's K-range stays fixed: G % ksplit == 0
  launch_gemv_kernel(qgemv_kernel<MT, D, U>, dim3(G), dim3(256), lds, st, a);
}

// Units per block: enough that one round of resident blocks covers the launch (every
// block stages its activations once, so fewer, longer-lived blocks amortise that), but at
// most 4: a block keeps only the next unit in flight, so longer queues (the vocab head
// at 8 or 16 units per block) leave the weight stream latency-bound (head 110 -> 75 us).
// With U units per block the grid is a whole number of blocks per CU, the fewest that hold
// the units (G = CUs x ceil(units / (CUs U))): the units of one CU's blocks then differ by
// one at most, where ceil(units / U) blocks leave some CUs a block (U units) more than others.
template <int MT, int D>
static void launch_md(const GemvArgs& a, size_t lds, hipStream_t st) {
  const int nunits = a.NT * a.ksplit;
  const int cap = g_cus * occupancy<MT, D, 1>(lds);
  const int need = (nunits + cap - 1) / cap;
  auto grid = [&](int U) { return std::min(nunits, g_cus * ((nunits + g_cus * U - 1) / (g_cus * U))); };
  if (need <= 1) launch_mdu<MT, D, 1>(a, lds, nunits, st);
  else if (need == 2) launch_mdu<MT, D, 2>(a, lds, grid(2), st);
  else launch_mdu<MT, D, 4>(a, lds, grid(4), st);
}

template <int MT>
static void launch_mt(const GemvArgs& a, int D, size_t lds, hipStream_t st) {
  switch (D) {
    case 1: launch_md<MT, 1>(a, lds, st); break;
    case 2: launch_md<MT, 2>(a, lds, st); break;
    case 3: launch_md<MT, 3>(a, lds, st); break;
    case 4: launch_md<MT, 4>(a, lds, st); break;
    default: launch_md<MT, 5>(a, lds, st); break;
  }
}

template <int MT, int D>
static void launch_mid_d(const GemvArgs& a, size_t lds, hipStream_t st) {
  int occ = 1;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, (const void*)qgemv_mid_kernel<MT, D>, MID_THREADS, lds) !=
          hipSuccess || occ < 1)
    occ = 1;
  const int groups = (a.NT + MID_WAVES - 1) / MID_WAVES;
  const int G1 = std::max(1, std::min(groups, device_cus() * occ / a.ksplit));
  launch_gemv_kernel(qgemv_mid_kernel<MT, D>, dim3(G1 * a.ksplit), dim3(MID_THREADS), lds, st, a);
}

template <int MT>
static void launch_mid(const GemvArgs& a, size_t lds, hipStream_t st) {
  if (a.kr <= 4) launch_mid_d<MT, 4>(a, lds, st);
  else if (a.kr <= 6) launch_mid_d<MT, 6>(a, lds, st);
  else launch_mid_d<MT, 8>(a, lds, st);
}

int gemv_launch(const GemvArgs& a, int MT, hipStream_t st) {
  (void)device_cus();
  const int Mr = std::min(a.M, 16 * MT);
  const size_t lds = MT > 1 ? mid_lds_bytes(Mr, a.kr, MT) : gemv_lds_bytes(Mr, a.kr, MT);
  if (lds > (size_t)GEMV_LDS_LIMIT) return fail(MC_E_INVALID, "gemv: K-range exceeds LDS");
  if (a.M < 1 || a.M > 16 * MT || (MT > 1 && a.M <= 16)) return fail(MC_E_INVALID, "gemv: M outside the m-tile class");
  if (a.K % 64 || a.GP != (a.K + 127) / 128 || a.NT != (a.N + 15) / 16) return fail(MC_E_INVALID, "gemv: bad shape");
  if (a.kr < 1 || a.kr > (MT > 1 ? MID_KMAX : GEMV_WAVES * 5) || a.ksplit != (a.GP + a.kr - 1) / a.kr)
    return fail(MC_E_INVALID, "gemv: bad K-range plan");
  if (a.norm_w && (!a.ss_in || a.ss_nt < 1 || a.ss_nt > 256 || a.ss_ld < a.ss_nt))
    return fail(MC_E_INVALID, "gemv: fused norm needs the producer's sums of squares (<= 256 tiles)");
  if (a.amax && a.epi != EPI_STORE) return fail(MC_E_INVALID, "gemv: argmax partials need the store epilogue");
  if (a.epi == EPI_RESIDUAL && (a.N % 16 || (a.ss_out && a.ss_ld_out < a.NT)))
    return fail(MC_E_INVALID, "gemv: residual epilogue needs N % 16 == 0");
  if ((a.ksplit > 1 || a.epi == EPI_RESIDUAL) &&
      (!a.part || a.part_floats < (size_t)a.ksplit * a.NT * MT * 64 * 4 || !a.counters || a.counters_n < a.NT))
    return fail(MC_E_INVALID, "gemv: split-K workspace smaller than the plan");
  const int D = (a.kr + GEMV_WAVES - 1) / GEMV_WAVES;  // group pairs per wave per unit
  switch (MT) {
    case 1: launch_mt<1>(a, D, lds, st); break;
    case 2: launch_mid<2>(a, lds, st); break;
    case 3: launch_mid<3>(a, lds, st); break;
    case 4: launch_mid<4>(a, lds, st); break;
    default: return fail(MC_E_INVALID, "gemv: unsupported m-tile count");
  }
  MC_HIP(hipGetLastError());
  return MC_OK;
}

template <int MT, int D>
static int setup_md() {
  const void* fns[] = {(const void*)qgemv_kernel<MT, D, 1>, (const void*)qgemv_kernel<MT, D, 2>,
                       (const void*)qgemv_kernel<MT, D, 4>};
  for (const void* f : fns) MC_HIP(hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, GEMV_LDS_LIMIT));
  return MC_OK;
}

template <int MT>
static int setup_mt() {
  int rc;
  if ((rc = setup_md<MT, 1>()) || (rc = setup_md<MT, 2>())) return rc;
  if constexpr (MT == 1) {
    if ((rc = setup_md<MT, 3>()) || (rc = setup_md<MT, 4>()) || (rc = setup_md<MT, 5>())) return rc;
  }
  return MC_OK;
}

// ---------------------------------------------------------------------------------------
// grouped (MoE) GEMV
// ---------------------------------------------------------------------------------------
constexpr int MOE_MAX_GP = 20;  // K <= 2560

constexpr int MOE_ROWS = 8;  // routed pairs staged at a time (a verify block routes ~1-3 per expert)

__host__ __device__ constexpr size_t moe_lds_bytes(int GP) {
  return (size_t)MOE_ROWS * xrow_stride(GP) * 2 + (size_t)16 * 2 * GP * 4;
}

// Block (slot, jb): touched expert act_e[slot], tiles jb, jb + nb, ... with the full K range;
// wave w of the block takes the block's tiles w, w + 4, ..., each as K-chunks of D group
// pairs accumulated in order, so the wave needs no partner to finish a tile and keeps
// the next chunk's weights (D KiB) in flight while it computes the current one.  The
// expert's pairs are taken MOE_ROWS at a time (rows of one m-tile; the LDS they need lets
// four blocks share a CU); for each such group the block stages the pairs' input rows.
template <int D>
__global__ void __launch_bounds__(256) moe_gemv_kernel(MoeGemvArgs a) {
  MC_DYN_LDS(smem);
  __shared__ int s_pairs[64];
  const int slot = blockIdx.x / a.nb, jb = blockIdx.x - slot * a.nb;
  // the slot's routing, all in one round trip (slot < max_active <= E: every read is inside
  // the arrays; a slot past the touched count returns below)
  const int n_act = *a.rt.n_active, e = a.rt.act_e[slot];
  const int p0 = a.rt.off[slot], p1 = a.rt.off[slot + 1];
  const int my_pair = threadIdx.x < 64 ? a.rt.slot_pairs[(size_t)slot * 64 + threadIdx.x] : 0;
  if (slot >= n_act || jb >= a.NT) return;  // uniform over the block
  const int np = p1 - p0;
  if (threadIdx.x < 64) s_pairs[threadIdx.x] = my_pair;
  __syncthreads();
  const int GP = a.GP, XS = xrow_stride(GP), cpr = GP * 16, ng = 2 * GP;
  const int nkc = (GP + D - 1) / D;  // K-chunks per tile
  uint16_t* xl = reinterpret_cast<uint16_t*>(smem);                            // [MOE_ROWS][XS]
  float* xsum = reinterpret_cast<float*>(smem + (size_t)MOE_ROWS * XS * 2);    // [2 GP][16]
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, c = lane >> 4, r16 = lane & 15;
  GemvArgs g;  // the expert's weights, for load_unit
  g.qw = a.qw + (size_t)e * a.qw_es;
  g.sb = a.sb + (size_t)e * a.sb_es;
  g.GP = GP;
  const unsigned cpr_magic = 0xFFFFFFFFu / (unsigned)cpr + 1u;
  const uint32_t mask = a.dq_mask;
  uint32_t magic;
  MC_TO_VGPR(magic, a.dq_magic);
  const int tstride = GEMV_WAVES * a.nb;
  const int t0 = jb + a.nb * wave;
  // units of this wave: u = tile index i (t = t0 + i tstride) x K-chunk kc, in order
  const int ntl = t0 < a.NT ? (a.NT - t0 + tstride - 1) / tstride : 0;
  const int nunits = ntl * nkc;
  auto unit_tile = [&](int u) { return t0 + (u / nkc) * tstride; };
  auto unit_gp0 = [&](int u) { return (u % nkc) * D; };
  auto unit_ngp = [&](int u) { return min(GP, unit_gp0(u) + D) - unit_gp0(u); };
  for (int q0 = 0; q0 < np; q0 += MOE_ROWS) {
    const int Mr = min(MOE_ROWS, np - q0);  // MFMA rows >= Mr read row Mr - 1 and are not stored
    WBuf<D> wa, wb;
    if (nunits > 0) load_unit<D, 1>(wa, g, unit_tile(0), unit_gp0(0), unit_ngp(0), 0, lane, r16);
    for (int i0 = 0; i0 < Mr * cpr; i0 += 256 * 4) {
      u32x4 v[4];
      int mm[4], cc[4];
      bool in[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int i = i0 + tid + 256 * j;
        in[j] = i < Mr * cpr;
        mm[j] = (int)__umulhi((unsigned)i, cpr_magic);
        cc[j] = i - mm[j] * cpr;
        v[j] = (u32x4){0u, 0u, 0u, 0u};
        if (in[j] && cc[j] * 8 < a.K) {
          const int row = s_pairs[q0 + mm[j]] / a.x_div;
          v[j] = *reinterpret_cast<const u32x4*>(a.x + (size_t)row * a.ldx + cc[j] * 8);
        }
      }
      float gs[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        if (in[j]) *reinterpret_cast<u32x4*>(xl + mm[j] * XS + cc[j] * 8) = v[j];
        float s0 = 0.f, s1 = 0.f;
#pragma unroll
        for (int h = 0; h < 4; ++h) {
          s0 += __uint_as_float(v[j][h] << 16);
          s1 += __uint_as_float(v[j][h] & 0xFFFF0000u);
        }
        gs[j] = in[j] ? s0 + s1 : 0.f;
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) gs[j] = sum8_lanes(gs[j]);
#pragma unroll
      for (int j = 0; j < 4; ++j)
        if (in[j] && (cc[j] & 7) == 0) xsum[(cc[j] >> 3) * 16 + mm[j]] = gs[j];
    }
    if (lane < 16 - Mr)
      for (int gl = wave; gl < ng; gl += GEMV_WAVES) xsum[gl * 16 + Mr + lane] = 0.f;
    lds_barrier();
    f32x4 acc[1] = {(f32x4){0.f, 0.f, 0.f, 0.f}};
    auto finish = [&](int u, const WBuf<D>& cur) {
      f32x4 part[1];
      // the chunk's pairs: compute_unit indexes the staged X from pair 0 of the K range
      compute_unit<1, D, 1>(part, cur, xl + unit_gp0(u) * 128, xsum + unit_gp0(u) * 2 * 16, XS, Mr, unit_ngp(u), 0, c,
                            r16, mask, magic);
      acc[0] += part[0];
      if (u % nkc != nkc - 1) return;
      const int t = unit_tile(u);
      const int n = t * 16 + r16;
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int m = 4 * c + v;
        const bool live = m < Mr;
        const int pr = live ? s_pairs[q0 + m] : 0;
        if (a.epi == EPI_SWIGLU) {
          const float up = __shfl_xor(acc[0][v], 1);
          if (live && !(r16 & 1) && n + 1 < a.N) a.y[(size_t)pr * a.ldy + (n >> 1)] = f32_to_bf16(silu_f(acc[0][v]) * up);
        } else if (live && n < a.N) {
          a.yf[(size_t)pr * a.ldy + n] = acc[0][v];
        }
      }
      acc[0] = (f32x4){0.f, 0.f, 0.f, 0.f};
    };
    for (int u = 0; u < nunits; u += 2) {
      {
        const int un = u + 1 < nunits ? u + 1 : u;  // the last unit re-reads itself
        load_unit<D, 1>(wb, g, unit_tile(un), unit_gp0(un), unit_ngp(un), 0, lane, r16);
        finish(u, wa);
      }
      if (u + 1 >= nunits) break;
      {
        const int un = u + 2 < nunits ? u + 2 : u + 1;
        load_unit<D, 1>(wa, g, unit_tile(un), unit_gp0(un), unit_ngp(un), 0, lane, r16);
        finish(u + 1, wb);
      }
    }
    // the staged rows are rewritten by the next group: every wave is past its last tile
    __builtin_amdgcn_s_waitcnt(0);
    lds_barrier();
  }
}

int moe_gemv_launch(const MoeGemvArgs& a, hipStream_t st) {
  if (a.K % 64 || a.GP != (a.K + 127) / 128 || a.NT != (a.N + 15) / 16 || a.GP > MOE_MAX_GP)
    return fail(MC_E_INVALID, "moe gemv: shape (K must be a multiple of 64, at most 2560)");
  if (a.nb < 1 || a.max_active < 1 || !a.rt.n_active || !a.rt.act_e || !a.rt.off || !a.rt.pairs || a.x_div < 1)
    return fail(MC_E_INVALID, "moe gemv: routing arguments");
  if ((a.epi == EPI_SWIGLU && (!a.y || a.N % 2)) || (a.epi == EPI_STORE && !a.yf) ||
      (a.epi != EPI_SWIGLU && a.epi != EPI_STORE))
    return fail(MC_E_INVALID, "moe gemv: epilogue");
  const size_t lds = moe_lds_bytes(a.GP);
  const dim3 grid((unsigned)(a.max_active * a.nb));
  // K-chunks of 4 group pairs: registers for three blocks per CU (measured faster than 8)
  hipLaunchKernelGGL(moe_gemv_kernel<4>, grid, dim3(256), lds, st, a);
  MC_HIP(hipGetLastError());
  return MC_OK;
}

// One block per row: sum of squares in a fixed order (thread partials, then a tree over
// the block), then bf16((x * r) * w).
__global__ void __launch_bounds__(256) rows_rmsnorm_kernel(const uint16_t* x, const uint16_t* w, int H, float eps,
                                                           uint16_t* xn) {
  __shared__ float part[256];
  const int t = blockIdx.x, tid = threadIdx.x;
  const uint16_t* xr = x + (size_t)t * H;
  float q = 0.f;
  for (int k = tid; k < H; k += 256) {
    const float v = bf16_to_f32(xr[k]);
    q += v * v;
  }
  part[tid] = q;
  __syncthreads();
  for (int s = 128; s > 0; s >>= 1) {
    if (tid < s) part[tid] += part[tid + s];
    __syncthreads();
  }
  const float r = 1.0f / sqrtf(part[0] / (float)H + eps);
  for (int k = tid; k < H; k += 256) xn[(size_t)t * H + k] = f32_to_bf16((bf16_to_f32(xr[k]) * r) * bf16_to_f32(w[k]));
}

int launch_rows_rmsnorm(const uint16_t* x, const uint16_t* w, int M, int H, float eps, uint16_t* xn, hipStream_t st) {
  if (M < 1) return MC_OK;
  hipLaunchKernelGGL(rows_rmsnorm_kernel, dim3(M), dim3(256), 0, st, x, w, H, eps, xn);
  MC_HIP(hipGetLastError());
  return MC_OK;
}

// Wave-wide reductions for the routing block: DPP moves within rows of 16 lanes (swap
// neighbours, swap pairs, mirror 8, mirror 16: every lane of a row then holds the row's
// result), then the four rows' results read into scalar registers -- no LDS round trips.
template <int CTRL>
__device__ inline unsigned dpp_u32(unsigned v) {
  return (unsigned)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xF, 0xF, false);
}
__device__ inline float route_wave_max(float v) {
  v = fmaxf(v, __uint_as_float(dpp_u32<0xB1>(__float_as_uint(v))));
  v = fmaxf(v, __uint_as_float(dpp_u32<0x4E>(__float_as_uint(v))));
  v = fmaxf(v, __uint_as_float(dpp_u32<0x141>(__float_as_uint(v))));
  v = fmaxf(v, __uint_as_float(dpp_u32<0x140>(__float_as_uint(v))));
  const unsigned u = __float_as_uint(v);
  return fmaxf(fmaxf(__uint_as_float((unsigned)__builtin_amdgcn_readlane((int)u, 0)),
                     __uint_as_float((unsigned)__builtin_amdgcn_readlane((int)u, 16))),
               fmaxf(__uint_as_float((unsigned)__builtin_amdgcn_readlane((int)u, 32)),
                     __uint_as_float((unsigned)__builtin_amdgcn_readlane((int)u, 48))));
}
__device__ inline float route_wave_sum(float v) {
  v += __uint_as_float(dpp_u32<0xB1>(__float_as_uint(v)));
  v += __uint_as_float(dpp_u32<0x4E>(__float_as_uint(v)));
  v += __uint_as_float(dpp_u32<0x141>(__float_as_uint(v)));
  v += __uint_as_float(dpp_u32<0x140>(__float_as_uint(v)));
  const unsigned u = __float_as_uint(v);
  return (__uint_as_float((unsigned)__builtin_amdgcn_readlane((int)u, 0)) +
          __uint_as_float((unsigned)__builtin_amdgcn_readlane((int)u, 16))) +
         (__uint_as_float((unsigned)__builtin_amdgcn_readlane((int)u, 32)) +
          __uint_as_float((unsigned)__builtin_amdgcn_readlane((int)u, 48)));
}
template <int CTRL>
__device__ inline unsigned long long dpp_max_u64(unsigned long long k) {
  const unsigned long long o = ((unsigned long long)dpp_u32<CTRL>((unsigned)(k >> 32)) << 32) | dpp_u32<CTRL>((unsigned)k);
  return o > k ? o : k;
}
__device__ inline unsigned long long route_wave_max_u64(unsigned long long k) {
  k = dpp_max_u64<0xB1>(k);
  k = dpp_max_u64<0x4E>(k);
  k = dpp_max_u64<0x141>(k);
  k = dpp_max_u64<0x140>(k);
  unsigned long long m = 0ull;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const unsigned long long x = ((unsigned long long)(unsigned)__builtin_amdgcn_readlane((int)(unsigned)(k >> 32), 16 * r) << 32) |
                                 (unsigned)__builtin_amdgcn_readlane((int)(unsigned)k, 16 * r);
    m = x > m ? x : m;
  }
  return m;
}

// One block of 16 waves.  Wave w routes tokens w, w + 16, ... (at most 4): the logits of
// all its tokens are loaded first (one memory round trip), then per token the E <= 256 bf16
// logits (4 per lane), softmax in fp32, TK rounds of the largest remaining probability
// (lowest expert on ties), weights renormalised over the selection in selection order.
// The selections stay in LDS: thread e counts expert e's pairs (16-byte LDS reads), a scan
// over the experts gives the touched list and the offsets, and thread e writes its pairs
// in ascending order.
constexpr int MOE_ROUTE_PAIRS = 64 * 8;  // M <= 64 tokens x TK <= 8
constexpr int MOE_ROUTE_WAVES = 16;
constexpr int MOE_ROUTE_TPW = 64 / MOE_ROUTE_WAVES;  // tokens per wave, at most
typedef int route_i4 __attribute__((ext_vector_type(4)));

__global__ void __launch_bounds__(64 * MOE_ROUTE_WAVES) moe_route_kernel(const uint16_t* logits, int M, int E, int TK,
                                                                         MoeRoute rt) {
  __shared__ __align__(16) int s_sel[MOE_ROUTE_PAIRS];
  __shared__ int s_cnt[256], s_act[256];
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  float lg[MOE_ROUTE_TPW][4];
#pragma unroll
  for (int u = 0; u < MOE_ROUTE_TPW; ++u) {
    const int t = wave + MOE_ROUTE_WAVES * u;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int ex = lane + 64 * j;
      lg[u][j] = t < M && ex < E ? bf16_to_f32(logits[(size_t)t * E + ex]) : -INFINITY;
    }
  }
#pragma unroll
  for (int u = 0; u < MOE_ROUTE_TPW; ++u) {
    const int t = wave + MOE_ROUTE_WAVES * u;
    if (t >= M) break;  // uniform per wave
    float p[4];
    float mx = -INFINITY;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      p[j] = lg[u][j];
      mx = fmaxf(mx, p[j]);
    }
    mx = route_wave_max(mx);
    float den = 0.f;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      p[j] = lane + 64 * j < E ? expf(p[j] - mx) : 0.f;
      den += p[j];
    }
    den = route_wave_sum(den);
#pragma unroll
    for (int j = 0; j < 4; ++j) p[j] /= den;
    unsigned taken = 0u;  // bit j: expert lane + 64 j already selected
    float wsum = 0.f, wmine = 0.f;
    for (int kk = 0; kk < TK; ++kk) {
      // key: probability bits (non-negative floats order as unsigned) over the inverted index
      unsigned long long best = 0ull;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int ex = lane + 64 * j;
        if (ex < E && !((taken >> j) & 1u)) {
          const unsigned long long k = ((unsigned long long)__float_as_uint(p[j]) << 32) | (0xFFFFFFFFu - (unsigned)ex);
          best = k > best ? k : best;
        }
      }
      best = route_wave_max_u64(best);
      const int ex = (int)(0xFFFFFFFFu - (unsigned)(best & 0xFFFFFFFFull));
      const float w = __uint_as_float((unsigned)(best >> 32));
      if ((ex & 63) == lane) taken |= 1u << (ex >> 6);
      wsum += w;
      if (lane == kk) wmine = w;  // lane kk keeps the kk-th selection's weight
      if (lane == 0) s_sel[t * TK + kk] = ex;
    }
    if (lane < TK) {
      rt.wts[t * TK + lane] = wmine / wsum;
    }
  }
  const int P = M * TK, P4 = (P + 3) / 4;
  if (tid < 4 * P4 - P) s_sel[P + tid] = -1;  // the last 16-byte group's padding
  __syncthreads();
  for (int i = tid; i < P; i += 64 * MOE_ROUTE_WAVES) rt.sel[i] = s_sel[i];
  const route_i4* sel4 = reinterpret_cast<const route_i4*>(s_sel);
  int n = 0;
  if (tid < E) {
#pragma unroll 8
    for (int i = 0; i < P4; ++i) {
      const route_i4 v = sel4[i];
      n += (v.x == tid) + (v.y == tid) + (v.z == tid) + (v.w == tid);
    }
  }
  if (tid < 256) {
    s_cnt[tid] = n;
    s_act[tid] = n > 0 ? 1 : 0;
  }
  __syncthreads();
  // exclusive offsets of the pair counts and of the touched experts: wave 0 scans the
  // 256 entries, 4 consecutive per lane (lane sums, then a 6-step inclusive lane scan)
  if (wave == 0) {
    int c[4], a[4], cs = 0, as = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      c[j] = s_cnt[4 * lane + j];
      a[j] = s_act[4 * lane + j];
      cs += c[j];
      as += a[j];
    }
    int ci = cs, ai = as;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int cu = __shfl_up(ci, o), au = __shfl_up(ai, o);
      if (lane >= o) {
        ci += cu;
        ai += au;
      }
    }
    int ce = ci - cs, ae = ai - as;  // exclusive prefix of this lane's first entry
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      s_cnt[4 * lane + j] = ce;  // exclusive offsets now
      s_act[4 * lane + j] = ae;
      ce += c[j];
      ae += a[j];
    }
    if (lane == 63) {
      rt.off[ai] = ci;
      *rt.n_active = ai;
    }
  }
  __syncthreads();
  if (tid < 256 && n > 0) {
    const int first = s_cnt[tid];  // exclusive offset of expert tid's pairs
    const int slot = s_act[tid];
    rt.act_e[slot] = tid;
    rt.off[slot] = first;
    int o = first;
    int32_t* sp = rt.slot_pairs + (size_t)slot * 64;
    for (int i = 0; i < P4; ++i) {
      const route_i4 v = sel4[i];
#pragma unroll
      for (int h = 0; h < 4; ++h)
        if (v[h] == tid) {
          sp[o - first] = 4 * i + h;
          rt.pairs[o++] = 4 * i + h;
        }
    }
  }
}

int launch_moe_route(const uint16_t* logits, int M, int E, int TK, const MoeRoute& rt, hipStream_t st) {
  if (E < 1 || E > 256 || TK < 1 || TK > 8 || TK > E) return fail(MC_E_INVALID, "moe route: experts (<= 256) / top-k (<= 8)");
  if (M < 1) return MC_OK;
  if (M * TK > MOE_ROUTE_PAIRS) return fail(MC_E_INVALID, "moe route: more than 64 tokens");
  hipLaunchKernelGGL(moe_route_kernel, dim3(1), dim3(64 * MOE_ROUTE_WAVES), 0, st, logits, M, E, TK, rt);
  MC_HIP(hipGetLastError());
  return MC_OK;
}

// Block per (row, 256 columns): thread n sums its pairs' outputs in kk order, adds the
// residual; 16-lane groups form the tile sums of squares of the new row.
__global__ void __launch_bounds__(256) moe_combine_kernel(uint16_t* x, const float* yd, const float* wts, int TK, int H,
                                                          float* ss) {
  const int t = blockIdx.y, n = blockIdx.x * 256 + threadIdx.x;
  float q = 0.f;
  if (n < H) {
    float mo = 0.f;
    for (int kk = 0; kk < TK; ++kk) mo += wts[t * TK + kk] * yd[((size_t)t * TK + kk) * H + n];
    uint16_t* xp = x + (size_t)t * H + n;
    const uint16_t h = f32_to_bf16(bf16_to_f32(*xp) + mo);
    *xp = h;
    const float r = bf16_to_f32(h);
    q = r * r;
  }
#pragma unroll
  for (int o = 1; o < 16; o <<= 1) q += __shfl_xor(q, o);
  if (n < H && (threadIdx.x & 15) == 0) ss[(size_t)t * (H / 16) + n / 16] = q;
}

int launch_moe_combine(uint16_t* x, const float* yd, const float* wts, int M, int TK, int H, float* ss, hipStream_t st) {
  if (H % 16) return fail(MC_E_INVALID, "moe combine: hidden size must be a multiple of 16");
  if (M < 1) return MC_OK;
  hipLaunchKernelGGL(moe_combine_kernel, dim3((H + 255) / 256, M), dim3(256), 0, st, x, yd, wts, TK, H, ss);
  MC_HIP(hipGetLastError());
  return MC_OK;
}

int gemv_setup_lds() {
  int rc;
  if ((rc = setup_mt<1>())) return rc;
  const void* mid[] = {(const void*)qgemv_mid_kernel<2, 4>, (const void*)qgemv_mid_kernel<2, 6>,
                       (const void*)qgemv_mid_kernel<2, 8>, (const void*)qgemv_mid_kernel<3, 4>,
                       (const void*)qgemv_mid_kernel<3, 6>, (const void*)qgemv_mid_kernel<3, 8>,
                       (const void*)qgemv_mid_kernel<4, 4>, (const void*)qgemv_mid_kernel<4, 6>,
                       (const void*)qgemv_mid_kernel<4, 8>};
  for (const void* f : mid) MC_HIP(hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, MID_LDS_CAP));
  const void* moe[] = {(const void*)moe_gemv_kernel<4>};
  for (const void* f : moe)
    MC_HIP(hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, (int)moe_lds_bytes(MOE_MAX_GP)));
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
  const int t = nd >> 4, r = nd & 15;
  const int gp = g >> 1, gi = g & 1;
  return tile_sb_word(t, r, gp, gi, L.GP);
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
