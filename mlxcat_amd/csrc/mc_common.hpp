// mc_common.hpp -- shared definitions for the gfx950 kernels and the C-ABI host code.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <algorithm>
#include <cstdio>
#include <string>

#include "../../include/mlxcat_hip.h"

// Dynamic LDS and register-placement hints.  The CPU emulation of the kernels (tests/emu)
// compiles the sources as host C++ and supplies its own definitions of these.
#ifndef MC_EMULATE
#define MC_DYN_LDS(name) extern __shared__ __align__(16) unsigned char name[]
#define MC_OPAQUE(x) asm volatile("" : "+v"(x))
#define MC_OPAQUE2(x, y) asm volatile("" : "+v"(x), "+v"(y))
#define MC_FENCE() asm volatile("" ::: "memory")
#define MC_TO_VGPR(dst, src) asm volatile("v_mov_b32 %0, %1" : "=v"(dst) : "s"(src))
#define MC_TRACE_TIMEOUT(site) ((void)0)
#endif

namespace mc {

// ---------------------------------------------------------------------------
// error plumbing
// ---------------------------------------------------------------------------
void set_error(const std::string& msg);
int fail(int code, const std::string& msg);
int hip_fail(hipError_t e, const char* what, const char* file, int line);

#define MC_HIP(expr)                                                      \
  do {                                                                    \
    hipError_t _e = (expr);                                               \
    if (_e != hipSuccess) return ::mc::hip_fail(_e, #expr, __FILE__, __LINE__); \
  } while (0)

// ---------------------------------------------------------------------------
// bf16 and hashing helpers, identical on host and device
// ---------------------------------------------------------------------------
__host__ __device__ inline float bf16_to_f32(uint16_t h) {
  return __builtin_bit_cast(float, (uint32_t)h << 16);
}
// Round to nearest even.  On the device this is gfx950's v_cvt_pk_bf16_f32; the host
// restatement gives the same bits for every non-NaN input.
__host__ __device__ inline uint16_t f32_to_bf16(float f) {
#if defined(__HIP_DEVICE_COMPILE__)
  return __builtin_bit_cast(uint16_t, (__bf16)f);
#else
  uint32_t u = __builtin_bit_cast(uint32_t, f);
  if ((u & 0x7F800000u) == 0x7F800000u && (u & 0x007FFFFFu)) return (uint16_t)((u >> 16) | 0x40);
  uint32_t r = u + 0x7FFFu + ((u >> 16) & 1u);
  return (uint16_t)(r >> 16);
#endif
}

// order-preserving 16-bit key of a bf16 value, with -0 folded into +0
__host__ __device__ inline uint32_t bf16_order_key(uint16_t h) {
  if ((h & 0x7FFFu) == 0) h = 0;
  return (h & 0x8000u) ? (uint32_t)(~h & 0xFFFFu) : (uint32_t)(h | 0x8000u);
}

// splitmix64 finalizer (Steele, Lea, Flood 2014)
__host__ __device__ inline uint64_t mix64(uint64_t z) {
  z += 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

// 32-bit uniform for (seed, per-row draw counter, position, kind); kind 0 = accept
// test, 1 = sample draw.
__host__ __device__ inline uint32_t uniform_u32(uint64_t seed, uint64_t counter, uint32_t pos,
                                                uint32_t kind) {
  uint64_t h = mix64(seed ^ 0x5851F42D4C957F2Dull);
  h = mix64(h ^ counter);
  h = mix64(h ^ (((uint64_t)pos << 8) | kind));
  return (uint32_t)(h >> 32);
}

// tensor ids of the synthetic generator
enum { T_Q = 0, T_K = 1, T_V = 2, T_O = 3, T_GATE = 4, T_UP = 5, T_DOWN = 6, T_IN_NORM = 7,
       T_POST_NORM = 8, T_Q_NORM = 9, T_K_NORM = 10, T_ROUTER = 11 };
inline uint64_t tensor_id(int layer, int which) { return ((uint64_t)(layer + 1) << 8) | (uint64_t)which; }
inline uint64_t expert_tensor_id(int layer, int expert, int which) {
  return 0x100000000ull | ((uint64_t)layer << 20) | ((uint64_t)expert << 4) | (uint64_t)which;
}
constexpr uint64_t TID_EMBED = 0xE0000001ull;
constexpr uint64_t TID_LM_HEAD = 0xE0000002ull;
constexpr uint64_t TID_FINAL_NORM = 0xE0000003ull;

// ---------------------------------------------------------------------------
// exp(x), x <= 0, with a fixed operation sequence: y = x*log2(e), n = rint(y),
// f = y - n, 2^f by the degree-7 Taylor polynomial in (f ln2) in Horner form
// with fused multiply-adds, exact ldexp.  Used for the integer acceptance masses
// so that CPU and GPU decisions agree bit for bit.
// ---------------------------------------------------------------------------
__device__ inline float exp_neg_det(float x) {
#pragma clang fp contract(off)
  if (!(x > -87.0f)) return 0.0f;
  const float LOG2E = 1.44269504088896341f;
  float y = x * LOG2E;
  float n = __builtin_rintf(y);
  float f = y - n;
  if (n < -40.0f) return 0.0f;
  float p = 1.52527338e-05f;
  p = __builtin_fmaf(p, f, 1.54035304e-04f);
  p = __builtin_fmaf(p, f, 1.33335581e-03f);
  p = __builtin_fmaf(p, f, 9.61812911e-03f);
  p = __builtin_fmaf(p, f, 5.55041087e-02f);
  p = __builtin_fmaf(p, f, 2.40226507e-01f);
  p = __builtin_fmaf(p, f, 6.93147181e-01f);
  p = __builtin_fmaf(p, f, 1.0f);
  return __builtin_ldexpf(p, (int)n);
}

__device__ inline uint64_t mass_of(float e) {
#pragma clang fp contract(off)
  return (uint64_t)__builtin_rintf(e * 4294967296.0f);
}

// ---------------------------------------------------------------------------
// packed weight layout ("tile layout") for the dequant GEMV
//
// A linear of N outputs and K inputs is stored as NT = ceil(N/16) row tiles by
// GP = ceil(K/128) group pairs.  Each (tile, group pair) is a 1 KiB block read by
// one wave with one 16-byte load per lane: lane l holds row 16t + (l & 15) and
// k-slot block c = l >> 4; its four words are [group 2gp, MFMA 0], [2gp, MFMA 1],
// [2gp+1, MFMA 0], [2gp+1, MFMA 1].  MFMA a of group g covers physical k =
// 64g + 32a + 8c + i, i = 0..7, i.e. exactly MLX word kw = 8g + 4a + c.  Within a
// word, element i sits at bits 4(i/2) for even i and 16 + 4(i/2) for odd i, so
// ((w << 3) >> 4p) & 0x00780078 | 0x3F803F80 puts the nibble pair in the top four mantissa
// bits of two bf16 ones: the pair (1 + q_2p / 16, 1 + q_2p+1 / 16).  A group's dot product
// then folds as s q.x + b sum(x) = 16 s (v.x) - 16 s sum(x) + b sum(x): the offset (1) is
// of the order of the signal (q / 16), so the fp32 accumulation of v.x loses no more than
// a bit to the cancellation (an offset of 128 with q in the low bits would lose about 4).
//
// Scales/biases: uint32 (scale bf16 | bias bf16 << 16) at
// sb[((t * 16 + r) * GP + gp) * 2 + gi] for row 16t + r, group 2gp + gi ([NT][16][GP][2]):
// the lane that owns weight row r of the tile reads one group pair's two groups with one
// 8-byte load, or two consecutive group pairs with one 16-byte load.
// Rows >= N and groups >= K/64 are zero (scale = bias = 0, so they add nothing).
// ---------------------------------------------------------------------------
__host__ __device__ inline size_t tile_sb_word(int t, int r, int gp, int gi, int GP) {
  return (((size_t)t * 16 + r) * GP + gp) * 2 + gi;
}
constexpr uint32_t DQ_MASK = 0x00780078u;   // the nibble pair at mantissa bits 3..6
constexpr uint32_t DQ_MAGIC = 0x3F803F80u;  // two bf16 ones
constexpr float DQ_STEP = 16.0f;            // v = 1 + q / DQ_STEP

struct QLinear {
  int N = 0, K = 0, NT = 0, GP = 0;
  uint32_t* qw = nullptr;  // NT * GP * 256 words
  uint32_t* sb = nullptr;  // NT * GP * 32 words
  size_t qw_words() const { return (size_t)NT * GP * 256; }
  size_t sb_words() const { return (size_t)NT * GP * 32; }
  // algorithmic bytes of the MLX format: N*K/2 nibbles + 4 bytes per group of 64
  double alg_bytes() const { return (double)N * K * 0.5 + (double)N * (K / 64) * 4.0; }
};

__host__ __device__ inline uint32_t permute_mlx_word(uint32_t w) {
  // MLX word: element i at bits 4i.  Tile word: even i at 4(i/2), odd i at 16 + 4(i/2).
  uint32_t out = 0;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    uint32_t q = (w >> (4 * i)) & 0xFu;
    int sh = (i & 1) ? 16 + 4 * (i >> 1) : 4 * (i >> 1);
    out |= q << sh;
  }
  return out;
}
__host__ __device__ inline uint32_t unpermute_tile_word(uint32_t w) {
  uint32_t out = 0;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    int sh = (i & 1) ? 16 + 4 * (i >> 1) : 4 * (i >> 1);
    uint32_t q = (w >> sh) & 0xFu;
    out |= q << (4 * i);
  }
  return out;
}

// synthetic MLX word / scale generation (matches the oracle's or_gen_linear)
__host__ __device__ inline uint32_t synth_mlx_word(uint64_t base, int n, int KW, int kw) {
  uint64_t idx = ((uint64_t)n * (uint64_t)KW + (uint64_t)kw) * 2u;
  uint64_t h0 = mix64(base ^ idx), h1 = mix64(base ^ (idx + 1));
  uint32_t w = 0;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    uint64_t h = j < 4 ? h0 : h1;
    uint32_t q = (uint32_t)__builtin_popcountll((h >> (15 * (j & 3))) & 0x7FFFull);
    w |= q << (4 * j);
  }
  return w;
}
__host__ __device__ inline uint32_t synth_scale_bias(uint64_t base, int n, int G, int g, int scale_exp) {
  uint64_t h = mix64(base ^ 0xA5A5A5A500000000ull ^ ((uint64_t)n * (uint64_t)G + (uint64_t)g));
  uint16_t sb = (uint16_t)(((uint32_t)(127 + scale_exp) << 7) | (0x28u + (uint32_t)(h & 0xFu)));
  float s = bf16_to_f32(sb);
  uint16_t bb = f32_to_bf16(-7.5f * s);
  return (uint32_t)sb | ((uint32_t)bb << 16);
}
inline uint64_t synth_base(uint64_t seed, uint64_t tid) { return mix64(seed ^ mix64(tid)); }

// Device-coherent 64-bit store / load (relaxed, agent scope: sc1 accesses).  Split-K and
// split-KV partials travel through these: a store is written through to the device's
// coherence point and a load misses the CU's L1, so a block on another XCD reads the
// value once the writer's arrival (an agent-scope atomic issued after the store has
// completed) is visible.
__device__ inline void st_coherent(float* p, float a, float b) {
  const unsigned long long v = (unsigned long long)__float_as_uint(a) | ((unsigned long long)__float_as_uint(b) << 32);
  __hip_atomic_store(reinterpret_cast<unsigned long long*>(p), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ inline float2 ld_coherent(const float* p) {
  const unsigned long long v =
      __hip_atomic_load(reinterpret_cast<const unsigned long long*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return make_float2(__uint_as_float((unsigned)v), __uint_as_float((unsigned)(v >> 32)));
}

// Sum over the 8 lanes (l & ~7) .. + 7, the same value in each: DPP quad swaps (xor 1, xor 2),
// then the half-row mirror (lane 7 - l of the other quad holds the other quad's sum).
__device__ inline float sum8_lanes(float v) {
  v += __uint_as_float((unsigned)__builtin_amdgcn_update_dpp(0, (int)__float_as_uint(v), 0xB1, 0xF, 0xF, false));
  v += __uint_as_float((unsigned)__builtin_amdgcn_update_dpp(0, (int)__float_as_uint(v), 0x4E, 0xF, 0xF, false));
  v += __uint_as_float((unsigned)__builtin_amdgcn_update_dpp(0, (int)__float_as_uint(v), 0x141, 0xF, 0xF, false));
  return v;
}

}  // namespace mc
