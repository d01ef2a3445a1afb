// mc_kernels.hip -- per-token kernels of the verify forward for gfx950:
// quantized-embedding gather, fused q/k-norm + RoPE + KV append, and
// split-KV GQA attention over each row's contiguous K/V (one query block per
// (row, kv head): the (K+1) verify positions x the GQA group share every key load).
//
// Semantics follow the mlx-lm decoder the reference runs (external to its tree):
// RMSNorm y = (x * rsqrt(mean(x^2) + eps)) * w, rotate-half RoPE with a per-row
// position (the reference's per-row RoPE offsets, Sources/MLXCat/TrackB/BatchCache.swift:123-139),
// causal attention where the query at position p sees keys [0, p]
// (Sources/MLXCat/TrackB/CausalMask.swift:4-28).
#include "mc_kernels.hpp"

#include <algorithm>

namespace mc {

typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

// ---------------------------------------------------------------------------
// embedding: dequantised row of the tile-layout [V, H] tensor, bf16(fma(s, q, b)).
// One thread per (token, 16 hidden elements); it also writes the 16 elements' sum of
// squares (ssq[m * ss_ld + t]): the RMSNorm partials of the first linear's input.
// ---------------------------------------------------------------------------
__global__ void embed_kernel(QLinear E, const int32_t* slot_tok, int M, int H, uint16_t* x, float* ssq, int ss_ld) {
  const int nt = H / 16;
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= M * nt) return;
  const int m = i / nt, tt = i - m * nt;
  int tok = slot_tok[m];
  if (tok < 0 || tok >= E.N) tok = 0;
  const int t = tok >> 4, r = tok & 15;
  float q = 0.f;
#pragma unroll
  for (int half = 0; half < 2; ++half) {
    const int kw = tt * 2 + half;
    const int g = kw >> 3, w8 = kw & 7, am = w8 >> 2, c = w8 & 3;
    const int gp = g >> 1, gi = g & 1;
    const uint32_t word = E.qw[(((size_t)t * E.GP + gp) * 64 + c * 16 + r) * 4 + gi * 2 + am];
    const uint32_t sbw = E.sb[tile_sb_word(t, r, gp, gi, E.GP)];
    const float s = bf16_to_f32((uint16_t)(sbw & 0xFFFFu)), b = bf16_to_f32((uint16_t)(sbw >> 16));
    uint32_t out[4];
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      const uint16_t h0 = f32_to_bf16(__builtin_fmaf(s, (float)((word >> (4 * p)) & 0xFu), b));       // element 2p
      const uint16_t h1 = f32_to_bf16(__builtin_fmaf(s, (float)((word >> (16 + 4 * p)) & 0xFu), b));  // element 2p + 1
      const float v0 = bf16_to_f32(h0), v1 = bf16_to_f32(h1);
      q += v0 * v0;
      q += v1 * v1;
      out[p] = (uint32_t)h0 | ((uint32_t)h1 << 16);
    }
    const u32x4 v = {out[0], out[1], out[2], out[3]};
    *reinterpret_cast<u32x4*>(x + (size_t)m * H + kw * 8) = v;
  }
  ssq[(size_t)m * ss_ld + tt] = q;
}

int launch_embed(const QLinear& E, const int32_t* slot_tok, int M, int H, uint16_t* x, float* ssq, int ss_ld,
                 hipStream_t st) {
  if (H % 16) return fail(MC_E_INVALID, "embed: hidden size must be a multiple of 16");
  const int total = M * (H / 16);
  hipLaunchKernelGGL(embed_kernel, dim3((total + 255) / 256), dim3(256), 0, st, E, slot_tok, M, H, x, ssq, ss_ld);
  MC_HIP(hipGetLastError());
  return MC_OK;
}

// ---------------------------------------------------------------------------
// block reductions (fixed order)
// ---------------------------------------------------------------------------
__device__ inline float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  return v;
}
__device__ inline float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
  return v;
}

// ---------------------------------------------------------------------------
// QB head vectors per wave at once (independent latency chains) in two steps, so that a
// caller can issue other loads in between: rope_load issues the loads of vector i (hp[i] at
// position pos[i]) and rope_finish normalises and rotates them.  Every load is unconditional,
// from an in-bounds address (lanes >= d/2 read lane 0's elements), and is selected afterwards:
// a load under a lane or ok[i] condition becomes a branch with its own wait, and the QB
// vectors would then load one round trip after another.  ok[i] false drops vector i; hp[i]
// and pos[i] must still address a readable vector.
template <int QB>
struct RopeRegs {
  uint16_t x1[QB], x2[QB], w1, w2;
  float cs[QB], sn[QB];
  bool v[QB];
};

template <int QB>
__device__ inline void rope_load(RopeRegs<QB>& g, const uint16_t* const (&hp)[QB], const int (&pos)[QB],
                                 const bool (&ok)[QB], const uint16_t* nw, const float* rope_cos,
                                 const float* rope_sin, int d, int lane) {
  const int hd = d >> 1;
  const int l = lane < hd ? lane : 0;
  const uint16_t* wp = nw ? nw : hp[0];  // without a norm the weights are read and not used
  g.w1 = wp[l];
  g.w2 = wp[l + hd];
#pragma unroll
  for (int i = 0; i < QB; ++i) {
    g.v[i] = ok[i] && lane < hd;
    g.x1[i] = hp[i][l];
    g.x2[i] = hp[i][l + hd];
    g.cs[i] = rope_cos[(size_t)pos[i] * hd + l];
    g.sn[i] = rope_sin[(size_t)pos[i] * hd + l];
  }
}

template <int QB>
__device__ inline void rope_finish(RopeRegs<QB>& g, bool norm, int d, float eps, int lane, uint16_t (&o1)[QB],
                                   uint16_t (&o2)[QB]) {
#pragma clang fp contract(off)
  // the weights are taken here, with the vectors: otherwise their loads sink into the norm
  // branch and start one round trip later
  asm volatile("" ::"v"((uint32_t)g.w1), "v"((uint32_t)g.w2));
  float x1[QB], x2[QB];
#pragma unroll
  for (int i = 0; i < QB; ++i) {
    x1[i] = g.v[i] ? bf16_to_f32(g.x1[i]) : 0.f;
    x2[i] = g.v[i] ? bf16_to_f32(g.x2[i]) : 0.f;
  }
  if (norm) {
    const float w1 = bf16_to_f32(g.w1), w2 = bf16_to_f32(g.w2);
    float ss[QB];
#pragma unroll
    for (int i = 0; i < QB; ++i) ss[i] = x1[i] * x1[i] + x2[i] * x2[i];
#pragma unroll
    for (int o = 32; o > 0; o >>= 1)
#pragma unroll
      for (int i = 0; i < QB; ++i) ss[i] += __shfl_xor(ss[i], o);
#pragma unroll
    for (int i = 0; i < QB; ++i) {
      const float r = 1.0f / sqrtf(ss[i] / (float)d + eps);
      if (g.v[i]) {
        x1[i] = bf16_to_f32(f32_to_bf16((x1[i] * r) * w1));
        x2[i] = bf16_to_f32(f32_to_bf16((x2[i] * r) * w2));
      }
    }
  }
#pragma unroll
  for (int i = 0; i < QB; ++i) {
    o1[i] = g.v[i] ? f32_to_bf16(x1[i] * g.cs[i] - x2[i] * g.sn[i]) : (uint16_t)0;
    o2[i] = g.v[i] ? f32_to_bf16(x1[i] * g.sn[i] + x2[i] * g.cs[i]) : (uint16_t)0;
  }
}

// ---------------------------------------------------------------------------
// q/k RMSNorm (Qwen3) + rotate-half RoPE of one head vector by one wave: lane < d/2 holds
// the rotation pair (lane, lane + d/2).  The standalone kernel below and the fused attention
// both go through rope_load / rope_finish, so a key (or query) has the same bits whichever
// path computes it.  Products are not contracted into fused multiply-adds: every step rounds
// where it is written.
// ---------------------------------------------------------------------------
__device__ inline void rope_pair(const uint16_t* hp, const uint16_t* nw, const float* rope_cos, const float* rope_sin,
                                 int d, int pos, float eps, int lane, uint16_t* o1, uint16_t* o2) {
  RopeRegs<1> g;
  const uint16_t* const hps[1] = {hp};
  const int ps[1] = {pos};
  const bool ok[1] = {true};
  rope_load<1>(g, hps, ps, ok, nw, rope_cos, rope_sin, d, lane);
  uint16_t a[1], b[1];
  rope_finish<1>(g, nw != nullptr, d, eps, lane, a, b);
  *o1 = a[0];
  *o2 = b[0];
}

// Grid (slot, head / 4), one wave per head: q heads to q_out, k heads and v heads appended
// to the cache at the slot's position.
__global__ void __launch_bounds__(256) qk_rope_append_kernel(const uint16_t* qkv, const uint16_t* q_norm,
                                                             const uint16_t* k_norm, const float* rope_cos,
                                                             const float* rope_sin, int nq, int nkv, int d,
                                                             float eps, const int32_t* slot_row,
                                                             const int32_t* slot_pos, KVLayer kv, uint16_t* q_out) {
  const int m = blockIdx.x;
  const int row = slot_row[m], pos = slot_pos[m];
  if (row < 0) return;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int hd = d >> 1;
  const int ntot = nq + 2 * nkv;
  const uint16_t* src = qkv + (size_t)m * ntot * d;
  const int hh = blockIdx.y * 4 + wave;  // one wave per head
  if (hh >= ntot) return;
  const uint16_t* hp = src + (size_t)hh * d;
  if (hh >= nq + nkv) {  // V head: copy into the cache
    const int h = hh - nq - nkv;
    uint16_t* dst = kv.v + ((size_t)row * nkv + h) * d * kv.cap + pos;
    for (int i = lane; i < d; i += 64) dst[(size_t)i * kv.cap] = hp[i];
    return;
  }
  const bool is_q = hh < nq;
  uint16_t o1, o2;
  rope_pair(hp, is_q ? q_norm : k_norm, rope_cos, rope_sin, d, pos, eps, lane, &o1, &o2);
  if (lane < hd) {
    uint16_t* dst = is_q ? q_out + (size_t)m * nq * d + (size_t)hh * d
                         : kv.k + (((size_t)row * nkv + (hh - nq)) * kv.cap + pos) * d;
    dst[lane] = o1;
    dst[lane + hd] = o2;
  }
}

int launch_qk_rope_append(const uint16_t* qkv, const uint16_t* q_norm, const uint16_t* k_norm, const float* rope_cos,
                          const float* rope_sin, int M, int nq, int nkv, int d, float eps, const int32_t* slot_row,
                          const int32_t* slot_pos, KVLayer kv, uint16_t* q_out, hipStream_t st) {
  if (d > 128 || (d & 1)) return fail(MC_E_INVALID, "head_dim must be even and <= 128");
  hipLaunchKernelGGL(qk_rope_append_kernel, dim3(M, (nq + 2 * nkv + 3) / 4), dim3(256), 0, st, qkv, q_norm, k_norm,
                     rope_cos, rope_sin, nq, nkv, d, eps, slot_row, slot_pos, kv, q_out);
  MC_HIP(hipGetLastError());
  return MC_OK;
}

// ---------------------------------------------------------------------------
// Split-KV attention, flash-decoding style, without LDS staging of K/V.  Grid
// (R * nkv, splits); block (row, kv head, split) covers keys [split S 64, (split+1) S 64)
// of the row, wave w its 64-key sub-chunks w, w + 4, ... (S >= 2: at S < 4 some waves
// have none and only join the merge).  K rows and V^T rows
// go straight from the cache into MFMA operands:
//   S^T[key][q] = K[key][:] . q[q][:]          v_mfma_f32_16x16x32_bf16 (A = 16 keys x 32 d,
//                                              B = 32 d x 16 queries)
//   O^T[d][q] += V^T[d][key] . P^T[key][q]     v_mfma_f32_16x16x16bf16_1k: the S^T accumulator
//                                              (lane: query l % 16, keys 4 (l / 16) + v) is the
//                                              P^T operand as it stands, split into bf16 hi + lo
// with a running max / sum per query (online softmax).  The four waves' (max, sum, o) are
// merged through LDS in wave order into one partial per (query, split); a query's result
// depends only on its own position and keys.
// ---------------------------------------------------------------------------
typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8_t;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4_t;
typedef short s16x4_t __attribute__((ext_vector_type(4)));
typedef short s16x8_t __attribute__((ext_vector_type(8)));
// query tiles of 16 per pass over the keys: every tile of a (row, kv head) in one pass
// (at most 4, 64 queries), so the keys and values are read once
inline int attn_tiles(int nqry) { return std::min(4, std::max(1, (nqry + 15) / 16)); }

// Merge of one query's split partials 0 .. ns - 1, in split order, for the output element
// pair (e0, e0 + 1): running max, rescaled sums (the arithmetic of the standalone merge
// kernel below, shared by the last-arriving block of the fused attention).
template <bool COHERENT>
__device__ inline float2 merge_splits(const float* pml, const float* po, int ns, int d, int e0) {
  float mx = -INFINITY, l = 0.f, a0 = 0.f, a1 = 0.f;
  constexpr int UN = 8;
  for (int c0 = 0; c0 < ns; c0 += UN) {
    float2 ml[UN], ov[UN];
#pragma unroll
    for (int u = 0; u < UN; ++u) {
      const int cc = c0 + u;
      ml[u] = make_float2(-INFINITY, 0.f);
      ov[u] = make_float2(0.f, 0.f);
      if (cc < ns) {
        ml[u] = COHERENT ? ld_coherent(pml + (size_t)cc * 2) : *reinterpret_cast<const float2*>(pml + (size_t)cc * 2);
        if (e0 < d)
          ov[u] = COHERENT ? ld_coherent(po + (size_t)cc * d + e0) : *reinterpret_cast<const float2*>(po + (size_t)cc * d + e0);
      }
    }
#pragma unroll
    for (int u = 0; u < UN; ++u) {
      const float cm = ml[u].x;
      if (cm == -INFINITY) continue;  // a split with no visible key
      const float nm = fmaxf(mx, cm);
      const float fo = (mx == -INFINITY) ? 0.f : __expf(mx - nm);
      const float fn = __expf(cm - nm);
      l = l * fo + ml[u].y * fn;
      a0 = a0 * fo + ov[u].x * fn;
      a1 = a1 * fo + ov[u].y * fn;
      mx = nm;
    }
  }
  const float inv = 1.0f / l;
  return make_float2(a0 * inv, a1 * inv);
}

// FUSE: the block also prepares its queries and the new keys, and the splits are merged by
// the last block of each (row, kv head) to arrive:
//   * q rows of the row's queries of this kv head (q-norm + RoPE, rope_pair) into LDS;
//   * the new keys / values whose positions fall in this block's key range (k-norm + RoPE)
//     appended to the cache, read back by the block's own waves after a barrier (each new
//     position lies in exactly one block's range);
//   * the block's partials stored device-coherent; an agent-scope arrival count per
//     (row, kv head); the last arrival merges every split in split order into att (the
//     standalone merge's arithmetic) and rearms the count.
// Queries and keys have the same bits as the standalone preparation kernel's; the merge
// weights each split by exp(m_sp - M) / L in one pass (the standalone merge rescales a running
// sum split by split), so attention outputs agree with the three-kernel path to rounding.

template <int D, bool FUSE, int TP>
__global__ void __launch_bounds__(256) attn_flash_kernel(const uint16_t* q, KVLayer kv, SlotView sv, int nq, int nkv,
                                                         float scale, int S, AttnWork w, AttnFuse f) {
  __shared__ float mrg[4][TP][16][D + 2];  // per wave: o[d], max, sum of each query of the pass
  __shared__ __align__(16) uint16_t qs[FUSE ? FUSE_QMAX * D : 8];
  __shared__ int s_last;
  const int G = nq / nkv;
  const int r = blockIdx.x / nkv, kh = blockIdx.x % nkv;
  const int split = blockIdx.y;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, c = lane >> 4, r16 = lane & 15;
  const size_t head = (size_t)r * nkv + kh;
  const uint16_t* kbase = kv.k + head * kv.cap * D;   // [pos][d]
  const uint16_t* vbase = kv.v + head * D * kv.cap;   // [d][pos]
  constexpr int NS = D / 32, NDB = D / 16;
  typedef unsigned u4 __attribute__((ext_vector_type(4)));
  // keys sc .. sc + 63 of the cache (inside the row's cap; keys >= kend are finite and masked)
  // in four 16-key MFMA blocks.  Slot j of block kb = 2 p + h holds key
  //   sc + 32 p + 8 (j / 4) + 4 h + j % 4,
  // so the 4 keys a lane holds of block 2p and the 4 of block 2p + 1 are 8 consecutive
  // positions: one 16-byte load of a V^T row serves both blocks (the sum over keys does
  // not depend on which slot holds which key, as long as K, the mask and V agree).
  bf16x8_t ka[4][4];
  s16x4_t va[NDB][4];
  auto key_of = [&](int kb, int j) { return 32 * (kb >> 1) + 8 * (j >> 2) + 4 * (kb & 1) + (j & 3); };
  auto load_kv = [&](int sc) {
#pragma unroll
    for (int kb = 0; kb < 4; ++kb)
#pragma unroll
      for (int s4 = 0; s4 < 4; ++s4)
        ka[kb][s4] = s4 < NS ? *reinterpret_cast<const bf16x8_t*>(kbase + (size_t)(sc + key_of(kb, r16)) * D + 32 * s4 + 8 * c)
                             : __builtin_bit_cast(bf16x8_t, (u4){0u, 0u, 0u, 0u});
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
      for (int p = 0; p < 2; ++p) {
        const s16x8_t v8 = *reinterpret_cast<const s16x8_t*>(vbase + (size_t)(16 * db + r16) * kv.cap + sc + 32 * p + 8 * c);
        va[db][2 * p] = (s16x4_t){v8[0], v8[1], v8[2], v8[3]};
        va[db][2 * p + 1] = (s16x4_t){v8[4], v8[5], v8[6], v8[7]};
      }
  };
  const int s0 = split * S * ATTN_CHUNK;
  const int sc_first = s0 + ATTN_CHUNK * wave;
  // the row's state, the three loads together (no branch between them)
  const int nv = sv.n_valid[r];
  const int base = sv.qbase[r];
  const int slot0 = sv.row_slot0[r];
  const int nqry = nv * G;
  if (nqry == 0) return;
  const int kend = base + nv;
  if (s0 >= kend) return;
  const int s1 = min(kend, s0 + S * ATTN_CHUNK);
  bool pre = false;  // this wave's first sub-chunk is already in registers
  if constexpr (FUSE) {
    // the queries of this wave and the new keys / values in this block's key range
    const size_t ldq = (size_t)(nq + 2 * nkv) * D;  // row stride of the qkv projections
    constexpr int HD = D / 2, QB = TP * 4, KB = 4;  // queries per wave: at most TP x 16 / 4
    const uint16_t* hq[QB];
    int pq[QB];
    bool oq[QB];
#pragma unroll
    for (int i = 0; i < QB; ++i) {  // queries wave + 4 i
      const int qi = wave + 4 * i;
      oq[i] = qi < nqry;
      const int qc = oq[i] ? qi : 0;
      const int j = qc / G, gh = qc - j * G;
      hq[i] = f.qkv + (size_t)(slot0 + j) * ldq + (size_t)(kh * G + gh) * D;
      pq[i] = base + j;
    }
    RopeRegs<QB> gq;
    rope_load<QB>(gq, hq, pq, oq, f.q_norm, f.rope_cos, f.rope_sin, D, lane);
    // the new keys and values in this block's key range: positions p0 + wave + 4 i
    const int p0 = max(s0, base);
    const uint16_t* hk[KB];
    int pk[KB];
    bool ok[KB];
#pragma unroll
    for (int i = 0; i < KB; ++i) {
      const int p = p0 + wave + 4 * i;
      ok[i] = p < s1;
      pk[i] = ok[i] ? p : p0;
      hk[i] = f.qkv + (size_t)(slot0 + pk[i] - base) * ldq + (size_t)(nq + kh) * D;
    }
    RopeRegs<KB> gk;
    uint16_t vv[KB][D / 64];
    if (p0 < s1) {
      rope_load<KB>(gk, hk, pk, ok, f.k_norm, f.rope_cos, f.rope_sin, D, lane);
#pragma unroll
      for (int i = 0; i < KB; ++i)
#pragma unroll
        for (int e = 0; e < D / 64; ++e) vv[i][e] = hk[i][(size_t)nkv * D + lane + 64 * e];  // stored only if ok[i]
    }
    // loads of the prologue first (the queries of this wave, the new keys / values), then the
    // first sub-chunk of cached keys when it holds no key of this step
    pre = sc_first < s1 && sc_first + ATTN_CHUNK <= base;
    if (pre) load_kv(sc_first);
    uint16_t o1[QB], o2[QB];
    rope_finish<QB>(gq, f.q_norm != nullptr, D, f.eps, lane, o1, o2);
#pragma unroll
    for (int i = 0; i < QB; ++i) {
      const int qi = wave + 4 * i;
      if (oq[i] && lane < HD) {
        qs[qi * D + lane] = o1[i];
        qs[qi * D + lane + HD] = o2[i];
      }
    }
    // batch b of new positions: p0 + 4 KB b + wave + 4 i (the first batch's loads are above)
    uint16_t* kw = kv.k + head * kv.cap * D;
    uint16_t* vw = kv.v + head * D * kv.cap;
    for (int b0 = p0; b0 < s1; b0 += 4 * KB) {
      if (b0 != p0) {
#pragma unroll
        for (int i = 0; i < KB; ++i) {
          const int p = b0 + wave + 4 * i;
          ok[i] = p < s1;
          pk[i] = ok[i] ? p : p0;
          hk[i] = f.qkv + (size_t)(slot0 + pk[i] - base) * ldq + (size_t)(nq + kh) * D;
        }
        rope_load<KB>(gk, hk, pk, ok, f.k_norm, f.rope_cos, f.rope_sin, D, lane);
#pragma unroll
        for (int i = 0; i < KB; ++i)
#pragma unroll
          for (int e = 0; e < D / 64; ++e) vv[i][e] = hk[i][(size_t)nkv * D + lane + 64 * e];  // stored only if ok[i]
      }
      uint16_t k1[KB], k2[KB];
      rope_finish<KB>(gk, f.k_norm != nullptr, D, f.eps, lane, k1, k2);
#pragma unroll
      for (int i = 0; i < KB; ++i) {
        if (!ok[i]) continue;
        if (lane < HD) {
          kw[(size_t)pk[i] * D + lane] = k1[i];
          kw[(size_t)pk[i] * D + lane + HD] = k2[i];
        }
#pragma unroll
        for (int e = 0; e < D / 64; ++e) vw[(size_t)(lane + 64 * e) * kv.cap + pk[i]] = vv[i][e];
      }
    }
    __syncthreads();  // the queries and this range's new keys are visible to every wave
  }
  const int nqt = (nqry + 15) / 16;
  for (int t0 = 0; t0 < nqt; t0 += TP) {
    // B operands: q rows of queries (t0 + tt) 16 + r16, d = 32 s + 8 c .. + 7
    bf16x8_t qb[TP][4];
    int qpos[TP];
#pragma unroll
    for (int tt = 0; tt < TP; ++tt) {
      const int qi = min((t0 + tt) * 16 + r16, nqry - 1);
      const int j = qi / G, gh = qi - j * G;
      qpos[tt] = (t0 + tt) * 16 + r16 < nqry ? base + j : -1;
      const uint16_t* qp = FUSE ? qs + (size_t)qi * D : q + ((size_t)(slot0 + j) * nq + kh * G + gh) * D;
#pragma unroll
      for (int s4 = 0; s4 < 4; ++s4)
        qb[tt][s4] = s4 < NS ? *reinterpret_cast<const bf16x8_t*>(qp + 32 * s4 + 8 * c)
                             : __builtin_bit_cast(bf16x8_t, (u4){0u, 0u, 0u, 0u});
    }
    float mrun[TP], lrun[TP];
    f32x4_t o[TP][NDB];
#pragma unroll
    for (int tt = 0; tt < TP; ++tt) {
      mrun[tt] = -INFINITY;
      lrun[tt] = 0.f;
#pragma unroll
      for (int db = 0; db < NDB; ++db) o[tt][db] = (f32x4_t){0.f, 0.f, 0.f, 0.f};
    }
    for (int sc = sc_first; sc < s1; sc += 4 * ATTN_CHUNK) {
      if (!(pre && t0 == 0 && sc == sc_first)) load_kv(sc);
#pragma unroll
      for (int tt = 0; tt < TP; ++tt) {
        if (t0 + tt >= nqt) break;
        f32x4_t st[4];
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) {
          f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int s4 = 0; s4 < NS; ++s4) acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ka[kb][s4], qb[tt][s4], acc, 0, 0, 0);
          st[kb] = acc;
        }
        float mloc = -INFINITY;
#pragma unroll
        for (int kb = 0; kb < 4; ++kb)
#pragma unroll
          for (int v = 0; v < 4; ++v) {
            const int key = sc + key_of(kb, 4 * c + v);
            const float x = key <= qpos[tt] ? st[kb][v] * scale : -INFINITY;
            st[kb][v] = x;
            mloc = fmaxf(mloc, x);
          }
        mloc = fmaxf(mloc, __shfl_xor(mloc, 16));
        mloc = fmaxf(mloc, __shfl_xor(mloc, 32));
        // a query that sees no key yet keeps max -inf, sum 0 and o 0 (alpha 0, every p 0):
        // no branch, the wave's shuffles and MFMAs stay uniform
        const float mnew = fmaxf(mrun[tt], mloc);
        const float alpha = mrun[tt] == -INFINITY ? 0.f : __expf(mrun[tt] - mnew);
        float lsum = 0.f;
        s16x4_t ph[4], pl[4];
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) {
          short hv[4], lv[4];
#pragma unroll
          for (int v = 0; v < 4; ++v) {
            const float pv = st[kb][v] == -INFINITY ? 0.f : __expf(st[kb][v] - mnew);
            lsum += pv;
            const uint16_t h = f32_to_bf16(pv);
            hv[v] = (short)h;
            lv[v] = (short)f32_to_bf16(pv - bf16_to_f32(h));
          }
          ph[kb] = (s16x4_t){hv[0], hv[1], hv[2], hv[3]};
          pl[kb] = (s16x4_t){lv[0], lv[1], lv[2], lv[3]};
        }
        lsum += __shfl_xor(lsum, 16);
        lsum += __shfl_xor(lsum, 32);
        lrun[tt] = lrun[tt] * alpha + lsum;
        mrun[tt] = mnew;
#pragma unroll
        for (int db = 0; db < NDB; ++db) {
          f32x4_t acc = o[tt][db];
#pragma unroll
          for (int v = 0; v < 4; ++v) acc[v] *= alpha;
#pragma unroll
          for (int kb = 0; kb < 4; ++kb) {
            acc = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(va[db][kb], ph[kb], acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(va[db][kb], pl[kb], acc, 0, 0, 0);
          }
          o[tt][db] = acc;
        }
      }
    }
    // ---- merge the four waves in wave order: one partial per (query, split) ----
#pragma unroll
    for (int tt = 0; tt < TP; ++tt) {
#pragma unroll
      for (int db = 0; db < NDB; ++db)
#pragma unroll
        for (int v = 0; v < 4; ++v) mrg[wave][tt][r16][16 * db + 4 * c + v] = o[tt][db][v];
      if (c == 0) {
        mrg[wave][tt][r16][D] = mrun[tt];
        mrg[wave][tt][r16][D + 1] = lrun[tt];
      }
    }
    __syncthreads();
    // thread: query (tt, qq) = tid / 8 + 32 i (TP x 16 queries), d slice 16 (tid % 8)
    for (int qsel = threadIdx.x >> 3; qsel < TP * 16; qsel += 32) {
      const int part = threadIdx.x & 7;
      const int tt = qsel >> 4, qq = qsel & 15;
      const int qi = (t0 + tt) * 16 + qq;
      if (t0 + tt < nqt && qi < nqry) {
        float mx = -INFINITY;
#pragma unroll
        for (int w2 = 0; w2 < 4; ++w2) mx = fmaxf(mx, mrg[w2][tt][qq][D]);
        float fw[4], l = 0.f;
#pragma unroll
        for (int w2 = 0; w2 < 4; ++w2) {
          const float m2 = mrg[w2][tt][qq][D];
          fw[w2] = m2 == -INFINITY ? 0.f : __expf(m2 - mx);
          l += mrg[w2][tt][qq][D + 1] * fw[w2];
        }
        const int jj = qi / G, gg = qi - jj * G;
        const size_t pidx = ((size_t)(slot0 + jj) * nq + kh * G + gg) * w.nchunk + split;
        for (int e = part * (D / 8); e < (part + 1) * (D / 8); e += 2) {
          float a[2] = {0.f, 0.f};
#pragma unroll
          for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int w2 = 0; w2 < 4; ++w2) a[h] += mrg[w2][tt][qq][e + h] * fw[w2];
          if constexpr (FUSE) st_coherent(w.part_o + pidx * D + e, a[0], a[1]);
          else {
            w.part_o[pidx * D + e] = a[0];
            w.part_o[pidx * D + e + 1] = a[1];
          }
        }
        if (part == 0) {
          if constexpr (FUSE) st_coherent(w.part_ml + pidx * 2, mx, l);
          else {
            w.part_ml[pidx * 2] = mx;
            w.part_ml[pidx * 2 + 1] = l;
          }
        }
      }
    }
    __syncthreads();
  }
  if constexpr (FUSE) {
    // arrival of this split (its partial stores complete first); the last one merges
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    const int nsplit = (kend + S * ATTN_CHUNK - 1) / (S * ATTN_CHUNK);
    if (threadIdx.x == 0)
      s_last = __hip_atomic_fetch_add(f.counters + head, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
               (unsigned)(nsplit - 1);
    __syncthreads();
    if (!s_last) return;
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    if (threadIdx.x == 0) __hip_atomic_store(f.counters + head, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    // Split sp of query qi gets the weight exp(m_sp - M) (M: the query's largest split max)
    // and the query 1 / L, L = sum_sp l_sp exp(m_sp - M); a query at position p holds keys in
    // splits 0 .. p / (S 64) only.  (m, l) of every (query, split) go to LDS first (one load
    // each, all in flight), the weights replace them, then every output element sums its
    // splits' partials with all of a batch's loads in flight.  The pass buffer is free.
    float2* mls = reinterpret_cast<float2*>(&mrg[0][0][0][0]);  // [nqry][nsplit]
    float* invl = reinterpret_cast<float*>(mls + nqry * nsplit);
    for (int i = threadIdx.x; i < nqry * nsplit; i += 256) {
      const int qi = i / nsplit, sp = i - qi * nsplit;
      const int jj = qi / G, gg = qi - jj * G;
      const size_t qh = (size_t)(slot0 + jj) * nq + kh * G + gg;
      mls[i] = sp <= (base + jj) / (S * ATTN_CHUNK) ? ld_coherent(w.part_ml + (qh * w.nchunk + sp) * 2)
                                                   : make_float2(-INFINITY, 0.f);
    }
    __syncthreads();
    for (int qi = threadIdx.x; qi < nqry; qi += 256) {
      float2* q2 = mls + qi * nsplit;
      float mx = -INFINITY;
      for (int sp = 0; sp < nsplit; ++sp) mx = fmaxf(mx, q2[sp].x);
      float l = 0.f;
      for (int sp = 0; sp < nsplit; ++sp) {
        const float e = q2[sp].x == -INFINITY ? 0.f : __expf(q2[sp].x - mx);
        l += q2[sp].y * e;
        q2[sp].x = e;
      }
      invl[qi] = 1.0f / l;
    }
    __syncthreads();
    // thread per (query, 4 elements): the splits' float4 partials, NB per round in flight
    constexpr int NB = 24;
    for (int it = threadIdx.x; it < nqry * (D / 4); it += 256) {
      const int qi = it / (D / 4), e0 = (it - qi * (D / 4)) * 4;
      const int jj = qi / G, gg = qi - jj * G;
      const size_t qh = (size_t)(slot0 + jj) * nq + kh * G + gg;
      const float* po = w.part_o + qh * w.nchunk * D + e0;
      const float2* q2 = mls + qi * nsplit;
      const int ns = (base + jj) / (S * ATTN_CHUNK) + 1;
      float acc[4] = {0.f, 0.f, 0.f, 0.f};
      for (int c0 = 0; c0 < ns; c0 += NB) {
        float2 ov[NB][2];
#pragma unroll
        for (int u = 0; u < NB; ++u) {
          ov[u][0] = ov[u][1] = make_float2(0.f, 0.f);
          if (c0 + u < ns) {
            ov[u][0] = ld_coherent(po + (size_t)(c0 + u) * D);
            ov[u][1] = ld_coherent(po + (size_t)(c0 + u) * D + 2);
          }
        }
#pragma unroll
        for (int u = 0; u < NB; ++u) {
          if (c0 + u >= ns) break;
          const float e = q2[c0 + u].x;
          acc[0] += ov[u][0].x * e;
          acc[1] += ov[u][0].y * e;
          acc[2] += ov[u][1].x * e;
          acc[3] += ov[u][1].y * e;
        }
      }
      const float il = invl[qi];
      uint2 o;
      o.x = (uint32_t)f32_to_bf16(acc[0] * il) | ((uint32_t)f32_to_bf16(acc[1] * il) << 16);
      o.y = (uint32_t)f32_to_bf16(acc[2] * il) | ((uint32_t)f32_to_bf16(acc[3] * il) << 16);
      *reinterpret_cast<uint2*>(f.att + qh * D + e0) = o;
    }
  }
}

// One wave per (slot, head): merge the split partials 0..ns-1 in split order with a running
// max (each lane owns d/64 output elements); loads of 8 splits are in flight at a time.
__global__ void __launch_bounds__(256) attn_merge_kernel(SlotView sv, int M, int nq, int d, int S, AttnWork w,
                                                         uint16_t* att) {
  const int wid = (blockIdx.x * blockDim.x + threadIdx.x) >> 6, lane = threadIdx.x & 63;
  if (wid >= M * nq) return;
  const int m = wid / nq, h = wid - m * nq;
  uint16_t* out = att + ((size_t)m * nq + h) * d;
  const int row = sv.slot_row[m];
  const int e0 = lane * 2;  // d <= 128: lane owns elements e0, e0 + 1
  if (row < 0) {
    if (e0 < d) *reinterpret_cast<uint32_t*>(out + e0) = 0u;
    return;
  }
  const int ns = sv.slot_pos[m] / (S * ATTN_CHUNK) + 1;
  const size_t qh = (size_t)m * nq + h;
  const float2 o = merge_splits<false>(w.part_ml + qh * w.nchunk * 2, w.part_o + qh * w.nchunk * d, ns, d, e0);
  if (e0 < d) *reinterpret_cast<uint32_t*>(out + e0) = (uint32_t)f32_to_bf16(o.x) | ((uint32_t)f32_to_bf16(o.y) << 16);
}

// 64-key sub-chunks per block: more when the grid would exceed about 1024 blocks (fewer
// partials to merge), at least 8 from 64 (row, kv head) pairs on (two sub-chunks per wave,
// 4x fewer partials; batch 8 at 2K keys 5.08 -> 4.89 ms per step, 8 rows at 512-4096 keys
// 6.71 -> 6.28 ms), else 3: a decode row spreads its heads over more CUs, while the
// last-arriving block's merge reads fewer partials.  Qwen3-4B shape, one row at ~2.3K keys,
// per step with a one-token verify / with six verify tokens: 2 sub-chunks 2.33 / 2.71 ms,
// 3: 2.33 / 2.64, 4: 2.34 / 2.63.
int attn_split(int R, int nkv, int nchunk, bool fused) {
  const int smin = R * nkv >= 64 ? 8 : 3;
  return std::max(smin, (R * nkv * nchunk + 1023) / 1024);
}

bool attn_fuse_ok(int R, int nkv, int nchunk, int max_q, int nq, int d) {
  const int nqry = max_q * (nq / nkv);
  if (nqry > FUSE_QMAX) return false;
  // the merging block keeps (m, l) per (query, split) and 1 / L per query in the pass buffer
  const int S = attn_split(R, nkv, nchunk, true), TP = attn_tiles(nqry);
  const size_t words = (size_t)TP * 16 * (2 * ((nchunk + S - 1) / S) + 1);
  return words <= (size_t)4 * TP * 16 * (d + 2);
}

template <int D, bool FUSE>
static void launch_flash(int TP, dim3 grid, hipStream_t st, const uint16_t* q, const KVLayer& kv, const SlotView& sv,
                         int nq, int nkv, float scale, int S, const AttnWork& w, const AttnFuse& f) {
  switch (TP) {
    case 1: hipLaunchKernelGGL((attn_flash_kernel<D, FUSE, 1>), grid, dim3(256), 0, st, q, kv, sv, nq, nkv, scale, S, w, f); break;
    case 2: hipLaunchKernelGGL((attn_flash_kernel<D, FUSE, 2>), grid, dim3(256), 0, st, q, kv, sv, nq, nkv, scale, S, w, f); break;
    case 3: hipLaunchKernelGGL((attn_flash_kernel<D, FUSE, 3>), grid, dim3(256), 0, st, q, kv, sv, nq, nkv, scale, S, w, f); break;
    default: hipLaunchKernelGGL((attn_flash_kernel<D, FUSE, 4>), grid, dim3(256), 0, st, q, kv, sv, nq, nkv, scale, S, w, f); break;
  }
}

int launch_attention(const uint16_t* q, KVLayer kv, const SlotView& sv, int R, int max_q, int nq, int nkv, int d,
                     int M, const AttnWork& w, const AttnFuse* fuse, uint16_t* att, hipStream_t st) {
  if (d != 64 && d != 128) return fail(MC_E_INVALID, "attention: head_dim must be 64 or 128");
  if (fuse && (!attn_fuse_ok(R, nkv, w.nchunk, max_q, nq, d) || !fuse->qkv || !fuse->counters || !fuse->att))
    return fail(MC_E_INVALID, "attention: the fused path takes at most 64 queries per (row, kv head)");
  const float scale = 1.0f / sqrtf((float)d);
  const int S = attn_split(R, nkv, w.nchunk, fuse != nullptr);
  const dim3 grid(R * nkv, (w.nchunk + S - 1) / S);
  const AttnFuse nf{};
  const AttnFuse& f = fuse ? *fuse : nf;
  const int TP = attn_tiles(max_q * (nq / nkv));
  if (d == 128) {
    if (fuse) launch_flash<128, true>(TP, grid, st, q, kv, sv, nq, nkv, scale, S, w, f);
    else launch_flash<128, false>(TP, grid, st, q, kv, sv, nq, nkv, scale, S, w, f);
  } else {
    if (fuse) launch_flash<64, true>(TP, grid, st, q, kv, sv, nq, nkv, scale, S, w, f);
    else launch_flash<64, false>(TP, grid, st, q, kv, sv, nq, nkv, scale, S, w, f);
  }
  MC_HIP(hipGetLastError());
  if (fuse) return MC_OK;
  hipLaunchKernelGGL(attn_merge_kernel, dim3((M * nq + 3) / 4), dim3(256), 0, st, sv, M, nq, d, S, w, att);
  MC_HIP(hipGetLastError());
  return MC_OK;
}

// ---------------------------------------------------------------------------
// the reference's scheduler test doubles (SchedulerSpeculativeDecodingTests.swift:225-261)
// ---------------------------------------------------------------------------
__global__ void fake_logits_kernel(int arch, const int32_t* slot_tok, int M, int V, uint16_t* logits) {
  const int m = blockIdx.x;
  const int tok = slot_tok[m];
  int nx = tok == 1 ? 2 : tok == 2 ? 3 : 1;
  if (arch == MC_ARCH_FAKE_MISMATCHING && tok == 3) nx = 4;
  for (int v = threadIdx.x; v < V; v += blockDim.x)
    logits[(size_t)m * V + v] = f32_to_bf16(v == nx ? 20.0f : -20.0f);
}

int launch_fake_logits(int arch, const int32_t* slot_tok, int M, int V, uint16_t* logits, hipStream_t st) {
  hipLaunchKernelGGL(fake_logits_kernel, dim3(M), dim3(256), 0, st, arch, slot_tok, M, V, logits);
  MC_HIP(hipGetLastError());
  return MC_OK;
}

// ---------------------------------------------------------------------------
// synthetic K/V (same hash as the oracle's or_kv_fill_synthetic)
// ---------------------------------------------------------------------------
__global__ void kv_synth_kernel(KVLayer kv, int layer, int row, int nkv, int d, int n, uint64_t seed) {
  const size_t total = (size_t)2 * nkv * n * d;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (size_t)gridDim.x * blockDim.x) {
    const int e = (int)(i % d);
    const size_t rest = i / d;
    const int p = (int)(rest % n);
    const size_t rest2 = rest / n;
    const int h = (int)(rest2 % nkv);
    const int wv = (int)(rest2 / nkv);
    const uint64_t a = ((((uint64_t)layer * 2 + wv) << 40) ^ ((uint64_t)row << 32) ^ ((uint64_t)h << 24) ^
                        ((uint64_t)p << 8));
    const uint64_t hh = mix64(seed ^ mix64(a) ^ (uint64_t)e);
    const uint32_t sign = (uint32_t)(hh & 1u), ex = 126u - (uint32_t)((hh >> 1) & 3u), mant = (uint32_t)((hh >> 3) & 0x7Fu);
    const uint16_t val = (uint16_t)((sign << 15) | (ex << 7) | mant);
    if (wv) kv.v[(((size_t)row * nkv + h) * d + e) * kv.cap + p] = val;
    else kv.k[(((size_t)row * nkv + h) * kv.cap + p) * d + e] = val;
  }
}

// One 64 x 64 tile (64 positions x 64 channels) of one head's V between the cache's layout,
// [d][cap] with the block at columns t0 .. t0 + n - 1, and a prefix block's [n][d]
// (to_block: cache -> block).  Reads and writes are both along the fastest axis of their
// array; the tile turns in LDS (row pitch 66 halves = 33 banks, so a column read is
// conflict-free).
__global__ void __launch_bounds__(256) kv_block_v_kernel(uint16_t* v, int cap, uint16_t* blk, int n, int d, int t0,
                                                         int to_block) {
  __shared__ uint16_t tile[64][66];
  const int h = blockIdx.z, p0 = blockIdx.x * 64, e0 = blockIdx.y * 64;
  uint16_t* vh = v + (size_t)h * d * cap + t0;
  uint16_t* bh = blk + (size_t)h * n * d;
  const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
  if (to_block) {
    for (int i = ty; i < 64; i += 4)  // tile[e - e0][p - p0]
      if (e0 + i < d && p0 + tx < n) tile[i][tx] = vh[(size_t)(e0 + i) * cap + p0 + tx];
    __syncthreads();
    for (int i = ty; i < 64; i += 4)
      if (p0 + i < n && e0 + tx < d) bh[(size_t)(p0 + i) * d + e0 + tx] = tile[tx][i];
  } else {
    for (int i = ty; i < 64; i += 4)  // tile[p - p0][e - e0]
      if (p0 + i < n && e0 + tx < d) tile[i][tx] = bh[(size_t)(p0 + i) * d + e0 + tx];
    __syncthreads();
    for (int i = ty; i < 64; i += 4)
      if (e0 + i < d && p0 + tx < n) vh[(size_t)(e0 + i) * cap + p0 + tx] = tile[tx][i];
  }
}

int launch_kv_block_v(uint16_t* v_row, int cap, uint16_t* blk, int nkv, int n, int d, int t0, bool to_block,
                      hipStream_t st) {
  if (n <= 0) return MC_OK;
  hipLaunchKernelGGL(kv_block_v_kernel, dim3((unsigned)((n + 63) / 64), (unsigned)((d + 63) / 64), (unsigned)nkv),
                     dim3(256), 0, st, v_row, cap, blk, n, d, t0, to_block ? 1 : 0);
  MC_HIP(hipGetLastError());
  return MC_OK;
}

int launch_kv_synth(KVLayer kv, int layer, int row, int nkv, int d, int n, uint64_t seed, hipStream_t st) {
  size_t total = (size_t)2 * nkv * n * d;
  size_t blocks = (total + 255) / 256;
  if (blocks > 16384) blocks = 16384;
  if (blocks < 1) blocks = 1;
  hipLaunchKernelGGL(kv_synth_kernel, dim3((unsigned)blocks), dim3(256), 0, st, kv, layer, row, nkv, d, n, seed);
  MC_HIP(hipGetLastError());
  return MC_OK;
}

}  // namespace mc
