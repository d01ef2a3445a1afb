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
// q/k RMSNorm (Qwen3) + rotate-half RoPE + KV append.  Grid (slot, head / 4), one
// wave per head; lane i handles the rotation pair (i, i + d/2) for d = 128.
// ---------------------------------------------------------------------------
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
  const int Nqkv = ntot * d;
  const uint16_t* src = qkv + (size_t)m * Nqkv;
  {
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
    const uint16_t* nw = is_q ? q_norm : k_norm;
    // d <= 128: lane < hd handles (lane, lane + hd)
    float x1 = 0.f, x2 = 0.f;
    if (lane < hd) {
      x1 = bf16_to_f32(hp[lane]);
      x2 = bf16_to_f32(hp[lane + hd]);
    }
    if (nw) {
      const float ss = wave_sum(x1 * x1 + x2 * x2);
      const float r = 1.0f / sqrtf(ss / (float)d + eps);
      if (lane < hd) {
        x1 = bf16_to_f32(f32_to_bf16((x1 * r) * bf16_to_f32(nw[lane])));
        x2 = bf16_to_f32(f32_to_bf16((x2 * r) * bf16_to_f32(nw[lane + hd])));
      }
    }
    if (lane < hd) {
      const float cs = rope_cos[(size_t)pos * hd + lane], sn = rope_sin[(size_t)pos * hd + lane];
      const uint16_t o1 = f32_to_bf16(x1 * cs - x2 * sn);
      const uint16_t o2 = f32_to_bf16(x1 * sn + x2 * cs);
      if (is_q) {
        uint16_t* dst = q_out + (size_t)m * nq * d + (size_t)hh * d;
        dst[lane] = o1;
        dst[lane + hd] = o2;
      } else {
        const int h = hh - nq;
        uint16_t* dst = kv.k + (((size_t)row * nkv + h) * kv.cap + pos) * d;
        dst[lane] = o1;
        dst[lane + hd] = o2;
      }
    }
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
constexpr int FA_TP = 2;  // query tiles of 16 per pass

template <int D>
__global__ void __launch_bounds__(256) attn_flash_kernel(const uint16_t* q, KVLayer kv, SlotView sv, int nq, int nkv,
                                                         float scale, int S, AttnWork w) {
  __shared__ float mrg[4][FA_TP][16][D + 2];  // per wave: o[d], max, sum of each query of the pass
  const int G = nq / nkv;
  const int r = blockIdx.x / nkv, kh = blockIdx.x % nkv;
  const int split = blockIdx.y;
  const int nv = sv.n_valid[r];
  const int nqry = nv * G;
  if (nqry == 0) return;
  const int base = sv.qbase[r];
  const int kend = base + nv;
  const int s0 = split * S * ATTN_CHUNK;
  if (s0 >= kend) return;
  const int s1 = min(kend, s0 + S * ATTN_CHUNK);
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, c = lane >> 4, r16 = lane & 15;
  const int slot0 = sv.row_slot0[r];
  const size_t head = (size_t)r * nkv + kh;
  const uint16_t* kbase = kv.k + head * kv.cap * D;   // [pos][d]
  const uint16_t* vbase = kv.v + head * D * kv.cap;   // [d][pos]
  constexpr int NS = D / 32, NDB = D / 16;
  typedef unsigned u4 __attribute__((ext_vector_type(4)));
  const int nqt = (nqry + 15) / 16;
  for (int t0 = 0; t0 < nqt; t0 += FA_TP) {
    // B operands: q rows of queries (t0 + tt) 16 + r16, d = 32 s + 8 c .. + 7
    bf16x8_t qb[FA_TP][4];
    int qpos[FA_TP];
#pragma unroll
    for (int tt = 0; tt < FA_TP; ++tt) {
      const int qi = min((t0 + tt) * 16 + r16, nqry - 1);
      const int j = qi / G, gh = qi - j * G;
      qpos[tt] = (t0 + tt) * 16 + r16 < nqry ? base + j : -1;
      const uint16_t* qp = q + ((size_t)(slot0 + j) * nq + kh * G + gh) * D;
#pragma unroll
      for (int s4 = 0; s4 < 4; ++s4)
        qb[tt][s4] = s4 < NS ? *reinterpret_cast<const bf16x8_t*>(qp + 32 * s4 + 8 * c)
                             : __builtin_bit_cast(bf16x8_t, (u4){0u, 0u, 0u, 0u});
    }
    float mrun[FA_TP], lrun[FA_TP];
    f32x4_t o[FA_TP][NDB];
#pragma unroll
    for (int tt = 0; tt < FA_TP; ++tt) {
      mrun[tt] = -INFINITY;
      lrun[tt] = 0.f;
#pragma unroll
      for (int db = 0; db < NDB; ++db) o[tt][db] = (f32x4_t){0.f, 0.f, 0.f, 0.f};
    }
    for (int sc = s0 + ATTN_CHUNK * wave; sc < s1; sc += 4 * ATTN_CHUNK) {
      // keys sc .. sc + 63 (inside the row's cap; keys >= kend are finite and masked)
      bf16x8_t ka[4][4];
#pragma unroll
      for (int kb = 0; kb < 4; ++kb)
#pragma unroll
        for (int s4 = 0; s4 < 4; ++s4)
          ka[kb][s4] = s4 < NS ? *reinterpret_cast<const bf16x8_t*>(kbase + (size_t)(sc + 16 * kb + r16) * D + 32 * s4 + 8 * c)
                               : __builtin_bit_cast(bf16x8_t, (u4){0u, 0u, 0u, 0u});
      s16x4_t va[NDB][4];
#pragma unroll
      for (int db = 0; db < NDB; ++db)
#pragma unroll
        for (int kb = 0; kb < 4; ++kb)
          va[db][kb] = *reinterpret_cast<const s16x4_t*>(vbase + (size_t)(16 * db + r16) * kv.cap + sc + 16 * kb + 4 * c);
#pragma unroll
      for (int tt = 0; tt < FA_TP; ++tt) {
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
            const int key = sc + 16 * kb + 4 * c + v;
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
    for (int tt = 0; tt < FA_TP; ++tt) {
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
    // thread: query (tt, qq) = tid / 8 (FA_TP x 16 = 32 queries), d slice 16 (tid % 8)
    {
      const int qsel = threadIdx.x >> 3, part = threadIdx.x & 7;
      const int tt = qsel >> 4, qq = qsel & 15;
      const int qi = (t0 + tt) * 16 + qq;
      if (t0 + tt < nqt && qi < nqry) {
        float mx = -INFINITY;
#pragma unroll
        for (int w2 = 0; w2 < 4; ++w2) mx = fmaxf(mx, mrg[w2][tt][qq][D]);
        float f[4], l = 0.f;
#pragma unroll
        for (int w2 = 0; w2 < 4; ++w2) {
          const float m2 = mrg[w2][tt][qq][D];
          f[w2] = m2 == -INFINITY ? 0.f : __expf(m2 - mx);
          l += mrg[w2][tt][qq][D + 1] * f[w2];
        }
        const int jj = qi / G, gg = qi - jj * G;
        const size_t pidx = ((size_t)(slot0 + jj) * nq + kh * G + gg) * w.nchunk + split;
        for (int e = part * (D / 8); e < (part + 1) * (D / 8); ++e) {
          float a = 0.f;
#pragma unroll
          for (int w2 = 0; w2 < 4; ++w2) a += mrg[w2][tt][qq][e] * f[w2];
          w.part_o[pidx * D + e] = a;
        }
        if (part == 0) {
          w.part_ml[pidx * 2] = mx;
          w.part_ml[pidx * 2 + 1] = l;
        }
      }
    }
    __syncthreads();
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
  const float* pml = w.part_ml + ((size_t)m * nq + h) * w.nchunk * 2;
  const float* po = w.part_o + ((size_t)m * nq + h) * w.nchunk * d;
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
        ml[u] = *reinterpret_cast<const float2*>(pml + (size_t)cc * 2);
        if (e0 < d) ov[u] = *reinterpret_cast<const float2*>(po + (size_t)cc * d + e0);
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
  if (e0 < d) {
    const float inv = 1.0f / l;
    *reinterpret_cast<uint32_t*>(out + e0) = (uint32_t)f32_to_bf16(a0 * inv) | ((uint32_t)f32_to_bf16(a1 * inv) << 16);
  }
}

int launch_attention(const uint16_t* q, KVLayer kv, const SlotView& sv, int R, int max_q, int nq, int nkv, int d,
                     int M, const AttnWork& w, uint16_t* att, hipStream_t st) {
  if (d != 64 && d != 128) return fail(MC_E_INVALID, "attention: head_dim must be 64 or 128");
  (void)max_q;
  const float scale = 1.0f / sqrtf((float)d);
  // 64-key sub-chunks per block: more when the grid would exceed about 1024 blocks (fewer
  // partials to merge), and at least 2 (a few (row, kv head) pairs: one decode row spreads
  // its 8 heads over more CUs, 10.0 -> 8.0 us per layer at 2K keys against 4) or 8 (64 or
  // more pairs: two sub-chunks per wave, 4x fewer partials; batch 8 at 2K keys
  // 5.08 -> 4.89 ms per step, 8 rows at 512-4096 keys 6.71 -> 6.28 ms).
  const int smin = R * nkv >= 64 ? 8 : 2;
  const int S = std::max(smin, (R * nkv * w.nchunk + 1023) / 1024);
  const dim3 grid(R * nkv, (w.nchunk + S - 1) / S);
  if (d == 128) hipLaunchKernelGGL(attn_flash_kernel<128>, grid, dim3(256), 0, st, q, kv, sv, nq, nkv, scale, S, w);
  else hipLaunchKernelGGL(attn_flash_kernel<64>, grid, dim3(256), 0, st, q, kv, sv, nq, nkv, scale, S, w);
  MC_HIP(hipGetLastError());
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
