// mc_kernels.hip -- per-token kernels of the verify forward for gfx950:
// quantized-embedding gather, RMSNorm, fused q/k-norm + RoPE + KV append, and
// split-KV GQA attention over each row's contiguous K/V (one query block per
// (row, kv head): the (K+1) verify positions x the GQA group share every key load).
//
// Semantics follow the mlx-lm decoder the reference runs (external to its tree):
// RMSNorm y = (x * rsqrt(mean(x^2) + eps)) * w, rotate-half RoPE with a per-row
// position (the reference's per-row RoPE offsets, Sources/MLXCat/TrackB/BatchCache.swift:123-139),
// causal attention where the query at position p sees keys [0, p]
// (Sources/MLXCat/TrackB/CausalMask.swift:4-28).
#include "mc_kernels.hpp"

namespace mc {

typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

// ---------------------------------------------------------------------------
// embedding: dequantised row of the tile-layout [V, H] tensor, bf16(fma(s, q, b))
// ---------------------------------------------------------------------------
__global__ void embed_kernel(QLinear E, const int32_t* slot_tok, int M, int H, uint16_t* x) {
  const int per_row = H / 8;
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= M * per_row) return;
  const int m = i / per_row, kw = i - m * per_row;
  int tok = slot_tok[m];
  if (tok < 0 || tok >= E.N) tok = 0;
  const int t = tok >> 4, r = tok & 15;
  const int g = kw >> 3, w8 = kw & 7, am = w8 >> 2, c = w8 & 3;
  const int gp = g >> 1, gi = g & 1;
  const uint32_t word = E.qw[(((size_t)t * E.GP + gp) * 64 + c * 16 + r) * 4 + gi * 2 + am];
  const uint32_t sbw = E.sb[(((size_t)t * E.GP + gp) * 4 + (r >> 2)) * 8 + gi * 4 + (r & 3)];
  const float s = bf16_to_f32((uint16_t)(sbw & 0xFFFFu)), b = bf16_to_f32((uint16_t)(sbw >> 16));
  uint32_t out[4];
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    const float q0 = (float)((word >> (4 * p)) & 0xFu);          // element 2p
    const float q1 = (float)((word >> (16 + 4 * p)) & 0xFu);     // element 2p + 1
    out[p] = (uint32_t)f32_to_bf16(__builtin_fmaf(s, q0, b)) | ((uint32_t)f32_to_bf16(__builtin_fmaf(s, q1, b)) << 16);
  }
  u32x4 v = {out[0], out[1], out[2], out[3]};
  *reinterpret_cast<u32x4*>(x + (size_t)m * H + kw * 8) = v;
}

int launch_embed(const QLinear& E, const int32_t* slot_tok, int M, int H, uint16_t* x, hipStream_t st) {
  const int total = M * (H / 8);
  hipLaunchKernelGGL(embed_kernel, dim3((total + 255) / 256), dim3(256), 0, st, E, slot_tok, M, H, x);
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
// RMSNorm: one 256-thread block per token
// ---------------------------------------------------------------------------
__global__ void __launch_bounds__(256) rmsnorm_kernel(const uint16_t* x, const uint16_t* w, int H, float eps,
                                                      uint16_t* y) {
  __shared__ float red[4];
  const int m = blockIdx.x, tid = threadIdx.x;
  const uint16_t* xr = x + (size_t)m * H;
  float ss = 0.f;
  for (int i = tid; i < H; i += 256) {
    const float v = bf16_to_f32(xr[i]);
    ss += v * v;
  }
  ss = wave_sum(ss);
  if ((tid & 63) == 0) red[tid >> 6] = ss;
  __syncthreads();
  const float tot = (red[0] + red[1]) + (red[2] + red[3]);
  const float r = 1.0f / sqrtf(tot / (float)H + eps);
  for (int i = tid; i < H; i += 256)
    y[(size_t)m * H + i] = f32_to_bf16((bf16_to_f32(xr[i]) * r) * bf16_to_f32(w[i]));
}

int launch_rmsnorm(const uint16_t* x, const uint16_t* w, int M, int H, float eps, uint16_t* y, hipStream_t st) {
  hipLaunchKernelGGL(rmsnorm_kernel, dim3(M), dim3(256), 0, st, x, w, H, eps, y);
  MC_HIP(hipGetLastError());
  return MC_OK;
}

// ---------------------------------------------------------------------------
// q/k RMSNorm (Qwen3) + rotate-half RoPE + KV append.  One block per slot, one
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
  for (int hh = wave; hh < ntot; hh += 4) {
    const uint16_t* hp = src + (size_t)hh * d;
    if (hh >= nq + nkv) {  // V head: copy into the cache
      const int h = hh - nq - nkv;
      uint16_t* dst = kv.v + (((size_t)row * nkv + h) * kv.cap + pos) * d;
      for (int i = lane; i < d; i += 64) dst[i] = hp[i];
      continue;
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
  hipLaunchKernelGGL(qk_rope_append_kernel, dim3(M), dim3(256), 0, st, qkv, q_norm, k_norm, rope_cos, rope_sin, nq,
                     nkv, d, eps, slot_row, slot_pos, kv, q_out);
  MC_HIP(hipGetLastError());
  return MC_OK;
}

// ---------------------------------------------------------------------------
// split-KV attention.  Grid (R * nkv, nchunk, qtiles); block 256.  A block loads a
// 64-key chunk of one (row, kv head) once and scores it against up to 16 queries
// (verify positions x GQA group), producing per-query partial (max, sum, o[d]).
// The combine pass merges chunks 0..nc-1 in order, so a query's result depends
// only on its own position and keys.
// ---------------------------------------------------------------------------
constexpr int KROW = 128 + 2;  // LDS row stride (bf16) for K / V chunks

__global__ void __launch_bounds__(256) attn_partial_kernel(const uint16_t* q, KVLayer kv, SlotView sv, int nq,
                                                           int nkv, int d, float scale, AttnWork w) {
  __shared__ uint16_t ks[ATTN_CHUNK * KROW];
  __shared__ uint16_t vs[ATTN_CHUNK * KROW];
  __shared__ float qs[ATTN_QTILE * 128];
  __shared__ float ps[ATTN_QTILE * ATTN_CHUNK];
  __shared__ float pm[ATTN_QTILE], pl[ATTN_QTILE];

  const int G = nq / nkv;
  const int r = blockIdx.x / nkv, kh = blockIdx.x % nkv;
  const int chunk = blockIdx.y, qt = blockIdx.z;
  const int nv = sv.n_valid[r];
  const int nqry = nv * G;
  if (qt * ATTN_QTILE >= nqry) return;
  const int base = sv.qbase[r];
  const int kend = base + nv;  // keys visible to the last query
  const int k0 = chunk * ATTN_CHUNK;
  if (k0 >= kend) return;
  const int nk = min(ATTN_CHUNK, kend - k0);
  const int tid = threadIdx.x;
  const int slot0 = sv.row_slot0[r];

  // stage K, V chunk
  const uint16_t* kbase = kv.k + (((size_t)r * nkv + kh) * kv.cap + k0) * d;
  const uint16_t* vbase = kv.v + (((size_t)r * nkv + kh) * kv.cap + k0) * d;
  for (int i = tid; i < nk * (d / 2); i += 256) {
    const int key = i / (d / 2), e = (i - key * (d / 2)) * 2;
    const uint32_t kk = *reinterpret_cast<const uint32_t*>(kbase + (size_t)key * d + e);
    const uint32_t vv = *reinterpret_cast<const uint32_t*>(vbase + (size_t)key * d + e);
    *reinterpret_cast<uint32_t*>(ks + key * KROW + e) = kk;
    *reinterpret_cast<uint32_t*>(vs + key * KROW + e) = vv;
  }
  // stage queries of this tile
  for (int i = tid; i < ATTN_QTILE * d; i += 256) {
    const int qi = i / d, e = i - qi * d;
    const int gq = qt * ATTN_QTILE + qi;
    float v = 0.f;
    if (gq < nqry) {
      const int j = gq / G, gh = gq - j * G;
      v = bf16_to_f32(q[(size_t)(slot0 + j) * nq * d + (size_t)(kh * G + gh) * d + e]);
    }
    qs[qi * 128 + e] = v;
  }
  __syncthreads();

  // scores: thread -> query qi = tid / 16, keys (tid % 16) + 16 i
  {
    const int qi = tid >> 4, kl = tid & 15;
    const int gq = qt * ATTN_QTILE + qi;
    const int qpos = (gq < nqry) ? base + gq / G : -1;
    float sc[ATTN_CHUNK / 16];
    float mx = -INFINITY;
#pragma unroll
    for (int i = 0; i < ATTN_CHUNK / 16; ++i) {
      const int key = kl + 16 * i;
      float s = -INFINITY;
      if (key < nk && k0 + key <= qpos) {
        float a0 = 0.f, a1 = 0.f;
        for (int e = 0; e < d; e += 2) {
          a0 += qs[qi * 128 + e] * bf16_to_f32(ks[key * KROW + e]);
          a1 += qs[qi * 128 + e + 1] * bf16_to_f32(ks[key * KROW + e + 1]);
        }
        s = (a0 + a1) * scale;
      }
      sc[i] = s;
      mx = fmaxf(mx, s);
    }
    // max / sum over the 16 lanes that share this query (lanes qi*16 .. qi*16+15)
#pragma unroll
    for (int o = 8; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 16));
    float l = 0.f;
#pragma unroll
    for (int i = 0; i < ATTN_CHUNK / 16; ++i) {
      const float p = (sc[i] == -INFINITY) ? 0.f : __expf(sc[i] - mx);
      ps[qi * ATTN_CHUNK + kl + 16 * i] = p;
      l += p;
    }
#pragma unroll
    for (int o = 8; o > 0; o >>= 1) l += __shfl_xor(l, o, 16);
    if (kl == 0) {
      pm[qi] = mx;
      pl[qi] = l;
    }
  }
  __syncthreads();

  // o[qi][e] = sum_key p[qi][key] v[key][e]; thread -> qi = tid / 16, e = (tid % 16) + 16 i
  {
    const int qi = tid >> 4, el = tid & 15;
    const int gq = qt * ATTN_QTILE + qi;
    if (gq < nqry) {
      const int j = gq / G, gh = gq - j * G;
      const int slot = slot0 + j;
      const int h = kh * G + gh;
      float* po = w.part_o + (((size_t)slot * nq + h) * w.nchunk + chunk) * d;
      for (int e = el; e < d; e += 16) {
        float a = 0.f;
        for (int key = 0; key < nk; ++key) a += ps[qi * ATTN_CHUNK + key] * bf16_to_f32(vs[key * KROW + e]);
        po[e] = a;
      }
      if (el == 0) {
        float* pml = w.part_ml + (((size_t)slot * nq + h) * w.nchunk + chunk) * 2;
        pml[0] = pm[qi];
        pml[1] = pl[qi];
      }
    }
  }
}

// one block (d threads) per (slot, head): merge chunks 0..nc-1 in order
__global__ void attn_combine_kernel(SlotView sv, int nq, int d, AttnWork w, uint16_t* att) {
  const int m = blockIdx.x, h = blockIdx.y, e = threadIdx.x;
  const int row = sv.slot_row[m];
  uint16_t* out = att + ((size_t)m * nq + h) * d;
  if (row < 0) {
    if (e < d) out[e] = 0;
    return;
  }
  const int pos = sv.slot_pos[m];
  const int nc = pos / ATTN_CHUNK + 1;
  const float* pml = w.part_ml + ((size_t)m * nq + h) * w.nchunk * 2;
  float mx = -INFINITY;
  for (int c = 0; c < nc; ++c) mx = fmaxf(mx, pml[c * 2]);
  float l = 0.f, acc = 0.f;
  const float* po = w.part_o + ((size_t)m * nq + h) * w.nchunk * d;
  for (int c = 0; c < nc; ++c) {
    const float cm = pml[c * 2];
    const float f = (cm == -INFINITY) ? 0.f : __expf(cm - mx);
    l += pml[c * 2 + 1] * f;
    if (e < d) acc += po[(size_t)c * d + e] * f;
  }
  if (e < d) out[e] = f32_to_bf16(acc / l);
}

int launch_attention(const uint16_t* q, KVLayer kv, const SlotView& sv, int R, int max_q, int nq, int nkv, int d,
                     int M, const AttnWork& w, uint16_t* att, hipStream_t st) {
  if (d > 128) return fail(MC_E_INVALID, "attention: head_dim > 128");
  const int G = nq / nkv;
  const int qtiles = (max_q * G + ATTN_QTILE - 1) / ATTN_QTILE;
  const float scale = 1.0f / sqrtf((float)d);
  hipLaunchKernelGGL(attn_partial_kernel, dim3(R * nkv, w.nchunk, qtiles), dim3(256), 0, st, q, kv, sv, nq, nkv, d,
                     scale, w);
  MC_HIP(hipGetLastError());
  hipLaunchKernelGGL(attn_combine_kernel, dim3(M, nq), dim3(128), 0, st, sv, nq, d, w, att);
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
    uint16_t* c = wv ? kv.v : kv.k;
    c[(((size_t)row * nkv + h) * kv.cap + p) * d + e] = (uint16_t)((sign << 15) | (ex << 7) | mant);
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
