// mc_step.hip -- the speculative step's control kernels for gfx950.
//
//   propose:  the n-gram proposer of ContinuousBatchGenerator.proposeSuffixTokens
//             (Sources/MLXCat/TrackB/BatchGenerator.swift:982-1010) for every row at
//             once, plus the step gate (canSpeculate :957-975, proposal limit :876-884)
//             and the verify-token layout (:897-898).  The sequential search "longest
//             suffix first, then the latest earlier non-overlapping occurrence" is the
//             lexicographic maximum of (min(l(e), n - e), e) over candidate ends e, where
//             l(e) is the backward match length at e; one block computes every l(e) in
//             parallel and max-reduces the packed key.
//   scan:     per (row, verify position): the values the position samples from (the
//             logits, or with logit bias / min_tokens / penalties the processed fp32
//             values of Sampling.swift:592-652), then greedy argmax (lowest index on
//             ties), or the integer-mass target distribution of a sampled row (top-p as
//             Sampling.swift:847-858 on T=1 masses, min-p, top-k, then temperature), the
//             accept test of the draft token (u < p(x), one-hot n-gram draft) and the
//             residual / bonus sample.
//   commit:   per row: the acceptance rule (the reference's all-or-nothing loop
//             :906-947, or longest-prefix / speculative sampling), KV rollback by length,
//             history append (:1012-1014), stats (:894-895,938,952) and finish reasons
//             (Scheduler.swift:372-401).
#include "mc_step.hpp"

namespace mc {

__device__ inline uint64_t umax64(uint64_t a, uint64_t b) { return a > b ? a : b; }

// ---------------------------------------------------------------------------
// n-gram search over one history (block of 256 threads); returns e* or -1
// ---------------------------------------------------------------------------
__device__ int ngram_best_end(const int32_t* ctx, int n, int max_suffix, int min_ctx, uint64_t* red) {
  const int tid = threadIdx.x;
  if (n < min_ctx) return -1;
  const int maxlen = min(max_suffix, n - 1);
  if (maxlen <= 0) return -1;
  uint64_t best = 0;
  for (int e = 1 + tid; e <= n - 1; e += blockDim.x) {
    const int lim = min(maxlen, min(e, n - e));
    int l = 0;
    while (l < lim && ctx[e - 1 - l] == ctx[n - 1 - l]) ++l;
    if (l > 0) best = umax64(best, ((uint64_t)l << 32) | (uint64_t)e);
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) best = umax64(best, (uint64_t)__shfl_xor((unsigned long long)best, o));
  if ((tid & 63) == 0) red[tid >> 6] = best;
  __syncthreads();
  uint64_t b = 0;
  for (int w = 0; w < (int)(blockDim.x >> 6); ++w) b = umax64(b, red[w]);
  __syncthreads();
  return b ? (int)(b & 0xFFFFFFFFu) : -1;
}

__global__ void __launch_bounds__(256) propose_kernel(StepState s) {
  __shared__ uint64_t red[8];
  __shared__ int s_nactive;
  const int r = blockIdx.x, tid = threadIdx.x;
  if (tid == 0) {
    int na = 0;
    for (int i = 0; i < s.R; ++i) na += s.active[i] != 0;
    s_nactive = na;
  }
  __syncthreads();
  int P = 0;
  const bool act = s.active[r] != 0;
  const int32_t* ctx = s.hist + (size_t)r * s.hcap;
  if (act && s.enabled && s.K > 0 && (!s.single_row_only || s_nactive == 1) && s.hist_len[r] >= s.min_ctx &&
      (!s.greedy_only || (s.temp[r] == 0.0f && !s.has_seed[r]))) {
    const int remaining = max(0, s.max_gen[r] - s.gen[r]);
    if (remaining > 1) {
      const int limit = min(s.K, remaining - 1);
      const int n = s.hist_len[r];
      if (limit > 0) {
        const int e = ngram_best_end(ctx, n, s.max_suffix, s.min_ctx, red);
        if (e > 0) P = min(limit, n - e);
        if (P > 0 && tid < P) s.drafts[r * s.K1 + tid] = ctx[e + tid];
        // the continuation token after the drafts (the forced schedule's correction)
        if (P > 0 && tid == 0 && s.dext) {
          const bool ext = e + P < n;
          s.dext[r] = ext ? 1 : 0;
          if (ext) s.drafts[r * s.K1 + P] = ctx[e + P];
        }
      }
    }
  }
  if (tid == 0) {
    if (P == 0 && s.dext) s.dext[r] = 0;
    s.nprop[r] = act ? P : 0;
    s.n_valid[r] = act ? P + 1 : 0;
    s.row_slot0[r] = r * s.K1;
    s.qbase[r] = s.kv_len[r];
  }
  __syncthreads();
  for (int j = tid; j < s.K1; j += blockDim.x) {
    const int slot = r * s.K1 + j;
    if (act && j <= P) {
      s.slot_tok[slot] = j == 0 ? s.cur[r] : s.drafts[r * s.K1 + j - 1];
      s.slot_row[slot] = r;
      s.slot_pos[slot] = s.kv_len[r] + j;
    } else {
      s.slot_tok[slot] = 0;
      s.slot_row[slot] = -1;
      s.slot_pos[slot] = 0;
    }
  }
}

int launch_propose(const StepState& s, hipStream_t st) {
  if (s.K1 > 256) return fail(MC_E_INVALID, "propose: K too large");
  hipLaunchKernelGGL(propose_kernel, dim3(s.R), dim3(256), 0, st, s);
  MC_HIP(hipGetLastError());
  return MC_OK;
}

__global__ void __launch_bounds__(256) ngram_standalone_kernel(const int32_t* hist, const int64_t* off, int max_suffix,
                                                               int min_ctx, const int32_t* limit, int out_stride,
                                                               int32_t* out, int32_t* out_len) {
  __shared__ uint64_t red[8];
  const int r = blockIdx.x;
  const int32_t* ctx = hist + off[r];
  const int n = (int)(off[r + 1] - off[r]);
  int P = 0;
  const int lim = limit[r];
  int e = -1;
  if (lim > 0) {
    e = ngram_best_end(ctx, n, max_suffix, min_ctx, red);
    if (e > 0) P = min(lim, n - e);
  }
  for (int j = threadIdx.x; j < P; j += blockDim.x) out[(size_t)r * out_stride + j] = ctx[e + j];
  if (threadIdx.x == 0) out_len[r] = P;
}

int launch_ngram_standalone(const int32_t* hist, const int64_t* off, int B, int max_suffix, int min_ctx,
                            const int32_t* limit, int out_stride, int32_t* out, int32_t* out_len, hipStream_t st) {
  hipLaunchKernelGGL(ngram_standalone_kernel, dim3(B), dim3(256), 0, st, hist, off, max_suffix, min_ctx, limit,
                     out_stride, out, out_len);
  MC_HIP(hipGetLastError());
  return MC_OK;
}

// ---------------------------------------------------------------------------
// acceptance scan
// ---------------------------------------------------------------------------
constexpr int SCAN_THREADS = 1024;

// order-preserving 32-bit key of an fp32 value (callers fold -0 into +0 first)
__device__ inline uint32_t key32(float v) {
  const uint32_t u = __float_as_uint(v);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
// floor(u * T / 2^32) for u < 2^32, T < 2^60
__device__ inline uint64_t mulhi32(uint32_t u, uint64_t T) {
  const uint64_t lo = (T & 0xFFFFFFFFull) * (uint64_t)u;
  const uint64_t hi = (T >> 32) * (uint64_t)u;
  return hi + (lo >> 32);
}

__device__ inline uint64_t block_sum_u64(uint64_t v, uint64_t* red) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += (uint64_t)__shfl_xor((unsigned long long)v, o);
  const int tid = threadIdx.x;
  __syncthreads();
  if ((tid & 63) == 0) red[tid >> 6] = v;
  __syncthreads();
  uint64_t t = 0;
  for (int w = 0; w < (int)(blockDim.x >> 6); ++w) t += red[w];
  __syncthreads();
  return t;
}

// exclusive prefix sum over the block's threads in thread order
__device__ inline uint64_t block_excl_scan_u64(uint64_t v, uint64_t* red) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  uint64_t x = v;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const uint64_t y = (uint64_t)__shfl_up((unsigned long long)x, o);
    if (lane >= o) x += y;
  }
  __syncthreads();
  if (lane == 63) red[w] = x;
  __syncthreads();
  uint64_t off = 0;
  for (int i = 0; i < w; ++i) off += red[i];
  __syncthreads();
  return off + x - v;
}

__device__ inline unsigned long long block_max_u64(unsigned long long v, uint64_t* red) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const unsigned long long w = (unsigned long long)__shfl_xor(v, o);
    v = w > v ? w : v;
  }
  const int tid = threadIdx.x;
  __syncthreads();
  if ((tid & 63) == 0) red[tid >> 6] = v;
  __syncthreads();
  unsigned long long t = 0ull;
  for (int w = 0; w < (int)(blockDim.x >> 6); ++w) t = red[w] > t ? red[w] : t;
  __syncthreads();
  return t;
}

__device__ inline float block_max_f(float v, float* red) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
  const int tid = threadIdx.x;
  __syncthreads();
  if ((tid & 63) == 0) red[tid >> 6] = v;
  __syncthreads();
  float t = -INFINITY;
  for (int w = 0; w < (int)(blockDim.x >> 6); ++w) t = fmaxf(t, red[w]);
  __syncthreads();
  return t;
}

// The values one (row, position) samples from: the bf16 logits in fp32, and for rows with
// logits processors or penalties (Sampling.swift:638-652, 592-636) the logit bias, the
// min_tokens EOS mask and the repetition / presence / frequency penalties over the
// generated tokens (the row's, then the drafts before this position).  -0 reads as +0.
struct PosVals {
  const uint16_t* lg = nullptr;
  int proc = 0;
  int nb = 0;                 // bias entries
  const int32_t* bt = nullptr;
  const float* bv = nullptr;
  int ne = 0;                 // EOS ids to mask (0 = no mask at this position)
  const int32_t* eos = nullptr;
  int pen = 0;
  float rp = 1.f, pp = 0.f, fp = 0.f;
  const int32_t* cnt = nullptr;  // [V] generated-token counts of the row (NULL: none generated)
  const int32_t* dr = nullptr;   // drafts before this position
  int nd = 0;
  __device__ float operator()(int i) const {
#pragma clang fp contract(off)
    float v = bf16_to_f32(lg[i]);
    if (proc) {
      for (int k = 0; k < nb; ++k)
        if (bt[k] == i) v = v + bv[k];
      for (int k = 0; k < ne; ++k)
        if (eos[k] == i) v = -INFINITY;
      if (pen) {
        int c = cnt ? cnt[i] : 0;
        for (int t = 0; t < nd; ++t) c += dr[t] == i;
        if (c > 0) {
          if (rp != 1.0f) v = v < 0.0f ? v * rp : v / rp;
          if (pp != 0.0f) v = v - pp;
          if (fp != 0.0f) v = v - (float)c * fp;
        }
      }
    }
    return v == 0.0f ? 0.0f : v;
  }
};

// argmax with the lowest index on ties
__device__ int block_argmax(const PosVals& pv, int V, float* redv, int* redi) {
  const int tid = threadIdx.x;
  float bv = -INFINITY;
  int bi = 0x7FFFFFFF;
  for (int i = tid; i < V; i += blockDim.x) {
    const float v = pv(i);
    if (v > bv || (v == bv && i < bi)) { bv = v; bi = i; }
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float ov = __shfl_xor(bv, o);
    const int oi = __shfl_xor(bi, o);
    if (ov > bv || (ov == bv && oi < bi)) { bv = ov; bi = oi; }
  }
  __syncthreads();
  if ((tid & 63) == 0) { redv[tid >> 6] = bv; redi[tid >> 6] = bi; }
  __syncthreads();
  float v = -INFINITY;
  int idx = 0x7FFFFFFF;
  for (int w = 0; w < (int)(blockDim.x >> 6); ++w)
    if (redv[w] > v || (redv[w] == v && redi[w] < idx)) { v = redv[w]; idx = redi[w]; }
  __syncthreads();
  return idx == 0x7FFFFFFF ? 0 : idx;
}

// Kept set and temperature mass total of one position (filters in the order of
// Sampling.swift:500-522): top-p keeps key32(v) >= kstar, min-p keeps v - m >= lmp, top-k
// keeps the top_k largest values, the lowest indices first among equal values.
struct DistDev {
  float m;          // max value
  uint32_t kstar;   // smallest kept key under top-p (0 = all kept)
  float lmp;        // log(min_p), -inf = off
  int has_k;
  int ksh;          // top-k compares key32 >> ksh
  uint32_t kk;      // ... against the k-th largest
  int kidx;         // largest kept index among keys equal to kk
  uint64_t total;   // kept temperature mass
};

__device__ inline bool dkept(const DistDev& d, float v, int i) {
#pragma clang fp contract(off)
  const uint32_t k = key32(v);
  if (k < d.kstar) return false;
  if (!(v - d.m >= d.lmp)) return false;
  if (d.has_k) {
    const uint32_t kt = k >> d.ksh;
    if (kt < d.kk || (kt == d.kk && i > d.kidx)) return false;
  }
  return true;
}

__device__ inline uint64_t tmass(const DistDev& d, float v, int i, float inv_t) {
#pragma clang fp contract(off)
  if (!dkept(d, v, i)) return 0;
  return mass_of(exp_neg_det((v - d.m) * inv_t));
}

// Radix selection over `nlev` 8-bit digits of the keys (2 for plain bf16 values, whose keys'
// low 16 bits carry nothing, 4 for processed fp32 values).
__device__ DistDev dist_build_dev(const PosVals& pv, int V, float inv_t, float top_p, int top_k, float lmp, int nlev,
                                  uint64_t* hist, uint64_t* red, float* redf, int* s_int, uint64_t* s_u64) {
#pragma clang fp contract(off)
  const int tid = threadIdx.x, nt = blockDim.x;
  DistDev d;
  float mx = -INFINITY;
  for (int i = tid; i < V; i += nt) mx = fmaxf(mx, pv(i));
  d.m = block_max_f(mx, redf);
  d.kstar = 0;
  d.lmp = lmp;
  if (top_p > 0.0f && top_p < 1.0f) {
    // Sampling.swift:847-858 on T=1 masses: the kept values are those >= the smallest value
    // whose strictly-larger values hold less than top_p of the mass
    uint32_t prefix = 0;
    uint64_t base = 0;
    double X = 0.0;
    bool ok = true;
    for (int lev = 0; lev < nlev; ++lev) {
      const int sh = 24 - 8 * lev;
      for (int b = tid; b < 256; b += nt) hist[b] = 0;
      __syncthreads();
      uint64_t t1 = 0;
      for (int i = tid; i < V; i += nt) {
        const float v = pv(i);
        const uint32_t k = key32(v);
        if (lev > 0 && (k >> (sh + 8)) != prefix) continue;
        const uint64_t w = mass_of(exp_neg_det(v - d.m));
        t1 += w;
        if (w) atomicAdd((unsigned long long*)&hist[(k >> sh) & 255u], (unsigned long long)w);
      }
      if (lev == 0)
        X = (double)top_p * (double)block_sum_u64(t1, red);
      else
        __syncthreads();
      if (tid == 0) {
        uint64_t cum = base, sb = base;
        int sel = -1;
        for (int b = 255; b >= 0; --b) {
          if (hist[b] == 0) continue;
          if (!((double)cum < X)) break;
          sel = b;
          sb = cum;
          cum += hist[b];
        }
        s_int[0] = sel;
        s_u64[0] = sb;
      }
      __syncthreads();
      const int sel = s_int[0];
      base = s_u64[0];
      __syncthreads();
      if (sel < 0) { ok = false; break; }  // block-uniform
      prefix = (prefix << 8) | (uint32_t)sel;
    }
    d.kstar = ok ? prefix << (32 - 8 * nlev) : 0u;
  }
  d.has_k = top_k > 0 && top_k < V;
  d.ksh = 32 - 8 * nlev;
  d.kk = 0;
  d.kidx = 0x7FFFFFFF;
  if (d.has_k) {
    // Sampling.swift:893-906: the top_k-th largest key, then the index cutoff among its ties
    unsigned* cnt = reinterpret_cast<unsigned*>(hist);
    uint32_t prefix = 0;
    int need = top_k;
    for (int lev = 0; lev < nlev; ++lev) {
      const int sh = 24 - 8 * lev;
      for (int b = tid; b < 256; b += nt) cnt[b] = 0u;
      __syncthreads();
      for (int i = tid; i < V; i += nt) {
        const uint32_t k = key32(pv(i));
        if (lev > 0 && (k >> (sh + 8)) != prefix) continue;
        atomicAdd(&cnt[(k >> sh) & 255u], 1u);
      }
      __syncthreads();
      if (tid == 0) {
        int cum = 0, sel = 0;
        for (int b = 255; b >= 0; --b) {
          if (cum + (int)cnt[b] >= need) { sel = b; break; }
          cum += (int)cnt[b];
        }
        s_int[1] = sel;
        s_int[2] = need - cum;
      }
      __syncthreads();
      prefix = (prefix << 8) | (uint32_t)s_int[1];
      need = s_int[2];
      __syncthreads();
    }
    d.kk = prefix;
    const int chunk = (V + nt - 1) / nt;
    const int b0 = min(V, tid * chunk), b1 = min(V, b0 + chunk);
    int c = 0;
    for (int i = b0; i < b1; ++i) c += (key32(pv(i)) >> d.ksh) == prefix;
    if (tid == 0) s_int[3] = 0x7FFFFFFF;
    const int start = (int)block_excl_scan_u64((uint64_t)c, red);
    if (start < need && need <= start + c) {
      int seen = start;
      for (int i = b0; i < b1; ++i)
        if ((key32(pv(i)) >> d.ksh) == prefix && ++seen == need) { s_int[3] = i; break; }
    }
    __syncthreads();
    d.kidx = s_int[3];
    __syncthreads();
  }
  uint64_t tt = 0;
  for (int i = tid; i < V; i += nt) tt += tmass(d, pv(i), i, inv_t);
  d.total = block_sum_u64(tt, red);
  return d;
}

// index-order inverse-CDF sample of floor(u * total' / 2^32), total' excluding `ex`
__device__ int dist_sample_dev(const DistDev& d, const PosVals& pv, int V, float inv_t, uint32_t u, int ex,
                               uint64_t wx, uint64_t* red, int* s_int) {
  const int tid = threadIdx.x, nt = blockDim.x;
  const uint64_t total = d.total - (ex >= 0 ? wx : 0);
  const uint64_t R = mulhi32(u, total);
  const int chunk = (V + nt - 1) / nt;
  const int b0 = min(V, tid * chunk), b1 = min(V, b0 + chunk);
  uint64_t cs = 0;
  for (int i = b0; i < b1; ++i)
    if (i != ex) cs += tmass(d, pv(i), i, inv_t);
  if (tid == 0) s_int[4] = -1;
  const uint64_t start = block_excl_scan_u64(cs, red);
  if (R >= start && R < start + cs) {
    uint64_t c = start;
    for (int i = b0; i < b1; ++i) {
      if (i == ex) continue;
      const uint64_t w = tmass(d, pv(i), i, inv_t);
      if (w == 0) continue;
      if (c + w > R) { s_int[4] = i; break; }
      c += w;
    }
  }
  __syncthreads();
  const int tok = s_int[4];
  __syncthreads();
  return tok < 0 ? 0 : tok;
}

__global__ void __launch_bounds__(SCAN_THREADS) accept_scan_kernel(StepState s, const uint16_t* logits, int row_filter) {
  __shared__ uint64_t hist[256];
  __shared__ uint64_t red[16];
  __shared__ float redf[16];
  __shared__ int redi[16];
  __shared__ int s_int[8];
  __shared__ uint64_t s_u64[2];
  __shared__ int32_t l_bt[16], l_eos[8], l_dr[256];
  __shared__ float l_bv[16];
  const int r = blockIdx.x, j = blockIdx.y;
  if (row_filter >= 0 && r != row_filter) return;
  if (!s.active[r] || j >= s.n_valid[r]) return;
  const int P = s.nprop[r];
  const int slot = s.row_slot0[r] + j;
  const int V = s.V;
  PosVals pv;
  pv.lg = logits + (size_t)slot * V;
  {
    const int flags = s.proc ? s.proc[r] : 0;
    pv.nb = (flags & 1) ? s.n_bias[r] : 0;
    pv.ne = ((flags & 2) && s.gen[r] + j < s.min_tokens[r]) ? s.n_eos[r] : 0;
    pv.pen = (flags & 4) ? 1 : 0;
    pv.proc = pv.nb > 0 || pv.ne > 0 || pv.pen;
  }
  if (pv.proc) {  // block-uniform
    const int tid = threadIdx.x;
    if (tid < pv.nb) {
      l_bt[tid] = s.bias_tok[r * 16 + tid];
      l_bv[tid] = s.bias_val[r * 16 + tid];
    }
    if (tid < pv.ne) l_eos[tid] = s.eos[r * 8 + tid];
    if (pv.pen && tid < j) l_dr[tid] = s.drafts[r * s.K1 + tid];
    __syncthreads();
    pv.bt = l_bt;
    pv.bv = l_bv;
    pv.eos = l_eos;
    pv.dr = l_dr;
    pv.nd = pv.pen ? j : 0;
    pv.rp = s.rep_pen[r];
    pv.pp = s.pres_pen[r];
    pv.fp = s.freq_pen[r];
    pv.cnt = s.gen_cnt ? s.gen_cnt + (size_t)r * V : nullptr;
  }
  if (s.temp[r] == 0.0f) {
    int t;
    if (s.amax && !pv.proc) {
      // max over the head's per-tile partials (value key << 32 | 0xFFFFFFFF - index)
      const unsigned long long* ap = s.amax + (size_t)slot * s.amax_nt;
      unsigned long long best = 0ull;
      for (int i = threadIdx.x; i < s.amax_nt; i += blockDim.x) best = ap[i] > best ? ap[i] : best;
      best = block_max_u64(best, red);
      t = (int)(0xFFFFFFFFull - (best & 0xFFFFFFFFull));
    } else {
      t = block_argmax(pv, V, redf, redi);
    }
    if (threadIdx.x == 0) s.scan_tok[r * s.K1 + j] = t;
    return;
  }
  const float inv_t = s.inv_temp[r];
  const DistDev d = dist_build_dev(pv, V, inv_t, s.top_p[r], s.top_k[r], s.min_p_log[r], pv.proc ? 4 : 2, hist, red,
                                   redf, s_int, s_u64);
  const uint64_t seed = s.seed[r], ctr = s.counter[r];
  const bool caller_u = s.use_uniforms && *s.use_uniforms;
  const uint32_t* uu = caller_u ? s.uniforms + ((size_t)r * s.K1 + j) * 2 : nullptr;
  const uint32_t u_acc = caller_u ? uu[0] : uniform_u32(seed, ctr, (uint32_t)j, 0u);
  const uint32_t u_smp = caller_u ? uu[1] : uniform_u32(seed, ctr, (uint32_t)j, 1u);
  const bool forced = s.forced && s.forced[r] >= 0;  // the draw after forced drafts excludes nothing
  if (j < P) {
    const int x = s.drafts[r * s.K1 + j];
    const uint64_t wx = tmass(d, pv(x), x, inv_t);
    const int acc = mulhi32(u_acc, d.total) < wx;
    const int res = forced ? dist_sample_dev(d, pv, V, inv_t, u_smp, -1, 0, red, s_int)
                           : dist_sample_dev(d, pv, V, inv_t, u_smp, x, wx, red, s_int);
    if (threadIdx.x == 0) {
      s.scan_acc[r * s.K1 + j] = acc;
      s.scan_res[r * s.K1 + j] = res;
    }
  } else {
    const int res = dist_sample_dev(d, pv, V, inv_t, u_smp, -1, 0, red, s_int);
    if (threadIdx.x == 0) s.scan_res[r * s.K1 + j] = res;
  }
}

int launch_accept_scan(const StepState& s, const uint16_t* logits, int row_filter, hipStream_t st) {
  if (s.K1 > 257) return fail(MC_E_INVALID, "accept scan: K too large");
  hipLaunchKernelGGL(accept_scan_kernel, dim3(s.R, s.K1), dim3(SCAN_THREADS), 0, st, s, logits, row_filter);
  MC_HIP(hipGetLastError());
  return MC_OK;
}

// ---------------------------------------------------------------------------
// commit: one thread per row
// ---------------------------------------------------------------------------
__device__ inline bool is_eos(const StepState& s, int r, int tok) {
  const int n = s.n_eos[r];
  for (int i = 0; i < n; ++i)
    if (s.eos[r * 8 + i] == tok) return true;
  return false;
}

// Acceptance decision of one row.  Writes the emitted tokens to `out`, returns their
// count; *keep = verified positions kept in the KV (current token + accepted drafts),
// *nacc = drafts accepted, *rejected = 1 when a proposal was (partly) rejected.
__device__ int decide_row(const StepState& s, int r, int32_t* out, int* keep, int* nacc, int* rejected) {
  const int P = s.nprop[r], K1 = s.K1;
  const int32_t* dr = s.drafts + r * K1;
  const int32_t* st = s.scan_tok + r * K1;
  const int32_t* sa = s.scan_acc + r * K1;
  const int32_t* sr = s.scan_res + r * K1;
  const bool greedy = s.temp[r] == 0.0f;
  const int rej = s.reject[r];
  int n = 0;
  *keep = 1;
  *nacc = 0;
  *rejected = 0;
  if (greedy && s.acceptance == MC_ACCEPT_ALL_OR_NOTHING) {
    if (P == 0) {
      out[n++] = st[0];
    } else {
      bool all = true;
      int na = 0;
      for (int pos = 0; pos <= P; ++pos) {
        const int t = st[pos];
        if (rej >= 0 && t == rej) { all = false; break; }        // :920-923
        if (pos < P && t != dr[pos]) { all = false; break; }    // :925-928
        out[na++] = t;
        if (is_eos(s, r, t)) break;                             // :932-934
      }
      if (!all) {
        *rejected = 1;                                          // :938
        out[0] = st[0];                                         // :939 the one-token decode: position 0
        // (bit-identical to a separate one-token forward within the M <= 16 class at the same
        // batch shape; across classes it agrees to rounding)
        n = 1;
      } else {
        n = na;
        *keep = P + 1;                                          // :942 adopt the verified positions
        *nacc = na > 1 ? na - 1 : 0;                            // :952
      }
    }
  } else if (s.forced && s.forced[r] >= 0) {
    // forced accept-length schedule (stress workloads): exactly min(f, P) drafts count as
    // accepted, up to an EOS or reject token among them, then the history's continuation
    // token after them (the next draft, or the one after the last draft), or the model's
    // token at that position when the history has none (sampled rows: drawn without
    // exclusion)
    int a = min(s.forced[r], P);
    bool stop = false;
    for (int pos = 0; pos < a; ++pos) {
      const int t = dr[pos];
      out[n++] = t;
      if (t == rej || is_eos(s, r, t)) { a = pos + 1; stop = true; break; }
    }
    if (!stop) out[n++] = (a < P || (P > 0 && s.dext[r])) ? dr[a] : (greedy ? st[a] : sr[a]);
    *keep = a + 1;
    *nacc = a;
    *rejected = (P > 0 && a < P) ? 1 : 0;
  } else {
    int a = 0;
    bool stop = false;
    for (int pos = 0; pos < P; ++pos) {
      int t;
      if (greedy) {
        t = st[pos];
        if (t != dr[pos] || t == rej) { out[n++] = t; stop = true; break; }
      } else {
        if (!sa[pos]) { out[n++] = sr[pos]; stop = true; break; }
        t = dr[pos];
      }
      out[n++] = t;
      ++a;
      if (t == rej || is_eos(s, r, t)) { stop = true; break; }
    }
    if (!stop) out[n++] = greedy ? st[P] : sr[P];
    *keep = a + 1;
    *nacc = a;
    *rejected = (P > 0 && a < P) ? 1 : 0;
  }
  return n;
}

__global__ void commit_kernel(StepState s, int row_filter) {
  const int r = blockIdx.x * blockDim.x + threadIdx.x;
  if (r >= s.R) return;
  if (row_filter >= 0 && r != row_filter) return;
  if (!s.active[r]) {
    s.out_cnt[r] = 0;
    s.out_fin[r] = 0;
    return;
  }
  const int P = s.nprop[r];
  int32_t* out = s.out_tok + r * s.K1;
  int keep, nacc, rejected;
  const int n = decide_row(s, r, out, &keep, &nacc, &rejected);
  if (P > 0) {
    atomicAdd(&s.stats[0], (unsigned long long)P);        // :895
    atomicAdd(&s.stats[1], (unsigned long long)nacc);     // :952
    atomicAdd(&s.stats[2], 1ull);                         // :894
    atomicAdd(&s.stats[3], (unsigned long long)rejected); // :938
  }
  s.counter[r] += 1;
  s.kv_len[r] = s.qbase[r] + keep;  // rollback: keep current token + accepted drafts
  int fin = 0, emitted = 0;
  int32_t* h = s.hist + (size_t)r * s.hcap;
  int32_t* cnt = (s.proc && (s.proc[r] & 4)) ? s.gen_cnt + (size_t)r * s.V : nullptr;
  for (int z = 0; z < n; ++z) {
    const int t = out[z];
    if (s.hist_len[r] < s.hcap) h[s.hist_len[r]++] = t;
    if (cnt) cnt[t] += 1;  // the penalties' token counts
    s.gen[r] += 1;
    ++emitted;
    fin = is_eos(s, r, t) ? 1 : (s.gen[r] >= s.max_gen[r] ? 2 : 0);
    if (fin) break;
  }
  s.cur[r] = out[n - 1];
  s.out_cnt[r] = emitted;
  s.out_fin[r] = fin;
  if (fin) s.active[r] = 0;
}

// decision only (mc_accept): no state update
__global__ void decide_kernel(StepState s, int32_t* n_emit, int32_t* keep_out, int32_t* nacc_out) {
  const int r = blockIdx.x * blockDim.x + threadIdx.x;
  if (r >= s.R) return;
  int keep, nacc, rejected;
  const int n = decide_row(s, r, s.out_tok + r * s.K1, &keep, &nacc, &rejected);
  n_emit[r] = n;
  keep_out[r] = keep;
  nacc_out[r] = nacc;
}

int launch_decide(const StepState& s, int32_t* n_emit, int32_t* keep_out, int32_t* nacc_out, hipStream_t st) {
  hipLaunchKernelGGL(decide_kernel, dim3((s.R + 63) / 64), dim3(64), 0, st, s, n_emit, keep_out, nacc_out);
  MC_HIP(hipGetLastError());
  return MC_OK;
}

// Rows of an acceptance over caller device buffers: drafts [B][K] -> the state's [B][K1]
// layout, proposal lengths, slot offsets.  A row whose n_draft or draft ids are out of range
// is run with no drafts and flagged in *err.
__global__ void accept_prep_kernel(StepState s, const int32_t* drafts, const int32_t* n_draft, int K, int32_t* err) {
  const int r = blockIdx.x * blockDim.x + threadIdx.x;
  if (r >= s.R) return;
  int P = n_draft[r];
  bool bad = P < 0 || P > K;
  if (!bad)
    for (int j = 0; j < P; ++j) {
      const int t = drafts[(size_t)r * K + j];
      bad = bad || t < 0 || t >= s.V;
    }
  if (bad) {
    P = 0;
    atomicAdd(err, 1);
  }
  for (int j = 0; j < s.K1; ++j) s.drafts[r * s.K1 + j] = j < P ? drafts[(size_t)r * K + j] : 0;
  s.nprop[r] = P;
  s.n_valid[r] = P + 1;
  s.row_slot0[r] = r * s.K1;
  s.active[r] = 1;
  s.forced[r] = -1;
  s.gen[r] = 0;
}

int launch_accept_prep(const StepState& s, const int32_t* drafts, const int32_t* n_draft, int K, int32_t* err,
                       hipStream_t st) {
  hipLaunchKernelGGL(accept_prep_kernel, dim3((s.R + 63) / 64), dim3(64), 0, st, s, drafts, n_draft, K, err);
  MC_HIP(hipGetLastError());
  return MC_OK;
}

int launch_commit(const StepState& s, int row_filter, hipStream_t st) {
  hipLaunchKernelGGL(commit_kernel, dim3((s.R + 63) / 64), dim3(64), 0, st, s, row_filter);
  MC_HIP(hipGetLastError());
  return MC_OK;
}

}  // namespace mc
