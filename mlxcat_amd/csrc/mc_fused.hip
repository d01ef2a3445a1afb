// mc_fused.hip -- the verify forward of M <= 8 tokens as one persistent kernel.
//
// Why: at bs=1 the forward is ~250 dependent phases of a few MB each.  As separate
// kernels every phase pays launch ramp, first-load latency and tail, and the HBM idles
// between them.  Here every phase is a set of work units that a fixed block / wave owns,
// and a unit's weights (or cached K/V) are loaded into registers as soon as the wave has
// finished its previous unit -- long before the unit's inputs exist.  Phases exchange
// activations through LL words (payload | tag << 32, 8-byte device-coherent stores); a
// consumer polls exactly the words it needs until all tags equal the tag of the producing
// phase of this call.  Each LL buffer is rewritten only by a phase that depends (through
// the data) on every reader of its previous contents, so no reader can see a newer value
// than the one it waits for.
//
// Block = 4 waves (one per SIMD, so a wave may hold 256 VGPRs + 256 AGPRs), one block
// per CU, grid = #CUs (all resident: the LDS footprint allows one block per CU).
//   waves 0..2  work units: a 16-row tile x K-range of a 4-bit linear (MFMA, the same
//               dequant arithmetic as mc_gemv), or 64 cached keys of one (row, kv head)
//               for attention (MFMA S^T = K Q^T and O^T = V^T P^T);
//   wave 3      split-K reductions (+ residual add + RMSNorm partials), attention
//               combine, embedding.
//   all waves   stage a phase's input in LDS: poll the LL words, then normalise / rotate
//               and form the per-group sums the dequant fold needs.
// Every wait is bounded: after FW_TIMEOUT the wave sets *err and leaves, and the others
// see *err (or time out themselves), so the kernel always ends.
#include "mc_fused.hpp"

#include <algorithm>
#include <vector>

namespace mc {

typedef unsigned long long u64;
typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4;
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x2 __attribute__((ext_vector_type(2)));
typedef __amdgpu_buffer_rsrc_t rsrc_t;

namespace {

constexpr int CP_NT = 2;    // cache policy: streamed once
constexpr int CP_SC1 = 16;  // cache policy: device-coherent (LL words)
constexpr int NWAVE = FW_THREADS / 64;
constexpr u64 FW_TIMEOUT = 20000000ull;  // 200 ms of the 100 MHz real-time counter

enum { OP_QKV = 0, OP_ATT = 1, OP_O = 2, OP_GU = 3, OP_DN = 4, OP_HEAD = 5 };
enum { TG_X = 0, TG_QKV = 1, TG_ATTP = 2, TG_ATT = 3, TG_OP = 4, TG_XO = 5, TG_ACT = 6, TG_DP = 7, TG_XD = 8 };

// tag of phase k of layer l in call ep (layer -1: the embedding); 62 layers at most
__device__ inline unsigned tagof(unsigned ep, int l, int k) { return ep * 1024u + (unsigned)((l + 1) * 16 + k); }

// ---- LDS layout (bytes); the GEMV staging and the attention staging alias ----
constexpr int XST = FW_UGP * 128 + 8;  // X row stride (bf16): 16 B pad against bank conflicts
constexpr int L_X = 0;                                        // [FW_MMAX][XST] bf16
constexpr int L_XSUM = L_X + FW_MMAX * XST * 2;               // [2 FW_UGP groups][16 tokens] f32
constexpr int L_RS = L_XSUM + 2 * FW_UGP * 16 * 4;            // [FW_MMAX] f32 RMSNorm scales
constexpr int L_NW = L_RS + FW_MMAX * 4;                      // [FW_UGP * 128] bf16 norm weights
constexpr int L_GEMV_END = L_NW + FW_UGP * 128 * 2;
constexpr int QS = 128 + 8;                                   // q / new-k row stride (bf16)
constexpr int VS = 32 + 8;                                    // new-V^T row stride (bf16)
constexpr int L_Q = 0;                                        // [FW_QROWS][QS] bf16 normed + rotated q
constexpr int L_KN = L_Q + FW_QROWS * QS * 2;                 // [32 keys][QS] bf16 new k (normed + rotated)
constexpr int L_VN = L_KN + 32 * QS * 2;                      // [128][VS] bf16 new v, transposed
constexpr int RAW_ROWS = 6 * FW_MMAX;                         // (GQA group + k + v) x tokens
constexpr int L_RAW = L_VN + 128 * VS * 2;                    // [RAW_ROWS][128] bf16 raw q / k / v
constexpr int L_RCS = L_RAW + RAW_ROWS * 128 * 2;             // [FW_MMAX][64] f32 rope cos
constexpr int L_RSN = L_RCS + FW_MMAX * 64 * 4;               // [FW_MMAX][64] f32 rope sin
constexpr int L_QKW = L_RSN + FW_MMAX * 64 * 4;               // [2][128] bf16 q_norm, k_norm
constexpr int L_MG = L_RAW;                                   // [FW_CW][FW_QROWS][128] f32 unit outputs
constexpr int L_ML = L_MG + FW_CW * FW_QROWS * 128 * 4;       // [FW_CW][FW_QROWS][2] f32 (max, sum)
constexpr int L_ATT_END = L_ML + FW_CW * FW_QROWS * 2 * 4;
constexpr int L_ROW = L_GEMV_END > L_ATT_END ? L_GEMV_END : L_ATT_END;  // [FW_MMAX][8] int row info
constexpr int L_FLAG = L_ROW + FW_MMAX * 8 * 4;                          // [8] int counters
constexpr int L_TOTAL = L_FLAG + 8 * 4;
static_assert(L_QKW + 512 <= L_ML, "attention staging overlaps the unit outputs");
static_assert(L_TOTAL <= 160 * 1024, "LDS budget");
// row info fields
enum { RI_T = 0, RI_NV = 1, RI_S0 = 2, RI_NPB = 3, RI_BASE = 4 };
// counters: every use of the staging area increments each by one per wave
enum { F_RAW = 0, F_PREP = 1, F_RES = 2, F_DONE = 3, F_NA = 4 };

// ---------------------------------------------------------------------------------------
// memory access: buffer descriptors (out-of-range loads read 0, stores are dropped)
// ---------------------------------------------------------------------------------------
__device__ inline rsrc_t mk(const void* p, size_t bytes) {
  const int n = bytes > 0x7FFFFFF0ull ? 0x7FFFFFF0 : (int)bytes;
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, n, 0x00020000);
}
__device__ inline u32x4 ld16_nt(rsrc_t r, unsigned off) { return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, CP_NT); }
__device__ inline u32x4 ld16(rsrc_t r, unsigned off) { return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0); }
__device__ inline u32x4 ld16_sc(rsrc_t r, unsigned off) { return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, CP_SC1); }
__device__ inline u32x2 ld8_sc(rsrc_t r, unsigned off) { return __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, CP_SC1); }
__device__ inline void st8_sc(rsrc_t r, unsigned off, unsigned data, unsigned tag) {
  __builtin_amdgcn_raw_buffer_store_b64((u32x2){data, tag}, r, off, 0, CP_SC1);
}
__device__ inline void st16_sc(rsrc_t r, unsigned off, u32x4 v) { __builtin_amdgcn_raw_buffer_store_b128(v, r, off, 0, CP_SC1); }

__device__ inline float lo_f(uint32_t w) { return __uint_as_float(w << 16); }
__device__ inline float hi_f(uint32_t w) { return __uint_as_float(w & 0xFFFF0000u); }
__device__ inline uint32_t pack2(float a, float b) { return (uint32_t)f32_to_bf16(a) | ((uint32_t)f32_to_bf16(b) << 16); }

__device__ inline bf16x8 dequant_word(uint32_t w, uint32_t mask, uint32_t magic) {
  u32x4 p;
  p.x = ((w << 3) & mask) | magic;
  p.y = ((w >> 1) & mask) | magic;
  p.z = ((w >> 5) & mask) | magic;
  p.w = ((w >> 9) & mask) | magic;
  return __builtin_bit_cast(bf16x8, p);
}
__device__ inline float silu_f(float z) { return z / (1.0f + __expf(-z)); }

// ---------------------------------------------------------------------------------------
// bounded waiting
// ---------------------------------------------------------------------------------------
struct Ctl {
  u64 t0;
  unsigned* err;
  int ab;  // wave-uniform: this wave has given up
};

// One wait iteration: sleep; every 32nd call look at *err and at the clock.  Returns true
// when the wave must give up.
__device__ inline bool spin(Ctl& c, int& it, int site) {
  (void)site;
  __builtin_amdgcn_s_sleep(2);
  if ((++it & 31) != 0) return false;
  bool bad = __hip_atomic_load(c.err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0u;
  if (!bad && wall_clock64() - c.t0 > FW_TIMEOUT) {
    if ((threadIdx.x & 63) == 0) __hip_atomic_fetch_or(c.err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    MC_TRACE_TIMEOUT(site);
    bad = true;
  }
  if (bad) c.ab = 1;
  return bad;
}

// LDS counters between the waves of a block (LDS operations only: no global fence)
__device__ inline void lds_signal(int* f) {
  MC_FENCE();
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): this wave's LDS writes are done
  if ((threadIdx.x & 63) == 0) __hip_atomic_fetch_add(f, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
  MC_FENCE();
}
__device__ inline bool lds_wait(int* f, int target, Ctl& c, int site) {
  int it = 0;
  while (__hip_atomic_load(f, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) < target)
    if (spin(c, it, site)) return false;
  MC_FENCE();
  return true;
}

// The thread index, re-materialised: address arithmetic derived from it cannot be hoisted
// out of the phase loop (the kernel would otherwise keep hundreds of lane constants live
// for the whole forward).
__device__ inline int fresh_tid() {
  int t = threadIdx.x;
  MC_OPAQUE(t);
  return t;
}

__device__ inline float wave_sum64(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  return v;
}

// ---------------------------------------------------------------------------------------
// work-unit assignment (identical in every wave; no communication)
// ---------------------------------------------------------------------------------------
// GEMV phase: K-range kr = b % ks, tiles t = bg + GB (w + FW_CW i) with bg = b / ks.
__device__ inline int gemv_tile(const FwLin& L, int G, int b, int w, int i) {
  const int GB = G / L.ks;
  if (b >= GB * L.ks) return -1;
  const int t = b / L.ks + GB * (w + FW_CW * i);
  return t < L.NT ? t : -1;
}
__device__ inline bool gemv_block_has(const FwLin& L, int G, int b) { return gemv_tile(L, G, b, 0, 0) >= 0; }

// attention: tasks (row, kv head, block part pb) in row-major order; task f is block
// f % G's round f / G; wave w of the round takes 64-key chunk pb * FW_CW + w of the row
// (chunks < nh: cached keys; chunk nh: the new keys; beyond: nothing).
struct AttTask {
  int r, h, pb, T, NV, S0, npb, nh;
};
__device__ inline bool att_task(const int* ri, int R, int nkv, int f, AttTask& t) {
  for (int r = 0; r < R; ++r) {
    const int npb = ri[r * 8 + RI_NPB], base = ri[r * 8 + RI_BASE];
    if (f >= base && f < base + nkv * npb) {
      const int rem = f - base;
      t.r = r;
      t.h = rem / npb;
      t.pb = rem - t.h * npb;
      t.T = ri[r * 8 + RI_T];
      t.NV = ri[r * 8 + RI_NV];
      t.S0 = ri[r * 8 + RI_S0];
      t.npb = npb;
      t.nh = (t.T + FW_AKEYS - 1) / FW_AKEYS;
      return true;
    }
  }
  return false;
}

// key index of A-operand row i of key block kb: the two key blocks of a 32-key slice
// interleave in fours so that the S^T rows a lane ends with are 8 consecutive keys --
// exactly the k-slots of its P^T operand and of its 16-byte V^T load.
__device__ inline int sigma(int kb, int i) { return 32 * (kb >> 1) + 8 * (i >> 2) + 4 * (kb & 1) + (i & 3); }

__device__ inline FwLin lin_of(const FwArgs& a, int op, int l) {
  if (op == OP_HEAD) return a.head;
  const FwLayer& Ly = a.layers[l];
  return op == OP_QKV ? Ly.qkv : op == OP_O ? Ly.o : op == OP_GU ? Ly.gu : Ly.dn;
}

// A compute wave's next unit that needs loads: (layer, op, round).
struct Unit {
  int l, op, i;
};

// Advance u to the first loading unit of wave w strictly after u (u.op = -1: from the start).
// Returns false when there is none.
__device__ __forceinline__ bool next_unit(const FwArgs& a, const int* ri, int na, int G, int b, int w, Unit& u) {
  int l, op, i;
  if (u.op < 0) {
    l = 0; op = OP_QKV; i = 0;
  } else {
    l = u.l; op = u.op; i = u.i + 1;
  }
  if (op != OP_HEAD && l >= a.L) { l = a.L; op = OP_HEAD; i = 0; }
  // at most 5 L + 1 phase steps
  while (true) {
    if (op == OP_HEAD) {
      if (a.with_head && gemv_tile(a.head, G, b, w, i) >= 0) { u = Unit{a.L, OP_HEAD, i}; return true; }
      return false;
    }
    if (op == OP_ATT) {
      for (;; ++i) {
        const int f = b + G * i;
        if (f >= na) break;
        AttTask t;
        if (!att_task(ri, a.R, a.nkv, f, t)) break;
        if (t.pb * FW_CW + w < t.nh) { u = Unit{l, op, i}; return true; }
      }
    } else {
      // rounds of one GEMV phase are consecutive: if round i is empty, so are the later ones
      if (gemv_tile(lin_of(a, op, l), G, b, w, i) >= 0) { u = Unit{l, op, i}; return true; }
    }
    ++op;
    i = 0;
    if (op > OP_DN) {
      ++l;
      op = l >= a.L ? OP_HEAD : OP_QKV;
      if (op == OP_HEAD) l = a.L;
    }
  }
}

// ---------------------------------------------------------------------------------------
// unit loads (registers ub[32] = 512 B per lane)
// ---------------------------------------------------------------------------------------
__device__ inline void issue_gemv(u32x4 (&ub)[32], const FwLin& L, int t, int kr, int lane) {
  const int gp0 = kr * L.ugp, ngp = min(L.ugp, L.GP - gp0);
  const rsrc_t rq = mk(L.qw, (size_t)L.NT * L.GP * 1024);
  const rsrc_t rs = mk(L.sb, (size_t)L.NT * 16 * L.GP * 8);
  // every slot is loaded unconditionally (a short K-range re-reads its last group pair):
  // conditional register writes would keep the previous unit's values alive as well
  const unsigned qoff = ((unsigned)(t * L.GP + gp0) * 64u + (unsigned)lane) * 16u;
#pragma unroll
  for (int j = 0; j < FW_UGP; ++j) ub[j] = ld16_nt(rq, qoff + (unsigned)min(j, ngp - 1) * 1024u);
  const unsigned soff = (unsigned)tile_sb_word(t, lane & 15, gp0, 0, L.GP) * 4u;
#pragma unroll
  for (int j = 0; j < FW_UGP / 2; ++j) ub[FW_UGP + j] = ld16(rs, soff + (unsigned)min(j, (ngp - 1) / 2) * 16u);
  ub[30] = ub[29];
  ub[31] = ub[29];
}

// 64 cached keys of (row r, kv head h) from key kbase: K rows in the sigma order (A operand
// of S^T = K Q^T), V^T rows (A operand of O^T = V^T P^T).
__device__ inline void issue_att(u32x4 (&ub)[32], const FwLayer& Ly, const FwArgs& a, int r, int h, int kbase,
                                 int lane) {
  const int c4 = lane >> 4, n = lane & 15;
  const size_t head = (size_t)r * a.nkv + h;
  const size_t bytes = (size_t)a.R * a.nkv * a.cap * a.d * 2;
  const rsrc_t rk = mk(Ly.k, bytes), rv = mk(Ly.v, bytes);
#pragma unroll
  for (int kb = 0; kb < 4; ++kb)
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const int key = kbase + sigma(kb, n);
      ub[kb * 4 + s] = ld16(rk, (unsigned)(((head * a.cap + key) * a.d + 32 * s + 8 * c4) * 2));
    }
#pragma unroll
  for (int db = 0; db < 8; ++db)
#pragma unroll
    for (int k2 = 0; k2 < 2; ++k2)
      ub[16 + db * 2 + k2] =
          ld16(rv, (unsigned)((((head * a.d + 16 * db + n) * a.cap) + kbase + 32 * k2 + 8 * c4) * 2));
}

__device__ __forceinline__ void issue_unit(u32x4 (&ub)[32], const FwArgs& a, const int* ri, int G, int b, int w, int lane, const Unit& u) {
  if (u.op == OP_ATT) {
    AttTask t;
    att_task(ri, a.R, a.nkv, b + G * u.i, t);
    issue_att(ub, a.layers[u.l], a, t.r, t.h, (t.pb * FW_CW + w) * FW_AKEYS, lane);
  } else {
    const FwLin L = lin_of(a, u.op, u.op == OP_HEAD ? 0 : u.l);
    issue_gemv(ub, L, gemv_tile(L, G, b, w, u.i), b % L.ks, lane);
  }
}

// ---------------------------------------------------------------------------------------
// GEMV unit: acc[v] = sum_k x[token 4c + v][k] W[16t + r16][k] over the K-range
// ---------------------------------------------------------------------------------------
__device__ inline f32x4 gemv_compute(const u32x4 (&ub)[32], int ngp, const unsigned char* lds, int M, int lane,
                                     uint32_t mask, uint32_t magic) {
  const int c = lane >> 4, r16 = lane & 15;
  const uint16_t* xrow = reinterpret_cast<const uint16_t*>(lds + L_X) + min(r16, M - 1) * XST + 8 * c;
  const float* xsum = reinterpret_cast<const float*>(lds + L_XSUM);
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int j = 0; j < FW_UGP; ++j) {
    if (j < ngp) {
      // the words pass through an empty asm here, so their dequantisation (4x the
      // registers) cannot be hoisted ahead of this group pair
      u32x4 wq = ub[j];
      u32x4 sbp = ub[FW_UGP + j / 2];
      MC_OPAQUE2(wq, sbp);
#pragma unroll
      for (int gi = 0; gi < 2; ++gi) {
        const bf16x8 wv0 = dequant_word(gi ? wq.z : wq.x, mask, magic);
        const bf16x8 wv1 = dequant_word(gi ? wq.w : wq.y, mask, magic);
        const uint32_t sbv = (j & 1) ? (gi ? sbp.w : sbp.z) : (gi ? sbp.y : sbp.x);
        const float sv = DQ_STEP * __uint_as_float(sbv << 16);
        const float bv = __uint_as_float(sbv & 0xFFFF0000u) - sv;
        const int kl = j * 128 + gi * 64;
        const bf16x8 xv0 = *reinterpret_cast<const bf16x8*>(xrow + kl);
        const bf16x8 xv1 = *reinterpret_cast<const bf16x8*>(xrow + kl + 32);
        f32x4 g = {0.f, 0.f, 0.f, 0.f};
        g = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xv0, wv0, g, 0, 0, 0);
        g = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xv1, wv1, g, 0, 0, 0);
        const f32x4 xs = *reinterpret_cast<const f32x4*>(xsum + (j * 2 + gi) * 16 + 4 * c);
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          acc[v] = __builtin_fmaf(sv, g[v], acc[v]);
          acc[v] = __builtin_fmaf(bv, xs[v], acc[v]);
        }
      }
      // keep the LDS reads of one group pair together (bounded register use)
      MC_FENCE();
    }
  }
  return acc;
}

// ---------------------------------------------------------------------------------------
// staging of a GEMV phase's input: LL rows [token][ldw words], words k0/2 .. (k0 + kl)/2
// ---------------------------------------------------------------------------------------
struct XIn {
  const u64* src;
  int ldw;             // words per token row of src
  unsigned tag;
  const uint16_t* nw;  // RMSNorm weights [K] (NULL: no norm)
  const u64* ss;       // [FW_MMAX][ssn] sums of squares per 16 columns (norm only)
  int ssn;
  int K;               // full input width (the norm's mean)
  float eps;
};

constexpr int XPP = (FW_MMAX * FW_UGP * 128 / 4 + FW_THREADS - 1) / FW_THREADS;  // 16-byte pairs per thread

template <bool CTL>
__device__ __forceinline__ bool stage_x(const XIn& in, int k0, int kl, int M, unsigned char* lds, int nst, Ctl& cx) {
  const int tid = fresh_tid(), lane = tid & 63, w = tid >> 6;
  int* fl = reinterpret_cast<int*>(lds + L_FLAG);
  const int ppr = kl / 4;  // pairs per token row
  const int np = M * ppr;
  const rsrc_t rx = mk(in.src, (size_t)FW_MMAX * in.ldw * 8);
  u32x4 v[XPP];
  unsigned pend = 0;
#pragma unroll
  for (int q = 0; q < XPP; ++q)
    if (tid + FW_THREADS * q < np) pend |= 1u << q;
  // control wave: the norm's sums of squares (2 pairs per lane per token) and weights
  const bool ctl = CTL && in.nw != nullptr;
  const rsrc_t rss = mk(in.ss, (size_t)FW_MMAX * in.ssn * 8);
  u32x4 sv[CTL ? 2 * FW_MMAX : 1];
  unsigned spend = 0;
  if (ctl) {
#pragma unroll
    for (int m = 0; m < FW_MMAX; ++m)
#pragma unroll
      for (int i = 0; i < 2; ++i)
        if (m < M && lane + 64 * i < in.ssn / 2) spend |= 1u << (m * 2 + i);
  }
  unsigned xoff[XPP];
#pragma unroll
  for (int q = 0; q < XPP; ++q) {
    const int p = min(tid + FW_THREADS * q, np - 1), m = p / ppr, pw = p - m * ppr;
    xoff[q] = ((unsigned)(m * in.ldw + k0 / 2) + 2u * (unsigned)pw) * 8u;
  }
  int it = 0;
  while (true) {
    // every round reloads all slots (unconditional register writes)
#pragma unroll
    for (int q = 0; q < XPP; ++q) v[q] = ld16_sc(rx, xoff[q]);
    if constexpr (CTL) {
      if (ctl) {
#pragma unroll
        for (int m = 0; m < FW_MMAX; ++m)
#pragma unroll
          for (int i = 0; i < 2; ++i)
            sv[m * 2 + i] = ld16_sc(rss, ((unsigned)(min(m, M - 1) * in.ssn) + 2u * (unsigned)min(lane + 64 * i, in.ssn / 2 - 1)) * 8u);
      }
    }
    pend = 0;
#pragma unroll
    for (int q = 0; q < XPP; ++q)
      if (tid + FW_THREADS * q < np && !(v[q].y == in.tag && v[q].w == in.tag)) pend |= 1u << q;
    if constexpr (CTL) {
      if (ctl) {
        const unsigned want = spend;
        spend = 0;
#pragma unroll
        for (int k = 0; k < 2 * FW_MMAX; ++k)
          if ((want >> k & 1u) && !(sv[k].y == in.tag && sv[k].w == in.tag)) spend |= 1u << k;
      }
    }
    if (!__any((pend | spend) != 0u)) break;
    if (spin(cx, it, 101)) return false;
  }
  // the previous use of the staging area is over
  if (!lds_wait(fl + F_DONE, NWAVE * (nst - 1), cx, 201)) return false;
  uint16_t* xl = reinterpret_cast<uint16_t*>(lds + L_X);
#pragma unroll
  for (int q = 0; q < XPP; ++q) {
    const int p = tid + FW_THREADS * q;
    if (p < np) {
      const int m = p / ppr, pw = p - m * ppr;
      *reinterpret_cast<u32x2*>(xl + m * XST + 4 * pw) = (u32x2){v[q].x, v[q].z};
    }
  }
  if constexpr (CTL) {
   if (ctl) {
    float* rs = reinterpret_cast<float*>(lds + L_RS);
#pragma unroll
    for (int m = 0; m < FW_MMAX; ++m) {
      if (m >= M) break;
      float s = 0.f;
#pragma unroll
      for (int i = 0; i < 2; ++i)
        if (lane + 64 * i < in.ssn / 2) s += __uint_as_float(sv[m * 2 + i].x) + __uint_as_float(sv[m * 2 + i].z);
      s = wave_sum64(s);
      if (lane == 0) rs[m] = 1.0f / sqrtf(s / (float)in.K + in.eps);
    }
    const rsrc_t rw = mk(in.nw, (size_t)in.K * 2);
    uint16_t* nwl = reinterpret_cast<uint16_t*>(lds + L_NW);
    for (int i = lane; i < kl / 8; i += 64)
      *reinterpret_cast<u32x4*>(nwl + 8 * i) = ld16(rw, (unsigned)(k0 + 8 * i) * 2u);
   }
  }
  lds_signal(fl + F_RAW);
  if (!lds_wait(fl + F_RAW, NWAVE * nst, cx, 202)) return false;
  // normalise (bf16((x r) w): a standalone RMSNorm's rounding) and the per-group sums
  const float* rs = reinterpret_cast<const float*>(lds + L_RS);
  const uint16_t* nwl = reinterpret_cast<const uint16_t*>(lds + L_NW);
  float* xsum = reinterpret_cast<float*>(lds + L_XSUM);
  const int cpr = kl / 8;  // 16-byte chunks per row
  const int nch = M * cpr;
  for (int base = 0; base < FW_MMAX * FW_UGP * 16; base += FW_THREADS) {
    if (base >= nch) break;
    const int i = base + tid;
    float gs = 0.f;
    if (i < nch) {
      const int m = i / cpr, ch = i - m * cpr;
      u32x4 x = *reinterpret_cast<const u32x4*>(xl + m * XST + 8 * ch);
      if (in.nw) {
        const float r = rs[m];
        const u32x4 wv = *reinterpret_cast<const u32x4*>(nwl + 8 * ch);
#pragma unroll
        for (int h = 0; h < 4; ++h) x[h] = pack2((lo_f(x[h]) * r) * lo_f(wv[h]), (hi_f(x[h]) * r) * hi_f(wv[h]));
        *reinterpret_cast<u32x4*>(xl + m * XST + 8 * ch) = x;
      }
      float q0 = 0.f, q1 = 0.f;
#pragma unroll
      for (int h = 0; h < 4; ++h) {
        q0 += lo_f(x[h]);
        q1 += hi_f(x[h]);
      }
      gs = q0 + q1;
    }
    // the 8 chunks of a 64-wide group are 8 consecutive lanes (cpr is a multiple of 8)
    gs += __shfl_xor(gs, 1);
    gs += __shfl_xor(gs, 2);
    gs += __shfl_xor(gs, 4);
    if (i < nch && (i & 7) == 0) {
      const int m = i / cpr, gl = (i - m * cpr) >> 3;
      xsum[gl * 16 + m] = gs;
    }
  }
  // token rows >= M of the group sums: zero
  for (int i = tid; i < (16 - M) * (kl / 64); i += FW_THREADS) xsum[(i / (16 - M)) * 16 + M + i % (16 - M)] = 0.f;
  lds_signal(fl + F_PREP);
  return true;
}

// ---------------------------------------------------------------------------------------
// GEMV phase
// ---------------------------------------------------------------------------------------
struct Epi {
  int kind;  // 0: bf16 pairs LL, 1: SwiGLU pairs LL, 2: f32 partial LL, 3: logits + argmax
  u64* out;
  int ldo;   // words per token row (kind 0/1), columns N (kind 2)
  unsigned tag;
};

__device__ inline void gemv_epilogue(const Epi& e, const FwArgs& a, const FwLin& L, f32x4 acc, int t, int kr, int lane) {
  const int c = lane >> 4, r16 = lane & 15;
  const int n = t * 16 + r16;
  const int M = a.M;
  if (e.kind == 0) {
    const rsrc_t ro = mk(e.out, (size_t)FW_MMAX * e.ldo * 8);
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const float other = __shfl_xor(acc[v], 1);
      const int m = 4 * c + v;
      if (!(r16 & 1) && m < M && n < L.N) st8_sc(ro, (unsigned)(m * e.ldo + n / 2) * 8u, pack2(acc[v], other), e.tag);
    }
  } else if (e.kind == 1) {
    // rows interleave (gate_i, up_i): even lanes form act_i, lanes 4p pair act_(2p), act_(2p+1)
    const rsrc_t ro = mk(e.out, (size_t)FW_MMAX * e.ldo * 8);
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const float up = __shfl_xor(acc[v], 1);
      const float av = bf16_to_f32(f32_to_bf16(silu_f(acc[v]) * up));
      const float av2 = __shfl_xor(av, 2);
      const int m = 4 * c + v;
      if ((r16 & 3) == 0 && m < M && n + 3 < L.N) st8_sc(ro, (unsigned)(m * e.ldo + n / 4) * 8u, pack2(av, av2), e.tag);
    }
  } else if (e.kind == 2) {
    const rsrc_t ro = mk(e.out, (size_t)L.ks * FW_MMAX * e.ldo * 8);
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int m = 4 * c + v;
      if (m < M && n < L.N) st8_sc(ro, (unsigned)((kr * FW_MMAX + m) * e.ldo + n) * 8u, __float_as_uint(acc[v]), e.tag);
    }
  } else {
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int m = 4 * c + v;
      const bool live = m < M && n < L.N;
      const uint16_t hv = f32_to_bf16(acc[v]);
      if (live) a.logits[(size_t)m * a.V + n] = hv;
      // tile argmax over 16 rows: key (value key << 16 | 15 - row), lowest row on ties
      unsigned key = live ? (bf16_order_key(hv) << 16) | (unsigned)(15 - r16) : 0u;
#pragma unroll
      for (int o = 1; o < 16; o <<= 1) key = max(key, (unsigned)__shfl_xor((int)key, o));
      if (m < M && r16 == 0 && key)
        a.amax[(size_t)m * L.NT + t] =
            ((u64)(key >> 16) << 32) | (0xFFFFFFFFull - (unsigned)(t * 16 + 15 - (int)(key & 15u)));
    }
  }
}

struct WaveState {
  u32x4 ub[32];
  Unit cur;
  bool has;  // cur is a loading unit whose loads are issued
};

// Load the registers of the wave's next unit; with none left, a fresh zero definition, so
// the previous unit's registers are dead on every path (no copies, no spills).
__device__ __forceinline__ void refill(WaveState& ws, const FwArgs& a, const int* ri, int G, int b, int w, int lane) {
  if (ws.has) {
    issue_unit(ws.ub, a, ri, G, b, w, lane, ws.cur);
  } else {
#pragma unroll
    for (int j = 0; j < 32; ++j) ws.ub[j] = (u32x4){0u, 0u, 0u, 0u};
  }
}

template <bool CTL>
__device__ __forceinline__ bool gemv_phase(const FwArgs& a, unsigned char* lds, Ctl& cx, int& nst, WaveState& ws, const int* ri, int na,
                           int op, int l, const XIn& in, const Epi& e, uint32_t mask, uint32_t magic) {
  const int tid = fresh_tid(), w = tid >> 6, lane = tid & 63;
  const int b = blockIdx.x, G = gridDim.x;
  const FwLin L = lin_of(a, op, op == OP_HEAD ? 0 : l);
  if (!gemv_block_has(L, G, b)) return true;
  ++nst;
  int* fl = reinterpret_cast<int*>(lds + L_FLAG);
  const int kr = b % L.ks;
  const int gp0 = kr * L.ugp, ngp = min(L.ugp, L.GP - gp0);
  if (!stage_x<CTL>(in, gp0 * 128, ngp * 128, a.M, lds, nst, cx)) return false;
  if constexpr (!CTL) {
    for (int i = 0;; ++i) {
      const int t = gemv_tile(L, G, b, w, i);
      if (t < 0) break;
      if (!ws.has || ws.cur.op != op || ws.cur.l != l || ws.cur.i != i) {
        // the unit schedule and the phase order disagree: a bug, never a wait
        if (lane == 0) __hip_atomic_fetch_or(a.err, 2u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        cx.ab = 1;
        return false;
      }
      if (i == 0 && !lds_wait(fl + F_PREP, NWAVE * nst, cx, 203)) return false;
      const f32x4 acc = gemv_compute(ws.ub, ngp, lds, a.M, lane, mask, magic);
      gemv_epilogue(e, a, L, acc, t, kr, lane);
      ws.has = next_unit(a, ri, na, G, b, w, ws.cur);
      refill(ws, a, ri, G, b, w, lane);
    }
  }
  lds_signal(fl + F_DONE);
  return true;
}

// ---------------------------------------------------------------------------------------
// attention phase
// ---------------------------------------------------------------------------------------
// One unit: the 32 query rows (GQA head gh x token j, row 8 gh + j) of the staged (row, kv
// head) against 64 cached keys from kbase (NEW = false, K / V^T in ub) or against the new
// keys (NEW = true, K / V^T in LDS).  Writes O^T (unnormalised), max and sum per row.
template <bool NEW>
__device__ __forceinline__ void att_unit(const u32x4 (&ub)[32], unsigned char* lds, int w, int lane, int kbase, int T, int NV,
                         float scale) {
  const int c4 = lane >> 4, n = lane & 15;
  const uint16_t* qs = reinterpret_cast<const uint16_t*>(lds + L_Q);
  const uint16_t* kn = reinterpret_cast<const uint16_t*>(lds + L_KN);
  const uint16_t* vn = reinterpret_cast<const uint16_t*>(lds + L_VN);
  float* mg = reinterpret_cast<float*>(lds + L_MG) + w * FW_QROWS * 128;
  float* ml = reinterpret_cast<float*>(lds + L_ML) + w * FW_QROWS * 2;
  constexpr int NKB = NEW ? 2 : 4;
#pragma unroll
  for (int qb = 0; qb < FW_QROWS / 16; ++qb) {
    bf16x8 qv[4];
#pragma unroll
    for (int s = 0; s < 4; ++s) qv[s] = *reinterpret_cast<const bf16x8*>(qs + (qb * 16 + n) * QS + 32 * s + 8 * c4);
    f32x4 S[NKB];
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb) {
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        bf16x8 kv;
        if (NEW) kv = *reinterpret_cast<const bf16x8*>(kn + sigma(kb, n) * QS + 32 * s + 8 * c4);
        else kv = __builtin_bit_cast(bf16x8, ub[kb * 4 + s]);
        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kv, qv[s], acc, 0, 0, 0);
      }
      S[kb] = acc;  // lane: S^T[key sigma(kb, 4 c4 + v)][query qb * 16 + n]
    }
    const int qrow = qb * 16 + n, jq = qrow & 7;
    float m = -INFINITY;
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int key = sigma(kb, 4 * c4 + v);
        const bool ok = NEW ? (key <= jq && key < NV) : (kbase + key < T);
        const float s = ok ? S[kb][v] * scale : -INFINITY;
        S[kb][v] = s;
        m = fmaxf(m, s);
      }
    m = fmaxf(m, __shfl_xor(m, 16));
    m = fmaxf(m, __shfl_xor(m, 32));
    float l = 0.f;
    bf16x8 ph[NKB / 2], pl[NKB / 2];
#pragma unroll
    for (int k2 = 0; k2 < NKB / 2; ++k2) {
      u32x4 hw, lw;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        // k-slot 8 c4 + 2e', 2e' + 1 of this slice: keys from block 2 k2 (e < 2) or 2 k2 + 1
        const int kb = 2 * k2 + (e >> 1);
        const int v0 = 2 * (e & 1);
        float pv[2];
#pragma unroll
        for (int z = 0; z < 2; ++z) {
          const float s = S[kb][v0 + z];
          pv[z] = (s == -INFINITY) ? 0.f : __expf(s - m);
          l += pv[z];
        }
        const uint16_t h0 = f32_to_bf16(pv[0]), h1 = f32_to_bf16(pv[1]);
        hw[e] = (uint32_t)h0 | ((uint32_t)h1 << 16);
        lw[e] = pack2(pv[0] - bf16_to_f32(h0), pv[1] - bf16_to_f32(h1));
      }
      ph[k2] = __builtin_bit_cast(bf16x8, hw);
      pl[k2] = __builtin_bit_cast(bf16x8, lw);
    }
    l += __shfl_xor(l, 16);
    l += __shfl_xor(l, 32);
#pragma unroll
    for (int db = 0; db < 8; ++db) {
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int k2 = 0; k2 < NKB / 2; ++k2) {
        bf16x8 vv;
        if (NEW) vv = *reinterpret_cast<const bf16x8*>(vn + (16 * db + n) * VS + 8 * c4);
        else vv = __builtin_bit_cast(bf16x8, ub[16 + db * 2 + k2]);
        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vv, ph[k2], acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vv, pl[k2], acc, 0, 0, 0);
      }
      // lane: O^T[dim 16 db + 4 c4 + v][query qrow]
      *reinterpret_cast<f32x4*>(mg + qrow * 128 + 16 * db + 4 * c4) = acc;
    }
    if (c4 == 0) {
      ml[qrow * 2] = m;
      ml[qrow * 2 + 1] = l;
    }
  }
}

template <bool CTL>
__device__ __forceinline__ bool att_phase(const FwArgs& a, unsigned char* lds, Ctl& cx, int& nst, int& nat, WaveState& ws,
                          const int* ri, int na, int l, unsigned ep) {
  const int tid = fresh_tid(), w = tid >> 6, lane = tid & 63;
  const int b = blockIdx.x, G = gridDim.x;
  int* fl = reinterpret_cast<int*>(lds + L_FLAG);
  const FwLayer& Ly = a.layers[l];
  const int g = a.nq / a.nkv;
  const int Nqkv = (a.nq + 2 * a.nkv) * a.d;
  const unsigned tq = tagof(ep, l, TG_QKV);
  const rsrc_t rq = mk(a.qkv, (size_t)FW_MMAX * (Nqkv / 2) * 8);
  for (int i = 0;; ++i) {
    const int f = b + G * i;
    if (f >= na) break;
    AttTask t;
    if (!att_task(ri, a.R, a.nkv, f, t)) break;
    ++nst;
    ++nat;
    // ---- raw q / k / v of the (row, kv head) for the NV new tokens: 32 pairs per head row ----
    const int nrow = (g + 2) * t.NV;
    const int np = nrow * 32;
    constexpr int APP = (RAW_ROWS * 32 + FW_THREADS - 1) / FW_THREADS;
    u32x4 v[APP];
    unsigned voff[APP];
#pragma unroll
    for (int q = 0; q < APP; ++q) {
      const int p = min(tid + FW_THREADS * q, np - 1), rr = p >> 5, pw = p & 31;
      const int hs = rr / t.NV, j = rr - hs * t.NV;
      const int hh = hs < g ? t.h * g + hs : (hs == g ? a.nq + t.h : a.nq + a.nkv + t.h);
      voff[q] = ((unsigned)((t.S0 + j) * (Nqkv / 2) + hh * (a.d / 2)) + 2u * (unsigned)pw) * 8u;
    }
    int it = 0;
    while (true) {
#pragma unroll
      for (int q = 0; q < APP; ++q) v[q] = ld16_sc(rq, voff[q]);
      unsigned pend = 0;
#pragma unroll
      for (int q = 0; q < APP; ++q)
        if (tid + FW_THREADS * q < np && !(v[q].y == tq && v[q].w == tq)) pend |= 1u << q;
      if (!__any(pend != 0u)) break;
      if (spin(cx, it, 102)) return false;
    }
    if (!lds_wait(fl + F_DONE, NWAVE * (nst - 1), cx, 204)) return false;
    uint16_t* raw = reinterpret_cast<uint16_t*>(lds + L_RAW);
#pragma unroll
    for (int q = 0; q < APP; ++q) {
      const int p = tid + FW_THREADS * q;
      if (p < np) *reinterpret_cast<u32x2*>(raw + (p >> 5) * 128 + 4 * (p & 31)) = (u32x2){v[q].x, v[q].z};
    }
    // zero the q / new-k / new-v^T operands (rows of absent tokens stay zero)
    {
      u32x4 z = {0u, 0u, 0u, 0u};
      for (int i2 = tid; i2 < (FW_QROWS * QS + 32 * QS + 128 * VS) / 8; i2 += FW_THREADS)
        reinterpret_cast<u32x4*>(lds + L_Q)[i2] = z;
    }
    if constexpr (CTL) {  // rope tables of the new positions, q / k norm weights
      float* cs = reinterpret_cast<float*>(lds + L_RCS);
      float* sn = reinterpret_cast<float*>(lds + L_RSN);
      for (int i2 = lane; i2 < t.NV * 64; i2 += 64) {
        const int j = i2 >> 6, e = i2 & 63;
        cs[i2] = a.rope_cos[(size_t)(t.T + j) * 64 + e];
        sn[i2] = a.rope_sin[(size_t)(t.T + j) * 64 + e];
      }
      uint16_t* qkw = reinterpret_cast<uint16_t*>(lds + L_QKW);
      for (int i2 = lane; i2 < 256; i2 += 64) {
        const uint16_t* src = i2 < 128 ? Ly.q_norm : Ly.k_norm;
        qkw[i2] = src ? src[i2 & 127] : (uint16_t)0;
      }
    }
    lds_signal(fl + F_RAW);
    if (!lds_wait(fl + F_RAW, NWAVE * nst, cx, 205)) return false;
    // ---- q / k norm + RoPE (a wave per head row; lane e rotates the pair (e, e + 64)) ----
    {
      const float* cs = reinterpret_cast<const float*>(lds + L_RCS);
      const float* sn = reinterpret_cast<const float*>(lds + L_RSN);
      const uint16_t* qkw = reinterpret_cast<const uint16_t*>(lds + L_QKW);
      uint16_t* qs = reinterpret_cast<uint16_t*>(lds + L_Q);
      uint16_t* kn = reinterpret_cast<uint16_t*>(lds + L_KN);
      uint16_t* vn = reinterpret_cast<uint16_t*>(lds + L_VN);
      const bool append = t.pb == t.npb - 1;  // this block holds the new keys: write them to the cache
      const size_t head = (size_t)t.r * a.nkv + t.h;
      for (int rr = w; rr < nrow; rr += NWAVE) {
        const int hs = rr / t.NV, j = rr - hs * t.NV;
        float x1 = bf16_to_f32(raw[rr * 128 + lane]), x2 = bf16_to_f32(raw[rr * 128 + lane + 64]);
        if (hs > g) {  // v
          vn[lane * VS + j] = f32_to_bf16(x1);
          vn[(lane + 64) * VS + j] = f32_to_bf16(x2);
          if (append) {
            Ly.v[(head * a.d + lane) * a.cap + t.T + j] = f32_to_bf16(x1);
            Ly.v[(head * a.d + lane + 64) * a.cap + t.T + j] = f32_to_bf16(x2);
          }
          continue;
        }
        const bool isq = hs < g;
        const uint16_t* nwp = (isq ? Ly.q_norm : Ly.k_norm) ? qkw + (isq ? 0 : 128) : nullptr;
        if (nwp) {
          const float ss = wave_sum64(x1 * x1 + x2 * x2);
          const float r = 1.0f / sqrtf(ss / (float)a.d + a.eps);
          x1 = bf16_to_f32(f32_to_bf16((x1 * r) * bf16_to_f32(nwp[lane])));
          x2 = bf16_to_f32(f32_to_bf16((x2 * r) * bf16_to_f32(nwp[lane + 64])));
        }
        const float c0 = cs[j * 64 + lane], s0 = sn[j * 64 + lane];
        const uint16_t o1 = f32_to_bf16(x1 * c0 - x2 * s0);
        const uint16_t o2 = f32_to_bf16(x1 * s0 + x2 * c0);
        if (isq) {
          qs[(hs * 8 + j) * QS + lane] = o1;
          qs[(hs * 8 + j) * QS + lane + 64] = o2;
        } else {
          kn[j * QS + lane] = o1;
          kn[j * QS + lane + 64] = o2;
          if (append) {
            uint16_t* kd = Ly.k + (head * a.cap + t.T + j) * a.d;
            kd[lane] = o1;
            kd[lane + 64] = o2;
          }
        }
      }
    }
    lds_signal(fl + F_PREP);
    // ---- units ----
    if constexpr (!CTL) {
      const int c = t.pb * FW_CW + w;
      if (!lds_wait(fl + F_PREP, NWAVE * nst, cx, 206)) return false;
      if (c < t.nh) {
        if (!ws.has || ws.cur.op != OP_ATT || ws.cur.l != l || ws.cur.i != i) {
          if (lane == 0) __hip_atomic_fetch_or(a.err, 2u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          cx.ab = 1;
          return false;
        }
        att_unit<false>(ws.ub, lds, w, lane, c * FW_AKEYS, t.T, t.NV, a.scale);
        ws.has = next_unit(a, ri, na, G, b, w, ws.cur);
        refill(ws, a, ri, G, b, w, lane);
      } else if (c == t.nh) {
        att_unit<true>(ws.ub, lds, w, lane, 0, t.T, t.NV, a.scale);
      } else {
        float* mg = reinterpret_cast<float*>(lds + L_MG) + w * FW_QROWS * 128;
        float* ml = reinterpret_cast<float*>(lds + L_ML) + w * FW_QROWS * 2;
        for (int i2 = lane; i2 < FW_QROWS * 128; i2 += 64) mg[i2] = 0.f;
        if (lane < FW_QROWS) {
          ml[lane * 2] = -INFINITY;
          ml[lane * 2 + 1] = 0.f;
        }
      }
    }
    lds_signal(fl + F_RES);
    if (!lds_wait(fl + F_RES, NWAVE * nat, cx, 207)) return false;
    // ---- merge the unit results (fixed wave order) into this block's partial ----
    for (int e2 = tid; e2 < FW_QROWS * 16; e2 += FW_THREADS) {
      const int qrow = e2 >> 4, d0 = 8 * (e2 & 15);
      const float* mg = reinterpret_cast<const float*>(lds + L_MG);
      const float* ml = reinterpret_cast<const float*>(lds + L_ML);
      float mx = -INFINITY;
#pragma unroll
      for (int u = 0; u < FW_CW; ++u) mx = fmaxf(mx, ml[(u * FW_QROWS + qrow) * 2]);
      float o[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
      float ls = 0.f;
#pragma unroll
      for (int u = 0; u < FW_CW; ++u) {
        const float mu = ml[(u * FW_QROWS + qrow) * 2];
        const float e = (mu == -INFINITY) ? 0.f : __expf(mu - mx);
        ls += e * ml[(u * FW_QROWS + qrow) * 2 + 1];
        const f32x4 p0 = *reinterpret_cast<const f32x4*>(mg + (u * FW_QROWS + qrow) * 128 + d0);
        const f32x4 p1 = *reinterpret_cast<const f32x4*>(mg + (u * FW_QROWS + qrow) * 128 + d0 + 4);
#pragma unroll
        for (int z = 0; z < 4; ++z) {
          o[z] += e * p0[z];
          o[4 + z] += e * p1[z];
        }
      }
      const unsigned tp = tagof(ep, l, TG_ATTP);
      const size_t pidx = ((size_t)t.r * a.nkv + t.h) * a.npb_cap + t.pb;
      const size_t nrec = (size_t)a.R * a.nkv * a.npb_cap * FW_QROWS;
      const rsrc_t ro = mk(a.ao, nrec * 128 * 8), rm = mk(a.aml, nrec * 2 * 8);
      const unsigned ob = (unsigned)((pidx * FW_QROWS + qrow) * 128 + d0) * 8u;
#pragma unroll
      for (int z = 0; z < 4; ++z)
        st16_sc(ro, ob + 16u * z, (u32x4){__float_as_uint(o[2 * z]), tp, __float_as_uint(o[2 * z + 1]), tp});
      if ((e2 & 15) == 0)
        st16_sc(rm, (unsigned)((pidx * FW_QROWS + qrow) * 2) * 8u, (u32x4){__float_as_uint(mx), tp, __float_as_uint(ls), tp});
    }
    lds_signal(fl + F_DONE);
  }
  return true;
}

// ---------------------------------------------------------------------------------------
// control-wave tasks
// ---------------------------------------------------------------------------------------
// combine the block partials of (slot s, head hq) in part order -> att (bf16 pairs LL)
__device__ __forceinline__ bool comb_tasks(const FwArgs& a, const int* ri, Ctl& cx, int l, unsigned ep) {
  const int lane = fresh_tid() & 63;
  const int b = blockIdx.x, G = gridDim.x;
  const int g = a.nq / a.nkv;
  const unsigned tp = tagof(ep, l, TG_ATTP), ta = tagof(ep, l, TG_ATT);
  const size_t nrec = (size_t)a.R * a.nkv * a.npb_cap * FW_QROWS;
  const rsrc_t ro = mk(a.ao, nrec * 128 * 8), rm = mk(a.aml, nrec * 2 * 8);
  const rsrc_t rat = mk(a.att, (size_t)FW_MMAX * (a.nq * a.d / 2) * 8);
  for (int f = b; f < a.M * a.nq; f += G) {
    const int s = f / a.nq, hq = f - s * a.nq;
    const int r = a.slot_row[s];
    const int rr = (r >= 0 && r < a.R) ? r : -1;
    int j = -1;
    if (rr >= 0) {
      j = s - ri[rr * 8 + RI_S0];
      if (j < 0 || j >= ri[rr * 8 + RI_NV]) j = -1;
    }
    float o0 = 0.f, o1 = 0.f, lsum = 1.f;
    if (j >= 0) {
      const int h = hq / g, gh = hq - h * g, qrow = gh * 8 + j;
      const int npb = ri[rr * 8 + RI_NPB];
      const size_t base = ((size_t)rr * a.nkv + h) * a.npb_cap;
      float mx = -INFINITY, ls = 0.f;
      // 8 parts per pass, merged in part order with a running max
      for (int p0 = 0; p0 < npb; p0 += 8) {
        const int cnt = min(8, npb - p0);
        u32x4 ov[8];
        u32x4 mv = {0u, 0u, 0u, 0u};
        unsigned pend = 0;
#pragma unroll
        for (int k = 0; k < 8; ++k)
          if (k < cnt) pend |= 1u << k;
        bool mpend = lane < cnt;
        int it = 0;
        while (true) {
#pragma unroll
          for (int k = 0; k < 8; ++k)
            if (pend >> k & 1u) ov[k] = ld16_sc(ro, (unsigned)(((base + p0 + k) * FW_QROWS + qrow) * 128 + 2 * lane) * 8u);
          if (mpend) mv = ld16_sc(rm, (unsigned)(((base + p0 + lane) * FW_QROWS + qrow) * 2) * 8u);
#pragma unroll
          for (int k = 0; k < 8; ++k)
            if ((pend >> k & 1u) && ov[k].y == tp && ov[k].w == tp) pend &= ~(1u << k);
          if (mpend && mv.y == tp && mv.w == tp) mpend = false;
          if (!__any(pend != 0u || mpend)) break;
          if (spin(cx, it, 103)) return false;
        }
#pragma unroll
        for (int k = 0; k < 8; ++k) {
          if (k >= cnt) break;
          const float mk_ = __uint_as_float(__shfl(mv.x, k)), lk = __uint_as_float(__shfl(mv.z, k));
          const float nm = fmaxf(mx, mk_);
          const float e_old = (mx == -INFINITY) ? 0.f : __expf(mx - nm);
          const float e_new = (mk_ == -INFINITY) ? 0.f : __expf(mk_ - nm);
          ls = ls * e_old + lk * e_new;
          o0 = o0 * e_old + __uint_as_float(ov[k].x) * e_new;
          o1 = o1 * e_old + __uint_as_float(ov[k].z) * e_new;
          mx = nm;
        }
      }
      lsum = ls;
    }
    const float inv = (j >= 0 && lsum > 0.f) ? 1.0f / lsum : 0.f;
    st8_sc(rat, (unsigned)(s * (a.nq * a.d / 2) + hq * (a.d / 2) + lane) * 8u, pack2(o0 * inv, o1 * inv), ta);
  }
  return true;
}

// split-K reduction of tile t + residual: x_new = bf16(x_old + sum_kr part[kr]); the new
// rows' sums of squares per 16 columns.  Lane (m = lane / 8, column pair lane % 8).
__device__ __forceinline__ bool reduce_tasks(const FwArgs& a, Ctl& cx, const FwLin& L, const u64* part, unsigned tpart,
                             unsigned txold, unsigned txnew) {
  const int lane = fresh_tid() & 63;
  const int b = blockIdx.x, G = gridDim.x;
  const int m = lane >> 3, cp = lane & 7;
  const int H = a.H;
  const rsrc_t rp = mk(part, (size_t)L.ks * FW_MMAX * H * 8);
  const rsrc_t rx = mk(a.x, (size_t)FW_MMAX * (H / 2) * 8);
  const rsrc_t rs = mk(a.xss, (size_t)FW_MMAX * (H / 16) * 8);
  for (int t = b; t < L.NT; t += G) {
    const int n0 = t * 16 + 2 * cp;
    const bool live = m < a.M;
    u32x4 pv[4];
    u32x2 xo = {0u, 0u};
    unsigned pend = 0;
    bool xpend = live;
#pragma unroll
    for (int k = 0; k < 4; ++k)
      if (live && k < L.ks) pend |= 1u << k;
    int it = 0;
    while (true) {
#pragma unroll
      for (int k = 0; k < 4; ++k)
        if (pend >> k & 1u) pv[k] = ld16_sc(rp, (unsigned)((k * FW_MMAX + m) * H + n0) * 8u);
      if (xpend) xo = ld8_sc(rx, (unsigned)(m * (H / 2) + n0 / 2) * 8u);
#pragma unroll
      for (int k = 0; k < 4; ++k)
        if ((pend >> k & 1u) && pv[k].y == tpart && pv[k].w == tpart) pend &= ~(1u << k);
      if (xpend && xo.y == txold) xpend = false;
      if (!__any(pend != 0u || xpend)) break;
      if (spin(cx, it, 104)) return false;
    }
    float s0 = 0.f, s1 = 0.f;
#pragma unroll
    for (int k = 0; k < 4; ++k)
      if (k < L.ks) {
        s0 += __uint_as_float(pv[k].x);
        s1 += __uint_as_float(pv[k].z);
      }
    const uint16_t h0 = f32_to_bf16(s0 + lo_f(xo.x)), h1 = f32_to_bf16(s1 + hi_f(xo.x));
    const float f0 = bf16_to_f32(h0), f1 = bf16_to_f32(h1);
    float q = f0 * f0 + f1 * f1;
    q += __shfl_xor(q, 1);
    q += __shfl_xor(q, 2);
    q += __shfl_xor(q, 4);
    if (live) {
      st8_sc(rx, (unsigned)(m * (H / 2) + n0 / 2) * 8u, (uint32_t)h0 | ((uint32_t)h1 << 16), txnew);
      if (cp == 0) st8_sc(rs, (unsigned)(m * (H / 16) + t) * 8u, __float_as_uint(q), txnew);
    }
  }
  return true;
}

// embedding rows of the M slots (dequantised bf16(fma(s, q, b))) and their sums of squares
__device__ __forceinline__ void embed_tasks(const FwArgs& a, unsigned ep) {
  const int lane = fresh_tid() & 63;
  const int b = blockIdx.x, G = gridDim.x;
  const int nt = a.H / 16;
  const unsigned tx = tagof(ep, -1, TG_X);
  const QLinear& E = a.embed;
  const rsrc_t rx = mk(a.x, (size_t)FW_MMAX * (a.H / 2) * 8);
  const rsrc_t rs = mk(a.xss, (size_t)FW_MMAX * nt * 8);
  for (int f = b * 64 + lane; f < a.M * nt; f += G * 64) {
    const int m = f / nt, tt = f - m * nt;
    int tok = a.slot_tok[m];
    if (tok < 0 || tok >= E.N) tok = 0;
    const int t = tok >> 4, r = tok & 15;
    float q = 0.f;
    uint32_t outw[8];
#pragma unroll
    for (int half = 0; half < 2; ++half) {
      const int kw = tt * 2 + half;
      const int gq = kw >> 3, w8 = kw & 7, am = w8 >> 2, c = w8 & 3;
      const int gp = gq >> 1, gi = gq & 1;
      const uint32_t word = E.qw[(((size_t)t * E.GP + gp) * 64 + c * 16 + r) * 4 + gi * 2 + am];
      const uint32_t sbw = E.sb[tile_sb_word(t, r, gp, gi, E.GP)];
      const float sc = bf16_to_f32((uint16_t)(sbw & 0xFFFFu)), bi = bf16_to_f32((uint16_t)(sbw >> 16));
#pragma unroll
      for (int p = 0; p < 4; ++p) {
        const uint16_t h0 = f32_to_bf16(__builtin_fmaf(sc, (float)((word >> (4 * p)) & 0xFu), bi));
        const uint16_t h1 = f32_to_bf16(__builtin_fmaf(sc, (float)((word >> (16 + 4 * p)) & 0xFu), bi));
        const float v0 = bf16_to_f32(h0), v1 = bf16_to_f32(h1);
        q += v0 * v0;
        q += v1 * v1;
        outw[half * 4 + p] = (uint32_t)h0 | ((uint32_t)h1 << 16);
      }
    }
#pragma unroll
    for (int k = 0; k < 4; ++k)
      st16_sc(rx, (unsigned)(m * (a.H / 2) + tt * 8 + 2 * k) * 8u, (u32x4){outw[2 * k], tx, outw[2 * k + 1], tx});
    st8_sc(rs, (unsigned)(m * nt + tt) * 8u, __float_as_uint(q), tx);
  }
}

}  // namespace

// ---------------------------------------------------------------------------------------
// the kernel
// ---------------------------------------------------------------------------------------
__global__ void __launch_bounds__(FW_THREADS) fused_forward_kernel(FwArgs a) {
  MC_DYN_LDS(lds);
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
  const int b = blockIdx.x, G = gridDim.x;
  Ctl cx;
  cx.t0 = wall_clock64();
  cx.err = a.err;
  cx.ab = 0;
  const unsigned ep = *a.epoch;
  int* fl = reinterpret_cast<int*>(lds + L_FLAG);
  int* ri = reinterpret_cast<int*>(lds + L_ROW);
  if (tid == 0) {
    for (int k = 0; k < 8; ++k) fl[k] = 0;
    int base = 0;
    for (int r = 0; r < a.R; ++r) {
      const int T = a.qbase[r], NV = a.n_valid[r];
      const int nh = (T + FW_AKEYS - 1) / FW_AKEYS;
      const int npb = NV > 0 ? (nh + 1 + FW_CW - 1) / FW_CW : 0;
      ri[r * 8 + RI_T] = T;
      ri[r * 8 + RI_NV] = NV;
      ri[r * 8 + RI_S0] = a.row_slot0[r];
      ri[r * 8 + RI_NPB] = npb;
      ri[r * 8 + RI_BASE] = base;
      base += a.nkv * npb;
    }
    fl[F_NA] = base;
  }
  __syncthreads();
  const int na = fl[F_NA];
  // dequant constants: one in an SGPR, the other in a VGPR (v_and_or_b32 reads one SGPR)
  const uint32_t mask = DQ_MASK;
  uint32_t magic;
  MC_TO_VGPR(magic, DQ_MAGIC);

  int nst = 0, nat = 0;
  WaveState ws;
  ws.has = false;
  if (w < FW_CW) {
    ws.cur = Unit{0, -1, 0};
    ws.has = next_unit(a, ri, na, G, b, w, ws.cur);
    refill(ws, a, ri, G, b, w, lane);
  } else {
    embed_tasks(a, ep);
  }
  // phases in order: per layer QKV, ATT, O, GU, DN; then the head
  for (int step = 0; step < 5 * a.L + (a.with_head ? 1 : 0); ++step) {
    const int l = step / 5, op = l == a.L ? OP_HEAD : step % 5;
    if (op == OP_ATT) {
      if (w == FW_CW) {
        if (!att_phase<true>(a, lds, cx, nst, nat, ws, ri, na, l, ep)) return;
        if (!comb_tasks(a, ri, cx, l, ep)) return;
      } else {
        if (!att_phase<false>(a, lds, cx, nst, nat, ws, ri, na, l, ep)) return;
      }
      continue;
    }
    const FwLayer* Ly = op == OP_HEAD ? nullptr : a.layers + l;
    const unsigned tx_in = l == 0 ? tagof(ep, -1, TG_X) : tagof(ep, l - 1, TG_XD);
    XIn in;
    Epi e;
    in.eps = a.eps;
    in.ss = a.xss;
    in.ssn = a.H / 16;
    if (op == OP_QKV || op == OP_GU || op == OP_HEAD) {
      in.src = a.x;
      in.ldw = a.H / 2;
      in.K = a.H;
      in.tag = op == OP_QKV ? tx_in : op == OP_GU ? tagof(ep, l, TG_XO) : tagof(ep, a.L - 1, TG_XD);
      in.nw = op == OP_QKV ? Ly->in_norm : op == OP_GU ? Ly->post_norm : a.final_norm;
    } else {
      in.src = op == OP_O ? a.att : a.act;
      in.ldw = op == OP_O ? a.nq * a.d / 2 : a.I / 2;
      in.K = op == OP_O ? a.nq * a.d : a.I;
      in.tag = op == OP_O ? tagof(ep, l, TG_ATT) : tagof(ep, l, TG_ACT);
      in.nw = nullptr;
    }
    if (op == OP_QKV) e = Epi{0, a.qkv, (a.nq + 2 * a.nkv) * a.d / 2, tagof(ep, l, TG_QKV)};
    else if (op == OP_GU) e = Epi{1, a.act, a.I / 2, tagof(ep, l, TG_ACT)};
    else if (op == OP_O) e = Epi{2, a.opart, a.H, tagof(ep, l, TG_OP)};
    else if (op == OP_DN) e = Epi{2, a.dpart, a.H, tagof(ep, l, TG_DP)};
    else e = Epi{3, nullptr, 0, 0u};
    if (w == FW_CW) {
      if (!gemv_phase<true>(a, lds, cx, nst, ws, ri, na, op, l, in, e, mask, magic)) return;
      if (op == OP_O && !reduce_tasks(a, cx, Ly->o, a.opart, tagof(ep, l, TG_OP), tx_in, tagof(ep, l, TG_XO))) return;
      if (op == OP_DN &&
          !reduce_tasks(a, cx, Ly->dn, a.dpart, tagof(ep, l, TG_DP), tagof(ep, l, TG_XO), tagof(ep, l, TG_XD)))
        return;
    } else {
      if (!gemv_phase<false>(a, lds, cx, nst, ws, ri, na, op, l, in, e, mask, magic)) return;
    }
  }
}

__global__ void epoch_bump_kernel(unsigned* epoch) {
  if (threadIdx.x == 0 && blockIdx.x == 0) *epoch = *epoch + 1u;
}

// ---------------------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------------------
FwLin fused_lin(const QLinear& L, int max_ks) {
  FwLin f;
  f.qw = L.qw;
  f.sb = L.sb;
  f.N = L.N;
  f.K = L.K;
  f.NT = L.NT;
  f.GP = L.GP;
  int ks = (L.GP + FW_UGP - 1) / FW_UGP;
  int ugp = (L.GP + ks - 1) / ks;
  ugp += ugp & 1;  // even: 16-byte scale/bias loads stay aligned
  ks = (L.GP + ugp - 1) / ugp;
  f.ks = ks;
  f.ugp = ugp;
  if (ks > max_ks) f.ks = 0;
  return f;
}

int fused_npb_cap(int cap) { return (cap / FW_AKEYS + 1 + FW_CW - 1) / FW_CW; }

bool fused_supported(const mc_model_config& c, int M, int cap, const char** why) {
  const char* r = nullptr;
  const int g = c.n_kv_heads > 0 ? c.n_q_heads / c.n_kv_heads : 0;
  if (M < 1 || M > FW_MMAX) r = "more than 8 tokens";
  else if (c.head_dim != 128) r = "head_dim != 128";
  else if (g < 1 || g > 4 || g * c.n_kv_heads != c.n_q_heads) r = "GQA group outside 1..4";
  else if (c.hidden % 256 || c.hidden > FW_UGP * 128) r = "hidden size (multiple of 256, <= 2560)";
  else if (c.intermediate % 256 || (c.n_q_heads * c.head_dim) % 256) r = "intermediate / attention width not a multiple of 256";
  else if (c.n_layers < 1 || c.n_layers > 62) r = "layer count";
  else if (c.n_experts > 0) r = "mixture of experts";
  else if (cap % FW_AKEYS) r = "cache stride";
  else {
    QLinear o, dn;
    o.N = c.hidden; o.K = c.n_q_heads * c.head_dim; o.GP = (o.K + 127) / 128;
    dn.N = c.hidden; dn.K = c.intermediate; dn.GP = (dn.K + 127) / 128;
    if (fused_lin(o, 4).ks == 0 || fused_lin(dn, 4).ks == 0) r = "split-K beyond 4 ranges";
  }
  if (why) *why = r;
  return r == nullptr;
}

size_t fused_lds_bytes() { return (size_t)L_TOTAL; }

int fused_grid(int device) {
  static int cached[64] = {0};
  if (device >= 0 && device < 64 && cached[device]) return cached[device];
  int cus = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess || cus <= 0) return 0;
  static bool attr = false;
  if (!attr) {
    if (hipFuncSetAttribute((const void*)fused_forward_kernel, hipFuncAttributeMaxDynamicSharedMemorySize, L_TOTAL) !=
        hipSuccess)
      return 0;
    attr = true;
  }
  int occ = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, (const void*)fused_forward_kernel, FW_THREADS, L_TOTAL) !=
          hipSuccess ||
      occ < 1)
    return 0;
  // one block per CU: every block must be resident at once (they wait on each other)
  if (device >= 0 && device < 64) cached[device] = cus;
  return cus;
}

int launch_fused_forward(const FwArgs& a, int grid, hipStream_t st) {
  if (grid < 1) return fail(MC_E_STATE, "fused forward: no resident grid on this device");
  hipLaunchKernelGGL(fused_forward_kernel, dim3(grid), dim3(FW_THREADS), L_TOTAL, st, a);
  MC_HIP(hipGetLastError());
  return MC_OK;
}

int launch_epoch_bump(unsigned* epoch, hipStream_t st) {
  hipLaunchKernelGGL(epoch_bump_kernel, dim3(1), dim3(64), 0, st, epoch);
  MC_HIP(hipGetLastError());
  return MC_OK;
}

}  // namespace mc
