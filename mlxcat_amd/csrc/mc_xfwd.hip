// mc_xfwd.hip -- the XCD-partitioned persistent verify forward (declarations and layout in
// mc_xfwd.hpp).
//
// Per layer every block runs the same phase sequence; XCD i works on its slice:
//   RX   x    = bf16(x1_prev + sum_j dpart_j)   columns [cb blk, cb (blk+1)), all 8 XCDs redundantly
//             (layer 0: the embedding rows); also the sums of squares of those columns
//   QKV  q, k, v of kv head i and its g q heads = rmsnorm(x) . Wqkv^T        (local)
//   ATT  per (row, 64-key chunk): q/k norm + RoPE, append the new keys, softmax partials
//   CMB  per (token, q head): merge the chunk partials in chunk order -> att  (local)
//   O    opart_i = att_i . Wo[:, heads of i]^T                               (read by every XCD)
//   RX1  x1 = bf16(x + sum_j opart_j)
//   GU   act_i = silu(g) u over act columns [128 pdn[i], 128 pdn[i+1])       (local)
//   DN   dpart_i = act_i . Wdn[:, same columns]^T                            (read by every XCD)
// then RX once more (the final residual stream) and the LM head over all 256 blocks.
//
// Exchange words: 8 bytes, (32-bit payload, 32-bit tag).  XCD-local words are written with
// plain stores (they stay in the XCD's L2) and read with device-scope (sc1) loads, which
// miss the CU's L1; words read by other XCDs are written with sc1 stores.  Every buffer is
// rewritten only by a phase that depends (through the data) on every reader of its previous
// contents, so a reader never sees a newer tag than the one it waits for.
//
// Every wait is bounded: after XF_TIMEOUT a wave sets *err and leaves; the others see *err
// (or time out themselves), so the kernel always ends.
#include "mc_xfwd.hpp"

#include <algorithm>

// LDS accesses of the loader waves go through inline asm: after a direct-to-LDS load the
// compiler would otherwise wait for every outstanding load before any LDS access.
#ifndef MC_EMULATE
#define XF_LDS_RD(addr, out) \
  asm volatile("ds_read_b32 %0, %1\n\ts_waitcnt lgkmcnt(0)" : "=v"(out) : "v"(addr) : "memory")
#define XF_LDS_WR(addr, val) asm volatile("ds_write_b32 %0, %1\n\ts_waitcnt lgkmcnt(0)" ::"v"(addr), "v"(val) : "memory")
#define XF_XCC_ID(out) asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID, 0, 4)" : "=s"(out))
// s_waitcnt immediates: vmcnt in bits 3:0 and 15:14, expcnt 6:4, lgkmcnt 11:8
#define XF_WAIT_VM_NF() __builtin_amdgcn_s_waitcnt(((2 * XF_NF) & 0xF) | (((2 * XF_NF) >> 4) << 14) | 0x70 | 0xF00)
#define XF_WAIT_VM0() __builtin_amdgcn_s_waitcnt(0x0F70)
// a wave-uniform value in a scalar register (v_readfirstlane with an SGPR result)
__device__ inline int xf_uniform(int v) {
  int r;
  asm volatile("v_readfirstlane_b32 %0, %1" : "=s"(r) : "v"(v));
  return r;
}
#define XF_UNIFORM(v) xf_uniform(v)
#else
#define XF_UNIFORM(v) (v)
#define XF_WAIT_VM_NF() ((void)0)
#define XF_WAIT_VM0() ((void)0)
#endif

namespace mc {

typedef unsigned long long u64;
typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8;
typedef __attribute__((__vector_size__(4 * sizeof(short)))) short s16x4;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4;
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x2 __attribute__((ext_vector_type(2)));
typedef __amdgpu_buffer_rsrc_t rsrc_t;
#ifdef MC_EMULATE
typedef void lds_void_t;
typedef unsigned char lds_u8_t;
#else
typedef __attribute__((address_space(3))) void lds_void_t;
typedef __attribute__((address_space(3))) unsigned char lds_u8_t;
#endif

namespace {

constexpr int CP_PLAIN = 0, CP_NT = 2, CP_SC1 = 16;
constexpr u64 XF_TIMEOUT = 20000000ull;  // 200 ms of the 100 MHz real-time counter
enum { TG_X = 0, TG_Q = 1, TG_R = 2, TG_A = 3, TG_O = 4, TG_X1 = 5, TG_U = 6, TG_D = 7 };
enum { OP_Q = 0, OP_O = 1, OP_U = 2, OP_D = 3, OP_HEAD = 4 };
enum { RX_EMBED = 0, RX_DOWN = 1, RX_O = 2 };
// control words at LDS offset 0 (ints)
enum { C_LOADED = 0, C_CONSUMED = 8, C_BAR = 16, C_XI = 17, C_J = 18, C_KVB = 20, C_ROWS = 24 };
// row info (8 ints per row, from C_ROWS)
enum { RI_T = 0, RI_NV = 1, RI_S0 = 2, RI_NCH = 3, RI_UB = 4 };
constexpr int CTL_BYTES = (C_ROWS + 8 * XF_MMAX) * 4;

// tag of phase k of layer l (l = 0 .. L; RX of layer L is the final residual stream)
__device__ inline unsigned tagof(unsigned ep, int l, int k) { return ep * 1024u + (unsigned)(l * 16 + k); }

// ---------------------------------------------------------------------------------------
// memory access (buffer descriptors: out-of-range loads read 0, stores are dropped)
// ---------------------------------------------------------------------------------------
__device__ inline rsrc_t mk(const void* p, size_t bytes) {
  const int n = bytes > 0x7FFFFFF0ull ? 0x7FFFFFF0 : (int)bytes;
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, n, 0x00020000);
}
// A buffer descriptor from a base and a size that the compiler may not know to be
// wave-uniform: both go through readfirstlane, so the descriptor lives in scalar registers
// (a descriptor in vector registers would make every buffer instruction a loop over lanes).
__device__ inline rsrc_t mk_uniform(const void* p, unsigned bytes) {
  const unsigned long long u = (unsigned long long)(uintptr_t)p;
  const unsigned lo = __builtin_amdgcn_readfirstlane((unsigned)u);
  const unsigned hi = __builtin_amdgcn_readfirstlane((unsigned)(u >> 32));
  const unsigned n = __builtin_amdgcn_readfirstlane(bytes);
  return mk(reinterpret_cast<const void*>((uintptr_t)(((unsigned long long)hi << 32) | lo)), n);
}

__device__ inline rsrc_t mkd(const void* p, size_t bytes) {
  return mk_uniform(p, (unsigned)(bytes > 0x7FFFFFF0ull ? 0x7FFFFFF0ull : bytes));
}

template <int CP>
__device__ inline u32x4 bld16(rsrc_t r, unsigned off) { return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, CP); }
template <int CP>
__device__ inline void bst8(rsrc_t r, unsigned off, unsigned data, unsigned tag) {
  __builtin_amdgcn_raw_buffer_store_b64((u32x2){data, tag}, r, off, 0, CP);
}
template <int CP>
__device__ inline void bst16(rsrc_t r, unsigned off, u32x4 v) { __builtin_amdgcn_raw_buffer_store_b128(v, r, off, 0, CP); }

__device__ inline float lo_f(uint32_t w) { return __uint_as_float(w << 16); }
__device__ inline float hi_f(uint32_t w) { return __uint_as_float(w & 0xFFFF0000u); }
__device__ inline uint32_t pack2(float a, float b) { return (uint32_t)f32_to_bf16(a) | ((uint32_t)f32_to_bf16(b) << 16); }
__device__ inline float bfr(float x) { return bf16_to_f32(f32_to_bf16(x)); }

__device__ inline bf16x8 dequant_word(uint32_t w, uint32_t mask, uint32_t magic) {
  u32x4 p;
  p.x = ((w << 3) & mask) | magic;
  p.y = ((w >> 1) & mask) | magic;
  p.z = ((w >> 5) & mask) | magic;
  p.w = ((w >> 9) & mask) | magic;
  return __builtin_bit_cast(bf16x8, p);
}
__device__ inline float silu_f(float z) { return z / (1.0f + __expf(-z)); }

__device__ inline unsigned lds_addr(const void* p) { return (unsigned)(uintptr_t)(const lds_u8_t*)p; }

// ---------------------------------------------------------------------------------------
// bounded waiting
// ---------------------------------------------------------------------------------------
struct Ctl {
  u64 t0;
  unsigned* err;
};
// One wait iteration; true when the wave must give up.
__device__ inline bool spin(Ctl& c, int& it) {
  __builtin_amdgcn_s_sleep(1);
  if ((++it & 15) != 0) return false;
  if (__hip_atomic_load(c.err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0u) return true;
  if (wall_clock64() - c.t0 > XF_TIMEOUT) {
    if ((threadIdx.x & 63) == 0) __hip_atomic_fetch_or(c.err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    MC_TRACE_TIMEOUT(it);
    return true;
  }
  return false;
}

__device__ inline float wave_sum64(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  return v;
}

// ---------------------------------------------------------------------------------------
// per-block context
// ---------------------------------------------------------------------------------------
struct Ctx {
  unsigned char* lds;
  int xi, j, gb, G;  // XCD, block within the XCD, block id over the grid, grid
  unsigned ep;
  Ctl cx;
  int w, lane;       // compute wave 0..7 / loader 0..3, lane
  int rc;            // ring chunks consumed (compute) or issued (loader)
  int nb;            // compute-wave barriers passed
  int M, wh;         // tokens of the launch; 1: the LM head runs
};

__device__ inline int* ctl_of(unsigned char* lds) { return reinterpret_cast<int*>(lds); }
__device__ inline const int* rows_of(unsigned char* lds) { return reinterpret_cast<const int*>(lds) + C_ROWS; }
// field f of row r's info, wave-uniform
__device__ inline int row_info(const int* ri, int r, int f) { return ri[r * 8 + f]; }
__device__ inline unsigned char* ring_of(const XArgs& a, unsigned char* lds, int w) {
  return lds + a.o_ring + (size_t)w * a.ring_slots * XF_SLOT;
}

// barrier of the 4 compute waves (LDS counter; the loaders never take part)
__device__ inline bool cw_barrier(Ctx& c) {
  int* bar = ctl_of(c.lds) + C_BAR;
  ++c.nb;
  MC_FENCE();
  __builtin_amdgcn_s_waitcnt(0xC07F);  // this wave's LDS accesses are done
  if (c.lane == 0) __hip_atomic_fetch_add(bar, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
  int it = 0;
  while (__hip_atomic_load(bar, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) < XF_NCW * c.nb)
    if (spin(c.cx, it)) return false;
  MC_FENCE();
  return true;
}

// ---------------------------------------------------------------------------------------
// phase descriptors (shared by the compute waves and the loaders, so that both walk the
// same sequence of ring chunks)
// ---------------------------------------------------------------------------------------
struct PD {
  XLin L;
  int ntl;    // XCD-local tiles (head: all tiles)
  int pk0;    // first group pair of the K range
  int np;     // group pairs
  int kind;   // OP_*
  int tbase;  // GU: first global tile
};

__device__ inline PD phase_desc(const XArgs& a, int op, int l, int xi) {
  PD p;
  p.kind = op;
  p.tbase = 0;
  const int g = a.nq / a.nkv;
  if (op == OP_HEAD) {
    p.L = a.head; p.ntl = a.head.NT; p.pk0 = 0; p.np = a.head.GP;
    return p;
  }
  const XLayer& Ly = a.layers[l];
  if (op == OP_Q) {
    p.L = Ly.qkv; p.ntl = (g + 2) * a.d / 16; p.pk0 = 0; p.np = Ly.qkv.GP;
  } else if (op == OP_O) {
    p.L = Ly.o; p.ntl = Ly.o.NT; p.np = g * a.d / 128; p.pk0 = xi * p.np;
  } else if (op == OP_U) {
    p.L = Ly.gu; p.tbase = 16 * a.pdn[xi]; p.ntl = 16 * (a.pdn[xi + 1] - a.pdn[xi]); p.pk0 = 0; p.np = Ly.gu.GP;
  } else {
    p.L = Ly.dn; p.ntl = Ly.dn.NT; p.pk0 = a.pdn[xi]; p.np = a.pdn[xi + 1] - a.pdn[xi];
  }
  return p;
}

// Tiles of this block in a phase: local index lt = first + k stride (k = 0 .. n - 1).
__device__ inline void block_tiles(const PD& p, const Ctx& c, int bpx, int& first, int& stride, int& n) {
  if (p.kind == OP_HEAD) {
    first = c.gb; stride = c.G;
  } else {
    first = c.j; stride = bpx;
  }
  n = p.ntl > first ? (p.ntl - first + stride - 1) / stride : 0;
}

// Global tile of XCD-local tile lt.
__device__ inline int global_tile(const XArgs& a, const PD& p, int xi, int lt) {
  if (p.kind == OP_Q) {
    const int g = a.nq / a.nkv, dt = a.d / 16, qt = g * dt;
    if (lt < qt) return xi * qt + lt;
    if (lt < qt + dt) return a.nq * dt + xi * dt + (lt - qt);
    return (a.nq + a.nkv) * dt + xi * dt + (lt - qt - dt);
  }
  return p.tbase + lt;
}

// Attention work of a row: chunks of 64 keys over [0, T + NV).
__device__ inline int att_chunks(int T, int NV) { return NV > 0 ? (T + NV + 63) / 64 : 0; }

// ---------------------------------------------------------------------------------------
// loader waves
// ---------------------------------------------------------------------------------------
#ifdef MC_EMULATE
__device__ inline void xf_publish(unsigned char* lds, int w, int v) { ctl_of(lds)[C_LOADED + w] = v; }
__device__ inline int xf_consumed(unsigned char* lds, int w) { return ctl_of(lds)[C_CONSUMED + w]; }
#else
__device__ inline void xf_publish(unsigned char* lds, int w, int v) { XF_LDS_WR(lds_addr(ctl_of(lds) + C_LOADED + w), v); }
__device__ inline int xf_consumed(unsigned char* lds, int w) {
  int v;
  XF_LDS_RD(lds_addr(ctl_of(lds) + C_CONSUMED + w), v);
  return v;
}
#endif

struct Loader {
  const XArgs* a;
  Ctx* c;
  unsigned char* ring;
  int cons;  // last seen consumed count
};

// Wait for a free slot; then the chunk's two loads: 1 KiB at (ra, offa + 16 lane) and, for
// weights, the 32 scale/bias words of the chunk's 16 rows x 2 groups (lanes < 32 at
// offs[lane]), else a 4-byte placeholder load, so that every chunk counts two loads.
__device__ inline bool push_chunk(Loader& L, rsrc_t ra, unsigned offa, bool with_sb, rsrc_t rs, unsigned offs) {
  Ctx& c = *L.c;
  const int RS = L.a->ring_slots;
  if (c.rc - L.cons >= RS) {
    XF_WAIT_VM0();
    xf_publish(c.lds, c.w, c.rc);
    int it = 0;
    while (c.rc - (L.cons = xf_consumed(c.lds, c.w)) >= RS)
      if (spin(c.cx, it)) return false;
  }
  unsigned char* slot = L.ring + (size_t)(c.rc % RS) * XF_SLOT;
  __builtin_amdgcn_raw_ptr_buffer_load_lds(ra, (lds_void_t*)slot, 16, offa + 16u * (unsigned)c.lane, 0, 0, CP_NT);
  if (with_sb) {
    if (c.lane < 32) __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_void_t*)(slot + 1024), 4, offs, 0, 0, CP_NT);
  } else {
    if (c.lane == 0) __builtin_amdgcn_raw_ptr_buffer_load_lds(ra, (lds_void_t*)(slot + 1024), 4, offa, 0, 0, CP_NT);
  }
  ++c.rc;
  XF_WAIT_VM_NF();
  if (c.rc > XF_NF) xf_publish(c.lds, c.w, c.rc - XF_NF);
  return true;
}

__device__ inline bool load_gemv(Loader& Ld, int op, int l) {
  const XArgs& a = *Ld.a;
  Ctx& c = *Ld.c;
  const PD p = phase_desc(a, op, l, c.xi);
  int first, stride, n;
  block_tiles(p, c, a.bpx, first, stride, n);
  if (n == 0) return true;
  const XLin& L = p.L;
  const rsrc_t rq = mkd(L.qw, (size_t)L.NT * L.GP * 1024);
  const rsrc_t rs = mkd(L.sb, (size_t)L.NT * L.GP * 32 * 4);
  for (int gs = 0; gs < n; gs += XF_TG) {
    const int tg = min(XF_TG, n - gs);
    for (int pi = c.w; pi < p.np; pi += XF_NCW) {
      const int gp = p.pk0 + pi;
      for (int ti = 0; ti < tg; ++ti) {
        const int t = global_tile(a, p, c.xi, first + stride * (gs + ti));
        const unsigned offa = (unsigned)(t * L.GP + gp) * 1024u;
        const unsigned offs = (unsigned)tile_sb_word(t, (c.lane >> 1) & 15, gp, c.lane & 1, L.GP) * 4u;
        if (!push_chunk(Ld, rq, offa, true, rs, offs)) return false;
      }
    }
  }
  return true;
}

__device__ inline bool load_att(Loader& Ld, int l) {
  const XArgs& a = *Ld.a;
  Ctx& c = *Ld.c;
  const XLayer& Ly = a.layers[l];
  const int* ri = rows_of(c.lds);
  const size_t kvb = (size_t)a.R * a.nkv * a.cap * a.d * 2;
  const rsrc_t rk = mkd(Ly.k, kvb), rv = mkd(Ly.v, kvb);
  for (int r = 0; r < a.R; ++r) {
    const int T = row_info(ri, r, RI_T), NV = row_info(ri, r, RI_NV), nch = row_info(ri, r, RI_NCH),
              ub = row_info(ri, r, RI_UB);
    for (int ch = 0; ch < nch; ++ch) {
      if ((ub + ch) % a.bpx != c.j) continue;
      const int s = 4 * ch + c.w;
      if (16 * s >= T + NV) continue;
      const size_t head = (size_t)r * a.nkv + c.xi;
      for (int k = 0; k < 4; ++k) {  // K rows 16 s + 4k .. + 3 (1 KiB contiguous)
        const unsigned off = (unsigned)(((head * a.cap) + 16 * s + 4 * k) * a.d * 2);
        if (!push_chunk(Ld, rk, off - 0u, false, rk, 0u)) return false;
      }
      for (int k = 0; k < 4; ++k) {  // V^T rows 32k .. 32k + 31, keys 16 s .. + 15 (two 16-byte halves a row)
        const int dd = 32 * k + (c.lane >> 1);
        const unsigned lane_off = (unsigned)((((head * a.d) + dd) * a.cap + 16 * s + 8 * (c.lane & 1)) * 2);
        // push_chunk adds 16 lane to the first load's offset: pass the per-lane offset minus that
        if (!push_chunk(Ld, rv, lane_off - 16u * (unsigned)c.lane, false, rv, 0u)) return false;
      }
    }
  }
  return true;
}

__device__ void loader_main(const XArgs& a, Ctx& c) {
  Loader Ld;
  Ld.a = &a;
  Ld.c = &c;
  Ld.ring = ring_of(a, c.lds, c.w);
  Ld.cons = 0;
  bool ok = true;
  for (int l = 0; ok && l < a.L; ++l) {
    ok = load_gemv(Ld, OP_Q, l) && load_att(Ld, l) && load_gemv(Ld, OP_O, l) && load_gemv(Ld, OP_U, l) &&
         load_gemv(Ld, OP_D, l);
  }
  if (ok && c.wh) ok = load_gemv(Ld, OP_HEAD, a.L);
  XF_WAIT_VM0();
  if (ok) xf_publish(c.lds, c.w, c.rc);
}

// ---------------------------------------------------------------------------------------
// compute waves: ring access
// ---------------------------------------------------------------------------------------
__device__ inline bool ring_wait(Ctx& c, int upto) {  // chunks [0, upto) landed
  const int* ld = ctl_of(c.lds) + C_LOADED + c.w;
  int it = 0;
  while (__hip_atomic_load(ld, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) < upto)
    if (spin(c.cx, it)) return false;
  MC_FENCE();
  return true;
}
__device__ inline void ring_release(Ctx& c, int upto) {
  MC_FENCE();
  __builtin_amdgcn_s_waitcnt(0xC07F);  // the slot reads are complete
  if (c.lane == 0)
    __hip_atomic_store(ctl_of(c.lds) + C_CONSUMED + c.w, upto, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}
__device__ inline const unsigned char* ring_slot(const XArgs& a, unsigned char* lds, int w, int chunk) {
  return ring_of(a, lds, w) + (size_t)(chunk % a.ring_slots) * XF_SLOT;
}

// ---------------------------------------------------------------------------------------
// RX: residual add of the eight partial sums (or the embedding), sums of squares
// ---------------------------------------------------------------------------------------
__device__ inline bool rx_phase(const XArgs& a, Ctx& c, int l, int kind) {
  const int tid = c.w * 64 + c.lane;
  const int M = c.M, H = a.H;
  const int cb = H / a.bpx, npair = cb / 2, items = M * npair;
  uint16_t* xprev = reinterpret_cast<uint16_t*>(c.lds + a.o_xprev);  // [MMAX][cb]
  float* red = reinterpret_cast<float*>(c.lds + a.o_red);
  const bool to_x1 = kind == RX_O;
  const unsigned tout = tagof(c.ep, l, to_x1 ? TG_X1 : TG_X);
  u64* outw = (to_x1 ? a.x1l : a.xl) + (size_t)c.xi * XF_MMAX * (H / 2);
  u64* outs = (to_x1 ? a.x1ss : a.xss) + (size_t)c.xi * a.bpx * XF_MMAX;
  const rsrc_t ro = mkd(outw, (size_t)XF_MMAX * (H / 2) * 8);
  const rsrc_t ros = mkd(outs, (size_t)a.bpx * XF_MMAX * 8);
  const u64* part = kind == RX_O ? a.opart : a.dpart;
  const unsigned tin = kind == RX_O ? tagof(c.ep, l, TG_O) : tagof(c.ep, l - 1, TG_D);
  const rsrc_t rp = mkd(part, (size_t)XF_XCD * XF_MMAX * H * 8);
  for (int it0 = tid; it0 < items; it0 += XF_NCW * 64) {
    const int m = it0 / npair, pp = it0 - m * npair;
    const int col = c.j * cb + 2 * pp;
    float v0, v1;
    if (kind == RX_EMBED) {
      int tok = a.slot_tok[m];
      if (tok < 0 || tok >= a.embed.N) tok = 0;
      const XLin& E = a.embed;
      const int t = tok >> 4, r = tok & 15;
      const int kw = col >> 3, g = kw >> 3, w8 = kw & 7, am = w8 >> 2, cc = w8 & 3, gp = g >> 1, gi = g & 1;
      const uint32_t word = E.qw[(((size_t)t * E.GP + gp) * 64 + cc * 16 + r) * 4 + gi * 2 + am];
      const uint32_t sbw = E.sb[tile_sb_word(t, r, gp, gi, E.GP)];
      const float sc = bf16_to_f32((uint16_t)(sbw & 0xFFFFu)), bi = bf16_to_f32((uint16_t)(sbw >> 16));
      // MLX element i of the word sits at 4(i/2) (even i) or 16 + 4(i/2) (odd i) of the tile word
      const int i0 = col & 7;  // even
      const float q0 = (float)((word >> (4 * (i0 >> 1))) & 0xFu);
      const float q1 = (float)((word >> (16 + 4 * (i0 >> 1))) & 0xFu);
      v0 = bfr(__builtin_fmaf(sc, q0, bi));
      v1 = bfr(__builtin_fmaf(sc, q1, bi));
    } else {
      u32x4 pv[XF_XCD];
      unsigned pend = (1u << XF_XCD) - 1u;
      int it = 0;
      while (true) {
#pragma unroll
        for (int x = 0; x < XF_XCD; ++x)
          if (pend >> x & 1u) pv[x] = bld16<CP_SC1>(rp, (unsigned)((x * XF_MMAX + m) * H + col) * 8u);
#pragma unroll
        for (int x = 0; x < XF_XCD; ++x)
          if ((pend >> x & 1u) && pv[x].y == tin && pv[x].w == tin) pend &= ~(1u << x);
        if (pend == 0u) break;
        if (spin(c.cx, it)) return false;
      }
      float s0 = 0.f, s1 = 0.f;
#pragma unroll
      for (int x = 0; x < XF_XCD; ++x) {
        s0 += __uint_as_float(pv[x].x);
        s1 += __uint_as_float(pv[x].z);
      }
      v0 = bfr(bf16_to_f32(xprev[m * cb + 2 * pp]) + s0);
      v1 = bfr(bf16_to_f32(xprev[m * cb + 2 * pp + 1]) + s1);
    }
    xprev[m * cb + 2 * pp] = f32_to_bf16(v0);
    xprev[m * cb + 2 * pp + 1] = f32_to_bf16(v1);
    bst8<CP_PLAIN>(ro, (unsigned)(m * (H / 2) + col / 2) * 8u, pack2(v0, v1), tout);
    red[it0] = v0 * v0 + v1 * v1;
  }
  if (!cw_barrier(c)) return false;
  if (tid < M) {
    float ss = 0.f;
    for (int pp = 0; pp < npair; ++pp) ss += red[tid * npair + pp];
    bst8<CP_PLAIN>(ros, (unsigned)(c.j * XF_MMAX + tid) * 8u, __float_as_uint(ss), tout);
  }
  return true;
}

// ---------------------------------------------------------------------------------------
// GEMV phases
// ---------------------------------------------------------------------------------------
struct XIn {
  const u64* src;      // token rows of this XCD's input
  int ldw;             // words per token row
  int ncol;            // columns staged (from column 0)
  unsigned tag;
  const uint16_t* nw;  // RMSNorm weights (NULL: no norm)
  const u64* ss;       // [bpx][MMAX] sums of squares (norm only)
  int kfull;           // the norm's width
};

constexpr int XQ = 3;  // 16-byte (4-column) input quads per thread, at most (ncol <= 3072)

// Stage the phase input as bf16 rows X[m][0 .. ncol) (RMS-normalised when in.nw).
__device__ inline bool stage_x(const XArgs& a, Ctx& c, const XIn& in) {
  const int tid = c.w * 64 + c.lane;
  const int M = c.M;
  uint16_t* X = reinterpret_cast<uint16_t*>(c.lds + a.o_x);
  const rsrc_t rx = mkd(in.src, (size_t)XF_MMAX * in.ldw * 8);
  // norm factors, computed redundantly by every compute wave: lanes take block partials
  float rn[XF_MMAX];
  if (in.nw) {
    const rsrc_t rs = mkd(in.ss, (size_t)a.bpx * XF_MMAX * 8);
    const int p = c.lane % a.bpx;
    u32x2 sv[XF_MMAX];
    unsigned pend = 0;
#pragma unroll
    for (int m = 0; m < XF_MMAX; ++m)
      if (m < M) pend |= 1u << m;
    int it = 0;
    while (true) {
#pragma unroll
      for (int m = 0; m < XF_MMAX; ++m)
        if (pend >> m & 1u) sv[m] = __builtin_amdgcn_raw_buffer_load_b64(rs, (unsigned)(p * XF_MMAX + m) * 8u, 0, CP_SC1);
#pragma unroll
      for (int m = 0; m < XF_MMAX; ++m)
        if ((pend >> m & 1u) && sv[m].y == in.tag) pend &= ~(1u << m);
      if (!__any(pend != 0u)) break;
      if (spin(c.cx, it)) return false;
    }
#pragma unroll
    for (int m = 0; m < XF_MMAX; ++m) {
      float s = m < M ? __uint_as_float(sv[m].x) : 0.f;
      // lanes 0 .. bpx - 1 hold one partial each (the others repeat them): butterfly over bpx
      for (int o = 1; o < a.bpx; o <<= 1) s += __shfl_xor(s, o);
      rn[m] = 1.0f / sqrtf(s / (float)in.kfull + a.eps);
    }
  }
  const int nq4 = in.ncol / 4;
  u32x4 v[XQ][XF_MMAX];
  unsigned pend = 0;
#pragma unroll
  for (int i = 0; i < XQ; ++i)
#pragma unroll
    for (int m = 0; m < XF_MMAX; ++m)
      if (tid + XF_CT * i < nq4 && m < M) pend |= 1u << (i * XF_MMAX + m);
  int it = 0;
  while (true) {
#pragma unroll
    for (int i = 0; i < XQ; ++i)
#pragma unroll
      for (int m = 0; m < XF_MMAX; ++m)
        if (pend >> (i * XF_MMAX + m) & 1u)
          v[i][m] = bld16<CP_SC1>(rx, (unsigned)(m * in.ldw + 2 * (tid + XF_CT * i)) * 8u);
#pragma unroll
    for (int i = 0; i < XQ; ++i)
#pragma unroll
      for (int m = 0; m < XF_MMAX; ++m)
        if ((pend >> (i * XF_MMAX + m) & 1u) && v[i][m].y == in.tag && v[i][m].w == in.tag) pend &= ~(1u << (i * XF_MMAX + m));
    if (!__any(pend != 0u)) break;
    if (spin(c.cx, it)) return false;
  }
  const rsrc_t rw = mkd(in.nw, (size_t)in.ncol * 2);
#pragma unroll
  for (int i = 0; i < XQ; ++i) {
    const int cq = tid + XF_CT * i;
    if (XF_CT * i >= nq4) break;  // uniform
    const bool live = cq < nq4;
    u32x2 wv = {0u, 0u};
    if (in.nw && live) wv = __builtin_amdgcn_raw_buffer_load_b64(rw, (unsigned)cq * 8u, 0, CP_PLAIN);
#pragma unroll
    for (int m = 0; m < XF_MMAX; ++m) {
      if (m < M && live) {
        uint32_t x0 = v[i][m].x, x1 = v[i][m].z;
        if (in.nw) {
          const float r = rn[m];
          x0 = pack2((lo_f(x0) * r) * lo_f(wv.x), (hi_f(x0) * r) * hi_f(wv.x));
          x1 = pack2((lo_f(x1) * r) * lo_f(wv.y), (hi_f(x1) * r) * hi_f(wv.y));
        }
        *reinterpret_cast<u32x2*>(X + m * a.xst + 4 * cq) = (u32x2){x0, x1};
      }
    }
  }
  return cw_barrier(c);
}

__device__ inline XIn gemv_input(const XArgs& a, const Ctx& c, int op, int l) {
  XIn in;
  const int g = a.nq / a.nkv;
  in.kfull = a.H;
  in.ss = nullptr;
  in.nw = nullptr;
  if (op == OP_Q || op == OP_HEAD) {
    in.src = a.xl + (size_t)c.xi * XF_MMAX * (a.H / 2);
    in.ldw = a.H / 2;
    in.ncol = a.H;
    in.tag = tagof(c.ep, op == OP_Q ? l : a.L, TG_X);
    in.nw = op == OP_Q ? a.layers[l].in_norm : a.final_norm;
    in.ss = a.xss + (size_t)c.xi * a.bpx * XF_MMAX;
  } else if (op == OP_U) {
    in.src = a.x1l + (size_t)c.xi * XF_MMAX * (a.H / 2);
    in.ldw = a.H / 2;
    in.ncol = a.H;
    in.tag = tagof(c.ep, l, TG_X1);
    in.nw = a.layers[l].post_norm;
    in.ss = a.x1ss + (size_t)c.xi * a.bpx * XF_MMAX;
  } else if (op == OP_O) {
    in.src = a.attl + (size_t)c.xi * XF_MMAX * (g * a.d / 2);
    in.ldw = g * a.d / 2;
    in.ncol = g * a.d;
    in.tag = tagof(c.ep, l, TG_A);
  } else {
    in.src = a.actl + (size_t)c.xi * XF_MMAX * a.act_w;
    in.ldw = a.act_w;
    in.ncol = 128 * (a.pdn[c.xi + 1] - a.pdn[c.xi]);
    in.tag = tagof(c.ep, l, TG_U);
  }
  return in;
}

// Epilogue of tile t (local lt) for lanes < 32: acc[v] = token 4c + v of weight row 16 t + r16.
__device__ inline void gemv_epilogue(const XArgs& a, const Ctx& c, const PD& p, int l, int lt, int t, f32x4 acc) {
  const int lane = c.lane, cq = lane >> 4, r16 = lane & 15;
  const int M = c.M, H = a.H, g = a.nq / a.nkv;
  const int n = t * 16 + r16;
  if (p.kind == OP_Q) {
    const int ldo = (g + 2) * a.d / 2;
    const rsrc_t ro = mkd(a.qkvl + (size_t)c.xi * XF_MMAX * ldo, (size_t)XF_MMAX * ldo * 8);
    const unsigned tag = tagof(c.ep, l, TG_Q);
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const float other = __shfl_xor(acc[v], 1);
      const int m = 4 * cq + v;
      if (lane < 32 && !(r16 & 1) && m < M) bst8<CP_PLAIN>(ro, (unsigned)(m * ldo + (lt * 16 + r16) / 2) * 8u, pack2(acc[v], other), tag);
    }
  } else if (p.kind == OP_U) {
    const rsrc_t ro = mkd(a.actl + (size_t)c.xi * XF_MMAX * a.act_w, (size_t)XF_MMAX * a.act_w * 8);
    const unsigned tag = tagof(c.ep, l, TG_U);
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      // rows interleave (gate_i, up_i): even lanes form act_i; lanes 4q pair act_2q, act_2q+1
      const float up = __shfl_xor(acc[v], 1);
      const float av = bfr(silu_f(acc[v]) * up);
      const float av2 = __shfl_xor(av, 2);
      const int m = 4 * cq + v;
      if (lane < 32 && (r16 & 3) == 0 && m < M)
        bst8<CP_PLAIN>(ro, (unsigned)(m * a.act_w + (8 * lt + r16 / 2) / 2) * 8u, pack2(av, av2), tag);
    }
  } else if (p.kind == OP_O || p.kind == OP_D) {
    u64* part = p.kind == OP_O ? a.opart : a.dpart;
    const rsrc_t ro = mkd(part, (size_t)XF_XCD * XF_MMAX * H * 8);
    const unsigned tag = tagof(c.ep, l, p.kind == OP_O ? TG_O : TG_D);
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int m = 4 * cq + v;
      if (lane < 32 && m < M && n < H) bst8<CP_SC1>(ro, (unsigned)((c.xi * XF_MMAX + m) * H + n) * 8u, __float_as_uint(acc[v]), tag);
    }
  } else {
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int m = 4 * cq + v;
      const bool live = lane < 32 && m < M && n < a.V;
      const uint16_t hv = f32_to_bf16(acc[v]);
      if (live) a.logits[(size_t)m * a.V + n] = hv;
      // tile argmax over 16 rows: key (value key << 16 | 15 - row), lowest row on ties
      unsigned key = live ? (bf16_order_key(hv) << 16) | (unsigned)(15 - r16) : 0u;
#pragma unroll
      for (int o = 1; o < 16; o <<= 1) key = max(key, (unsigned)__shfl_xor((int)key, o));
      if (lane < 32 && m < M && r16 == 0 && key)
        a.amax[(size_t)m * p.L.NT + t] =
            ((u64)(key >> 16) << 32) | (0xFFFFFFFFull - (unsigned)(t * 16 + 15 - (int)(key & 15u)));
    }
  }
}

// One group pair of TG tiles: the pair's activations (x0..x3, the 4 k-blocks of 32), the
// group sums of the activations (formed by the MFMA against ones: every column of
// C = X . 1 is the row sum), then the TG ring chunks: dequantise, 4 MFMAs, fold the affine
// scale/bias per group.  Branch-free, so the tiles' MFMA chains interleave.
template <int TG>
__device__ __forceinline__ void gemv_pair(const unsigned char* ring, int slot0, int RS, int lane, int r16,
                                          f32x4 (&acc)[XF_TG], bf16x8 x0, bf16x8 x1, bf16x8 x2, bf16x8 x3,
                                          uint32_t mask, uint32_t magic) {
  const bf16x8 ones = __builtin_bit_cast(bf16x8, (u32x4){0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u});
  f32x4 xs0 = {0.f, 0.f, 0.f, 0.f}, xs1 = {0.f, 0.f, 0.f, 0.f};
  xs0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(x0, ones, xs0, 0, 0, 0);
  xs1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(x2, ones, xs1, 0, 0, 0);
  xs0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(x1, ones, xs0, 0, 0, 0);
  xs1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(x3, ones, xs1, 0, 0, 0);
  u32x4 wq[TG];
  u32x2 sb[TG];
#pragma unroll
  for (int ti = 0; ti < TG; ++ti) {
    int sl = slot0 + ti;
    if (sl >= RS) sl -= RS;
    const unsigned char* slot = ring + sl * XF_SLOT;
    wq[ti] = *reinterpret_cast<const u32x4*>(slot + 16 * lane);
    sb[ti] = *reinterpret_cast<const u32x2*>(slot + 1024 + 8 * r16);
  }
#pragma unroll
  for (int ti = 0; ti < TG; ++ti) {
    f32x4 g0 = {0.f, 0.f, 0.f, 0.f}, g1 = {0.f, 0.f, 0.f, 0.f};
    g0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(x0, dequant_word(wq[ti].x, mask, magic), g0, 0, 0, 0);
    g1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(x2, dequant_word(wq[ti].z, mask, magic), g1, 0, 0, 0);
    g0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(x1, dequant_word(wq[ti].y, mask, magic), g0, 0, 0, 0);
    g1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(x3, dequant_word(wq[ti].w, mask, magic), g1, 0, 0, 0);
    const float s0 = DQ_STEP * __uint_as_float(sb[ti].x << 16), b0 = __uint_as_float(sb[ti].x & 0xFFFF0000u) - s0;
    const float s1 = DQ_STEP * __uint_as_float(sb[ti].y << 16), b1 = __uint_as_float(sb[ti].y & 0xFFFF0000u) - s1;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      float t0 = __builtin_fmaf(s0, g0[v], acc[ti][v]);
      t0 = __builtin_fmaf(b0, xs0[v], t0);
      t0 = __builtin_fmaf(s1, g1[v], t0);
      acc[ti][v] = __builtin_fmaf(b1, xs1[v], t0);
    }
  }
}

__device__ inline bool gemv_phase(const XArgs& a, Ctx& c, int op, int l) {
  const PD p = phase_desc(a, op, l, c.xi);
  int first, stride, n;
  block_tiles(p, c, a.bpx, first, stride, n);
  if (n == 0) return true;
  if (!stage_x(a, c, gemv_input(a, c, op, l))) return false;
  const int lane = c.lane, cq = lane >> 4, r16 = lane & 15;
  const int row = min(r16, c.M - 1);
  const uint16_t* X = reinterpret_cast<const uint16_t*>(c.lds + a.o_x) + row * a.xst + 8 * cq;
  f32x4* exch = reinterpret_cast<f32x4*>(c.lds + a.o_exch);
  const unsigned char* ring = ring_of(a, c.lds, c.w);
  const int RS = a.ring_slots;
  int slot = c.rc % RS;  // ring slot of the next chunk
  const uint32_t mask = DQ_MASK;
  uint32_t magic;
  MC_TO_VGPR(magic, DQ_MAGIC);
  for (int gs = 0; gs < n; gs += XF_TG) {
    const int tg = min(XF_TG, n - gs);
    f32x4 acc[XF_TG];
#pragma unroll
    for (int ti = 0; ti < XF_TG; ++ti) acc[ti] = (f32x4){0.f, 0.f, 0.f, 0.f};
    for (int pi = c.w; pi < p.np; pi += XF_NCW) {
      const bf16x8 x0 = *reinterpret_cast<const bf16x8*>(X + pi * 128);
      const bf16x8 x1 = *reinterpret_cast<const bf16x8*>(X + pi * 128 + 32);
      const bf16x8 x2 = *reinterpret_cast<const bf16x8*>(X + pi * 128 + 64);
      const bf16x8 x3 = *reinterpret_cast<const bf16x8*>(X + pi * 128 + 96);
      if (!ring_wait(c, c.rc + tg)) return false;
      switch (tg) {
        case 5: gemv_pair<5>(ring, slot, RS, lane, r16, acc, x0, x1, x2, x3, mask, magic); break;
        case 4: gemv_pair<4>(ring, slot, RS, lane, r16, acc, x0, x1, x2, x3, mask, magic); break;
        case 3: gemv_pair<3>(ring, slot, RS, lane, r16, acc, x0, x1, x2, x3, mask, magic); break;
        case 2: gemv_pair<2>(ring, slot, RS, lane, r16, acc, x0, x1, x2, x3, mask, magic); break;
        default: gemv_pair<1>(ring, slot, RS, lane, r16, acc, x0, x1, x2, x3, mask, magic); break;
      }
      c.rc += tg;
      slot += tg;
      if (slot >= RS) slot -= RS;
      ring_release(c, c.rc);
    }
    // exchange the waves' partials (tokens 0..7 live in lanes 0..31)
    if (lane < 32) {
#pragma unroll
      for (int ti = 0; ti < XF_TG; ++ti)
        if (ti < tg) exch[(ti * XF_NCW + c.w) * 32 + lane] = acc[ti];
    }
    if (!cw_barrier(c)) return false;
    for (int ti = c.w; ti < tg; ti += XF_NCW) {
      const int ln = lane & 31;
      f32x4 s = exch[(ti * XF_NCW + 0) * 32 + ln];
#pragma unroll
      for (int w2 = 1; w2 < XF_NCW; ++w2) s += exch[(ti * XF_NCW + w2) * 32 + ln];
      const int lt = first + stride * (gs + ti);
      gemv_epilogue(a, c, p, l, lt, global_tile(a, p, c.xi, lt), s);
    }
    // the next group of this phase rewrites the exchange area; the next phase's first
    // write to it follows that phase's staging barrier
    if (gs + XF_TG < n && !cw_barrier(c)) return false;
  }
  return true;
}

// ---------------------------------------------------------------------------------------
// attention
// ---------------------------------------------------------------------------------------
// staging area (aliases X): raw [48][128] bf16, q [4][8][XF_QS], kn [8][XF_QS], vn [8][128],
// rope cos/sin [8][64] f32, q/k norm weights [2][128]
constexpr int A_RAW = 0;
constexpr int A_Q = A_RAW + 48 * 128 * 2;
constexpr int A_KN = A_Q + 4 * 8 * XF_QS * 2;
constexpr int A_VN = A_KN + 8 * XF_QS * 2;
constexpr int A_CS = A_VN + 8 * 128 * 2;
constexpr int A_SN = A_CS + 8 * 64 * 4;
constexpr int A_NW = A_SN + 8 * 64 * 4;
constexpr int A_END = A_NW + 2 * 128 * 2;

__device__ inline bool att_unit(const XArgs& a, Ctx& c, int l, int r, int ch) {
  const int tid = c.w * 64 + c.lane, lane = c.lane, w = c.w;
  const int* ri = rows_of(c.lds);
  const int T = row_info(ri, r, RI_T), NV = row_info(ri, r, RI_NV), S0 = row_info(ri, r, RI_S0);
  const int g = a.nq / a.nkv, d = a.d;
  const XLayer& Ly = a.layers[l];
  unsigned char* st = c.lds + a.o_x;
  uint16_t* raw = reinterpret_cast<uint16_t*>(st + A_RAW);
  uint16_t* qs = reinterpret_cast<uint16_t*>(st + A_Q);
  uint16_t* kn = reinterpret_cast<uint16_t*>(st + A_KN);
  uint16_t* vn = reinterpret_cast<uint16_t*>(st + A_VN);
  float* cs = reinterpret_cast<float*>(st + A_CS);
  float* sn = reinterpret_cast<float*>(st + A_SN);
  uint16_t* nwl = reinterpret_cast<uint16_t*>(st + A_NW);
  int* kvb = ctl_of(c.lds) + C_KVB;
  // ---- raw q (g heads), k, v rows of the NV new tokens: 32 quads (16 bytes = 2 words) a row ----
  {
    const int ldq = (g + 2) * d / 2;
    const rsrc_t rq = mkd(a.qkvl + (size_t)c.xi * XF_MMAX * ldq, (size_t)XF_MMAX * ldq * 8);
    const unsigned tq = tagof(c.ep, l, TG_Q);
    const int nrow = (g + 2) * NV, np = nrow * 32;
    constexpr int APP = (48 * 32 + XF_CT - 1) / XF_CT;
    u32x4 v[APP];
    unsigned pend = 0;
#pragma unroll
    for (int q = 0; q < APP; ++q)
      if (tid + XF_CT * q < np) pend |= 1u << q;
    int it = 0;
    while (true) {
#pragma unroll
      for (int q = 0; q < APP; ++q)
        if (pend >> q & 1u) {
          const int p = tid + XF_CT * q, rr = p >> 5, pw = p & 31;
          const int hs = rr / NV, jj = rr - hs * NV;
          v[q] = bld16<CP_SC1>(rq, (unsigned)((S0 + jj) * ldq + hs * (d / 2) + 2 * pw) * 8u);
        }
#pragma unroll
      for (int q = 0; q < APP; ++q)
        if ((pend >> q & 1u) && v[q].y == tq && v[q].w == tq) pend &= ~(1u << q);
      if (!__any(pend != 0u)) break;
      if (spin(c.cx, it)) return false;
    }
#pragma unroll
    for (int q = 0; q < APP; ++q) {
      const int p = tid + XF_CT * q;
      if (p < np) *reinterpret_cast<u32x2*>(raw + (p >> 5) * 128 + 4 * (p & 31)) = (u32x2){v[q].x, v[q].z};
    }
    for (int i2 = tid; i2 < NV * 64; i2 += XF_CT) {
      const int jj = i2 >> 6, e = i2 & 63;
      cs[i2] = a.rope_cos[(size_t)(T + jj) * 64 + e];
      sn[i2] = a.rope_sin[(size_t)(T + jj) * 64 + e];
    }
    for (int i2 = tid; i2 < 256; i2 += XF_CT) {
      const uint16_t* src = i2 < 128 ? Ly.q_norm : Ly.k_norm;
      nwl[i2] = src ? src[i2 & 127] : (uint16_t)0;
    }
  }
  if (!cw_barrier(c)) return false;
  // ---- q / k norm + RoPE: rows rr = w + 4 k of a wave, lane e rotates the pair (e, e + 64);
  // the rows' sums of squares are reduced together (independent shuffle chains) ----
  {
    const int nrow = (g + 2) * NV;
    constexpr int RPW = (6 * XF_MMAX + XF_NCW - 1) / XF_NCW;  // rows per wave, at most
    float x1[RPW], x2[RPW], ss[RPW];
#pragma unroll
    for (int k = 0; k < RPW; ++k) {
      const int rr = min(w + XF_NCW * k, nrow - 1);
      x1[k] = bf16_to_f32(raw[rr * 128 + lane]);
      x2[k] = bf16_to_f32(raw[rr * 128 + lane + 64]);
      ss[k] = x1[k] * x1[k] + x2[k] * x2[k];
    }
    if (Ly.q_norm) {
#pragma unroll
      for (int o = 32; o > 0; o >>= 1)
#pragma unroll
        for (int k = 0; k < RPW; ++k) ss[k] += __shfl_xor(ss[k], o);
    }
#pragma unroll
    for (int k = 0; k < RPW; ++k) {
      const int rr = w + XF_NCW * k;
      if (rr >= nrow) break;
      const int hs = rr / NV, jj = rr - hs * NV;
      float y1 = x1[k], y2 = x2[k];
      if (hs > g) {  // v
        vn[jj * 128 + lane] = f32_to_bf16(y1);
        vn[jj * 128 + lane + 64] = f32_to_bf16(y2);
        continue;
      }
      const bool isq = hs < g;
      if (Ly.q_norm) {
        const uint16_t* nwp = nwl + (isq ? 0 : 128);
        const float rr2 = 1.0f / sqrtf(ss[k] / (float)d + a.eps);
        y1 = bfr((y1 * rr2) * bf16_to_f32(nwp[lane]));
        y2 = bfr((y2 * rr2) * bf16_to_f32(nwp[lane + 64]));
      }
      const float c0 = cs[jj * 64 + lane], s0 = sn[jj * 64 + lane];
      const uint16_t o1 = f32_to_bf16(y1 * c0 - y2 * s0);
      const uint16_t o2 = f32_to_bf16(y1 * s0 + y2 * c0);
      uint16_t* dst = isq ? qs + (hs * 8 + jj) * XF_QS : kn + jj * XF_QS;
      dst[lane] = o1;
      dst[lane + 64] = o2;
    }
  }
  if (!cw_barrier(c)) return false;
  // ---- this wave's 16-key sub-block: patch in the new keys, append them to the cache ----
  const int s = 4 * ch + w;
  const bool valid = w < XF_G && 16 * s < T + NV;
  if (valid) {
    if (!ring_wait(c, c.rc + 8)) return false;
    const int lo = max(16 * s, T), hi = min(16 * s + 16, T + NV);
    const size_t head = (size_t)r * a.nkv + c.xi;
    for (int pos = lo; pos < hi; ++pos) {
      const int jj = pos - T, kk = pos - 16 * s;
      unsigned char* ks = const_cast<unsigned char*>(ring_slot(a, c.lds, w, c.rc + (kk >> 2))) + (kk & 3) * 256;
      const uint32_t kw = *reinterpret_cast<const uint32_t*>(kn + jj * XF_QS + 2 * lane);
      *reinterpret_cast<uint32_t*>(ks + 4 * lane) = kw;
      *reinterpret_cast<uint32_t*>(Ly.k + ((head * a.cap + pos) * d) + 2 * lane) = kw;
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        const int dd = lane + 64 * hh;
        const uint16_t vv = vn[jj * 128 + dd];
        uint16_t* vs = reinterpret_cast<uint16_t*>(const_cast<unsigned char*>(ring_slot(a, c.lds, w, c.rc + 4 + (dd >> 5))));
        vs[(dd & 31) * 16 + kk] = vv;
        Ly.v[(head * d + dd) * a.cap + pos] = vv;
      }
    }
  }
  if (lane == 0 && w < XF_G) kvb[w] = valid ? c.rc : -1;
  if (!cw_barrier(c)) return false;
  // ---- GQA head gq = w (waves 0..3) against the chunk's 64 keys ----
  if (w < XF_G) {
    const int gq = w, n = lane & 15, c4 = lane >> 4;
    const int qrow = min(n, NV - 1);
    bf16x8 qv[4];
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) qv[kk] = *reinterpret_cast<const bf16x8*>(qs + (gq * 8 + qrow) * XF_QS + 32 * kk + 8 * c4);
    f32x4 S[4];
    int base[4];
#pragma unroll
    for (int sb = 0; sb < 4; ++sb) {
      base[sb] = kvb[sb];
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
      if (base[sb] >= 0) {
        const unsigned char* kslot = ring_slot(a, c.lds, sb, base[sb] + (n >> 2)) + (n & 3) * 256;
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) {
          const bf16x8 kv = *reinterpret_cast<const bf16x8*>(kslot + (32 * kk + 8 * c4) * 2);
          acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kv, qv[kk], acc, 0, 0, 0);
        }
      }
      S[sb] = acc;  // lane: S^T[key 16 (4 ch + sb) + 4 c4 + v][query n]
    }
    float mx = -INFINITY;
#pragma unroll
    for (int sb = 0; sb < 4; ++sb)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int pos = 16 * (4 * ch + sb) + 4 * c4 + v;
        const bool ok = base[sb] >= 0 && n < NV && pos <= T + n && pos < T + NV;
        const float sv = ok ? S[sb][v] * a.scale : -INFINITY;
        S[sb][v] = sv;
        mx = fmaxf(mx, sv);
      }
    mx = fmaxf(mx, __shfl_xor(mx, 16));
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    float lsum = 0.f;
    s16x4 ph[4], pl[4];
#pragma unroll
    for (int sb = 0; sb < 4; ++sb) {
      uint16_t hv[4], lv[4];
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const float sv = S[sb][v];
        const float pv = (sv == -INFINITY) ? 0.f : __expf(sv - mx);
        lsum += pv;
        hv[v] = f32_to_bf16(pv);
        lv[v] = f32_to_bf16(pv - bf16_to_f32(hv[v]));
      }
      ph[sb] = (s16x4){(short)hv[0], (short)hv[1], (short)hv[2], (short)hv[3]};
      pl[sb] = (s16x4){(short)lv[0], (short)lv[1], (short)lv[2], (short)lv[3]};
    }
    lsum += __shfl_xor(lsum, 16);
    lsum += __shfl_xor(lsum, 32);
    f32x4 o[8];
#pragma unroll
    for (int db = 0; db < 8; ++db) o[db] = (f32x4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int sb = 0; sb < 4; ++sb) {
      if (base[sb] < 0) continue;
#pragma unroll
      for (int db = 0; db < 8; ++db) {
        const int dd = 16 * db + n;
        const unsigned char* vslot = ring_slot(a, c.lds, sb, base[sb] + 4 + (dd >> 5));
        const s16x4 vv = *reinterpret_cast<const s16x4*>(vslot + ((dd & 31) * 16 + 4 * c4) * 2);
        o[db] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(vv, ph[sb], o[db], 0, 0, 0);
        o[db] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(vv, pl[sb], o[db], 0, 0, 0);
      }
    }
    // record (o unnormalised, max, sum) of query n of head gq: lane holds o[16 db + 4 c4 + v]
    const size_t rec0 = ((((size_t)c.xi * a.R + r) * a.nch_cap + ch) * 32 + gq * 8 + n) * XF_REC;
    const rsrc_t rr = mkd(a.rec, (size_t)XF_XCD * a.R * a.nch_cap * 32 * XF_REC * 8);
    const unsigned tr = tagof(c.ep, l, TG_R);
    if (n < NV) {
#pragma unroll
      for (int db = 0; db < 8; ++db) {
        const unsigned off = (unsigned)(rec0 + 16 * db + 4 * c4) * 8u;
        bst16<CP_PLAIN>(rr, off, (u32x4){__float_as_uint(o[db][0]), tr, __float_as_uint(o[db][1]), tr});
        bst16<CP_PLAIN>(rr, off + 16u, (u32x4){__float_as_uint(o[db][2]), tr, __float_as_uint(o[db][3]), tr});
      }
      if (c4 == 0) bst16<CP_PLAIN>(rr, (unsigned)(rec0 + 128) * 8u, (u32x4){__float_as_uint(mx), tr, __float_as_uint(lsum), tr});
    }
  }
  if (!cw_barrier(c)) return false;
  if (valid) {
    c.rc += 8;
    ring_release(c, c.rc);
  }
  return true;
}

__device__ inline bool att_phase(const XArgs& a, Ctx& c, int l) {
  const int* ri = rows_of(c.lds);
  for (int r = 0; r < a.R; ++r) {
    const int nch = row_info(ri, r, RI_NCH), ub = row_info(ri, r, RI_UB);
    for (int ch = 0; ch < nch; ++ch) {
      if ((ub + ch) % a.bpx != c.j) continue;
      if (!att_unit(a, c, l, r, ch)) return false;
    }
  }
  return true;
}

// merge the chunk records of (slot, q head) -> att (bf16 pairs).  A block's unit is shared
// by its 4 waves (wave w takes chunks w, w + 4, ...); the 4 partials meet in LDS and wave 0
// merges them in wave order.  Every slot of the launch gets its words (zeros for slots
// outside the rows' valid tokens): the o projection stages all M slots.
__device__ inline bool comb_phase(const XArgs& a, Ctx& c, int l) {
  const int* ri = rows_of(c.lds);
  const int lane = c.lane, w = c.w, g = a.nq / a.nkv;
  const unsigned tr = tagof(c.ep, l, TG_R), ta = tagof(c.ep, l, TG_A);
  const rsrc_t rr = mkd(a.rec, (size_t)XF_XCD * a.R * a.nch_cap * 32 * XF_REC * 8);
  const int ldo = g * a.d / 2;
  const rsrc_t ro = mkd(a.attl + (size_t)c.xi * XF_MMAX * ldo, (size_t)XF_MMAX * ldo * 8);
  f32x4* cm = reinterpret_cast<f32x4*>(c.lds + a.o_cm);  // [4 waves][64 lanes] (max, sum, o0, o1)
  constexpr int CPW = 9;  // chunks a wave merges per pass
  for (int u = c.j; u < c.M * g; u += a.bpx) {
    const int s = u / g, gq = u - s * g;
    const int r = a.slot_row[s];
    int jj = -1, nch = 0;
    if (r >= 0 && r < a.R) {
      jj = s - row_info(ri, r, RI_S0);
      nch = row_info(ri, r, RI_NCH);
      if (jj < 0 || jj >= row_info(ri, r, RI_NV)) jj = -1;
    }
    float mx = -INFINITY, ls = 0.f, o0 = 0.f, o1 = 0.f;
    if (jj >= 0) {
      for (int p0 = w; p0 < nch; p0 += XF_NCW * CPW) {
        u32x4 ov[CPW], mv[CPW];
        unsigned pend = 0;
#pragma unroll
        for (int k2 = 0; k2 < CPW; ++k2)
          if (p0 + XF_NCW * k2 < nch) pend |= 1u << k2;
        const unsigned all = pend;
        int it = 0;
        while (true) {
#pragma unroll
          for (int k2 = 0; k2 < CPW; ++k2)
            if (pend >> k2 & 1u) {
              const size_t rec0 =
                  ((((size_t)c.xi * a.R + r) * a.nch_cap + p0 + XF_NCW * k2) * 32 + gq * 8 + jj) * XF_REC;
              ov[k2] = bld16<CP_SC1>(rr, (unsigned)(rec0 + 2 * lane) * 8u);
              mv[k2] = bld16<CP_SC1>(rr, (unsigned)(rec0 + 128) * 8u);
            }
#pragma unroll
          for (int k2 = 0; k2 < CPW; ++k2)
            if ((pend >> k2 & 1u) && ov[k2].y == tr && ov[k2].w == tr && mv[k2].y == tr && mv[k2].w == tr)
              pend &= ~(1u << k2);
          if (!__any(pend != 0u)) break;
          if (spin(c.cx, it)) return false;
        }
#pragma unroll
        for (int k2 = 0; k2 < CPW; ++k2) {
          if (!(all >> k2 & 1u)) break;
          const float mk_ = __uint_as_float(mv[k2].x), lk = __uint_as_float(mv[k2].z);
          const float nm = fmaxf(mx, mk_);
          const float e_old = (mx == -INFINITY) ? 0.f : __expf(mx - nm);
          const float e_new = (mk_ == -INFINITY) ? 0.f : __expf(mk_ - nm);
          ls = ls * e_old + lk * e_new;
          o0 = o0 * e_old + __uint_as_float(ov[k2].x) * e_new;
          o1 = o1 * e_old + __uint_as_float(ov[k2].z) * e_new;
          mx = nm;
        }
      }
    }
    cm[w * 64 + lane] = (f32x4){mx, ls, o0, o1};
    if (!cw_barrier(c)) return false;
    if (w == 0) {
      float M2 = -INFINITY, L2 = 0.f, O0 = 0.f, O1 = 0.f;
#pragma unroll
      for (int w2 = 0; w2 < XF_NCW; ++w2) {
        const f32x4 q = cm[w2 * 64 + lane];
        const float nm = fmaxf(M2, q[0]);
        const float e_old = (M2 == -INFINITY) ? 0.f : __expf(M2 - nm);
        const float e_new = (q[0] == -INFINITY) ? 0.f : __expf(q[0] - nm);
        L2 = L2 * e_old + q[1] * e_new;
        O0 = O0 * e_old + q[2] * e_new;
        O1 = O1 * e_old + q[3] * e_new;
        M2 = nm;
      }
      const float inv = L2 > 0.f ? 1.0f / L2 : 0.f;
      bst8<CP_PLAIN>(ro, (unsigned)(s * ldo + gq * (a.d / 2) + lane) * 8u, pack2(O0 * inv, O1 * inv), ta);
    }
    if (u + a.bpx < c.M * g && !cw_barrier(c)) return false;  // cm is rewritten by the next unit
  }
  return true;
}

__device__ void compute_main(const XArgs& a, Ctx& c) {
  for (int l = 0; l < a.L; ++l) {
    if (!rx_phase(a, c, l, l == 0 ? RX_EMBED : RX_DOWN)) return;
    if (!gemv_phase(a, c, OP_Q, l)) return;
    if (!att_phase(a, c, l)) return;
    if (!comb_phase(a, c, l)) return;
    if (!gemv_phase(a, c, OP_O, l)) return;
    if (!rx_phase(a, c, l, RX_O)) return;
    if (!gemv_phase(a, c, OP_U, l)) return;
    if (!gemv_phase(a, c, OP_D, l)) return;
  }
  if (!rx_phase(a, c, a.L, RX_DOWN)) return;
  if (c.wh) gemv_phase(a, c, OP_HEAD, a.L);
}

}  // namespace

// ---------------------------------------------------------------------------------------
// the kernel
// ---------------------------------------------------------------------------------------
__global__ void __launch_bounds__(XF_THREADS) xfwd_kernel(const XArgs* __restrict__ ap, int M, int with_head) {
  MC_DYN_LDS(lds);
  const XArgs& a = *ap;
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
  int* ctl = ctl_of(lds);
  if (tid == 0) {
    unsigned xi;
#ifdef MC_EMULATE
    xi = blockIdx.x % XF_XCD;
#else
    XF_XCC_ID(xi);
#endif
    unsigned jj = 0xFFFFFFFFu;
    if (xi < (unsigned)XF_XCD) jj = __hip_atomic_fetch_add(a.xcd_ctr + xi, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (xi >= (unsigned)XF_XCD || jj >= (unsigned)a.bpx) {
      __hip_atomic_fetch_or(a.err, 4u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      xi = 0xFFFFu;
    }
    for (int k = 0; k < C_ROWS; ++k) ctl[k] = 0;
    ctl[C_XI] = (int)xi;
    ctl[C_J] = (int)jj;
    int ub = 0;
    for (int r = 0; r < a.R; ++r) {
      const int T = a.qbase[r], NV = a.n_valid[r];
      int* ri = ctl + C_ROWS + r * 8;
      ri[RI_T] = T;
      ri[RI_NV] = NV;
      ri[RI_S0] = a.row_slot0[r];
      ri[RI_NCH] = att_chunks(T, NV);
      ri[RI_UB] = ub;
      ub += ri[RI_NCH];
    }
  }
  __syncthreads();
  // values read back from memory are wave-uniform: say so (readfirstlane), so that every
  // address derived from them stays scalar (a buffer descriptor the compiler must assume to
  // vary across lanes turns each buffer instruction into a loop over lanes)
  Ctx c;
  c.lds = lds;
  c.xi = XF_UNIFORM(ctl[C_XI]);
  c.j = XF_UNIFORM(ctl[C_J]);
  if (c.xi < 0 || c.xi >= XF_XCD) return;
  c.gb = c.xi * a.bpx + c.j;
  c.G = XF_XCD * a.bpx;
  c.ep = (unsigned)XF_UNIFORM((int)*a.epoch);
  c.cx.t0 = wall_clock64();
  c.cx.err = a.err;
  c.w = w < XF_NCW ? w : w - XF_NCW;
  c.lane = lane;
  c.rc = 0;
  c.nb = 0;
  c.M = M;
  c.wh = with_head;
  if (w >= XF_NCW) loader_main(a, c);
  else compute_main(a, c);
}

__global__ void xfwd_epoch_kernel(unsigned* epoch, unsigned* xcd_ctr) {
  if (blockIdx.x == 0) {
    if (threadIdx.x == 0) *epoch = *epoch + 1u;
    if (threadIdx.x < XF_XCD) xcd_ctr[threadIdx.x] = 0u;
  }
}

// ---------------------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------------------
bool xfwd_supported(const mc_model_config& c, int R, int cap, int cus, const char** why) {
  const char* r = nullptr;
  const int g = c.n_kv_heads > 0 ? c.n_q_heads / c.n_kv_heads : 0;
  if (cus % XF_XCD || cus < XF_XCD) r = "CU count is not a multiple of the XCD count";
  else if (c.n_experts > 0) r = "mixture of experts";
  else if (c.n_kv_heads != XF_XCD) r = "kv heads != XCD count";
  else if (g != XF_G || g * c.n_kv_heads != c.n_q_heads) r = "GQA group != 4";
  else if (c.head_dim != 128) r = "head_dim != 128";
  else if (c.hidden % 256 || c.hidden > XF_CT * 4 * XQ || (c.hidden / (cus / XF_XCD)) % 2) r = "hidden size";
  else if (c.intermediate % 128) r = "intermediate not a multiple of 128";
  else if (c.n_layers < 1 || c.n_layers > 62) r = "layer count";
  else if (c.n_experts > 0) r = "mixture of experts";
  else if (R < 1 || R > XF_MMAX) r = "more than 8 rows";
  else if (cap % 64) r = "cache stride";
  if (why) *why = r;
  return r == nullptr;
}

bool xfwd_plan(XArgs& a) {
  const int H = a.H, g = a.nq / a.nkv;
  const int GPd = a.I / 128;
  int mx = 0;
  for (int x = 0; x <= XF_XCD; ++x) a.pdn[x] = x * GPd / XF_XCD;
  for (int x = 0; x < XF_XCD; ++x) mx = std::max(mx, a.pdn[x + 1] - a.pdn[x]);
  a.act_w = mx * 64;
  const int kst = std::max(std::max(H, g * a.d), 128 * mx);
  if (kst > XF_CT * 4 * XQ) return false;  // staging: XQ quads of 4 columns per compute thread
  const int cb = H / a.bpx;
  auto al = [](int x) { return (x + 15) & ~15; };
  int o = CTL_BYTES;
  o = al(o);
  a.o_xprev = o; o += al(XF_MMAX * cb * 2);
  a.o_red = o; o += al(XF_MMAX * (cb / 2) * 4);
  a.o_exch = o; o += XF_TG * XF_NCW * 32 * 16;
  a.o_cm = o; o += XF_NCW * 64 * 16;
  a.o_xsum = o;
  a.xst = kst + 8;
  a.o_x = o; o += al(std::max(XF_MMAX * a.xst * 2, A_END));
  a.o_ring = o;
  const int limit = 160 * 1024;
  a.ring_slots = (limit - o) / (XF_NCW * XF_SLOT);
  if (a.ring_slots < XF_NF + 2) return false;  // and at least the 8 chunks of an attention sub-block
  a.lds_bytes = o + a.ring_slots * XF_NCW * XF_SLOT;
  return true;
}

int launch_xfwd(const XArgs* dev_args, int lds_bytes, int M, int with_head, int grid, hipStream_t st) {
  static bool attr = false;
  if (!attr) {
    MC_HIP(hipFuncSetAttribute((const void*)xfwd_kernel, hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024));
    attr = true;
  }
  hipLaunchKernelGGL(xfwd_kernel, dim3(grid), dim3(XF_THREADS), lds_bytes, st, dev_args, M, with_head);
  MC_HIP(hipGetLastError());
  return MC_OK;
}

int launch_xfwd_epoch(unsigned* epoch, unsigned* xcd_ctr, hipStream_t st) {
  hipLaunchKernelGGL(xfwd_epoch_kernel, dim3(1), dim3(64), 0, st, epoch, xcd_ctr);
  MC_HIP(hipGetLastError());
  return MC_OK;
}

}  // namespace mc
