// Host emulation of the HIP device facilities and runtime calls the library uses, so that
// mlxcat_amd/csrc/*.hip compile as host C++ and run on the CPU (tests/emu).  Test
// infrastructure only.
//
// Every GPU lane runs as its own coroutine (emu_runtime.cpp).  Wave-wide operations
// (shuffles, votes, the MFMA) are collectives: the 64 lanes of a wave deposit their
// operands, the last to arrive computes, all continue.  Buffer loads / stores check their
// range like the hardware (out-of-range loads read 0, stores are dropped) and every
// out-of-range access is counted.  Runtime calls are synchronous: a kernel runs to
// completion inside hipLaunchKernelGGL.
#pragma once
#include <math.h>
#include <stddef.h>
#include <stdint.h>
#include <string.h>

#include <algorithm>
#include <cmath>
#include <functional>

#define MC_EMULATE 1
#define __host__
#define __device__
#define __global__
#define __forceinline__ inline
#define __launch_bounds__(...)
#define __align__(x) __attribute__((aligned(x)))
#define __shared__ static  // blocks of an ordinary kernel run one group at a time (see run_kernel)

// ---------------------------------------------------------------------------------------
// runtime types
// ---------------------------------------------------------------------------------------
typedef int hipError_t;
enum {
  hipSuccess = 0,
  hipErrorInvalidValue = 1,
  hipErrorOutOfMemory = 2,
  hipErrorEmu = 999,
};
typedef struct emu_stream* hipStream_t;
typedef struct emu_event* hipEvent_t;
typedef struct emu_graph* hipGraph_t;
typedef struct emu_graph* hipGraphExec_t;
enum hipMemcpyKind { hipMemcpyHostToDevice, hipMemcpyDeviceToHost, hipMemcpyDeviceToDevice, hipMemcpyHostToHost };
enum hipFuncAttribute { hipFuncAttributeMaxDynamicSharedMemorySize };
enum hipDeviceAttribute_t { hipDeviceAttributeMultiprocessorCount };
enum hipStreamCaptureMode { hipStreamCaptureModeThreadLocal };
#define hipStreamNonBlocking 1u
#define hipHostMallocDefault 0u
struct float2 {
  float x, y;
};
inline float2 make_float2(float a, float b) { return float2{a, b}; }
struct uint2 {
  unsigned x, y;
};
struct dim3 {
  unsigned x, y, z;
  dim3(unsigned a = 1, unsigned b = 1, unsigned c = 1) : x(a), y(b), z(c) {}
};

hipError_t hipMalloc(void** p, size_t n);
hipError_t hipFree(void* p);
hipError_t hipMemset(void* p, int v, size_t n);
hipError_t hipMemcpy(void* d, const void* s, size_t n, hipMemcpyKind k);
hipError_t hipMemcpyAsync(void* d, const void* s, size_t n, hipMemcpyKind k, hipStream_t st);
hipError_t hipMemcpy2D(void* d, size_t dp, const void* s, size_t sp, size_t w, size_t h, hipMemcpyKind k);
hipError_t hipMemcpy2DAsync(void* d, size_t dp, const void* s, size_t sp, size_t w, size_t h, hipMemcpyKind k,
                             hipStream_t st);
hipError_t hipHostMalloc(void** p, size_t n, unsigned flags);
hipError_t hipHostFree(void* p);
hipError_t hipSetDevice(int d);
hipError_t hipGetDevice(int* d);
hipError_t hipGetDeviceCount(int* n);
hipError_t hipDeviceGetAttribute(int* v, hipDeviceAttribute_t a, int d);
hipError_t hipStreamCreateWithFlags(hipStream_t* s, unsigned f);
hipError_t hipStreamDestroy(hipStream_t s);
hipError_t hipStreamSynchronize(hipStream_t s);
// a __device__ array is host memory here: its address is the symbol's
#define HIP_SYMBOL(x) (&(x))
inline hipError_t hipGetSymbolAddress(void** p, const void* sym) {
  *p = const_cast<void*>(sym);
  return hipSuccess;
}
hipError_t hipGetLastError();
const char* hipGetErrorString(hipError_t e);
hipError_t hipFuncSetAttribute(const void* f, hipFuncAttribute a, int v);
hipError_t hipOccupancyMaxActiveBlocksPerMultiprocessor(int* n, const void* f, int threads, size_t lds);
hipError_t hipEventCreate(hipEvent_t* e);
hipError_t hipEventDestroy(hipEvent_t e);
hipError_t hipEventRecord(hipEvent_t e, hipStream_t s);
hipError_t hipEventElapsedTime(float* ms, hipEvent_t a, hipEvent_t b);
hipError_t hipStreamBeginCapture(hipStream_t s, hipStreamCaptureMode m);
hipError_t hipStreamEndCapture(hipStream_t s, hipGraph_t* g);
hipError_t hipGraphInstantiate(hipGraphExec_t* e, hipGraph_t g, void*, void*, size_t);
hipError_t hipGraphLaunch(hipGraphExec_t e, hipStream_t s);
hipError_t hipGraphDestroy(hipGraph_t g);
hipError_t hipGraphExecDestroy(hipGraphExec_t e);

// ---------------------------------------------------------------------------------------
// device side
// ---------------------------------------------------------------------------------------
#define __HIP_MEMORY_SCOPE_WORKGROUP 3
#define __HIP_MEMORY_SCOPE_AGENT 4

typedef unsigned emu_u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned emu_u32x2 __attribute__((ext_vector_type(2)));

struct __amdgpu_buffer_rsrc_t {
  char* base;
  uint32_t num;
};

namespace emu {
struct Idx {
  unsigned x, y, z;
};
extern Idx* g_tid;
extern Idx* g_bid;
extern Idx* g_gdim;
extern Idx* g_bdim;

float shfl_xor_f(float v, int mask);
int shfl_xor_i(int v, int mask);
unsigned long long shfl_xor_u64(unsigned long long v, int mask);
unsigned shfl_u(unsigned v, int src);
unsigned long long shfl_idx_u64(unsigned long long v, int src);
int any(int pred);
unsigned long long ballot(int pred);
void wave_sync();
void block_sync();
void spin_yield();
unsigned long long clock();
void mfma_16x16x32_bf16(const void* a, const void* b, const float* c, float* d);
void mfma_16x16x16_bf16(const void* a, const void* b, const float* c, float* d);
void dma(__amdgpu_buffer_rsrc_t r, void* lds, unsigned size, unsigned off);
emu_u32x4 bload16(__amdgpu_buffer_rsrc_t r, unsigned off);
emu_u32x2 bload8(__amdgpu_buffer_rsrc_t r, unsigned off);
unsigned bload4(__amdgpu_buffer_rsrc_t r, unsigned off);
void bstore8(emu_u32x2 v, __amdgpu_buffer_rsrc_t r, unsigned off);
void bstore16(emu_u32x4 v, __amdgpu_buffer_rsrc_t r, unsigned off);
unsigned char* block_lds();
void trace_timeout(int site);
// Runs body on every lane of the grid.  A persistent kernel (its blocks wait on each
// other) needs all blocks live at once; other kernels run in groups of blocks.
void run_kernel(const void* kernel, dim3 grid, dim3 block, size_t lds, const std::function<void()>& body);

template <class K, class... A>
void launch(K kernel, dim3 grid, dim3 block, size_t lds, hipStream_t, A... args) {
  run_kernel((const void*)kernel, grid, block, lds, [=]() { kernel(args...); });
}
}  // namespace emu

#define hipLaunchKernelGGL(kernel, grid, block, lds, stream, ...) \
  emu::launch(kernel, dim3(grid), dim3(block), (size_t)(lds), stream, __VA_ARGS__)
#define hipExtLaunchKernelGGL(kernel, grid, block, lds, stream, ev0, ev1, flags, ...) \
  ((void)(ev0), (void)(ev1), emu::launch(kernel, dim3(grid), dim3(block), (size_t)(lds), stream, __VA_ARGS__))

#define threadIdx (*emu::g_tid)
#define blockIdx (*emu::g_bid)
#define gridDim (*emu::g_gdim)
#define blockDim (*emu::g_bdim)

inline unsigned __umulhi(unsigned a, unsigned b) { return (unsigned)(((unsigned long long)a * b) >> 32); }
inline float __shfl_xor(float v, int mask, int width = 64) {
  (void)width;
  return emu::shfl_xor_f(v, mask);
}
inline int __shfl_xor(int v, int mask, int width = 64) {
  (void)width;
  return emu::shfl_xor_i(v, mask);
}
inline unsigned long long __shfl_xor(unsigned long long v, int mask, int width = 64) {
  (void)width;
  return emu::shfl_xor_u64(v, mask);
}
inline unsigned __shfl(unsigned v, int src) { return emu::shfl_u(v, src); }
// lane l reads lane l - delta; lanes below delta keep their own value
inline unsigned long long __shfl_up(unsigned long long v, unsigned delta, int width = 64) {
  (void)width;
  const int l = (int)(threadIdx.x & 63), s = l - (int)delta;
  return emu::shfl_idx_u64(v, s < 0 ? l : s);
}
// DPP moves used by the kernels: quad_perm (ctrl < 0x100) and the half-row mirror (0x141),
// every row and bank enabled
inline int emu_dpp(int src, int ctrl) {
  const int l = (int)(threadIdx.x & 63);
  int s;
  if (ctrl < 0x100) s = (l & ~3) | ((ctrl >> (2 * (l & 3))) & 3);
  else if (ctrl == 0x141) s = (l & ~7) | (7 - (l & 7));
  else if (ctrl == 0x140) s = (l & ~15) | (15 - (l & 15));
  else abort();
  return (int)emu::shfl_u((unsigned)src, s);
}
#define __builtin_amdgcn_update_dpp(old, src, ctrl, rm, bm, bc) emu_dpp((src), (ctrl))
#define __builtin_amdgcn_readlane(v, l) ((int)emu::shfl_u((unsigned)(v), (l)))
inline int __any(int pred) { return emu::any(pred); }
inline unsigned long long __ballot(int pred) { return emu::ballot(pred); }
inline int __ffsll(long long x) { return __builtin_ffsll(x); }
inline void __syncthreads() { emu::block_sync(); }
inline unsigned long long wall_clock64() { return emu::clock(); }
inline float __expf(float x) { return expf(x); }
inline unsigned __float_as_uint(float f) {
  unsigned u;
  memcpy(&u, &f, 4);
  return u;
}
inline float __uint_as_float(unsigned u) {
  float f;
  memcpy(&f, &u, 4);
  return f;
}
inline unsigned atomicAdd(unsigned* p, unsigned v) { return __atomic_fetch_add(p, v, __ATOMIC_SEQ_CST); }
inline int atomicAdd(int* p, int v) { return __atomic_fetch_add(p, v, __ATOMIC_SEQ_CST); }
inline unsigned long long atomicAdd(unsigned long long* p, unsigned long long v) {
  return __atomic_fetch_add(p, v, __ATOMIC_SEQ_CST);
}
using std::max;
using std::min;

#define __builtin_amdgcn_s_sleep(n) emu::spin_yield()
#define __builtin_amdgcn_readfirstlane(x) (x)  // every lane of a wave holds the same value here
#define __builtin_amdgcn_s_waitcnt(n) emu::wave_sync()
#define __builtin_amdgcn_wave_barrier() emu::wave_sync()
#define __builtin_amdgcn_s_barrier() emu::block_sync()
#define __builtin_amdgcn_fence(...) ((void)0)
#define __builtin_nontemporal_load(p) (*(p))
#define __builtin_amdgcn_make_buffer_rsrc(p, stride, num, flags) \
  (__amdgpu_buffer_rsrc_t{(char*)(p), (uint32_t)(num)})
// variadic: the stored value may be a compound literal with commas
inline emu_u32x4 emu_bl16(__amdgpu_buffer_rsrc_t r, unsigned off, int, int) { return emu::bload16(r, off); }
inline emu_u32x2 emu_bl8(__amdgpu_buffer_rsrc_t r, unsigned off, int, int) { return emu::bload8(r, off); }
inline unsigned emu_bl4(__amdgpu_buffer_rsrc_t r, unsigned off, int, int) { return emu::bload4(r, off); }
inline void emu_bs8(emu_u32x2 v, __amdgpu_buffer_rsrc_t r, unsigned off, int, int) { emu::bstore8(v, r, off); }
inline void emu_bs16(emu_u32x4 v, __amdgpu_buffer_rsrc_t r, unsigned off, int, int) { emu::bstore16(v, r, off); }
#define __builtin_amdgcn_raw_buffer_load_b128(...) emu_bl16(__VA_ARGS__)
#define __builtin_amdgcn_raw_buffer_load_b64(...) emu_bl8(__VA_ARGS__)
#define __builtin_amdgcn_raw_buffer_load_b32(...) emu_bl4(__VA_ARGS__)
#define __builtin_amdgcn_raw_buffer_store_b64(...) emu_bs8(__VA_ARGS__)
#define __builtin_amdgcn_raw_buffer_store_b128(...) emu_bs16(__VA_ARGS__)

template <class V, class C>
inline C emu_mfma6(const V& a, const V& b, const C& c, int, int, int) {
  float cin[4], dout[4];
  memcpy(cin, &c, 16);
  emu::mfma_16x16x32_bf16(&a, &b, cin, dout);
  C d;
  memcpy(&d, dout, 16);
  return d;
}
#define __builtin_amdgcn_mfma_f32_16x16x32_bf16(...) emu_mfma6(__VA_ARGS__)
template <class V, class C>
inline C emu_mfma16(const V& a, const V& b, const C& c, int, int, int) {
  float cin[4], dout[4];
  memcpy(cin, &c, 16);
  emu::mfma_16x16x16_bf16(&a, &b, cin, dout);
  C d;
  memcpy(&d, dout, 16);
  return d;
}
#define __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(...) emu_mfma16(__VA_ARGS__)
// buffer load straight into LDS: lane l writes its size bytes at lds + l size
inline void emu_dma(__amdgpu_buffer_rsrc_t r, void* lds, unsigned size, unsigned voff, unsigned soff, unsigned off,
                    unsigned) {
  emu::dma(r, lds, size, voff + soff + off);
}
#define __builtin_amdgcn_raw_ptr_buffer_load_lds(...) emu_dma(__VA_ARGS__)

#define __hip_atomic_load(p, order, scope) __atomic_load_n((p), __ATOMIC_SEQ_CST)
#define __hip_atomic_store(p, v, order, scope) __atomic_store_n((p), (v), __ATOMIC_SEQ_CST)
#define __hip_atomic_fetch_add(p, v, order, scope) __atomic_fetch_add((p), (v), __ATOMIC_SEQ_CST)
#define __hip_atomic_fetch_or(p, v, order, scope) __atomic_fetch_or((p), (v), __ATOMIC_SEQ_CST)

// the kernels' dynamic-LDS declaration and register-placement hints
#define MC_DYN_LDS(name) unsigned char* name = emu::block_lds()
#define MC_OPAQUE(x) ((void)0)
#define MC_OPAQUE2(x, y) ((void)0)
#define MC_FENCE() ((void)0)
#define MC_TO_VGPR(dst, src) ((dst) = (src))
#define MC_TRACE_TIMEOUT(site) emu::trace_timeout(site)
