// CPU emulation runtime for the library's kernels (see include/hip/hip_runtime.h).
// Test infrastructure only.
//
// "Device" memory is host memory that ends at a PROT_NONE page, so an out-of-bounds
// access faults here as it would on the GPU; the fault handler names the allocation and
// the lane.  Each GPU lane is a ucontext coroutine; lanes yield at wave collectives,
// block barriers and spin-waits, so memory operations between yield points are atomic.
#include <execinfo.h>
#include <signal.h>
#include <sys/mman.h>
#include <ucontext.h>
#include <unistd.h>

#include <cstdio>
#include <cstdlib>
#include <map>
#include <string>
#include <vector>

#include <hip/hip_runtime.h>

#include "emu.hpp"

// ---------------------------------------------------------------------------------------
// memory
// ---------------------------------------------------------------------------------------
namespace {
struct Region {
  char* p;
  size_t n;
  char* base;
  size_t len;
  std::string name;
};
std::map<char*, Region> g_regions;  // by start
const size_t PAGE = 4096;
}  // namespace

namespace emu {
void* dalloc(size_t bytes, const char* name) {
  const size_t sz = (bytes + 15) & ~(size_t)15;
  const size_t np = (sz + PAGE - 1) / PAGE + 2;
  char* base = (char*)mmap(nullptr, np * PAGE, PROT_READ | PROT_WRITE, MAP_PRIVATE | MAP_ANONYMOUS, -1, 0);
  if (base == MAP_FAILED) abort();
  mprotect(base, PAGE, PROT_NONE);
  mprotect(base + (np - 1) * PAGE, PAGE, PROT_NONE);
  char* p = base + (np - 1) * PAGE - sz;  // ends at the guard page
  g_regions[p] = Region{p, sz, base, np * PAGE, name ? name : "device"};
  return p;
}
void dfree(void* p) {
  auto it = g_regions.find((char*)p);
  if (it == g_regions.end()) return;
  munmap(it->second.base, it->second.len);
  g_regions.erase(it);
}
static const Region* region_near(const char* a) {
  const Region* best = nullptr;
  for (auto& kv : g_regions) {
    const Region& R = kv.second;
    if (a >= R.base && a < R.base + R.len) return &R;
    if (!best || std::abs(a - R.p) < std::abs(a - best->p)) best = &R;
  }
  return best;
}
}  // namespace emu

// ---------------------------------------------------------------------------------------
// lanes, waves, blocks
// ---------------------------------------------------------------------------------------
namespace emu {
Idx* g_tid;
Idx* g_bid;
Idx* g_gdim;
Idx* g_bdim;
long long oob_loads = 0, oob_stores = 0;
unsigned long long vclock = 0;

namespace {
struct Lane {
  ucontext_t ctx;
  char* stack = nullptr;
  Idx tid, bid;
  int block = 0, wave = 0, lane = 0;
  bool done = false;
};
enum { K_NONE, K_SHFL_F, K_SHFL_I, K_SHFL_U64, K_SHFL_U, K_ANY, K_BALLOT, K_SYNC, K_MFMA, K_MFMA16 };
struct Wave {
  int kind = K_NONE, arrived = 0;
  unsigned gen = 0;
  float f[64], fo[64];
  int i[64], io[64], src[64];
  unsigned long long q[64], qo[64];
  unsigned u[64], uo[64];
  uint16_t A[64][8], B[64][8];
  float C[64][4], D[64][4];
};
struct Block {
  unsigned char* lds = nullptr;
  int arrived = 0, nthreads = 0;
  unsigned gen = 0;
};
std::vector<Lane> lanes;
std::vector<Wave> waves;
std::vector<Block> blocks;
int cur = -1;
ucontext_t sched;
Idx gdim, bdim;
int waves_per_block = 4;
const std::function<void()>* g_body = nullptr;
const void* g_persistent[4] = {nullptr, nullptr, nullptr, nullptr};

void yield() { swapcontext(&lanes[(size_t)cur].ctx, &sched); }
Wave& my_wave() { return waves[(size_t)(lanes[(size_t)cur].block * waves_per_block + lanes[(size_t)cur].wave)]; }
int my_lane() { return lanes[(size_t)cur].lane; }

void arrive(Wave& W, int kind, void (*compute)(Wave&)) {
  const Lane& L = lanes[(size_t)cur];
  if (W.arrived == 0) W.kind = kind;
  else if (W.kind != kind) {
    fprintf(stderr, "EMU: wave collective mismatch (kind %d vs %d) at block %d wave %d\n", kind, W.kind, L.block,
            L.wave);
    abort();
  }
  const size_t base = (size_t)L.block * (size_t)(waves_per_block * 64) + (size_t)L.wave * 64;
  for (int k = 0; k < 64; ++k)
    if (lanes[base + (size_t)k].done) {
      fprintf(stderr, "EMU: lanes of block %d wave %d left while the others entered a collective\n", L.block, L.wave);
      abort();
    }
  const unsigned g = W.gen;
  if (++W.arrived == 64) {
    compute(W);
    W.arrived = 0;
    ++W.gen;
  } else {
    while (W.gen == g) yield();
  }
}
}  // namespace

float shfl_xor_f(float v, int mask) {
  Wave& W = my_wave();
  const int l = my_lane();
  W.f[l] = v;
  W.src[l] = l ^ mask;
  arrive(W, K_SHFL_F, [](Wave& w) {
    for (int k = 0; k < 64; ++k) w.fo[k] = w.f[(w.src[k] >= 0 && w.src[k] < 64) ? w.src[k] : k];
  });
  return W.fo[l];
}
int shfl_xor_i(int v, int mask) {
  Wave& W = my_wave();
  const int l = my_lane();
  W.i[l] = v;
  W.src[l] = l ^ mask;
  arrive(W, K_SHFL_I, [](Wave& w) {
    for (int k = 0; k < 64; ++k) w.io[k] = w.i[(w.src[k] >= 0 && w.src[k] < 64) ? w.src[k] : k];
  });
  return W.io[l];
}
unsigned long long shfl_xor_u64(unsigned long long v, int mask) {
  Wave& W = my_wave();
  const int l = my_lane();
  W.q[l] = v;
  W.src[l] = l ^ mask;
  arrive(W, K_SHFL_U64, [](Wave& w) {
    for (int k = 0; k < 64; ++k) w.qo[k] = w.q[(w.src[k] >= 0 && w.src[k] < 64) ? w.src[k] : k];
  });
  return W.qo[l];
}
unsigned long long shfl_idx_u64(unsigned long long v, int src) {
  Wave& W = my_wave();
  const int l = my_lane();
  W.q[l] = v;
  W.src[l] = src;
  arrive(W, K_SHFL_U64, [](Wave& w) {
    for (int k = 0; k < 64; ++k) w.qo[k] = w.q[(w.src[k] >= 0 && w.src[k] < 64) ? w.src[k] : k];
  });
  return W.qo[l];
}
unsigned shfl_u(unsigned v, int src) {
  Wave& W = my_wave();
  const int l = my_lane();
  W.u[l] = v;
  W.src[l] = src & 63;
  arrive(W, K_SHFL_U, [](Wave& w) {
    for (int k = 0; k < 64; ++k) w.uo[k] = w.u[w.src[k]];
  });
  return W.uo[l];
}
int any(int pred) {
  Wave& W = my_wave();
  const int l = my_lane();
  W.i[l] = pred != 0;
  arrive(W, K_ANY, [](Wave& w) {
    int a = 0;
    for (int k = 0; k < 64; ++k) a |= w.i[k];
    for (int k = 0; k < 64; ++k) w.io[k] = a;
  });
  return W.io[l];
}
unsigned long long ballot(int pred) {
  Wave& W = my_wave();
  const int l = my_lane();
  W.i[l] = pred != 0;
  arrive(W, K_BALLOT, [](Wave& w) {
    unsigned long long m = 0;
    for (int k = 0; k < 64; ++k) m |= (unsigned long long)(w.i[k] != 0) << k;
    for (int k = 0; k < 64; ++k) w.qo[k] = m;
  });
  return W.qo[l];
}
void wave_sync() {
  arrive(my_wave(), K_SYNC, [](Wave&) {});
}
void block_sync() {
  Block& B = blocks[(size_t)lanes[(size_t)cur].block];
  const unsigned g = B.gen;
  if (++B.arrived == B.nthreads) {
    B.arrived = 0;
    ++B.gen;
  } else {
    while (B.gen == g) yield();
  }
}
void spin_yield() { yield(); }
unsigned long long clock() { return vclock; }
unsigned char* block_lds() { return blocks[(size_t)lanes[(size_t)cur].block].lds; }

static float bf(uint16_t h) {
  const uint32_t u = (uint32_t)h << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}
// v_mfma_f32_16x16x32_bf16: lane l holds A[l % 16][8 (l / 16) + i], B[8 (l / 16) + i][l % 16],
// C / D [4 (l / 16) + v][l % 16]
void mfma_16x16x32_bf16(const void* a, const void* b, const float* c, float* d) {
  Wave& W = my_wave();
  const int l = my_lane();
  memcpy(W.A[l], a, 16);
  memcpy(W.B[l], b, 16);
  memcpy(W.C[l], c, 16);
  arrive(W, K_MFMA, [](Wave& w) {
    float A[16][32], B[32][16], C[16][16];
    for (int k = 0; k < 64; ++k)
      for (int i = 0; i < 8; ++i) {
        A[k % 16][8 * (k / 16) + i] = bf(w.A[k][i]);
        B[8 * (k / 16) + i][k % 16] = bf(w.B[k][i]);
      }
    for (int k = 0; k < 64; ++k)
      for (int v = 0; v < 4; ++v) C[4 * (k / 16) + v][k % 16] = w.C[k][v];
    for (int m = 0; m < 16; ++m)
      for (int n = 0; n < 16; ++n) {
        double s = C[m][n];
        for (int k = 0; k < 32; ++k) s += (double)A[m][k] * (double)B[k][n];
        C[m][n] = (float)s;
      }
    for (int k = 0; k < 64; ++k)
      for (int v = 0; v < 4; ++v) w.D[k][v] = C[4 * (k / 16) + v][k % 16];
  });
  memcpy(d, W.D[l], 16);
}

// v_mfma_f32_16x16x16_bf16: lane l holds A[l % 16][4 (l / 16) + i], B[4 (l / 16) + i][l % 16],
// C / D [4 (l / 16) + v][l % 16]
void mfma_16x16x16_bf16(const void* a, const void* b, const float* c, float* d) {
  Wave& W = my_wave();
  const int l = my_lane();
  memcpy(W.A[l], a, 8);
  memcpy(W.B[l], b, 8);
  memcpy(W.C[l], c, 16);
  arrive(W, K_MFMA16, [](Wave& w) {
    float A[16][16], B[16][16], C[16][16];
    for (int k = 0; k < 64; ++k)
      for (int i = 0; i < 4; ++i) {
        A[k % 16][4 * (k / 16) + i] = bf(w.A[k][i]);
        B[4 * (k / 16) + i][k % 16] = bf(w.B[k][i]);
      }
    for (int k = 0; k < 64; ++k)
      for (int v = 0; v < 4; ++v) C[4 * (k / 16) + v][k % 16] = w.C[k][v];
    for (int m = 0; m < 16; ++m)
      for (int n = 0; n < 16; ++n) {
        double s = C[m][n];
        for (int k = 0; k < 16; ++k) s += (double)A[m][k] * (double)B[k][n];
        C[m][n] = (float)s;
      }
    for (int k = 0; k < 64; ++k)
      for (int v = 0; v < 4; ++v) w.D[k][v] = C[4 * (k / 16) + v][k % 16];
  });
  memcpy(d, W.D[l], 16);
}

void dma(__amdgpu_buffer_rsrc_t r, void* lds, unsigned size, unsigned off) {
  unsigned char* dst = (unsigned char*)lds + (size_t)my_lane() * size;
  if ((uint64_t)off + size > r.num) {
    ++oob_loads;
    memset(dst, 0, size);
    return;
  }
  memcpy(dst, r.base + off, size);
}

// Offsets at or past 0x80000000 are the kernels' deliberate masked-off loads (zero, as the
// hardware's range check returns); other out-of-range offsets are counted as faults.
constexpr unsigned MASKED = 0x80000000u;
unsigned bload4(__amdgpu_buffer_rsrc_t r, unsigned off) {
  unsigned v = 0u;
  if ((uint64_t)off + 4 > r.num) {
    if (off < MASKED) ++oob_loads;
    return v;
  }
  memcpy(&v, r.base + off, 4);
  return v;
}
emu_u32x4 bload16(__amdgpu_buffer_rsrc_t r, unsigned off) {
  emu_u32x4 v = {0u, 0u, 0u, 0u};
  if ((uint64_t)off + 16 > r.num) {
    if (off < MASKED) ++oob_loads;
    return v;
  }
  memcpy(&v, r.base + off, 16);
  return v;
}
emu_u32x2 bload8(__amdgpu_buffer_rsrc_t r, unsigned off) {
  emu_u32x2 v = {0u, 0u};
  if ((uint64_t)off + 8 > r.num) {
    if (off < MASKED) ++oob_loads;
    return v;
  }
  memcpy(&v, r.base + off, 8);
  return v;
}
void bstore8(emu_u32x2 v, __amdgpu_buffer_rsrc_t r, unsigned off) {
  if ((uint64_t)off + 8 > r.num) {
    ++oob_stores;
    return;
  }
  memcpy(r.base + off, &v, 8);
}
void bstore16(emu_u32x4 v, __amdgpu_buffer_rsrc_t r, unsigned off) {
  if ((uint64_t)off + 16 > r.num) {
    ++oob_stores;
    return;
  }
  memcpy(r.base + off, &v, 16);
}

void trace_timeout(int site) {
  const Lane& L = lanes[(size_t)cur];
  if (L.lane != 0) return;
  fprintf(stderr, "EMU: timeout at wait site %d: block %d wave %d\n", site, L.block, L.wave);
}

void set_persistent(const void* kernel) {
  for (auto& p : g_persistent)
    if (!p || p == kernel) {
      p = kernel;
      return;
    }
}

static void lane_main() {
  (*g_body)();
  lanes[(size_t)cur].done = true;  // returns to the scheduler through uc_link
}

static std::vector<char*> stack_pool;
static const size_t STACK = 256 * 1024;

// run blocks [b0, b1) of the grid to completion; false on a deadlock
static bool run_blocks(size_t b0, size_t b1, dim3 grid, dim3 block, size_t lds) {
  const int T = (int)(block.x * block.y * block.z);
  waves_per_block = (T + 63) / 64;
  const size_t nb = b1 - b0;
  lanes.assign(nb * (size_t)waves_per_block * 64, Lane{});
  waves.assign(nb * (size_t)waves_per_block, Wave{});
  blocks.assign(nb, Block{});
  for (size_t k = 0; k < nb; ++k) {
    blocks[k].nthreads = T;
    blocks[k].lds = (unsigned char*)dalloc(std::max<size_t>(lds, 16), "lds");
    memset(blocks[k].lds, 0xA5, std::max<size_t>(lds, 16));  // LDS starts as garbage
  }
  while (stack_pool.size() < lanes.size()) stack_pool.push_back((char*)malloc(STACK));
  size_t live = 0;
  for (size_t i = 0; i < lanes.size(); ++i) {
    Lane& L = lanes[i];
    const size_t bl = i / ((size_t)waves_per_block * 64);
    const int t = (int)(i % ((size_t)waves_per_block * 64));
    L.block = (int)bl;
    L.wave = t / 64;
    L.lane = t % 64;
    const size_t gb = b0 + bl;
    L.bid = Idx{(unsigned)(gb % grid.x), (unsigned)((gb / grid.x) % grid.y), (unsigned)(gb / (grid.x * grid.y))};
    L.tid = Idx{(unsigned)(t % block.x), (unsigned)((t / block.x) % block.y), (unsigned)(t / (block.x * block.y))};
    L.done = t >= T;  // padding lanes of a partial wave never run
    if (L.done) continue;
    ++live;
    L.stack = stack_pool[i];
    getcontext(&L.ctx);
    L.ctx.uc_stack.ss_sp = L.stack;
    L.ctx.uc_stack.ss_size = STACK;
    L.ctx.uc_link = &sched;
    makecontext(&L.ctx, lane_main, 0);
  }
  unsigned long long rounds = 0;
  while (live > 0) {
    for (size_t i = 0; i < lanes.size(); ++i) {
      Lane& L = lanes[i];
      if (L.done) continue;
      cur = (int)i;
      g_tid = &L.tid;
      g_bid = &L.bid;
      swapcontext(&sched, &L.ctx);
    }
    vclock += 1000;  // virtual time: 1000 ticks per round, whatever the lane count
    if (++rounds > 4000000ull) return false;
    live = 0;
    for (auto& L : lanes) live += !L.done;
  }
  for (auto& B : blocks) dfree(B.lds);
  cur = -1;
  return true;
}

void run_kernel(const void* kernel, dim3 grid, dim3 block, size_t lds, const std::function<void()>& body) {
  g_body = &body;
  gdim = Idx{grid.x, grid.y, grid.z};
  bdim = Idx{block.x, block.y, block.z};
  g_gdim = &gdim;
  g_bdim = &bdim;
  const size_t nblocks = (size_t)grid.x * grid.y * grid.z;
  // blocks of ordinary kernels run one at a time (their __shared__ arrays are static);
  // a persistent kernel (its LDS is per block) needs every block live at once
  bool persistent = false;
  for (const void* p : g_persistent) persistent |= p && p == kernel;
  const size_t group = persistent ? nblocks : 1;
  if (persistent && getenv("EMU_TRACE_PERSISTENT"))
    fprintf(stderr, "EMU: persistent launch, %zu blocks of %u threads\n", nblocks, block.x * block.y * block.z);
  for (size_t b0 = 0; b0 < nblocks; b0 += group)
    if (!run_blocks(b0, std::min(nblocks, b0 + group), grid, block, lds)) {
      fprintf(stderr, "EMU: deadlock in a kernel launch\n");
      abort();
    }
}
}  // namespace emu

// ---------------------------------------------------------------------------------------
// fault handler
// ---------------------------------------------------------------------------------------
static void on_segv(int, siginfo_t* si, void*) {
  const char* a = (const char*)si->si_addr;
  fprintf(stderr, "EMU: fault at %p", (const void*)a);
  if (const auto* R = emu::region_near(a))
    fprintf(stderr, " near %s [%p, +%zu) offset %lld", R->name.c_str(), (void*)R->p, R->n, (long long)(a - R->p));
  if (emu::cur >= 0) {
    const auto& L = emu::lanes[(size_t)emu::cur];
    fprintf(stderr, " lane: block (%u,%u) wave %d lane %d", L.bid.x, L.bid.y, L.wave, L.lane);
  }
  fprintf(stderr, "\n");
  void* fr[32];
  const int n = backtrace(fr, 32);
  backtrace_symbols_fd(fr, n, 2);
  _exit(3);
}

void emu::install_fault_handler() {
  struct sigaction sa;
  memset(&sa, 0, sizeof sa);
  sa.sa_sigaction = on_segv;
  sa.sa_flags = SA_SIGINFO | SA_ONSTACK;
  static char altstack[1 << 16];
  stack_t ss{altstack, 0, sizeof altstack};
  sigaltstack(&ss, nullptr);
  sigaction(SIGSEGV, &sa, nullptr);
  sigaction(SIGBUS, &sa, nullptr);
}

// ---------------------------------------------------------------------------------------
// runtime calls: synchronous
// ---------------------------------------------------------------------------------------
struct emu_event {
  int dummy;
};
struct emu_graph {
  int dummy;
};
struct emu_stream {
  int dummy;
};

hipError_t hipMalloc(void** p, size_t n) {
  *p = emu::dalloc(n, "hipMalloc");
  return hipSuccess;
}
hipError_t hipFree(void* p) {
  emu::dfree(p);
  return hipSuccess;
}
hipError_t hipMemset(void* p, int v, size_t n) {
  memset(p, v, n);
  return hipSuccess;
}
hipError_t hipMemcpy(void* d, const void* s, size_t n, hipMemcpyKind) {
  memmove(d, s, n);
  return hipSuccess;
}
hipError_t hipMemcpyAsync(void* d, const void* s, size_t n, hipMemcpyKind k, hipStream_t) { return hipMemcpy(d, s, n, k); }
hipError_t hipMemcpy2D(void* d, size_t dp, const void* s, size_t sp, size_t w, size_t h, hipMemcpyKind) {
  for (size_t r = 0; r < h; ++r) memmove((char*)d + r * dp, (const char*)s + r * sp, w);
  return hipSuccess;
}
hipError_t hipMemcpy2DAsync(void* d, size_t dp, const void* s, size_t sp, size_t w, size_t h, hipMemcpyKind k,
                             hipStream_t) {
  return hipMemcpy2D(d, dp, s, sp, w, h, k);
}
hipError_t hipHostMalloc(void** p, size_t n, unsigned) {
  *p = malloc(n ? n : 1);
  return hipSuccess;
}
hipError_t hipHostFree(void* p) {
  free(p);
  return hipSuccess;
}
hipError_t hipSetDevice(int) { return hipSuccess; }
hipError_t hipGetDevice(int* d) {
  *d = 0;
  return hipSuccess;
}
hipError_t hipGetDeviceCount(int* n) {
  *n = 1;
  return hipSuccess;
}
hipError_t hipDeviceGetAttribute(int* v, hipDeviceAttribute_t, int) {
  const char* e = getenv("EMU_CUS");
  *v = e ? atoi(e) : 16;
  return hipSuccess;
}
hipError_t hipStreamCreateWithFlags(hipStream_t* s, unsigned) {
  *s = new emu_stream{0};
  return hipSuccess;
}
hipError_t hipStreamDestroy(hipStream_t s) {
  delete s;
  return hipSuccess;
}
hipError_t hipStreamSynchronize(hipStream_t) { return hipSuccess; }
hipError_t hipGetLastError() { return hipSuccess; }
const char* hipGetErrorString(hipError_t) { return "emulated error"; }
hipError_t hipFuncSetAttribute(const void*, hipFuncAttribute, int) { return hipSuccess; }
hipError_t hipOccupancyMaxActiveBlocksPerMultiprocessor(int* n, const void*, int, size_t) {
  *n = 1;
  return hipSuccess;
}
hipError_t hipEventCreate(hipEvent_t* e) {
  *e = new emu_event{0};
  return hipSuccess;
}
hipError_t hipEventDestroy(hipEvent_t e) {
  delete e;
  return hipSuccess;
}
hipError_t hipEventRecord(hipEvent_t, hipStream_t) { return hipSuccess; }
hipError_t hipEventElapsedTime(float* ms, hipEvent_t, hipEvent_t) {
  *ms = 0.f;
  return hipSuccess;
}
// no graph capture here: the step runs eagerly (MC_STEP_EAGER=1)
hipError_t hipStreamBeginCapture(hipStream_t, hipStreamCaptureMode) { return hipErrorEmu; }
hipError_t hipStreamEndCapture(hipStream_t, hipGraph_t* g) {
  *g = nullptr;
  return hipErrorEmu;
}
hipError_t hipGraphInstantiate(hipGraphExec_t*, hipGraph_t, void*, void*, size_t) { return hipErrorEmu; }
hipError_t hipGraphLaunch(hipGraphExec_t, hipStream_t) { return hipErrorEmu; }
hipError_t hipGraphDestroy(hipGraph_t) { return hipSuccess; }
hipError_t hipGraphExecDestroy(hipGraphExec_t) { return hipSuccess; }
