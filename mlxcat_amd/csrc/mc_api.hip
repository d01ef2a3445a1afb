// mc_api.hip -- the C ABI (include/mlxcat_hip.h): model and batch handles, the verify
// forward, the fused speculative step captured as one HIP graph per batch, and the
// standalone proposer / acceptance entry points.  Host code only; the kernels live in
// mc_gemv.hip, mc_kernels.hip and mc_step.hip.
#include <algorithm>
#include <cmath>
#include <type_traits>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

#include "mc_gemv.hpp"
#include "mc_kernels.hpp"
#include "mc_step.hpp"

namespace mc {

static thread_local std::string g_err;
void set_error(const std::string& msg) { g_err = msg; }
int fail(int code, const std::string& msg) {
  g_err = msg;
  return code;
}
int hip_fail(hipError_t e, const char* what, const char* file, int line) {
  char buf[512];
  snprintf(buf, sizeof buf, "HIP error '%s' in %s (%s:%d)", hipGetErrorString(e), what, file, line);
  g_err = buf;
  return e == hipErrorOutOfMemory ? MC_E_NOMEM : MC_E_HIP;
}

static int g_device = 0;
// Prompt prefill chunk: the reference's idle-time chunk (Scheduler.swift:670-800 uses 512
// tokens idle, 2048 busy); more than 64 tokens run the linears through the large-M GEMM.
constexpr int PREFILL_CHUNK = 512;

// State of mc_accept_noalloc: a file-scope device array, one copy per GPU, held until the
// process ends and shared by every call on that GPU.  Host code never names it as an
// address: hipGetSymbolAddress gives each device's copy (resolved once per device, with
// that device current), and only that pointer reaches kernels and copies.
constexpr size_t NOALLOC_SCRATCH_BYTES = 64 * 1024;
constexpr int NOALLOC_MAX_ROWS = 64, NOALLOC_MAX_DRAFTS = 16, NOALLOC_MAX_DEVICES = 64;
static __device__ __align__(256) unsigned char scratch[NOALLOC_SCRATCH_BYTES];
static void* g_scratch_ptr[NOALLOC_MAX_DEVICES] = {};

static int resolve_scratch(int device) {  // `device` must be current
  if (device < 0 || device >= NOALLOC_MAX_DEVICES) return fail(MC_E_INVALID, "device index beyond the scratch table");
  if (g_scratch_ptr[device]) return MC_OK;
  void* p = nullptr;
  const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
  if (e != hipSuccess) return hip_fail(e, "hipGetSymbolAddress(scratch)", __FILE__, __LINE__);
  g_scratch_ptr[device] = p;
  return MC_OK;
}

template <typename T>
static int dev_alloc(T** p, size_t n) {
  *p = nullptr;
  if (n == 0) n = 1;
  hipError_t e = hipMalloc((void**)p, n * sizeof(T));
  if (e != hipSuccess) return hip_fail(e, "hipMalloc", __FILE__, __LINE__);
  return MC_OK;
}
template <typename T>
static int dev_zero(T** p, size_t n) {
  int rc = dev_alloc(p, n);
  if (rc) return rc;
  MC_HIP(hipMemset(*p, 0, (n ? n : 1) * sizeof(T)));
  return MC_OK;
}

static int qlinear_alloc(QLinear* L, int N, int K) {
  if (N <= 0 || K <= 0 || K % 64) return fail(MC_E_INVALID, "linear: K must be a positive multiple of 64");
  L->N = N;
  L->K = K;
  L->NT = (N + 15) / 16;
  L->GP = (K + 127) / 128;
  int rc = dev_zero(&L->qw, L->qw_words());
  if (rc) return rc;
  return dev_zero(&L->sb, L->sb_words());
}
static void qlinear_free(QLinear* L) {
  if (L->qw) (void)hipFree(L->qw);
  if (L->sb) (void)hipFree(L->sb);
  L->qw = nullptr;
  L->sb = nullptr;
}

}  // namespace mc

using namespace mc;

// ---------------------------------------------------------------------------
// model
// ---------------------------------------------------------------------------
struct mc_model {
  mc_model_config cfg{};
  int device = 0;
  bool fake = false;
  struct Layer {
    QLinear qkv, o, gateup, down;
    // Qwen3-MoE: the router and every expert's interleaved gate/up and down (expert e's
    // tiles at e * qw_words() / e * sb_words() of the N x K shape the linear records)
    QLinear router, egu, edn;
    uint16_t *in_norm = nullptr, *post_norm = nullptr, *q_norm = nullptr, *k_norm = nullptr;
  };
  std::vector<Layer> layers;
  QLinear embed, lm_head;
  uint16_t* final_norm = nullptr;
  hipStream_t st = nullptr;
  const QLinear& head() const { return cfg.tied_embeddings ? embed : lm_head; }
  bool moe() const { return cfg.arch == MC_ARCH_QWEN3_MOE; }
};

// Expert e of a linear holding every expert's tiles.
static QLinear expert_view(const QLinear& all, int e) {
  QLinear v = all;
  v.qw = all.qw + (size_t)e * all.qw_words();
  v.sb = all.sb + (size_t)e * all.sb_words();
  return v;
}

static int experts_alloc(QLinear* L, int E, int N, int K) {
  if (N <= 0 || K <= 0 || K % 64) return fail(MC_E_INVALID, "expert linear: K must be a positive multiple of 64");
  L->N = N;
  L->K = K;
  L->NT = (N + 15) / 16;
  L->GP = (K + 127) / 128;
  int rc = dev_zero(&L->qw, L->qw_words() * (size_t)E);
  if (rc) return rc;
  return dev_zero(&L->sb, L->sb_words() * (size_t)E);
}

extern "C" const char* mc_last_error(void) { return g_err.c_str(); }

extern "C" int mc_set_device(int device) {
  int n = 0;
  MC_HIP(hipGetDeviceCount(&n));
  if (device < 0 || device >= n) return fail(MC_E_INVALID, "mc_set_device: no such device");
  g_device = device;
  MC_HIP(hipSetDevice(device));
  return resolve_scratch(device);
}

static int norm_ones(uint16_t** p, int n) {
  int rc = dev_alloc(p, (size_t)n);
  if (rc) return rc;
  std::vector<uint16_t> h((size_t)n, (uint16_t)0x3F80);
  MC_HIP(hipMemcpy(*p, h.data(), (size_t)n * 2, hipMemcpyHostToDevice));
  return MC_OK;
}

extern "C" int mc_model_create(const mc_model_config* cfg, mc_model** out) {
  if (!cfg || !out) return fail(MC_E_INVALID, "mc_model_create: null argument");
  *out = nullptr;
  MC_HIP(hipSetDevice(g_device));
  auto* m = new mc_model();
  m->cfg = *cfg;
  m->device = g_device;
  const auto& c = *cfg;
  if (c.arch == MC_ARCH_FAKE_REPEATING || c.arch == MC_ARCH_FAKE_MISMATCHING) {
    if (c.vocab < 8) { delete m; return fail(MC_E_INVALID, "fake model needs vocab >= 8"); }
    m->fake = true;
    *out = m;
    return MC_OK;
  }
  if (c.arch != MC_ARCH_QWEN3 && c.arch != MC_ARCH_LLAMA && c.arch != MC_ARCH_QWEN3_MOE) {
    delete m;
    return fail(MC_E_INVALID, "mc_model_create: architecture not supported by this build");
  }
  if (c.n_layers <= 0 || c.hidden % 64 || c.hidden > 4096 || (c.head_dim != 64 && c.head_dim != 128) || c.n_kv_heads <= 0 ||
      c.n_q_heads % c.n_kv_heads || c.intermediate % 64 || c.vocab <= 0 || (c.n_q_heads * c.head_dim) % 64) {
    delete m;
    return fail(MC_E_INVALID, "mc_model_create: unsupported shape");
  }
  if (c.arch == MC_ARCH_QWEN3_MOE &&
      (c.n_experts < 1 || c.n_experts > 256 || c.n_experts_per_tok < 1 || c.n_experts_per_tok > 8 ||
       c.n_experts_per_tok > c.n_experts || c.moe_intermediate <= 0 || c.moe_intermediate % 64 ||
       c.moe_intermediate > 2560 || c.hidden > 2560)) {
    delete m;
    return fail(MC_E_INVALID, "mc_model_create: unsupported MoE shape (<= 256 experts, top-k <= 8, hidden and expert "
                              "width multiples of 64, <= 2560)");
  }
  int rc = MC_OK;
  MC_HIP(hipStreamCreateWithFlags(&m->st, hipStreamNonBlocking));
  const int H = c.hidden, d = c.head_dim, nq = c.n_q_heads, nkv = c.n_kv_heads, I = c.intermediate;
  m->layers.resize((size_t)c.n_layers);
  for (auto& L : m->layers) {
    if ((rc = qlinear_alloc(&L.qkv, (nq + 2 * nkv) * d, H))) break;
    if ((rc = qlinear_alloc(&L.o, H, nq * d))) break;
    if (c.arch == MC_ARCH_QWEN3_MOE) {
      if ((rc = qlinear_alloc(&L.router, c.n_experts, H))) break;
      if ((rc = experts_alloc(&L.egu, c.n_experts, 2 * c.moe_intermediate, H))) break;
      if ((rc = experts_alloc(&L.edn, c.n_experts, H, c.moe_intermediate))) break;
    } else {
      if ((rc = qlinear_alloc(&L.gateup, 2 * I, H))) break;
      if ((rc = qlinear_alloc(&L.down, H, I))) break;
    }
    if ((rc = norm_ones(&L.in_norm, H)) || (rc = norm_ones(&L.post_norm, H))) break;
    if (c.arch == MC_ARCH_QWEN3 || c.arch == MC_ARCH_QWEN3_MOE) {
      if ((rc = norm_ones(&L.q_norm, d)) || (rc = norm_ones(&L.k_norm, d))) break;
    }
  }
  if (!rc) rc = qlinear_alloc(&m->embed, c.vocab, H);
  if (!rc && !c.tied_embeddings) rc = qlinear_alloc(&m->lm_head, c.vocab, H);
  if (!rc) rc = norm_ones(&m->final_norm, H);
  if (!rc) rc = gemv_setup_lds();
  if (rc) {
    mc_model_destroy(m);
    return rc;
  }
  *out = m;
  return MC_OK;
}

extern "C" void mc_model_destroy(mc_model* m) {
  if (!m) return;
  (void)hipSetDevice(m->device);
  for (auto& L : m->layers) {
    qlinear_free(&L.qkv);
    qlinear_free(&L.o);
    qlinear_free(&L.gateup);
    qlinear_free(&L.down);
    qlinear_free(&L.router);
    qlinear_free(&L.egu);
    qlinear_free(&L.edn);
    for (uint16_t* p : {L.in_norm, L.post_norm, L.q_norm, L.k_norm})
      if (p) (void)hipFree(p);
  }
  qlinear_free(&m->embed);
  qlinear_free(&m->lm_head);
  if (m->final_norm) (void)hipFree(m->final_norm);
  if (m->st) (void)hipStreamDestroy(m->st);
  delete m;
}

// Where an MLX tensor lands inside the fused tile tensors: (linear, row offset, row stride, rows).
// expert >= 0 names one expert's gate / up / down of a Qwen3-MoE layer.
static int linear_slot(mc_model* m, int layer, int which, int expert, QLinear* L, int* off, int* stride, int* rows, int* K) {
  const auto& c = m->cfg;
  const int H = c.hidden, d = c.head_dim, nq = c.n_q_heads, nkv = c.n_kv_heads, I = c.intermediate;
  if (expert >= 0 && (!m->moe() || expert >= c.n_experts)) return fail(MC_E_INVALID, "no such expert");
  if (which == MC_W_EMBED) { *L = m->embed; *off = 0; *stride = 1; *rows = c.vocab; *K = H; return MC_OK; }
  if (which == MC_W_LM_HEAD) {
    if (c.tied_embeddings) return fail(MC_E_INVALID, "tied model has no separate lm_head");
    *L = m->lm_head; *off = 0; *stride = 1; *rows = c.vocab; *K = H; return MC_OK;
  }
  if (layer < 0 || layer >= c.n_layers) return fail(MC_E_INVALID, "layer out of range");
  auto& Ly = m->layers[(size_t)layer];
  if (m->moe() && (which == MC_W_GATE || which == MC_W_UP || which == MC_W_DOWN)) {
    if (expert < 0) return fail(MC_E_INVALID, "MoE layer: gate / up / down need an expert index");
    const int MI = c.moe_intermediate;
    if (which == MC_W_DOWN) { *L = expert_view(Ly.edn, expert); *off = 0; *stride = 1; *rows = H; *K = MI; return MC_OK; }
    *L = expert_view(Ly.egu, expert); *off = which == MC_W_UP ? 1 : 0; *stride = 2; *rows = MI; *K = H;
    return MC_OK;
  }
  if (expert >= 0) return fail(MC_E_INVALID, "only gate / up / down have experts");
  switch (which) {
    case MC_W_Q: *L = Ly.qkv; *off = 0; *stride = 1; *rows = nq * d; *K = H; return MC_OK;
    case MC_W_K: *L = Ly.qkv; *off = nq * d; *stride = 1; *rows = nkv * d; *K = H; return MC_OK;
    case MC_W_V: *L = Ly.qkv; *off = (nq + nkv) * d; *stride = 1; *rows = nkv * d; *K = H; return MC_OK;
    case MC_W_O: *L = Ly.o; *off = 0; *stride = 1; *rows = H; *K = nq * d; return MC_OK;
    case MC_W_GATE: *L = Ly.gateup; *off = 0; *stride = 2; *rows = I; *K = H; return MC_OK;
    case MC_W_UP: *L = Ly.gateup; *off = 1; *stride = 2; *rows = I; *K = H; return MC_OK;
    case MC_W_DOWN: *L = Ly.down; *off = 0; *stride = 1; *rows = H; *K = I; return MC_OK;
    case MC_W_ROUTER:
      if (!m->moe()) return fail(MC_E_INVALID, "dense model has no router");
      *L = Ly.router; *off = 0; *stride = 1; *rows = c.n_experts; *K = H; return MC_OK;
    default: return fail(MC_E_INVALID, "unknown linear slot");
  }
}

extern "C" int mc_model_set_linear(mc_model* m, int32_t layer, int32_t which, int32_t expert, const uint32_t* wq,
                                   const uint16_t* scales, const uint16_t* biases) {
  if (!m || !wq || !scales || !biases) return fail(MC_E_INVALID, "mc_model_set_linear: null argument");
  if (m->fake) return fail(MC_E_STATE, "fake model has no weights");
  MC_HIP(hipSetDevice(m->device));
  QLinear L;
  int off, stride, rows, K;
  int rc = linear_slot(m, layer, which, expert, &L, &off, &stride, &rows, &K);
  if (rc) return rc;
  uint32_t* dq;
  uint16_t *ds, *db;
  const size_t nw = (size_t)rows * (K / 8), ns = (size_t)rows * (K / 64);
  if ((rc = dev_alloc(&dq, nw))) return rc;
  if ((rc = dev_alloc(&ds, ns))) { (void)hipFree(dq); return rc; }
  if ((rc = dev_alloc(&db, ns))) { (void)hipFree(dq); (void)hipFree(ds); return rc; }
  hipError_t e = hipMemcpy(dq, wq, nw * 4, hipMemcpyHostToDevice);
  if (e == hipSuccess) e = hipMemcpy(ds, scales, ns * 2, hipMemcpyHostToDevice);
  if (e == hipSuccess) e = hipMemcpy(db, biases, ns * 2, hipMemcpyHostToDevice);
  if (e == hipSuccess) {
    rc = qlinear_repack(L, off, stride, rows, dq, ds, db, m->st);
    if (!rc) e = hipStreamSynchronize(m->st);
  }
  (void)hipFree(dq);
  (void)hipFree(ds);
  (void)hipFree(db);
  if (e != hipSuccess) return hip_fail(e, "mc_model_set_linear", __FILE__, __LINE__);
  return rc;
}

extern "C" int mc_model_get_linear(mc_model* m, int32_t layer, int32_t which, int32_t expert, uint32_t* wq,
                                   uint16_t* scales, uint16_t* biases) {
  if (!m || !wq || !scales || !biases) return fail(MC_E_INVALID, "mc_model_get_linear: null argument");
  if (m->fake) return fail(MC_E_STATE, "fake model has no weights");
  MC_HIP(hipSetDevice(m->device));
  QLinear L;
  int off, stride, rows, K;
  int rc = linear_slot(m, layer, which, expert, &L, &off, &stride, &rows, &K);
  if (rc) return rc;
  uint32_t* dq;
  uint16_t *ds, *db;
  const size_t nw = (size_t)rows * (K / 8), ns = (size_t)rows * (K / 64);
  if ((rc = dev_alloc(&dq, nw))) return rc;
  if ((rc = dev_alloc(&ds, ns))) { (void)hipFree(dq); return rc; }
  if ((rc = dev_alloc(&db, ns))) { (void)hipFree(dq); (void)hipFree(ds); return rc; }
  rc = qlinear_export(L, off, stride, rows, dq, ds, db, m->st);
  hipError_t e = hipSuccess;
  if (!rc) e = hipStreamSynchronize(m->st);
  if (!rc && e == hipSuccess) e = hipMemcpy(wq, dq, nw * 4, hipMemcpyDeviceToHost);
  if (!rc && e == hipSuccess) e = hipMemcpy(scales, ds, ns * 2, hipMemcpyDeviceToHost);
  if (!rc && e == hipSuccess) e = hipMemcpy(biases, db, ns * 2, hipMemcpyDeviceToHost);
  (void)hipFree(dq);
  (void)hipFree(ds);
  (void)hipFree(db);
  if (e != hipSuccess) return hip_fail(e, "mc_model_get_linear", __FILE__, __LINE__);
  return rc;
}

extern "C" int mc_model_set_norm(mc_model* m, int32_t layer, int32_t which, const uint16_t* w) {
  if (!m || !w) return fail(MC_E_INVALID, "mc_model_set_norm: null argument");
  if (m->fake) return fail(MC_E_STATE, "fake model has no weights");
  MC_HIP(hipSetDevice(m->device));
  const auto& c = m->cfg;
  uint16_t* dst = nullptr;
  int n = 0;
  if (which == MC_N_FINAL) {
    dst = m->final_norm;
    n = c.hidden;
  } else {
    if (layer < 0 || layer >= c.n_layers) return fail(MC_E_INVALID, "layer out of range");
    auto& L = m->layers[(size_t)layer];
    switch (which) {
      case MC_N_INPUT: dst = L.in_norm; n = c.hidden; break;
      case MC_N_POST: dst = L.post_norm; n = c.hidden; break;
      case MC_N_Q: dst = L.q_norm; n = c.head_dim; break;
      case MC_N_K: dst = L.k_norm; n = c.head_dim; break;
      default: return fail(MC_E_INVALID, "unknown norm slot");
    }
    if (!dst) return fail(MC_E_INVALID, "this architecture has no such norm");
  }
  MC_HIP(hipMemcpy(dst, w, (size_t)n * 2, hipMemcpyHostToDevice));
  return MC_OK;
}

// synthetic norm weights: bf16 1 + (h % 32 - 16) / 128 (matches the oracle)
static std::vector<uint16_t> synth_norm(uint64_t seed, uint64_t tid, int n) {
  std::vector<uint16_t> w((size_t)n);
  const uint64_t base = mix64(seed ^ mix64(tid ^ 0x4E4F524Dull));
  for (int i = 0; i < n; ++i) {
    const uint64_t h = mix64(base ^ (uint64_t)i);
    const int k = (int)(h % 32u) - 16;
    w[(size_t)i] = f32_to_bf16(1.0f + (float)k / 128.0f);
  }
  return w;
}

extern "C" int mc_model_init_synthetic(mc_model* m, uint64_t seed) {
  if (!m) return fail(MC_E_INVALID, "mc_model_init_synthetic: null model");
  if (m->fake) return MC_OK;
  MC_HIP(hipSetDevice(m->device));
  const auto& c = m->cfg;
  const int d = c.head_dim, nq = c.n_q_heads, nkv = c.n_kv_heads, I = c.intermediate, H = c.hidden;
  int rc;
  for (int l = 0; l < c.n_layers; ++l) {
    auto& L = m->layers[(size_t)l];
    if ((rc = qlinear_synth(L.qkv, 0, 1, nq * d, synth_base(seed, tensor_id(l, T_Q)), -7, m->st))) return rc;
    if ((rc = qlinear_synth(L.qkv, nq * d, 1, nkv * d, synth_base(seed, tensor_id(l, T_K)), -7, m->st))) return rc;
    if ((rc = qlinear_synth(L.qkv, (nq + nkv) * d, 1, nkv * d, synth_base(seed, tensor_id(l, T_V)), -7, m->st))) return rc;
    if ((rc = qlinear_synth(L.o, 0, 1, H, synth_base(seed, tensor_id(l, T_O)), -7, m->st))) return rc;
    if (m->moe()) {
      const int MI = c.moe_intermediate;
      if ((rc = qlinear_synth(L.router, 0, 1, c.n_experts, synth_base(seed, tensor_id(l, T_ROUTER)), -7, m->st))) return rc;
      for (int e = 0; e < c.n_experts; ++e) {
        const QLinear gu = expert_view(L.egu, e), dn = expert_view(L.edn, e);
        if ((rc = qlinear_synth(gu, 0, 2, MI, synth_base(seed, expert_tensor_id(l, e, T_GATE)), -7, m->st))) return rc;
        if ((rc = qlinear_synth(gu, 1, 2, MI, synth_base(seed, expert_tensor_id(l, e, T_UP)), -7, m->st))) return rc;
        if ((rc = qlinear_synth(dn, 0, 1, H, synth_base(seed, expert_tensor_id(l, e, T_DOWN)), -7, m->st))) return rc;
      }
    } else {
      if ((rc = qlinear_synth(L.gateup, 0, 2, I, synth_base(seed, tensor_id(l, T_GATE)), -7, m->st))) return rc;
      if ((rc = qlinear_synth(L.gateup, 1, 2, I, synth_base(seed, tensor_id(l, T_UP)), -7, m->st))) return rc;
      if ((rc = qlinear_synth(L.down, 0, 1, H, synth_base(seed, tensor_id(l, T_DOWN)), -7, m->st))) return rc;
    }
    auto w = synth_norm(seed, tensor_id(l, T_IN_NORM), H);
    MC_HIP(hipMemcpy(L.in_norm, w.data(), (size_t)H * 2, hipMemcpyHostToDevice));
    w = synth_norm(seed, tensor_id(l, T_POST_NORM), H);
    MC_HIP(hipMemcpy(L.post_norm, w.data(), (size_t)H * 2, hipMemcpyHostToDevice));
    if (L.q_norm) {
      w = synth_norm(seed, tensor_id(l, T_Q_NORM), d);
      MC_HIP(hipMemcpy(L.q_norm, w.data(), (size_t)d * 2, hipMemcpyHostToDevice));
      w = synth_norm(seed, tensor_id(l, T_K_NORM), d);
      MC_HIP(hipMemcpy(L.k_norm, w.data(), (size_t)d * 2, hipMemcpyHostToDevice));
    }
  }
  if ((rc = qlinear_synth(m->embed, 0, 1, c.vocab, synth_base(seed, TID_EMBED), -7, m->st))) return rc;
  if (!c.tied_embeddings && (rc = qlinear_synth(m->lm_head, 0, 1, c.vocab, synth_base(seed, TID_LM_HEAD), -7, m->st)))
    return rc;
  auto w = synth_norm(seed, TID_FINAL_NORM, H);
  MC_HIP(hipMemcpy(m->final_norm, w.data(), (size_t)H * 2, hipMemcpyHostToDevice));
  MC_HIP(hipStreamSynchronize(m->st));
  return MC_OK;
}

// ---------------------------------------------------------------------------
// batch
// ---------------------------------------------------------------------------
struct mc_batch {
  mc_model* m = nullptr;
  int R = 0, cap = 0, K = 0, K1 = 1, hcap = 0, Mmax = 0;
  mc_spec_config spec{};
  hipStream_t st = nullptr;
  std::vector<KVLayer> kv;
  uint16_t* kv_mem = nullptr;
  float *rope_cos = nullptr, *rope_sin = nullptr;
  uint16_t *x = nullptr, *qkv = nullptr, *q = nullptr, *att = nullptr, *act = nullptr,
           *logits = nullptr;
  float* gemv_part = nullptr;
  unsigned* gemv_cnt = nullptr;
  size_t gemv_part_n = 0;  // floats
  int gemv_cnt_n = 0;
  float* ssq = nullptr;  // [Mmax][hidden / 16]: per-tile sums of squares of the residual stream
  uint16_t* xn = nullptr;  // [Mmax][hidden]: normalised rows for the M > 64 GEMM (allocated when Mmax > 64)
  unsigned long long* amax = nullptr;  // [Mmax][vocab tiles]: greedy argmax partials of the head
  // Qwen3-MoE: normalised rows, router logits, routing, per-pair expert outputs
  uint16_t *moe_xn = nullptr, *moe_logits = nullptr, *moe_act = nullptr;
  float* moe_out = nullptr;   // [Mmax * TK][hidden] down-projection output of each pair
  int32_t* moe_i32 = nullptr; // n_active per layer [L] | act_e [E] | off [E + 1] | pairs, sel [Mmax * TK]
  float* moe_wts = nullptr;   // [Mmax * TK]
  AttnWork aw{};
  unsigned* attn_cnt = nullptr;  // [R * n_kv] split arrivals of the fused attention, zero at rest
  StepState s;
  void* scratch = nullptr;  // one allocation for the small StepState arrays
  size_t scratch_words = 0;
  // the per-row arrays inside `scratch` that a row's state consists of (mc_batch_filter
  // moves them with the row): offset and width in 32-bit words, value of an empty row
  struct RowArr { size_t off; int w; int32_t empty; };
  std::vector<RowArr> row_arrs;
  // pinned staging
  int32_t* h_i32 = nullptr;  // general staging
  size_t h_i32_n = 0;
  int32_t* h_out = nullptr;  // [R*K1 tok | R cnt | R fin | R nprop | R kv_len]
  hipGraphExec_t graph = nullptr;
  hipGraph_t graph_def = nullptr;
  std::vector<int32_t> widths;
  std::vector<int32_t> kv_len_host;
  uint64_t unseeded = 0;
  bool forced_none = true;  // the device's forced accept-length schedule is all -1
  bool uniforms_on = false; // the device reads caller uniforms
  int last_M = 0;           // token slots of the last forward (mc_batch_read_attention)
  int32_t* gen_cnt = nullptr;  // [R][V] generated-token counts (rows with penalties)
  // profiling
  bool profiling = false;
  std::vector<hipEvent_t> ev;
  size_t ev_used = 0;
  struct Rec { int kind; size_t e0, e1; double bytes; };
  std::vector<Rec> recs;
  double prof_ms[3] = {0, 0, 0}, prof_bytes[3] = {0, 0, 0};
  int prof_launch[3] = {0, 0, 0};
};

static void batch_free(mc_batch* b) {
  if (!b) return;
  (void)hipSetDevice(b->m->device);
  if (b->graph) (void)hipGraphExecDestroy(b->graph);
  if (b->graph_def) (void)hipGraphDestroy(b->graph_def);
  for (void* p : {(void*)b->kv_mem, (void*)b->rope_cos, (void*)b->rope_sin, (void*)b->x, (void*)b->qkv,
                  (void*)b->q, (void*)b->att, (void*)b->act, (void*)b->logits, (void*)b->gemv_part,
                  (void*)b->gemv_cnt, (void*)b->ssq, (void*)b->amax, (void*)b->aw.part_o, (void*)b->aw.part_ml, (void*)b->attn_cnt, b->scratch, (void*)b->gen_cnt,
                  (void*)b->moe_xn, (void*)b->moe_logits, (void*)b->moe_act, (void*)b->moe_out, (void*)b->moe_i32,
                  (void*)b->moe_wts, (void*)b->xn})
    if (p) (void)hipFree(p);
  if (b->h_i32) (void)hipHostFree(b->h_i32);
  if (b->h_out) (void)hipHostFree(b->h_out);
  for (auto e : b->ev) (void)hipEventDestroy(e);
  if (b->st) (void)hipStreamDestroy(b->st);
  delete b;
}

extern "C" void mc_batch_destroy(mc_batch* b) { batch_free(b); }

static int stage_i32(mc_batch* b, size_t n) {
  if (n <= b->h_i32_n) return MC_OK;
  if (b->h_i32) MC_HIP(hipHostFree(b->h_i32));
  b->h_i32 = nullptr;
  MC_HIP(hipHostMalloc((void**)&b->h_i32, n * 4, hipHostMallocDefault));
  b->h_i32_n = n;
  return MC_OK;
}

extern "C" int mc_batch_create(mc_model* m, int32_t max_rows, int32_t max_ctx, int32_t max_draft,
                               const mc_spec_config* spec, mc_batch** out) {
  if (!m || !out || !spec) return fail(MC_E_INVALID, "mc_batch_create: null argument");
  if (max_rows <= 0 || max_rows > 1024 || max_ctx <= 1 || max_draft < 0 || max_draft > 64)
    return fail(MC_E_INVALID, "mc_batch_create: bad sizes");
  *out = nullptr;
  MC_HIP(hipSetDevice(m->device));
  auto* b = new mc_batch();
  b->m = m;
  b->spec = *spec;
  if (b->spec.max_proposal_tokens < 0) b->spec.max_proposal_tokens = 0;  // BatchGenerator.swift:23-25
  if (b->spec.max_suffix_tokens < 1) b->spec.max_suffix_tokens = 1;
  if (b->spec.min_context_tokens < 2) b->spec.min_context_tokens = 2;
  if (b->spec.max_proposal_tokens > max_draft) b->spec.max_proposal_tokens = max_draft;
  b->R = max_rows;
  b->cap = max_ctx;
  b->K = b->spec.enabled ? b->spec.max_proposal_tokens : 0;
  b->K1 = b->K + 1;
  b->hcap = max_ctx + b->K1 + 1;
  b->Mmax = std::max(b->R * b->K1, PREFILL_CHUNK);
  b->kv_len_host.assign((size_t)b->R, 0);
  const auto& c = m->cfg;
  int rc = MC_OK;
  MC_HIP(hipStreamCreateWithFlags(&b->st, hipStreamNonBlocking));
  const int V = c.vocab;
  const int M = b->Mmax;
  if (!m->fake) {
    const int H = c.hidden, d = c.head_dim, nq = c.n_q_heads, nkv = c.n_kv_heads, I = c.intermediate;
    const int kcap = (max_ctx + 63) / 64 * 64;  // position stride of the cache
    const size_t per = (size_t)b->R * nkv * (size_t)kcap * d;
    if ((rc = dev_zero(&b->kv_mem, per * 2 * (size_t)c.n_layers))) { batch_free(b); return rc; }
    b->kv.resize((size_t)c.n_layers);
    for (int l = 0; l < c.n_layers; ++l) {
      b->kv[(size_t)l].k = b->kv_mem + per * 2 * (size_t)l;
      b->kv[(size_t)l].v = b->kv_mem + per * (2 * (size_t)l + 1);
      b->kv[(size_t)l].cap = kcap;
    }
    // RoPE table in double precision, rounded to float (shared definition with the oracle)
    const int hd = d / 2;
    std::vector<float> cs((size_t)max_ctx * hd), sn((size_t)max_ctx * hd);
    for (int p = 0; p < max_ctx; ++p)
      for (int i = 0; i < hd; ++i) {
        const double inv = std::pow((double)c.rope_theta, -2.0 * (double)i / (double)d);
        const double a = (double)p * inv;
        cs[(size_t)p * hd + i] = (float)std::cos(a);
        sn[(size_t)p * hd + i] = (float)std::sin(a);
      }
    if ((rc = dev_alloc(&b->rope_cos, cs.size())) || (rc = dev_alloc(&b->rope_sin, sn.size()))) { batch_free(b); return rc; }
    MC_HIP(hipMemcpy(b->rope_cos, cs.data(), cs.size() * 4, hipMemcpyHostToDevice));
    MC_HIP(hipMemcpy(b->rope_sin, sn.data(), sn.size() * 4, hipMemcpyHostToDevice));
    const size_t Nqkv = (size_t)(nq + 2 * nkv) * d;
    if ((rc = dev_zero(&b->x, (size_t)M * H)) ||
        (rc = dev_zero(&b->qkv, (size_t)M * Nqkv)) || (rc = dev_zero(&b->q, (size_t)M * nq * d)) ||
        (rc = dev_zero(&b->att, (size_t)M * nq * d)) || (rc = dev_zero(&b->act, (size_t)M * I))) {
      batch_free(b);
      return rc;
    }
    // split-K workspace: the largest plan over every linear and m-tile class.  Units with
    // a residual epilogue leave a partial here even with one K-range, so every plan counts.
    size_t part = 1;
    int maxnt = 1;
    auto acc_plan = [&](const QLinear& L) {
      for (int MT = 1; MT <= 4; ++MT) {
        int kr, ks;
        gemv_plan(L, MT, &kr, &ks);
        part = std::max(part, (size_t)ks * L.NT * MT * 64 * 4);
      }
      maxnt = std::max(maxnt, L.NT);
      if (M > 64) {  // the large-M GEMM's split-K plans
        size_t qp;
        int qc;
        qgemm_workspace(L.NT, L.GP, M, &qp, &qc);
        part = std::max(part, qp);
        maxnt = std::max(maxnt, qc);
      }
    };
    for (auto& L : m->layers)
      for (const QLinear* q : {&L.qkv, &L.o, &L.gateup, &L.down, &L.router})
        if (q->N > 0) acc_plan(*q);
    acc_plan(m->head());
    b->gemv_part_n = part;
    b->gemv_cnt_n = maxnt;
    if ((rc = dev_alloc(&b->gemv_part, part)) || (rc = dev_zero(&b->gemv_cnt, (size_t)maxnt)) ||
        (rc = dev_zero(&b->ssq, (size_t)(H / 16) * M)) || (M > 64 && (rc = dev_zero(&b->xn, (size_t)M * H))) ||
        (rc = dev_zero(&b->amax, (size_t)M * m->head().NT))) {
      batch_free(b);
      return rc;
    }
    b->aw.nchunk = (max_ctx + ATTN_CHUNK - 1) / ATTN_CHUNK;
    if ((rc = dev_alloc(&b->aw.part_o, (size_t)M * nq * b->aw.nchunk * d)) ||
        (rc = dev_alloc(&b->aw.part_ml, (size_t)M * nq * b->aw.nchunk * 2)) ||
        (rc = dev_zero(&b->attn_cnt, (size_t)b->R * nkv))) {
      batch_free(b);
      return rc;
    }
    if (m->moe()) {
      const size_t E = (size_t)c.n_experts, P = (size_t)M * c.n_experts_per_tok;
      if ((rc = dev_zero(&b->moe_xn, (size_t)M * H)) || (rc = dev_zero(&b->moe_logits, (size_t)M * E)) ||
          (rc = dev_zero(&b->moe_act, P * c.moe_intermediate)) || (rc = dev_zero(&b->moe_out, P * H)) ||
          (rc = dev_zero(&b->moe_i32, (size_t)c.n_layers + 2 * E + 1 + 2 * P + 64 * E)) || (rc = dev_zero(&b->moe_wts, P))) {
        batch_free(b);
        return rc;
      }
    }
  }
  if ((rc = dev_zero(&b->logits, (size_t)M * V))) { batch_free(b); return rc; }

  // small per-row state in one zeroed allocation
  StepState& s = b->s;
  s.R = b->R; s.K = b->K; s.K1 = b->K1; s.hcap = b->hcap; s.V = V;
  s.enabled = b->spec.enabled; s.max_suffix = b->spec.max_suffix_tokens; s.min_ctx = b->spec.min_context_tokens;
  s.acceptance = b->spec.acceptance; s.single_row_only = b->spec.single_row_only; s.greedy_only = b->spec.greedy_only;
  const size_t R = (size_t)b->R, RK = R * b->K1, Ms = (size_t)M;
  size_t words = 0;
  auto take = [&](size_t n) { size_t o = words; words += (n + 1) & ~(size_t)1; return o; };  // 8-byte aligned in u32 units
  const size_t o_active = take(R), o_hist = take(R * b->hcap), o_hlen = take(R), o_gen = take(R), o_max = take(R),
               o_cur = take(R), o_temp = take(R), o_topp = take(R), o_invt = take(R),
               o_hseed = take(R), o_seed = take(2 * R), o_ctr = take(2 * R), o_eos = take(8 * R), o_neos = take(R),
               o_rej = take(R), o_dr = take(RK), o_stok = take(Ms), o_srow = take(Ms),
               o_spos = take(Ms), o_rs0 = take(R), o_nv = take(R), o_qb = take(R), o_sct = take(RK),
               o_sca = take(RK), o_scr = take(RK), o_forced = take(R), o_stats = take(8),
               o_topk = take(R), o_mpl = take(R), o_rp = take(R), o_pp = take(R), o_fp = take(R),
               o_mint = take(R), o_nb = take(R), o_bt = take(16 * R), o_bv = take(16 * R), o_proc = take(R),
               o_uni = take(2 * RK), o_useu = take(2), o_dext = take(R),
               // what a step returns, contiguous so that one copy brings it to the host:
               // [RK tokens | R counts | R finish | R proposal lengths | R KV lengths]
               o_otok = take(RK + 4 * R), o_ocnt = o_otok + RK, o_ofin = o_ocnt + R, o_np = o_ofin + R,
               o_kv = o_np + R;
  uint32_t* base;
  if ((rc = dev_zero(&base, words))) { batch_free(b); return rc; }
  b->scratch = base;
  b->scratch_words = words;
  for (auto [o, w] : {std::pair<size_t, int>{o_active, 1}, {o_hist, b->hcap}, {o_hlen, 1}, {o_gen, 1}, {o_max, 1},
                      {o_cur, 1}, {o_temp, 1}, {o_topp, 1}, {o_invt, 1}, {o_hseed, 1}, {o_seed, 2}, {o_ctr, 2},
                      {o_eos, 8}, {o_neos, 1}, {o_topk, 1}, {o_mpl, 1}, {o_rp, 1}, {o_pp, 1}, {o_fp, 1},
                      {o_mint, 1}, {o_nb, 1}, {o_bt, 16}, {o_bv, 16}, {o_proc, 1}, {o_kv, 1}})
    b->row_arrs.push_back({o, w, 0});
  b->row_arrs.push_back({o_rej, 1, -1});
  b->row_arrs.push_back({o_forced, 1, -1});
  auto I32 = [&](size_t o) { return reinterpret_cast<int32_t*>(base + o); };
  s.active = I32(o_active); s.hist = I32(o_hist); s.hist_len = I32(o_hlen); s.gen = I32(o_gen); s.max_gen = I32(o_max);
  s.cur = I32(o_cur); s.kv_len = I32(o_kv); s.temp = reinterpret_cast<float*>(base + o_temp);
  s.top_p = reinterpret_cast<float*>(base + o_topp); s.inv_temp = reinterpret_cast<float*>(base + o_invt);
  s.has_seed = I32(o_hseed); s.seed = reinterpret_cast<uint64_t*>(base + o_seed);
  s.counter = reinterpret_cast<uint64_t*>(base + o_ctr); s.eos = I32(o_eos); s.n_eos = I32(o_neos);
  s.reject = I32(o_rej); s.drafts = I32(o_dr); s.nprop = I32(o_np); s.slot_tok = I32(o_stok);
  s.slot_row = I32(o_srow); s.slot_pos = I32(o_spos); s.row_slot0 = I32(o_rs0); s.n_valid = I32(o_nv);
  s.qbase = I32(o_qb); s.scan_tok = I32(o_sct); s.scan_acc = I32(o_sca); s.scan_res = I32(o_scr);
  s.forced = I32(o_forced); s.out_tok = I32(o_otok); s.out_cnt = I32(o_ocnt); s.out_fin = I32(o_ofin);
  s.stats = reinterpret_cast<unsigned long long*>(base + o_stats);
  auto F32 = [&](size_t o) { return reinterpret_cast<float*>(base + o); };
  s.top_k = I32(o_topk); s.min_p_log = F32(o_mpl); s.rep_pen = F32(o_rp); s.pres_pen = F32(o_pp);
  s.freq_pen = F32(o_fp); s.min_tokens = I32(o_mint); s.n_bias = I32(o_nb); s.bias_tok = I32(o_bt);
  s.bias_val = F32(o_bv); s.proc = I32(o_proc);
  s.uniforms = reinterpret_cast<const uint32_t*>(base + o_uni); s.use_uniforms = I32(o_useu); s.dext = I32(o_dext);
  if ((rc = dev_zero(&b->gen_cnt, R * (size_t)V))) { batch_free(b); return rc; }
  s.gen_cnt = b->gen_cnt;
  if (!m->fake) { s.amax = b->amax; s.amax_nt = m->head().NT; }
  // forced = -1 (none), reject = -1
  {
    std::vector<int32_t> neg(R, -1);
    MC_HIP(hipMemcpy(s.forced, neg.data(), R * 4, hipMemcpyHostToDevice));
    MC_HIP(hipMemcpy(s.reject, neg.data(), R * 4, hipMemcpyHostToDevice));
  }
  if ((rc = stage_i32(b, std::max<size_t>(4096, (size_t)b->hcap + 16)))) { batch_free(b); return rc; }
  MC_HIP(hipHostMalloc((void**)&b->h_out, (RK + 4 * R) * 4, hipHostMallocDefault));
  *out = b;
  return MC_OK;
}

// --------------------------- forward --------------------------------------
static int prof_begin(mc_batch* b, size_t* e0) {
  if (!b->profiling) return MC_OK;
  if (b->ev_used + 2 > b->ev.size()) {
    for (int i = 0; i < 64; ++i) {
      hipEvent_t e;
      MC_HIP(hipEventCreate(&e));
      b->ev.push_back(e);
    }
  }
  *e0 = b->ev_used++;
  MC_HIP(hipEventRecord(b->ev[*e0], b->st));
  return MC_OK;
}
static int prof_end(mc_batch* b, size_t e0, int kind, double bytes) {
  if (!b->profiling) return MC_OK;
  const size_t e1 = b->ev_used++;
  MC_HIP(hipEventRecord(b->ev[e1], b->st));
  b->recs.push_back({kind, e0, e1, bytes});
  return MC_OK;
}
// One GEMV / GEMM kernel timed by its own launch (start and end of its execution, not the
// dispatch gap before it): the next such launch on this thread records into two events.
static int prof_kernel(mc_batch* b, int kind, double bytes) {
  if (!b->profiling) return MC_OK;
  if (b->ev_used + 2 > b->ev.size()) {
    for (int i = 0; i < 64; ++i) {
      hipEvent_t e;
      MC_HIP(hipEventCreate(&e));
      b->ev.push_back(e);
    }
  }
  const size_t e0 = b->ev_used++, e1 = b->ev_used++;
  gemv_time_next_launch(b->ev[e0], b->ev[e1]);
  b->recs.push_back({kind, e0, e1, bytes});
  return MC_OK;
}

// Algorithmic HBM bytes of one forward over M slots: every linear's packed weights
// (0.5625 B per weight), the cached K/V read, the new K/V written, the bf16 logits.
static double forward_alg_bytes(const mc_batch* b, int M, bool with_head) {
  const mc_model* m = b->m;
  const auto& c = m->cfg;
  double w = 0;
  for (const auto& L : m->layers) w += L.qkv.alg_bytes() + L.o.alg_bytes() + L.gateup.alg_bytes() + L.down.alg_bytes();
  if (with_head) w += m->head().alg_bytes() + (double)M * c.vocab * 2;
  double ctx = 0;
  for (int r = 0; r < b->R; ++r) ctx += b->kv_len_host[(size_t)r];
  const double kv_row = (double)c.n_layers * 2 * c.n_kv_heads * c.head_dim * 2;
  return w + ctx * kv_row + (double)M * kv_row;
}

// One linear over M tokens, in launches of at most 64.  norm_w: the input rows are the
// residual stream b->x, RMS-normalised with these weights inside the linear from the
// per-tile sums of squares in b->ssq (rows ss_m0 ...).  EPI_RESIDUAL writes the new rows'
// sums of squares to b->ssq.
static int run_gemv(mc_batch* b, const QLinear& L, const uint16_t* x, int ldx, const uint16_t* norm_w, uint16_t* y,
                    int ldy, int M, int epi, int ss_m0 = 0, unsigned long long* amax = nullptr) {
  const auto& c = b->m->cfg;
  const int H = c.hidden;
  if (M > 64) {  // one GEMM over every token (the input rows normalised first when the linear has a norm)
    const uint16_t* xin = x;
    int ldxin = ldx;
    int rc;
    if (norm_w) {
      if ((rc = launch_rows_rmsnorm(x, norm_w, M, H, c.rms_eps, b->xn, b->st))) return rc;
      xin = b->xn;
      ldxin = H;
    }
    GemvArgs a;
    a.qw = L.qw; a.sb = L.sb;
    a.x = xin; a.ldx = ldxin;
    if (epi == EPI_RESIDUAL) {
      a.ss_out = b->ssq + (size_t)ss_m0 * (H / 16); a.ss_ld_out = H / 16;
    }
    a.y = y; a.ldy = ldy;
    a.M = M; a.N = L.N; a.K = L.K; a.NT = L.NT; a.GP = L.GP;
    a.epi = epi;
    a.amax = amax;
    a.part = b->gemv_part; a.part_floats = b->gemv_part_n;
    a.counters = b->gemv_cnt; a.counters_n = b->gemv_cnt_n;
    if ((rc = prof_kernel(b, 0, L.alg_bytes()))) return rc;
    rc = qgemm_launch(a, b->st);
    gemv_time_next_launch(nullptr, nullptr);  // consumed by the launch, or dropped on an error
    return rc;
  }
  for (int m0 = 0; m0 < M; m0 += 64) {
    const int mc = std::min(64, M - m0);
    const int MT = (mc + 15) / 16;
    GemvArgs a;
    a.qw = L.qw; a.sb = L.sb;
    a.x = x + (size_t)m0 * ldx; a.ldx = ldx;
    if (norm_w) {
      a.norm_w = norm_w;
      a.ss_in = b->ssq + (size_t)(ss_m0 + m0) * (H / 16); a.ss_nt = H / 16; a.ss_ld = H / 16; a.eps = c.rms_eps;
    }
    if (epi == EPI_RESIDUAL) {
      a.ss_out = b->ssq + (size_t)(ss_m0 + m0) * (H / 16); a.ss_ld_out = H / 16;
    }
    a.y = y + (size_t)m0 * ldy; a.ldy = ldy;
    a.M = mc; a.N = L.N; a.K = L.K; a.NT = L.NT; a.GP = L.GP;
    gemv_plan(L, MT, &a.kr, &a.ksplit);
    a.part = b->gemv_part; a.part_floats = b->gemv_part_n;
    a.counters = b->gemv_cnt; a.counters_n = b->gemv_cnt_n; a.epi = epi;
    if (amax) a.amax = amax + (size_t)m0 * L.NT;
    int rc = prof_kernel(b, 0, L.alg_bytes());
    if (rc) return rc;
    rc = gemv_launch(a, MT, b->st);
    gemv_time_next_launch(nullptr, nullptr);
    if (rc) return rc;
  }
  return MC_OK;
}

// Routing of layer l: its touched-expert count stays at moe_i32[l] (read back for the
// byte count of a profiled step); the lists are rewritten by every layer.
static MoeRoute moe_route_of(mc_batch* b, int l) {
  const auto& c = b->m->cfg;
  const size_t E = (size_t)c.n_experts, P = (size_t)b->Mmax * c.n_experts_per_tok;
  int32_t* p = b->moe_i32;
  MoeRoute rt;
  rt.n_active = p + l;
  p += c.n_layers;
  rt.act_e = p; p += E;
  rt.off = p; p += E + 1;
  rt.pairs = p; p += P;
  rt.sel = p; p += P;
  rt.slot_pairs = p;
  rt.wts = b->moe_wts;
  return rt;
}

// Blocks per touched expert: 4 of its 16-row tiles per block (one per wave).  Qwen3-30B-A3B
// shape, 4 rows x 5 tokens, per step: 4 tiles 7.24 ms, 8 tiles 7.69, 2 tiles 7.71, 16 tiles 9.25.
static int moe_blocks_per_expert(const QLinear& L) { return std::max(1, std::min(L.NT, (L.NT + 3) / 4)); }

// The Qwen3-MoE MLP of layer l over M tokens (Qwen3MoeSparseMoeBlock, EXTERNAL to the
// reference tree): post-attention RMSNorm, router, softmax top-k with renormalised weights,
// each touched expert's SwiGLU MLP over its tokens, the weighted sum added to the residual.
static int moe_mlp(mc_batch* b, int l, int M) {
  const mc_model* m = b->m;
  const auto& c = m->cfg;
  const auto& L = m->layers[(size_t)l];
  const int H = c.hidden, E = c.n_experts, TK = c.n_experts_per_tok, MI = c.moe_intermediate;
  int rc;
  for (int m0 = 0; m0 < M; m0 += 64) {
    const int mc = std::min(64, M - m0);
    uint16_t* x = b->x + (size_t)m0 * H;
    if ((rc = launch_rows_rmsnorm(x, L.post_norm, mc, H, c.rms_eps, b->moe_xn, b->st))) return rc;
    if ((rc = run_gemv(b, L.router, b->moe_xn, H, nullptr, b->moe_logits, E, mc, EPI_STORE))) return rc;
    const MoeRoute rt = moe_route_of(b, l);
    if ((rc = launch_moe_route(b->moe_logits, mc, E, TK, rt, b->st))) return rc;
    size_t e0 = 0;
    if ((rc = prof_begin(b, &e0))) return rc;
    MoeGemvArgs a;
    a.rt = rt;
    a.max_active = std::min(E, mc * TK);
    a.qw = L.egu.qw; a.sb = L.egu.sb; a.qw_es = L.egu.qw_words(); a.sb_es = L.egu.sb_words();
    a.N = L.egu.N; a.K = L.egu.K; a.NT = L.egu.NT; a.GP = L.egu.GP;
    a.x = b->moe_xn; a.ldx = H; a.x_div = TK;
    a.epi = EPI_SWIGLU; a.y = b->moe_act; a.ldy = MI;
    a.nb = moe_blocks_per_expert(L.egu);
    if ((rc = moe_gemv_launch(a, b->st))) return rc;
    a.qw = L.edn.qw; a.sb = L.edn.sb; a.qw_es = L.edn.qw_words(); a.sb_es = L.edn.sb_words();
    a.N = L.edn.N; a.K = L.edn.K; a.NT = L.edn.NT; a.GP = L.edn.GP;
    a.x = b->moe_act; a.ldx = MI; a.x_div = 1;
    a.epi = EPI_STORE; a.y = nullptr; a.yf = b->moe_out; a.ldy = H;
    a.nb = moe_blocks_per_expert(L.edn);
    if ((rc = moe_gemv_launch(a, b->st))) return rc;
    if ((rc = prof_end(b, e0, 0, 0.0))) return rc;
    if ((rc = launch_moe_combine(x, b->moe_out, rt.wts, mc, TK, H, b->ssq + (size_t)m0 * (H / 16), b->st))) return rc;
  }
  return MC_OK;
}

// Forward over M slots already described in the StepState slot arrays.  Logits are
// produced for slots [lg0, lg0 + lgn) into b->logits rows [lg0, lg0 + lgn).
static int forward_slots(mc_batch* b, int M, int max_q, int lg0, int lgn) {
  mc_model* m = b->m;
  const auto& c = m->cfg;
  const StepState& s = b->s;
  int rc;
  b->last_M = m->fake ? 0 : M;
  if (m->fake) {
    if (lgn > 0) return launch_fake_logits(c.arch, s.slot_tok + lg0, lgn, c.vocab, b->logits + (size_t)lg0 * c.vocab, b->st);
    return MC_OK;
  }
  const int H = c.hidden, d = c.head_dim, nq = c.n_q_heads, nkv = c.n_kv_heads, I = c.intermediate;
  const int Nqkv = (nq + 2 * nkv) * d;
  SlotView sv{s.slot_tok, s.slot_row, s.slot_pos, s.row_slot0, s.n_valid, s.qbase};
  // Attention with the q/k preparation and the split merge inside (one launch per layer
  // instead of three) whenever a row's queries of one kv head fit its query buffer, except
  // for many (row, kv head) pairs over short splits: every split block repeats its queries'
  // preparation, which at 64 pairs x 512-key splits costs more than the two launches it
  // saves (8 rows, K = 5: 5.30 ms fused against 5.03 ms per step; 8 Llama-3-8B rows: 6.50
  // against 6.30), while 32 rows x 16K keys (4160-key splits) and a single row gain from it.
  const int S_attn = attn_split(b->R, nkv, b->aw.nchunk, true);
  const bool fuse = attn_fuse_ok(b->R, nkv, b->aw.nchunk, max_q, nq, d) && (b->R * nkv < 64 || S_attn >= 16);
  if ((rc = launch_embed(m->embed, s.slot_tok, M, H, b->x, b->ssq, H / 16, b->st)))
    return rc;
  for (int l = 0; l < c.n_layers; ++l) {
    const auto& L = m->layers[(size_t)l];
    if ((rc = run_gemv(b, L.qkv, b->x, H, L.in_norm, b->qkv, Nqkv, M, EPI_STORE))) return rc;
    AttnFuse fz;
    if (fuse) {
      fz.qkv = b->qkv; fz.q_norm = L.q_norm; fz.k_norm = L.k_norm; fz.rope_cos = b->rope_cos; fz.rope_sin = b->rope_sin;
      fz.eps = c.rms_eps; fz.counters = b->attn_cnt; fz.att = b->att;
    } else if ((rc = launch_qk_rope_append(b->qkv, L.q_norm, L.k_norm, b->rope_cos, b->rope_sin, M, nq, nkv, d, c.rms_eps,
                                           s.slot_row, s.slot_pos, b->kv[(size_t)l], b->q, b->st))) {
      return rc;
    }
    size_t e0 = 0;
    if ((rc = prof_begin(b, &e0))) return rc;
    if ((rc = launch_attention(b->q, b->kv[(size_t)l], sv, b->R, max_q, nq, nkv, d, M, b->aw, fuse ? &fz : nullptr, b->att,
                               b->st)))
      return rc;
    if ((rc = prof_end(b, e0, 1, 0.0))) return rc;
    if ((rc = run_gemv(b, L.o, b->att, nq * d, nullptr, b->x, H, M, EPI_RESIDUAL))) return rc;
    if (m->moe()) {
      if ((rc = moe_mlp(b, l, M))) return rc;
      continue;
    }
    if ((rc = run_gemv(b, L.gateup, b->x, H, L.post_norm, b->act, I, M, EPI_SWIGLU))) return rc;
    if ((rc = run_gemv(b, L.down, b->act, I, nullptr, b->x, H, M, EPI_RESIDUAL))) return rc;
  }
  if (lgn > 0) {
    if ((rc = run_gemv(b, m->head(), b->x + (size_t)lg0 * H, H, m->final_norm, b->logits + (size_t)lg0 * c.vocab, c.vocab, lgn,
                       EPI_STORE, lg0, b->amax + (size_t)lg0 * m->head().NT)))
      return rc;
  }
  return MC_OK;
}

static int upload_i32(mc_batch* b, int32_t* dst, const int32_t* src, size_t n) {
  int rc = stage_i32(b, n);
  if (rc) return rc;
  MC_HIP(hipStreamSynchronize(b->st));  // staging buffer reuse
  memcpy(b->h_i32, src, n * 4);
  MC_HIP(hipMemcpyAsync(dst, b->h_i32, n * 4, hipMemcpyHostToDevice, b->st));
  MC_HIP(hipStreamSynchronize(b->st));
  return MC_OK;
}

// Describe counts[i] new tokens of rows[i] as slots (packed), with qbase = kv_len.
static int set_slots(mc_batch* b, int nrows, const int32_t* rows, const int32_t* counts, const int32_t* tokens, int* M) {
  const int R = b->R;
  int total = 0;
  for (int i = 0; i < nrows; ++i) total += counts[i];
  std::vector<int32_t> tok((size_t)total), row((size_t)total), pos((size_t)total), rs0((size_t)R, 0), nv((size_t)R, 0),
      qb((size_t)R, 0);
  for (int r = 0; r < R; ++r) qb[(size_t)r] = b->kv_len_host[(size_t)r];
  int o = 0;
  for (int i = 0; i < nrows; ++i) {
    const int r = rows[i];
    rs0[(size_t)r] = o;
    nv[(size_t)r] = counts[i];
    for (int j = 0; j < counts[i]; ++j, ++o) {
      tok[(size_t)o] = tokens[o];
      row[(size_t)o] = r;
      pos[(size_t)o] = b->kv_len_host[(size_t)r] + j;
    }
  }
  int rc;
  if ((rc = upload_i32(b, b->s.slot_tok, tok.data(), tok.size()))) return rc;
  if ((rc = upload_i32(b, b->s.slot_row, row.data(), row.size()))) return rc;
  if ((rc = upload_i32(b, b->s.slot_pos, pos.data(), pos.size()))) return rc;
  if ((rc = upload_i32(b, b->s.row_slot0, rs0.data(), rs0.size()))) return rc;
  if ((rc = upload_i32(b, b->s.n_valid, nv.data(), nv.size()))) return rc;
  if ((rc = upload_i32(b, b->s.qbase, qb.data(), qb.size()))) return rc;
  *M = total;
  return MC_OK;
}

static int set_row_i32(mc_batch* b, int32_t* arr, int row, int32_t v) { return upload_i32(b, arr + row, &v, 1); }

static int sync_kv_len(mc_batch* b) {
  MC_HIP(hipStreamSynchronize(b->st));
  MC_HIP(hipMemcpy(b->kv_len_host.data(), b->s.kv_len, (size_t)b->R * 4, hipMemcpyDeviceToHost));
  return MC_OK;
}

extern "C" int mc_forward(mc_batch* b, int32_t nrows, const int32_t* rows, const int32_t* counts,
                          const int32_t* tokens, uint16_t* logits_host) {
  if (!b || (nrows > 0 && (!rows || !counts || !tokens))) return fail(MC_E_INVALID, "mc_forward: null argument");
  MC_HIP(hipSetDevice(b->m->device));
  int rc = sync_kv_len(b);
  if (rc) return rc;
  int total = 0;
  std::vector<int> seen((size_t)b->R, 0);
  for (int i = 0; i < nrows; ++i) {
    const int r = rows[i];
    if (r < 0 || r >= b->R || seen[(size_t)r]++) return fail(MC_E_INVALID, "mc_forward: bad or repeated row");
    if (counts[i] < 0) return fail(MC_E_INVALID, "mc_forward: negative count");
    if (b->kv_len_host[(size_t)r] + counts[i] > b->cap) return fail(MC_E_CAPACITY, "mc_forward: context capacity exceeded");
    total += counts[i];
  }
  if (total == 0) return MC_OK;
  if (total > b->Mmax) return fail(MC_E_CAPACITY, "mc_forward: too many tokens for one call");
  int M;
  if ((rc = set_slots(b, nrows, rows, counts, tokens, &M))) return rc;
  int maxq = 0;
  for (int i = 0; i < nrows; ++i) maxq = std::max(maxq, (int)counts[i]);
  if ((rc = forward_slots(b, M, maxq, 0, logits_host ? M : 0))) return rc;
  // advance kv_len
  for (int i = 0; i < nrows; ++i) b->kv_len_host[(size_t)rows[i]] += counts[i];
  if ((rc = upload_i32(b, b->s.kv_len, b->kv_len_host.data(), (size_t)b->R))) return rc;
  if (logits_host) {
    MC_HIP(hipMemcpyAsync(logits_host, b->logits, (size_t)M * b->m->cfg.vocab * 2, hipMemcpyDeviceToHost, b->st));
  }
  MC_HIP(hipStreamSynchronize(b->st));
  return MC_OK;
}

// --------------------------- admission ------------------------------------
// Host image of one row's sampler options, validated (mc_sampling in include/mlxcat_hip.h).
struct RowSampling {
  float temp = 0.f, top_p = 0.f, inv_t = 0.f, min_p_log = -INFINITY, rp = 1.f, pp = 0.f, fp = 0.f;
  int32_t top_k = 0, min_tokens = 0, n_bias = 0, proc = 0, n_eos = 0;
  int32_t bias_tok[16] = {0};
  float bias_val[16] = {0};
  int32_t eos[8] = {0};
};

static int row_sampling(const mc_sampling* sp, int V, RowSampling* o) {
  const float vals[] = {sp->temperature, sp->top_p, sp->min_p, sp->repetition_penalty, sp->presence_penalty,
                        sp->frequency_penalty};
  for (float v : vals)
    if (!std::isfinite(v)) return fail(MC_E_INVALID, "sampling: non-finite parameter");
  if (sp->temperature < 0.f || sp->top_k < 0 || sp->min_p < 0.f || sp->min_p > 1.f || sp->repetition_penalty < 0.f ||
      sp->n_bias < 0 || sp->n_bias > 16)
    return fail(MC_E_INVALID, "sampling: parameter out of range");
  for (int i = 0; i < sp->n_bias; ++i)
    if (!std::isfinite(sp->bias_value[i])) return fail(MC_E_INVALID, "sampling: non-finite logit bias");
  o->temp = sp->temperature;
  o->top_p = sp->top_p;
  o->inv_t = sp->temperature != 0.0f ? 1.0f / sp->temperature : 0.0f;
  o->top_k = sp->top_k;
  o->min_p_log = sp->min_p > 0.0f ? logf(sp->min_p) : -INFINITY;
  o->rp = sp->repetition_penalty == 0.0f ? 1.0f : sp->repetition_penalty;
  o->pp = sp->presence_penalty;
  o->fp = sp->frequency_penalty;
  o->min_tokens = std::max(0, sp->min_tokens);
  o->n_eos = std::max(0, std::min(8, sp->n_eos));
  for (int i = 0; i < o->n_eos; ++i) o->eos[i] = sp->eos[i];
  for (int i = 0; i < sp->n_bias; ++i)  // ids outside the vocabulary are ignored (Sampling.swift:698)
    if (sp->bias_token[i] >= 0 && sp->bias_token[i] < V) {
      o->bias_tok[o->n_bias] = sp->bias_token[i];
      o->bias_val[o->n_bias++] = sp->bias_value[i];
    }
  o->proc = (o->n_bias > 0 ? 1 : 0) | (o->min_tokens > 0 && o->n_eos > 0 ? 2 : 0) |
            (o->rp != 1.0f || o->pp != 0.0f || o->fp != 0.0f ? 4 : 0);
  return MC_OK;
}

static int set_row_f32(mc_batch* b, float* arr, int row, float v) {
  int32_t w;
  memcpy(&w, &v, 4);
  return upload_i32(b, reinterpret_cast<int32_t*>(arr) + row, &w, 1);
}

// Per-row sampler state; `counted` are the tokens generated so far (the penalties' counts).
static int set_row_sampling(mc_batch* b, int row, const mc_sampling* sp, const int32_t* counted, int n_counted) {
  StepState& s = b->s;
  RowSampling q;
  int rc;
  if ((rc = row_sampling(sp, s.V, &q))) return rc;
  if ((rc = set_row_f32(b, s.temp, row, q.temp))) return rc;
  if ((rc = set_row_f32(b, s.top_p, row, q.top_p))) return rc;
  if ((rc = set_row_f32(b, s.inv_temp, row, q.inv_t))) return rc;
  if ((rc = set_row_i32(b, s.has_seed, row, sp->has_seed ? 1 : 0))) return rc;
  // unseeded rows: a per-batch stream keyed by admission order (global seed 7)
  const uint64_t seed = sp->has_seed ? sp->seed : mix64(7ull ^ mix64(++b->unseeded));
  int32_t rowv[4];
  const uint64_t two[2] = {seed, 0};
  memcpy(rowv, two, 16);
  if ((rc = upload_i32(b, reinterpret_cast<int32_t*>(s.seed + row), rowv, 2))) return rc;
  if ((rc = upload_i32(b, reinterpret_cast<int32_t*>(s.counter + row), rowv + 2, 2))) return rc;
  if ((rc = upload_i32(b, s.eos + row * 8, q.eos, 8))) return rc;
  if ((rc = set_row_i32(b, s.n_eos, row, q.n_eos))) return rc;
  if ((rc = set_row_i32(b, s.reject, row, sp->reject_token))) return rc;
  if ((rc = set_row_i32(b, s.top_k, row, q.top_k))) return rc;
  if ((rc = set_row_f32(b, s.min_p_log, row, q.min_p_log))) return rc;
  if ((rc = set_row_f32(b, s.rep_pen, row, q.rp))) return rc;
  if ((rc = set_row_f32(b, s.pres_pen, row, q.pp))) return rc;
  if ((rc = set_row_f32(b, s.freq_pen, row, q.fp))) return rc;
  if ((rc = set_row_i32(b, s.min_tokens, row, q.min_tokens))) return rc;
  if ((rc = set_row_i32(b, s.n_bias, row, q.n_bias))) return rc;
  if ((rc = upload_i32(b, s.bias_tok + row * 16, q.bias_tok, 16))) return rc;
  int32_t bv[16];
  memcpy(bv, q.bias_val, sizeof bv);
  if ((rc = upload_i32(b, reinterpret_cast<int32_t*>(s.bias_val) + row * 16, bv, 16))) return rc;
  if ((rc = set_row_i32(b, s.proc, row, q.proc))) return rc;
  if (q.proc & 4) {  // the row's generated-token counts
    std::vector<int32_t> c((size_t)s.V, 0);
    for (int i = 0; i < n_counted; ++i)
      if (counted[i] >= 0 && counted[i] < s.V) c[(size_t)counted[i]]++;
    if ((rc = upload_i32(b, b->gen_cnt + (size_t)row * s.V, c.data(), c.size()))) return rc;
  }
  return MC_OK;
}

static int check_row(mc_batch* b, int row) {
  if (row < 0 || row >= b->R) return fail(MC_E_INVALID, "row out of range");
  return MC_OK;
}

// Admission with the first n_cached prompt positions' K/V already in the row (0: none).
static int insert_row(mc_batch* b, int32_t row, const int32_t* prompt, int32_t n_prompt, int32_t n_cached,
                      int32_t max_tokens, const mc_sampling* sp, int32_t* first_token, int32_t* finished) {
  if (!b || !prompt || !sp || n_prompt < 1 || max_tokens < 1) return fail(MC_E_INVALID, "mc_batch_insert: bad argument");
  int rc = check_row(b, row);
  if (rc) return rc;
  if (n_cached < 0 || n_cached >= n_prompt)
    return fail(MC_E_INVALID, "mc_batch_insert: n_cached must lie in [0, n_prompt - 1]");
  if ((size_t)n_prompt + (size_t)max_tokens + (size_t)b->K1 + 1 > (size_t)b->cap)
    return fail(MC_E_CAPACITY, "mc_batch_insert: prompt + max_tokens exceeds the context capacity");
  MC_HIP(hipSetDevice(b->m->device));
  if ((rc = sync_kv_len(b))) return rc;
  if (n_cached > 0 && (b->m->fake || b->kv_len_host[(size_t)row] != n_cached))
    return fail(MC_E_STATE, "mc_batch_insert: the row's K/V length must equal n_cached");
  StepState& s = b->s;
  const int V = b->m->cfg.vocab;
  for (int i = 0; i < n_prompt; ++i)
    if (prompt[i] < 0 || prompt[i] >= V) return fail(MC_E_INVALID, "mc_batch_insert: token id out of range");
  if ((rc = set_row_i32(b, s.active, row, 0))) return rc;
  b->kv_len_host[(size_t)row] = n_cached;
  // prefill all but the last prompt token (Scheduler.swift:722-739), in chunks; a prefix hit
  // resumes at the matched count (Scheduler.swift:960-990, prefillRange matched ..< count)
  int done = n_cached;
  while (done < n_prompt - 1) {
    const int cnt = std::min(PREFILL_CHUNK, n_prompt - 1 - done);
    int M;
    if ((rc = set_slots(b, 1, &row, &cnt, prompt + done, &M))) return rc;
    if ((rc = forward_slots(b, M, cnt, 0, 0))) return rc;
    b->kv_len_host[(size_t)row] += cnt;
    done += cnt;
  }
  if (n_prompt - 1 > n_cached) b->widths.push_back(1);
  // last prompt token with logits, then first-token sampling through the acceptance kernels
  {
    const int one = 1;
    int M;
    if ((rc = set_slots(b, 1, &row, &one, prompt + n_prompt - 1, &M))) return rc;
    if ((rc = forward_slots(b, M, 1, 0, 1))) return rc;
  }
  if ((rc = upload_i32(b, s.hist + (size_t)row * b->hcap, prompt, (size_t)n_prompt))) return rc;
  if ((rc = set_row_i32(b, s.hist_len, row, n_prompt))) return rc;
  if ((rc = set_row_i32(b, s.gen, row, 0))) return rc;
  if ((rc = set_row_i32(b, s.max_gen, row, max_tokens))) return rc;
  if ((rc = set_row_i32(b, s.cur, row, prompt[n_prompt - 1]))) return rc;
  if ((rc = set_row_i32(b, s.kv_len, row, n_prompt - 1))) return rc;
  if ((rc = set_row_i32(b, s.nprop, row, 0))) return rc;
  if ((rc = set_row_sampling(b, row, sp, nullptr, 0))) return rc;
  if ((rc = set_row_i32(b, s.active, row, 1))) return rc;
  if ((rc = launch_accept_scan(s, b->logits, row, b->st))) return rc;
  if ((rc = launch_commit(s, row, b->st))) return rc;
  int32_t res[2];
  MC_HIP(hipMemcpyAsync(&res[0], s.out_tok + (size_t)row * b->K1, 4, hipMemcpyDeviceToHost, b->st));
  MC_HIP(hipMemcpyAsync(&res[1], s.out_fin + row, 4, hipMemcpyDeviceToHost, b->st));
  MC_HIP(hipStreamSynchronize(b->st));
  b->kv_len_host[(size_t)row] = n_prompt;
  if (first_token) *first_token = res[0];
  if (finished) *finished = res[1];
  return MC_OK;
}

extern "C" int mc_batch_insert(mc_batch* b, int32_t row, const int32_t* prompt, int32_t n_prompt, int32_t max_tokens,
                               const mc_sampling* sp, int32_t* first_token, int32_t* finished) {
  return insert_row(b, row, prompt, n_prompt, 0, max_tokens, sp, first_token, finished);
}

extern "C" int mc_batch_insert_cached(mc_batch* b, int32_t row, const int32_t* prompt, int32_t n_prompt,
                                      int32_t n_cached, int32_t max_tokens, const mc_sampling* sp,
                                      int32_t* first_token, int32_t* finished) {
  return insert_row(b, row, prompt, n_prompt, n_cached, max_tokens, sp, first_token, finished);
}

extern "C" int mc_batch_fill_synthetic_kv(mc_batch* b, int32_t row, int32_t n, uint64_t seed) {
  if (!b) return fail(MC_E_INVALID, "null batch");
  int rc = check_row(b, row);
  if (rc) return rc;
  if (n < 0 || n > b->cap) return fail(MC_E_CAPACITY, "fill_synthetic_kv: n exceeds capacity");
  MC_HIP(hipSetDevice(b->m->device));
  const auto& c = b->m->cfg;
  if (!b->m->fake)
    for (int l = 0; l < c.n_layers; ++l)
      if ((rc = launch_kv_synth(b->kv[(size_t)l], l, row, c.n_kv_heads, c.head_dim, n, seed, b->st))) return rc;
  if ((rc = set_row_i32(b, b->s.kv_len, row, n))) return rc;
  b->kv_len_host[(size_t)row] = n;
  MC_HIP(hipStreamSynchronize(b->st));
  return MC_OK;
}

extern "C" int mc_batch_insert_prefilled(mc_batch* b, int32_t row, const int32_t* ctx, int32_t n_ctx,
                                         int32_t max_tokens, const mc_sampling* sp) {
  if (!b || !ctx || !sp || n_ctx < 1 || max_tokens < 1) return fail(MC_E_INVALID, "insert_prefilled: bad argument");
  int rc = check_row(b, row);
  if (rc) return rc;
  MC_HIP(hipSetDevice(b->m->device));
  if ((rc = sync_kv_len(b))) return rc;
  if (b->kv_len_host[(size_t)row] != n_ctx - 1) return fail(MC_E_STATE, "insert_prefilled: kv_len must equal n_ctx - 1");
  if ((size_t)n_ctx + (size_t)max_tokens + (size_t)b->K1 + 1 > (size_t)b->cap)
    return fail(MC_E_CAPACITY, "insert_prefilled: context + max_tokens exceeds capacity");
  StepState& s = b->s;
  if ((rc = upload_i32(b, s.hist + (size_t)row * b->hcap, ctx, (size_t)n_ctx))) return rc;
  if ((rc = set_row_i32(b, s.hist_len, row, n_ctx))) return rc;
  if ((rc = set_row_i32(b, s.gen, row, 1))) return rc;
  if ((rc = set_row_i32(b, s.max_gen, row, max_tokens))) return rc;
  if ((rc = set_row_i32(b, s.cur, row, ctx[n_ctx - 1]))) return rc;
  // the current token counts as generated (generatedTokenHistory holds it)
  if ((rc = set_row_sampling(b, row, sp, ctx + n_ctx - 1, 1))) return rc;
  return set_row_i32(b, s.active, row, 1);
}

extern "C" int mc_batch_remove(mc_batch* b, int32_t row) {
  if (!b) return fail(MC_E_INVALID, "null batch");
  int rc = check_row(b, row);
  if (rc) return rc;
  MC_HIP(hipSetDevice(b->m->device));
  return set_row_i32(b, b->s.active, row, 0);
}

extern "C" int mc_batch_rollback(mc_batch* b, int32_t row, int32_t n) {
  if (!b) return fail(MC_E_INVALID, "null batch");
  int rc = check_row(b, row);
  if (rc) return rc;
  if (n < 0) return fail(MC_E_INVALID, "rollback: negative count");
  MC_HIP(hipSetDevice(b->m->device));
  if ((rc = sync_kv_len(b))) return rc;
  const int len = b->kv_len_host[(size_t)row];
  b->kv_len_host[(size_t)row] = len - std::min(n, len);
  return set_row_i32(b, b->s.kv_len, row, b->kv_len_host[(size_t)row]);
}

extern "C" int mc_batch_trim(mc_batch* b, int32_t n) {
  if (!b) return fail(MC_E_INVALID, "null batch");
  if (n < 0) return fail(MC_E_INVALID, "trim: negative count");
  MC_HIP(hipSetDevice(b->m->device));
  int rc = sync_kv_len(b);
  if (rc) return rc;
  int idx = 0;
  for (int v : b->kv_len_host) idx = std::max(idx, v);
  const int trimmed = std::min(idx, n);  // BatchCache.swift:406
  if (trimmed <= 0) return 0;
  for (auto& v : b->kv_len_host) v -= std::min(trimmed, v);  // per-row: min(trimmed, row length)
  if ((rc = upload_i32(b, b->s.kv_len, b->kv_len_host.data(), (size_t)b->R))) return rc;
  return trimmed;
}

// The copies that make row i hold what row rows[i] held, for i < n (a row may be listed more
// than once): (dst, src) pairs in execution order, where -1 names one spare row.  A copy runs
// once no pending copy still reads its destination; when only cycles remain, one destination
// is parked in the spare first (each row is written at most once, so the copies form trees
// and at most one cycle per connected part, and the spare is free again before the next
// cycle needs it).
static std::vector<std::pair<int, int>> plan_row_moves(const int32_t* rows, int n, int R) {
  std::vector<int> src((size_t)n), readers((size_t)R, 0);
  std::vector<char> pending((size_t)n, 0);
  int left = 0;
  for (int i = 0; i < n; ++i) {
    src[(size_t)i] = rows[i];
    if (rows[i] != i) { pending[(size_t)i] = 1; readers[(size_t)rows[i]]++; ++left; }
  }
  std::vector<std::pair<int, int>> out;
  while (left > 0) {
    bool moved = false;
    for (int i = 0; i < n; ++i)
      if (pending[(size_t)i] && readers[(size_t)i] == 0) {
        out.push_back({i, src[(size_t)i]});
        if (src[(size_t)i] >= 0) readers[(size_t)src[(size_t)i]]--;
        pending[(size_t)i] = 0;
        --left;
        moved = true;
      }
    if (moved) continue;
    int i = 0;  // every pending copy lies on a cycle: park one destination
    while (!pending[(size_t)i]) ++i;
    out.push_back({-1, i});
    for (int j = 0; j < n; ++j)
      if (pending[(size_t)j] && src[(size_t)j] == i) src[(size_t)j] = -1;
    readers[(size_t)i] = 0;
  }
  return out;
}

// K/V positions [0, len) of one layer from (sk, sv) to (dk, dv): K blocks [n_kv][cap][d],
// V blocks [n_kv][d][cap] with each side's own position stride.
// Position stride of a batch's K/V cache: max_ctx rounded up to a 64-key sub-chunk (the
// attention reads whole sub-chunks), not max_ctx itself.
static int kv_stride(const mc_batch* b) { return b->kv.empty() ? b->cap : b->kv[0].cap; }

static int copy_kv_block(uint16_t* dk, uint16_t* dv, int dcap, const uint16_t* sk, const uint16_t* sv, int scap,
                         int len, int nkv, int d, hipStream_t st) {
  if (len <= 0) return MC_OK;
  MC_HIP(hipMemcpy2DAsync(dk, (size_t)dcap * d * 2, sk, (size_t)scap * d * 2, (size_t)len * d * 2, (size_t)nkv,
                          hipMemcpyDeviceToDevice, st));
  MC_HIP(hipMemcpy2DAsync(dv, (size_t)dcap * 2, sv, (size_t)scap * 2, (size_t)len * 2, (size_t)nkv * d,
                          hipMemcpyDeviceToDevice, st));
  return MC_OK;
}

// BatchCache.swift:217-246 filter(keeping:): the listed rows, in the order given (a row may be
// listed twice, as take() allows), become rows 0 .. n-1 with their K/V, lengths, token
// histories and sampler state; the other rows are left empty (inactive, no K/V).  Rows here
// have no left padding to drop.
extern "C" int mc_batch_filter(mc_batch* b, const int32_t* rows, int32_t n) {
  if (!b || (n > 0 && !rows)) return fail(MC_E_INVALID, "filter: null argument");
  if (n < 0 || n > b->R) return fail(MC_E_INVALID, "filter: row count out of range");
  for (int i = 0; i < n; ++i)
    if (rows[i] < 0 || rows[i] >= b->R) return fail(MC_E_INVALID, "filter: row out of range");
  MC_HIP(hipSetDevice(b->m->device));
  int rc = sync_kv_len(b);
  if (rc) return rc;
  const int R = b->R;
  const auto& c = b->m->cfg;
  const int nkv = c.n_kv_heads, d = c.head_dim, V = b->s.V, cap = kv_stride(b);
  const size_t kv_row = (size_t)nkv * cap * d;  // elements of one row's K (and of its V) in one layer
  const bool kv = !b->m->fake;
  // K/V and generated-token counts: row blocks moved in place, through one spare block
  const auto plan = plan_row_moves(rows, n, R);
  uint16_t* spare = nullptr;
  int32_t* spare_cnt = nullptr;
  if (std::any_of(plan.begin(), plan.end(), [](const std::pair<int, int>& p) { return p.first < 0; })) {
    if ((kv && hipMalloc((void**)&spare, 2 * kv_row * 2) != hipSuccess) ||
        hipMalloc((void**)&spare_cnt, (size_t)V * 4) != hipSuccess) {
      if (spare) (void)hipFree(spare);
      return fail(MC_E_NOMEM, "filter: no device memory for the spare row");
    }
  }
  // the per-row state arrays (lengths included)
  std::vector<uint32_t> h(b->scratch_words), o;
  if (hipMemcpy(h.data(), b->scratch, h.size() * 4, hipMemcpyDeviceToHost) == hipSuccess) {
    o = h;
    for (const auto& a : b->row_arrs)
      for (int i = 0; i < R; ++i)
        for (int e = 0; e < a.w; ++e)
          o[a.off + (size_t)i * a.w + e] = i < n ? h[a.off + (size_t)rows[i] * a.w + e] : (uint32_t)a.empty;
    if (hipMemcpy(b->scratch, o.data(), o.size() * 4, hipMemcpyHostToDevice) != hipSuccess)
      rc = fail(MC_E_HIP, "filter: state upload failed");
  } else {
    rc = fail(MC_E_HIP, "filter: state download failed");
  }
  // positions each copy moves (the source's length at that point of the plan)
  std::vector<int> lens(b->kv_len_host), move_len;
  int spare_len = 0;
  for (const auto& [dst, src] : plan) {
    const int len = src < 0 ? spare_len : lens[(size_t)src];
    move_len.push_back(len);
    if (dst < 0) spare_len = len; else lens[(size_t)dst] = len;
  }
  // layer by layer, the whole plan through a one-layer spare; then the counts
  for (int l = 0; kv && !rc && l < c.n_layers; ++l) {
    const KVLayer& L = b->kv[(size_t)l];
    for (size_t i = 0; i < plan.size() && !rc; ++i) {
      const auto [dst, src] = plan[i];
      uint16_t* dk = dst < 0 ? spare : L.k + (size_t)dst * kv_row;
      uint16_t* dv = dst < 0 ? spare + kv_row : L.v + (size_t)dst * kv_row;
      const uint16_t* sk = src < 0 ? spare : L.k + (size_t)src * kv_row;
      const uint16_t* sv = src < 0 ? spare + kv_row : L.v + (size_t)src * kv_row;
      rc = copy_kv_block(dk, dv, cap, sk, sv, cap, move_len[i], nkv, d, b->st);
    }
  }
  for (size_t i = 0; i < plan.size() && !rc; ++i) {
    const auto [dst, src] = plan[i];
    int32_t* dc = dst < 0 ? spare_cnt : b->gen_cnt + (size_t)dst * V;
    const int32_t* sc = src < 0 ? spare_cnt : b->gen_cnt + (size_t)src * V;
    if (hipMemcpyAsync(dc, sc, (size_t)V * 4, hipMemcpyDeviceToDevice, b->st) != hipSuccess)
      rc = fail(MC_E_HIP, "filter: copy failed");
  }
  const hipError_t e = hipStreamSynchronize(b->st);
  if (spare) (void)hipFree(spare);
  if (spare_cnt) (void)hipFree(spare_cnt);
  if (rc) return rc;
  if (e != hipSuccess) return fail(MC_E_HIP, "filter: copy failed");
  return sync_kv_len(b);  // the lengths moved with the state arrays
}

// BatchCache.swift:196-215 extract(_:): one row's K/V (positions [0, kv_len)) copied into row
// dst_row of dst, a batch of the same model; that row becomes inactive with this K/V and
// length, ready for mc_batch_insert_prefilled.
extern "C" int mc_batch_extract_kv(mc_batch* b, int32_t row, mc_batch* dst, int32_t dst_row) {
  if (!b || !dst) return fail(MC_E_INVALID, "extract_kv: null batch");
  int rc = check_row(b, row);
  if (rc || (rc = check_row(dst, dst_row))) return rc;
  const auto &c = b->m->cfg, &dc = dst->m->cfg;
  if (b->m->device != dst->m->device || c.n_layers != dc.n_layers || c.n_kv_heads != dc.n_kv_heads ||
      c.head_dim != dc.head_dim || b->m->fake != dst->m->fake)
    return fail(MC_E_INVALID, "extract_kv: the batches' models differ in K/V shape or device");
  if (b == dst && row == dst_row) return MC_OK;
  MC_HIP(hipSetDevice(b->m->device));
  if ((rc = sync_kv_len(dst)) || (rc = sync_kv_len(b))) return rc;
  const int len = b->kv_len_host[(size_t)row];
  if (len > dst->cap) return fail(MC_E_CAPACITY, "extract_kv: the row's K/V exceeds the destination's capacity");
  if ((rc = set_row_i32(dst, dst->s.active, dst_row, 0))) return rc;
  if (!b->m->fake) {
    const int scap = kv_stride(b), dcap = kv_stride(dst);
    const size_t skv = (size_t)c.n_kv_heads * scap * c.head_dim, dkv = (size_t)c.n_kv_heads * dcap * c.head_dim;
    for (int l = 0; l < c.n_layers; ++l) {
      const KVLayer &S = b->kv[(size_t)l], &D = dst->kv[(size_t)l];
      if ((rc = copy_kv_block(D.k + (size_t)dst_row * dkv, D.v + (size_t)dst_row * dkv, dcap,
                              S.k + (size_t)row * skv, S.v + (size_t)row * skv, scap, len, c.n_kv_heads,
                              c.head_dim, b->st)))
        return rc;
    }
    MC_HIP(hipStreamSynchronize(b->st));
  }
  dst->kv_len_host[(size_t)dst_row] = len;
  return set_row_i32(dst, dst->s.kv_len, dst_row, len);
}

// Prefix blocks (TrackA/BlockAwarePrefixCache.swift:140-162 payloadForBlock, :57-85
// reconstructCache): positions [t0, t0 + n) of one row's K/V in the reference's per-layer
// state layout, keys and values each [n_layers][n_kv][n][d] bf16 (layer l's slice
// state[0 or 1][0, :, t0 ..< t0 + n, :]).  Both go through a device staging buffer in the
// block layout, moved to or from the host by one plain copy each: K rows are contiguous in
// the cache and move by device-side strided copies; V is stored [d][cap] per head and
// turns through a device transpose.
static int kv_block_io(mc_batch* b, int row, int t0, int n, uint16_t* keys, uint16_t* values, bool to_host) {
  const auto& c = b->m->cfg;
  const int nkv = c.n_kv_heads, d = c.head_dim, cap = kv_stride(b), L = c.n_layers;
  const size_t per_layer = (size_t)nkv * n * d, kv_row = (size_t)nkv * cap * d, total = per_layer * L;
  uint16_t* stage = nullptr;  // [2][L][nkv][n][d]: keys, then values
  MC_HIP(hipMalloc((void**)&stage, total * 2 * 2));
  int rc = MC_OK;
  hipError_t e = hipSuccess;
  if (!to_host) {
    e = hipMemcpyAsync(stage, keys, total * 2, hipMemcpyHostToDevice, b->st);
    if (e == hipSuccess) e = hipMemcpyAsync(stage + total, values, total * 2, hipMemcpyHostToDevice, b->st);
  }
  for (int l = 0; l < L && rc == MC_OK && e == hipSuccess; ++l) {
    const KVLayer& kv = b->kv[(size_t)l];
    uint16_t* krow = kv.k + (size_t)row * kv_row + (size_t)t0 * d;  // head h at + h cap d
    uint16_t* vrow = kv.v + (size_t)row * kv_row;
    uint16_t *sk = stage + per_layer * l, *sv = stage + total + per_layer * l;
    if (to_host)
      e = hipMemcpy2DAsync(sk, (size_t)n * d * 2, krow, (size_t)cap * d * 2, (size_t)n * d * 2, (size_t)nkv,
                           hipMemcpyDeviceToDevice, b->st);
    else
      e = hipMemcpy2DAsync(krow, (size_t)cap * d * 2, sk, (size_t)n * d * 2, (size_t)n * d * 2, (size_t)nkv,
                           hipMemcpyDeviceToDevice, b->st);
    if (e == hipSuccess) rc = launch_kv_block_v(vrow, cap, sv, nkv, n, d, t0, to_host, b->st);
  }
  if (to_host && rc == MC_OK && e == hipSuccess) {
    e = hipMemcpyAsync(keys, stage, total * 2, hipMemcpyDeviceToHost, b->st);
    if (e == hipSuccess) e = hipMemcpyAsync(values, stage + total, total * 2, hipMemcpyDeviceToHost, b->st);
  }
  if (rc == MC_OK && e != hipSuccess) rc = fail(MC_E_HIP, hipGetErrorString(e));
  const hipError_t es = hipStreamSynchronize(b->st);
  const hipError_t ef = hipFree(stage);
  if (rc == MC_OK && es != hipSuccess) rc = fail(MC_E_HIP, hipGetErrorString(es));
  if (rc == MC_OK && ef != hipSuccess) rc = fail(MC_E_HIP, hipGetErrorString(ef));
  return rc;
}

extern "C" int mc_batch_export_kv_block(mc_batch* b, int32_t row, int32_t t0, int32_t n, uint16_t* keys,
                                        uint16_t* values) {
  if (!b || !keys || !values) return fail(MC_E_INVALID, "export_kv_block: null argument");
  int rc = check_row(b, row);
  if (rc) return rc;
  if (b->m->fake) return fail(MC_E_STATE, "export_kv_block: fake model has no K/V");
  if (t0 < 0 || n < 1) return fail(MC_E_INVALID, "export_kv_block: bad range");
  MC_HIP(hipSetDevice(b->m->device));
  if ((rc = sync_kv_len(b))) return rc;
  if ((int64_t)t0 + n > b->kv_len_host[(size_t)row])
    return fail(MC_E_INVALID, "export_kv_block: range past the row's K/V length");
  return kv_block_io(b, row, t0, n, keys, values, true);
}

extern "C" int mc_batch_import_kv_block(mc_batch* b, int32_t row, int32_t t0, int32_t n, const uint16_t* keys,
                                        const uint16_t* values) {
  if (!b || !keys || !values) return fail(MC_E_INVALID, "import_kv_block: null argument");
  int rc = check_row(b, row);
  if (rc) return rc;
  if (b->m->fake) return fail(MC_E_STATE, "import_kv_block: fake model has no K/V");
  if (t0 < 0 || n < 1) return fail(MC_E_INVALID, "import_kv_block: bad range");
  MC_HIP(hipSetDevice(b->m->device));
  if ((rc = sync_kv_len(b))) return rc;
  if (t0 > b->kv_len_host[(size_t)row])
    return fail(MC_E_INVALID, "import_kv_block: t0 past the row's K/V length (blocks go in order)");
  if ((int64_t)t0 + n > b->cap) return fail(MC_E_CAPACITY, "import_kv_block: block past the row's capacity");
  if ((rc = set_row_i32(b, b->s.active, row, 0))) return rc;
  if ((rc = kv_block_io(b, row, t0, n, const_cast<uint16_t*>(keys), const_cast<uint16_t*>(values), false))) return rc;
  b->kv_len_host[(size_t)row] = t0 + n;
  return set_row_i32(b, b->s.kv_len, row, t0 + n);
}

extern "C" int mc_batch_kv_len(mc_batch* b, int32_t row, int32_t* len) {
  if (!b || !len) return fail(MC_E_INVALID, "null argument");
  int rc = check_row(b, row);
  if (rc) return rc;
  MC_HIP(hipSetDevice(b->m->device));
  if ((rc = sync_kv_len(b))) return rc;
  *len = b->kv_len_host[(size_t)row];
  return MC_OK;
}

extern "C" int mc_batch_read_kv(mc_batch* b, int32_t layer, int32_t row, int32_t which_v, uint16_t* out) {
  if (!b || !out) return fail(MC_E_INVALID, "null argument");
  int rc = check_row(b, row);
  if (rc) return rc;
  if (b->m->fake) return fail(MC_E_STATE, "fake model has no KV");
  const auto& c = b->m->cfg;
  if (layer < 0 || layer >= c.n_layers) return fail(MC_E_INVALID, "layer out of range");
  MC_HIP(hipSetDevice(b->m->device));
  if ((rc = sync_kv_len(b))) return rc;
  const int len = b->kv_len_host[(size_t)row];
  const KVLayer& kv = b->kv[(size_t)layer];
  const int d = c.head_dim;
  if (!which_v) {
    for (int h = 0; h < c.n_kv_heads; ++h)
      MC_HIP(hipMemcpy(out + (size_t)h * len * d, kv.k + (((size_t)row * c.n_kv_heads + h) * kv.cap) * d,
                       (size_t)len * d * 2, hipMemcpyDeviceToHost));
    return MC_OK;
  }
  // V is stored transposed ([d][cap] per head): copy the d rows, then transpose
  std::vector<uint16_t> tmp((size_t)d * len);
  for (int h = 0; h < c.n_kv_heads; ++h) {
    if (len > 0)
      MC_HIP(hipMemcpy2D(tmp.data(), (size_t)len * 2, kv.v + ((size_t)row * c.n_kv_heads + h) * d * kv.cap,
                         (size_t)kv.cap * 2, (size_t)len * 2, (size_t)d, hipMemcpyDeviceToHost));
    uint16_t* o = out + (size_t)h * len * d;
    for (int e = 0; e < d; ++e)
      for (int p = 0; p < len; ++p) o[(size_t)p * d + e] = tmp[(size_t)e * len + p];
  }
  return MC_OK;
}

extern "C" int mc_batch_read_attention(mc_batch* b, int32_t M, uint16_t* out) {
  if (!b || !out || M < 0) return fail(MC_E_INVALID, "read_attention: bad argument");
  if (M > b->last_M) return fail(MC_E_STATE, "read_attention: the last forward had fewer token slots");
  MC_HIP(hipSetDevice(b->m->device));
  MC_HIP(hipStreamSynchronize(b->st));
  const auto& c = b->m->cfg;
  MC_HIP(hipMemcpy(out, b->att, (size_t)M * c.n_q_heads * c.head_dim * 2, hipMemcpyDeviceToHost));
  return MC_OK;
}

extern "C" int mc_batch_read_router(mc_batch* b, int32_t M, uint16_t* out) {
  if (!b || !out || M < 0) return fail(MC_E_INVALID, "read_router: bad argument");
  const auto& c = b->m->cfg;
  if (!b->moe_logits) return fail(MC_E_STATE, "read_router: not a mixture-of-experts model");
  if (M > b->last_M || M > 64) return fail(MC_E_STATE, "read_router: the last forward's last 64-token chunk has fewer slots");
  MC_HIP(hipSetDevice(b->m->device));
  MC_HIP(hipStreamSynchronize(b->st));
  MC_HIP(hipMemcpy(out, b->moe_logits, (size_t)M * c.n_experts * 2, hipMemcpyDeviceToHost));
  return MC_OK;
}

extern "C" int mc_batch_read_logits(mc_batch* b, int32_t slot0, int32_t n, uint16_t* out) {
  if (!b || !out || slot0 < 0 || n < 0) return fail(MC_E_INVALID, "read_logits: bad argument");
  const int V = b->m->cfg.vocab;
  const int M = b->m->fake ? b->R * b->K1 : b->last_M;
  if (slot0 + n > M) return fail(MC_E_STATE, "read_logits: the last forward had fewer token slots");
  MC_HIP(hipSetDevice(b->m->device));
  MC_HIP(hipStreamSynchronize(b->st));
  MC_HIP(hipMemcpy(out, b->logits + (size_t)slot0 * V, (size_t)n * V * 2, hipMemcpyDeviceToHost));
  return MC_OK;
}

extern "C" int mc_batch_history(mc_batch* b, int32_t row, int32_t* out, int32_t cap, int32_t* len) {
  if (!b || !len) return fail(MC_E_INVALID, "null argument");
  int rc = check_row(b, row);
  if (rc) return rc;
  MC_HIP(hipSetDevice(b->m->device));
  MC_HIP(hipStreamSynchronize(b->st));
  int32_t n = 0;
  MC_HIP(hipMemcpy(&n, b->s.hist_len + row, 4, hipMemcpyDeviceToHost));
  *len = n;
  if (out && cap > 0)
    MC_HIP(hipMemcpy(out, b->s.hist + (size_t)row * b->hcap, (size_t)std::min(n, cap) * 4, hipMemcpyDeviceToHost));
  return MC_OK;
}

// --------------------------- the step -------------------------------------
static int enqueue_step(mc_batch* b) {
  int rc;
  const StepState& s = b->s;
  if ((rc = launch_propose(s, b->st))) return rc;
  const int M = b->R * b->K1;
  if ((rc = forward_slots(b, M, b->K1, 0, M))) return rc;
  if ((rc = launch_accept_scan(s, b->logits, -1, b->st))) return rc;
  return launch_commit(s, -1, b->st);
}

extern "C" int mc_step(mc_batch* b, const int32_t* forced_accept, const uint32_t* uniforms, int32_t* out_tokens,
                       int32_t* out_counts, int32_t* out_finish) {
  if (!b) return fail(MC_E_INVALID, "null batch");
  MC_HIP(hipSetDevice(b->m->device));
  int rc;
  const int R = b->R, K1 = b->K1;
  // caller uniforms (the captured step reads them through a device flag)
  if (uniforms) {
    if ((rc = upload_i32(b, reinterpret_cast<int32_t*>(const_cast<uint32_t*>(b->s.uniforms)),
                         reinterpret_cast<const int32_t*>(uniforms), (size_t)2 * R * K1)))
      return rc;
  }
  if ((uniforms != nullptr) != b->uniforms_on) {
    const int32_t on = uniforms ? 1 : 0;
    if ((rc = upload_i32(b, const_cast<int32_t*>(b->s.use_uniforms), &on, 1))) return rc;
    b->uniforms_on = uniforms != nullptr;
  }
  // forced accept-length schedule (or none)
  // (uploaded only when it differs from the all-none schedule already on the device)
  if (forced_accept || !b->forced_none) {
    std::vector<int32_t> f((size_t)R, -1);
    if (forced_accept)
      for (int r = 0; r < R; ++r) f[(size_t)r] = forced_accept[r] < 0 ? -1 : forced_accept[r];
    if ((rc = upload_i32(b, b->s.forced, f.data(), (size_t)R))) return rc;
    b->forced_none = forced_accept == nullptr;
  }
  // MC_STEP_EAGER=1 launches the step's kernels directly instead of replaying the captured
  // graph (same kernels; used under profilers that do not follow graph launches).
  static const bool eager = [] {
    const char* e = getenv("MC_STEP_EAGER");
    return e && e[0] == '1';
  }();
  if (eager && !b->profiling) {
    if ((rc = enqueue_step(b))) return rc;
  } else if (b->profiling) {
    b->ev_used = 0;
    b->recs.clear();
    size_t e0 = 0;
    if ((rc = prof_begin(b, &e0))) return rc;
    if ((rc = enqueue_step(b))) return rc;
    if ((rc = prof_end(b, e0, 2, 0.0))) return rc;
  } else {
    if (!b->graph) {
      MC_HIP(hipStreamBeginCapture(b->st, hipStreamCaptureModeThreadLocal));
      rc = enqueue_step(b);
      hipGraph_t g = nullptr;
      hipError_t e = hipStreamEndCapture(b->st, &g);
      if (rc) {
        if (g) (void)hipGraphDestroy(g);
        return rc;
      }
      if (e != hipSuccess) return hip_fail(e, "hipStreamEndCapture", __FILE__, __LINE__);
      b->graph_def = g;
      MC_HIP(hipGraphInstantiate(&b->graph, g, nullptr, nullptr, 0));
    }
    MC_HIP(hipGraphLaunch(b->graph, b->st));
    b->last_M = b->m->fake ? 0 : R * K1;  // the replayed forward's slots
  }
  const StepState& s = b->s;
  int32_t* h = b->h_out;
  // tokens, counts, finish reasons, proposal and KV lengths sit contiguously on the device
  MC_HIP(hipMemcpyAsync(h, s.out_tok, (size_t)(R * K1 + 4 * R) * 4, hipMemcpyDeviceToHost, b->st));
  MC_HIP(hipStreamSynchronize(b->st));
  if (out_tokens) memcpy(out_tokens, h, (size_t)R * K1 * 4);
  if (out_counts) memcpy(out_counts, h + R * K1, (size_t)R * 4);
  if (out_finish) memcpy(out_finish, h + R * K1 + R, (size_t)R * 4);
  for (int r = 0; r < R; ++r) {
    if (h[R * K1 + r] > 0) b->widths.push_back(h[R * K1 + 2 * R + r] + 1);
    b->kv_len_host[(size_t)r] = h[R * K1 + 3 * R + r];
  }
  if (b->profiling) {
    for (int k = 0; k < 3; ++k) { b->prof_ms[k] = 0; b->prof_bytes[k] = 0; b->prof_launch[k] = 0; }
    for (const auto& rec : b->recs) {
      float ms = 0;
      MC_HIP(hipEventElapsedTime(&ms, b->ev[rec.e0], b->ev[rec.e1]));
      b->prof_ms[rec.kind] += ms;
      b->prof_bytes[rec.kind] += rec.bytes;
      b->prof_launch[rec.kind] += 1;
    }
  }
  return MC_OK;
}

extern "C" int mc_batch_stats(mc_batch* b, mc_spec_stats* out) {
  if (!b || !out) return fail(MC_E_INVALID, "null argument");
  MC_HIP(hipSetDevice(b->m->device));
  MC_HIP(hipStreamSynchronize(b->st));
  unsigned long long v[4];
  MC_HIP(hipMemcpy(v, b->s.stats, sizeof v, hipMemcpyDeviceToHost));
  out->proposed = (int64_t)v[0];
  out->accepted = (int64_t)v[1];
  out->proposal_batches = (int64_t)v[2];
  out->rejected_batches = (int64_t)v[3];
  return MC_OK;
}

extern "C" int mc_batch_call_widths(mc_batch* b, int32_t* out, int32_t cap) {
  if (!b) return fail(MC_E_INVALID, "null batch");
  const int n = (int)b->widths.size();
  for (int i = 0; i < n && i < cap && out; ++i) out[i] = b->widths[(size_t)i];
  return n;
}

extern "C" int mc_batch_set_profiling(mc_batch* b, int32_t enabled) {
  if (!b) return fail(MC_E_INVALID, "null batch");
  b->profiling = enabled != 0;
  return MC_OK;
}

extern "C" int mc_batch_profile(mc_batch* b, int32_t kind, double* ms, double* bytes, int32_t* launches) {
  if (!b || kind < 0 || kind > 2) return fail(MC_E_INVALID, "bad argument");
  if (ms) *ms = b->prof_ms[kind];
  if (bytes) *bytes = b->prof_bytes[kind];
  if (launches) *launches = b->prof_launch[kind];
  return MC_OK;
}

// --------------------------- standalone proposer / acceptance -------------
extern "C" int mc_ngram_propose(const int32_t* hist, const int64_t* hist_off, int32_t B, int32_t max_suffix,
                                int32_t min_context, const int32_t* limit, int32_t out_stride, int32_t* out,
                                int32_t* out_len) {
  if (!hist_off || !limit || !out || !out_len || B < 0) return fail(MC_E_INVALID, "mc_ngram_propose: null argument");
  if (B == 0) return MC_OK;
  for (int r = 0; r < B; ++r)
    if (limit[r] > out_stride || hist_off[r + 1] < hist_off[r]) return fail(MC_E_INVALID, "mc_ngram_propose: bad limit/offsets");
  max_suffix = std::max(1, max_suffix);
  min_context = std::max(2, min_context);
  MC_HIP(hipSetDevice(g_device));
  const size_t nh = (size_t)hist_off[B];
  int32_t *dh = nullptr, *dl = nullptr, *dout = nullptr, *dlen = nullptr;
  int64_t* doff = nullptr;
  int rc = MC_OK;
  hipStream_t st;
  MC_HIP(hipStreamCreateWithFlags(&st, hipStreamNonBlocking));
  if (!(rc = dev_alloc(&dh, nh)) && !(rc = dev_alloc(&doff, (size_t)B + 1)) && !(rc = dev_alloc(&dl, (size_t)B)) &&
      !(rc = dev_alloc(&dout, (size_t)B * std::max(1, out_stride))) && !(rc = dev_alloc(&dlen, (size_t)B))) {
    hipError_t e = hipSuccess;
    if (nh) e = hipMemcpy(dh, hist, nh * 4, hipMemcpyHostToDevice);
    if (e == hipSuccess) e = hipMemcpy(doff, hist_off, ((size_t)B + 1) * 8, hipMemcpyHostToDevice);
    if (e == hipSuccess) e = hipMemcpy(dl, limit, (size_t)B * 4, hipMemcpyHostToDevice);
    if (e != hipSuccess) rc = hip_fail(e, "mc_ngram_propose upload", __FILE__, __LINE__);
    if (!rc) rc = launch_ngram_standalone(dh, doff, B, max_suffix, min_context, dl, out_stride, dout, dlen, st);
    if (!rc) {
      e = hipStreamSynchronize(st);
      if (e == hipSuccess) e = hipMemcpy(out_len, dlen, (size_t)B * 4, hipMemcpyDeviceToHost);
      if (e == hipSuccess) e = hipMemcpy(out, dout, (size_t)B * out_stride * 4, hipMemcpyDeviceToHost);
      if (e != hipSuccess) rc = hip_fail(e, "mc_ngram_propose", __FILE__, __LINE__);
    }
  }
  for (void* p : {(void*)dh, (void*)doff, (void*)dl, (void*)dout, (void*)dlen})
    if (p) (void)hipFree(p);
  (void)hipStreamDestroy(st);
  return rc;
}

extern "C" int mc_accept(const uint16_t* logits, int32_t vocab, int32_t B, const int64_t* row_off,
                         const int32_t* drafts, int32_t draft_stride, const int32_t* n_draft, const mc_sampling* sp,
                         const int32_t* generated, const int64_t* gen_off, const uint64_t* counter,
                         const uint32_t* uniforms, int32_t acceptance, int32_t* out_tokens, int32_t* n_emit,
                         int32_t* kv_keep, int32_t* n_accepted) {
  if (!logits || !row_off || !n_draft || !sp || !counter || !out_tokens || !n_emit || !kv_keep || !n_accepted || B <= 0 ||
      vocab <= 0 || row_off[0] != 0 || draft_stride < 0 || (!drafts && draft_stride > 0) ||
      (generated && !gen_off))
    return fail(MC_E_INVALID, "mc_accept: bad argument");
  int K = 0;
  for (int r = 0; r < B; ++r) {
    if (n_draft[r] < 0 || n_draft[r] > draft_stride) return fail(MC_E_INVALID, "mc_accept: bad n_draft");
    if (row_off[r + 1] - row_off[r] != n_draft[r] + 1) return fail(MC_E_INVALID, "mc_accept: row_off must give n_draft+1 rows");
    for (int j = 0; j < n_draft[r]; ++j) {
      const int32_t t = drafts[(size_t)r * draft_stride + j];
      if (t < 0 || t >= vocab) return fail(MC_E_INVALID, "mc_accept: draft token out of range");
    }
    if (generated && (gen_off[r + 1] < gen_off[r] || gen_off[0] != 0))
      return fail(MC_E_INVALID, "mc_accept: gen_off must be non-decreasing from 0");
    K = std::max(K, n_draft[r]);
  }
  if (K + 1 > 257) return fail(MC_E_INVALID, "mc_accept: at most 256 drafts per row");
  MC_HIP(hipSetDevice(g_device));
  const int K1 = K + 1;
  // device state laid out as a StepState with row r's logits at slots r*K1 + j
  StepState s;
  s.R = B; s.K = K; s.K1 = K1; s.V = vocab; s.acceptance = acceptance; s.hcap = 1;
  std::vector<int32_t> h_nprop((size_t)B), h_nv((size_t)B), h_rs0((size_t)B), h_act((size_t)B, 1), h_dr((size_t)B * K1, 0),
      h_eos((size_t)B * 8, 0), h_neos((size_t)B), h_rej((size_t)B), h_hs((size_t)B), h_forced((size_t)B, -1),
      h_topk((size_t)B), h_mint((size_t)B), h_nb((size_t)B), h_bt((size_t)B * 16, 0), h_proc((size_t)B), h_gen((size_t)B, 0),
      h_useu(1, uniforms ? 1 : 0);
  std::vector<float> h_t((size_t)B), h_tp((size_t)B), h_it((size_t)B), h_mpl((size_t)B), h_rp((size_t)B), h_pp((size_t)B),
      h_fp((size_t)B), h_bv((size_t)B * 16, 0.f);
  std::vector<uint64_t> h_seed((size_t)B), h_ctr((size_t)B);
  std::vector<uint32_t> h_uni(uniforms ? (size_t)B * K1 * 2 : 1, 0u);
  bool any_pen = false;
  for (int r = 0; r < B; ++r) {
    RowSampling q;
    int rc0 = row_sampling(&sp[r], vocab, &q);
    if (rc0) return rc0;
    h_nprop[(size_t)r] = n_draft[r];
    h_nv[(size_t)r] = n_draft[r] + 1;
    h_rs0[(size_t)r] = r * K1;
    for (int j = 0; j < n_draft[r]; ++j) h_dr[(size_t)r * K1 + j] = drafts[(size_t)r * draft_stride + j];
    h_t[(size_t)r] = q.temp;
    h_tp[(size_t)r] = q.top_p;
    h_it[(size_t)r] = q.inv_t;
    h_hs[(size_t)r] = sp[r].has_seed;
    h_seed[(size_t)r] = sp[r].seed;
    h_ctr[(size_t)r] = counter[r];
    for (int i = 0; i < q.n_eos; ++i) h_eos[(size_t)r * 8 + i] = q.eos[i];
    h_neos[(size_t)r] = q.n_eos;
    h_rej[(size_t)r] = sp[r].reject_token;
    h_topk[(size_t)r] = q.top_k;
    h_mpl[(size_t)r] = q.min_p_log;
    h_rp[(size_t)r] = q.rp;
    h_pp[(size_t)r] = q.pp;
    h_fp[(size_t)r] = q.fp;
    h_mint[(size_t)r] = q.min_tokens;
    h_nb[(size_t)r] = q.n_bias;
    for (int i = 0; i < 16; ++i) {
      h_bt[(size_t)r * 16 + i] = q.bias_tok[i];
      h_bv[(size_t)r * 16 + i] = q.bias_val[i];
    }
    h_proc[(size_t)r] = q.proc;
    any_pen = any_pen || (q.proc & 4);
    h_gen[(size_t)r] = generated ? (int32_t)(gen_off[r + 1] - gen_off[r]) : 0;
    if (uniforms)
      for (int j = 0; j <= n_draft[r]; ++j)
        for (int k = 0; k < 2; ++k)
          h_uni[((size_t)r * K1 + j) * 2 + k] = uniforms[((size_t)r * (draft_stride + 1) + j) * 2 + k];
  }
  // generated-token counts of the rows with penalties
  std::vector<int32_t> h_cnt(any_pen ? (size_t)B * vocab : 1, 0);
  if (any_pen && generated)
    for (int r = 0; r < B; ++r) {
      if (!(h_proc[(size_t)r] & 4)) continue;
      for (int64_t i = gen_off[r]; i < gen_off[r + 1]; ++i)
        if (generated[i] >= 0 && generated[i] < vocab) h_cnt[(size_t)r * vocab + generated[i]]++;
    }
  std::vector<uint16_t> h_lg((size_t)B * K1 * vocab, 0);
  for (int r = 0; r < B; ++r)
    memcpy(&h_lg[(size_t)r * K1 * vocab], logits + (size_t)row_off[r] * vocab, (size_t)(n_draft[r] + 1) * vocab * 2);
  std::vector<void*> allocs;
  int rc = MC_OK;
  auto up = [&](auto** dst, const auto& src) -> int {
    using T = typename std::remove_reference<decltype(src)>::type::value_type;
    T* p = nullptr;
    int r2 = dev_alloc(&p, src.size());
    if (r2) return r2;
    allocs.push_back(p);
    MC_HIP(hipMemcpy(p, src.data(), src.size() * sizeof(T), hipMemcpyHostToDevice));
    *dst = p;
    return MC_OK;
  };
  uint16_t* dlg = nullptr;
  int32_t *d_emit = nullptr, *d_keep = nullptr, *d_nacc = nullptr;
  std::vector<int32_t> zeros_rk((size_t)B * K1, 0), zeros_r((size_t)B, 0);
  if (!rc) rc = up(&dlg, h_lg);
  if (!rc) rc = up(&s.nprop, h_nprop);
  if (!rc) rc = up(&s.n_valid, h_nv);
  if (!rc) rc = up(&s.row_slot0, h_rs0);
  if (!rc) rc = up(&s.active, h_act);
  if (!rc) rc = up(&s.drafts, h_dr);
  if (!rc) rc = up(&s.temp, h_t);
  if (!rc) rc = up(&s.top_p, h_tp);
  if (!rc) rc = up(&s.inv_temp, h_it);
  if (!rc) rc = up(&s.has_seed, h_hs);
  if (!rc) rc = up(&s.seed, h_seed);
  if (!rc) rc = up(&s.counter, h_ctr);
  if (!rc) rc = up(&s.eos, h_eos);
  if (!rc) rc = up(&s.n_eos, h_neos);
  if (!rc) rc = up(&s.reject, h_rej);
  if (!rc) rc = up(&s.forced, h_forced);
  if (!rc) rc = up(&s.top_k, h_topk);
  if (!rc) rc = up(&s.min_p_log, h_mpl);
  if (!rc) rc = up(&s.rep_pen, h_rp);
  if (!rc) rc = up(&s.pres_pen, h_pp);
  if (!rc) rc = up(&s.freq_pen, h_fp);
  if (!rc) rc = up(&s.min_tokens, h_mint);
  if (!rc) rc = up(&s.n_bias, h_nb);
  if (!rc) rc = up(&s.bias_tok, h_bt);
  if (!rc) rc = up(&s.bias_val, h_bv);
  if (!rc) rc = up(&s.proc, h_proc);
  if (!rc) rc = up(&s.gen, h_gen);
  if (!rc) rc = up(&s.gen_cnt, h_cnt);
  {
    uint32_t* du = nullptr;
    int32_t* df = nullptr;
    if (!rc) rc = up(&du, h_uni);
    if (!rc) rc = up(&df, h_useu);
    s.uniforms = du;
    s.use_uniforms = df;
  }
  if (!rc) rc = up(&s.scan_tok, zeros_rk);
  if (!rc) rc = up(&s.scan_acc, zeros_rk);
  if (!rc) rc = up(&s.scan_res, zeros_rk);
  if (!rc) rc = up(&s.out_tok, zeros_rk);
  if (!rc) rc = up(&d_emit, zeros_r);
  if (!rc) rc = up(&d_keep, zeros_r);
  if (!rc) rc = up(&d_nacc, zeros_r);
  hipStream_t st = nullptr;
  if (!rc) {
    hipError_t e = hipStreamCreateWithFlags(&st, hipStreamNonBlocking);
    if (e != hipSuccess) rc = hip_fail(e, "stream", __FILE__, __LINE__);
  }
  if (!rc) rc = launch_accept_scan(s, dlg, -1, st);
  if (!rc) rc = launch_decide(s, d_emit, d_keep, d_nacc, st);
  if (!rc) {
    std::vector<int32_t> otok((size_t)B * K1);
    hipError_t e = hipStreamSynchronize(st);
    if (e == hipSuccess) e = hipMemcpy(otok.data(), s.out_tok, otok.size() * 4, hipMemcpyDeviceToHost);
    if (e == hipSuccess) e = hipMemcpy(n_emit, d_emit, (size_t)B * 4, hipMemcpyDeviceToHost);
    if (e == hipSuccess) e = hipMemcpy(kv_keep, d_keep, (size_t)B * 4, hipMemcpyDeviceToHost);
    if (e == hipSuccess) e = hipMemcpy(n_accepted, d_nacc, (size_t)B * 4, hipMemcpyDeviceToHost);
    if (e != hipSuccess) rc = hip_fail(e, "mc_accept", __FILE__, __LINE__);
    if (!rc)
      for (int r = 0; r < B; ++r)
        for (int j = 0; j < n_emit[r]; ++j) out_tokens[(size_t)r * (draft_stride + 1) + j] = otok[(size_t)r * K1 + j];
  }
  if (st) (void)hipStreamDestroy(st);
  for (void* p : allocs) (void)hipFree(p);
  return rc;
}

// ---- acceptance over caller device buffers, allocating nothing ----
extern "C" int mc_accept_noalloc(const uint16_t* logits, int32_t vocab, int32_t B, int32_t K, const int32_t* drafts,
                                 const int32_t* n_draft, const mc_sampling* sp, const uint64_t* counter,
                                 const uint32_t* uniforms, int32_t acceptance, int32_t* out_tokens, int32_t* n_emit,
                                 int32_t* kv_keep, int32_t* n_accepted) {
  if (!logits || !n_draft || !sp || !counter || !out_tokens || !n_emit || !kv_keep || !n_accepted || B <= 0 ||
      vocab <= 0 || K < 0 || (K > 0 && !drafts))
    return fail(MC_E_INVALID, "mc_accept_noalloc: bad argument");
  if (B > NOALLOC_MAX_ROWS || K > NOALLOC_MAX_DRAFTS)
    return fail(MC_E_CAPACITY, "mc_accept_noalloc: at most 64 rows and 16 drafts per row");
  int rc;
  RowSampling q[NOALLOC_MAX_ROWS];
  for (int r = 0; r < B; ++r)
    if ((rc = row_sampling(&sp[r], vocab, &q[r]))) return rc;
  MC_HIP(hipSetDevice(g_device));
  if ((rc = resolve_scratch(g_device))) return rc;
  const int K1 = K + 1;
  const size_t R = (size_t)B, RK = R * K1;
  // layout in 32-bit words: the part the prep kernel fills, then the part copied from the host
  size_t words = 0;
  auto take = [&](size_t n) { size_t o = words; words += (n + 1) & ~(size_t)1; return o; };
  const size_t o_np = take(R), o_nv = take(R), o_rs0 = take(R), o_act = take(R), o_dr = take(RK), o_forced = take(R),
               o_gen = take(R), o_sct = take(RK), o_sca = take(RK), o_scr = take(RK);
  const size_t host0 = words;
  const size_t o_temp = take(R), o_topp = take(R), o_invt = take(R), o_hseed = take(R), o_seed = take(2 * R),
               o_ctr = take(2 * R), o_eos = take(8 * R), o_neos = take(R), o_rej = take(R), o_topk = take(R),
               o_mpl = take(R), o_rp = take(R), o_pp = take(R), o_fp = take(R), o_mint = take(R), o_nb = take(R),
               o_bt = take(16 * R), o_bv = take(16 * R), o_proc = take(R), o_useu = take(2), o_err = take(2);
  if (words * 4 > NOALLOC_SCRATCH_BYTES) return fail(MC_E_CAPACITY, "mc_accept_noalloc: scratch too small");
  // the host part, staged in a per-thread buffer
  static thread_local uint32_t himg[NOALLOC_SCRATCH_BYTES / 4];
  uint32_t* h = himg - host0;  // h[o] for o >= host0
  memset(himg, 0, (words - host0) * 4);
  auto put_f = [&](size_t o, float v) { memcpy(&h[o], &v, 4); };
  auto put_i = [&](size_t o, int32_t v) { memcpy(&h[o], &v, 4); };
  for (int r = 0; r < B; ++r) {
    put_f(o_temp + r, q[r].temp);
    put_f(o_topp + r, q[r].top_p);
    put_f(o_invt + r, q[r].inv_t);
    put_i(o_hseed + r, sp[r].has_seed);
    memcpy(&h[o_seed + 2 * r], &sp[r].seed, 8);
    memcpy(&h[o_ctr + 2 * r], &counter[r], 8);
    for (int i = 0; i < 8; ++i) put_i(o_eos + 8 * r + i, q[r].eos[i]);
    put_i(o_neos + r, q[r].n_eos);
    put_i(o_rej + r, sp[r].reject_token);
    put_i(o_topk + r, q[r].top_k);
    put_f(o_mpl + r, q[r].min_p_log);
    put_f(o_rp + r, q[r].rp);
    put_f(o_pp + r, q[r].pp);
    put_f(o_fp + r, q[r].fp);
    put_i(o_mint + r, q[r].min_tokens);
    put_i(o_nb + r, q[r].n_bias);
    for (int i = 0; i < 16; ++i) {
      put_i(o_bt + 16 * r + i, q[r].bias_tok[i]);
      put_f(o_bv + 16 * r + i, q[r].bias_val[i]);
    }
    put_i(o_proc + r, q[r].proc);
  }
  put_i(o_useu, uniforms ? 1 : 0);
  uint32_t* base = static_cast<uint32_t*>(g_scratch_ptr[g_device]);
  auto I32 = [&](size_t o) { return reinterpret_cast<int32_t*>(base + o); };
  auto F32 = [&](size_t o) { return reinterpret_cast<float*>(base + o); };
  StepState s;
  s.R = B; s.K = K; s.K1 = K1; s.V = vocab; s.acceptance = acceptance; s.hcap = 1;
  s.nprop = I32(o_np); s.n_valid = I32(o_nv); s.row_slot0 = I32(o_rs0); s.active = I32(o_act); s.drafts = I32(o_dr);
  s.forced = I32(o_forced); s.gen = I32(o_gen); s.scan_tok = I32(o_sct); s.scan_acc = I32(o_sca);
  s.scan_res = I32(o_scr); s.temp = F32(o_temp); s.top_p = F32(o_topp); s.inv_temp = F32(o_invt);
  s.has_seed = I32(o_hseed); s.seed = reinterpret_cast<uint64_t*>(base + o_seed);
  s.counter = reinterpret_cast<uint64_t*>(base + o_ctr); s.eos = I32(o_eos); s.n_eos = I32(o_neos);
  s.reject = I32(o_rej); s.top_k = I32(o_topk); s.min_p_log = F32(o_mpl); s.rep_pen = F32(o_rp);
  s.pres_pen = F32(o_pp); s.freq_pen = F32(o_fp); s.min_tokens = I32(o_mint); s.n_bias = I32(o_nb);
  s.bias_tok = I32(o_bt); s.bias_val = F32(o_bv); s.proc = I32(o_proc); s.use_uniforms = I32(o_useu);
  s.uniforms = uniforms;  // caller's [B][K + 1][2]
  s.gen_cnt = nullptr;    // no generated history: penalties see the drafts only
  s.out_tok = out_tokens; // caller's [B][K + 1]
  hipStream_t st = nullptr;
  MC_HIP(hipMemcpyAsync(base + host0, himg, (words - host0) * 4, hipMemcpyHostToDevice, st));
  if ((rc = launch_accept_prep(s, drafts, n_draft, K, I32(o_err), st))) return rc;
  if ((rc = launch_accept_scan(s, logits, -1, st))) return rc;
  if ((rc = launch_decide(s, n_emit, kv_keep, n_accepted, st))) return rc;
  int32_t err = 0;
  MC_HIP(hipMemcpyAsync(&err, I32(o_err), 4, hipMemcpyDeviceToHost, st));
  MC_HIP(hipStreamSynchronize(st));
  if (err) return fail(MC_E_INVALID, "mc_accept_noalloc: n_draft or a draft id out of range");
  return MC_OK;
}
