// CPU run of the persistent forward kernel (mlxcat_amd/csrc/mc_fused.hip compiled as host
// C++ against include/hip/hip_runtime.h), checked against the oracle: logits within
// 2e-2 abs + 1e-2 rel, and the K/V the kernel appends.  Test infrastructure.
// The kernel runs on the CPU emulation (emu_runtime.cpp): every lane a coroutine, "device"
// buffers ending at a guard page so an out-of-bounds access faults as on the GPU.
//
// usage: fused_emu <scenario> <grid>   scenario 0: 1 row, 6 tokens, 1000 cached positions
//                                      scenario 1: 3 rows of (3, 1, 3) tokens, mixed contexts
//                                      scenario 2: 1 row, 8 tokens, 40 cached positions
//                                      scenario 3: Qwen3-4B shape (2 layers), 1 row, 6 tokens,
//                                                  40 cached positions (split-K 2 and 4)
// prints one line per checked quantity; exit status 0 when everything matches.
#include <cstdio>
#include <cstdlib>
#include <string>
#include <vector>

#include "../../mlxcat_amd/csrc/mc_fused.hip"
#include "emu.hpp"

extern "C" {
#include "../../oracle/oracle.h"
}

using namespace mc;

// the library's error plumbing (mc_api.hip is not part of this harness)
namespace mc {
int fail(int code, const std::string& msg) {
  fprintf(stderr, "error %d: %s\n", code, msg.c_str());
  return code;
}
int hip_fail(hipError_t e, const char* what, const char* file, int line) {
  fprintf(stderr, "hip error %d in %s (%s:%d)\n", e, what, file, line);
  return -2;
}
}  // namespace mc

static void* dalloc(size_t bytes, const char* name) {
  void* p = emu::dalloc(bytes, name);
  memset(p, 0, bytes);
  return p;
}

// ---------------------------------------------------------------------------------------
// the model, taken from the oracle (same seeded tensors), in the GPU's tile layout
// ---------------------------------------------------------------------------------------
static const uint64_t SEED = 1234;

static size_t tile_word(const QLinear& L, int nd, int kw) {
  const int t = nd >> 4, r = nd & 15;
  const int g = kw >> 3, w8 = kw & 7, am = w8 >> 2, c = w8 & 3;
  const int gp = g >> 1, gi = g & 1;
  return (((size_t)t * L.GP + gp) * 64 + c * 16 + r) * 4 + gi * 2 + am;
}

static QLinear new_linear(int N, int K, const char* name) {
  QLinear L;
  L.N = N;
  L.K = K;
  L.NT = (N + 15) / 16;
  L.GP = (K + 127) / 128;
  L.qw = (uint32_t*)dalloc(L.qw_words() * 4, name);
  L.sb = (uint32_t*)dalloc(L.sb_words() * 4, name);
  return L;
}

// rows row_off + n * row_stride of L <- the oracle tensor (N rows of K inputs)
static void put(QLinear& L, or_model* om, int layer, int which, int row_off, int row_stride) {
  const uint32_t* wq;
  const uint16_t *s, *b;
  int N, K;
  if (or_model_linear(om, layer, which, -1, &wq, &s, &b, &N, &K)) abort();
  const int KW = K / 8, G = K / 64;
  for (int n = 0; n < N; ++n) {
    const int nd = row_off + n * row_stride;
    for (int kw = 0; kw < KW; ++kw) L.qw[tile_word(L, nd, kw)] = permute_mlx_word(wq[(size_t)n * KW + kw]);
    for (int g = 0; g < G; ++g)
      L.sb[tile_sb_word(nd >> 4, nd & 15, g >> 1, g & 1, L.GP)] =
          (uint32_t)s[(size_t)n * G + g] | ((uint32_t)b[(size_t)n * G + g] << 16);
  }
}

static uint16_t* norm(uint64_t tid, int n, const char* name) {
  uint16_t* w = (uint16_t*)dalloc((size_t)n * 2, name);
  or_gen_norm(SEED, tid, n, w);
  return w;
}

struct Scenario {
  int R;
  std::vector<int> T, NV;
};

int main(int argc, char** argv) {
  const int scen = argc > 1 ? atoi(argv[1]) : 0;
  const int G = argc > 2 ? atoi(argv[2]) : 8;
  emu::install_fault_handler();
  emu::set_persistent((const void*)fused_forward_kernel);

  // head_dim 128, GQA group 2, widths multiples of 256: the smallest shape the kernel serves
  mc_model_config c{};
  c.arch = 0; c.n_layers = 2; c.hidden = 256; c.n_q_heads = 4; c.n_kv_heads = 2; c.head_dim = 128;
  c.intermediate = 512; c.vocab = 4096; c.tied_embeddings = 1; c.rms_eps = 1e-6f; c.rope_theta = 1e6f;
  Scenario sc;
  int max_ctx = 1100;
  if (scen == 0) sc = Scenario{1, {1000}, {6}};
  else if (scen == 1) sc = Scenario{3, {30, 9, 300}, {3, 1, 3}};
  else if (scen == 2) sc = Scenario{1, {40}, {8}};
  else {
    c.hidden = 2560; c.n_q_heads = 32; c.n_kv_heads = 8; c.intermediate = 9728; c.vocab = 151936;
    sc = Scenario{1, {40}, {6}};
    max_ctx = 256;
  }
  const char* why = nullptr;
  const int cap = (max_ctx + 63) / 64 * 64;
  int M = 0;
  for (int v : sc.NV) M += v;
  if (!fused_supported(c, M, cap, &why)) {
    fprintf(stderr, "unsupported: %s\n", why);
    return 2;
  }
  or_config oc{c.arch, c.n_layers, c.hidden, c.n_q_heads, c.n_kv_heads, c.head_dim, c.intermediate, c.vocab,
               c.tied_embeddings, c.rms_eps, c.rope_theta, 0, 0, 0};
  or_model* om = or_model_create(&oc, SEED, max_ctx, sc.R);
  const int H = c.hidden, d = c.head_dim, nq = c.n_q_heads, nkv = c.n_kv_heads, I = c.intermediate, V = c.vocab;
  const int Lyr = c.n_layers;

  // weights
  std::vector<FwLayer> layers((size_t)Lyr);
  for (int l = 0; l < Lyr; ++l) {
    QLinear qkv = new_linear((nq + 2 * nkv) * d, H, "qkv"), o = new_linear(H, nq * d, "o");
    QLinear gu = new_linear(2 * I, H, "gateup"), dn = new_linear(H, I, "down");
    put(qkv, om, l, OR_T_Q, 0, 1);
    put(qkv, om, l, OR_T_K, nq * d, 1);
    put(qkv, om, l, OR_T_V, (nq + nkv) * d, 1);
    put(o, om, l, OR_T_O, 0, 1);
    put(gu, om, l, OR_T_GATE, 0, 2);
    put(gu, om, l, OR_T_UP, 1, 2);
    put(dn, om, l, OR_T_DOWN, 0, 1);
    FwLayer& f = layers[(size_t)l];
    f.qkv = fused_lin(qkv, 1);
    f.o = fused_lin(o, 4);
    f.gu = fused_lin(gu, 1);
    f.dn = fused_lin(dn, 4);
    f.in_norm = norm(or_tensor_id(l, OR_T_IN_NORM), H, "in_norm");
    f.post_norm = norm(or_tensor_id(l, OR_T_POST_NORM), H, "post_norm");
    f.q_norm = norm(or_tensor_id(l, OR_T_Q_NORM), d, "q_norm");
    f.k_norm = norm(or_tensor_id(l, OR_T_K_NORM), d, "k_norm");
    f.k = (uint16_t*)dalloc((size_t)sc.R * nkv * cap * d * 2, "kcache");
    f.v = (uint16_t*)dalloc((size_t)sc.R * nkv * cap * d * 2, "vcache");
  }
  QLinear emb = new_linear(V, H, "embed");
  put(emb, om, -1, 0, 0, 1);
  FwLayer* dlayers = (FwLayer*)dalloc(layers.size() * sizeof(FwLayer), "layers");
  memcpy(dlayers, layers.data(), layers.size() * sizeof(FwLayer));

  // cached context: the oracle's synthetic K/V, copied into the kernel's layouts
  for (int r = 0; r < sc.R; ++r) {
    or_kv_fill_synthetic(om, r, sc.T[(size_t)r], 77 + r);
    const int T = sc.T[(size_t)r];
    std::vector<uint16_t> kv((size_t)nkv * T * d);
    for (int l = 0; l < Lyr; ++l)
      for (int w = 0; w < 2; ++w) {
        or_kv_read(om, l, r, w, kv.data());
        for (int h = 0; h < nkv; ++h)
          for (int p = 0; p < T; ++p)
            for (int e = 0; e < d; ++e) {
              const uint16_t x = kv[((size_t)h * T + p) * d + e];
              const size_t head = (size_t)r * nkv + h;
              if (w) layers[(size_t)l].v[(head * d + e) * cap + p] = x;
              else layers[(size_t)l].k[(head * cap + p) * d + e] = x;
            }
      }
  }
  float* rc = (float*)dalloc((size_t)max_ctx * d / 2 * 4, "rope_cos");
  float* rs = (float*)dalloc((size_t)max_ctx * d / 2 * 4, "rope_sin");
  memcpy(rc, or_model_rope_cos(om), (size_t)max_ctx * d / 2 * 4);
  memcpy(rs, or_model_rope_sin(om), (size_t)max_ctx * d / 2 * 4);

  // LL buffers and the rest of the arguments, as fused_setup lays them out
  const int npb = fused_npb_cap(cap);
  const size_t mm = FW_MMAX, Nqkv = (size_t)(nq + 2 * nkv) * d;
  FwArgs a;
  a.x = (unsigned long long*)dalloc(mm * H / 2 * 8, "x");
  a.xss = (unsigned long long*)dalloc(mm * H / 16 * 8, "xss");
  a.qkv = (unsigned long long*)dalloc(mm * Nqkv / 2 * 8, "qkv");
  a.att = (unsigned long long*)dalloc(mm * nq * d / 2 * 8, "att");
  a.act = (unsigned long long*)dalloc(mm * I / 2 * 8, "act");
  a.opart = (unsigned long long*)dalloc((size_t)layers[0].o.ks * mm * H * 8, "opart");
  a.dpart = (unsigned long long*)dalloc((size_t)layers[0].dn.ks * mm * H * 8, "dpart");
  a.ao = (unsigned long long*)dalloc((size_t)sc.R * nkv * npb * FW_QROWS * d * 8, "ao");
  a.aml = (unsigned long long*)dalloc((size_t)sc.R * nkv * npb * FW_QROWS * 2 * 8, "aml");
  a.npb_cap = npb;
  a.layers = dlayers;
  a.L = Lyr;
  a.embed = emb;
  a.head = fused_lin(emb, 1);
  a.final_norm = norm(OR_TID_FINAL_NORM, H, "final_norm");
  a.H = H; a.nq = nq; a.nkv = nkv; a.d = d; a.I = I; a.V = V;
  a.eps = c.rms_eps;
  a.scale = 1.0f / sqrtf((float)d);
  a.rope_cos = rc;
  a.rope_sin = rs;
  a.cap = cap;
  a.R = sc.R;
  a.M = M;
  a.with_head = 1;
  int32_t* slot_tok = (int32_t*)dalloc(mm * 4, "slot_tok");
  int32_t* slot_row = (int32_t*)dalloc(mm * 4, "slot_row");
  int32_t* row_slot0 = (int32_t*)dalloc((size_t)sc.R * 4, "row_slot0");
  int32_t* n_valid = (int32_t*)dalloc((size_t)sc.R * 4, "n_valid");
  int32_t* qbase = (int32_t*)dalloc((size_t)sc.R * 4, "qbase");
  a.slot_tok = slot_tok; a.slot_row = slot_row; a.row_slot0 = row_slot0; a.n_valid = n_valid; a.qbase = qbase;
  a.logits = (uint16_t*)dalloc((size_t)M * V * 2, "logits");
  a.amax = (unsigned long long*)dalloc((size_t)M * a.head.NT * 8, "amax");
  unsigned* ctl = (unsigned*)dalloc(8, "ctl");
  ctl[0] = 1;
  a.epoch = ctl;
  a.err = ctl + 1;

  int bad = 0;
  uint64_t rng = 0x9E3779B97F4A7C15ull;
  for (int call = 0; call < 2; ++call) {
    // tokens and slots (rows packed in order)
    std::vector<int32_t> toks((size_t)M), rows, counts;
    for (auto& t : toks) {
      rng = or_mix64(rng);
      t = (int32_t)(rng % (uint64_t)V);
    }
    int s0 = 0;
    for (int r = 0; r < sc.R; ++r) {
      row_slot0[r] = s0;
      n_valid[r] = sc.NV[(size_t)r];
      qbase[r] = or_kv_len(om, r);
      for (int j = 0; j < sc.NV[(size_t)r]; ++j) slot_row[s0 + j] = r;
      s0 += sc.NV[(size_t)r];
      rows.push_back(r);
      counts.push_back(sc.NV[(size_t)r]);
    }
    for (int m = 0; m < M; ++m) slot_tok[m] = toks[(size_t)m];
    if (launch_fused_forward(a, G, nullptr)) {
      printf("call %d: launch failed\n", call);
      return 1;
    }
    ctl[0] += 1;  // the epoch bump kernel
    printf("call %d: err word %u, out-of-range buffer loads %lld stores %lld\n", call, ctl[1], emu::oob_loads,
           emu::oob_stores);
    bad += ctl[1] != 0 || emu::oob_loads != 0 || emu::oob_stores != 0;
    // oracle
    std::vector<uint16_t> want((size_t)M * V);
    or_forward(om, (int)rows.size(), rows.data(), counts.data(), toks.data(), want.data());
    int outside = 0;
    double maxerr = 0;
    for (size_t i = 0; i < want.size(); ++i) {
      const double g = bf16_to_f32(a.logits[i]), w = bf16_to_f32(want[i]);
      const double e = fabs(g - w);
      maxerr = std::max(maxerr, e);
      if (!(e <= 2e-2 + 1e-2 * fabs(w))) ++outside;
    }
    printf("call %d: logits %d of %zu outside 2e-2 + 1e-2 rel, max err %.4g\n", call, outside, want.size(), maxerr);
    bad += outside > 0;
    // appended K / V
    int kv_out = 0;
    for (int r = 0; r < sc.R; ++r) {
      const int T1 = or_kv_len(om, r);
      std::vector<uint16_t> kv((size_t)nkv * T1 * d);
      for (int l = 0; l < Lyr; ++l)
        for (int w = 0; w < 2; ++w) {
          or_kv_read(om, l, r, w, kv.data());
          for (int h = 0; h < nkv; ++h)
            for (int p = qbase[r]; p < T1; ++p)
              for (int e = 0; e < d; ++e) {
                const size_t head = (size_t)r * nkv + h;
                const uint16_t g = w ? layers[(size_t)l].v[(head * d + e) * cap + p] : layers[(size_t)l].k[(head * cap + p) * d + e];
                const double x = bf16_to_f32(g), y = bf16_to_f32(kv[((size_t)h * T1 + p) * d + e]);
                if (!(fabs(x - y) <= 2e-2 + 1e-2 * fabs(y))) ++kv_out;
              }
        }
    }
    printf("call %d: appended K/V values outside the tolerance: %d\n", call, kv_out);
    bad += kv_out > 0;
  }
  printf("%s\n", bad ? "FAIL" : "OK");
  or_model_destroy(om);
  return bad ? 1 : 0;
}
