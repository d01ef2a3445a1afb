// The library's C ABI running on the CPU emulation (all kernels and the host code of
// mlxcat_amd/csrc compiled as host C++), checked against the oracle.  Test infrastructure.
//
// usage: lib_emu <case>
//   case 0: small head_dim-128 model; 40-token prefill, then verify blocks of 6, 1 and 8
//           tokens; logits and the whole K/V against the oracle
//   case 1: the same as case 0 (kept for the numbering of older notes)
//   case 2: Qwen3-4B shape (2 layers): 40-token prefill, a 6-token verify
//   case 3: case 0 with 32 q / 8 kv heads, hidden 512 (GQA group 4, eight kv heads)
//   case 4: the case-3 model through mc_step (verify blocks with padding slots; MC_STEP_EAGER=1)
//   case 5: a small Qwen3-MoE model (16 experts, top-4)
//   case 6: the case-0 model, 12 rows: one verify block of 12 x 6 = 72 tokens (the M > 64 GEMM)
// exit status 0 when everything matches.
#include <cstdio>
#include <cstdlib>
#include <cmath>
#include <cstring>
#include <string>
#include <vector>

#include "../../include/mlxcat_hip.h"
#include "emu.hpp"

extern "C" {
#include "../../oracle/oracle.h"
}

static int g_bad = 0;

static void check(int rc, const char* what) {
  if (rc < 0) {
    printf("%s: error %d: %s\n", what, rc, mc_last_error());
    exit(1);
  }
}

static float bf(uint16_t h) {
  const uint32_t u = (uint32_t)h << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

// bf16 values against the oracle's: count outside 2e-2 abs + 1e-2 rel
static void compare(const char* what, const uint16_t* got, const uint16_t* want, size_t n, size_t allowed) {
  size_t out = 0;
  double mx = 0;
  for (size_t i = 0; i < n; ++i) {
    const double g = bf(got[i]), w = bf(want[i]), e = fabs(g - w);
    mx = e > mx ? e : mx;
    if (!(e <= 2e-2 + 1e-2 * fabs(w))) ++out;
  }
  printf("%s: %zu of %zu outside the tolerance (max err %.4g)\n", what, out, n, mx);
  if (out > allowed) ++g_bad;
}

int main(int argc, char** argv) {
  const int cs = argc > 1 ? atoi(argv[1]) : 0;
  emu::install_fault_handler();
  check(mc_set_device(0), "set_device");
  mc_model_config c{};
  c.arch = 0; c.n_layers = 2; c.hidden = 256; c.n_q_heads = 4; c.n_kv_heads = 2; c.head_dim = 128;
  c.intermediate = 512; c.vocab = 4096; c.tied_embeddings = 1; c.rms_eps = 1e-6f; c.rope_theta = 1e6f;
  if (cs == 2) {
    c.hidden = 2560; c.n_q_heads = 32; c.n_kv_heads = 8; c.intermediate = 9728; c.vocab = 151936;
  }
  if (cs == 3) {  // 8 kv heads, GQA group 4
    c.hidden = 512; c.n_q_heads = 32; c.n_kv_heads = 8; c.intermediate = 1024; c.vocab = 4096;
  }
  if (cs == 4) {  // speculative steps: padding slots
    c.hidden = 512; c.n_q_heads = 32; c.n_kv_heads = 8; c.intermediate = 1024; c.vocab = 4096;
  }
  if (cs == 5) {  // Qwen3-MoE: 16 experts of width 128, top-4 (a 40-token prefill gives experts > 16 pairs)
    c.arch = MC_ARCH_QWEN3_MOE; c.n_experts = 16; c.n_experts_per_tok = 4; c.moe_intermediate = 128;
  }
  const uint64_t SEED = 1234;
  const int ctx = 256, V = c.vocab;
  mc_model* m = nullptr;
  check(mc_model_create(&c, &m), "model_create");
  check(mc_model_init_synthetic(m, SEED), "init_synthetic");
  mc_spec_config spec{1, 5, 3, 8, 1, 0, 0};
  mc_batch* b = nullptr;
  check(mc_batch_create(m, 1, ctx, 5, &spec, &b), "batch_create");
  if (cs == 4) {
    // a prompt without repeats (no drafts: one valid slot of six) and a repeating one
    // (drafts), each stepped twice from a fresh batch (the two runs must agree)
    std::vector<std::vector<int32_t>> outs;
    for (int pass = 0; pass < 4; ++pass) {
      mc_batch* bb = nullptr;
      check(mc_batch_create(m, 1, ctx, 5, &spec, &bb), "batch_create");
      std::vector<int32_t> prompt(48);
      for (int i = 0; i < 48; ++i) prompt[(size_t)i] = pass < 2 ? (i * 37 + 11) % V : 100 + (i % 8);
      mc_sampling sp{};
      sp.reject_token = -1;
      int32_t first = 0, fin = 0;
      check(mc_batch_insert(bb, 0, prompt.data(), 48, 24, &sp, &first, &fin), "insert");
      std::vector<int32_t> toks{first};
      for (int st = 0; st < 6; ++st) {
        int32_t ot[6], cnt[1], f[1];
        check(mc_step(bb, nullptr, ot, cnt, f), "step");
        for (int k = 0; k < cnt[0]; ++k) toks.push_back(ot[k]);
        if (cnt[0] == 0) break;
      }
      printf("pass %d (%s): %zu tokens:", pass, pass < 2 ? "no repeats" : "repeats", toks.size());
      for (int t : toks) printf(" %d", t);
      printf("\n");
      outs.push_back(toks);
      mc_batch_destroy(bb);
    }
    if (outs[0] != outs[1] || outs[2] != outs[3]) { printf("repeated runs differ\n"); ++g_bad; }
    printf("out-of-range buffer accesses: loads %lld stores %lld\n", emu::oob_loads, emu::oob_stores);
    if (emu::oob_loads || emu::oob_stores) ++g_bad;
    printf("%s\n", g_bad ? "FAIL" : "OK");
    return g_bad ? 1 : 0;
  }
  or_config oc{c.arch, c.n_layers, c.hidden, c.n_q_heads, c.n_kv_heads, c.head_dim, c.intermediate, c.vocab,
               c.tied_embeddings, c.rms_eps, c.rope_theta, c.n_experts, c.n_experts_per_tok, c.moe_intermediate};
  if (cs == 6) {
    const int R = 12, W = 6;
    mc_batch* bb = nullptr;
    check(mc_batch_create(m, R, ctx, W - 1, &spec, &bb), "batch_create");
    or_model* om6 = or_model_create(&oc, SEED, ctx, R);
    uint64_t rng6 = 0x7777ull;
    auto toks6 = [&](int n) {
      std::vector<int32_t> t((size_t)n);
      for (auto& x : t) { rng6 = or_mix64(rng6); x = (int32_t)(rng6 % (uint64_t)V); }
      return t;
    };
    for (int32_t r = 0; r < R; ++r) {  // prefill: 10 + r tokens per row
      const int32_t n = 10 + r;
      auto t = toks6(n);
      check(mc_forward(bb, 1, &r, &n, t.data(), nullptr), "prefill");
      or_forward(om6, 1, &r, &n, t.data(), nullptr);
    }
    std::vector<int32_t> rows(R), cnts(R, W);
    for (int r = 0; r < R; ++r) rows[(size_t)r] = r;
    auto t = toks6(R * W);
    std::vector<uint16_t> got((size_t)R * W * V), want(got.size());
    check(mc_forward(bb, R, rows.data(), cnts.data(), t.data(), got.data()), "verify");
    or_forward(om6, R, rows.data(), cnts.data(), t.data(), want.data());
    compare("verify 12 x 6 logits", got.data(), want.data(), got.size(), 0);
    for (int l = 0; l < c.n_layers; ++l)
      for (int wv = 0; wv < 2; ++wv) {
        int32_t len = 0;
        check(mc_batch_kv_len(bb, 11, &len), "kv_len");
        std::vector<uint16_t> g2((size_t)c.n_kv_heads * len * c.head_dim), w2(g2.size());
        check(mc_batch_read_kv(bb, l, 11, wv, g2.data()), "read_kv");
        or_kv_read(om6, l, 11, wv, w2.data());
        const std::string what = "row 11 kv layer " + std::to_string(l) + (wv ? " V" : " K");
        compare(what.c_str(), g2.data(), w2.data(), g2.size(), 0);
      }
    printf("out-of-range buffer accesses: loads %lld stores %lld\n", emu::oob_loads, emu::oob_stores);
    if (emu::oob_loads || emu::oob_stores) ++g_bad;
    printf("%s\n", g_bad ? "FAIL" : "OK");
    return g_bad ? 1 : 0;
  }
  or_model* om = or_model_create(&oc, SEED, ctx, 1);
  uint64_t rng = 0x1234567ull;
  auto tokens = [&](int n) {
    std::vector<int32_t> t((size_t)n);
    for (auto& x : t) {
      rng = or_mix64(rng);
      x = (int32_t)(rng % (uint64_t)V);
    }
    return t;
  };
  const int32_t row0 = 0;
  {
    const int32_t n = 40;
    auto t = tokens(n);
    check(mc_forward(b, 1, &row0, &n, t.data(), nullptr), "prefill");
    or_forward(om, 1, &row0, &n, t.data(), nullptr);
    printf("prefill done\n");
  }
  const std::vector<int> widths = cs == 2 ? std::vector<int>{6} : std::vector<int>{6, 1, 8};
  for (int w : widths) {
    auto t = tokens(w);
    std::vector<uint16_t> got((size_t)w * V), want((size_t)w * V);
    const int32_t n = w;
    check(mc_forward(b, 1, &row0, &n, t.data(), got.data()), "verify");
    or_forward(om, 1, &row0, &n, t.data(), want.data());
    const std::string what = "verify " + std::to_string(w) + " logits";
    compare(what.c_str(), got.data(), want.data(), got.size(), cs == 2 ? got.size() / 1000 : 0);
  }
  int32_t len = 0;
  check(mc_batch_kv_len(b, 0, &len), "kv_len");
  printf("kv_len %d (oracle %d)\n", len, or_kv_len(om, 0));
  if (len != or_kv_len(om, 0)) ++g_bad;
  for (int l = 0; l < c.n_layers; ++l)
    for (int wv = 0; wv < 2; ++wv) {
      std::vector<uint16_t> got((size_t)c.n_kv_heads * len * c.head_dim), want(got.size());
      check(mc_batch_read_kv(b, l, 0, wv, got.data()), "read_kv");
      or_kv_read(om, l, 0, wv, want.data());
      const std::string what = "kv layer " + std::to_string(l) + (wv ? " V" : " K");
      compare(what.c_str(), got.data(), want.data(), got.size(), 0);
    }
  printf("out-of-range buffer accesses: loads %lld stores %lld\n", emu::oob_loads, emu::oob_stores);
  if (emu::oob_loads || emu::oob_stores) ++g_bad;
  mc_batch_destroy(b);
  mc_model_destroy(m);
  or_model_destroy(om);
  printf("%s\n", g_bad ? "FAIL" : "OK");
  return g_bad ? 1 : 0;
}
