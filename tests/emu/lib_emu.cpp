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
//   case 7: mc_accept with random sampler options against or_accept_row
//   case 8: mc_accept_noalloc against mc_accept, two calls
//   case 9: the case-4 model, 4 rows: mc_batch_filter (a 3-cycle; a repeated row) and
//           mc_batch_extract_kv + mc_batch_insert_prefilled against an unfiltered batch
//   case 10: the case-4 model: prefix blocks exported, imported, and mc_batch_insert_cached
// exit status 0 when everything matches.
#include <cstdio>
#include <cstdlib>
#include <cmath>
#include <cstring>
#include <string>
#include <vector>

#include "../../include/mlxcat_hip.h"
#include "emu.hpp"
#include <hip/hip_runtime.h>

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

// case 7: mc_accept over host logits with random sampler options (temperature, top-p,
// top-k, min-p, logit bias, min_tokens, penalties over generated histories, caller or
// derived uniforms) against or_accept_row, token for token.
static uint64_t rng_state = 0x1234567ull;
static uint32_t rnd(uint32_t n) { return (uint32_t)(or_mix64(rng_state++) % n); }

static int accept_case(int argc_trials) {
  const int V = 3000, B = 6, KD = 5;
  const int trials = argc_trials > 0 ? argc_trials : 12;
  for (int trial = 0; trial < trials; ++trial) {
    std::vector<int32_t> nd(B), dr((size_t)B * KD, 0);
    std::vector<int64_t> off(B + 1, 0), goff(B + 1, 0);
    std::vector<int32_t> gen;
    std::vector<mc_sampling> sp(B);
    std::vector<or_sampling> osp(B);
    std::vector<uint64_t> ctr(B);
    const bool use_u = trial % 2 == 1;
    std::vector<uint32_t> uni((size_t)B * (KD + 1) * 2);
    for (auto& u : uni) u = (uint32_t)or_mix64(rng_state++);
    for (int r = 0; r < B; ++r) {
      nd[r] = (int)rnd(KD + 1);
      off[r + 1] = off[r] + nd[r] + 1;
      ctr[r] = rnd(100);
      mc_sampling q;
      memset(&q, 0, sizeof q);
      const float temps[] = {0.f, 0.7f, 1.0f, 1.5f};
      const float tops[] = {0.f, 0.9f, 0.5f};
      const int topks[] = {0, 1, 5, 50};
      const float minps[] = {0.f, 0.05f, 0.3f};
      const float reps[] = {1.f, 1.3f, 0.8f, 0.f};
      q.temperature = temps[rnd(4)];
      q.top_p = tops[rnd(3)];
      q.top_k = topks[rnd(4)];
      q.min_p = minps[rnd(3)];
      q.repetition_penalty = reps[rnd(4)];
      q.presence_penalty = rnd(2) ? 0.5f : 0.f;
      q.frequency_penalty = rnd(2) ? 0.25f : 0.f;
      q.min_tokens = 0;  // set below, around the generated count
      q.has_seed = 1;
      q.seed = or_mix64(trial * 100 + r);
      q.n_eos = (int)rnd(3);
      for (int i = 0; i < q.n_eos; ++i) q.eos[i] = (int)rnd(rnd(2) ? 12 : 40);
      q.reject_token = -1;
      q.n_bias = (int)rnd(4);
      for (int i = 0; i < q.n_bias; ++i) {
        q.bias_token[i] = rnd(8) == 0 ? V + 5 : (int)rnd(40);
        q.bias_value[i] = rnd(2) ? 2.5f : -1.75f;
      }
      // generated tokens from a small pool (counts above 1), drafts often from it too
      const int ng = (int)rnd(16);
      for (int i = 0; i < ng; ++i) gen.push_back((int)rnd(12));
      goff[r + 1] = goff[r] + ng;
      if (rnd(2)) q.min_tokens = ng + (int)rnd(4);  // the mask ends inside the verify block
      for (int j = 0; j < nd[r]; ++j) dr[(size_t)r * KD + j] = (int)rnd(rnd(2) ? 12 : 40);
      sp[r] = q;
      static_assert(sizeof(mc_sampling) == sizeof(or_sampling), "same layout");
      memcpy(&osp[r], &q, sizeof q);
    }
    // logits: few distinct bf16 values (ties everywhere), the first 40 ids larger
    std::vector<uint16_t> lg((size_t)off[B] * V);
    for (size_t i = 0; i < lg.size(); ++i) {
      const int id = (int)(i % V);
      const float v = id < 12 ? (float)((int)rnd(12) + 6) * 0.5f
                      : id < 40 ? (float)((int)rnd(24) - 4) * 0.5f : (float)((int)rnd(16) - 20) * 0.5f;
      lg[i] = or_f32_to_bf16(v);
    }
    std::vector<int32_t> out((size_t)B * (KD + 1)), ne(B), keep(B), nacc(B);
    check(mc_accept(lg.data(), V, B, off.data(), dr.data(), KD, nd.data(), sp.data(), gen.data(), goff.data(),
                    ctr.data(), use_u ? uni.data() : nullptr, trial % 3 == 0 ? 0 : 1, out.data(), ne.data(), keep.data(),
                    nacc.data()),
          "mc_accept");
    for (int r = 0; r < B; ++r) {
      std::vector<int32_t> want(KD + 1);
      int wk, wn, wr;
      const int n = or_accept_row(lg.data() + (size_t)off[r] * V, V, dr.data() + (size_t)r * KD, nd[r], &osp[r],
                                  gen.data() + goff[r], (int)(goff[r + 1] - goff[r]), sp[r].seed, ctr[r],
                                  use_u ? uni.data() + (size_t)r * (KD + 1) * 2 : nullptr, trial % 3 == 0 ? 0 : 1, -1, 0,
                                  want.data(), &wk, &wn, &wr);
      bool same = n == ne[r] && wk == keep[r] && wn == nacc[r];
      for (int j = 0; same && j < n; ++j) same = want[j] == out[(size_t)r * (KD + 1) + j];
      if (!same) {
        ++g_bad;
        printf("trial %d row %d: T %.2f top_p %.2f top_k %d min_p %.2f rp %.2f pp %.2f fp %.2f min_tokens %d "
               "bias %d: got n %d keep %d acc %d [%d %d], want n %d keep %d acc %d [%d %d]\n",
               trial, r, sp[r].temperature, sp[r].top_p, sp[r].top_k, sp[r].min_p, sp[r].repetition_penalty,
               sp[r].presence_penalty, sp[r].frequency_penalty, sp[r].min_tokens, sp[r].n_bias, ne[r], keep[r],
               nacc[r], out[(size_t)r * (KD + 1)], ne[r] > 1 ? out[(size_t)r * (KD + 1) + 1] : -1, n, wk, wn, want[0],
               n > 1 ? want[1] : -1);
      }
    }
    printf("trial %d done\n", trial);
    fflush(stdout);
  }
  printf("out-of-range buffer accesses: loads %lld stores %lld\n", emu::oob_loads, emu::oob_stores);
  if (emu::oob_loads || emu::oob_stores) ++g_bad;
  printf("%s\n", g_bad ? "FAIL" : "OK");
  return g_bad ? 1 : 0;
}

// case 8: mc_accept_noalloc against mc_accept (no generated history) on the same inputs,
// two calls in a row, the second smaller; caller uniforms on the second.
template <class T>
static T* dev_copy(const std::vector<T>& h) {
  T* d = nullptr;
  check(hipMalloc((void**)&d, h.size() * sizeof(T)) == hipSuccess ? 0 : -1, "hipMalloc");
  check(hipMemcpy(d, h.data(), h.size() * sizeof(T), hipMemcpyHostToDevice) == hipSuccess ? 0 : -1, "copy");
  return d;
}

static int noalloc_case() {
  const int V = 3000;
  const int shapes[2][2] = {{6, 5}, {3, 2}};  // (B, K)
  for (int call = 0; call < 2; ++call) {
    const int B = shapes[call][0], K = shapes[call][1], K1 = K + 1;
    std::vector<int32_t> nd(B), dr((size_t)B * std::max(K, 1), 0);
    std::vector<mc_sampling> sp(B);
    std::vector<uint64_t> ctr(B);
    std::vector<uint32_t> uni((size_t)B * K1 * 2);
    for (auto& u : uni) u = (uint32_t)or_mix64(rng_state++);
    std::vector<uint16_t> lg((size_t)B * K1 * V);
    for (size_t i = 0; i < lg.size(); ++i) {
      const int id = (int)(i % V);
      lg[i] = or_f32_to_bf16(id < 12 ? (float)((int)rnd(12) + 6) * 0.5f : (float)((int)rnd(16) - 20) * 0.5f);
    }
    for (int r = 0; r < B; ++r) {
      nd[r] = (int)rnd(K + 1);
      for (int j = 0; j < nd[r]; ++j) {  // mostly the position's argmax: long accepted prefixes
        const uint16_t* row = lg.data() + ((size_t)r * K1 + j) * V;
        int am = 0;
        for (int i = 1; i < V; ++i)
          if (bf(row[i]) > bf(row[am])) am = i;
        dr[(size_t)r * K + j] = rnd(4) ? am : (int)rnd(12);
      }
      mc_sampling q;
      memset(&q, 0, sizeof q);
      q.temperature = r % 2 ? 0.8f : 0.f;
      q.top_p = r % 3 == 1 ? 0.9f : 0.f;
      q.top_k = r == 3 ? 4 : 0;
      q.presence_penalty = r == 2 ? 1.0f : 0.f;
      q.n_bias = r == 4 ? 1 : 0;
      q.bias_token[0] = 5;
      q.bias_value[0] = 3.0f;
      q.has_seed = 1;
      q.seed = 900 + r;
      q.reject_token = -1;
      sp[r] = q;
      ctr[r] = rnd(50);
    }
    // mc_accept over host buffers: row r's logits rows at r*K1 .. r*K1 + nd[r]
    std::vector<int64_t> off(B + 1, 0);
    std::vector<uint16_t> packed;
    for (int r = 0; r < B; ++r) {
      off[r + 1] = off[r] + nd[r] + 1;
      packed.insert(packed.end(), lg.begin() + (size_t)r * K1 * V, lg.begin() + ((size_t)r * K1 + nd[r] + 1) * V);
    }
    const uint32_t* use_u = call == 1 ? uni.data() : nullptr;
    std::vector<int32_t> want((size_t)B * K1, -7), wne(B), wkeep(B), wnacc(B);
    check(mc_accept(packed.data(), V, B, off.data(), dr.data(), K, nd.data(), sp.data(), nullptr, nullptr, ctr.data(),
                    use_u, 1, want.data(), wne.data(), wkeep.data(), wnacc.data()),
          "mc_accept");
    uint16_t* d_lg = dev_copy(lg);
    int32_t* d_dr = dev_copy(dr);
    int32_t* d_nd = dev_copy(nd);
    uint32_t* d_u = dev_copy(uni);
    std::vector<int32_t> zeros((size_t)B * K1, -7), zr(B, 0);
    int32_t *d_out = dev_copy(zeros), *d_ne = dev_copy(zr), *d_keep = dev_copy(zr), *d_nacc = dev_copy(zr);
    check(mc_accept_noalloc(d_lg, V, B, K, d_dr, d_nd, sp.data(), ctr.data(), call == 1 ? d_u : nullptr, 1, d_out, d_ne,
                            d_keep, d_nacc),
          "mc_accept_noalloc");
    std::vector<int32_t> got((size_t)B * K1), ne(B), keep(B), nacc(B);
    hipMemcpy(got.data(), d_out, got.size() * 4, hipMemcpyDeviceToHost);
    hipMemcpy(ne.data(), d_ne, B * 4, hipMemcpyDeviceToHost);
    hipMemcpy(keep.data(), d_keep, B * 4, hipMemcpyDeviceToHost);
    hipMemcpy(nacc.data(), d_nacc, B * 4, hipMemcpyDeviceToHost);
    for (int r = 0; r < B; ++r) {
      bool same = ne[r] == wne[r] && keep[r] == wkeep[r] && nacc[r] == wnacc[r];
      for (int j = 0; same && j < ne[r]; ++j) same = got[(size_t)r * K1 + j] == want[(size_t)r * K1 + j];
      printf("call %d row %d: n %d keep %d acc %d %s\n", call, r, ne[r], keep[r], nacc[r], same ? "same" : "DIFFERENT");
      if (!same) ++g_bad;
    }
    for (void* p : {(void*)d_lg, (void*)d_dr, (void*)d_nd, (void*)d_u, (void*)d_out, (void*)d_ne, (void*)d_keep,
                    (void*)d_nacc})
      hipFree(p);
  }
  printf("%s\n", g_bad ? "FAIL" : "OK");
  return g_bad ? 1 : 0;
}

// case 9: rows moved by mc_batch_filter keep producing what they produce in a batch that was
// not filtered, and a row's K/V extracted into another batch continues the same way.
static std::vector<int32_t> case9_prompt(int r, int V) {
  std::vector<int32_t> p((size_t)(40 + 4 * r));
  for (size_t i = 0; i < p.size(); ++i) p[i] = r == 2 ? (int32_t)((i * 37 + 11) % V) : 100 + r + (int32_t)(i % (5 + r));
  return p;
}
static mc_sampling case9_sampling(int r) {
  mc_sampling sp{};
  sp.reject_token = -1;
  if (r == 1) { sp.temperature = 0.8f; sp.has_seed = 1; sp.seed = 77; sp.presence_penalty = 0.5f; }
  return sp;
}
static std::vector<std::vector<int32_t>> case9_steps(mc_batch* b, int R, int K1, int n) {
  std::vector<std::vector<int32_t>> out((size_t)R);
  for (int st = 0; st < n; ++st) {
    std::vector<int32_t> ot((size_t)R * K1), cnt((size_t)R), f((size_t)R);
    check(mc_step(b, nullptr, nullptr, ot.data(), cnt.data(), f.data()), "step");
    for (int r = 0; r < R; ++r)
      for (int k = 0; k < cnt[(size_t)r]; ++k) out[(size_t)r].push_back(ot[(size_t)r * K1 + k]);
  }
  return out;
}
static bool case9_same_kv(mc_batch* a, int ra, mc_batch* b, int rb, const mc_model_config& c) {
  int32_t la = 0, lb = 0;
  check(mc_batch_kv_len(a, ra, &la), "kv_len");
  check(mc_batch_kv_len(b, rb, &lb), "kv_len");
  if (la != lb) return false;
  for (int l = 0; l < c.n_layers; ++l)
    for (int wv = 0; wv < 2; ++wv) {
      std::vector<uint16_t> x((size_t)c.n_kv_heads * la * c.head_dim), y(x.size());
      check(mc_batch_read_kv(a, l, ra, wv, x.data()), "read_kv");
      check(mc_batch_read_kv(b, l, rb, wv, y.data()), "read_kv");
      if (x != y) return false;
    }
  return true;
}
static int filter_case(mc_model* m, const mc_model_config& c) {
  const int R = 4, K = 4, K1 = K + 1, ctx = 256, V = c.vocab;
  mc_spec_config spec{1, K, 3, 8, 1, 0, 0};
  auto make = [&]() {
    mc_batch* b = nullptr;
    check(mc_batch_create(m, R, ctx, K, &spec, &b), "batch_create");
    for (int r = 0; r < R; ++r) {
      auto p = case9_prompt(r, V);
      mc_sampling sp = case9_sampling(r);
      int32_t first = 0, fin = 0;
      check(mc_batch_insert(b, r, p.data(), (int32_t)p.size(), 40, &sp, &first, &fin), "insert");
    }
    case9_steps(b, R, K1, 2);
    return b;
  };
  mc_batch* ref = make();
  const std::vector<std::vector<int32_t>> plans{{2, 0, 1}, {1, 3, 3, 0}, {}};
  std::vector<mc_batch*> fb;
  for (const auto& keep : plans) {
    mc_batch* b = make();
    check(mc_batch_filter(b, keep.data(), (int32_t)keep.size()), "filter");
    for (size_t i = 0; i < keep.size(); ++i)
      if (!case9_same_kv(b, (int)i, ref, keep[i], c)) { printf("filter: row %zu K/V differs\n", i); ++g_bad; }
    for (int i = (int)keep.size(); i < R; ++i) {
      int32_t len = -1;
      check(mc_batch_kv_len(b, i, &len), "kv_len");
      if (len != 0) { printf("filter: dropped row %d keeps %d positions\n", i, len); ++g_bad; }
    }
    fb.push_back(b);
  }
  // extract row 3 of the reference batch into a one-row batch, admitted from its history
  mc_batch* one = nullptr;
  check(mc_batch_create(m, 1, ctx, K, &spec, &one), "batch_create");
  check(mc_batch_extract_kv(ref, 3, one, 0), "extract_kv");
  if (!case9_same_kv(one, 0, ref, 3, c)) { printf("extract: K/V differs\n"); ++g_bad; }
  int32_t hl = 0;
  check(mc_batch_history(ref, 3, nullptr, 0, &hl), "history");
  std::vector<int32_t> hist((size_t)hl);
  check(mc_batch_history(ref, 3, hist.data(), hl, &hl), "history");
  mc_sampling sp3 = case9_sampling(3);
  check(mc_batch_insert_prefilled(one, 0, hist.data(), hl, 40, &sp3), "insert_prefilled");
  const auto want = case9_steps(ref, R, K1, 3);
  for (size_t p = 0; p < plans.size(); ++p) {
    const auto got = case9_steps(fb[p], R, K1, 3);
    for (int i = 0; i < R; ++i) {
      const bool kept = i < (int)plans[p].size();
      const auto& w = kept ? want[(size_t)plans[p][(size_t)i]] : std::vector<int32_t>{};
      printf("plan %zu row %d (%s): %zu tokens%s\n", p, i, kept ? "kept" : "empty", got[(size_t)i].size(),
             got[(size_t)i] == w ? "" : "  DIFFERS");
      if (got[(size_t)i] != w) ++g_bad;
    }
    mc_batch_destroy(fb[p]);
  }
  const auto got1 = case9_steps(one, 1, K1, 3);
  printf("extracted row: %zu tokens (%zu in the batch)%s\n", got1[0].size(), want[3].size(),
         got1[0] == want[3] ? "" : "  DIFFERS");
  if (got1[0] != want[3] || want[3].empty()) ++g_bad;
  // errors: a row out of range, a capacity too small
  const int32_t bad[1] = {R};
  if (mc_batch_filter(ref, bad, 1) != MC_E_INVALID) { printf("filter accepted row %d\n", R); ++g_bad; }
  mc_batch* tiny = nullptr;
  check(mc_batch_create(m, 1, 64, K, &spec, &tiny), "batch_create");
  if (mc_batch_extract_kv(ref, 3, tiny, 0) != MC_E_CAPACITY) { printf("extract ignored capacity\n"); ++g_bad; }
  mc_batch_destroy(tiny);
  mc_batch_destroy(one);
  mc_batch_destroy(ref);
  printf("out-of-range buffer accesses: loads %lld stores %lld\n", emu::oob_loads, emu::oob_stores);
  if (emu::oob_loads || emu::oob_stores) ++g_bad;
  printf("%s\n", g_bad ? "FAIL" : "OK");
  return g_bad ? 1 : 0;
}

// case 10: prefix blocks: a row's K/V exported in the reference's block layout equals
// mc_batch_read_kv; the blocks imported into another batch's row read back the same, and
// mc_batch_insert_cached admits the row on top of them (the resumed prefill then has other
// M than the full one, so the tokens after it are not compared here)
static int prefix_case(mc_model* m, const mc_model_config& c) {
  // capacities that are not multiples of 64 (the cache's position stride rounds them up)
  const int K = 4, K1 = K + 1, V = c.vocab, B = 64, N = 150;
  const int nkv = c.n_kv_heads, d = c.head_dim, L = c.n_layers;
  mc_spec_config spec{1, K, 3, 8, 1, 0, 0};
  std::vector<int32_t> p((size_t)N);
  for (int i = 0; i < N; ++i) p[(size_t)i] = i >= 120 ? p[(size_t)i - 90] : (i * 29 + 7) % V;
  mc_batch *a = nullptr, *b = nullptr;
  check(mc_batch_create(m, 2, 250, K, &spec, &a), "batch_create");
  check(mc_batch_create(m, 2, 190, K, &spec, &b), "batch_create");
  mc_sampling sp{};
  sp.reject_token = -1;
  int32_t first_a = 0, first_b = 0, fin = 0;
  check(mc_batch_insert(a, 0, p.data(), N, 30, &sp, &first_a, &fin), "insert");
  check(mc_batch_insert(b, 0, p.data(), 40, 30, &sp, &first_b, &fin), "insert");
  std::vector<std::vector<uint16_t>> full((size_t)2 * L);
  for (int l = 0; l < L; ++l)
    for (int wv = 0; wv < 2; ++wv) {
      full[(size_t)2 * l + wv].resize((size_t)nkv * N * d);
      check(mc_batch_read_kv(a, l, 0, wv, full[(size_t)2 * l + wv].data()), "read_kv");
    }
  const int ranges[3][2] = {{0, B}, {B, B}, {5, 37}};
  for (const auto& rg : ranges) {
    const int t0 = rg[0], n = rg[1];
    std::vector<uint16_t> k((size_t)L * nkv * n * d), v(k.size());
    check(mc_batch_export_kv_block(a, 0, t0, n, k.data(), v.data()), "export_kv_block");
    size_t diff = 0;
    for (int l = 0; l < L; ++l)
      for (int h = 0; h < nkv; ++h)
        for (int t = 0; t < n; ++t)
          for (int e = 0; e < d; ++e) {
            const size_t o = (((size_t)l * nkv + h) * n + t) * d + e, f = ((size_t)h * N + t0 + t) * d + e;
            diff += k[o] != full[(size_t)2 * l][f];
            diff += v[o] != full[(size_t)2 * l + 1][f];
          }
    printf("export [%d, %d): %zu elements differ\n", t0, t0 + n, diff);
    if (diff) ++g_bad;
    if (t0 % B == 0) check(mc_batch_import_kv_block(b, 1, t0, n, k.data(), v.data()), "import_kv_block");
  }
  int32_t len = 0;
  check(mc_batch_kv_len(b, 1, &len), "kv_len");
  size_t diff = 0;
  for (int l = 0; l < L; ++l)
    for (int wv = 0; wv < 2; ++wv) {
      std::vector<uint16_t> x((size_t)nkv * len * d);
      check(mc_batch_read_kv(b, l, 1, wv, x.data()), "read_kv");
      for (int h = 0; h < nkv; ++h)
        for (int t = 0; t < len; ++t)
          for (int e = 0; e < d; ++e)
            diff += x[((size_t)h * len + t) * d + e] != full[(size_t)2 * l + wv][((size_t)h * N + t) * d + e];
    }
  printf("imported row: %d positions, %zu elements differ\n", len, diff);
  if (len != 2 * B || diff) ++g_bad;
  if (mc_batch_insert_cached(b, 1, p.data(), N, 2 * B + 1, 30, &sp, &first_b, &fin) != MC_E_STATE) {
    printf("insert_cached accepted a wrong n_cached\n");
    ++g_bad;
  }
  check(mc_batch_insert_cached(b, 1, p.data(), N, 2 * B, 30, &sp, &first_b, &fin), "insert_cached");
  check(mc_batch_kv_len(b, 1, &len), "kv_len");
  printf("insert_cached: first token %d (full prefill %d), K/V length %d\n", first_b, first_a, len);
  if (len != N) ++g_bad;
  std::vector<int32_t> ot((size_t)2 * K1), cnt(2), f(2);
  for (int st = 0; st < 2; ++st) check(mc_step(b, nullptr, nullptr, ot.data(), cnt.data(), f.data()), "step");
  // extract and filter between these strides: the K/V must read back the same
  mc_batch* e = nullptr;
  check(mc_batch_create(m, 1, 170, K, &spec, &e), "batch_create");
  check(mc_batch_extract_kv(a, 0, e, 0), "extract_kv");
  if (!case9_same_kv(e, 0, a, 0, c)) { printf("extract across strides: K/V differs\n"); ++g_bad; }
  const int32_t keep[2] = {1, 0};
  check(mc_batch_filter(b, keep, 2), "filter");
  mc_batch* a2 = nullptr;
  check(mc_batch_create(m, 2, 250, K, &spec, &a2), "batch_create");
  check(mc_batch_extract_kv(a, 0, a2, 1), "extract_kv");
  check(mc_batch_filter(a2, keep, 2), "filter");
  if (!case9_same_kv(a2, 0, a, 0, c)) { printf("filter: K/V differs\n"); ++g_bad; }
  mc_batch_destroy(a2);
  mc_batch_destroy(e);
  mc_batch_destroy(a);
  mc_batch_destroy(b);
  printf("out-of-range buffer accesses: loads %lld stores %lld\n", emu::oob_loads, emu::oob_stores);
  if (emu::oob_loads || emu::oob_stores) ++g_bad;
  printf("%s\n", g_bad ? "FAIL" : "OK");
  return g_bad ? 1 : 0;
}

int main(int argc, char** argv) {
  const int cs = argc > 1 ? atoi(argv[1]) : 0;
  emu::install_fault_handler();
  check(mc_set_device(0), "set_device");
  if (cs == 7) return accept_case(argc > 2 ? atoi(argv[2]) : 0);
  if (cs == 8) return noalloc_case();
  mc_model_config c{};
  c.arch = 0; c.n_layers = 2; c.hidden = 256; c.n_q_heads = 4; c.n_kv_heads = 2; c.head_dim = 128;
  c.intermediate = 512; c.vocab = 4096; c.tied_embeddings = 1; c.rms_eps = 1e-6f; c.rope_theta = 1e6f;
  if (cs == 2) {
    c.hidden = 2560; c.n_q_heads = 32; c.n_kv_heads = 8; c.intermediate = 9728; c.vocab = 151936;
  }
  if (cs == 3) {  // 8 kv heads, GQA group 4
    c.hidden = 512; c.n_q_heads = 32; c.n_kv_heads = 8; c.intermediate = 1024; c.vocab = 4096;
  }
  if (cs == 4 || cs == 9 || cs == 10) {  // speculative steps: padding slots
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
  if (cs == 9) return filter_case(m, c);
  if (cs == 10) return prefix_case(m, c);
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
        check(mc_step(bb, nullptr, nullptr, ot, cnt, f), "step");
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
  const std::vector<int> widths = cs == 2 ? std::vector<int>{6} : cs == 3 ? std::vector<int>{6, 1, 8, 12, 16} : std::vector<int>{6, 1, 8};
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
