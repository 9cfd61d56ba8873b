// C++ tests of the host interface (yasakani-for-mac_amd/host/yskn_sampler.hpp),
// written like the reference's own Rust unit tests
// (crates/yskn-ref/src/output_head_sampler.rs:252-310) so that the two read
// side by side. Every sampling test runs on the GPU through the C ABI.
//
//   test_sampler [--cpu]   --cpu: only the tests that need no device
#include <cmath>
#include <cstdio>
#include <cstring>
#include <limits>
#include <string>
#include <vector>

#include "../../yasakani-for-mac_amd/host/yskn_sampler.hpp"

using namespace yskn;

static int g_failures = 0;
#define CHECK(cond)                                                              \
  do {                                                                           \
    if (!(cond)) {                                                               \
      std::printf("  FAILED %s:%d: %s\n", __FILE__, __LINE__, #cond);            \
      ++g_failures;                                                              \
    }                                                                            \
  } while (0)

template <class T>
static T unwrap(const Result<T>& r) {
  if (r.is_err()) {
    std::printf("  FAILED unwrap: %s\n", r.error().message.c_str());
    ++g_failures;
    return T{};
  }
  return r.value();
}

static uint64_t bits(double x) {
  uint64_t b;
  std::memcpy(&b, &x, 8);
  return b;
}

// ---- output_head_sampler.rs:256-262 -----------------------------------------
static void raw_order_ties_are_broken_by_token_id() {
  CHECK(unwrap(greedy({-0.0f, 0.0f})) == 0u);
  CHECK((unwrap(top_tokens({2.0f, 3.0f, 3.0f, -1.0f}, 3)) == std::vector<uint32_t>{1, 2, 0}));
  const Result<uint32_t> nan = greedy({std::numeric_limits<float>::quiet_NaN()});
  CHECK(nan.is_err() && nan.error().kind == Error::Kind::NonFinite);
  CHECK(greedy({-std::numeric_limits<float>::infinity()}).is_err());
}

// ---- output_head_sampler.rs:264-284 -----------------------------------------
static void seed_and_absolute_position_are_the_only_sampling_state() {
  std::vector<float> logits;
  for (int index = 0; index < 32; ++index) logits.push_back((float)(index % 7) / 8.0f);
  for (SamplingVersion version : {SamplingVersion::Gumbel, SamplingVersion::InverseCumulative}) {
    SamplingParameters p;
    p.seed = 0x112345678ull;
    p.version = version;
    const Sampler sampler = Sampler::sampled(p);
    std::vector<uint32_t> expected, actual(20);
    for (uint64_t position = 100; position < 120; ++position) expected.push_back(unwrap(sampler.sample(logits, position)));
    for (uint64_t position = 119; position + 1 > 100; --position)
      actual[position - 100] = unwrap(sampler.sample(logits, position));
    CHECK(actual == expected);
    bool varies = false;
    for (size_t i = 1; i < expected.size(); ++i) varies = varies || expected[i] != expected[i - 1];
    CHECK(varies);
  }
}

// ---- output_head_sampler.rs:286-299 -----------------------------------------
static void truncation_retains_at_least_the_top_candidate() {
  for (SamplingVersion version : {SamplingVersion::Gumbel, SamplingVersion::InverseCumulative}) {
    SamplingParameters p;
    p.top_k = 3;
    p.min_p = 1.0;
    p.version = version;
    const Sampler sampler = Sampler::sampled(p);
    for (uint64_t position = 0; position < 16; ++position) CHECK(unwrap(sampler.sample({1.0f, 3.0f, 2.0f}, position)) == 1u);
  }
}

// ---- output_head_sampler.rs:301-310 -----------------------------------------
static void loss_is_invariant_to_an_exact_constant_logit_shift() {
  const double first = unwrap(negative_log_likelihood({1.0f, 2.0f, -1.0f}, 1));
  const double shifted = unwrap(negative_log_likelihood({17.0f, 18.0f, 15.0f}, 1));
  CHECK(bits(first) == bits(shifted));
  CHECK(bits(unwrap(negative_log_likelihood({4.0f}, 0))) == bits(0.0));
}

// ---- parameters (output_head_sampler.rs:30-75), no device needed ------------
static void parameters_follow_the_reference_rules() {
  const SamplingParameters d;
  CHECK(d.temperature == 1.0 && d.top_p == 0.95 && d.top_k == 20 && d.min_p == 0.0 && d.seed == 0);
  CHECK(d.version == SamplingVersion::Gumbel);
  const SamplingParameters p = unwrap(SamplingParameters::from_thousandths(700, 900, 50));
  CHECK(p.temperature == 700 / 1000.0 && p.top_p == 900 / 1000.0 && p.min_p == 50 / 1000.0);
  CHECK(SamplingParameters::from_thousandths(0, 900, 0).is_err());     // temperature must be positive
  CHECK(SamplingParameters::from_thousandths(700, 0, 0).is_err());     // top_p in (0, 1]
  CHECK(SamplingParameters::from_thousandths(700, 1001, 0).is_err());
  CHECK(SamplingParameters::from_thousandths(700, 900, 1001).is_err());  // min_p in [0, 1]
  SamplingParameters q;
  q.top_k = 21;
  CHECK(q.validate(248320).is_err());
  q.top_k = 20;
  CHECK(q.validate(19).is_err());  // top_k <= vocabulary size
  CHECK(q.validate(20).is_ok());
  q.temperature = std::numeric_limits<double>::quiet_NaN();
  const Result<Unit> e = q.validate(20);
  CHECK(e.is_err() && e.error().kind == Error::Kind::InvalidInput);
  CHECK(e.error().message.find("temperature") != std::string::npos);
}

// ---- Selector (speculation.rs:123-139) ------------------------------------------
static void samplers_are_selectors() {
  std::vector<float> logits(1000);
  for (size_t i = 0; i < logits.size(); ++i) logits[i] = std::sin(0.37f * (float)i) * 4.0f;
  Sampler g = Sampler::greedy();
  Selector& sel = g;
  CHECK(unwrap(sel.select(logits, 5)) == unwrap(greedy(logits)));
  SamplingParameters p;
  p.seed = 42;
  Sampler s = Sampler::sampled(p);
  Selector& sel2 = s;
  const uint32_t a = unwrap(sel2.select(logits, 7));
  CHECK(a == unwrap(s.sample(logits, 7)));
  const std::vector<uint32_t> top = unwrap(top_tokens(logits, 20));
  bool in_top = false;
  for (uint32_t t : top) in_top = in_top || t == a;
  CHECK(in_top);  // top_k = 20 by default
  CHECK(s.sample({}, 1).is_err());
}

// ---- accept loop (speculation.rs:483-523) ----------------------------------------
static void verify_block_equals_token_at_a_time_selection() {
  const size_t V = 3000, M = 8;
  std::vector<float> logits(M * V);
  uint64_t z = 0x1234;
  for (float& x : logits) {
    z = z * 6364136223846793005ull + 1442695040888963407ull;
    x = (float)((double)(z >> 11) * (1.0 / 9007199254740992.0) * 12.0 - 6.0);
  }
  SamplingParameters p;
  p.seed = 99;
  const Sampler sampler = Sampler::sampled(p);
  const uint64_t base = 1000;
  std::vector<uint32_t> sel(M);
  for (size_t j = 0; j < M; ++j)
    sel[j] = unwrap(sampler.sample(std::vector<float>(logits.begin() + j * V, logits.begin() + (j + 1) * V), base + j + 1));
  for (size_t agree = 0; agree < M; ++agree) {
    // drafts that match the first `agree` selections, then differ
    std::vector<uint32_t> drafts(M - 1);
    for (size_t j = 0; j + 1 < M; ++j) drafts[j] = j < agree ? sel[j] : (sel[j] + 1) % (uint32_t)V;
    const VerifyResult r = unwrap(verify_block(p, false, logits, M, drafts, base, {}));
    const size_t expect_acc = agree < M - 1 ? agree : M - 1;
    CHECK(r.accepted == expect_acc);
    CHECK(r.emitted == expect_acc + 1);
    CHECK(r.token == sel[expect_acc]);
    CHECK(!r.stop_eos);
    for (size_t j = 0; j < M; ++j) CHECK(r.selected[j] == sel[j]);
  }
  // an EOS id among the emitted tokens ends the block
  std::vector<uint32_t> drafts(sel.begin(), sel.end() - 1);
  const VerifyResult r = unwrap(verify_block(p, false, logits, M, drafts, base, {sel[2]}));
  size_t first = 0;
  while (sel[first] != sel[2]) ++first;  // an earlier row may select the same id
  CHECK(r.stop_eos && r.emitted == first + 1 && r.token == sel[2]);
}

int main(int argc, char** argv) {
  const bool cpu_only = argc > 1 && std::strcmp(argv[1], "--cpu") == 0;
  struct Test {
    const char* name;
    void (*fn)();
    bool device;
  } tests[] = {
      {"parameters_follow_the_reference_rules", parameters_follow_the_reference_rules, false},
      {"raw_order_ties_are_broken_by_token_id", raw_order_ties_are_broken_by_token_id, true},
      {"seed_and_absolute_position_are_the_only_sampling_state", seed_and_absolute_position_are_the_only_sampling_state, true},
      {"truncation_retains_at_least_the_top_candidate", truncation_retains_at_least_the_top_candidate, true},
      {"loss_is_invariant_to_an_exact_constant_logit_shift", loss_is_invariant_to_an_exact_constant_logit_shift, true},
      {"samplers_are_selectors", samplers_are_selectors, true},
      {"verify_block_equals_token_at_a_time_selection", verify_block_equals_token_at_a_time_selection, true},
  };
  for (const Test& t : tests) {
    if (cpu_only && t.device) continue;
    const int before = g_failures;
    std::printf("%s\n", t.name);
    std::fflush(stdout);
    t.fn();
    std::printf("  %s\n", g_failures == before ? "ok" : "FAILED");
    std::fflush(stdout);
  }
  std::printf(g_failures == 0 ? "ALL PASSED\n" : "%d FAILURES\n", g_failures);
  return g_failures == 0 ? 0 : 1;
}
