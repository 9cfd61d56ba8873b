// smp_api.hip -- host side of the C ABI declared in include/yskn_smp.h.
//
// Validation mirrors the reference: SamplingParameters::validate
// (crates/yskn-ref/src/output_head_sampler.rs:56-75), validate_logits
// (:94-101), and the C ABI's 0 / negative status with a thread-local last
// error (src/c_api.cpp:11-14). The handle owns only scratch memory,
// allocated once at create (the engine's pattern, src/engine35.cpp:336-347).
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

#include "../../include/yskn_smp.h"
#include "smp_internal.hpp"

using namespace yskn;

namespace {

thread_local std::string g_error;

int fail(int code, const std::string& msg) {
  g_error = msg;
  return code;
}

int hip_fail(hipError_t e, const char* what) {
  g_error = std::string(what) + ": " + hipGetErrorString(e);
  return YSKN_SMP_EDEVICE;
}

}  // namespace

struct yskn_smp {
  int32_t max_rows = 0;
  int32_t max_vocab = 0;
  uint32_t flags = 0;
  int device = 0;
  std::vector<DevParams> params;  // host copy of the device parameters, 1 or max_rows entries
  bool params_shared = true;
  DevParams* d_params = nullptr;
  int32_t* d_status = nullptr;
  uint32_t* d_vcount = nullptr;
  uint32_t* d_vresult = nullptr;
  uint64_t* d_dense_a = nullptr;
  uint64_t* d_dense_b = nullptr;
  double* d_dense_w = nullptr;
  int64_t dense_ld = 0;
  uint2* d_pen_words = nullptr;
  int64_t pw_ld = 0;
  uint32_t* d_pen_cnt = nullptr;
  int32_t* d_pen_len = nullptr;
  unsigned long long* d_stats = nullptr;
  uint64_t* d_exp_cand = nullptr;  // [max_rows][SEG_MAX][EXP_CAP]
  SegMeta* d_exp_meta = nullptr;   // [max_rows][SEG_MAX]
  uint32_t* d_segcnt = nullptr;    // [max_rows]
  // host-slice convenience buffers
  float* d_host_logits = nullptr;
  uint64_t* d_host_pos = nullptr;
  uint32_t* d_host_out = nullptr;
  int32_t last_rows = 0;
  // the last call was a verify: its pass status is in the caller's result
  const yskn_smp_verify_result* last_verify = nullptr;
  int last_kind = 0;  // KIND_*: which call's messages yskn_smp_sync reports
};

namespace {

yskn_smp_params default_params() {
  yskn_smp_params p;
  std::memset(&p, 0, sizeof p);
  p.temperature_milli = 1000;
  p.top_p_milli = 950;
  p.top_k = 20;
  p.min_p_milli = 0;
  p.seed = 0;
  p.version = YSKN_SMP_VERSION_GUMBEL;
  p.repetition_penalty = 1.0f;
  p.presence_penalty = 0.0f;
  p.frequency_penalty = 0.0f;
  return p;
}

bool finite_f(float x) {
  uint32_t b;
  std::memcpy(&b, &x, 4);
  return (b & 0x7f800000u) != 0x7f800000u;
}

// |l - M| <= 2 * FLT_MAX for finite binary32 logits, so (l - M) / T cannot
// overflow binary64 unless T < 2 * FLT_MAX / DBL_MAX ~ 3.8e-270.
bool needs_zcheck(const DevParams& d) { return !d.greedy && d.temperature < 1e-260; }

DevParams to_device(const yskn_smp_params& p) {
  DevParams d;
  std::memset(&d, 0, sizeof d);
  // binary64 division by 1000.0, not multiplication by 0.001
  d.temperature = (double)p.temperature_milli / 1000.0;
  d.top_p = (double)p.top_p_milli / 1000.0;
  d.min_p = (double)p.min_p_milli / 1000.0;
  d.seed = p.seed;
  d.top_k = p.top_k;
  d.version = p.version;
  d.greedy = p.temperature_milli == 0 ? 1 : 0;
  d.rep = p.repetition_penalty;
  d.pres = p.presence_penalty;
  d.freq = p.frequency_penalty;
  d.penalize = (p.repetition_penalty != 1.0f || p.presence_penalty != 0.0f ||
                p.frequency_penalty != 0.0f)
                   ? 1
                   : 0;
  d.zcheck = needs_zcheck(d) ? 1 : 0;
  return d;
}

DevParams to_device(const yskn_smp_params_f64& p) {
  DevParams d;
  std::memset(&d, 0, sizeof d);
  d.temperature = p.temperature;
  d.top_p = p.top_p;
  d.min_p = p.min_p;
  d.seed = p.seed;
  d.top_k = p.top_k;
  d.version = p.version;
  d.greedy = p.greedy ? 1 : 0;
  d.rep = p.repetition_penalty;
  d.pres = p.presence_penalty;
  d.freq = p.frequency_penalty;
  d.penalize = (p.repetition_penalty != 1.0f || p.presence_penalty != 0.0f ||
                p.frequency_penalty != 0.0f)
                   ? 1
                   : 0;
  d.zcheck = needs_zcheck(d) ? 1 : 0;
  return d;
}

bool finite_d(double x) { return x - x == 0.0; }

// SamplingParameters::validate (output_head_sampler.rs:56-75), same order and
// messages; greedy rows are not validated (Sampler::Greedy has no parameters),
// penalties are the extension's.
int validate(const DevParams& p, int64_t vocab, uint32_t flags) {
  if (!p.greedy) {
    if (!finite_d(p.temperature) || !(p.temperature > 0.0))
      return fail(YSKN_SMP_EINVAL, "invalid input: temperature must be finite and positive");
    if (!finite_d(p.top_p) || !(p.top_p > 0.0) || p.top_p > 1.0)
      return fail(YSKN_SMP_EINVAL, "invalid input: top_p must be in (0, 1]");
    if (!finite_d(p.min_p) || !(p.min_p >= 0.0 && p.min_p <= 1.0))
      return fail(YSKN_SMP_EINVAL, "invalid input: min_p must be in [0, 1]");
    if (flags & YSKN_SMP_FLAG_EXTENDED_TOP_K) {
      if ((int64_t)p.top_k > vocab)
        return fail(YSKN_SMP_EINVAL, "invalid input: top_k must be in 0..=vocabulary size");
    } else if (p.top_k == 0 || p.top_k > 20 || (int64_t)p.top_k > vocab) {
      return fail(YSKN_SMP_EINVAL, "invalid input: top_k must be in 1..=min(20, vocabulary size)");
    }
    if (p.version != YSKN_SMP_VERSION_GUMBEL && p.version != YSKN_SMP_VERSION_INVERSE_CDF)
      return fail(YSKN_SMP_EINVAL, "invalid input: version must be 2 or 3");
  }
  if (!finite_f(p.rep) || !(p.rep > 0.0f) || !finite_f(p.pres) || !finite_f(p.freq))
    return fail(YSKN_SMP_EINVAL, "invalid input: penalties must be finite, repetition > 0");
  return YSKN_SMP_OK;
}

int validate(const yskn_smp_params& p, int64_t vocab, uint32_t flags) {
  if (p.temperature_milli != 0) {
    // thousandths are range-checked before the division
    if (p.top_p_milli < 1 || p.top_p_milli > 1000)
      return fail(YSKN_SMP_EINVAL, "invalid input: top_p must be in (0, 1]");
    if (p.min_p_milli > 1000) return fail(YSKN_SMP_EINVAL, "invalid input: min_p must be in [0, 1]");
  }
  return validate(to_device(p), vocab, flags);
}

int validate(const yskn_smp_params_f64& p, int64_t vocab, uint32_t flags) {
  return validate(to_device(p), vocab, flags);
}

template <typename T>
hipError_t alloc(T** p, size_t n) {
  return hipMalloc((void**)p, n * sizeof(T) + 256);
}

int check_common(yskn_smp_handle h, const void* logits, int32_t dtype, int32_t rows,
                 int32_t vocab, int64_t ld) {
  if (!h) return fail(YSKN_SMP_EINVAL, "invalid input: null handle");
  if (!logits) return fail(YSKN_SMP_EINVAL, "invalid input: null logits");
  if (dtype != YSKN_SMP_F32 && dtype != YSKN_SMP_BF16)
    return fail(YSKN_SMP_EINVAL, "invalid input: dtype must be YSKN_SMP_F32 or YSKN_SMP_BF16");
  if (vocab <= 0)
    return fail(YSKN_SMP_EINVAL, "invalid input: logits must contain a nonempty u32-indexed vocabulary");
  if (vocab > h->max_vocab)
    return fail(YSKN_SMP_ERANGE, "vocabulary larger than the handle's max_vocab");
  if (rows <= 0 || rows > h->max_rows) return fail(YSKN_SMP_ERANGE, "rows outside 1..=max_rows");
  if (ld < vocab) return fail(YSKN_SMP_EINVAL, "invalid input: ld < vocab");
  return YSKN_SMP_OK;
}

int check_params_for(yskn_smp_handle h, int32_t rows, int32_t vocab) {
  const int n = h->params_shared ? 1 : rows;
  for (int r = 0; r < n; ++r) {
    const int st = validate(h->params[r], vocab, h->flags);
    if (st) return st;
  }
  return YSKN_SMP_OK;
}

bool any_penalty(yskn_smp_handle h, int32_t rows) {
  const int n = h->params_shared ? 1 : rows;
  for (int r = 0; r < n; ++r) {
    if (h->params[r].penalize) return true;
  }
  return false;
}

// Segments per row. A block streams one segment; small batches split rows so
// that the call spreads over the CUs: about one 2,048-logit chunk per wave,
// and at most 256 blocks in all, one per CU (a block's LDS fills a CU), so
// that every block is resident from the start: a block queued behind a CU
// held by a long finish (the dense path) would hold back its row. From 192
// rows on, each row is one block.
// YSKN_SMP_SEGMENTS=n (1..32) fixes the count for measurements.
int segments_for(int32_t rows, int32_t vocab) {
  static const int forced = [] {
    const char* e = std::getenv("YSKN_SMP_SEGMENTS");
    return e ? std::atoi(e) : 0;
  }();
  const int nch = (vocab + WSEG - 1) / WSEG;
  int s;
  if (forced > 0) {
    s = forced;
  } else if (rows >= 192) {
    s = 1;
  } else {
    const int by_chunks = (nch + NW - 1) / NW;
    const int by_blocks = 256 / rows > 1 ? 256 / rows : 1;
    s = by_chunks < by_blocks ? by_chunks : by_blocks;
  }
  if (s > SEG_MAX) s = SEG_MAX;
  if (s > nch) s = nch;
  return s < 1 ? 1 : s;
}

SmpArgs base_args(yskn_smp_handle h, const void* logits, int32_t rows, int32_t vocab,
                  int64_t ld) {
  SmpArgs a;
  std::memset(&a, 0, sizeof a);
  a.logits = logits;
  a.ld = ld;
  a.V = vocab;
  a.rows = rows;
  a.mode = MODE_SAMPLE;
  a.pos_mode = POS_ARRAY;
  a.prm = h->d_params;
  a.prm_shared = h->params_shared ? 1 : 0;
  a.n_draws = 1;
  a.status = h->d_status;
  a.pen_words = h->d_pen_words;
  a.pw_ld = h->pw_ld;
  a.pen_cnt = h->d_pen_cnt;
  a.pen_len = h->d_pen_len;
  a.dense_a = h->d_dense_a;
  a.dense_b = h->d_dense_b;
  a.dense_w = h->d_dense_w;
  a.dense_ld = h->dense_ld;
  a.force_dense = (h->flags & YSKN_SMP_FLAG_FORCE_DENSE) ? 1 : 0;
  a.stats = h->d_stats;
  a.nseg = segments_for(rows, vocab);
  a.exp_cand = h->d_exp_cand;
  a.exp_meta = h->d_exp_meta;
  a.segcnt = h->d_segcnt;
  return a;
}

bool vector_ok(const void* logits, int32_t dtype, int64_t ld) {
  const size_t es = dtype == YSKN_SMP_F32 ? 4 : 2;
  return ((uintptr_t)logits % 16 == 0) && ((ld * (int64_t)es) % 16 == 0);
}

enum { KIND_SAMPLE = 0, KIND_SHORTLIST = 1, KIND_TOP16 = 2, KIND_CHOOSE = 3 };

int launch(yskn_smp_handle h, SmpArgs& a, int32_t dtype, bool pen, const yskn_smp_aux* aux,
           hipStream_t st) {
  if (pen) {
    PenArgs p;
    std::memset(&p, 0, sizeof p);
    p.history = aux ? aux->history : nullptr;
    p.history_len = aux ? aux->history_len : nullptr;
    p.history_ld = aux ? aux->history_ld : 0;
    p.V = a.V;
    p.rows = a.rows;
    p.words = h->d_pen_words;
    p.pw_ld = h->pw_ld;
    p.cnt = h->d_pen_cnt;
    p.len = h->d_pen_len;
    p.prm = h->d_params;
    p.prm_shared = a.prm_shared;
    hipError_t e = launch_penalty_prep(p, st);
    if (e != hipSuccess) return hip_fail(e, "penalty preparation launch");
  }
  a.vec = dtype != 2 && vector_ok(a.logits, dtype, a.ld) ? 1 : 0;
  hipError_t e = launch_sample(a, dtype == 2 ? 2 : (dtype == YSKN_SMP_F32 ? 0 : 1), a.vec != 0, pen, st);
  if (e != hipSuccess) return hip_fail(e, "sampler launch");
  h->last_rows = a.rows;
  h->last_verify = a.mode == MODE_VERIFY ? (const yskn_smp_verify_result*)a.vresult : nullptr;
  h->last_kind = KIND_SAMPLE;
  return YSKN_SMP_OK;
}

int draft_rows(yskn_smp_handle h, int32_t rows) {
  if (!h) return fail(YSKN_SMP_EINVAL, "invalid input: null handle");
  if (rows <= 0 || rows > h->max_rows) return fail(YSKN_SMP_ERANGE, "rows outside 1..=max_rows");
  return YSKN_SMP_OK;
}

int draft_launched(yskn_smp_handle h, hipError_t e, int32_t rows, int kind) {
  if (e != hipSuccess) return hip_fail(e, "draft selection launch");
  h->last_rows = rows;
  h->last_verify = nullptr;
  h->last_kind = kind;
  return YSKN_SMP_OK;
}

// The optional outputs and the penalty history of yskn_smp_aux into the
// launch arguments; *pen tells whether the penalty kernel must run.
int apply_aux(yskn_smp_handle h, SmpArgs& a, const yskn_smp_aux* aux, int32_t rows, bool* pen) {
  *pen = false;
  if (!aux) {
    if (any_penalty(h, rows)) return fail(YSKN_SMP_EINVAL, "invalid input: penalties need a history");
    return YSKN_SMP_OK;
  }
  if (aux->n_logprobs < 0 || aux->n_logprobs > a.V)
    return fail(YSKN_SMP_EINVAL, "invalid input: n_logprobs must be in 0..=vocab");
  if (aux->n_logprobs > 0 && (!aux->logprob_ids || !aux->logprobs))
    return fail(YSKN_SMP_EINVAL, "invalid input: n_logprobs > 0 needs both output arrays");
  if ((aux->top8_ids == nullptr) != (aux->top8_vals == nullptr) ||
      (aux->top20_ids == nullptr) != (aux->top20_vals == nullptr))
    return fail(YSKN_SMP_EINVAL, "invalid input: top lists need both ids and values");
  a.argmax = aux->argmax;
  a.top8_ids = aux->top8_ids;
  a.top8_vals = aux->top8_vals;
  a.top20_ids = aux->top20_ids;
  a.top20_vals = aux->top20_vals;
  a.n_lp = aux->n_logprobs;
  a.lp_ids = aux->logprob_ids;
  a.lp_vals = aux->logprobs;
  a.row_status = aux->row_status;
  a.want_mass = a.n_lp > 0 ? 1 : 0;
  if (any_penalty(h, rows)) {
    if (!aux->history || !aux->history_len)
      return fail(YSKN_SMP_EINVAL, "invalid input: penalties need a history");
    if (aux->history_ld < 0) return fail(YSKN_SMP_EINVAL, "invalid input: history_ld must be >= 0");
    *pen = true;
  }
  return YSKN_SMP_OK;
}

}  // namespace

extern "C" {

const char* yskn_smp_last_error(void) { return g_error.c_str(); }

const char* yskn_smp_version(void) { return "yskn_smp 0.1 (gfx950)"; }

int yskn_smp_validate_params(const yskn_smp_params* params, int32_t vocab, uint32_t flags) {
  if (!params) return fail(YSKN_SMP_EINVAL, "invalid input: null params");
  return validate(*params, vocab, flags);
}

int yskn_smp_validate_params_f64(const yskn_smp_params_f64* params, int32_t vocab, uint32_t flags) {
  if (!params) return fail(YSKN_SMP_EINVAL, "invalid input: null params");
  return validate(*params, vocab, flags);
}

int yskn_smp_create(int32_t max_rows, int32_t max_vocab, uint32_t flags, yskn_smp_handle* out) {
  if (!out) return fail(YSKN_SMP_EINVAL, "invalid input: null output handle");
  *out = nullptr;
  if (max_rows <= 0) return fail(YSKN_SMP_EINVAL, "invalid input: max_rows must be positive");
  if (max_vocab <= 0)
    return fail(YSKN_SMP_EINVAL, "invalid input: logits must contain a nonempty u32-indexed vocabulary");
  if ((int64_t)max_vocab > VMAX)
    return fail(YSKN_SMP_ERANGE, "vocabulary larger than 4,194,304");
  yskn_smp* h = new yskn_smp();
  h->max_rows = max_rows;
  h->max_vocab = max_vocab;
  h->flags = flags;
  h->params.assign(1, to_device(default_params()));
  h->params_shared = true;
  if (hipGetDevice(&h->device) != hipSuccess) h->device = 0;
  const size_t R = (size_t)max_rows;
  h->dense_ld = ((int64_t)max_vocab + 63) / 64 * 64;
  h->pw_ld = ((int64_t)max_vocab + 31) / 32;
  hipError_t e = hipSuccess;
  auto step = [&](hipError_t r) {
    if (e == hipSuccess) e = r;
  };
  step(alloc(&h->d_params, R));
  step(alloc(&h->d_status, R));
  step(alloc(&h->d_vcount, 4));
  step(alloc(&h->d_vresult, 4));
  step(alloc(&h->d_dense_a, R * (size_t)h->dense_ld));
  step(alloc(&h->d_dense_b, R * (size_t)h->dense_ld));
  step(alloc(&h->d_dense_w, R * (size_t)h->dense_ld));
  step(alloc(&h->d_pen_words, R * (size_t)h->pw_ld));
  step(alloc(&h->d_pen_cnt, R * (size_t)HCAP));
  step(alloc(&h->d_pen_len, R));
  step(alloc(&h->d_stats, (size_t)STAT_COUNT));
  step(alloc(&h->d_exp_cand, R * SEG_MAX * EXP_CAP));
  step(alloc(&h->d_exp_meta, R * SEG_MAX));
  step(alloc(&h->d_segcnt, R));
  step(alloc(&h->d_host_logits, (size_t)max_vocab));
  step(alloc(&h->d_host_pos, 1));
  step(alloc(&h->d_host_out, 1));
  if (e == hipSuccess) step(hipMemset(h->d_status, 0, R * sizeof(int32_t)));
  if (e == hipSuccess) step(hipMemset(h->d_vcount, 0, 4 * sizeof(uint32_t)));
  if (e == hipSuccess) step(hipMemset(h->d_pen_len, 0, R * sizeof(int32_t)));
  if (e == hipSuccess) step(hipMemset(h->d_stats, 0, STAT_COUNT * sizeof(unsigned long long)));
  if (e == hipSuccess) step(hipMemset(h->d_segcnt, 0, R * sizeof(uint32_t)));
  if (e == hipSuccess) {
    step(hipMemcpy(h->d_params, h->params.data(), sizeof(DevParams), hipMemcpyHostToDevice));
  }
  if (e != hipSuccess) {
    yskn_smp_destroy(h);
    return hip_fail(e, "yskn_smp_create");
  }
  *out = h;
  return YSKN_SMP_OK;
}

void yskn_smp_destroy(yskn_smp_handle h) {
  if (!h) return;
  void* ptrs[] = {h->d_params,
                  h->d_status,     h->d_vcount,    h->d_vresult,     h->d_dense_a,
                  h->d_dense_b,    h->d_dense_w,   h->d_pen_words,
                  h->d_pen_cnt,    h->d_pen_len,   h->d_stats,       h->d_host_logits,
                  h->d_host_pos,   h->d_host_out,  h->d_exp_cand,    h->d_exp_meta,
                  h->d_segcnt};
  for (void* p : ptrs)
    if (p) (void)hipFree(p);
  delete h;
}

extern "C++" {
namespace {

// Validated device parameters -> handle (host copy + device copy).
template <typename P>
int set_params_impl(yskn_smp_handle h, const P* params, int32_t n, const char* what) {
  if (!h || !params) return fail(YSKN_SMP_EINVAL, "invalid input: null handle or params");
  if (n != 1 && (n < 1 || n > h->max_rows))
    return fail(YSKN_SMP_EINVAL, "invalid input: n must be 1 or 1..=max_rows");
  for (int i = 0; i < n; ++i) {
    const int st = validate(params[i], h->max_vocab, h->flags);
    if (st) return st;
  }
  std::vector<DevParams> d(n);
  for (int i = 0; i < n; ++i) d[i] = to_device(params[i]);
  // Like the reference setter: drain outstanding work, then copy.
  hipError_t e = hipDeviceSynchronize();
  if (e == hipSuccess) e = hipMemcpy(h->d_params, d.data(), n * sizeof(DevParams), hipMemcpyHostToDevice);
  if (e != hipSuccess) return hip_fail(e, what);
  h->params.assign(d.begin(), d.end());
  h->params_shared = n == 1;
  return YSKN_SMP_OK;
}

}  // namespace
}  // extern "C++"

int yskn_smp_set_params(yskn_smp_handle h, const yskn_smp_params* params, int32_t n) {
  return set_params_impl(h, params, n, "yskn_smp_set_params");
}

int yskn_smp_set_params_f64(yskn_smp_handle h, const yskn_smp_params_f64* params, int32_t n) {
  return set_params_impl(h, params, n, "yskn_smp_set_params_f64");
}

int yskn_smp_sample(yskn_smp_handle h, const void* logits, int32_t dtype, int32_t rows,
                    int32_t vocab, int64_t ld, const uint64_t* positions, int32_t n_draws,
                    uint32_t* out_ids, const yskn_smp_aux* aux, void* stream) {
  int st = check_common(h, logits, dtype, rows, vocab, ld);
  if (st) return st;
  if (!h->params_shared && rows > (int32_t)h->params.size())
    return fail(YSKN_SMP_EINVAL, "invalid input: fewer per-row parameter sets than rows");
  if (out_ids && (!positions || n_draws < 1))
    return fail(YSKN_SMP_EINVAL, "invalid input: out_ids needs positions and n_draws >= 1");
  st = check_params_for(h, rows, vocab);
  if (st) return st;
  SmpArgs a = base_args(h, logits, rows, vocab, ld);
  a.positions = positions;
  a.n_draws = n_draws < 1 ? 1 : n_draws;
  a.out_ids = out_ids;
  bool pen = false;
  st = apply_aux(h, a, aux, rows, &pen);
  if (st) return st;
  return launch(h, a, dtype, pen, aux, (hipStream_t)stream);
}

int yskn_smp_sample_at(yskn_smp_handle h, const void* logits, int32_t dtype, int32_t rows,
                       int32_t vocab, int64_t ld, const uint64_t* base_position,
                       const uint8_t* row_depth, int32_t row0, uint32_t* out_ids,
                       const yskn_smp_aux* aux, const yskn_smp_advance* advance, void* stream) {
  int st = check_common(h, logits, dtype, rows, vocab, ld);
  if (st) return st;
  if (!base_position || !out_ids)
    return fail(YSKN_SMP_EINVAL, "invalid input: null base_position or out_ids");
  if (row0 < 0) return fail(YSKN_SMP_EINVAL, "invalid input: row0 must be >= 0");
  if (advance && (!advance->position || !advance->token))
    return fail(YSKN_SMP_EINVAL, "invalid input: advance needs both a position and a token");
  if (advance && rows != 1)
    return fail(YSKN_SMP_EINVAL, "invalid input: advance is defined for one row");
  if (!h->params_shared && rows > (int32_t)h->params.size())
    return fail(YSKN_SMP_EINVAL, "invalid input: fewer per-row parameter sets than rows");
  st = check_params_for(h, rows, vocab);
  if (st) return st;
  SmpArgs a = base_args(h, logits, rows, vocab, ld);
  a.pos_mode = POS_BASE;
  a.base_position = base_position;
  a.row_depth = row_depth;
  a.row0 = row0;
  a.n_draws = 1;
  a.out_ids = out_ids;
  if (advance) {
    a.adv_pos = advance->position;
    a.adv_tok = advance->token;
  }
  bool pen = false;
  st = apply_aux(h, a, aux, rows, &pen);
  if (st) return st;
  return launch(h, a, dtype, pen, aux, (hipStream_t)stream);
}

int yskn_smp_sample_head(yskn_smp_handle h, const yskn_smp_head* head, int32_t rows, int32_t vocab,
                         const uint64_t* positions, int32_t n_draws, uint32_t* out_ids,
                         const yskn_smp_aux* aux, void* stream) {
  if (!head) return fail(YSKN_SMP_EINVAL, "invalid input: null head");
  int st = check_common(h, head->acc, YSKN_SMP_F32, rows, vocab, head->acc_ld);
  if (st) return st;
  if (!head->unit_scale || !head->block_sums || !head->tau)
    return fail(YSKN_SMP_EINVAL, "invalid input: head needs unit_scale, block_sums and tau");
  if (head->n_blocks < 1 || head->n_blocks > 64)
    return fail(YSKN_SMP_EINVAL, "invalid input: head n_blocks must be in 1..=64");
  if (!finite_f(head->width) || !(head->width > 0.0f))
    return fail(YSKN_SMP_EINVAL, "invalid input: head width must be finite and positive");
  if (!finite_f(head->epsilon) || !(head->epsilon > 0.0f))
    return fail(YSKN_SMP_EINVAL, "invalid model: epsilon must be finite and positive");
  if (head->logits_out && head->logits_ld < vocab)
    return fail(YSKN_SMP_EINVAL, "invalid input: head logits_ld < vocab");
  if (head->clear_acc && !head->logits_out)
    return fail(YSKN_SMP_EINVAL, "invalid input: clearing the accumulators needs logits_out");
  if (!h->params_shared && rows > (int32_t)h->params.size())
    return fail(YSKN_SMP_EINVAL, "invalid input: fewer per-row parameter sets than rows");
  if (out_ids && (!positions || n_draws < 1))
    return fail(YSKN_SMP_EINVAL, "invalid input: out_ids needs positions and n_draws >= 1");
  st = check_params_for(h, rows, vocab);
  if (st) return st;
  SmpArgs a = base_args(h, head->acc, rows, vocab, head->acc_ld);
  a.positions = positions;
  a.n_draws = n_draws < 1 ? 1 : n_draws;
  a.out_ids = out_ids;
  a.head_tau = head->tau;
  a.head_us = head->unit_scale;
  a.head_sums = head->block_sums;
  a.head_nblk = head->n_blocks;
  a.head_width = head->width;
  a.head_eps = head->epsilon;
  a.head_out = head->logits_out;
  a.head_out_ld = head->logits_ld;
  a.head_clear = head->clear_acc ? 1 : 0;
  bool pen = false;
  st = apply_aux(h, a, aux, rows, &pen);
  if (st) return st;
  return launch(h, a, 2, pen, aux, (hipStream_t)stream);
}

int yskn_smp_argmax(yskn_smp_handle h, const void* logits, int32_t dtype, int32_t rows,
                    int32_t vocab, int64_t ld, uint32_t* out_ids, void* stream) {
  int st = check_common(h, logits, dtype, rows, vocab, ld);
  if (st) return st;
  if (!out_ids) return fail(YSKN_SMP_EINVAL, "invalid input: null output");
  SmpArgs a = base_args(h, logits, rows, vocab, ld);
  a.argmax = out_ids;
  return launch(h, a, dtype, false, nullptr, (hipStream_t)stream);
}

int yskn_smp_top_tokens(yskn_smp_handle h, const void* logits, int32_t dtype, int32_t rows,
                        int32_t vocab, int64_t ld, int32_t count, uint32_t* out_ids,
                        float* out_vals, void* stream) {
  int st = check_common(h, logits, dtype, rows, vocab, ld);
  if (st) return st;
  if (count < 1) return fail(YSKN_SMP_EINVAL, "invalid input: count must be at least 1");
  if (count > vocab) return fail(YSKN_SMP_EINVAL, "invalid input: top-token count exceeds vocabulary");
  if (!out_ids) return fail(YSKN_SMP_EINVAL, "invalid input: null output");
  SmpArgs a = base_args(h, logits, rows, vocab, ld);
  a.topn = count;
  a.topn_ids = out_ids;
  a.topn_vals = out_vals;
  return launch(h, a, dtype, false, nullptr, (hipStream_t)stream);
}

int yskn_smp_nll(yskn_smp_handle h, const void* logits, int32_t dtype, int32_t rows,
                 int32_t vocab, int64_t ld, const uint32_t* targets, double* out_nll,
                 void* stream) {
  int st = check_common(h, logits, dtype, rows, vocab, ld);
  if (st) return st;
  if (!targets || !out_nll) return fail(YSKN_SMP_EINVAL, "invalid input: null targets or output");
  SmpArgs a = base_args(h, logits, rows, vocab, ld);
  a.nll_targets = targets;
  a.nll_out = out_nll;
  a.want_mass = 1;
  return launch(h, a, dtype, false, nullptr, (hipStream_t)stream);
}

int yskn_smp_verify(yskn_smp_handle h, const void* target_logits, int32_t dtype, int32_t M,
                    int32_t vocab, int64_t ld, const uint32_t* drafts,
                    const uint64_t* base_position, const uint32_t* eos_ids, int32_t n_eos,
                    uint32_t* out_ids, yskn_smp_verify_result* result, const yskn_smp_aux* aux,
                    const yskn_smp_advance* commit, void* stream) {
  int st = check_common(h, target_logits, dtype, M, vocab, ld);
  if (st) return st;
  if (!base_position || !out_ids || !result)
    return fail(YSKN_SMP_EINVAL, "invalid input: null base_position, out_ids or result");
  if (M > 1 && !drafts) return fail(YSKN_SMP_EINVAL, "invalid input: null drafts");
  if (n_eos < 0 || (n_eos > 0 && !eos_ids)) return fail(YSKN_SMP_EINVAL, "invalid input: eos ids");
  if (commit && (!commit->position || !commit->token))
    return fail(YSKN_SMP_EINVAL, "invalid input: commit needs both a position and a token");
  if (!h->params_shared && M > (int32_t)h->params.size())
    return fail(YSKN_SMP_EINVAL, "invalid input: fewer per-row parameter sets than rows");
  st = check_params_for(h, M, vocab);
  if (st) return st;
  SmpArgs a = base_args(h, target_logits, M, vocab, ld);
  a.mode = MODE_VERIFY;
  a.pos_mode = POS_BASE;
  a.base_position = base_position;
  a.out_ids = out_ids;
  a.drafts = drafts;
  a.eos = eos_ids;
  a.n_eos = n_eos;
  a.vresult = (uint32_t*)result;
  a.vcount = h->d_vcount;
  if (commit) {
    a.adv_pos = commit->position;
    a.adv_tok = commit->token;
  }
  bool pen = false;
  st = apply_aux(h, a, aux, M, &pen);
  if (st) return st;
  return launch(h, a, dtype, pen, aux, (hipStream_t)stream);
}

int yskn_smp_draft_shortlist(yskn_smp_handle h, const float* scores, int32_t rows, int32_t vocab,
                             int64_t ld, int32_t count, uint32_t* out_ids, int64_t out_ld,
                             int32_t* row_status, void* stream) {
  int st = draft_rows(h, rows);
  if (st) return st;
  if (!scores || !out_ids) return fail(YSKN_SMP_EINVAL, "invalid input: null scores or output");
  if (vocab <= 0) return fail(YSKN_SMP_EINVAL, "invalid input: empty vocabulary");
  if (ld < vocab) return fail(YSKN_SMP_EINVAL, "invalid input: ld < vocab");
  if (count < 16 || count > 2048 || count % 8 != 0 || count > vocab)
    return fail(YSKN_SMP_EINVAL, "invalid input: shortlist must be 16..2048, multiple of 8 and <= vocabulary");
  if (out_ld < count) return fail(YSKN_SMP_EINVAL, "invalid input: out_ld < count");
  DraftShortlistArgs a;
  std::memset(&a, 0, sizeof a);
  a.scores = scores;
  a.ld = ld;
  a.V = vocab;
  a.rows = rows;
  a.count = count;
  a.out = out_ids;
  a.out_ld = out_ld;
  a.status = h->d_status;
  a.row_status = row_status;
  return draft_launched(h, launch_draft_shortlist(a, (hipStream_t)stream), rows, KIND_SHORTLIST);
}

int yskn_smp_draft_top16(yskn_smp_handle h, const uint32_t* tokens, const float* scores,
                         int32_t rows, int32_t n, int64_t ld, uint32_t* out_tokens,
                         float* out_scores, int32_t* row_status, void* stream) {
  int st = draft_rows(h, rows);
  if (st) return st;
  if (!tokens || !scores || !out_tokens) return fail(YSKN_SMP_EINVAL, "invalid input: null candidates or output");
  if (n < 16) return fail(YSKN_SMP_EINVAL, "invalid input: top16 requires >=16 finite candidates");
  if (n > TOP16_NMAX) return fail(YSKN_SMP_ERANGE, "top16 takes at most 4,096 candidates per row");
  if (ld < n) return fail(YSKN_SMP_EINVAL, "invalid input: ld < n");
  DraftTop16Args a;
  std::memset(&a, 0, sizeof a);
  a.tokens = tokens;
  a.scores = scores;
  a.ld = ld;
  a.n = n;
  a.rows = rows;
  a.out_tokens = out_tokens;
  a.out_scores = out_scores;
  a.status = h->d_status;
  a.row_status = row_status;
  return draft_launched(h, launch_draft_top16(a, (hipStream_t)stream), rows, KIND_TOP16);
}

int yskn_smp_draft_choose(yskn_smp_handle h, const float* scores, const uint32_t* tokens,
                          int32_t rows, int64_t ld, const yskn_smp_draft_choice* choice,
                          const uint64_t* positions, uint32_t* out_tokens, int32_t* alt,
                          float* margin, int32_t* alt3, int32_t* row_status, void* stream) {
  int st = draft_rows(h, rows);
  if (st) return st;
  if (!scores || !tokens || !out_tokens || !choice)
    return fail(YSKN_SMP_EINVAL, "invalid input: null candidates, choice or output");
  if (ld < 16) return fail(YSKN_SMP_EINVAL, "invalid input: choice needs 16 finite candidates");
  const bool sampled = choice->sampled != 0;
  if (sampled && choice->temperature_thousandths == 0)
    return fail(YSKN_SMP_EINVAL, "invalid input: draft temperature must be positive");
  if (sampled && !positions) return fail(YSKN_SMP_EINVAL, "invalid input: a sampled choice needs positions");
  DraftChooseArgs a;
  std::memset(&a, 0, sizeof a);
  a.scores = scores;
  a.tokens = tokens;
  a.ld = ld;
  a.rows = rows;
  a.sampled = sampled ? 1 : 0;
  a.seed = choice->seed;
  // a binary64 multiply, not a division (draft_head.rs:354-356)
  a.temperature = 0.001 * (double)choice->temperature_thousandths;
  a.positions = positions;
  a.out = out_tokens;
  a.alt = alt;
  a.margin = margin;
  a.alt3 = alt3;
  a.status = h->d_status;
  a.row_status = row_status;
  return draft_launched(h, launch_draft_choose(a, (hipStream_t)stream), rows, KIND_CHOOSE);
}

int yskn_smp_sync(yskn_smp_handle h, void* stream) {
  if (!h) return fail(YSKN_SMP_EINVAL, "invalid input: null handle");
  hipError_t e = hipStreamSynchronize((hipStream_t)stream);
  if (e != hipSuccess) return hip_fail(e, "yskn_smp_sync");
  std::vector<int32_t> s(h->last_rows > 0 ? h->last_rows : 1, 0);
  if (h->last_rows > 0) {
    e = hipMemcpy(s.data(), h->d_status, h->last_rows * sizeof(int32_t), hipMemcpyDeviceToHost);
    if (e != hipSuccess) return hip_fail(e, "yskn_smp_sync");
  }
  if (h->last_verify) {
    // a verify fails only on the rows its accept walk reached
    yskn_smp_verify_result r;
    e = hipMemcpy(&r, h->last_verify, sizeof r, hipMemcpyDeviceToHost);
    if (e != hipSuccess) return hip_fail(e, "yskn_smp_sync");
    s.assign(1, r.status);
  }
  for (int32_t v : s) {
    if (v == YSKN_SMP_OK) continue;
    // the reference's messages (draft_head.rs:240-249,285-300,326-336)
    if (h->last_kind == KIND_SHORTLIST) return fail(v, "non-finite value in draft approximate scores");
    if (h->last_kind == KIND_TOP16)
      return fail(v, "invalid input: top16 requires >=16 finite candidates and no duplicate draft candidates");
    if (h->last_kind == KIND_CHOOSE) return fail(v, "invalid input: choice needs 16 finite candidates");
    if (v == YSKN_SMP_ENONFINITE) return fail(v, "non-finite value in logits");
    if (v == YSKN_SMP_EINVAL)
      return fail(v, "invalid input: token outside the vocabulary, invalid history or prediction position overflow");
    if (v != YSKN_SMP_OK) return fail(v, "sampler row failed");
  }
  return YSKN_SMP_OK;
}

int yskn_smp_get_stats(yskn_smp_handle h, uint64_t* out, int32_t n) {
  if (!h || !out || n < 0) return fail(YSKN_SMP_EINVAL, "invalid input: null handle or output");
  unsigned long long v[STAT_COUNT];
  hipError_t e = hipDeviceSynchronize();
  if (e == hipSuccess) e = hipMemcpy(v, h->d_stats, sizeof v, hipMemcpyDeviceToHost);
  if (e != hipSuccess) return hip_fail(e, "yskn_smp_get_stats");
  const int m = n < STAT_COUNT ? n : STAT_COUNT;
  for (int i = 0; i < m; ++i) out[i] = v[i];
  return m;
}

int yskn_smp_select_host(yskn_smp_handle h, const float* host_logits, int32_t vocab,
                         uint64_t prediction_position, uint32_t* out_token) {
  if (!h || !host_logits || !out_token) return fail(YSKN_SMP_EINVAL, "invalid input: null argument");
  if (vocab <= 0)
    return fail(YSKN_SMP_EINVAL, "invalid input: logits must contain a nonempty u32-indexed vocabulary");
  if (vocab > h->max_vocab) return fail(YSKN_SMP_ERANGE, "vocabulary larger than the handle's max_vocab");
  hipError_t e = hipMemcpy(h->d_host_logits, host_logits, (size_t)vocab * 4, hipMemcpyHostToDevice);
  if (e == hipSuccess) e = hipMemcpy(h->d_host_pos, &prediction_position, 8, hipMemcpyHostToDevice);
  if (e != hipSuccess) return hip_fail(e, "yskn_smp_select_host");
  const bool shared = h->params_shared;
  int st = check_params_for(h, 1, vocab);
  if (st) return st;
  SmpArgs a = base_args(h, h->d_host_logits, 1, vocab, vocab);
  a.prm_shared = 1;
  (void)shared;
  a.positions = h->d_host_pos;
  a.out_ids = h->d_host_out;
  if (any_penalty(h, 1)) return fail(YSKN_SMP_EINVAL, "invalid input: penalties need yskn_smp_sample");
  st = launch(h, a, YSKN_SMP_F32, false, nullptr, nullptr);
  if (st) return st;
  st = yskn_smp_sync(h, nullptr);
  if (st) return st;
  e = hipMemcpy(out_token, h->d_host_out, 4, hipMemcpyDeviceToHost);
  if (e != hipSuccess) return hip_fail(e, "yskn_smp_select_host");
  return YSKN_SMP_OK;
}

}  // extern "C"
