/*
 * yskn_oracle.c -- CPU restatement of YASAKANI's per-step sampling path.
 *
 * TEST INFRASTRUCTURE ONLY (see yskn_oracle.h): the checker for the HIP
 * sampler, never part of the product path.
 *
 * Sources restated (all paths relative to the reference repository):
 *   crates/yskn-ref/src/portable_math.rs:52-58,224-364   exp_d, log_d
 *   crates/yskn-ref/src/output_head_sampler.rs:21-250     sampler, NLL
 *   crates/yskn-ref/src/speculation.rs:483-523            acceptance loop
 *   crates/yskn-ref/src/draft_head.rs:219-379             draft shortlist, top 16, coupling
 *   crates/yskn-ref/src/portable_math.rs:61-111           sqrt_rn, rsqrt
 *   crates/yskn-ref/src/residual_norm_mlp.rs:37-46        inverse RMS of the head input
 *   crates/yskn-ref/src/compressed_linear.rs:329-340      head scale restoration
 *   docs/spec/06_OUTPUT_HEAD_SAMPLER.md:21-230            normative text
 *
 * Compile with -ffp-contract=off and without -ffast-math: each binary64
 * multiply and add below must round separately.
 */
#define _GNU_SOURCE
#include "yskn_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------------ */
/* Bit helpers (portable_math.rs:52-58).                                     */
/* ------------------------------------------------------------------------ */
static inline uint64_t bits_of(double x) {
  uint64_t b;
  memcpy(&b, &x, sizeof b);
  return b;
}
static inline double from_bits(uint64_t b) {
  double x;
  memcpy(&x, &b, sizeof x);
  return x;
}
static inline double hilo(uint32_t hi, uint32_t lo) {
  return from_bits(((uint64_t)hi << 32) | (uint64_t)lo);
}
static inline uint32_t f32_bits(float x) {
  uint32_t b;
  memcpy(&b, &x, sizeof b);
  return b;
}
static inline int f32_finite(float x) { return (f32_bits(x) & 0x7f800000u) != 0x7f800000u; }

/* ------------------------------------------------------------------------ */
/* exp_d: portable_math.rs:224-283. fdlibm e_exp.c method: argument
 * reduction x = k*ln2 + r with ln2 split in a hi/lo pair, a degree-5
 * minimax polynomial in r*r for R(r*r), and reconstruction
 * 1 - ((lo - r*c/(2-c)) - hi) scaled by 2^k through the exponent word. */
/* ------------------------------------------------------------------------ */
static double scale_exp_word(double value, int32_t adjustment) {
  /* portable_math.rs:285-291: add adjustment to the exponent field of the
   * high word with wrapping 32-bit integer arithmetic. */
  uint64_t b = bits_of(value);
  uint32_t hi = (uint32_t)(b >> 32);
  uint32_t adj = hi + (uint32_t)adjustment * 1048576u;
  return hilo(adj, (uint32_t)b);
}

double yo_exp_d(double value) {
  const uint64_t b = bits_of(value);
  const uint32_t hi = (uint32_t)(b >> 32);
  const uint32_t lo = (uint32_t)b;
  const int neg = (hi >> 31) != 0;
  const uint32_t ahi = hi & 0x7fffffffu;
  if (ahi >= 0x40862e42u) {
    if (ahi >= 0x7ff00000u) {
      if (((ahi & 0x000fffffu) | lo) != 0) return value + value; /* NaN */
      return neg ? 0.0 : value;                                  /* +-inf */
    }
    if (value > hilo(0x40862e42u, 0xfefa39efu)) return INFINITY;
    if (value < hilo(0xc0874910u, 0xd52d3051u)) return 0.0;
  }
  const double ln2_hi = hilo(0x3fe62e42u, 0xfee00000u);
  const double ln2_lo = hilo(0x3dea39efu, 0x35793c76u);
  double h = 0.0, l = 0.0, r = value;
  int32_t k = 0;
  if (ahi > 0x3fd62e42u) {
    if (ahi < 0x3ff0a2b2u) {
      h = value - (neg ? -ln2_hi : ln2_hi);
      l = neg ? -ln2_lo : ln2_lo;
      k = neg ? -1 : 1;
    } else {
      /* truncation toward zero, as Rust's `as i32` for this bounded range */
      double t = hilo(0x3ff71547u, 0x652b82feu) * value;
      t = t + (neg ? -0.5 : 0.5);
      k = (int32_t)t;
      const double kf = (double)k;
      double kh = kf * ln2_hi;
      h = value - kh;
      l = kf * ln2_lo;
    }
    r = h - l;
  } else if (ahi < 0x3e300000u) {
    return 1.0 + value;
  }
  const double s = r * r;
  /* Horner nesting with a rounding after every product and sum. */
  double poly = s * hilo(0x3e663769u, 0x72bea4d0u);
  poly = hilo(0xbebbbd41u, 0xc5d26bf1u) + poly;
  poly = s * poly;
  poly = hilo(0x3f11566au, 0xaf25de2cu) + poly;
  poly = s * poly;
  poly = hilo(0xbf66c16cu, 0x16bebd93u) + poly;
  poly = s * poly;
  poly = hilo(0x3fc55555u, 0x5555553eu) + poly;
  double sp = s * poly;
  const double c = r - sp;
  if (k == 0) {
    double rc = r * c;
    double q = rc / (c - 2.0);
    return 1.0 - (q - r);
  }
  double rc = r * c;
  double q = rc / (2.0 - c);
  double y = 1.0 - ((l - q) - h);
  if (k >= -1021) return scale_exp_word(y, k);
  return scale_exp_word(y, k + 1000) * hilo(0x01700000u, 0u);
}

/* ------------------------------------------------------------------------ */
/* log_d: portable_math.rs:297-364. fdlibm e_log.c method: x = 2^k (1+f)
 * with sqrt(2)/2 < 1+f < sqrt(2), s = f/(2+f), log(1+f) = f - s*(f - R(s))
 * with R split in even/odd polynomials of s^2. No zero special case: +-0
 * flow through the subnormal branch and return finite values. */
/* ------------------------------------------------------------------------ */
double yo_log_d(double value) {
  int32_t hx = (int32_t)(uint32_t)(bits_of(value) >> 32);
  int32_t k = 0;
  if (hx < 0x00100000) {
    value = value * hilo(0x43500000u, 0u); /* 2^54 */
    k = -54;
    hx = (int32_t)(uint32_t)(bits_of(value) >> 32);
  }
  k += (hx >> 20) - 1023; /* arithmetic shift, as Rust's i32 >> */
  hx &= 0x000fffff;
  const int32_t i = (hx + 0x00095f64) & 0x00100000;
  value = hilo((uint32_t)(hx | (i ^ 0x3ff00000)), (uint32_t)bits_of(value));
  k += i >> 20;
  const double ln2_hi = hilo(0x3fe62e42u, 0xfee00000u);
  const double ln2_lo = hilo(0x3dea39efu, 0x35793c76u);
  const double f = value - 1.0;
  if ((0x000fffff & (2 + hx)) < 3) {
    if (f == 0.0) {
      if (k == 0) return 0.0;
      const double dk = (double)k;
      double a = dk * ln2_hi;
      double b2 = dk * ln2_lo;
      return a + b2;
    }
    double ff = f * f;
    double t = hilo(0x3fd55555u, 0x55555555u) * f;
    t = 0.5 - t;
    const double R = ff * t;
    if (k == 0) return f - R;
    const double dk = (double)k;
    double a = dk * ln2_hi;
    double b2 = dk * ln2_lo;
    return a - ((R - b2) - f);
  }
  const double s = f / (2.0 + f);
  const double dk = (double)k;
  const double z = s * s;
  const double w = z * z;
  const int32_t j = (hx - 0x0006147a) | (0x0006b851 - hx);
  /* even terms: w*(Lg2 + w*(Lg4 + w*Lg6)) */
  double t2 = w * hilo(0x3fc39a09u, 0xd078c69fu);
  t2 = hilo(0x3fcc71c5u, 0x1d8e78afu) + t2;
  t2 = w * t2;
  t2 = hilo(0x3fd99999u, 0x9997fa04u) + t2;
  t2 = w * t2;
  /* odd terms: z*(Lg1 + w*(Lg3 + w*(Lg5 + w*Lg7))) */
  double t1 = w * hilo(0x3fc2f112u, 0xdf3e5244u);
  t1 = hilo(0x3fc74664u, 0x96cb03deu) + t1;
  t1 = w * t1;
  t1 = hilo(0x3fd24924u, 0x94229359u) + t1;
  t1 = w * t1;
  t1 = hilo(0x3fe55555u, 0x55555593u) + t1;
  t1 = z * t1;
  const double R = t1 + t2;
  if (j > 0) {
    double hfsq = 0.5 * f;
    hfsq = hfsq * f;
    if (k == 0) {
      double u = hfsq + R;
      u = s * u;
      u = hfsq - u;
      return f - u;
    }
    double u = hfsq + R;
    u = s * u;
    double b2 = dk * ln2_lo;
    u = u + b2;
    u = hfsq - u;
    u = u - f;
    double a = dk * ln2_hi;
    return a - u;
  }
  if (k == 0) {
    double u = f - R;
    u = s * u;
    return f - u;
  }
  double u = f - R;
  u = s * u;
  double b2 = dk * ln2_lo;
  u = u - b2;
  u = u - f;
  double a = dk * ln2_hi;
  return a - u;
}

/* ------------------------------------------------------------------------ */
/* Hash and noise: output_head_sampler.rs:214-228; spec 06 section 6.        */
/* ------------------------------------------------------------------------ */
uint64_t yo_mix64(uint64_t z) {
  z += 0x9e3779b97f4a7c15ull;
  z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
  z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
  return z ^ (z >> 31);
}

double yo_gumbel(uint64_t seed, uint64_t position, uint32_t token) {
  const uint64_t a = yo_mix64(seed);
  const uint64_t b = yo_mix64(a ^ position);
  const uint64_t h = yo_mix64(b ^ ((uint64_t)token * 0xd6e8feb86659fd93ull));
  double u = (double)(h >> 11) + 0.5;
  u = u * (1.0 / 9007199254740992.0);
  return -yo_log_d(-yo_log_d(u));
}

double yo_uniform_v2(uint64_t seed, uint64_t position) {
  const uint64_t h = yo_mix64(yo_mix64(seed) ^ position);
  return (double)(h >> 11) * (1.0 / 9007199254740992.0);
}

/* ------------------------------------------------------------------------ */
/* Parameters: output_head_sampler.rs:30-75.                                  */
/* ------------------------------------------------------------------------ */
void yo_default_params(yo_params* p) {
  p->temperature = 1.0;
  p->top_p = 0.95;
  p->top_k = 20;
  p->min_p = 0.0;
  p->seed = 0;
  p->version = YO_VERSION_GUMBEL;
  p->extension_top_k = 0;
}

int yo_validate(const yo_params* p, uint64_t V) {
  if (!isfinite(p->temperature) || p->temperature <= 0.0) return YO_EINVAL;
  if (!isfinite(p->top_p) || p->top_p <= 0.0 || p->top_p > 1.0) return YO_EINVAL;
  if (!isfinite(p->min_p) || !(p->min_p >= 0.0 && p->min_p <= 1.0)) return YO_EINVAL;
  if (p->version != YO_VERSION_GUMBEL && p->version != YO_VERSION_INVERSE_CDF) return YO_EINVAL;
  if (p->extension_top_k) {
    if (p->top_k > V) return YO_EINVAL;
  } else {
    if (p->top_k == 0 || p->top_k > 20 || p->top_k > V) return YO_EINVAL;
  }
  return YO_OK;
}

int yo_params_from_thousandths(uint32_t t, uint32_t tp, uint32_t mp, yo_params* out) {
  yo_default_params(out);
  /* Division, not multiplication by 0.001 (output_head_sampler.rs:46-49). */
  out->temperature = (double)t / 1000.0;
  out->top_p = (double)tp / 1000.0;
  out->min_p = (double)mp / 1000.0;
  return yo_validate(out, 20);
}

/* ------------------------------------------------------------------------ */
/* Selection: output_head_sampler.rs:94-134.                                 */
/* ------------------------------------------------------------------------ */
int yo_validate_logits(const float* logits, uint64_t V) {
  if (V == 0 || V > 0xffffffffull) return YO_EINVAL;
  for (uint64_t i = 0; i < V; ++i)
    if (!f32_finite(logits[i])) return YO_ENONFINITE;
  return YO_OK;
}

int yo_greedy(const float* logits, uint64_t V, uint32_t* out) {
  int st = yo_validate_logits(logits, V);
  if (st) return st;
  uint64_t sel = 0;
  for (uint64_t t = 1; t < V; ++t)
    if (logits[t] > logits[sel]) sel = t; /* strict: smaller id keeps ties */
  *out = (uint32_t)sel;
  return YO_OK;
}

/* Comparator of output_head_sampler.rs:124-132: larger logit first, then
 * smaller id. qsort_r's context carries the logits. */
static int cmp_tokens(const void* a, const void* b, void* ctx) {
  const float* lg = (const float*)ctx;
  const uint32_t l = *(const uint32_t*)a, r = *(const uint32_t*)b;
  if (lg[l] > lg[r]) return -1;
  if (lg[l] < lg[r]) return 1;
  return l < r ? -1 : (l > r ? 1 : 0);
}

static uint32_t* sorted_tokens(const float* logits, uint64_t V) {
  uint32_t* ids = (uint32_t*)malloc(V * sizeof(uint32_t));
  if (!ids) return NULL;
  for (uint64_t i = 0; i < V; ++i) ids[i] = (uint32_t)i;
  qsort_r(ids, V, sizeof(uint32_t), cmp_tokens, (void*)logits);
  return ids;
}

int yo_top_tokens(const float* logits, uint64_t V, uint64_t count, uint32_t* out) {
  int st = yo_validate_logits(logits, V);
  if (st) return st;
  if (count > V) return YO_EINVAL;
  uint32_t* ids = sorted_tokens(logits, V);
  if (!ids) return YO_EINVAL;
  memcpy(out, ids, count * sizeof(uint32_t));
  free(ids);
  return YO_OK;
}

/* ------------------------------------------------------------------------ */
/* sample(): output_head_sampler.rs:136-212. `cands` is the full sorted    */
/* order; the first k entries are the candidates.                             */
/* ------------------------------------------------------------------------ */
typedef struct truncation {
  uint64_t k, n, retained;
  double* adjusted;
  double* weights;
  double total;
} truncation;

static int truncate_candidates(const float* logits, const uint32_t* cands, uint64_t k,
                               const yo_params* p, truncation* tr) {
  tr->k = k;
  tr->adjusted = (double*)malloc(k * sizeof(double));
  tr->weights = (double*)malloc(k * sizeof(double));
  if (!tr->adjusted || !tr->weights) return YO_EINVAL;
  const double maximum = (double)logits[cands[0]];
  double total = 0.0;
  for (uint64_t j = 0; j < k; ++j) {
    /* widen, subtract, divide: three separately rounded steps */
    double diff = (double)logits[cands[j]] - maximum;
    double value = diff / p->temperature;
    if (!isfinite(value)) return YO_ENONFINITE;
    double w = yo_exp_d(value);
    if (!isfinite(w)) return YO_ENONFINITE;
    tr->adjusted[j] = value;
    tr->weights[j] = w;
    total = total + w; /* serial, in candidate order */
  }
  tr->total = total;
  uint64_t retained = k;
  double prefix = 0.0;
  for (uint64_t j = 0; j < k; ++j) {
    prefix = prefix + tr->weights[j];
    double threshold = p->top_p * total;
    if (prefix >= threshold) {
      retained = j + 1;
      break;
    }
  }
  tr->n = retained;
  if (p->min_p > 0.0) {
    uint64_t m = 1;
    while (m < retained && tr->weights[m] >= p->min_p) ++m;
    retained = m;
  }
  tr->retained = retained;
  return YO_OK;
}

static int draw(const uint32_t* cands, const truncation* tr, uint64_t position,
                const yo_params* p, uint64_t* pick, yo_diag* diag) {
  uint64_t selected = tr->retained - 1;
  if (p->version == YO_VERSION_GUMBEL) {
    double best = -INFINITY;
    for (uint64_t j = 0; j < tr->retained; ++j) {
      double cand = tr->adjusted[j] + yo_gumbel(p->seed, position, cands[j]);
      if (!isfinite(cand)) return YO_ENONFINITE;
      if (cand > best) {
        best = cand;
        selected = j;
      }
    }
  } else {
    double mass = 0.0;
    for (uint64_t j = 0; j < tr->retained; ++j) mass = mass + tr->weights[j];
    const double uniform = yo_uniform_v2(p->seed, position);
    const double threshold = uniform * mass;
    if (diag) {
      diag->kept = mass;
      diag->uniform = uniform;
      diag->threshold = threshold;
    }
    double prefix = 0.0;
    for (uint64_t j = 0; j < tr->retained; ++j) {
      prefix = prefix + tr->weights[j];
      if (threshold < prefix) {
        selected = j;
        break;
      }
    }
  }
  *pick = selected;
  return YO_OK;
}

static void free_truncation(truncation* tr) {
  free(tr->adjusted);
  free(tr->weights);
}

int yo_sample(const float* logits, uint64_t V, uint64_t position, const yo_params* p,
              uint32_t* out, yo_diag* diag) {
  int st = yo_validate_logits(logits, V);
  if (st) return st;
  st = yo_validate(p, V);
  if (st) return st;
  const uint64_t k = p->top_k == 0 ? V : p->top_k;
  uint32_t* cands = sorted_tokens(logits, V);
  if (!cands) return YO_EINVAL;
  truncation tr = {0};
  st = truncate_candidates(logits, cands, k, p, &tr);
  uint64_t pick = 0;
  if (diag) {
    diag->kept = 0.0;
    diag->uniform = 0.0;
    diag->threshold = 0.0;
  }
  if (!st) st = draw(cands, &tr, position, p, &pick, diag);
  if (!st) {
    *out = cands[pick];
    if (diag) {
      diag->k = tr.k;
      diag->n_top_p = tr.n;
      diag->retained = tr.retained;
      diag->pick = pick;
      diag->total = tr.total;
    }
  }
  free_truncation(&tr);
  free(cands);
  return st;
}

int yo_sample_positions(const float* logits, uint64_t V, const uint64_t* positions, uint64_t n,
                        const yo_params* p, uint32_t* out) {
  int st = yo_validate_logits(logits, V);
  if (st) return st;
  st = yo_validate(p, V);
  if (st) return st;
  const uint64_t k = p->top_k == 0 ? V : p->top_k;
  uint32_t* cands = sorted_tokens(logits, V);
  if (!cands) return YO_EINVAL;
  truncation tr = {0};
  st = truncate_candidates(logits, cands, k, p, &tr);
  for (uint64_t i = 0; !st && i < n; ++i) {
    uint64_t pick = 0;
    st = draw(cands, &tr, positions[i], p, &pick, NULL);
    if (!st) out[i] = cands[pick];
  }
  free_truncation(&tr);
  free(cands);
  return st;
}

/* ------------------------------------------------------------------------ */
/* NLL: output_head_sampler.rs:230-250.                                       */
/* ------------------------------------------------------------------------ */
int yo_mass(const float* logits, uint64_t V, double* mass, float* maximum) {
  int st = yo_validate_logits(logits, V);
  if (st) return st;
  float mx = -INFINITY;
  for (uint64_t i = 0; i < V; ++i) mx = fmaxf(mx, logits[i]);
  double m = 0.0;
  for (uint64_t i = 0; i < V; ++i) {
    double d = (double)logits[i] - (double)mx;
    m = m + yo_exp_d(d); /* ascending token order */
  }
  *mass = m;
  *maximum = mx;
  return YO_OK;
}

int yo_nll(const float* logits, uint64_t V, uint32_t target, double* out) {
  double mass;
  float mx;
  int st = yo_mass(logits, V, &mass, &mx);
  if (st) return st;
  if ((uint64_t)target >= V) return YO_EINVAL;
  double a = (double)mx - (double)logits[target];
  double loss = a + yo_log_d(mass);
  if (!isfinite(loss)) return YO_ENONFINITE;
  *out = loss;
  return YO_OK;
}

int yo_top_logprobs(const float* logits, uint64_t V, uint64_t n, uint32_t* ids,
                    double* logprobs) {
  double mass;
  float mx;
  int st = yo_mass(logits, V, &mass, &mx);
  if (st) return st;
  if (n > V) return YO_EINVAL;
  st = yo_top_tokens(logits, V, n, ids);
  if (st) return st;
  const double lm = yo_log_d(mass);
  for (uint64_t i = 0; i < n; ++i) {
    double a = (double)mx - (double)logits[ids[i]];
    double loss = a + lm;
    logprobs[i] = -loss;
  }
  return YO_OK;
}

/* ------------------------------------------------------------------------ */
/* EXTENSIONS: bf16 widening and penalties.                                  */
/* ------------------------------------------------------------------------ */
void yo_bf16_to_f32(const uint16_t* in, float* out, uint64_t n) {
  for (uint64_t i = 0; i < n; ++i) {
    uint32_t b = (uint32_t)in[i] << 16;
    memcpy(&out[i], &b, sizeof b);
  }
}

int yo_apply_penalties(float* logits, uint64_t V, const uint32_t* history, uint64_t len,
                       float rep, float pres, float freq) {
  if (!(rep > 0.0f) || !f32_finite(rep) || !f32_finite(pres) || !f32_finite(freq))
    return YO_EINVAL;
  uint32_t* count = (uint32_t*)calloc(V ? V : 1, sizeof(uint32_t));
  if (!count) return YO_EINVAL;
  for (uint64_t i = 0; i < len; ++i) {
    if ((uint64_t)history[i] >= V) {
      free(count);
      return YO_EINVAL;
    }
    count[history[i]] += 1;
  }
  for (uint64_t v = 0; v < V; ++v) {
    const uint32_t c = count[v];
    if (c == 0) continue;
    float l = logits[v];
    if (rep != 1.0f) l = l > 0.0f ? l / rep : l * rep;
    float fc = freq * (float)c;
    l = l - fc;
    l = l - pres;
    logits[v] = l;
  }
  free(count);
  return YO_OK;
}

/* ------------------------------------------------------------------------ */
/* Speculative acceptance: speculation.rs:483-523.                           */
/* ------------------------------------------------------------------------ */
int yo_verify(const float* rows, uint64_t M, uint64_t V, uint64_t ld, const uint32_t* guesses,
              uint64_t base_position, const yo_params* p, int greedy, const uint32_t* eos_ids,
              uint64_t n_eos, uint32_t* selected, uint64_t* emitted, uint64_t* accepted,
              int* stop_eos) {
  uint64_t em = 0, acc = 0;
  int eos = 0;
  for (uint64_t row = 0; row < M; ++row) {
    /* checked_add: no wrap past 2^64 - 1 (speculation.rs:489-497) */
    if (base_position > UINT64_MAX - (row + 1)) return YO_EINVAL;
    const uint64_t pos = base_position + row + 1;
    uint32_t sel = 0;
    int st = greedy ? yo_greedy(rows + row * ld, V, &sel)
                    : yo_sample(rows + row * ld, V, pos, p, &sel, NULL);
    if (st) return st;
    selected[row] = sel;
    ++em;
    const int matched = row + 1 < M && guesses[row] == sel;
    acc += (uint64_t)matched;
    for (uint64_t e = 0; e < n_eos; ++e)
      if (eos_ids[e] == sel) eos = 1;
    if (eos || !matched) break;
  }
  *emitted = em;
  *accepted = acc;
  *stop_eos = eos;
  return YO_OK;
}

/* ------------------------------------------------------------------------ */
/* Draft coupling: draft_head.rs:325-379.                                    */
/* ------------------------------------------------------------------------ */
int yo_draft_choose_ex(const float* scores, const uint32_t* tokens, int greedy, uint64_t seed,
                       uint32_t temperature_thousandths, uint64_t position, uint32_t* out,
                       yo_draft_diag* diag) {
  for (int i = 0; i < 16; ++i)
    if (!f32_finite(scores[i])) return YO_EINVAL;
  /* greedy part: first strictly larger score in input order (:331-336) */
  int best = 0;
  for (int i = 1; i < 16; ++i)
    if (scores[i] > scores[best]) best = i;
  if (greedy) {
    *out = tokens[best];
    return YO_OK;
  }
  if (temperature_thousandths == 0) return YO_EINVAL;
  int order[16];
  for (int i = 0; i < 16; ++i) order[i] = i;
  /* insertion sort by (score desc, token asc); 16 entries (:346-353) */
  for (int i = 1; i < 16; ++i) {
    int o = order[i], j = i;
    while (j > 0) {
      int q = order[j - 1];
      int before = scores[o] > scores[q] || (scores[o] == scores[q] && tokens[o] < tokens[q]);
      if (!before) break;
      order[j] = q;
      --j;
    }
    order[j] = o;
  }
  /* binary64 multiply by 0.001, not division (draft_head.rs:354-355) */
  const double temperature = 0.001 * (double)temperature_thousandths;
  double z[16], w[16];
  for (int i = 0; i < 16; ++i) {
    double d = (double)scores[i] - (double)scores[order[0]];
    z[i] = d / temperature;
    w[i] = yo_exp_d(z[i]);
  }
  double total = 0.0;
  for (int i = 0; i < 16; ++i) total = total + w[order[i]];
  double prefix = 0.0, maximum = -INFINITY;
  int member[16] = {0};
  for (int t = 0; t < 16; ++t) {
    const int i = order[t];
    /* membership is decided before this candidate's weight is added (:368-377) */
    double lim = 0.95 * total;
    if (prefix < lim) {
      member[i] = 1;
      double score = z[i] + yo_gumbel(seed, position, tokens[i]);
      if (score > maximum) {
        maximum = score;
        best = i;
      }
    }
    prefix = prefix + w[i];
  }
  if (diag) {
    diag->temperature = temperature;
    diag->total = total;
    for (int i = 0; i < 16; ++i) {
      diag->z[i] = z[i];
      diag->w[i] = w[i];
      diag->order[i] = order[i];
      diag->member[i] = member[i];
    }
  }
  *out = tokens[best];
  return YO_OK;
}

int yo_draft_choose(const float* scores, const uint32_t* tokens, uint64_t seed,
                    uint32_t temperature_thousandths, uint64_t position, uint32_t* out) {
  return yo_draft_choose_ex(scores, tokens, 0, seed, temperature_thousandths, position, out, NULL);
}

/* ------------------------------------------------------------------------ */
/* Draft shortlist and top 16: draft_head.rs:219-300.                        */
/* ------------------------------------------------------------------------ */
/* Order-preserving key without canonicalising -0 (draft_head.rs:219-226). */
static inline uint32_t draft_key(float x) {
  const uint32_t u = f32_bits(x);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

/* Highest bin b with (count of bins > b) + hist[b] >= need; *above = count of
 * bins > b (draft_head.rs:227-236). */
static uint64_t cutoff_bin(const uint64_t* hist, uint64_t nbins, uint64_t need, uint64_t* above) {
  uint64_t a = 0;
  for (uint64_t b = nbins; b-- > 0;) {
    if (a + hist[b] >= need) {
      *above = a;
      return b;
    }
    a += hist[b];
  }
  *above = a;
  return 0;
}

int yo_shortlist(const float* scores, uint64_t V, uint64_t count, uint32_t* out) {
  for (uint64_t i = 0; i < V; ++i)
    if (!f32_finite(scores[i])) return YO_ENONFINITE;
  if (count < 16 || count > 2048 || count % 8 != 0 || count > V || V > 0x7fffffffull)
    return YO_EINVAL;
  uint64_t* h1 = (uint64_t*)calloc(1024, sizeof(uint64_t));
  uint64_t* h2 = (uint64_t*)calloc(2048, sizeof(uint64_t));
  if (!h1 || !h2) {
    free(h1);
    free(h2);
    return YO_EINVAL;
  }
  for (uint64_t i = 0; i < V; ++i) h1[draft_key(scores[i]) >> 22] += 1;
  uint64_t above1 = 0, above2 = 0;
  const uint64_t first = cutoff_bin(h1, 1024, count, &above1);
  for (uint64_t i = 0; i < V; ++i) {
    const uint32_t k = draft_key(scores[i]);
    if ((uint64_t)(k >> 22) == first) h2[(k >> 11) & 2047u] += 1;
  }
  const uint64_t second = cutoff_bin(h2, 2048, count - above1, &above2);
  const uint32_t prefix = (uint32_t)((first << 11) | second);
  uint64_t n = 0;
  for (uint64_t i = 0; i < V; ++i)
    if ((draft_key(scores[i]) >> 11) > prefix) out[n++] = (uint32_t)i;
  for (uint64_t i = 0; i < V && n < count; ++i)
    if ((draft_key(scores[i]) >> 11) == prefix) out[n++] = (uint32_t)i;
  free(h1);
  free(h2);
  return n == count ? YO_OK : YO_EINVAL;
}

int yo_top16(const uint32_t* tokens, const float* scores, uint64_t n, uint32_t* out_tokens,
             float* out_scores) {
  if (n < 16) return YO_EINVAL;
  for (uint64_t i = 0; i < n; ++i)
    if (!f32_finite(scores[i])) return YO_EINVAL;
  uint64_t* idx = (uint64_t*)malloc(n * sizeof(uint64_t));
  if (!idx) return YO_EINVAL;
  for (uint64_t i = 0; i < n; ++i) idx[i] = i;
  /* insertion sort by (score desc, token asc): n is a shortlist (<= 2048) */
  for (uint64_t i = 1; i < n; ++i) {
    const uint64_t o = idx[i];
    uint64_t j = i;
    while (j > 0) {
      const uint64_t q = idx[j - 1];
      const int before = scores[o] > scores[q] || (scores[o] == scores[q] && tokens[o] < tokens[q]);
      if (!before) break;
      idx[j] = q;
      --j;
    }
    idx[j] = o;
  }
  /* distinct tokens are required (draft_head.rs:292-299): equal tokens end up
   * adjacent only when their scores are equal too, so compare every pair */
  int dup = 0;
  for (uint64_t i = 0; i < n && !dup; ++i)
    for (uint64_t j = i + 1; j < n; ++j)
      if (tokens[i] == tokens[j]) {
        dup = 1;
        break;
      }
  if (!dup) {
    for (int i = 0; i < 16; ++i) {
      out_tokens[i] = tokens[idx[i]];
      out_scores[i] = scores[idx[i]];
    }
  }
  free(idx);
  return dup ? YO_EINVAL : YO_OK;
}

/* ------------------------------------------------------------------------ */
/* Head epilogue: spec 06 section 2; compressed_linear.rs:329-340;          */
/* residual_norm_mlp.rs:37-46; portable_math.rs:61-111.                      */
/* ------------------------------------------------------------------------ */
/* Correctly rounded binary32 square root from an integer square root: for a
 * normalised radicand m * 2^(2e) with m < 2^48, r = isqrt(m) has 24 or 25
 * significant bits; the remainder m - r^2 decides round-to-nearest exactly
 * (a halfway case would need m = (r + 1/2)^2, impossible for an integer m). */
static uint64_t isqrt_u64(uint64_t m) {
  uint64_t r = 0, bit = 1ull << 62;
  while (bit > m) bit >>= 2;
  while (bit) {
    if (m >= r + bit) {
      m -= r + bit;
      r = (r >> 1) + bit;
    } else {
      r >>= 1;
    }
    bit >>= 2;
  }
  return r;
}

float yo_sqrt_rn(float value) {
  const uint32_t b = f32_bits(value);
  if ((b & 0x7fffffffu) == 0 || b == 0x7f800000u) return value; /* +-0, +inf */
  if ((b & 0x80000000u) || (b & 0x7f800000u) == 0x7f800000u) return NAN;
  uint64_t sig;
  int e; /* value = sig * 2^e */
  if ((b >> 23) == 0) {
    sig = b & 0x007fffffu;
    e = -149;
  } else {
    sig = (b & 0x007fffffu) | 0x00800000u;
    e = (int)(b >> 23) - 150;
  }
  /* scale sig to [2^46, 2^48) with an even exponent */
  int lz = __builtin_clzll(sig); /* sig < 2^24 */
  int shift = (63 - lz <= 46) ? (46 - (63 - lz)) : 0;
  int ee = e - shift;
  if (ee & 1) {
    shift += 1;
    ee -= 1;
  }
  const uint64_t m = sig << shift; /* m in [2^46, 2^48) */
  uint64_t r = isqrt_u64(m);        /* in [2^23, 2^24] */
  const uint64_t rem = m - r * r;
  if (rem > r) r += 1;              /* m - r^2 > r + 1/4 <=> m > (r + 1/2)^2 */
  int ex = ee / 2;                  /* sqrt(value) ~ r * 2^ex */
  if (r == (1ull << 24)) {
    r >>= 1;
    ex += 1;
  }
  /* r in [2^23, 2^24): value bits = (ex + 23 + 127) << 23 | (r - 2^23) */
  const uint32_t out = ((uint32_t)(ex + 23 + 127) << 23) | ((uint32_t)r & 0x007fffffu);
  float f;
  memcpy(&f, &out, 4);
  return f;
}

float yo_rsqrt(float value) {
  volatile float s = yo_sqrt_rn(value);
  return 1.0f / s;
}

int yo_inverse_rms(const float* block_sums, uint64_t n_blocks, float width, float epsilon,
                   float* out) {
  float total = 0.0f;
  for (uint64_t b = 0; b < n_blocks; ++b) total = total + block_sums[b];
  if (!f32_finite(total)) return YO_ENONFINITE;
  float q = total / width;
  float arg = q + epsilon;
  if (!f32_finite(arg)) return YO_ENONFINITE;
  float r = yo_rsqrt(arg);
  if (!f32_finite(r)) return YO_ENONFINITE;
  *out = r;
  return YO_OK;
}

int yo_head_logits(const int64_t* acc, const float* tau, uint64_t V, float unit_scale,
                   float inverse_rms, float* out) {
  if (!f32_finite(inverse_rms)) return YO_ENONFINITE;
  int bad = 0;
  for (uint64_t v = 0; v < V; ++v) {
    float x = (float)acc[v]; /* one round-to-nearest conversion */
    x = x * unit_scale;
    x = x * inverse_rms;
    x = x * tau[v];
    out[v] = x;
    bad |= !f32_finite(x);
  }
  return bad ? YO_ENONFINITE : YO_OK;
}
