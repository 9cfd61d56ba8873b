/*
 * yskn_oracle.h -- CPU restatement of YASAKANI's per-step sampling path.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the checker for the HIP sampler:
 * only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
 * load it. The product path never calls it and never falls back to it.
 *
 * Every function restates one function of the reference's scalar
 * specification (Rust crate crates/yskn-ref), citing file:line. Functions
 * marked EXTENSION implement behaviour the reference does not have; their
 * semantics are defined here and are "parity unpinned" against the reference
 * (they are pinned only by the properties the tests check).
 *
 * Build: plain C11, -O3 -ffp-contract=off, no -ffast-math. Every binary64
 * operation is a separately rounded IEEE operation, as the reference's
 * portable math requires (crates/yskn-ref/src/portable_math.rs:1-7).
 */
#ifndef YSKN_ORACLE_H
#define YSKN_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes. Same numbering as the product C-ABI (include/yskn_smp.h). */
#define YO_OK 0
#define YO_EINVAL (-1)    /* Error::InvalidInput (crates/yskn-ref/src/lib.rs:42) */
#define YO_ENONFINITE (-2) /* Error::NonFinite (crates/yskn-ref/src/lib.rs:43) */

/* SamplingVersion (output_head_sampler.rs:14-18): 2 = InverseCumulative, 3 = Gumbel. */
#define YO_VERSION_INVERSE_CDF 2
#define YO_VERSION_GUMBEL 3

/* SamplingParameters (output_head_sampler.rs:21-41). */
typedef struct yo_params {
  double temperature;
  double top_p;
  uint64_t top_k;  /* 0 = disabled (k = V); only with extension_top_k */
  double min_p;
  uint64_t seed;
  int version;     /* YO_VERSION_* */
  int extension_top_k; /* EXTENSION: lift the 1..=20 cap to 1..=V, 0 = disabled */
} yo_params;

/* Diagnostics of one sample() call: sizes of the truncation stages. */
typedef struct yo_diag {
  uint64_t k;        /* candidate count after top-k */
  uint64_t n_top_p;  /* retained after top-p */
  uint64_t retained; /* retained after min-p */
  uint64_t pick;     /* selected candidate index */
  double total;      /* serial binary64 total of the top-k weights */
  double kept;       /* version 2: serial binary64 mass of the retained weights */
  double uniform;    /* version 2: the position-keyed uniform */
  double threshold;  /* version 2: uniform * kept */
} yo_diag;

/* ---- portable math (portable_math.rs:224-364) ---------------------------- */
double yo_exp_d(double value);
double yo_log_d(double value);

/* ---- hashing and noise (output_head_sampler.rs:214-228) ------------------ */
uint64_t yo_mix64(uint64_t value);
double yo_gumbel(uint64_t seed, uint64_t position, uint32_t token);
/* Version-2 uniform (output_head_sampler.rs:196-197). */
double yo_uniform_v2(uint64_t seed, uint64_t position);

/* ---- parameters (output_head_sampler.rs:43-75) --------------------------- */
void yo_default_params(yo_params* p);
int yo_params_from_thousandths(uint32_t temperature, uint32_t top_p, uint32_t min_p,
                               yo_params* out);
int yo_validate(const yo_params* p, uint64_t vocabulary_size);

/* ---- selection (output_head_sampler.rs:94-212) --------------------------- */
int yo_validate_logits(const float* logits, uint64_t V);
int yo_greedy(const float* logits, uint64_t V, uint32_t* out);
int yo_top_tokens(const float* logits, uint64_t V, uint64_t count, uint32_t* out);
int yo_sample(const float* logits, uint64_t V, uint64_t position, const yo_params* p,
              uint32_t* out, yo_diag* diag);
/* Many positions over one logits row (one sort, one draw per position). */
int yo_sample_positions(const float* logits, uint64_t V, const uint64_t* positions,
                        uint64_t n, const yo_params* p, uint32_t* out);

/* ---- loss / logprobs (output_head_sampler.rs:230-250) -------------------- */
int yo_nll(const float* logits, uint64_t V, uint32_t target, double* out);
/* Serial ascending-id binary64 mass sum_v exp_d(l_v - max) and the max. */
int yo_mass(const float* logits, uint64_t V, double* mass, float* maximum);
/* EXTENSION: ids of the n highest raw logits (top_tokens order) and their
 * logprobs -nll(id) = (l - max) - log_d(mass). */
int yo_top_logprobs(const float* logits, uint64_t V, uint64_t n, uint32_t* ids,
                    double* logprobs);

/* ---- EXTENSION: bf16 logits and penalties -------------------------------- */
/* Exact widening, crates/yskn-format/src/floats.rs:55-57. */
void yo_bf16_to_f32(const uint16_t* in, float* out, uint64_t n);
/* Repetition/presence/frequency penalties over a token history, in place:
 * for every token with count c > 0 in history:
 *   if rep != 1: l = l > 0 ? l / rep : l * rep     (binary32, RN)
 *   l = l - freq * (float)c                          (binary32 mul, then sub)
 *   l = l - pres                                      (binary32 sub)            */
int yo_apply_penalties(float* logits, uint64_t V, const uint32_t* history, uint64_t len,
                       float repetition, float presence, float frequency);

/* ---- speculative acceptance (speculation.rs:483-523) --------------------- */
/* rows: M logits rows of length V, stride ld. guesses: M-1 draft tokens.
 * Row j is sampled at prediction position base_position + j + 1.
 * Outputs: selected[j] for the rows that the reference samples (it stops at the
 * first mismatch or EOS); *emitted = number of tokens pushed; *accepted = number
 * of guesses that matched among emitted rows; *stop_eos = 1 if an EOS stopped it.
 * greedy != 0 uses Greedy instead of the sampler. */
/* A prediction position past 2^64 - 1 fails with YO_EINVAL when the loop
 * reaches its row (speculation.rs:489-497); rows after the first mismatch are
 * never sampled, so their logits are never validated (:520-522). */
int yo_verify(const float* rows, uint64_t M, uint64_t V, uint64_t ld, const uint32_t* guesses,
              uint64_t base_position, const yo_params* p, int greedy, const uint32_t* eos_ids,
              uint64_t n_eos, uint32_t* selected, uint64_t* emitted, uint64_t* accepted,
              int* stop_eos);

/* ---- draft coupling (draft_head.rs:325-379) ------------------------------ */
/* Sampled choice among 16 draft candidates with Gumbel coupling. */
int yo_draft_choose(const float* scores, const uint32_t* tokens, uint64_t seed,
                    uint32_t temperature_thousandths, uint64_t position, uint32_t* out);

/* Intermediates of one draft choice, for pinning the arithmetic. */
typedef struct yo_draft_diag {
  double temperature; /* 0.001 * thousandths (binary64 multiply) */
  double z[16];       /* (score_i - score_top) / temperature, input order */
  double w[16];       /* exp_d(z_i), input order */
  double total;       /* serial sum of w in (score desc, token asc) order */
  int order[16];      /* input indices in (score desc, token asc) order */
  int member[16];     /* 1 if candidate i entered the Gumbel argmax */
} yo_draft_diag;
/* greedy != 0: DraftChoice::Greedy (first highest score in input order);
 * otherwise DraftChoice::Sampled { seed, temperature_thousandths }. diag may be
 * NULL (it is filled only for a sampled choice). */
int yo_draft_choose_ex(const float* scores, const uint32_t* tokens, int greedy, uint64_t seed,
                       uint32_t temperature_thousandths, uint64_t position, uint32_t* out,
                       yo_draft_diag* diag);

/* ---- draft shortlist and top 16 (draft_head.rs:219-300) ------------------ */
/* Two-stage histogram cutoff over order-preserving keys (1,024 bins of
 * key >> 22, then 2,048 bins of (key >> 11) & 2047 inside the cutoff bin);
 * ids above the cutoff prefix in ascending id order, then cutoff-prefix ids in
 * ascending id order until `count` (16..2048, multiple of 8, <= V). */
int yo_shortlist(const float* scores, uint64_t V, uint64_t count, uint32_t* out);
/* The 16 best of n >= 16 distinct (token, score) candidates in
 * (score desc, token asc) order. */
int yo_top16(const uint32_t* tokens, const float* scores, uint64_t n, uint32_t* out_tokens,
             float* out_scores);

/* ---- head epilogue (spec 06 section 2; compressed_linear.rs:311-346;
 *      residual_norm_mlp.rs:37-46; portable_math.rs:61-111) ---------------- */
/* Correctly rounded binary32 square root (portable_math.rs:61-106). */
float yo_sqrt_rn(float value);
/* 1 / sqrt_rn(value), the division rounded separately (portable_math.rs:108-111). */
float yo_rsqrt(float value);
/* inverse_rms = rsqrt(fold_add32(block_sums[0..n_blocks]) / width + epsilon),
 * the fold starting from +0 (residual_norm_mlp.rs:37-46). Returns YO_ENONFINITE
 * if the sum, the argument or the result is not finite. */
int yo_inverse_rms(const float* block_sums, uint64_t n_blocks, float width, float epsilon,
                   float* out);
/* logit[v] = ((float)acc[v] * unit_scale) * inverse_rms * tau[v], each product
 * a separately rounded binary32 multiply, one RN int64 -> binary32 conversion
 * (compressed_linear.rs:329-340). YO_ENONFINITE if any logit is not finite. */
int yo_head_logits(const int64_t* acc, const float* tau, uint64_t V, float unit_scale,
                   float inverse_rms, float* out);

#ifdef __cplusplus
}
#endif

#endif /* YSKN_ORACLE_H */
