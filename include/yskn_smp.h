/*
 * yskn_smp.h -- C ABI of the MI355X (gfx950) sampling library.
 *
 * The per-step logits -> token path of YASAKANI as a thin C ABI in the shape
 * of the reference's include/yskn_abi.h: an opaque handle, int status
 * (0 = success, negative = failure), a thread-local last-error string,
 * caller-owned device buffers and an explicit HIP stream. No C++ or torch
 * types cross this boundary.
 *
 * Semantics follow the reference's scalar specification
 * (crates/yskn-ref/src/output_head_sampler.rs) bit for bit: selected token ids,
 * top-k index sets, argmax and accepted-draft counts are identical to it on the
 * same logits, parameters and prediction positions.
 *
 * Threading: a handle is used by one host thread at a time (the reference's
 * "one engine per thread", crates/yskn-cli/src/lib.rs:1). Calls on one handle
 * must be issued to one stream or otherwise ordered: the handle's workspace is
 * shared by its calls.
 */
#ifndef YSKN_SMP_H
#define YSKN_SMP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes --------------------------------------------------------
 * The reference returns Result<_, Error> (crates/yskn-ref/src/lib.rs:37-45)
 * and, at its C ABI, 0 / -1 plus yskn_last_error() (src/c_api.cpp:11-14). */
#define YSKN_SMP_OK 0
#define YSKN_SMP_EINVAL (-1)     /* Error::InvalidInput */
#define YSKN_SMP_ENONFINITE (-2) /* Error::NonFinite("logits") */
#define YSKN_SMP_ERANGE (-3)     /* vocabulary (max 4,194,304) or rows beyond the handle's limits */
#define YSKN_SMP_EDEVICE (-4)    /* HIP runtime failure */

/* ---- handle flags ------------------------------------------------------- */
/* Lift the reference's 1..=20 top_k cap (output_head_sampler.rs:68-72) to
 * 1..=V, with top_k = 0 meaning "disabled" (k = V). Without this flag top_k
 * outside 1..=min(20, V) is rejected exactly like the reference. */
#define YSKN_SMP_FLAG_EXTENDED_TOP_K 0x1u
/* Test hook: route every row through the exact large-candidate ("dense")
 * path even when the compact path would serve it. Results are identical. */
#define YSKN_SMP_FLAG_FORCE_DENSE 0x2u

/* ---- logits element type ------------------------------------------------ */
#define YSKN_SMP_F32 0
#define YSKN_SMP_BF16 1 /* widened exactly: bits << 16 (crates/yskn-format/src/floats.rs:55-57) */

/* ---- sampler versions (output_head_sampler.rs:14-18; spec 06 sections 6-7) */
#define YSKN_SMP_VERSION_INVERSE_CDF 2
#define YSKN_SMP_VERSION_GUMBEL 3

typedef struct yskn_smp* yskn_smp_handle;

/* Per-row sampling parameters. Replaces the reference's Q35SmpParams
 * (src/q35.hpp:114-116) set through yskn_set_opt keys 10/11/12/13/16/29
 * (src/engine35.cpp:946-959) and yskn-ref SamplingParameters
 * (output_head_sampler.rs:21-41). Stored values are binary64
 * thousandths / 1000.0 (division, output_head_sampler.rs:46-49). */
typedef struct yskn_smp_params {
  uint32_t temperature_milli; /* 0 = greedy (real_engine.rs:241-243); else T = value / 1000.0 */
  uint32_t top_p_milli;       /* 1..1000 */
  uint32_t top_k;             /* 1..min(20, V); with EXTENDED_TOP_K: 0 (disabled) or 1..V */
  uint32_t min_p_milli;       /* 0..1000 */
  uint64_t seed;              /* full 64-bit seed (the C setter supplies uint64(uint32(v))) */
  int32_t version;            /* YSKN_SMP_VERSION_GUMBEL (default) or _INVERSE_CDF */
  /* EXTENSION (no reference counterpart): penalties over the token history
   * passed to yskn_smp_sample. For every token with count c > 0 in the row's
   * history, in binary32 round-to-nearest:
   *   if repetition != 1: l = l > 0 ? l / repetition : l * repetition
   *   l = l - frequency * (float)c;  l = l - presence
   * applied to the (widened) logit before every other stage. */
  float repetition_penalty; /* 1 = off; must be > 0 */
  float presence_penalty;   /* 0 = off */
  float frequency_penalty;  /* 0 = off */
} yskn_smp_params;

/* The same parameters with binary64 fields, exactly as the Rust
 * SamplingParameters holds them (output_head_sampler.rs:21-28), for callers
 * whose values are not thousandths. greedy != 0 is Sampler::Greedy
 * (output_head_sampler.rs:77-82); its other fields are then ignored. */
typedef struct yskn_smp_params_f64 {
  double temperature; /* finite, > 0 */
  double top_p;       /* (0, 1] */
  double min_p;       /* [0, 1] */
  uint32_t top_k;     /* as yskn_smp_params.top_k */
  int32_t greedy;
  uint64_t seed;
  int32_t version;
  float repetition_penalty; /* EXTENSION, as yskn_smp_params */
  float presence_penalty;
  float frequency_penalty;
} yskn_smp_params_f64;

/* Optional outputs and inputs of yskn_smp_sample. Every pointer is a device
 * pointer or NULL. Replaces the optional outputs of Q35SmpArgs
 * (top_val/top_idx [rows*8], topk_val/topk_idx [rows*20]; src/q35.hpp:117-120)
 * and the argmax of ArgmaxArgs (src/args.hpp:24-30). */
typedef struct yskn_smp_aux {
  uint32_t* argmax;      /* [rows] greedy id: larger logit, then smaller id */
  uint32_t* top8_ids;    /* [rows*8] highest raw logits, (value desc, id asc) */
  float* top8_vals;      /* [rows*8] */
  uint32_t* top20_ids;   /* [rows*20] */
  float* top20_vals;     /* [rows*20] */
  /* EXTENSION: the n_logprobs highest raw logits with their logprobs
   * l - max - log(sum_v exp(l_v - max)) in binary64 (the negated
   * negative_log_likelihood of output_head_sampler.rs:230-250). */
  int32_t n_logprobs;    /* 0..vocab (above 64: the row takes the exact dense path) */
  uint32_t* logprob_ids; /* [rows*n_logprobs] */
  double* logprobs;      /* [rows*n_logprobs] */
  int32_t* row_status;   /* [rows] per-row YSKN_SMP_* status */
  /* EXTENSION: token history for the penalties: row r uses
   * history[r*history_ld .. + history_len[r]]. history_ld = 0 shares one
   * history among all rows; history_ld < 0 is rejected. A row whose
   * history_len is negative, above 16,384, above a positive history_ld, or
   * that holds an id >= vocab fails with YSKN_SMP_EINVAL. The caller must
   * size the buffer for the rows' lengths. */
  const uint32_t* history;
  const int32_t* history_len; /* [rows] */
  int64_t history_ld;
} yskn_smp_aux;

/* Device-side position/token advance: the reference sampler's adv_pos /
 * adv_tok (src/q35.hpp:118; src/q35_sample.cu:206) and Engine35::commit
 * (src/engine35.cpp:1319-1329) without a host round trip. Both pointers are
 * device pointers; `position` may be the same counter the call reads its
 * base position from (it is read before it is advanced). */
typedef struct yskn_smp_advance {
  uint64_t* position; /* advanced by the number of tokens emitted */
  uint32_t* token;    /* set to the last emitted token */
} yskn_smp_advance;

/* Result of a speculative verification; mirrors the accept loop of
 * crates/yskn-ref/src/speculation.rs:483-523 and src/specx.cpp:376-440. */
typedef struct yskn_smp_verify_result {
  uint32_t accepted; /* drafts equal to the selected token among emitted rows */
  uint32_t emitted;  /* tokens produced: accepted drafts + correction or bonus */
  uint32_t token;    /* last emitted token: the correction, or the bonus token */
  int32_t stop_eos;  /* 1 if an EOS id ended the pass */
  /* YSKN_SMP_OK, or the status of the first row the accept walk reached that
   * failed (then accepted = emitted = 0 and token = 0xFFFFFFFF) */
  int32_t status;
} yskn_smp_verify_result;

/* Thread-local description of the last failure on this thread
 * (src/c_api.cpp:11-14 yskn_last_error). Never NULL. */
const char* yskn_smp_last_error(void);

/* Create a sampler for up to max_rows rows of up to max_vocab logits. The
 * handle owns only scratch memory (candidates, counters, sort buffers),
 * allocated once here like the engine's buffers (src/engine35.cpp:336-347).
 * Initial parameters are the reference defaults (output_head_sampler.rs:30-41:
 * T 1.0, top-p 0.95, top-k 20, min-p 0, seed 0, Gumbel). */
int yskn_smp_create(int32_t max_rows, int32_t max_vocab, uint32_t flags, yskn_smp_handle* out);
void yskn_smp_destroy(yskn_smp_handle h);

/* Set sampling parameters: n = 1 applies one set to every row (the
 * reference's single Q35SmpParams per launch); n = rows gives each row its own
 * set (EXTENSION). Validates like SamplingParameters::validate
 * (output_head_sampler.rs:56-75) against max_vocab; the top_k <= V check is
 * repeated at every call against the call's V. Synchronous, like
 * yskn_set_opt's cudaMemcpy (src/engine35.cpp:946-959). */
int yskn_smp_set_params(yskn_smp_handle h, const yskn_smp_params* params, int32_t n);

/* yskn_smp_set_params with binary64 values: the Rust SamplingParameters
 * fields as they are (output_head_sampler.rs:21-28), validated by the rules
 * of SamplingParameters::validate (output_head_sampler.rs:56-75). */
int yskn_smp_set_params_f64(yskn_smp_handle h, const yskn_smp_params_f64* params, int32_t n);

/* Sample one token per (row, draw). Replaces launch_q35_smp
 * (src/q35.hpp:113-122; src/q35_sample.cu:210-214) and yskn-ref
 * Sampler::sample (output_head_sampler.rs:86-92). Rows whose temperature is 0
 * are greedy.
 *   logits     device [rows x ld] elements of dtype (YSKN_SMP_F32 | _BF16)
 *   positions  device [rows x n_draws] absolute prediction positions
 *              (input position + 1; speculation.rs:490-492, spec 06 section 5)
 *   out_ids    device [rows x n_draws]
 *   aux        optional outputs/inputs (may be NULL)
 * n_draws > 1 draws several positions from the same row (one candidate
 * extraction). Asynchronous on `stream`; per-row errors land in
 * aux->row_status and in the handle (see yskn_smp_sync). */
int yskn_smp_sample(yskn_smp_handle h, const void* logits, int32_t dtype, int32_t rows,
                    int32_t vocab, int64_t ld, const uint64_t* positions, int32_t n_draws,
                    uint32_t* out_ids, const yskn_smp_aux* aux, void* stream);

/* Sample one token per row at device-resident positions: the position form
 * and advance of launch_q35_smp (src/q35_sample.cu:180-181,206;
 * Q35SmpArgs d_pos / wk / row0 / adv_pos / adv_tok, src/q35.hpp:117-118).
 * Row r is sampled at prediction position
 *     *base_position + depth + 1,  depth = row_depth ? row_depth[row0 + r] : row0 + r
 * with checked unsigned 64-bit arithmetic: a position past 2^64 - 1 fails the
 * row with YSKN_SMP_EINVAL (speculation.rs:489-497). One draw per row.
 *   base_position  device [1]
 *   row_depth      device [row0 + rows] depth table (may be NULL)
 *   advance        optional (may be NULL): only for rows = 1; after the row is
 *                  sampled, *advance->position += 1 and *advance->token = id
 *                  (a failed row advances nothing).
 * Asynchronous on `stream`, like yskn_smp_sample. */
int yskn_smp_sample_at(yskn_smp_handle h, const void* logits, int32_t dtype, int32_t rows,
                       int32_t vocab, int64_t ld, const uint64_t* base_position,
                       const uint8_t* row_depth, int32_t row0, uint32_t* out_ids,
                       const yskn_smp_aux* aux, const yskn_smp_advance* advance, void* stream);

/* The output head's epilogue fused into the sampler: instead of binary32
 * logits the call reads the head's int64 accumulators and forms every logit
 * while streaming, in the reference's exact order
 *     inverse_rms = 1 / sqrt_rn(fold_add32(block_sums[row]) / width + epsilon)
 *     logit[v]    = (((float)acc[row][v] * unit_scale[row]) * inverse_rms) * tau[v]
 * (one round-to-nearest int64 -> binary32 conversion, each product separately
 * rounded; spec 06 section 2, docs/spec/06_OUTPUT_HEAD_SAMPLER.md:31-55;
 * src/misc_kernels.cu:57-73 with src/a8_prologue.cuh:10-15 argmax_stage1 /
 * xsum_combine; crates/yskn-ref/src/compressed_linear.rs:329-340 and
 * residual_norm_mlp.rs:37-46 with the portable rsqrt, portable_math.rs:61-111).
 * A non-finite sum, argument, inverse RMS or logit fails the row with
 * YSKN_SMP_ENONFINITE, as require_finite does there. */
typedef struct yskn_smp_head {
  const int64_t* acc;       /* device [rows x acc_ld] int64 accumulators */
  int64_t acc_ld;           /* >= vocab */
  const float* unit_scale;  /* device [rows] the common XSUM scale (row quantum) */
  const float* block_sums;  /* device [rows x n_blocks] stored block sums of squares */
  int32_t n_blocks;         /* 1..64 (10 for a width of 5,120) */
  float width;              /* finite, > 0: the hidden width (5,120) */
  float epsilon;            /* finite, > 0 */
  const float* tau;         /* device [vocab] per-token weight scale */
  float* logits_out;        /* optional device [rows x logits_ld]: the logits, written once */
  int64_t logits_ld;        /* >= vocab when logits_out is set */
  int32_t clear_acc;        /* 1: zero each accumulator once read, like xsum_combine
                               (src/a8_prologue.cuh:10-12); needs logits_out */
} yskn_smp_head;

/* yskn_smp_sample on head accumulators (see yskn_smp_head): the same
 * positions, draws, outputs and errors, with the logits formed in the
 * sampler's own sweep instead of being written and read again by a separate
 * epilogue launch (the reference's argmax_stage1 -> smp2_kernel pair,
 * src/engine35.cpp:810-821). */
int yskn_smp_sample_head(yskn_smp_handle h, const yskn_smp_head* head, int32_t rows, int32_t vocab,
                         const uint64_t* positions, int32_t n_draws, uint32_t* out_ids,
                         const yskn_smp_aux* aux, void* stream);

/* Greedy argmax per row: greedy() (output_head_sampler.rs:103-113),
 * launch_argmax (src/args.hpp:24-30; src/misc_kernels.cu:57-96).
 * Like the two entry points below, a pure function of the logits: the
 * handle's sampling parameters (penalties included) are not used. */
int yskn_smp_argmax(yskn_smp_handle h, const void* logits, int32_t dtype, int32_t rows,
                    int32_t vocab, int64_t ld, uint32_t* out_ids, void* stream);

/* The `count` (1..vocab) highest raw logits per row in (value desc, id asc)
 * order: top_tokens() (output_head_sampler.rs:115-134), launch_topk8
 * (src/args.hpp:43-45; src/misc_kernels.cu:100-147). Counts above 64 take
 * the exact dense path (the count-th key by radix selection over the row,
 * then a stable sort of the elements at or above it in the handle's scratch):
 * correct for any count, slower. */
int yskn_smp_top_tokens(yskn_smp_handle h, const void* logits, int32_t dtype, int32_t rows,
                        int32_t vocab, int64_t ld, int32_t count, uint32_t* out_ids,
                        float* out_vals, void* stream);

/* Negative log-likelihood of targets[row]: negative_log_likelihood()
 * (output_head_sampler.rs:230-250), launch_nll (src/misc_kernels.cu:150-166).
 * Binary64 output. */
int yskn_smp_nll(yskn_smp_handle h, const void* logits, int32_t dtype, int32_t rows,
                 int32_t vocab, int64_t ld, const uint32_t* targets, double* out_nll,
                 void* stream);

/* One-launch speculative verification of M rows: row j is sampled at
 * prediction position *base_position + j + 1 (checked like the reference's
 * accept loop) with the handle's parameters (one set, or one per row),
 * drafts[j] (j < M-1) is accepted while it equals the selected token, and the
 * first mismatch's selection (or the bonus when all match) ends the pass; an
 * EOS id among the emitted tokens stops it. A failed row (non-finite logits,
 * position overflow, invalid history) fails the pass only when the walk
 * reaches it. Replaces the per-row Selector loop of speculation.rs:483-523,
 * the host accept loop of src/specx.cpp:376-440 and, with `commit`, the
 * commit of Engine35::commit (src/engine35.cpp:1319-1329).
 *   target_logits device [M x ld]; drafts device [M-1]; base_position device [1]
 *   eos_ids device [n_eos] (may be NULL when n_eos = 0)
 *   out_ids device [M] selected token per row; result device [1]
 *   aux     optional per-row outputs of yskn_smp_sample (argmax, top-8,
 *           top-20, logprobs, row status: yskn_verify's out_argmax / top_ids /
 *           top_vals, include/yskn_abi.h:39,55) and the penalty history
 *   commit  optional: when the pass succeeds, *commit->position += emitted
 *           and *commit->token = the last emitted token */
int yskn_smp_verify(yskn_smp_handle h, const void* target_logits, int32_t dtype, int32_t M,
                    int32_t vocab, int64_t ld, const uint32_t* drafts,
                    const uint64_t* base_position, const uint32_t* eos_ids, int32_t n_eos,
                    uint32_t* out_ids, yskn_smp_verify_result* result, const yskn_smp_aux* aux,
                    const yskn_smp_advance* commit, void* stream);

/* ---- Draft-side selection ------------------------------------------------
 * The drafter's three selection steps, each a pure function of its inputs
 * (the handle's sampling parameters are not used). rows <= the handle's
 * max_rows; every row gets a status (yskn_smp_sync reports the first
 * failure; row_status, when not NULL, receives all of them). */

/* The drafter's shortlist of `count` token ids from its approximate scores:
 * shortlist() (crates/yskn-ref/src/draft_head.rs:219-282). Two histogram
 * passes (1,024 bins of the order-preserving key's top 10 bits, then 2,048
 * bins of the next 11 inside the cut-off bin) fix a 21-bit prefix; every id
 * above it is kept, in ascending id order, then the lowest ids of the tie
 * bucket, ascending, up to `count`. Replaces the SHEAD histogram/collect
 * kernels (src/q35_bdraft.cu:861-898), whose atomic tie-bucket order this
 * removes (the result is a function of the scores alone).
 *   scores device [rows x ld] f32; count in 16..=2048, a multiple of 8,
 *   <= vocab; out_ids device [rows x out_ld] (out_ld >= count).
 *   Row status YSKN_SMP_ENONFINITE for a non-finite score (its out_ids are
 *   all 0xffffffff). */
int yskn_smp_draft_shortlist(yskn_smp_handle h, const float* scores, int32_t rows, int32_t vocab,
                             int64_t ld, int32_t count, uint32_t* out_ids, int64_t out_ld,
                             int32_t* row_status, void* stream);

/* The 16 best of n rescored candidates under (score desc, token asc):
 * top16() (draft_head.rs:284-305); bdr_sk_top16_kernel
 * (src/q35_bdraft.cu:928). n in 16..=4096. Row status YSKN_SMP_EINVAL
 * for a non-finite score or a repeated token (outputs 0xffffffff / -inf).
 *   tokens, scores device [rows x ld]; out_tokens device [rows x 16];
 *   out_scores device [rows x 16] or NULL (the candidates' own scores). */
int yskn_smp_draft_top16(yskn_smp_handle h, const uint32_t* tokens, const float* scores,
                         int32_t rows, int32_t n, int64_t ld, uint32_t* out_tokens,
                         float* out_scores, int32_t* row_status, void* stream);

/* DraftChoice (draft_head.rs:307-323). */
typedef struct yskn_smp_draft_choice {
  int32_t sampled;                  /* 0: DraftChoice::Greedy; 1: Sampled */
  uint32_t temperature_thousandths; /* Sampled: > 0 (the reference default is 850) */
  uint64_t seed;                    /* Sampled */
} yskn_smp_draft_choice;

/* The draft token among 16 candidates per row: choose()
 * (draft_head.rs:325-379). Greedy: the first strictly larger score in input
 * order. Sampled: candidates ordered by (score desc, token asc), binary64
 * temperature 0.001 * thousandths, weights exp_d((s - s_top) / T), members
 * while the serial prefix before them is below 0.95 * total, then the
 * largest z + gumbel(seed, positions[row], token) among members, the
 * earliest winning ties. Replaces the coupling of bdr_select(3)_kernel
 * (src/q35_bdraft.cu:318-475) with the reference's portable exp_d.
 *   scores, tokens device [rows x ld] (16 used, ld >= 16)
 *   positions device [rows] prediction positions (Sampled; may be NULL for
 *   Greedy); out_tokens device [rows]
 *   alt, margin, alt3 device [rows] or NULL: the runner-up, the score gap
 *   to it and the third choice, as launch_bdr_select returns them
 *   (q35_bdraft.cu:437-450; -1 / 1e30 when absent).
 *   Row status YSKN_SMP_EINVAL for a non-finite score. */
int yskn_smp_draft_choose(yskn_smp_handle h, const float* scores, const uint32_t* tokens,
                          int32_t rows, int64_t ld, const yskn_smp_draft_choice* choice,
                          const uint64_t* positions, uint32_t* out_tokens, int32_t* alt,
                          float* margin, int32_t* alt3, int32_t* row_status, void* stream);

/* Synchronise `stream` and return the first per-row error of the handle's
 * last call (YSKN_SMP_OK if none), setting yskn_smp_last_error(). After a
 * verify it returns the pass's status (yskn_smp_verify_result.status). */
int yskn_smp_sync(yskn_smp_handle h, void* stream);

/* Host-slice convenience with the exact signature semantics of the Rust
 * trait Selector::select(&mut self, logits: &[f32], prediction_position: u64)
 * (crates/yskn-ref/src/speculation.rs:123-139): copies `vocab` host logits to
 * the device, samples with row-0 parameters, returns the token synchronously. */
int yskn_smp_select_host(yskn_smp_handle h, const float* host_logits, int32_t vocab,
                         uint64_t prediction_position, uint32_t* out_token);

/* Profiling counters of the handle, cumulative since create (no counterpart
 * in the reference, which has no sampler-level instrumentation): out[0] rows
 * finished, out[1] rows served by the exact large-candidate path, out[2]
 * those of them whose cut was certified without sorting the row, out[3]
 * candidates sorted by the row blocks. Synchronises the device.
 * Returns the number of counters written (<= n) or a negative status. */
int yskn_smp_get_stats(yskn_smp_handle h, uint64_t* out, int32_t n);

/* Validate parameters on the host without a device (the reference's
 * SamplingParameters::validate, output_head_sampler.rs:56-75). */
int yskn_smp_validate_params(const yskn_smp_params* params, int32_t vocab, uint32_t flags);

/* The same for binary64 parameters (SamplingParameters::validate on the
 * Rust fields as they are, NaN and infinities included). */
int yskn_smp_validate_params_f64(const yskn_smp_params_f64* params, int32_t vocab, uint32_t flags);

/* Device-math test hook, the counterpart of the reference's yskn_pm_test
 * (src/pm_test.cu:30-52): evaluates one device primitive of the sampler on n
 * inputs (host buffers in and out; the call synchronises).
 *   fn 10: exp_d   binary64 -> binary64   (portable_math.rs:224-283)
 *   fn 11: log_d   binary64 -> binary64   (portable_math.rs:297-364)
 *   fn 12: gumbel  (seed, position, token) u64 triples -> binary64
 *                  (output_head_sampler.rs:221-228)
 *   fn 13: version-2 uniform (seed, position) u64 pairs -> binary64 (:196-197)
 *   fn 14: mix64   u64 -> u64 (:214-219)
 *   fn 15: the certified dense tail's polynomial exp, binary64 -> binary64
 *          (no counterpart in the reference: bounded, not bit-exact)
 *   fn 16: the same tail's binary32 version-3 score from (z binary32 bits,
 *          position key mix64(mix64(seed) ^ position), token) u64 triples ->
 *          binary32 bits (no counterpart in the reference: bounded)
 *   fn 8:  serial binary64 prefix sums S_j = (..(w_0 + w_1) + ..) + w_j of n
 *          weights (w_0 = 1 >= w_j >= 0), as the tail computes them in
 *          parallel (output_head_sampler.rs:157-175)
 *   fn 6:  rsqrt   binary32 bits base + i -> binary32 bits (portable_math.rs:108-111)
 *   fn 7:  sqrt_rn binary32 bits base + i -> binary32 bits (portable_math.rs:61-106)
 * n in 1..2^28. Returns 0 or a negative status. */
int yskn_smp_pm_test(int32_t fn, uint64_t base, const void* host_in, void* host_out, int64_t n);

/* Library version string. */
const char* yskn_smp_version(void);

#ifdef __cplusplus
}
#endif

#endif /* YSKN_SMP_H */
