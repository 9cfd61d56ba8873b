// smp_internal.hpp -- structures shared by the sampler's kernels and its
// host-side C ABI. Nothing here crosses the public boundary.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace yskn {

// Geometry. One block of 8 wave64s per row; each wave streams the row's
// 2,048-logit chunks w, w + 8, w + 16, ... (32 values per lane, coalesced
// 16-byte loads, two chunks in flight).
constexpr int NT = 512;            // threads per row block (8 wave64s)
constexpr int NW = NT / 64;        // waves per row block
constexpr int EPT = 32;            // elements per lane per chunk
constexpr int WSEG = 64 * EPT;     // elements per chunk
constexpr int CAP = 4096;          // candidates a row block sorts in LDS
constexpr int BUFCAP = 8192;       // candidates a row block's append buffer holds
constexpr int DLANES = 16;         // lanes with survivors above which a chunk is deferred
constexpr int DEFCAP = 512;        // deferred chunks a row block records
constexpr int KBMAX = 64;          // largest "small" top-k / list length
// Segments: a row split over several blocks exports, per segment, every
// candidate at or above the segment's own certified threshold (at most
// EXP_CAP of them; more send the row to the dense path) for the row's last
// block to finish. SEG_MAX * EXP_CAP fits the append buffer.
constexpr int SEG_MAX = 32;
constexpr int EXP_CAP = 256;
constexpr int HCAP = 16384;        // history tokens per row for the penalties
constexpr int64_t VMAX = 4194304;  // largest vocabulary

// Binary64 log-domain cut for the serial-sum argument: a weight exp_d(z)
// with z < -37.5 is below 2^-53 and cannot change a running binary64 sum
// that is already >= 1.
constexpr double ZCUT = -37.5;
// Terms exp(l - m) with l < m - ZMASS are left out of the logprob mass: at
// most V * e^-40 < 7e-11 relative for V <= 4,194,304.
constexpr float ZMASS = 40.0f;

// Wave flags.
constexpr uint32_t F_NONFINITE = 1u;
constexpr uint32_t F_INVALID = 4u;

// Status codes (public values of include/yskn_smp.h).
constexpr int32_t ST_OK = 0;
constexpr int32_t ST_EINVAL = -1;
constexpr int32_t ST_ENONFINITE = -2;

// Sampling parameters of one row, as the device reads them.
struct DevParams {
  double temperature;  // temperature_milli / 1000.0
  double top_p;        // top_p_milli / 1000.0
  double min_p;        // min_p_milli / 1000.0
  uint64_t seed;
  uint32_t top_k;      // 0 = disabled
  int32_t version;     // 2 | 3
  int32_t greedy;      // temperature_milli == 0
  int32_t penalize;    // any penalty active
  float rep, pres, freq;
  // The temperature is so small that (l - M) / T can overflow binary64 for
  // some finite binary32 logits: the row takes the exact dense path, which
  // checks the weakest candidate's z like the reference does.
  int32_t zcheck;
};

// What a segment hands to the block that finishes its row.
struct SegMeta {
  uint32_t count;     // candidates exported (> EXP_CAP: overflow, none kept)
  uint32_t flags;     // F_* seen in the segment
  uint32_t mkey;      // the segment's largest key (0: none finite)
  uint32_t theta;     // the segment's certified KB-th key: no larger than the row's
  double mass;        // sum of exp(l - mref) over the segment's mass terms
  float mref;         // reference point of that mass (-inf: no terms)
  uint32_t part;      // the segment's share of the certified tail's first pass is in its slot
};

// Counters for profiling the path (cumulative since create).
enum StatIndex {
  STAT_ROWS = 0,      // rows finished
  STAT_DENSE_ROWS,    // rows served by the exact large-candidate path
  STAT_CERT_ROWS,     // of those, rows whose cut was certified without a sort
  STAT_CANDIDATES,    // candidates sorted by the row blocks
  STAT_COUNT
};

enum Mode { MODE_SAMPLE = 0, MODE_VERIFY = 1 };

// Where a row's prediction position comes from.
enum PosMode {
  POS_ARRAY = 0,  // positions[row * n_draws + d]
  POS_BASE = 1,   // *base_position + depth + 1, depth = row_depth ? row_depth[row0 + row] : row0 + row
};

// Words of the verify result (the public yskn_smp_verify_result).
enum VerifyWord { VR_ACCEPTED = 0, VR_EMITTED, VR_TOKEN, VR_STOP_EOS, VR_STATUS, VR_WORDS };

struct SmpArgs {
  const void* logits;
  int64_t ld;  // elements between rows
  int32_t V;
  int32_t rows;
  int32_t mode;
  const DevParams* prm;
  int32_t prm_shared;
  int32_t n_draws;
  int32_t nseg;                  // segments (blocks) per row, 1..SEG_MAX
  uint64_t* exp_cand;            // [rows][nseg][EXP_CAP] exported candidates
  SegMeta* exp_meta;             // [rows][nseg]
  uint32_t* segcnt;              // [rows] arrivals of the row's segments (left at 0)
  // Head accumulators as the input (element type 2; spec 06 section 2): the
  // logits are ((float)acc * unit_scale) * inverse_rms * tau, formed while
  // streaming. `logits` then points at the int64 accumulators, `ld` is their
  // row stride in elements.
  const float* head_tau;         // [V]
  const float* head_us;          // [rows] common XSUM scale
  const float* head_sums;        // [rows][head_nblk] stored block sums of squares
  int32_t head_nblk;
  float head_width, head_eps;
  float* head_out;               // optional [rows][head_out_ld] logits written out
  int64_t head_out_ld;
  int32_t head_clear;            // zero the accumulators once read (needs head_out)
  int32_t pos_mode;              // PosMode
  const uint64_t* positions;     // [rows * n_draws] (POS_ARRAY)
  const uint64_t* base_position; // POS_BASE: row r at *base + depth(r) + 1
  const uint8_t* row_depth;      // POS_BASE: optional depth table, indexed row0 + r
  int32_t row0;
  uint64_t* adv_pos;             // optional: advanced by the tokens emitted
  uint32_t* adv_tok;             // optional: set to the last emitted token
  uint32_t* out_ids;             // [rows * n_draws] or NULL
  uint32_t* argmax;
  uint32_t* top8_ids;
  float* top8_vals;
  uint32_t* top20_ids;
  float* top20_vals;
  int32_t topn;                  // generic top list (top_tokens API)
  uint32_t* topn_ids;
  float* topn_vals;
  int32_t n_lp;
  uint32_t* lp_ids;
  double* lp_vals;
  const uint32_t* nll_targets;
  double* nll_out;
  int32_t want_mass;
  int32_t* status;       // handle's [rows]
  int32_t* row_status;   // caller's [rows] or NULL
  // penalties
  const uint2* pen_words;      // [rows][pw_ld] {membership bits, distinct ids below}
  int64_t pw_ld;
  const uint32_t* pen_cnt;     // [rows][HCAP] count of each distinct id, in id order
  const int32_t* pen_len;      // [rows] distinct ids, -1 = invalid history
  // workspace
  uint64_t* dense_a;    // [rows][dense_ld]
  uint64_t* dense_b;
  double* dense_w;
  int64_t dense_ld;
  int32_t force_dense;
  int32_t vec;          // rows are 16-byte aligned with ld a multiple of 16 bytes
  unsigned long long* stats;
  // verify
  const uint32_t* drafts;
  const uint32_t* eos;
  int32_t n_eos;
  uint32_t* vresult;  // VR_WORDS words
  uint32_t* vcount;
};

struct PenArgs {
  const uint32_t* history;
  const int32_t* history_len;
  int64_t history_ld;
  int32_t V;
  int32_t rows;
  uint2* words;
  int64_t pw_ld;
  uint32_t* cnt;
  int32_t* len;
  const DevParams* prm;
  int32_t prm_shared;
};

// Draft-side selection (smp_draft.hip).
constexpr int TOP16_NMAX = 4096;  // candidates per row of the top-16 kernel

struct DraftShortlistArgs {
  const float* scores;  // [rows][ld]
  int64_t ld;
  int32_t V;
  int32_t rows;
  int32_t count;
  uint32_t* out;  // [rows][out_ld]
  int64_t out_ld;
  int32_t* status;      // [rows], always written
  int32_t* row_status;  // [rows] or NULL
};

struct DraftTop16Args {
  const uint32_t* tokens;  // [rows][ld]
  const float* scores;     // [rows][ld]
  int64_t ld;
  int32_t n;
  int32_t rows;
  uint32_t* out_tokens;  // [rows][16]
  float* out_scores;     // [rows][16] or NULL
  int32_t* status;
  int32_t* row_status;
};

struct DraftChooseArgs {
  const float* scores;     // [rows][ld], 16 used
  const uint32_t* tokens;  // [rows][ld], 16 used
  int64_t ld;
  int32_t rows;
  int32_t sampled;
  uint64_t seed;
  double temperature;        // 0.001 * thousandths, binary64
  const uint64_t* positions;  // [rows] (sampled only)
  uint32_t* out;             // [rows]
  int32_t* alt;              // [rows] or NULL
  float* margin;             // [rows] or NULL
  int32_t* alt3;             // [rows] or NULL
  int32_t* status;
  int32_t* row_status;
};

// Host-side launchers (smp_kernels.hip, smp_draft.hip).
hipError_t launch_sample(const SmpArgs& a, int dtype, bool vec, bool pen, hipStream_t st);
hipError_t launch_penalty_prep(const PenArgs& a, hipStream_t st);
// Test hook: the exact serial prefix sums of c binary64 weights (w[0] = 1 >=
// w[j] >= 0) by the block-parallel scan the tail uses; one block.
hipError_t launch_prefix_test(const double* w, double* S, int64_t c, hipStream_t st);
hipError_t launch_draft_shortlist(const DraftShortlistArgs& a, hipStream_t st);
hipError_t launch_draft_top16(const DraftTop16Args& a, hipStream_t st);
hipError_t launch_draft_choose(const DraftChooseArgs& a, hipStream_t st);

}  // namespace yskn
