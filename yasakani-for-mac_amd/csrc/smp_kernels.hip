// smp_kernels.hip -- gfx950 kernels of the per-step sampling path.
//
// One launch per call (two with penalties):
//
//  smp_row    one block of 8 wave64s per row. The waves stream the row in
//             2,048-logit chunks (32 values per lane, coalesced 16-byte
//             loads, two chunks in flight) and keep only the elements that
//             can matter to the reference algorithm: (a) elements whose
//             binary64 weight exp_d((l - M)/T) can reach 2^-53 (smaller
//             weights are absorbed by the reference's serial binary64 sums,
//             whose running value is >= 1) and (b) a superset of the row's
//             top-KB by value. The row's running maximum and top-KB bound
//             live in LDS, so every wave filters with the row's bounds as they
//             stand; the kept elements go to an LDS candidate buffer, which
//             the block then sorts by (value desc, id asc) before running the
//             reference's serial binary64 truncation and draw
//             (output_head_sampler.rs:136-212). Rows with more candidates
//             than LDS holds take the exact "dense" path: radix select, stable
//             LSD radix sort in global scratch, same tail.
//  smp_penalty_prep (penalties only) turns each row's history into
//             membership words over the vocabulary and per-id counts.
//
// Ordering is (value desc, id asc) everywhere, as output_head_sampler.rs:
// 124-132; -0 and +0 compare equal (keys canonicalise -0 to +0) and ties go
// to the smaller id, never to atomic arrival order.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "smp_internal.hpp"
#include "smp_math.hpp"

namespace yskn {

constexpr int32_t YSKN_V3 = 3;

// Pointers typed with their address space (3: LDS, 1: global). Stores through
// them cannot be merged into one generic (flat) store when the two kinds sit
// in neighbouring branches; a flat access counts against both the vector
// memory and the LDS counters, so every wait after it becomes a full wait.
typedef __attribute__((address_space(3))) uint64_t lds_u64;
typedef __attribute__((address_space(1))) uint64_t global_u64;
typedef __attribute__((ext_vector_type(4))) uint32_t u32x4;
typedef __attribute__((address_space(3))) u32x4 lds_u4;

// ---------------------------------------------------------------------------
// keys and packing
// ---------------------------------------------------------------------------
// Order-preserving key of binary32 bits; -0 is mapped to +0 first. Real
// logits have keys >= 0x007fffff; key 0 marks padding.
__device__ __forceinline__ uint32_t f2key(uint32_t b) {
  b = (b == 0x80000000u) ? 0u : b;
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}
__device__ __forceinline__ float key2f(uint32_t k) {
  const uint32_t b = (k & 0x80000000u) ? (k & 0x7fffffffu) : ~k;
  return __uint_as_float(b);
}
// (key, id) packed so that a larger u64 is earlier in (value desc, id asc).
__device__ __forceinline__ uint64_t pack(uint32_t key, uint32_t id) {
  return ((uint64_t)key << 32) | (uint64_t)(~id);
}
__device__ __forceinline__ uint32_t pk_key(uint64_t p) { return (uint32_t)(p >> 32); }
__device__ __forceinline__ uint32_t pk_id(uint64_t p) { return ~(uint32_t)p; }

// Key of the smallest binary32 value L with L <= M + ZCUT * T, i.e. every
// element whose weight can reach 2^-53 has key >= the result.
__device__ __forceinline__ uint32_t relevance_key(float M, double T) {
  const double L = (double)M + ZCUT * T;
  if (!(L > -3.4028234663852886e38)) return 1u;
  const float Lf = __double2float_rd(L);
  const uint32_t k = f2key(__float_as_uint(Lf));
  return k < 1u ? 1u : k;
}

// The binary32 value t with {v : v >= t} == {v : f2key(v) >= theta} over
// finite values: key thresholds at or below the key of -FLT_MAX keep every
// finite value; 0xffffffff (a NaN pattern) keeps none.
__device__ __forceinline__ float key_threshold_float(uint32_t theta) {
  if (theta <= 0x00800000u) return -3.4028234663852886e38f;
  return key2f(theta);
}

// ---------------------------------------------------------------------------
// wave64 / block reductions
// ---------------------------------------------------------------------------
__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const uint64_t w = __shfl_xor(v, o);
    v = v > w ? v : w;
  }
  return v;
}
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const uint32_t w = __shfl_xor(v, o);
    v = v > w ? v : w;
  }
  return v;
}
__device__ __forceinline__ uint32_t wave_min_u32(uint32_t v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const uint32_t w = __shfl_xor(v, o);
    v = v < w ? v : w;
  }
  return v;
}
// Wave-wide maximum through DPP (VALU only, no LDS round trips): an
// inclusive max-scan inside each row of 16 lanes (row_shr 1, 2, 4, 8; lanes
// shifted in from outside the row read 0, the identity), then row_bcast:15
// and row_bcast:31 carry the rows' totals upward. Lane 63 ends with the
// maximum of all 64 lanes; it is returned (uniform) to every lane.
template <int CTRL, int ROWS>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, ROWS, 0xf, false);
}
__device__ __forceinline__ uint32_t wave_max_dpp(uint32_t v) {
  uint32_t t;
  t = dpp_u32<0x111, 0xf>(v); v = v > t ? v : t;  // row_shr:1
  t = dpp_u32<0x112, 0xf>(v); v = v > t ? v : t;  // row_shr:2
  t = dpp_u32<0x114, 0xf>(v); v = v > t ? v : t;  // row_shr:4
  t = dpp_u32<0x118, 0xf>(v); v = v > t ? v : t;  // row_shr:8
  t = dpp_u32<0x142, 0xa>(v); v = v > t ? v : t;  // row_bcast:15 into rows 1, 3
  t = dpp_u32<0x143, 0xc>(v); v = v > t ? v : t;  // row_bcast:31 into rows 2, 3
  return (uint32_t)__builtin_amdgcn_readlane((int)v, 63);
}
// Wave-wide minimum (the maximum of the complements).
__device__ __forceinline__ uint32_t wave_min_u32_dpp(uint32_t v) { return ~wave_max_dpp(~v); }
// Number of lanes below this one whose bit is set in the wave mask m.
__device__ __forceinline__ uint32_t lanes_below(uint64_t m) {
  return __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
}
__device__ __forceinline__ double wave_sum_f64(double v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  return v;
}
// A 64-bit value moved by one DPP pattern (both halves; lanes the pattern
// does not write read 0).
template <int CTRL, int ROWS>
__device__ __forceinline__ uint64_t dpp_u64(uint64_t v) {
  const uint32_t lo = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)v, CTRL, ROWS, 0xf, false);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)(v >> 32), CTRL, ROWS, 0xf, false);
  return ((uint64_t)hi << 32) | lo;
}
__device__ __forceinline__ uint64_t lane_u64(uint64_t v, int j) {
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)v, j);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(v >> 32), j);
  return ((uint64_t)hi << 32) | lo;
}
// Wave-wide binary64 sum through DPP (scan within rows of 16, then row
// broadcasts; no LDS round trips), returned to every lane. The adds are not
// in serial order: for the logprob mass only, never for a top-p total.
__device__ __forceinline__ double wave_sum_f64_dpp(double v) {
  auto add = [](double a, uint64_t b) { return a + __longlong_as_double((long long)b); };
  v = add(v, dpp_u64<0x111, 0xf>((uint64_t)__double_as_longlong(v)));  // row_shr:1
  v = add(v, dpp_u64<0x112, 0xf>((uint64_t)__double_as_longlong(v)));  // row_shr:2
  v = add(v, dpp_u64<0x114, 0xf>((uint64_t)__double_as_longlong(v)));  // row_shr:4
  v = add(v, dpp_u64<0x118, 0xf>((uint64_t)__double_as_longlong(v)));  // row_shr:8
  v = add(v, dpp_u64<0x142, 0xa>((uint64_t)__double_as_longlong(v)));  // row_bcast:15
  v = add(v, dpp_u64<0x143, 0xc>((uint64_t)__double_as_longlong(v)));  // row_bcast:31
  return __longlong_as_double((long long)lane_u64((uint64_t)__double_as_longlong(v), 63));
}
// Wave-wide maximum of 64-bit values through DPP, returned to every lane.
__device__ __forceinline__ uint64_t wave_max_u64_dpp(uint64_t v) {
  uint64_t t;
  t = dpp_u64<0x111, 0xf>(v);
  v = v > t ? v : t;
  t = dpp_u64<0x112, 0xf>(v);
  v = v > t ? v : t;
  t = dpp_u64<0x114, 0xf>(v);
  v = v > t ? v : t;
  t = dpp_u64<0x118, 0xf>(v);
  v = v > t ? v : t;
  t = dpp_u64<0x142, 0xa>(v);
  v = v > t ? v : t;
  t = dpp_u64<0x143, 0xc>(v);
  v = v > t ? v : t;
  return lane_u64(v, 63);
}
// The largest t with at least k (1 <= k <= 64) lanes holding a value >= t:
// the k-th largest of the 64 values (0 if fewer than k are nonzero), found
// bit by bit from the top with one ballot per bit.
__device__ __forceinline__ uint32_t wave_kth_largest_radix(uint32_t x, int k) {
  uint32_t t = 0u;
#pragma unroll
  for (int b = 31; b >= 0; --b) {
    const uint32_t u = t | (1u << b);
    if (__popcll(__ballot(x >= u)) >= (uint32_t)k) t = u;
  }
  return t;
}
// k-th largest (1 <= k <= 256) of up to four values per lane (zeros for
// absent ones): the same bitwise ballot radix select over 256 values.
__device__ __forceinline__ uint32_t wave_kth_largest_radix4(const uint32_t (&x)[4], int k) {
  uint32_t t = 0u;
#pragma unroll
  for (int b = 31; b >= 0; --b) {
    const uint32_t u = t | (1u << b);
    uint32_t c = 0u;
#pragma unroll
    for (int q = 0; q < 4; ++q) c += (uint32_t)__popcll(__ballot(x[q] >= u));
    if (c >= (uint32_t)k) t = u;
  }
  return t;
}
__device__ __forceinline__ int wave_sum_int(int v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  return v;
}
__device__ __forceinline__ int wave_incl_scan(int x, int lane) {
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int y = __shfl_up(x, o);
    if (lane >= o) x += y;
  }
  return x;
}

// k-th largest (1 <= k <= 64) of one value per lane: bitonic sort of the
// 64 lane values (ascending) through cross-lane shuffles, then lane 64 - k.
__device__ __forceinline__ uint32_t wave_kth_largest(uint32_t v, int k) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int size = 2; size <= 64; size <<= 1) {
#pragma unroll
    for (int j = size >> 1; j > 0; j >>= 1) {
      const uint32_t o = __shfl_xor(v, j);
      const bool take_min = ((lane & size) == 0) == ((lane & j) == 0);
      v = take_min ? (v < o ? v : o) : (v > o ? v : o);
    }
  }
  return __shfl(v, 64 - k);
}

// Ascending bitonic sort of one value per lane across the wave: lane i
// returns the i-th smallest.
__device__ __forceinline__ uint32_t wave_sort_asc(uint32_t v) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int size = 2; size <= 64; size <<= 1) {
#pragma unroll
    for (int j = size >> 1; j > 0; j >>= 1) {
      const uint32_t o = __shfl_xor(v, j);
      const bool take_min = ((lane & size) == 0) == ((lane & j) == 0);
      v = take_min ? (v < o ? v : o) : (v > o ? v : o);
    }
  }
  return v;
}

// The ka-th and kb-th largest (1 <= ka, kb <= 64) of one value per lane.
__device__ __forceinline__ void wave_kth_pair(uint32_t v, int ka, int kb, uint32_t* a, uint32_t* b) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int size = 2; size <= 64; size <<= 1) {
#pragma unroll
    for (int j = size >> 1; j > 0; j >>= 1) {
      const uint32_t o = __shfl_xor(v, j);
      const bool take_min = ((lane & size) == 0) == ((lane & j) == 0);
      v = take_min ? (v < o ? v : o) : (v > o ? v : o);
    }
  }
  *a = __shfl(v, 64 - ka);
  *b = __shfl(v, 64 - kb);
}

// Block-wide reductions through a small LDS array (NW entries). Every
// thread must call them; the result is returned to every thread.
__device__ uint64_t block_max_u64(uint64_t v, uint64_t* red) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  v = wave_max_u64(v);
  __syncthreads();
  if (lane == 0) red[wave] = v;
  __syncthreads();
  uint64_t r = red[0];
#pragma unroll
  for (int w = 1; w < NW; ++w) r = r > red[w] ? r : red[w];
  return r;
}
__device__ double block_sum_f64(double v, double* red) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  v = wave_sum_f64(v);
  __syncthreads();
  if (lane == 0) red[wave] = v;
  __syncthreads();
  double r = 0.0;
#pragma unroll
  for (int w = 0; w < NW; ++w) r += red[w];
  return r;
}
__device__ int block_sum_int(int v, int* red) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  v = wave_sum_int(v);
  __syncthreads();
  if (lane == 0) red[wave] = v;
  __syncthreads();
  int r = 0;
#pragma unroll
  for (int w = 0; w < NW; ++w) r += red[w];
  return r;
}
// Exclusive block scan of per-thread counts; returns the offset, *total the sum.
__device__ int block_excl_scan(int cnt, int* red, int* total) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int inc = wave_incl_scan(cnt, lane);
  __syncthreads();
  if (lane == 63) red[wave] = inc;
  __syncthreads();
  int base = 0, tot = 0;
#pragma unroll
  for (int w = 0; w < NW; ++w) {
    const int t = red[w];
    base += (w < wave) ? t : 0;
    tot += t;
  }
  *total = tot;
  return base + inc - cnt;
}

// ---------------------------------------------------------------------------
// logit loading (binary32 or bf16, optional penalties)
// ---------------------------------------------------------------------------
struct RowCtx {
  const char* base;        // row start
  // element type 2 (head accumulators)
  const int64_t* acc;      // the row's accumulators
  int64_t* accw;           // the same, to clear (or NULL)
  const float* tau;        // [V]
  float us, r;             // common scale, inverse RMS of the row
  const float* lout;       // the row's logits written out (re-reads), or NULL
  float* loutw;            // the same, to write (or NULL)
  // Penalty words of the row (or NULL): word w holds the history membership
  // bits of ids 32w..32w+31 and the number of distinct history ids below 32w,
  // the index into pcnt of the word's first member.
  const uint2* pw;
  const uint32_t* pcnt;
  float rep, pres, freq;
};

// History count of a member id whose penalty word is w.
__device__ __forceinline__ uint32_t pen_count(const RowCtx& r, uint2 w, uint32_t v) {
  return r.pcnt[w.y + __popc(w.x & ((1u << (v & 31)) - 1u))];
}

// Penalties in binary32 round-to-nearest, each operation separately rounded.
__device__ __forceinline__ uint32_t penalize(uint32_t bits, uint32_t c, const RowCtx& r) {
  float l = __uint_as_float(bits);
  if (r.rep != 1.0f) l = (l > 0.0f) ? __fdiv_rn(l, r.rep) : __fmul_rn(l, r.rep);
  const float fc = __fmul_rn(r.freq, (float)c);
  l = __fsub_rn(l, fc);
  l = __fsub_rn(l, r.pres);
  return __float_as_uint(l);
}

// Head logit i from its int64 accumulator in the reference's exact order:
// one round-to-nearest int64 -> binary32 conversion, then three separately
// rounded binary32 multiplies (compressed_linear.rs:329-340; spec 06 section
// 2; src/misc_kernels.cu:63-69).
__device__ __forceinline__ float head_value(const RowCtx& r, int64_t i) {
  float x = (float)r.acc[i];
  x = __fmul_rn(x, r.us);
  x = __fmul_rn(x, r.r);
  return __fmul_rn(x, r.tau[i]);
}

template <int DT>
__device__ __forceinline__ uint32_t raw_bits(const RowCtx& r, int64_t i) {
  if (DT == 0) return ((const uint32_t*)r.base)[i];
  if (DT == 1) return (uint32_t)((const uint16_t*)r.base)[i] << 16;
  // a head row re-read: the logits written out, or formed again
  if (r.lout) return __float_as_uint(r.lout[i]);
  return __float_as_uint(head_value(r, i));
}

template <int DT, bool PEN>
__device__ __forceinline__ uint32_t value_bits(const RowCtx& r, int64_t i) {
  uint32_t b = raw_bits<DT>(r, i);
  if (PEN && r.pw) {
    const uint2 w = r.pw[i >> 5];
    if ((w.x >> (i & 31)) & 1u) b = penalize(b, pen_count(r, w, (uint32_t)i), r);
  }
  return b;
}

__device__ __forceinline__ bool nonfinite_bits(uint32_t b) { return (b & 0x7f800000u) == 0x7f800000u; }

// ---------------------------------------------------------------------------
// Per-row configuration derived from the parameters.
// ---------------------------------------------------------------------------
struct RowPlan {
  int64_t k_eff;  // candidates of top-k (V when disabled)
  int KB;         // length of the raw-order prefix the row needs
  int KL;         // length of the waves' lists in the stream: min(KB, KBMAX); a
                  // row with KB > KBMAX takes the dense path (exact KB-th key)
  bool need_rel;  // large-k sampling: needs every relevant element
  bool sampled;   // not greedy and ids requested
};

__device__ __forceinline__ RowPlan make_plan(const SmpArgs& A, const DevParams& P) {
  RowPlan p;
  p.sampled = A.out_ids != nullptr && !P.greedy;
  p.k_eff = (P.top_k == 0) ? (int64_t)A.V : (int64_t)P.top_k;
  int kb = 1;
  if (p.sampled && p.k_eff <= KBMAX) kb = (int)p.k_eff;
  if (A.top8_ids && kb < 8) kb = 8;
  if (A.top20_ids && kb < 20) kb = 20;
  if (A.topn_ids && kb < A.topn) kb = A.topn;
  if (A.n_lp > kb) kb = A.n_lp;
  if (kb > A.V) kb = A.V;
  p.KB = kb;
  p.KL = kb < KBMAX ? kb : KBMAX;
  p.need_rel = p.sampled && p.k_eff > KBMAX;
  return p;
}

// Prediction position of draw d of a row. The base form is checked like the
// reference's accept loop (checked_add, speculation.rs:489-497): *ok is false
// when base + depth + 1 passes 2^64 - 1. Depth comes from the row table or
// the row index (q35_sample.cu:180-181; spec 06 section 5).
__device__ __forceinline__ uint64_t position_of(const SmpArgs& A, int row, int d, bool* ok) {
  if (A.pos_mode == POS_BASE) {
    const uint64_t depth = A.row_depth ? (uint64_t)A.row_depth[A.row0 + row] : (uint64_t)(A.row0 + row);
    const uint64_t b = *A.base_position;
    *ok = b <= ~0ull - (depth + 1u);
    return b + depth + 1u;
  }
  *ok = true;
  return A.positions[(int64_t)row * A.n_draws + d];
}
__device__ __forceinline__ uint64_t position_of(const SmpArgs& A, int row, int d) {
  bool ok;
  return position_of(A, row, d, &ok);
}

// ---------------------------------------------------------------------------
// Exact serial binary64 prefix sums, in parallel.
//
// The reference sums the candidates' weights serially in candidate order
// (output_head_sampler.rs:157-175): S_j = (..(w_0 + w_1) + ..) + w_j, each
// add rounded to nearest-even. Here w_0 = 1 >= w_j >= 0, so S_j >= 1 and
// every w_j <= S_{j-1}. While the sum stays in one binade [2^e, 2^(e+1)),
// each add rounds to the grid of that binade's unit u = 2^(e-52): w_j adds
// round(w_j / u) units, exactly, and depends on the running sum only when
// w_j / u = q + 1/2 is a tie, which goes to the even unit count (a function
// of the sum's parity). A tile of weights is therefore a composition of
// functions of one parity bit, scanned across the block; the first element
// whose sum leaves the binade is added with a real binary64 add, which
// starts the next binade (an add can cross at most one, since w_j <= S).
// ---------------------------------------------------------------------------
struct PFun {
  uint64_t d0, d1;  // units added to a running sum of even / odd unit count
  uint32_t p;       // bit b: parity of the result from input parity b
};
__device__ __forceinline__ PFun pf_identity() { return PFun{0ull, 0ull, 2u}; }
// `a` first, then `b`
__device__ __forceinline__ PFun pf_then(const PFun& a, const PFun& b) {
  const uint32_t a0 = a.p & 1u, a1 = (a.p >> 1) & 1u;
  PFun r;
  r.d0 = a.d0 + (a0 ? b.d1 : b.d0);
  r.d1 = a.d1 + (a1 ? b.d1 : b.d0);
  const uint32_t b0 = b.p & 1u, b1 = (b.p >> 1) & 1u;
  r.p = (a0 ? b1 : b0) | ((a1 ? b1 : b0) << 1);
  return r;
}
// the add of a weight worth x = w / u units (x >= 0, exact)
__device__ __forceinline__ PFun pf_weight(double x) {
  const double q = floor(x);  // exact, as is x - q
  const double f = x - q;
  const uint64_t qi = (uint64_t)q;
  PFun r;
  if (f == 0.5) {
    // s + q + 1/2 rounds to whichever of s + q, s + q + 1 is even
    r.d0 = qi + (qi & 1ull);
    r.d1 = qi + ((qi + 1ull) & 1ull);
    r.p = 0u;
  } else {
    const uint64_t d = qi + (f > 0.5 ? 1ull : 0ull);
    r.d0 = d;
    r.d1 = d;
    const uint32_t b = (uint32_t)(d & 1ull);
    r.p = b | ((b ^ 1u) << 1);
  }
  return r;
}
__device__ __forceinline__ PFun pf_shfl_up(const PFun& x, int o) {
  PFun y;
  y.d0 = (uint64_t)__shfl_up((unsigned long long)x.d0, o);
  y.d1 = (uint64_t)__shfl_up((unsigned long long)x.d1, o);
  y.p = (uint32_t)__shfl_up((int)x.p, o);
  return y;
}

struct PScanShared {
  PFun wave[NW];
  double s;     // the sum before the next element
  int64_t j0;   // the next element
  int64_t jc;   // the first element of the tile whose sum leaves the binade
};

// S[j] for j < c (S may alias w: every element is read before it is
// written). Block-wide.
__device__ void exact_prefix(const double* w, double* S, int64_t c, PScanShared* ps) {
  constexpr int PT = 8;  // elements per thread and tile
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  if (tid == 0) {
    const double s0 = w[0];
    S[0] = s0;
    ps->s = s0;
    ps->j0 = 1;
  }
  __syncthreads();
  for (;;) {
    const int64_t j0 = ps->j0;
    if (j0 >= c) break;  // (block-uniform)
    const double s = ps->s;
    const uint64_t sb = (uint64_t)__double_as_longlong(s);
    const int E = (int)(sb >> 52);  // biased exponent: s >= 1 is normal
    const uint64_t su = (sb & 0x000fffffffffffffull) | 0x0010000000000000ull;  // s / u
    const int sh = 1075 - E;                                                    // w / u = w * 2^sh
    const double u = __longlong_as_double((long long)((uint64_t)(E - 52) << 52));
    const int64_t jb = j0 + (int64_t)tid * PT;
    const int64_t je = j0 + (int64_t)NT * PT < c ? j0 + (int64_t)NT * PT : c;  // tile end
    __syncthreads();  // ps->s and ps->j0 read
    if (tid == 0) ps->jc = INT64_MAX;
    double wv[PT];  // (the per-element functions are formed again where needed)
    PFun mine = pf_identity();
#pragma unroll
    for (int q = 0; q < PT; ++q) {
      const int64_t j = jb + q;
      wv[q] = j < je ? w[j] : 0.0;
      if (j < je) mine = pf_then(mine, pf_weight(ldexp(wv[q], sh)));
    }
    // exclusive scan of the threads' functions, in thread order
    PFun inc = mine;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const PFun y = pf_shfl_up(inc, o);
      if (lane >= o) inc = pf_then(y, inc);
    }
    PFun before = pf_shfl_up(inc, 1);
    if (lane == 0) before = pf_identity();
    if (lane == 63) ps->wave[wave] = inc;
    __syncthreads();
    PFun pre = pf_identity();
    for (int k = 0; k < wave; ++k) pre = pf_then(pre, ps->wave[k]);
    pre = pf_then(pre, before);
    // this thread's sums in units of u; the first that leaves the binade
    const uint32_t p0 = (uint32_t)(su & 1ull);
    const uint64_t acc0 = p0 ? pre.d1 : pre.d0;
    const uint32_t pp0 = (pre.p >> p0) & 1u;
    uint32_t p = pp0;
    uint64_t acc = acc0;
    int64_t my_jc = INT64_MAX;
    double s_prev_c = 0.0, w_c = 0.0, s_last = 0.0;
#pragma unroll
    for (int q = 0; q < PT; ++q) {
      const int64_t j = jb + q;
      if (j < je) {
        const uint64_t a0 = acc;
        const PFun f = pf_weight(ldexp(wv[q], sh));
        acc += p ? f.d1 : f.d0;
        p = (f.p >> p) & 1u;
        if (my_jc == INT64_MAX && su + acc >= (1ull << 53)) {
          my_jc = j;
          s_prev_c = (double)(su + a0) * u;
          w_c = wv[q];
        }
        if (j == je - 1) s_last = (double)(su + acc) * u;
      }
    }
    if (my_jc != INT64_MAX) atomicMin((unsigned long long*)&ps->jc, (unsigned long long)my_jc);
    __syncthreads();
    const int64_t jc = ps->jc;
    const int64_t jw = jc < je ? jc : je;  // elements below jw stay in the binade
    p = pp0;
    acc = acc0;
#pragma unroll
    for (int q = 0; q < PT; ++q) {
      const int64_t j = jb + q;
      if (j < jw) {
        const PFun f = pf_weight(ldexp(wv[q], sh));
        acc += p ? f.d1 : f.d0;
        p = (f.p >> p) & 1u;
        S[j] = (double)(su + acc) * u;
      }
    }
    if (jc < je) {
      if (my_jc == jc) {
        const double sn = s_prev_c + w_c;  // the serial add itself
        S[jc] = sn;
        ps->s = sn;
        ps->j0 = jc + 1;
      }
    } else if (je - 1 >= jb && je - 1 < jb + PT) {
      ps->s = s_last;
      ps->j0 = je;
    }
    __syncthreads();
  }
}

// First j in [lo, hi) with S[j] >= t (strict: S[j] > t), or hi; S is
// non-decreasing. One wave, 64 probes per round. Every lane returns it.
__device__ __forceinline__ int64_t first_reaching(const double* S, int64_t lo, int64_t hi, double t, bool strict) {
  const int lane = threadIdx.x & 63;
  while (hi - lo > 64) {
    const int64_t step = (hi - lo + 63) / 64;
    int64_t idx = lo + (int64_t)(lane + 1) * step - 1;
    if (idx > hi - 1) idx = hi - 1;
    const double v = S[idx];
    const uint64_t m = __ballot(strict ? v > t : v >= t);
    if (!m) return hi;
    const int64_t L = (int64_t)__builtin_ctzll(m);
    const int64_t nlo = lo + L * step;
    const int64_t nhi = lo + (L + 1) * step;
    lo = nlo;
    hi = nhi < hi ? nhi : hi;
  }
  const int64_t idx = lo + lane;
  const bool in = idx < hi;
  const double v = in ? S[idx] : 0.0;
  const uint64_t m = __ballot(in && (strict ? v > t : v >= t));
  return m ? lo + (int64_t)__builtin_ctzll(m) : hi;
}
// First j in [lo, hi) with w[j] < t, or hi; w is non-increasing.
__device__ __forceinline__ int64_t first_below(const double* w, int64_t lo, int64_t hi, double t) {
  const int lane = threadIdx.x & 63;
  while (hi - lo > 64) {
    const int64_t step = (hi - lo + 63) / 64;
    int64_t idx = lo + (int64_t)(lane + 1) * step - 1;
    if (idx > hi - 1) idx = hi - 1;
    const uint64_t m = __ballot(w[idx] < t);
    if (!m) return hi;
    const int64_t L = (int64_t)__builtin_ctzll(m);
    const int64_t nhi = lo + (L + 1) * step;
    lo = lo + L * step;
    hi = nhi < hi ? nhi : hi;
  }
  const int64_t idx = lo + lane;
  const bool in = idx < hi;
  const uint64_t m = __ballot(in && w[in ? idx : lo] < t);
  return m ? lo + (int64_t)__builtin_ctzll(m) : hi;
}

// ---------------------------------------------------------------------------
// Truncation and draw on the first c sorted candidates (output_head_sampler.rs
// :136-212). cand/w are generic pointers (LDS or global scratch); w is
// overwritten with the prefix sums.
// ---------------------------------------------------------------------------
struct TailShared {
  int64_t retained;
  double mass;  // serial binary64 sum of the retained weights (version 2)
  PScanShared scan;
};

__device__ __forceinline__ void sample_tail(const SmpArgs& A, const DevParams& P, int row, const uint64_t* cand,
                            double* w, int64_t c, TailShared* ts, double* redd, int* redi,
                            uint64_t* redu) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const double T = P.temperature;
  const float v0 = key2f(pk_key(cand[0]));
  // weights: widen, subtract, divide, exp_d -- in candidate order
  for (int64_t j = tid; j < c; j += NT) {
    const double z = ((double)key2f(pk_key(cand[j])) - (double)v0) / T;
    w[j] = exp_d_inline(z);
  }
  __syncthreads();
  // min-p relative to w_0 = 1: the first j >= 1 with w_j < min_p ends the
  // kept prefix (the weights do not increase along the candidates)
  if (wave == 0) {
    const int64_t m = P.min_p > 0.0 ? first_below(w, 1, c, P.min_p) : c;
    if (lane == 0) ts->retained = m;
  }
  __syncthreads();
  // the serial prefix sums, exactly
  exact_prefix(w, w, c, &ts->scan);
  if (wave == 0) {
    const double total = w[c - 1];
    // top-p: the first n with prefix_{n-1} >= top_p * total (:160-166)
    const int64_t n = first_reaching(w, 0, c, P.top_p * total, false);
    int64_t r = n < c ? n + 1 : c;
    const int64_t m = ts->retained;
    if (m < r) r = m;
    if (lane == 0) {
      ts->retained = r;
      ts->mass = w[r - 1];  // the retained mass: the same serial sum (:191)
    }
  }
  __syncthreads();
  const int64_t r = ts->retained;
  const int nd = A.mode == MODE_VERIFY ? 1 : A.n_draws;
  if (P.version == YSKN_V3 && (nd == 1 || r > 64)) {
    // each draw over the candidates in parallel: argmax of z + g with the
    // earliest candidate winning ties (strict > in candidate order)
    for (int d = 0; d < nd; ++d) {
      const uint64_t pk = position_key(P.seed, position_of(A, row, d));
      double best = -__builtin_inf();
      int64_t bj = r - 1;
      for (int64_t j = tid; j < r; j += NT) {
        const uint64_t cj = cand[j];
        const double z = ((double)key2f(pk_key(cj)) - (double)v0) / T;
        const double s = z + gumbel_from_key(pk, pk_id(cj));
        if (s > best || (s == best && j < bj)) {
          best = s;
          bj = j;
        }
      }
#pragma unroll
      for (int o = 32; o > 0; o >>= 1) {
        const double ob = __shfl_xor(best, o);
        const int64_t oj = __shfl_xor((long long)bj, o);
        if (ob > best || (ob == best && oj < bj)) {
          best = ob;
          bj = oj;
        }
      }
      __syncthreads();
      if (lane == 0) {
        redd[wave] = best;
        redu[wave] = (uint64_t)bj;
      }
      __syncthreads();
      if (tid == 0) {
        double b = redd[0];
        int64_t jj = (int64_t)redu[0];
        for (int q = 1; q < NW; ++q) {
          if (redd[q] > b || (redd[q] == b && (int64_t)redu[q] < jj)) {
            b = redd[q];
            jj = (int64_t)redu[q];
          }
        }
        A.out_ids[(int64_t)row * A.n_draws + d] = pk_id(cand[jj]);
      }
    }
    __syncthreads();
    return;
  }
  if (P.version == YSKN_V3) {
    // several draws over at most 64 candidates: one thread per draw
    for (int d = tid; d < nd; d += NT) {
      const uint64_t pk = position_key(P.seed, position_of(A, row, d));
      double best = -__builtin_inf();
      int64_t pick = r - 1;
      for (int64_t j = 0; j < r; ++j) {
        const uint64_t cj = cand[j];
        const double z = ((double)key2f(pk_key(cj)) - (double)v0) / T;
        const double s = z + gumbel_from_key(pk, pk_id(cj));
        if (s > best) {
          best = s;
          pick = j;
        }
      }
      A.out_ids[(int64_t)row * A.n_draws + d] = pk_id(cand[pick]);
    }
    __syncthreads();
    return;
  }
  // version 2: draw d picks the first j with u_d * mass < prefix_j
  // (:196-207), by a search of the prefix sums; one wave per draw
  for (int d = wave; d < nd; d += NW) {
    const double t = uniform_v2(P.seed, position_of(A, row, d)) * ts->mass;
    const int64_t j = first_reaching(w, 0, r, t, true);
    if (lane == 0) A.out_ids[(int64_t)row * A.n_draws + d] = pk_id(cand[j < r ? j : r - 1]);
  }
  __syncthreads();
}

// ---------------------------------------------------------------------------
// The same truncation and draw by one wave, for one draw over c <= 64
// sorted candidates (the common case): candidate j in lane j; weights and
// scores in one parallel pass; the reference's serial binary64 sums run in
// candidate order over values broadcast from the lanes (readlane).
// ---------------------------------------------------------------------------
__device__ __forceinline__ double lane_f64(double x, int j) {
  const uint64_t b = (uint64_t)__double_as_longlong(x);
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)b, j);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(b >> 32), j);
  return __longlong_as_double((long long)(((uint64_t)hi << 32) | lo));
}

// pre: LDS scratch of at least 128 binary64 values. With `have_pre`, pre[j]
// and pre[64 + j] already hold candidate j's weight and (version 3) score,
// computed by other waves while the candidates were being ranked; otherwise
// the weights are computed here and written to pre[j].
__device__ __forceinline__ void sample_tail_wave(const SmpArgs& A, const DevParams& P, int row,
                                                 const uint64_t* cand, int c, uint64_t pos, double* pre,
                                                 bool have_pre) {
  const int lane = threadIdx.x & 63;
  const double T = P.temperature;
  const float v0 = key2f(pk_key(cand[0]));
  const bool in = lane < c;
  const uint64_t cj = in ? cand[lane] : 0ull;
  double w = 0.0, sc = -__builtin_inf();
  if (in) {
    if (have_pre) {
      w = pre[lane];
      if (P.version == YSKN_V3) sc = pre[64 + lane];
    } else {
      const double z = ((double)key2f(pk_key(cj)) - (double)v0) / T;  // widen, subtract, divide
      w = exp_d_inline(z);
      if (P.version == YSKN_V3) sc = z + gumbel_from_key<true>(position_key(P.seed, pos), pk_id(cj));
    }
  }
  // The serial binary64 prefix sums in candidate order, one pass: lane j
  // keeps prefix_j = (..((w_0 + w_1) + w_2) ..) + w_j; the total is the last.
  // The weights are read from LDS by every lane at once (broadcast reads,
  // eight issued ahead of their adds), so the chain is the adds alone.
  if (!have_pre && in) pre[lane] = w;  // (the wave's own LDS writes precede its reads)
  double prefix = 0.0, pre_j = 0.0;
  for (int j0 = 0; j0 < c; j0 += 8) {
    double v[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) v[k] = pre[j0 + k];  // (c <= 64 < CAP: in bounds)
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      if (j0 + k < c) {
        prefix = prefix + v[k];
        pre_j = lane == j0 + k ? prefix : pre_j;
      }
    }
  }
  // top-p: the first n with prefix_{n-1} >= top_p * total
  const double thr = P.top_p * prefix;
  const uint64_t reach = __ballot(in && pre_j >= thr);
  int n = reach ? (int)__builtin_ctzll(reach) + 1 : c;
  // min-p relative to w_0 = 1: the first j >= 1 with w_j < min_p ends it
  if (P.min_p > 0.0) {
    const uint64_t below = __ballot(lane >= 1 && lane < n && w < P.min_p);
    if (below) n = (int)__builtin_ctzll(below);
  }
  int pick = n - 1;
  if (P.version == YSKN_V3) {
    // argmax of z + g over the retained candidates; the earliest wins ties
    // (order-preserving 64-bit keys of the scores, -0 taken as +0)
    uint64_t key = 0ull;
    if (lane < n) {
      const uint64_t b = (uint64_t)__double_as_longlong(sc == 0.0 ? 0.0 : sc);
      key = (b >> 63) ? ~b : (b | 0x8000000000000000ull);
    }
    const uint64_t best = wave_max_u64_dpp(key);
    const uint64_t hit = __ballot(lane < n && key == best);
    if (hit) pick = (int)__builtin_ctzll(hit);
  } else {
    // the retained mass is prefix_{n-1} (the same serial sum); the first
    // j with t < prefix_j is drawn
    const double mass = lane_f64(pre_j, n - 1);
    const double t = uniform_v2(P.seed, pos) * mass;
    const uint64_t hit = __ballot(lane < n && t < pre_j);
    if (hit) pick = (int)__builtin_ctzll(hit);
  }
  const uint32_t id = pk_id((uint64_t)(((uint64_t)(uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(cj >> 32), pick) << 32) |
                                       (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)cj, pick)));
  if (lane == 0) A.out_ids[(int64_t)row * A.n_draws] = id;
}

// ---------------------------------------------------------------------------
// Dense path: exact sorted order of every element with key >= theta_D.
// ---------------------------------------------------------------------------
// The exact need-th largest key of the row (1 <= need <= V): four 8-bit
// radix passes from the top over the whole row. hist: 256 LDS words, bc: 2.
// Block-wide; every thread returns the key.
// Histogram increment of an 8-bit `bin` for the valid lanes of a wave:
// lanes with equal bins are found with one ballot per bit and the lowest of
// them adds their number (one LDS atomic per distinct bin, not per lane:
// concentrated keys would otherwise serialise on a few counters).
__device__ __forceinline__ uint64_t bin_peers(uint32_t bin, bool valid) {
  uint64_t peers = __ballot(valid);
#pragma unroll
  for (int b = 0; b < 8; ++b) {
    const bool bit = (bin >> b) & 1u;
    const uint64_t bal = __ballot(bit);
    peers &= bit ? bal : ~bal;
  }
  return peers;
}
__device__ __forceinline__ void hist_add8(uint32_t* hist, uint32_t bin, bool valid) {
  const int lane = threadIdx.x & 63;
  const uint64_t peers = bin_peers(bin, valid);
  if (valid && (peers & ((1ull << lane) - 1ull)) == 0ull) atomicAdd(&hist[bin], (uint32_t)__popcll(peers));
}

// The exact need-th largest key of the row (1 <= need <= V): four 8-bit
// radix passes from the top over the whole row. hist: 256 LDS words, bc: 2.
// Block-wide; every thread returns the key.
template <int DT, bool PEN>
__device__ __forceinline__ uint32_t radix_kth_key(const RowCtx& rc, int V, int64_t need_in, uint32_t* hist,
                                                  uint32_t* bc) {
  const int tid = threadIdx.x;
  uint32_t prefix = 0, mask = 0;
  int64_t need = need_in;
  for (int pass = 0; pass < 4; ++pass) {
    const int shift = 24 - 8 * pass;
    for (int i = tid; i < 256; i += NT) hist[i] = 0;
    __syncthreads();
    for (int64_t i0 = 0; i0 < V; i0 += NT) {
      const int64_t i = i0 + tid;
      const uint32_t k = i < V ? f2key(value_bits<DT, PEN>(rc, i)) : 0u;
      hist_add8(hist, (k >> shift) & 255u, i < V && (k & mask) == prefix);
    }
    __syncthreads();
    if (tid == 0) {
      int64_t cum = 0;
      int dsel = 0;
      for (int d = 255; d >= 0; --d) {
        const int64_t h = (int64_t)hist[d];
        if (cum + h >= need) {
          dsel = d;
          need -= cum;
          break;
        }
        cum += h;
      }
      bc[0] = (uint32_t)dsel;
      bc[1] = (uint32_t)need;
    }
    __syncthreads();
    prefix |= bc[0] << shift;
    mask |= 255u << shift;
    need = (int64_t)bc[1];
    __syncthreads();
  }
  return prefix;
}

// Order-preserving compaction of the row's elements with key >= theta
// (theta >= 1) into da as packed (key, id) entries, ids ascending. Tiles of
// NT * 8 elements read coalesced: element (q, t) is tile + q * NT + t, and
// its rank counts the kept elements of rows q' < q, of the waves before t's
// in row q and of the lanes below it. lds: 65 words. Returns the count.
template <int DT, bool PEN>
__device__ int64_t dense_compact(const RowCtx& rc, int V, uint32_t theta, uint64_t* da, uint32_t* lds) {
  constexpr int PER = 8;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  uint32_t* cnt = lds;              // [PER][NW] counts, then offsets
  uint32_t* tot = lds + PER * NW;
  const uint64_t below = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  int64_t n = 0;
  for (int64_t base = 0; base < V; base += (int64_t)NT * PER) {
    uint32_t keys[PER];
    uint64_t m[PER];
    // every load issued (clamped index) so that all PER are in flight together
#pragma unroll
    for (int q = 0; q < PER; ++q) {
      const int64_t i = base + (int64_t)q * NT + tid;
      keys[q] = value_bits<DT, PEN>(rc, i < V ? i : (int64_t)V - 1);
    }
#pragma unroll
    for (int q = 0; q < PER; ++q) {
      const int64_t i = base + (int64_t)q * NT + tid;
      keys[q] = i < V ? f2key(keys[q]) : 0u;
    }
#pragma unroll
    for (int q = 0; q < PER; ++q) {
      m[q] = __ballot(keys[q] >= theta);
      if (lane == 0) cnt[q * NW + wave] = (uint32_t)__popcll(m[q]);
    }
    __syncthreads();
    if (wave == 0) {
      static_assert(PER * NW == 64, "one (row, wave) count per lane");
      const uint32_t c0 = cnt[lane];
      const uint32_t inc = (uint32_t)wave_incl_scan((int)c0, lane);
      cnt[lane] = inc - c0;
      if (lane == 63) *tot = inc;
    }
    __syncthreads();
#pragma unroll
    for (int q = 0; q < PER; ++q) {
      if (keys[q] >= theta)
        da[n + cnt[q * NW + wave] + (uint32_t)__popcll(m[q] & below)] =
            pack(keys[q], (uint32_t)(base + (int64_t)q * NT + tid));
    }
    n += *tot;
    __syncthreads();
  }
  return n;
}

// Stable sort of n packed (key, id) entries by key, descending (equal keys
// keep their order): LSD passes on the key bytes, digit 255 - byte, between
// a and b; a pass whose digit is the same for every entry is skipped; the
// result ends in a. One pass over the entries first counts all four digit
// histograms (plain LDS atomics: no order is needed there). A pass takes
// tiles of NT * 8 entries: wave w holds the
// tile's entries w * 512 + 64 q + lane (q < 8) and counts their digits;
// each entry's place in the tile, in (digit, wave, slot, lane) order, puts
// it in the LDS tile buffer, which is then written out in order: a digit's
// entries of the tile are one contiguous run of the destination.
// lds: 5,888 words; sbuf: NT * 8 entries. Block-wide.
__device__ __forceinline__ void lsd_sort_desc(uint64_t* a, uint64_t* b, int64_t n, uint32_t* lds, uint64_t* sbuf) {
  constexpr int PER = 8;
  constexpr int64_t TILE = (int64_t)NT * PER;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  uint32_t* gb = lds;                      // [4][256] digit counts, then running bases
  uint32_t* wc = lds + 1024;               // [NW][256] per-wave digit counts / cursors
  uint32_t* wo = lds + 1024 + NW * 256;    // [256][NW] per-wave offsets within a digit
  uint32_t* ts = lds + 1024 + 2 * NW * 256;        // [256] the tile's digit starts
  uint32_t* tc = lds + 1024 + 2 * NW * 256 + 256;  // [256] the tile's digit counts
  uint32_t* skip = lds + 1024 + 2 * NW * 256 + 512;  // [4] one digit only
  for (int i = tid; i < 1024; i += NT) gb[i] = 0u;
  __syncthreads();
  for (int64_t i = tid; i < n; i += NT) {
    const uint32_t key = (uint32_t)(a[i] >> 32);
#pragma unroll
    for (int p = 0; p < 4; ++p) atomicAdd(&gb[p * 256 + (255u - ((key >> (8 * p)) & 255u))], 1u);
  }
  __syncthreads();
  if (wave < 4) {
    // exclusive scan of pass `wave`'s 256 counts, four per lane
    uint32_t c[4], loc = 0u;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      c[q] = gb[wave * 256 + lane * 4 + q];
      loc += c[q];
    }
    const bool one = __ballot(c[0] == (uint32_t)n || c[1] == (uint32_t)n || c[2] == (uint32_t)n ||
                              c[3] == (uint32_t)n) != 0ull;
    const uint32_t inc = (uint32_t)wave_incl_scan((int)loc, lane);
    uint32_t run = inc - loc;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      gb[wave * 256 + lane * 4 + q] = run;
      run += c[q];
    }
    if (lane == 0) skip[wave] = one ? 1u : 0u;
  }
  __syncthreads();
  const uint64_t below = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  uint64_t* src = a;
  uint64_t* dst = b;
  for (int p = 0; p < 4; ++p) {
    if (skip[p]) continue;  // (block-uniform)
    const int shift = 32 + 8 * p;
    for (int64_t t0 = 0; t0 < n; t0 += TILE) {
      const int64_t tn = n - t0 < TILE ? n - t0 : TILE;
      uint64_t e[PER];
      uint32_t d[PER];
      uint64_t pm[PER];
      const int64_t wb = t0 + (int64_t)wave * 64 * PER;
#pragma unroll
      for (int q = 0; q < PER; ++q) {
        const int64_t i = wb + q * 64 + lane;
        e[q] = i < n ? src[i] : 0ull;
      }
      for (int i = lane; i < 256; i += 64) wc[wave * 256 + i] = 0u;
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
#pragma unroll
      for (int q = 0; q < PER; ++q) {
        const bool v = wb + q * 64 + lane < n;
        d[q] = 255u - (uint32_t)((e[q] >> shift) & 255u);
        pm[q] = bin_peers(d[q], v);
        if (v && (pm[q] & below) == 0ull) atomicAdd(&wc[wave * 256 + d[q]], (uint32_t)__popcll(pm[q]));
      }
      __syncthreads();
      if (wave == 0) {
        // digits 4 lane .. 4 lane + 3: offsets of the waves within each
        // digit, the tile's digit counts and (scanned) starts
        uint32_t loc = 0u;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const int dd = lane * 4 + k;
          uint32_t run = 0u;
#pragma unroll
          for (int w = 0; w < NW; ++w) {
            const uint32_t c = wc[w * 256 + dd];
            wo[dd * NW + w] = run;
            wc[w * 256 + dd] = 0u;
            run += c;
          }
          tc[dd] = run;
          loc += run;
        }
        const uint32_t inc = (uint32_t)wave_incl_scan((int)loc, lane);
        uint32_t st = inc - loc;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          ts[lane * 4 + k] = st;
          st += tc[lane * 4 + k];
        }
      }
      __syncthreads();
#pragma unroll
      for (int q = 0; q < PER; ++q) {
        const bool v = wb + q * 64 + lane < n;
        const int lead = v ? (int)__builtin_ctzll(pm[q]) : lane;
        uint32_t old = 0u;
        if (v && lead == lane) old = atomicAdd(&wc[wave * 256 + d[q]], (uint32_t)__popcll(pm[q]));
        old = (uint32_t)__shfl((int)old, lead);
        if (v) sbuf[ts[d[q]] + wo[d[q] * NW + wave] + old + (uint32_t)__popcll(pm[q] & below)] = e[q];
      }
      __syncthreads();
      for (int i = tid; i < (int)tn; i += NT) {
        const uint64_t x = sbuf[i];
        const uint32_t dd = 255u - (uint32_t)((x >> shift) & 255u);
        dst[gb[p * 256 + dd] + (uint32_t)i - ts[dd]] = x;
      }
      __syncthreads();
      if (tid < 256) gb[p * 256 + tid] += tc[tid];
      __syncthreads();
    }
    uint64_t* t = src;
    src = dst;
    dst = t;
  }
  if (src != a) {
    for (int64_t i = tid; i < n; i += NT) a[i] = src[i];
    __syncthreads();
  }
}

static_assert(BUFCAP >= NT * 8, "the append buffer holds a sort tile");
static_assert(2 * CAP >= 5888, "the candidate array holds the sort's counters");
static_assert(2 * CAP >= 2 * SEG_MAX + 2 + 256, "the weights array holds the segment import's tables");

// The dense path's candidates: every element with key >= theta, sorted
// (value desc, id asc) in dense_a. theta is the smaller of the KB-th
// largest key and, for large-k sampling, the relevance key; when at least
// KB elements reach the relevance key, the KB-th largest is among them and
// needs no selection pass. lds: 5,888 words; sbuf: NT * 8 entries.
template <int DT, bool PEN>
__device__ __forceinline__ int64_t dense_build(const SmpArgs& A, const RowCtx& rc, int row, uint32_t theta_rel,
                                               bool need_rel, int KB, uint32_t* lds, uint64_t* sbuf) {
  const int V = A.V;
  uint64_t* da = A.dense_a + (int64_t)row * A.dense_ld;
  uint64_t* db = A.dense_b + (int64_t)row * A.dense_ld;
  int64_t n = 0;
  if (need_rel) n = dense_compact<DT, PEN>(rc, V, theta_rel < 1u ? 1u : theta_rel, da, lds);
  if (!need_rel || n < (int64_t)KB) {
    uint32_t theta = radix_kth_key<DT, PEN>(rc, V, KB, lds, lds + 256);
    if (need_rel && theta_rel < theta) theta = theta_rel;
    if (theta < 1u) theta = 1u;
    n = dense_compact<DT, PEN>(rc, V, theta, da, lds);
  }
  lsd_sort_desc(da, db, n, lds, sbuf);
  return n;
}

// ---------------------------------------------------------------------------
// Shared per-row set-up of both kernels.
// ---------------------------------------------------------------------------
template <bool PEN>
__device__ __forceinline__ RowCtx make_rowctx(const SmpArgs& A, const DevParams& P, int row,
                                              int dtype_bytes, uint32_t* flags) {
  RowCtx rc;
  rc.base = (const char*)A.logits + (int64_t)row * A.ld * dtype_bytes;
  rc.acc = nullptr;
  rc.accw = nullptr;
  rc.tau = nullptr;
  rc.us = 0.0f;
  rc.r = 0.0f;
  rc.lout = nullptr;
  rc.loutw = nullptr;
  if (A.head_tau) {
    // inverse RMS of the row: the stored block sums folded from +0, divided
    // by the width, plus epsilon, then 1 / sqrt_rn (residual_norm_mlp.rs:
    // 37-46; portable_math.rs:108-111); every stage must stay finite
    const float* S = A.head_sums + (int64_t)row * A.head_nblk;
    float tot = 0.0f;
    for (int b = 0; b < A.head_nblk; ++b) tot = __fadd_rn(tot, S[b]);
    const float arg = __fadd_rn(__fdiv_rn(tot, A.head_width), A.head_eps);
    const float r = rsqrt_rn_f32(arg);
    if (nonfinite_bits(__float_as_uint(tot)) || nonfinite_bits(__float_as_uint(arg)) ||
        nonfinite_bits(__float_as_uint(r)))
      *flags |= F_NONFINITE;
    rc.acc = (const int64_t*)rc.base;
    if (A.head_clear) rc.accw = (int64_t*)rc.base;
    rc.tau = A.head_tau;
    rc.us = A.head_us[row];
    rc.r = r;
    if (A.head_out) {
      rc.loutw = A.head_out + (int64_t)row * A.head_out_ld;
      rc.lout = rc.loutw;
    }
  }
  rc.pw = nullptr;
  rc.pcnt = nullptr;
  rc.rep = P.rep;
  rc.pres = P.pres;
  rc.freq = P.freq;
  if (PEN && P.penalize) {
    if (A.pen_len[row] < 0) {
      *flags |= F_INVALID;
    } else {
      rc.pw = A.pen_words + (int64_t)row * A.pw_ld;
      rc.pcnt = A.pen_cnt + (int64_t)row * HCAP;
    }
  }
  return rc;
}

// Order-preserving final threshold of a row: a block or wave with bounds
// (m, kb) keeps key >= threshold(m, kb); the threshold never decreases as
// the bounds grow, so bounds seen early give supersets of the final set.
__device__ __forceinline__ uint32_t row_threshold(const RowPlan& plan, const DevParams& P,
                                                  float m, uint32_t kb) {
  uint32_t t = kb;
  if (plan.need_rel) {
    const uint32_t tr = relevance_key(m, P.temperature);
    t = tr < t ? tr : t;
  }
  return t < 1u ? 1u : t;
}

// ---------------------------------------------------------------------------
// Descending bitonic sort of n <= CAP packed candidates held in LDS `a`.
// Element i = r * NT + tid lives in register v[r] of its thread. A
// compare-exchange stage with partner distance j runs through wave shuffles
// for j < 64, inside a thread's registers for j >= NT, and through LDS (two
// barriers) only for 64 <= j < NT.
// ---------------------------------------------------------------------------
__device__ __forceinline__ uint64_t cx_pick(uint64_t mine, uint64_t other, uint32_t i, uint32_t j,
                                            uint32_t k) {
  // descending network: the lower index of a pair in a "descending" block
  // (i & k == 0) keeps the larger value
  const bool take_max = ((i & j) == 0) == ((i & k) == 0);
  return take_max ? (mine > other ? mine : other) : (mine < other ? mine : other);
}

__device__ void sort_desc(uint64_t* a, int n) {
  const int tid = threadIdx.x;
  int n2 = NT;
  while (n2 < n) n2 <<= 1;
  const int R = n2 / NT;  // 1..8
  uint64_t v[CAP / NT];
#pragma unroll
  for (int r = 0; r < CAP / NT; ++r) {
    const int i = r * NT + tid;
    v[r] = (r < R && i < n) ? a[i] : 0ull;
  }
  for (int k = 2; k <= n2; k <<= 1) {
    for (int j = k >> 1; j > 0; j >>= 1) {
      if (j >= NT) {
        const int jr = j / NT;
#pragma unroll
        for (int r = 0; r < CAP / NT; ++r) {
          // pairs (r, r ^ jr) inside the thread; handle each pair once
#pragma unroll
          for (int q = 1; q < CAP / NT; q <<= 1) {
            if (q == jr && r < R && (r & q) == 0) {
              const uint32_t i = (uint32_t)(r * NT + tid);
              const uint64_t lo = v[r], hi = v[r | q];
              v[r] = cx_pick(lo, hi, i, (uint32_t)j, (uint32_t)k);
              v[r | q] = cx_pick(hi, lo, i + (uint32_t)j, (uint32_t)j, (uint32_t)k);
            }
          }
        }
      } else if (j >= 64) {
        __syncthreads();
#pragma unroll
        for (int r = 0; r < CAP / NT; ++r)
          if (r < R) a[r * NT + tid] = v[r];
        __syncthreads();
#pragma unroll
        for (int r = 0; r < CAP / NT; ++r) {
          if (r < R) {
            const uint32_t i = (uint32_t)(r * NT + tid);
            v[r] = cx_pick(v[r], a[i ^ (uint32_t)j], i, (uint32_t)j, (uint32_t)k);
          }
        }
      } else {
#pragma unroll
        for (int r = 0; r < CAP / NT; ++r) {
          if (r < R) {
            const uint32_t i = (uint32_t)(r * NT + tid);
            v[r] = cx_pick(v[r], __shfl_xor(v[r], j), i, (uint32_t)j, (uint32_t)k);
          }
        }
      }
    }
  }
  __syncthreads();
#pragma unroll
  for (int r = 0; r < CAP / NT; ++r)
    if (r < R) a[r * NT + tid] = v[r];
  __syncthreads();
}

// Descending sort of n <= 512 packed candidates in LDS `a` (distinct
// values), `b` is LDS scratch of n entries. n <= 64: one wave sorts in
// registers. Otherwise each wave sorts a 64-element run in registers and
// every element's final position is its position in its run plus, for each
// other run, the number of larger elements there (binary search).
__device__ __forceinline__ uint64_t wave_sort_desc_u64(uint64_t v) {
  const uint32_t lane = threadIdx.x & 63;
#pragma unroll
  for (int size = 2; size <= 64; size <<= 1) {
#pragma unroll
    for (int j = size >> 1; j > 0; j >>= 1) v = cx_pick(v, __shfl_xor(v, j), lane, (uint32_t)j, (uint32_t)size);
  }
  return v;
}

__device__ void sort_desc_small(uint64_t* a, uint64_t* b, int n) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  if (n <= 64) {
    if (wave == 0) {
      const uint64_t v = wave_sort_desc_u64(lane < n ? a[lane] : 0ull);
      if (lane < n) a[lane] = v;
    }
    __syncthreads();
    return;
  }
  const int runs = (n + 63) / 64;
  uint64_t v = 0ull;
  if (wave < runs) {
    v = wave_sort_desc_u64(tid < n ? a[tid] : 0ull);
    a[tid] = v;  // run `wave`, descending, zeros (absent) last
  }
  __syncthreads();
  if (wave < runs && v != 0ull) {
    int rank = lane;
    for (int w = 0; w < runs; ++w) {
      if (w == wave) continue;
      const uint64_t* run = a + w * 64;
      int lo = 0, hi = 64;  // first position whose value is below v
      while (lo < hi) {
        const int mid = (lo + hi) >> 1;
        if (run[mid] > v) lo = mid + 1; else hi = mid;
      }
      rank += lo;
    }
    b[rank] = v;
  }
  __syncthreads();
  for (int i = tid; i < n; i += NT) a[i] = b[i];
  __syncthreads();
}

// Descending sort of NT < n <= 2 NT packed candidates in LDS `a` (distinct
// values, nonzero), `b` LDS scratch of n entries: each wave sorts two
// 64-element runs in registers, and every element's final position is its
// position in its run plus, for each other run, the number of larger
// elements there (binary search), as in sort_desc_small.
__device__ void sort_desc_runs2(uint64_t* a, uint64_t* b, int n) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int runs = (n + 63) / 64;  // 9..16
  uint64_t v[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int run = wave + h * NW;
    const int i = run * 64 + lane;
    v[h] = 0ull;
    if (run < runs) {
      v[h] = wave_sort_desc_u64(i < n ? a[i] : 0ull);
      a[i] = v[h];  // run `run`, descending, zeros (absent) last
    }
  }
  __syncthreads();
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int run = wave + h * NW;
    if (run < runs && v[h] != 0ull) {
      int rank = lane;
      for (int w = 0; w < runs; ++w) {
        if (w == run) continue;
        const uint64_t* r = a + w * 64;
        int lo = 0, hi = 64;  // first position whose value is below v
        while (lo < hi) {
          const int mid = (lo + hi) >> 1;
          if (r[mid] > v[h]) lo = mid + 1; else hi = mid;
        }
        rank += lo;
      }
      b[rank] = v[h];
    }
  }
  __syncthreads();
  for (int i = tid; i < n; i += NT) a[i] = b[i];
  __syncthreads();
}

// The exact k-th largest key among n >= k packed entries in LDS: four 8-bit
// radix passes from the top. Each wave adds its lanes' digits with one LDS
// atomic per distinct digit (ballot-matched peers), and every wave picks the
// next digit from the histogram itself, so a pass costs one barrier; the
// three histograms rotate (hist: 768 LDS words), the one of pass p - 1
// cleared after pass p's barrier. Block-wide; every thread returns the key.
__device__ uint32_t lds_kth_key(const uint64_t* buf, uint32_t n, uint32_t k, uint32_t* hist) {
  const int tid = threadIdx.x, lane = tid & 63;
  for (int i = tid; i < 3 * 256; i += NT) hist[i] = 0u;
  __syncthreads();
  uint32_t prefix = 0u, mask = 0u, need = k;
  for (int pass = 0; pass < 4; ++pass) {
    const int shift = 24 - 8 * pass;
    uint32_t* const h = hist + (pass % 3) * 256;
    for (uint32_t i0 = 0; i0 < n; i0 += NT) {
      const uint32_t i = i0 + (uint32_t)tid;
      const uint32_t kk = i < n ? pk_key(buf[i]) : 0u;
      hist_add8(h, (kk >> shift) & 255u, i < n && (kk & mask) == prefix);
    }
    __syncthreads();
    // (the histogram of pass 0 serves again in pass 3)
    if (pass == 1)
      for (int i = tid; i < 256; i += NT) hist[i] = 0u;
    uint32_t hq[4], own = 0u;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      hq[q] = h[4 * lane + q];
      own += hq[q];
    }
    // suffix sum: entries in the bins of this lane and every higher lane
    uint32_t suf = own;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const uint32_t t = __shfl_down(suf, o);
      if (lane + o < 64) suf += t;
    }
    const uint64_t reach = __ballot(suf >= need);
    uint32_t dsel = 0u, nn = 1u;  // (fewer than k entries: the caller does not ask for that)
    if (reach) {
      const int L = 63 - __builtin_clzll(reach);  // the highest lane still holding the k-th
      uint32_t cum = suf - own;                     // entries in higher lanes' bins
      uint32_t d = 4u * (uint32_t)lane;
#pragma unroll
      for (int q = 3; q >= 0; --q) {
        if (cum + hq[q] >= need) {
          d = 4u * (uint32_t)lane + (uint32_t)q;
          break;
        }
        cum += hq[q];
      }
      dsel = (uint32_t)__builtin_amdgcn_readlane((int)d, L);
      nn = (uint32_t)__builtin_amdgcn_readlane((int)(need - cum), L);
    }
    prefix |= dsel << shift;
    mask |= 255u << shift;
    need = nn;
  }
  return prefix;
}

// ---------------------------------------------------------------------------
// LDS of a row block (136 KB in all with the small arrays: one block per CU).
// ---------------------------------------------------------------------------
struct RowLds {
  uint64_t buf[BUFCAP];    // append buffer of candidates (unordered)
  uint64_t cand[CAP];      // the candidates that pass the final bounds, sorted
  double w[CAP];           // weights of the tail; scratch of the sorts
  uint4 def[DEFCAP];           // deferred chunks: (chunk, largest key, second key, id of the largest)
  uint32_t lists[NW * 8];      // each wave's 8 largest list entries, after the stream
};

// Raw bits of chunk c (2,048 logits) of a row into kb; nothing for c >= nch.
// Element (q, j) of this lane is eb + q * 64 * GRP + j.
// For element type 2, `first` marks the chunk's first read: the head logits
// are formed from the accumulators, written out and the accumulators
// cleared when asked; later reads use the written logits (raw_bits).
template <int DT, bool VEC>
__device__ __forceinline__ void load_chunk(const RowCtx& rc, int32_t V, int nch, int c, int lane,
                                           uint32_t (&kb)[EPT], bool first = true) {
  constexpr int GRP = (DT == 1) ? 8 : 4;
  constexpr int NGRP = EPT / GRP;
  if (c >= nch) return;
  const uint32_t w0 = (uint32_t)c * WSEG;
  const uint32_t eb = w0 + (uint32_t)lane * GRP;
  if (DT == 2) {
    const int32_t lim = V - (int32_t)eb;
#pragma unroll
    for (int q = 0; q < NGRP; ++q) {
#pragma unroll
      for (int j = 0; j < GRP; ++j) {
        const int32_t o = q * 64 * GRP + j;
        uint32_t b = 0u;
        if (o < lim) {
          const int64_t i = (int64_t)eb + o;
          if (first) {
            const float f = head_value(rc, i);
            if (rc.loutw) rc.loutw[i] = f;
            if (rc.accw) rc.accw[i] = 0;
            b = __float_as_uint(f);
          } else {
            b = raw_bits<DT>(rc, i);
          }
        }
        kb[q * GRP + j] = b;
      }
    }
    return;
  }
  if (VEC && w0 + WSEG <= (uint32_t)V) {
    const uint4* src = (const uint4*)(rc.base + (size_t)eb * (DT == 0 ? 4 : 2));
#pragma unroll
    for (int q = 0; q < NGRP; ++q) {
      const uint4 v = src[q * 64];
      if (DT == 0) {
        kb[q * 4 + 0] = v.x;
        kb[q * 4 + 1] = v.y;
        kb[q * 4 + 2] = v.z;
        kb[q * 4 + 3] = v.w;
      } else {
        kb[q * 8 + 0] = v.x << 16;
        kb[q * 8 + 1] = v.x & 0xffff0000u;
        kb[q * 8 + 2] = v.y << 16;
        kb[q * 8 + 3] = v.y & 0xffff0000u;
        kb[q * 8 + 4] = v.z << 16;
        kb[q * 8 + 5] = v.z & 0xffff0000u;
        kb[q * 8 + 6] = v.w << 16;
        kb[q * 8 + 7] = v.w & 0xffff0000u;
      }
    }
  } else {
    // offsets o of this lane lie inside the row iff o < lim (compared
    // against immediates: no per-element index registers)
    const int32_t lim = V - (int32_t)eb;
#pragma unroll
    for (int q = 0; q < NGRP; ++q) {
#pragma unroll
      for (int j = 0; j < GRP; ++j) {
        const int32_t o = q * 64 * GRP + j;
        kb[q * GRP + j] = o < lim ? raw_bits<DT>(rc, eb + (uint32_t)o) : 0u;
      }
    }
  }
}

// Raw bits of chunk c through 16-byte buffer loads, no guards: the caller
// ensures the row starts 16-byte aligned and that every 16-byte group of the
// chunk lies either wholly inside the row or wholly past its end (the
// ragged last chunk comes here only when the row length is a whole number of
// groups). The resource spans exactly the row: groups past its end are out
// of range and return zeros without touching memory (chunk_values ignores
// them). The loads take a uniform
// chunk offset in an SGPR and loop-invariant lane offsets in VGPRs, so the
// stream spends no vector instructions on addresses. With `live` false the
// same loads go through a resource of size 0: every one is out of range. Issuing the same loads on every path, and keeping address
// arithmetic out of the destination registers, lets the compiler wait for
// exactly the buffer it is about to read, with the other still in flight.
template <int DT>
__device__ __forceinline__ void load_full(const char* row_base, int32_t V, int c, bool live, int lane,
                                          uint32_t (&kb)[EPT]) {
  if (DT == 2) return;  // head rows are not streamed through buffer loads
  constexpr int GRP = (DT == 0) ? 4 : 8;
  constexpr int NGRP = EPT / GRP;
  const __amdgpu_buffer_rsrc_t rs =
      __builtin_amdgcn_make_buffer_rsrc((void*)row_base, (short)0, live ? V * (DT == 0 ? 4 : 2) : 0, 0x00020000);
  const int soff = live ? c * WSEG * (DT == 0 ? 4 : 2) : 0;
#pragma unroll
  for (int q = 0; q < NGRP; ++q) {
    const __attribute__((ext_vector_type(4))) uint32_t v =
        __builtin_amdgcn_raw_buffer_load_b128(rs, lane * 16 + (q & 3) * 1024, soff + (q >> 2) * 4096, 0);
    if (DT == 0) {
      kb[q * 4 + 0] = v.x;
      kb[q * 4 + 1] = v.y;
      kb[q * 4 + 2] = v.z;
      kb[q * 4 + 3] = v.w;
    } else {
      kb[q * 8 + 0] = v.x << 16;
      kb[q * 8 + 1] = v.x & 0xffff0000u;
      kb[q * 8 + 2] = v.y << 16;
      kb[q * 8 + 3] = v.y & 0xffff0000u;
      kb[q * 8 + 4] = v.z << 16;
      kb[q * 8 + 5] = v.z & 0xffff0000u;
      kb[q * 8 + 6] = v.w << 16;
      kb[q * 8 + 7] = v.w & 0xffff0000u;
    }
  }
}

// Chunk c's raw bits -> binary32 value bits in place (penalties applied,
// absent elements -inf); non-finite test and lane maximum.
template <int DT, bool PEN>
__device__ __forceinline__ void chunk_values(const RowCtx& rc, int32_t V, int c, int lane,
                                             uint32_t (&kb)[EPT], float& lmax, bool& bad) {
  constexpr int GRP = (DT == 1) ? 8 : 4;
  constexpr int NGRP = EPT / GRP;
  const uint32_t w0 = (uint32_t)c * WSEG;
  const uint32_t eb = w0 + (uint32_t)lane * GRP;
  if (!PEN && w0 + WSEG <= (uint32_t)V) {
    // a full chunk without penalties: the raw bits are the values
#pragma unroll
    for (int i = 0; i < EPT; ++i) {
      const float v = __uint_as_float(kb[i]);
      bad |= __builtin_amdgcn_class(v, 0x207) != 0;  // signaling/quiet NaN, +-inf
      lmax = fmaxf(lmax, v);
    }
    return;
  }
  const bool full = w0 + WSEG <= (uint32_t)V;
  const int32_t lim = V - (int32_t)eb;
#pragma unroll
  for (int q = 0; q < NGRP; ++q) {
    uint2 pw = make_uint2(0u, 0u);
    if (PEN && rc.pw && q * 64 * GRP < lim) pw = rc.pw[(eb + q * 64 * GRP) >> 5];
#pragma unroll
    for (int j = 0; j < GRP; ++j) {
      const int32_t o = q * 64 * GRP + j;
      uint32_t b = kb[q * GRP + j];
      float v = -__builtin_inff();
      if (full || o < lim) {
        if (PEN && rc.pw && ((pw.x >> ((eb + o) & 31)) & 1u)) {
          b = penalize(b, pen_count(rc, pw, eb + (uint32_t)o), rc);
        }
        v = __uint_as_float(b);
        bad |= __builtin_amdgcn_class(v, 0x207) != 0;  // signaling/quiet NaN, +-inf
      }
      kb[q * GRP + j] = __float_as_uint(v);
      lmax = fmaxf(lmax, v);
    }
  }
}

// The first NSTASH deferred chunks keep their converted values in LDS, in
// the candidate and weight arrays (unused until the finish): their second
// pass reads LDS instead of memory. Slot s holds lane l's values
// 4q .. 4q + 3 at uint4 s * 512 + q * 64 + l.
constexpr uint32_t NSTASH = (CAP * 16) / (WSEG * 4);
__device__ __forceinline__ void stash_chunk(RowLds& fl, uint32_t s, int lane, const uint32_t (&kb)[EPT]) {
  lds_u4* S = (lds_u4*)fl.cand + s * 512u + (uint32_t)lane;
#pragma unroll
  for (int q = 0; q < EPT / 4; ++q) {
    u32x4 v;
    v.x = kb[4 * q];
    v.y = kb[4 * q + 1];
    v.z = kb[4 * q + 2];
    v.w = kb[4 * q + 3];
    S[q * 64] = v;
  }
}
__device__ __forceinline__ void unstash_chunk(RowLds& fl, uint32_t s, int lane, uint32_t (&kb)[EPT]) {
  const lds_u4* S = (const lds_u4*)fl.cand + s * 512u + (uint32_t)lane;
#pragma unroll
  for (int q = 0; q < EPT / 4; ++q) {
    const u32x4 v = S[q * 64];
    kb[4 * q] = v.x;
    kb[4 * q + 1] = v.y;
    kb[4 * q + 2] = v.z;
    kb[4 * q + 3] = v.w;
  }
}

// Per-wave streaming state.
struct WaveState {
  uint32_t wkey;    // largest key this wave has seen (uniform)
  float m_ref;      // reference point of the wave's logprob mass (uniform)
  double acc;       // per lane: sum of exp(l - m_ref) over l >= m_ref - ZMASS
  bool bad;         // per lane: a non-finite value was seen
  uint32_t spill_cap;  // slots of the row's spill area
};

// Shared streaming state of a row block.
// The bounds the waves share sit in one array so that a wave reads all of
// them with a single LDS load (lane i reads word i).
constexpr int BW_THETA = 0;       // best top-KB bound any wave has certified
constexpr int BW_Q = 1;           // BW_Q + w: wave w's ceil(KB/8)-th list value
constexpr int BW_MKEY = 1 + NW;   // running row maximum key
constexpr int BW_N = 2 + NW;
static_assert(BW_N <= 16, "the shared bounds are read by the lanes of one DPP row");

struct RowShared {
  uint32_t count;      // entries appended (beyond BUFCAP they went to the spill area)
  uint32_t flags;      // F_* of the row
  uint32_t bw[BW_N];   // shared bounds (BW_*)
  uint32_t ndef;       // deferred chunks recorded (may exceed DEFCAP: those were not deferred)
  uint32_t ctr;        // compaction counter
  uint32_t next;       // next chunk of the stream not yet claimed by a wave
};

// The element pass of chunk_filter: mass terms of the values >= lo, and
// the values >= thf (when keep) appended in order from slot slot0. With
// SPILL the slots reach past BUFCAP: those go to the row's spill area
// (dropped past its end, which sends the row to the dense path). The
// common chunk takes the LDS-only copy, which holds no global store.
template <int GRP, int NGRP, bool SPILL>
__device__ __forceinline__ void chunk_pass(const uint32_t (&kb)[EPT], const float (&gmax)[NGRP], float tany,
                                           float lo, float thf, bool keep, uint32_t eb, uint32_t slot0,
                                           WaveState& ws, RowLds& fl, uint64_t* spill) {
  uint32_t cur = slot0;
  const bool mass = lo != __builtin_inff();
#pragma unroll
  for (int q = 0; q < NGRP; ++q) {
    if (!__ballot(gmax[q] >= tany)) continue;
    if (mass) {
      // the group's mass terms, independent of one another (no branch, no
      // serial chain through the accumulator): a binary64 pairwise sum,
      // then one add to the lane's accumulator
      double t[GRP];
#pragma unroll
      for (int j = 0; j < GRP; ++j) {
        const float v = __uint_as_float(kb[q * GRP + j]);
        const float e = __builtin_amdgcn_exp2f((v - ws.m_ref) * 1.4426950408889634f);
        t[j] = v >= lo ? (double)e : 0.0;
      }
#pragma unroll
      for (int h = GRP / 2; h > 0; h >>= 1) {
#pragma unroll
        for (int j = 0; j < h; ++j) t[j] = t[j] + t[j + h];
      }
      ws.acc += t[0];
    }
    if (!keep) continue;
#pragma unroll
    for (int j = 0; j < GRP; ++j) {
      const float v = __uint_as_float(kb[q * GRP + j]);
      const bool k = v >= thf;
      const uint64_t km = __ballot(k);
      if (!km) continue;
      const uint32_t slot = cur + lanes_below(km);
      if (k) {
        const uint64_t e = pack(f2key(__float_as_uint(v)), eb + (uint32_t)(q * 64 * GRP + j));
        if (!SPILL || slot < (uint32_t)BUFCAP) {
          ((lds_u64*)fl.buf)[slot] = e;
        } else if (slot - (uint32_t)BUFCAP < ws.spill_cap) {
          __builtin_nontemporal_store(e, &((global_u64*)spill)[slot - BUFCAP]);
        }
      }
      cur += (uint32_t)__popcll(km);
    }
  }
}

// Mass terms (if mass) and candidates of chunk c for threshold thr. Work is
// skipped per chunk (its maximum), then per load group (GRP consecutive
// values of a lane), then per element slot, wherever no lane holds a value
// >= min(threshold, m_ref - ZMASS); the chunk's survivors are counted first
// and reserve their slots with one LDS atomic (the buffer has no holes).
// Mass terms are binary32
// exponentials accumulated in binary64: next to the row maximum's term (1.0)
// the small terms must not be rounded away, since the top token's logprob is
// -log(1 + their sum). Slots beyond BUFCAP go to the row's spill area in
// global memory (each element is appended at most once, so V entries always
// suffice); that rare path ends with a full wait, so the common path holds
// only LDS stores and the compiler can keep the prefetched chunk in flight.
// A chunk where more than defer_lanes lanes hold survivors (the running
// bounds are still low; 64: never) is deferred instead: recorded with its largest key and read again at the
// end, and only if that key reaches the final bound.
template <int DT>
__device__ __forceinline__ void chunk_filter(int c, int lane, const uint32_t (&kb)[EPT], uint32_t thr,
                                             uint32_t mk, bool mass, uint32_t lk, uint32_t cmax, int defer_lanes,
                                             WaveState& ws, RowShared& sh, RowLds& fl, uint64_t* spill) {
  constexpr int GRP = (DT == 1) ? 8 : 4;
  constexpr int NGRP = EPT / GRP;
  if (mk == 0u) return;  // nothing finite seen yet: the row is rejected anyway
  const float thf = key_threshold_float(thr);
  float lo = __builtin_inff();
  if (mass) {
    const float Mt = key2f(mk);
    if (Mt > ws.m_ref) {
      if (ws.m_ref != -__builtin_inff()) ws.acc *= exp((double)ws.m_ref - (double)Mt);
      ws.m_ref = Mt;
    }
    lo = ws.m_ref - ZMASS;
  }
  float tany = fminf(thf, lo);
  // nothing in the chunk reaches the lower of the two cuts: no work at all
  // (lk: this lane's largest key, 0 for none; cmax: the chunk's, 0 if not
  // known yet)
  const float lkf = lk == 0u ? -__builtin_inff() : key2f(lk);
  if (!__ballot(lkf >= tany)) return;
  float gmax[NGRP];
  float lmax = -__builtin_inff();
#pragma unroll
  for (int q = 0; q < NGRP; ++q) {
    float g = __uint_as_float(kb[q * GRP]);
#pragma unroll
    for (int j = 1; j < GRP; ++j) g = fmaxf(g, __uint_as_float(kb[q * GRP + j]));
    gmax[q] = g;
    lmax = fmaxf(lmax, g);
  }
  bool keep_any = true;
  if (defer_lanes < 64 && __popcll(__ballot(lmax >= thf)) > defer_lanes) {
    uint32_t idx = 0;
    if (lane == 0) idx = atomicAdd(&sh.ndef, 1u);
    idx = (uint32_t)__builtin_amdgcn_readfirstlane((int)idx);
    if (idx < (uint32_t)DEFCAP) {
      if (cmax == 0u) cmax = wave_max_dpp(lk);
      // The chunk's two largest keys and the id of the largest: after the
      // stream it is read again only if the second reaches the final bound
      // (when only the largest does, that one element is appended then).
      // Per lane: its largest value, where it is, and its second (a value
      // equal to the largest counts as the second).
      float m1 = -__builtin_inff(), m2 = -__builtin_inff();
      int p1 = 0;
#pragma unroll
      for (int e = 0; e < EPT; ++e) {
        const float v = __uint_as_float(kb[e]);
        const bool up = v > m1;
        m2 = up ? m1 : fmaxf(m2, v);
        p1 = up ? e : p1;
        m1 = up ? v : m1;
      }
      const int L = (int)__builtin_ctzll(__ballot(lk == cmax));  // a lane holding the chunk maximum
      const uint32_t k2 = m2 == -__builtin_inff() ? 0u : f2key(__float_as_uint(m2));
      const uint32_t sec = wave_max_dpp(lane == L ? k2 : lk);
      const uint32_t pos = (uint32_t)(c * WSEG + lane * GRP + (p1 / GRP) * 64 * GRP + p1 % GRP);
      const uint32_t id1 = (uint32_t)__builtin_amdgcn_readlane((int)pos, L);
      // (chunk, stash slot + 1 or 0) in the record's first word
      uint32_t code = (uint32_t)c;
      if (idx < NSTASH) {
        stash_chunk(fl, idx, lane, kb);
        code |= (idx + 1u) << 16;
      }
      if (lane == 0) fl.def[idx] = make_uint4(code, cmax, sec, id1);
      keep_any = false;
      tany = lo;
      if (!(key2f(cmax) >= tany)) return;
    }
  }
  const uint32_t eb = (uint32_t)c * WSEG + (uint32_t)lane * GRP;
  uint32_t base = 0u, total = 0u;
  if (keep_any) {
#pragma unroll
    for (int q = 0; q < NGRP; ++q) {
      if (!__ballot(gmax[q] >= thf)) continue;
#pragma unroll
      for (int j = 0; j < GRP; ++j) total += (uint32_t)__popcll(__ballot(__uint_as_float(kb[q * GRP + j]) >= thf));
    }
    if (total) {
      if (lane == 0) base = atomicAdd(&sh.count, total);
      base = (uint32_t)__builtin_amdgcn_readfirstlane((int)base);
    }
  }
  if (base + total <= (uint32_t)BUFCAP) {
    chunk_pass<GRP, NGRP, false>(kb, gmax, tany, lo, thf, keep_any, eb, base, ws, fl, spill);
  } else {
    chunk_pass<GRP, NGRP, true>(kb, gmax, tany, lo, thf, keep_any, eb, base, ws, fl, spill);
    // the rare spill stores end with a full wait, so the common path holds
    // only LDS stores and the compiler keeps the prefetched chunk in flight
    __builtin_amdgcn_s_waitcnt(0);
  }
}

// Order-free parallel compaction: appends to dst the entries of src[0, n)
// with key >= thr, at most cap in all; *ctr counts every qualifying entry
// (reset first if `reset`). Returns *ctr (every thread). With STOP a wave
// stops once the count has passed cap (the caller only needs to know that
// it did; the count returned is then some value above cap). Block-wide.
template <bool STOP = false>
__device__ __forceinline__ uint32_t compact_entries(const uint64_t* src, uint32_t n, uint64_t* dst,
                                                    uint32_t cap, uint32_t thr, uint32_t* ctr, bool reset) {
  const int tid = threadIdx.x, lane = tid & 63;
  if (reset) {
    __syncthreads();
    if (tid == 0) *ctr = 0u;
  }
  __syncthreads();
  for (uint32_t i0 = 0; i0 < n; i0 += NT) {
    if (STOP && __builtin_amdgcn_readfirstlane(
                    (int)__hip_atomic_load(ctr, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP)) > (int)cap)
      break;
    const uint32_t i = i0 + (uint32_t)tid;
    uint64_t e = 0;
    bool keep = false;
    if (i < n) {
      e = src[i];
      keep = pk_key(e) >= thr;
    }
    const uint64_t m = __ballot(keep);
    if (m) {
      const int first = (int)__builtin_ctzll(m);
      uint32_t base = 0;
      if (lane == first) base = atomicAdd(ctr, (uint32_t)__popcll(m));
      base = (uint32_t)__builtin_amdgcn_readlane((int)base, first);
      const uint32_t slot = base + lanes_below(m);
      if (keep && slot < cap) dst[slot] = e;
    }
  }
  __syncthreads();
  const uint32_t r = *ctr;
  __syncthreads();
  return r;
}

// ---------------------------------------------------------------------------
// The tail of a large-candidate row without sorting the row (top-k disabled
// or above the relevant count, version 3, lists of at most KBMAX entries).
//
// The reference sorts the candidates, forms w_j = exp_d(z_j), cuts at the
// first serial binary64 prefix S_j >= top_p * total and at the first w_j
// below min-p, and draws over the kept prefix (output_head_sampler.rs
// :136-190). Only the cut needs the order, and only near it:
//  1. every relevant weight, and a count, is added into one of CB_NB buckets
//     of an absolute grid of the values (grid_bucket: an interval of the
//     candidate order each). A segmented row's blocks add their shares
//     before they hand over (cert_share: weights relative to the segment's
//     maximum, buckets relative to its grid cell); the finishing block
//     shifts and scales them into place. Otherwise the finishing block reads
//     the row once for this;
//  2. a second pass collects the bucket in which the running bucket sums
//     cross top_p * total, the buckets that hold the first KB candidates
//     (the lists) and the bucket that holds the min-p threshold, finds the
//     largest key below that bucket, and writes out the entries kept
//     whichever cut holds (those before both buckets); the cut and head
//     collections are sorted in LDS;
//  3. the sums are not the reference's serial binary64 sum: other order,
//     weights from exp_approx (within 2^-46 relative) of z' = (l - M) * (1 / T)
//     or of the segment's (l - Ms) * (1 / T) times exp_approx((Ms - M) * (1 / T))
//     instead of exp_d of z = (l - M) / T: within 2^-43 of w each for
//     |z| <= 40. Every prefix or total formed here is within
//     E = 2^-53 R (4n + 2 CB_NB + 2 CAP + 64) + 2^-42 R
//     of the serial value it stands for (R the total, n the counted
//     elements: each serial addition, each bucket, merge and scan addition,
//     each addition of the walk through the collected bucket and the top-p
//     product round by at most 2^-53 R; the weights add at most 2^-43 R). A
//     cut is taken only when every compare it rests on holds with a margin
//     of 2E, and min-p's only when no weight of the threshold bucket lies
//     within 2^-40 (relative) of min-p and the threshold is not within 10^-6
//     grid steps of a bucket edge (every weight outside that bucket is then
//     at least 9e-9 away from min-p, relative); otherwise, or when a
//     collection does not fit, the function returns 0 and the caller sorts
//     the row (the exact path);
//  4. the kept candidates are a prefix of the order: the second pass writes
//     out those before the collected buckets, the sorted cut bucket (top-p
//     cut) or the threshold bucket (min-p cut) adds its part. A draw takes
//     the largest binary32 score (within SC_TOL of z + g, score_approx)
//     over them, then the exact binary64 z + g of the entries within
//     2 SC_TOL of it, ties to the earlier candidate (the reference's strict
//     > in candidate order).
// Passes over the row keep the next tile's loads in flight while a tile is
// processed. The total is also summed in a second order; a difference
// beyond the bound fails the certification too. On success fl.cand holds
// the first KB candidates, sorted, out_ids the draws, and the return value
// is the number of counted elements. Block-wide.
// ---------------------------------------------------------------------------
constexpr int CB_NB = 4096;       // buckets of the certified tail
constexpr float SC_TOL = 1e-4f;   // bound on |score_approx - (z + g)|
constexpr int DRB = 8;            // entries per thread and round of the draw passes
constexpr int BCAP = 2016;        // entries of the min-p threshold bucket kept in LDS
constexpr int64_t CSLOT = CB_NB + CB_NB / 2 + 8;  // doubles of a segment's share in the row's scratch
static_assert(CB_NB % NT == 0, "bucket array in whole rounds of the block");

// Bucket of value l on the absolute grid of step 1/c: F(M) - F(l) with
// F(x) = floor(x c) (fm = F(M)), the values CB_NB - 1 or more steps below in
// the last bucket (a NaN too). With c = CB_NB / (37.5 T) every relevant value
// lands in 0..CB_NB - 1; the bucket does not decrease along the candidate
// order, and a segment's bucket relative to its own F(Ms) is this one shifted
// by F(M) - F(Ms).
__device__ __forceinline__ uint32_t grid_bucket(double fm, double l, double c) {
  const double t = fm - floor(l * c);  // >= 0: no value exceeds the maximum
  return t < (double)(CB_NB - 1) ? (t > 0.0 ? (uint32_t)t : 0u) : (uint32_t)(CB_NB - 1);
}

// Entries j0 + q * NT + tid of the compacted kept set (clamped: all DRB
// loads issued together).
__device__ __forceinline__ void draw_load(const uint64_t* da, int64_t nk, int64_t j0, uint64_t (&v)[DRB]) {
#pragma unroll
  for (int q = 0; q < DRB; ++q) {
    const int64_t j = j0 + (int64_t)q * NT + (int64_t)threadIdx.x;
    v[q] = da[j < nk ? j : nk - 1];
  }
}

struct CertShared {
  double R;            // sum of the bucket sums
  double a_cut;        // bucket sums before the cut bucket
  double a_star;       // bucket sums before the min-p threshold bucket
  double p_lo, p_hi;   // prefix before and through the cut candidate
  uint32_t n;          // counted elements
  uint32_t bcut, ccut; // cut bucket, elements before it
  uint32_t btop, ctop; // last bucket of the head, elements through it
  uint32_t ncut, ntop; // entries collected
  uint32_t nb;         // entries of the threshold bucket collected
  uint32_t nk;         // kept entries written
  int32_t j0;          // cut position in the sorted cut bucket (-1: not found)
  uint32_t kb[6];      // key bounds of the second pass (lower_key)
};

// The smallest key in [lo, f2key(+inf)] whose value lies in bucket x or a
// lower one. Over non-NaN values the bucket does not increase with the key
// (grid_bucket is F(M) - floor(l c), clamped), so the keys of buckets <= x
// are exactly those at or above this one; +inf is in bucket 0.
__device__ __forceinline__ uint32_t lower_key(double fm, double c, uint32_t x, uint32_t lo) {
  uint32_t hi = 0xff800000u;  // f2key(+inf)
  while (lo < hi) {
    const uint32_t mid = lo + (hi - lo) / 2u;
    if (grid_bucket(fm, (double)key2f(mid), c) <= x) hi = mid;
    else lo = mid + 1u;
  }
  return lo;
}

// Raw bits of elements base + q * NT + tid. Every load is issued, at a
// clamped index, so that all PER are in flight together (a load behind a
// per-element branch waits for the one before it); the bits are turned into
// keys only where they are used (cert_keys), so that the loads of the next
// tile stay in flight while a tile is processed.
template <int DT, bool PEN, int PER>
__device__ __forceinline__ void cert_load(const RowCtx& rc, int64_t V, int64_t base, uint32_t (&b)[PER]) {
#pragma unroll
  for (int q = 0; q < PER; ++q) {
    const int64_t i = base + (int64_t)q * NT + (int64_t)threadIdx.x;
    b[q] = value_bits<DT, PEN>(rc, i < V ? i : V - 1);
  }
}
// Keys of those elements (0 past the end).
template <int PER>
__device__ __forceinline__ void cert_keys(int64_t V, int64_t base, const uint32_t (&b)[PER], uint32_t (&k)[PER]) {
#pragma unroll
  for (int q = 0; q < PER; ++q) {
    const int64_t i = base + (int64_t)q * NT + (int64_t)threadIdx.x;
    k[q] = i < V ? f2key(b[q]) : 0u;
  }
}

// Step 1 over elements [e0, e1) with weights relative to maximum Mw and
// buckets relative to fw = F(Mw), relevant = key >= trel, into hw / hc
// (LDS, cleared here). Returns the thread's sum of the weights.
template <int DT, bool PEN>
__device__ __forceinline__ double cert_pass1(const RowCtx& rc, int64_t e0, int64_t e1, float Mw, double fw, double c,
                                             double invT, uint32_t trel, double* hw, uint32_t* hc) {
  constexpr int P1 = 8;
  const int tid = threadIdx.x;
  for (int i = tid; i < CB_NB; i += NT) {
    hw[i] = 0.0;
    hc[i] = 0u;
  }
  __syncthreads();
  const double Mwd = (double)Mw;
  double ws = 0.0;
  uint32_t nx[P1];
  cert_load<DT, PEN, P1>(rc, e1, e0, nx);
  for (int64_t base = e0; base < e1; base += (int64_t)NT * P1) {
    uint32_t kk[P1];
    cert_keys<P1>(e1, base, nx, kk);
    if (base + (int64_t)NT * P1 < e1) cert_load<DT, PEN, P1>(rc, e1, base + (int64_t)NT * P1, nx);
    // every element's weight and bucket first, outside the branches, so
    // that the elements' dependent chains interleave
    double wv[P1];
    uint32_t bv[P1];
#pragma unroll
    for (int q = 0; q < P1; ++q) {
      const double l = (double)key2f(kk[q]);
      wv[q] = exp_approx((l - Mwd) * invT);
      bv[q] = grid_bucket(fw, l, c);
      ws += kk[q] >= trel ? wv[q] : 0.0;
    }
#pragma unroll
    for (int q = 0; q < P1; ++q) {
      if (kk[q] >= trel) {
        atomicAdd(&hw[bv[q]], wv[q]);
        atomicAdd(&hc[bv[q]], 1u);
      }
    }
  }
  __syncthreads();
  return ws;
}

// A segment of a row headed for the certified tail (its export overflowed)
// adds its share of step 1 before it hands over: its elements relevant to
// its own maximum Ms (a superset of the row's relevant ones: the extra ones
// lie CB_NB - 1 or more grid steps below M, in the last bucket), weights
// relative to Ms, buckets relative to F(Ms), into its slot of the row's
// scratch. Returns false, writing nothing, when the slot does not fit the
// scratch or the grid is too fine for exact integer steps. Block-wide.
template <int DT, bool PEN>
__device__ __forceinline__ bool cert_share(const SmpArgs& A, const DevParams& P, const RowCtx& rc, int row, int seg,
                                           int nseg, float Ms, int64_t e0, int64_t e1, RowLds& fl, double* redd) {
  const double T = P.temperature, invT = 1.0 / T, c = (double)CB_NB / (37.5 * T);
  const double msc = (double)Ms * c;
  if ((int64_t)nseg * CSLOT > A.dense_ld || !(fabs(msc) < 0x1p30)) return false;
  double* hw = (double*)fl.buf;
  uint32_t* hc = (uint32_t*)(fl.buf + CB_NB);
  __syncthreads();  // (the export read the append buffer)
  double ws = cert_pass1<DT, PEN>(rc, e0, e1, Ms, floor(msc), c, invT, relevance_key(Ms, T), hw, hc);
  ws = block_sum_f64(ws, redd);
  double* slot = A.dense_w + (int64_t)row * A.dense_ld + (int64_t)seg * CSLOT;
  uint32_t* sc = (uint32_t*)(slot + CB_NB);
  for (int i = threadIdx.x; i < CB_NB; i += NT) {
    slot[i] = hw[i];
    sc[i] = hc[i];
  }
  if (threadIdx.x == 0) slot[CB_NB + CB_NB / 2] = ws;
  __syncthreads();
  return true;
}

template <int DT, bool PEN>
__device__ __forceinline__ int64_t dense_certified(const SmpArgs& A, const DevParams& P, const RowCtx& rc,
                                                   int row, int nseg, float M, uint32_t trel, const RowPlan& plan,
                                                   RowLds& fl, double* redd, uint64_t* redu) {
  constexpr int P2 = 16;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int V = A.V;
  const double T = P.temperature;
  const double invT = 1.0 / T;
  const double Md = (double)M;
  const double c = (double)CB_NB / (37.5 * T);
  const double fm = floor(Md * c);
  double* hw = (double*)fl.buf;                            // [CB_NB] bucket sums
  uint32_t* hc = (uint32_t*)(fl.buf + CB_NB);              // [CB_NB] bucket counts
  CertShared* cs = (CertShared*)(fl.buf + CB_NB + CB_NB / 2);
  uint64_t* bkt = fl.buf + CB_NB + CB_NB / 2 + 32;         // [BCAP] the min-p threshold bucket
  uint64_t* top = fl.cand;                                 // the head buckets
  uint64_t* cut = (uint64_t*)fl.w;                         // the cut bucket
  static_assert(CB_NB + CB_NB / 2 + 32 + BCAP <= BUFCAP && sizeof(CertShared) <= 32 * 8, "certified tail LDS layout");
  // the min-p threshold l* = M + T log(min_p) and its bucket
  const bool minp = P.min_p > 0.0;
  const double lstar = Md + T * log(P.min_p > 0.0 ? P.min_p : 1.0);
  const double lsc = lstar * c;
  const double fr = lsc - floor(lsc);
  const uint32_t bstar = minp ? grid_bucket(fm, lstar, c) : (uint32_t)CB_NB;
  if (!(fabs(Md * c) < 0x1p30) || (minp && (!(fabs(lsc) < 0x1p30) || fr < 1e-6 || fr > 1.0 - 1e-6 ||
                                            bstar >= (uint32_t)(CB_NB - 2))))
    return 0;  // (uniform)
  // 1. the bucket sums: the segments' shares, shifted and scaled, or one pass
  bool merged = false;
  if (nseg > 1) {
    const SegMeta* mt = A.exp_meta + (int64_t)row * nseg;
    bool all = true;
    for (int s = 0; s < nseg; ++s) all = all && mt[s].part != 0u && mt[s].mkey != 0u;
    merged = all;
  }
  double wrel = 0.0;
  if (merged) {
    const SegMeta* mt = A.exp_meta + (int64_t)row * nseg;
    for (int i = tid; i < CB_NB; i += NT) {
      hw[i] = 0.0;
      hc[i] = 0u;
    }
    __syncthreads();
    for (int s = 0; s < nseg; ++s) {
      const double Ms = (double)key2f(mt[s].mkey);
      const double o = fm - floor(Ms * c);  // >= 0: Ms <= M
      const double f = exp_approx((Ms - Md) * invT);
      const double* slot = A.dense_w + (int64_t)row * A.dense_ld + (int64_t)s * CSLOT;
      const uint32_t* sc = (const uint32_t*)(slot + CB_NB);
      constexpr int MQ = CB_NB / NT;  // a thread's buckets of the share: all loads in flight together
      uint32_t cv[MQ];
      double hv[MQ];
#pragma unroll
      for (int q = 0; q < MQ; ++q) {
        cv[q] = sc[q * NT + tid];
        hv[q] = slot[q * NT + tid];
      }
#pragma unroll
      for (int q = 0; q < MQ; ++q) {
        if (cv[q]) {
          const double bt = (double)(q * NT + tid) + o;  // >= 0: o = F(M) - F(Ms) >= 0
          const uint32_t b = bt < (double)(CB_NB - 1) ? (bt > 0.0 ? (uint32_t)bt : 0u) : (uint32_t)(CB_NB - 1);
          atomicAdd(&hw[b], f * hv[q]);
          atomicAdd(&hc[b], cv[q]);
        }
      }
      wrel += f * slot[CB_NB + CB_NB / 2];  // (every thread: the same sum)
    }
    __syncthreads();
  } else {
    wrel = cert_pass1<DT, PEN>(rc, 0, V, M, fm, c, invT, trel, hw, hc);
    wrel = block_sum_f64(wrel, redd);  // the total once more, in another order (a cross-check)
  }
  if (tid == 0) {
    cs->ncut = 0u;
    cs->ntop = 0u;
    cs->nb = 0u;
    cs->nk = 0u;
  }
  // the running sums over the buckets (wave 0; lane l owns buckets 64l..64l+63)
  if (wave == 0) {
    const int b0 = lane * 64;
    double sw = 0.0;
    uint32_t sc = 0u;
    for (int i = 0; i < 64; ++i) {
      sw += hw[b0 + i];
      sc += hc[b0 + i];
    }
    double ew = sw;
    uint32_t ec = sc;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const double tw = __shfl_up(ew, o);
      const uint32_t tc = (uint32_t)__shfl_up((int)ec, o);
      if (lane >= o) {
        ew += tw;
        ec += tc;
      }
    }
    const double R = __shfl(ew, 63);
    const uint32_t n = (uint32_t)__shfl((int)ec, 63);
    const double tau = P.top_p * R;
    double a = ew - sw;
    uint32_t cn = ec - sc;
    int fcut = -1, ftop = -1;
    double acut = 0.0, astar = 0.0;
    uint32_t ccut = 0u, ctop = 0u;
    for (int i = 0; i < 64; ++i) {
      const double wb = hw[b0 + i];
      const uint32_t cb = hc[b0 + i];
      if (fcut < 0 && a + wb >= tau) {
        fcut = b0 + i;
        acut = a;
        ccut = cn;
      }
      if (ftop < 0 && cn + cb >= (uint32_t)plan.KB) {
        ftop = b0 + i;
        ctop = cn + cb;
      }
      if ((uint32_t)(b0 + i) == bstar) astar = a;
      a += wb;
      cn += cb;
    }
    const uint64_t mc = __ballot(fcut >= 0), mt = __ballot(ftop >= 0);
    const int lc = mc ? (int)__builtin_ctzll(mc) : 0, lt = mt ? (int)__builtin_ctzll(mt) : 0;
    const int bcut = __shfl(fcut, lc), btop = __shfl(ftop, lt);
    const double a_cut = __shfl(acut, lc);
    const uint32_t c_cut = (uint32_t)__shfl((int)ccut, lc), c_top = (uint32_t)__shfl((int)ctop, lt);
    if ((uint32_t)lane == (bstar >> 6) && bstar < (uint32_t)CB_NB) cs->a_star = astar;
    if (lane == 0) {
      cs->R = R;
      cs->n = n;
      cs->bcut = mc ? (uint32_t)bcut : (uint32_t)CB_NB;
      cs->a_cut = a_cut;
      cs->ccut = c_cut;
      cs->btop = mt ? (uint32_t)btop : (uint32_t)CB_NB;
      cs->ctop = c_top;
    }
  }
  __syncthreads();
  const uint32_t n = cs->n, bcut = cs->bcut, btop = cs->btop;
  // the candidates are the relevant elements (top-k at or above their
  // count); the collected buckets lie above the last one (which may hold
  // counted elements below the relevance cut) and fit the LDS collections
  if (n == 0u || plan.k_eff < (int64_t)n || bcut >= (uint32_t)(CB_NB - 1) || btop >= (uint32_t)(CB_NB - 1) ||
      hc[bcut] > (uint32_t)CAP || cs->ctop > (uint32_t)CAP ||
      (minp && bstar != bcut && hc[bstar] > (uint32_t)BCAP)) {
    __syncthreads();
    return 0;
  }
  // 2. collect the cut bucket, the head and the threshold bucket; the
  // largest key below the threshold bucket; write out the entries before
  // both collected buckets (kept whichever cut holds: with the min-p cut,
  // S_(m-1) < top_p * total - E puts every kept entry at or before the cut
  // bucket and the kept set ends in the threshold bucket; with the top-p cut
  // the kept set ends in the cut bucket, at or before the threshold bucket)
  uint64_t* da = A.dense_a + (int64_t)row * A.dense_ld;
  const uint32_t bw = bcut < bstar ? bcut : bstar;
  uint32_t kbelow = 0u;
  // Every bucket set the pass asks about is an interval of relevant keys
  // (lower_key; no value here is NaN or infinite: such a row is flagged
  // non-finite and does not reach this tail), so elements are classified by
  // key compares alone: kb[0] written (b < bw), [kb[1], kb[2]) the cut
  // bucket, [kb[3], kb[4]) the threshold bucket (below kb[3]: b > bstar),
  // kb[5] the head (b <= btop). A bound of a bucket below 0 is no key.
  if (tid < 6) {
    const int64_t x = tid == 0 ? (int64_t)bw - 1 : tid == 1 ? (int64_t)bcut : tid == 2 ? (int64_t)bcut - 1
                    : tid == 3 ? (int64_t)bstar : tid == 4 ? (int64_t)bstar - 1 : (int64_t)btop;
    cs->kb[tid] = x < 0 ? 0xffffffffu : lower_key(fm, c, (uint32_t)x, trel);
  }
  __syncthreads();
  const uint32_t kw = cs->kb[0], kc0 = cs->kb[1], kc1 = cs->kb[2], ks0 = cs->kb[3], ks1 = cs->kb[4],
                 kt = cs->kb[5];
  {
    // one tile of NT * P2 elements (keys 0 past the end: not relevant)
    auto tile = [&](const uint32_t (&kk)[P2], int64_t base) {
      // the tile's written entries reserved by one LDS atomic per wave (the
      // whole wave is active), then stored in element order
      uint64_t wq[P2];
      uint32_t nw = 0u;
#pragma unroll
      for (int q = 0; q < P2; ++q) {
        wq[q] = __ballot(kk[q] >= kw);  // (kw >= trel: written entries are relevant)
        nw += (uint32_t)__popcll(wq[q]);
      }
      uint32_t s0 = 0u;
      if (nw) {
        if (lane == 0) s0 = atomicAdd(&cs->nk, nw);
        s0 = (uint32_t)__builtin_amdgcn_readfirstlane((int)s0);
      }
#pragma unroll
      for (int q = 0; q < P2; ++q) {
        const uint32_t k = kk[q];
        const uint64_t e = pack(k, (uint32_t)(base + (int64_t)q * NT + tid));
        if ((wq[q] >> lane) & 1ull) da[s0 + lanes_below(wq[q])] = e;
        s0 += (uint32_t)__popcll(wq[q]);
        if (k >= trel) {
          if (k < ks0 && k > kbelow) kbelow = k;  // b > bstar
          if (k >= kc0 && k < kc1) {
            const uint32_t s = atomicAdd(&cs->ncut, 1u);
            if (s < (uint32_t)CAP) cut[s] = e;
          } else if (k >= ks0 && k < ks1) {
            const uint32_t s = atomicAdd(&cs->nb, 1u);
            if (s < (uint32_t)BCAP) bkt[s] = e;
          }
          if (k >= kt) {
            const uint32_t s = atomicAdd(&cs->ntop, 1u);
            if (s < (uint32_t)CAP) top[s] = e;
          }
        }
      }
    };
    // two tiles in flight (loads at clamped indices: in range past the end)
    constexpr int64_t TL = (int64_t)NT * P2;
    uint32_t la[P2], lb[P2];
    cert_load<DT, PEN, P2>(rc, V, 0, la);
    cert_load<DT, PEN, P2>(rc, V, TL, lb);
    for (int64_t base = 0; base < V; base += 2 * TL) {
      uint32_t kk[P2];
      cert_keys<P2>(V, base, la, kk);
      if (base + 2 * TL < V) cert_load<DT, PEN, P2>(rc, V, base + 2 * TL, la);
      tile(kk, base);
      cert_keys<P2>(V, base + TL, lb, kk);
      if (base + 3 * TL < V) cert_load<DT, PEN, P2>(rc, V, base + 3 * TL, lb);
      tile(kk, base + TL);
    }
  }
  kbelow = (uint32_t)block_max_u64((uint64_t)kbelow, redu);
  __syncthreads();
  const uint32_t ncut = cs->ncut, ntop = cs->ntop;
  const uint32_t nb = bstar == bcut ? ncut : cs->nb;
  const uint64_t* const sb = bstar == bcut ? cut : bkt;  // the threshold bucket's entries
  if (ncut != hc[bcut] || ntop != cs->ctop || (minp && bstar != bcut && nb != hc[bstar])) {
    __syncthreads();
    return 0;
  }
  __syncthreads();
  // (the bucket sums are not read again: their array is the small sorts'
  // scratch)
  if (ntop <= (uint32_t)NT) sort_desc_small(top, (uint64_t*)hw, (int)ntop);
  else if (ntop <= 2u * NT) sort_desc_runs2(top, (uint64_t*)hw, (int)ntop);
  else sort_desc(top, (int)ntop);
  if (ncut <= (uint32_t)NT) sort_desc_small(cut, (uint64_t*)hw, (int)ncut);
  else if (ncut <= 2u * NT) sort_desc_runs2(cut, (uint64_t*)hw, (int)ncut);
  else sort_desc(cut, (int)ncut);
  // the first candidate min-p drops: the largest key below min-p in the
  // threshold bucket, else the largest key below that bucket
  const double mp_lo = P.min_p * (1.0 - 0x1p-40), mp_hi = P.min_p * (1.0 + 0x1p-40);
  uint32_t kfb = 0u;
  bool amb = false;
  if (minp) {
    for (uint32_t j = (uint32_t)tid; j < nb; j += NT) {
      const uint32_t k = pk_key(sb[j]);
      const double w = exp_approx(((double)key2f(k) - Md) * invT);
      if (w < mp_lo && k > kfb) kfb = k;
      amb |= w >= mp_lo && w <= mp_hi;
    }
    kfb = (uint32_t)block_max_u64((uint64_t)kfb, redu);
    amb = block_max_u64(amb ? 1ull : 0ull, redu) != 0ull;
    if (kfb == 0u) kfb = kbelow;
  }
  double pfb = 0.0;  // the threshold bucket's weights above kfb
  if (minp && kfb) {
    for (uint32_t j = (uint32_t)tid; j < nb; j += NT) {
      const uint32_t k = pk_key(sb[j]);
      if (k > kfb) pfb += exp_approx(((double)key2f(k) - Md) * invT);
    }
  }
  pfb = block_sum_f64(pfb, redd);
  // the cut bucket's weights, in candidate order
  for (uint32_t j = (uint32_t)tid; j < ncut; j += NT) hw[j] = exp_approx(((double)key2f(pk_key(cut[j])) - Md) * invT);
  __syncthreads();
  // 3. the cut, certified
  const double R = cs->R;
  const double marg = 2.0 * ((R * 0x1p-53) * (4.0 * (double)n + 2.0 * CB_NB + 2.0 * CAP + 64.0) + R * 0x1p-42);
  const double tau = P.top_p * R;
  int mode = 0;  // 0: not certified, 1: min-p cut, 2: top-p cut
  if (amb) {
    mode = 0;
  } else if (kfb) {
    const double pm = cs->a_star + pfb;  // the weights of the candidates min-p keeps
    if (pm < tau - marg && bstar <= bcut) mode = 1;
    else if (pm >= tau + marg && bcut <= bstar) mode = 2;
  } else {
    mode = (!minp || bcut <= bstar) ? 2 : 0;
  }
  if (mode == 2) {
    if (wave == 0) {
      const uint32_t K = (ncut + 63u) / 64u;
      const uint32_t j0 = (uint32_t)lane * K;
      const uint32_t j1 = j0 + K < ncut ? j0 + K : ncut;
      double s = 0.0;
      for (uint32_t j = j0; j < j1; ++j) s += hw[j];
      double e = s;
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) {
        const double t = __shfl_up(e, o);
        if (lane >= o) e += t;
      }
      double run = cs->a_cut + (e - s), lo = 0.0, hi = 0.0;
      int found = -1;
      for (uint32_t j = j0; j < j1; ++j) {
        const double prev = run;
        run += hw[j];
        if (found < 0 && run >= tau) {
          found = (int)j;
          lo = prev;
          hi = run;
        }
      }
      const uint64_t mf = __ballot(found >= 0);
      const int lf = mf ? (int)__builtin_ctzll(mf) : 0;
      const int f = __shfl(found, lf);
      const double flo = __shfl(lo, lf), fhi = __shfl(hi, lf);
      if (lane == 0) {
        cs->j0 = mf ? f : -1;
        cs->p_lo = flo;
        cs->p_hi = fhi;
      }
    }
    __syncthreads();
    if (cs->j0 < 0 || !(cs->p_hi >= tau + marg) || !(cs->p_lo < tau - marg)) mode = 0;
  }
  if (!(fabs(wrel - R) <= marg)) mode = 0;  // the two sums disagree beyond their bounds
  if (mode == 0) {
    __syncthreads();
    return 0;
  }
  // 4. the kept entries of the last bucket join those written in pass 2:
  // with the top-p cut the cut bucket's first j0 + 1, with the min-p cut the
  // threshold bucket's entries above kfb
  {
    const int32_t j0 = mode == 2 ? cs->j0 : -1;
    const uint32_t m4 = mode == 2 ? ncut : nb;
    const uint64_t* const s4 = mode == 2 ? cut : sb;
    for (uint32_t j = (uint32_t)tid; j < m4; j += NT) {
      const uint64_t e = s4[j];
      if (mode == 2 ? (int32_t)j <= j0 : pk_key(e) > kfb) da[atomicAdd(&cs->nk, 1u)] = e;
    }
  }
  __syncthreads();
  const int64_t nk = (int64_t)cs->nk;
  const float Mf = M, invTf = (float)invT;
  const int nd = A.mode == MODE_VERIFY ? 1 : A.n_draws;
  for (int d = 0; d < nd; ++d) {
    const uint64_t pk = position_key(P.seed, position_of(A, row, d));
    // the largest binary32 score (and each thread's two largest, with the
    // entry of the first) ...
    float s1 = -__builtin_inff(), s2 = -__builtin_inff();
    uint64_t e1 = 0ull;
    uint64_t nv[DRB];  // the next round's entries, in flight while a round is scored
    if (nk > 0) draw_load(da, nk, 0, nv);
    for (int64_t j0 = 0; j0 < nk; j0 += (int64_t)NT * DRB) {
      uint64_t ev[DRB];
#pragma unroll
      for (int q = 0; q < DRB; ++q) ev[q] = nv[q];
      if (j0 + (int64_t)NT * DRB < nk) draw_load(da, nk, j0 + (int64_t)NT * DRB, nv);
#pragma unroll
      for (int q = 0; q < DRB; ++q) {
        const uint64_t e = ev[q];
        const float s = score_approx((key2f(pk_key(e)) - Mf) * invTf, pk, pk_id(e));
        const float sv = j0 + (int64_t)q * NT + tid < nk ? s : -__builtin_inff();
        const bool up = sv > s1;
        s2 = up ? s1 : (sv > s2 ? sv : s2);
        e1 = up ? e : e1;
        s1 = up ? sv : s1;
      }
    }
    float smax = s1;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
      const float t = __shfl_xor(smax, o);
      smax = t > smax ? t : smax;
    }
    __syncthreads();
    if (lane == 0) redd[wave] = (double)smax;
    __syncthreads();
    double sm = redd[0];
#pragma unroll
    for (int q = 1; q < NW; ++q) sm = redd[q] > sm ? redd[q] : sm;
    const float thr = (float)sm - 2.0f * SC_TOL;
    // ... then the exact z + g of the entries within 2 SC_TOL of it: each
    // thread's first when no thread has a second there (the common case),
    // else every entry again
    double best = -__builtin_inf();
    uint64_t be = 0ull;
    const bool again = block_max_u64(s2 >= thr ? 1ull : 0ull, redu) != 0ull;
    if (!again && s1 >= thr && s1 != -__builtin_inff()) {
      best = ((double)key2f(pk_key(e1)) - Md) / T + gumbel_from_key(pk, pk_id(e1));
      be = e1;
    }
    if (again && nk > 0) draw_load(da, nk, 0, nv);
    for (int64_t j0 = 0; again && j0 < nk; j0 += (int64_t)NT * DRB) {
      uint64_t ev[DRB];
#pragma unroll
      for (int q = 0; q < DRB; ++q) ev[q] = nv[q];
      if (j0 + (int64_t)NT * DRB < nk) draw_load(da, nk, j0 + (int64_t)NT * DRB, nv);
      uint32_t hit = 0u;
#pragma unroll
      for (int q = 0; q < DRB; ++q) {
        const uint64_t e = ev[q];
        const float s = score_approx((key2f(pk_key(e)) - Mf) * invTf, pk, pk_id(e));
        hit |= (j0 + (int64_t)q * NT + tid < nk && s >= thr) ? (1u << q) : 0u;
      }
      while (hit) {  // the few entries near the largest score: exact binary64 z + g
        const int q = __builtin_ctz(hit);
        hit &= hit - 1u;
        uint64_t e = ev[0];
#pragma unroll
        for (int r = 1; r < DRB; ++r) e = r == q ? ev[r] : e;
        const double z = ((double)key2f(pk_key(e)) - Md) / T;
        const double x = z + gumbel_from_key(pk, pk_id(e));
        if (x > best || (x == best && e > be)) {
          best = x;
          be = e;
        }
      }
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
      const double ob = __shfl_xor(best, o);
      const uint64_t oe = (uint64_t)__shfl_xor((long long)be, o);
      if (ob > best || (ob == best && oe > be)) {
        best = ob;
        be = oe;
      }
    }
    __syncthreads();
    if (lane == 0) {
      redd[wave] = best;
      redu[wave] = be;
    }
    __syncthreads();
    if (tid == 0) {
      double b = redd[0];
      uint64_t e = redu[0];
      for (int q = 1; q < NW; ++q) {
        if (redd[q] > b || (redd[q] == b && redu[q] > e)) {
          b = redd[q];
          e = redu[q];
        }
      }
      A.out_ids[(int64_t)row * A.n_draws + d] = pk_id(e);
    }
  }
  __syncthreads();
  return (int64_t)n;
}

// ---------------------------------------------------------------------------
// smp_row: one block of 8 wave64s per row, streaming the whole row.
//
// The row is read in chunks of 2,048 logits (32 values per lane, 16-byte
// buffer loads), two per wave in flight; the waves claim chunks as they
// free their buffers and share bounds and the row maximum through LDS
// atomics, with no barrier in the stream. Each wave filters its chunks with
// the bounds as they stand and appends the elements that can matter to an
// LDS buffer. After the stream the same block sorts the candidates and runs
// the reference's truncation and draw: no second launch, no traffic between
// blocks. CERT: the form of the smaller launches, whose rows may be split
// into segments (one block each, the last one finishing the row) and whose
// dense rows try the certified tail; without it, one block per row.
// ---------------------------------------------------------------------------
template <int DT, bool VEC, bool PEN, bool CERT>
__global__ __launch_bounds__(NT) void smp_row(SmpArgs Ain) {
  // The large-launch form serves one feature set: sampling at explicit
  // positions, one draw per row, lists of at most KBMAX entries, no
  // advance, no NLL targets, nothing forced (the host sends every other
  // launch to the general form). Pinning those fields leaves the rest out
  // of that kernel's code.
  SmpArgs A = Ain;
  if constexpr (!CERT) {
    A.nseg = 1;
    A.mode = MODE_SAMPLE;
    A.n_draws = 1;
    A.pos_mode = POS_ARRAY;
    A.adv_pos = nullptr;
    A.adv_tok = nullptr;
    A.nll_targets = nullptr;
    A.force_dense = 0;
  }
  __shared__ RowLds fl;
  __shared__ RowShared sh;
  __shared__ uint64_t red_u64[NW];
  __shared__ double red_f64[NW];
  __shared__ int red_int[NW];
  __shared__ float s_mref[SEG_MAX];   // mass terms: one per wave, or one per segment
  __shared__ double s_mass[SEG_MAX];
  __shared__ int32_t s_last;          // this block finishes the row
  __shared__ TailShared ts;
  __shared__ uint64_t s_pos;       // position of the row's first draw
  __shared__ int32_t s_pos_ok;     // that position is representable
  __shared__ uint32_t s_rank[64];  // ranks of up to 64 final candidates
  __shared__ double s_wpre[64];    // their weights, in compaction order
  __shared__ double s_spre[64];    // their version-3 scores, in compaction order

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  // A row is split into nseg segments of whole chunks, one block each; with
  // nseg = 1 the block streams the whole row and finishes it directly.
  const int nseg = A.nseg;
  const int row = (int)blockIdx.x / nseg;
  const int seg = (int)blockIdx.x - row * nseg;
  const int32_t V = A.V;
  // The wave's first two chunks are requested before anything else: they
  // need only the row's address, while the parameters take dependent scalar
  // loads (microseconds at the start of a launch).
  constexpr int ES = DT == 0 ? 4 : (DT == 1 ? 2 : 8);  // bytes per input element
  const char* const row_base = (const char*)A.logits + (int64_t)row * A.ld * ES;
  const int nch = (V + WSEG - 1) / WSEG;
  const int cb = (int)(((int64_t)seg * nch) / nseg);       // this block's chunks [cb, ce)
  const int ce = (int)(((int64_t)(seg + 1) * nch) / nseg);
  // Chunks [cb, sfull) are read by the double-buffered stream with
  // range-checked buffer loads: every chunk of an aligned row, the ragged
  // last one included when the row is a whole number of 16-byte groups (a
  // group straddling the row end would make one 16-byte load only partly in
  // range: that chunk goes to the guarded loads after the stream, like every
  // chunk of an unaligned row).
  const bool whole_groups = ((uint32_t)V * (uint32_t)ES) % 16u == 0u;
  const int nfull = VEC ? (whole_groups ? nch : V / WSEG) : 0;
  const int sfull = nfull < ce ? nfull : ce;
  uint32_t buf0[EPT], buf1[EPT];
  load_full<DT>(row_base, V, cb + wave, cb + wave < sfull, lane, buf0);
  __builtin_amdgcn_sched_barrier(0);  // buf0's loads first: the stream waits for them first
  load_full<DT>(row_base, V, cb + wave + NW, cb + wave + NW < sfull, lane, buf1);
  __builtin_amdgcn_sched_barrier(0);  // both chunks in flight before any other work
  const DevParams P = A.prm[A.prm_shared ? 0 : row];
  const RowPlan plan = make_plan(A, P);
  // the exact dense path from the start: forced, or a prefix longer than the
  // waves' lists (top-N or logprob counts above KBMAX)
  const bool fdense = CERT && (A.force_dense != 0 || plan.KB > KBMAX);  // (the large form: KB <= KBMAX)
  uint32_t wflags = 0;
  const RowCtx rc = make_rowctx<PEN>(A, P, row, ES, &wflags);
  if (tid == 0) {
    sh.count = 0u;
    sh.flags = 0u;
    sh.ndef = 0u;
    sh.next = (uint32_t)cb + 2u * NW;  // chunks cb .. cb + 2 NW - 1 are the waves' first two
  }
  if (tid < BW_N) sh.bw[tid] = 0u;
  if (tid < 64) s_rank[tid] = 0u;
  if (tid == 64) sh.ctr = 0u;
  // each segment appends past BUFCAP into its own share of the row's spill area
  const int64_t spill_share = A.dense_ld / nseg;
  uint64_t* const spill = A.dense_b + (int64_t)row * A.dense_ld + (int64_t)seg * spill_share;

  WaveState ws;
  ws.wkey = 0u;
  ws.m_ref = -__builtin_inff();
  ws.acc = 0.0;
  ws.bad = false;
  ws.spill_cap = (uint32_t)spill_share;
  __syncthreads();  // shared state initialised

  // Each wave keeps the KB largest lane maxima of its chunks so far, sorted
  // descending in lanes 0..KB-1 (distinct elements: KB of them are at or
  // above the list's last value, which is therefore a valid top-KB bound).
  // Waves share the best such bound and the row maximum through LDS atomics;
  // nothing in the stream waits for another wave.
  // A lane maximum at or below the row's certified bound th_row cannot be
  // among the row's top KB and does not enter the list: any KB distinct
  // elements certify their smallest value as a bound, so the lists stay
  // valid while the row bound filters what reaches them.
  uint32_t lst = 0u, theta_w = 0u, q_pub = 0u, th_row = 0u;
  uint32_t thr_mk = 0u, thr_th = 0u, thr_c = 1u;  // the last row threshold and its inputs
  uint32_t theta_pub = 0u;                          // theta_w as last published
  const int qidx = (plan.KL + NW - 1) / NW - 1;
  // per chunk: up to its two largest lane maxima enter the list. Each entry
  // costs a wave-wide reduction on the stream's critical path (the waves'
  // first chunks at the start most of all). Early on the list is short, so
  // the waves' first chunks meet no bound and are deferred (kept in LDS);
  // the bound builds up from the waves' shared ceil(KB/8)-th entries, and
  // the final one comes from the union of their lists. (On 256 x 248,320
  // logits with KB = 20, inserting the first chunk's top KB at once cost
  // about 4 us per launch, eight per later chunk about 0.5 us.)
  // A segmented row gives each wave about one chunk: its first chunk then
  // inserts all its KB largest lane maxima, so that a certified bound exists
  // at once (otherwise the segment would export every element).
  const int r_next = plan.KL < 2 ? plan.KL : 2;
  const int r_first = nseg > 1 ? plan.KL : r_next;

  // Below lo_f nothing can matter to this wave: no lane maximum would enter
  // its list (lo_f <= its KB-th value), no value would be a candidate
  // (lo_f <= the threshold it last used) or a mass term (lo_f <= m_ref -
  // ZMASS). A chunk whose values all lie below it costs its conversion and
  // one comparison; the bounds only rise, so a stale lo_f is merely low.
  float lo_f = -__builtin_inff();

  // One chunk: c from X. In the stream, the wave claims its next chunk and
  // prefetches it into X (the claim is an LDS atomic issued first, its
  // result read last, so that its latency is hidden); returns that chunk.
  // `live`: X holds chunk c (false for a buffer whose claim fell past the
  // streamed chunks: nothing was loaded into it).
  auto step = [&](uint32_t (&X)[EPT], int c, bool first, bool stream, bool live) -> int {
    uint32_t ticket = 0u;
    if (stream && lane == 0) ticket = atomicAdd(&sh.next, 1u);
    float lmax = -__builtin_inff();
    if (live) chunk_values<DT, PEN>(rc, V, c, lane, X, lmax, ws.bad);
    if (live && (first || __ballot(lmax >= lo_f))) {
      const uint32_t lk = lmax == -__builtin_inff() ? 0u : f2key(__float_as_uint(lmax));
      // The chunk maximum (a DPP reduction) only when a lane maximum may
      // enter the list or raise the wave's maximum.
      uint32_t cmax = 0u;
      const uint32_t lb = theta_w > th_row ? theta_w : th_row;
      if (first || __ballot(lk > lb || lk > ws.wkey)) {
        uint32_t rk = lk;
        const int rr = first ? r_first : r_next;
        if (first && rr > 2) {
          // The wave's first chunk with the list empty (th_row = theta_w =
          // 0): the list becomes the rr largest nonzero lane maxima, equal
          // values once per lane, in one step -- the rr-th largest by a
          // ballot radix select, each qualifying lane's rank by (value desc,
          // lane asc) over the qualifying lanes, and one lane permute.
          cmax = wave_max_dpp(lk);
          const int nz = __popcll(__ballot(lk != 0u));
          const uint32_t kth = nz > rr ? wave_kth_largest_radix(lk, rr) : 1u;
          const uint64_t in = __ballot(lk != 0u && lk >= kth);
          uint32_t rank = 0u;
          for (uint64_t rem = in; rem; rem &= rem - 1ull) {
            const int b = __builtin_ctzll(rem);
            const uint32_t vb = (uint32_t)__builtin_amdgcn_readlane((int)lk, b);
            rank += (vb > lk || (vb == lk && b < lane)) ? 1u : 0u;
          }
          const bool put = ((in >> lane) & 1ull) != 0ull && rank < (uint32_t)rr;
          const uint32_t got = (uint32_t)__builtin_amdgcn_ds_permute((int)((put ? rank : 63u) * 4u), (int)lk);
          const int nput = __popcll(in) < rr ? __popcll(in) : rr;
          lst = lane < nput ? got : 0u;
          theta_w = (uint32_t)__builtin_amdgcn_readlane((int)lst, plan.KL - 1);
        } else {
          for (int i = 0; i < rr; ++i) {
            const uint32_t m = wave_max_dpp(rk);
            if (i == 0) cmax = m;
            if (m <= theta_w || m <= th_row) break;  // 0, cannot enter the full list, or below the row bound
            // insert m: entries >= m keep their lanes, the rest move up by one
            const uint32_t pos = (uint32_t)__popcll(__ballot(lane < plan.KL && lst >= m));
            const uint32_t up = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)lst, 0x138, 0xf, 0xf, false);  // wave_shr:1
            lst = (uint32_t)lane < pos ? lst : ((uint32_t)lane == pos ? m : up);
            theta_w = (uint32_t)__builtin_amdgcn_readlane((int)lst, plan.KL - 1);
            const uint64_t eq = __ballot(rk == m);
            if (lane == (int)__builtin_ctzll(eq)) rk = 0u;
          }
        }
        if (cmax > ws.wkey) {
          ws.wkey = cmax;
          if (lane == 0) atomicMax(&sh.bw[BW_MKEY], cmax);
        }
      }
      if (theta_w > theta_pub) {
        // every bound a wave uses must reach the shared one: the final
        // bound is taken from it and may not be lower
        theta_pub = theta_w;
        if (lane == 0) atomicMax(&sh.bw[BW_THETA], theta_w);
      }
      {
        const uint32_t qw = (uint32_t)__builtin_amdgcn_readlane((int)lst, qidx);
        if (qw > q_pub) {
          q_pub = qw;
          if (lane == 0) atomicMax(&sh.bw[BW_Q + wave], qw);
        }
      }
      // Every shared bound in one LDS load (a workgroup-scope atomic read:
      // a volatile access through a generic pointer would become a flat load
      // that waits for every outstanding global load -- the prefetch). Two
      // certified bounds: the best single wave's KB-th value, and the minimum
      // over the waves of their ceil(KB/8)-th values (each wave has that many
      // elements at or above it: 8 * ceil(KB/8) >= KB in all).
      const uint32_t bw = lane < BW_N ? __hip_atomic_load(&sh.bw[lane], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP)
                                      : 0u;
      uint32_t qv = (lane >= BW_Q && lane < BW_Q + NW) ? bw : 0xffffffffu;
      {
        uint32_t t;
        t = (uint32_t)__builtin_amdgcn_update_dpp(-1, (int)qv, 0x111, 0xf, 0xf, false);  // row_shr:1
        qv = qv < t ? qv : t;
        t = (uint32_t)__builtin_amdgcn_update_dpp(-1, (int)qv, 0x112, 0xf, 0xf, false);  // row_shr:2
        qv = qv < t ? qv : t;
        t = (uint32_t)__builtin_amdgcn_update_dpp(-1, (int)qv, 0x114, 0xf, 0xf, false);  // row_shr:4
        qv = qv < t ? qv : t;
        t = (uint32_t)__builtin_amdgcn_update_dpp(-1, (int)qv, 0x118, 0xf, 0xf, false);  // row_shr:8
        qv = qv < t ? qv : t;
      }
      const uint32_t qmin = (uint32_t)__builtin_amdgcn_readlane((int)qv, 15);
      uint32_t th = (uint32_t)__builtin_amdgcn_readlane((int)bw, BW_THETA);
      th = th > theta_w ? th : theta_w;
      th = qmin > th ? qmin : th;
      uint32_t mk = (uint32_t)__builtin_amdgcn_readlane((int)bw, BW_MKEY);
      mk = mk > ws.wkey ? mk : ws.wkey;
      // the row threshold changes only with (mk, th): computed again only then
      if (mk != thr_mk || th != thr_th) {
        thr_mk = mk;
        thr_th = th;
        thr_c = fdense ? 0xffffffffu : row_threshold(plan, P, key2f(mk), th);
      }
      const uint32_t thr = thr_c;
      // (a wave's first chunk has about KB lanes with survivors by
      // construction -- the lane maxima that set its first bound -- so its
      // deferral limit is raised by KB)
      chunk_filter<DT>(c, lane, X, thr, mk, A.want_mass != 0, lk, cmax, first ? DLANES + plan.KL : DLANES, ws,
                       sh, fl, spill);
      th_row = th;
      const float lo_list = key_threshold_float(theta_w > th ? theta_w : th);
      const float lo_cand = key_threshold_float(thr);
      const float lo_mass = A.want_mass ? ws.m_ref - ZMASS : __builtin_inff();
      lo_f = mk == 0u ? -__builtin_inff() : fminf(fminf(lo_list, lo_cand), lo_mass);
    }
    int nx = sfull;
    if (stream) {
      nx = __builtin_amdgcn_readfirstlane((int)ticket);
      load_full<DT>(rc.base, V, nx, nx < sfull, lane, X);
    }
    return nx;
  };
  // The first draw's position: a global load waits behind the other rows'
  // streams (microseconds), so it is read now, at the start, by the last
  // wave; the chunks it meanwhile leaves go to the other waves.
  // (a uniform branch: a scalar load, which leaves the vector-memory
  // counter, and so the stream's waits, alone)
  if (wave == NW - 1 && A.out_ids != nullptr) {
    bool ok;
    const uint64_t p0 = position_of(A, row, 0, &ok);
    if (lane == 0) {
      s_pos = p0;
      s_pos_ok = ok ? 1 : 0;
    }
  }
  // Chunks [cb, sfull) are handed out as the waves free their buffers: wave
  // w starts with chunks cb + w and cb + w + NW (already requested) and then
  // claims the next unclaimed chunk, so that a wave slowed by heavy chunks
  // takes fewer of them. At every step the buffer read is the older of the
  // two in flight; a claim past sfull ends the wave's stream (claims only
  // grow, so the other buffer's chunk, claimed earlier, was the smaller).
  bool wfirst = true;  // the wave has filtered no chunk yet
  {
    int c0 = cb + wave, c1 = cb + wave + NW;
    while (c0 < sfull) {
      c0 = step(buf0, c0, wfirst, true, true);
      wfirst = false;
      // (c1 may be past the streamed chunks: then nothing but the claim)
      c1 = step(buf1, c1, false, true, c1 < sfull);
    }
  }
  // the remaining chunks of the segment, round robin over the waves
  {
    const int tb = sfull > cb ? sfull : cb;
    for (int c = tb + wave; c < ce; c += NW) {
      load_chunk<DT, VEC>(rc, V, nch, c, lane, buf0);
      step(buf0, c, wfirst, false, true);
      wfirst = false;
    }
  }
  // A final bound from the union of the waves' lists: the KB-th largest of
  // their top 8 entries (64 distinct elements). It is at least the minimum
  // over the waves of their ceil(KB/8)-th values, and sh.bw[BW_THETA] keeps
  // the best single-wave bound: no bound used in the stream exceeds the
  // final one (every improvement was published), which keeps the buffer
  // complete down to it.
  if (lane < 8) fl.lists[wave * 8 + lane] = lane < plan.KL ? lst : 0u;
  // The wave's own results, which the deferred chunks below do not change
  // (they add no mass terms and find no new maximum).
  if (__ballot(ws.bad)) wflags |= F_NONFINITE;
  {
    const double wm = A.want_mass ? wave_sum_f64_dpp(ws.acc) : 0.0;
    if (lane == 0) {
      if (wflags) atomicOr(&sh.flags, wflags);
      s_mref[wave] = ws.m_ref;
      s_mass[wave] = wm;
    }
  }
  __syncthreads();  // every append, deferral, list, maximum and mass term is in LDS
  // every wave ranks the union itself (the same value in all): no second barrier
  uint32_t theta = sh.bw[BW_THETA];
  {
    const uint32_t t = wave_kth_largest_radix(fl.lists[lane], plan.KL);
    theta = t > theta ? t : theta;
  }
  // Deferred chunks against the final bound: one whose second largest key
  // reaches it is read again and filtered with that bound; one where only
  // its largest does hands that element over directly (wave 0); the rest
  // hold nothing at or above it. Entry i is read again by wave i % NW; each
  // wave keeps two of its chunks in flight (the stream's buffers are free).
  if (!fdense) {
    const uint32_t mkf = sh.bw[BW_MKEY];
    const uint32_t thr_f = row_threshold(plan, P, key2f(mkf), theta);
    const uint32_t nd = sh.ndef < (uint32_t)DEFCAP ? sh.ndef : (uint32_t)DEFCAP;
    if (wave == 0) {
      bool spilled = false;
      for (uint32_t i0 = 0; i0 < nd; i0 += 64) {
        const uint32_t i = i0 + (uint32_t)lane;
        const uint4 d = i < nd ? fl.def[i] : make_uint4(0u, 0u, 0u, 0u);
        const bool one = i < nd && d.y >= thr_f && d.z < thr_f;
        const uint64_t m = __ballot(one);
        if (m) {
          uint32_t base = 0u;
          if (lane == 0) base = atomicAdd(&sh.count, (uint32_t)__popcll(m));
          base = (uint32_t)__builtin_amdgcn_readfirstlane((int)base);
          const uint32_t slot = base + lanes_below(m);
          if (one) {
            const uint64_t e = pack(d.y, d.w);
            if (slot < (uint32_t)BUFCAP) {
              ((lds_u64*)fl.buf)[slot] = e;
            } else if (slot - (uint32_t)BUFCAP < ws.spill_cap) {
              __builtin_nontemporal_store(e, &((global_u64*)spill)[slot - BUFCAP]);
              spilled = true;
            }
          }
        }
      }
      if (__ballot(spilled)) __builtin_amdgcn_s_waitcnt(0);
    }
    // (every wave sees the same entries: the condition is block-uniform)
    bool any = false;
    for (uint32_t i = (uint32_t)lane; i < nd; i += 64) any = any || fl.def[i].z >= thr_f;
    if (__ballot(any)) {
      auto next = [&](uint32_t from) -> uint32_t {
        for (uint32_t i = from; i < nd; i += NW)
          if (fl.def[i].z >= thr_f) return i;
        return nd;
      };
      // a stashed chunk comes from LDS, converted already; the others from
      // memory again
      auto fetch = [&](uint32_t (&X)[EPT], uint32_t i) {
        const uint32_t code = fl.def[i].x;
        if ((code >> 16) == 0u) load_chunk<DT, VEC>(rc, V, nch, (int)(code & 0xffffu), lane, X, false);
      };
      auto redo = [&](uint32_t (&X)[EPT], uint32_t i) {
        const uint32_t code = fl.def[i].x;
        const int cc = (int)(code & 0xffffu);
        float lmax = -__builtin_inff();
        if ((code >> 16) != 0u) {
          unstash_chunk(fl, (code >> 16) - 1u, lane, X);
#pragma unroll
          for (int k = 0; k < EPT; ++k) lmax = fmaxf(lmax, __uint_as_float(X[k]));
        } else {
          bool bad = false;
          chunk_values<DT, PEN>(rc, V, cc, lane, X, lmax, bad);
        }
        const uint32_t lkr = lmax == -__builtin_inff() ? 0u : f2key(__float_as_uint(lmax));
        chunk_filter<DT>(cc, lane, X, thr_f, mkf, false, lkr, fl.def[i].y, 64, ws, sh, fl, spill);
      };
      uint32_t ia = next((uint32_t)wave);
      uint32_t ib = ia < nd ? next(ia + NW) : nd;
      if (ia < nd) fetch(buf0, ia);
      if (ib < nd) fetch(buf1, ib);
      while (ia < nd) {
        redo(buf0, ia);
        const uint32_t ic = ib < nd ? next(ib + NW) : nd;
        if (ic < nd) fetch(buf0, ic);
        if (ib >= nd) break;
        redo(buf1, ib);
        const uint32_t id = ic < nd ? next(ic + NW) : nd;
        if (id < nd) fetch(buf1, id);
        ia = ic;
        ib = id;
      }
    }
    if (nd) __syncthreads();  // the deferred chunks' appends are in the buffer
  }

  // ---- segments: hand the candidates to the row's last block -------------
  // A segment's certified bound and maximum are no larger than the row's, so
  // its threshold is no larger than the row's final one: every element of the
  // row at or above that final threshold is exported by its segment (unless
  // a segment overflows EXP_CAP: then the row takes the dense path). The
  // row's top-KB are among the exports, so the last block ranks the union
  // itself for the final bound.
  int n_mass = NW;  // mass terms in s_mref / s_mass
  if (nseg > 1) {
    const uint32_t mk_s = sh.bw[BW_MKEY];
    const uint32_t theta_s = fdense ? 0xffffffffu : row_threshold(plan, P, key2f(mk_s), theta);
    uint64_t* const xc = A.exp_cand + ((int64_t)row * nseg + seg) * EXP_CAP;
    const uint32_t cnt = sh.count;
    uint32_t nx;
    // (an export past EXP_CAP is of no use: the compaction stops there)
    if (cnt <= (uint32_t)BUFCAP) {
      nx = compact_entries<true>(fl.buf, cnt, xc, EXP_CAP, theta_s, &sh.ctr, true);
    } else if ((int64_t)(cnt - (uint32_t)BUFCAP) <= spill_share) {
      compact_entries<true>(fl.buf, BUFCAP, xc, EXP_CAP, theta_s, &sh.ctr, true);
      nx = compact_entries<true>(spill, cnt - (uint32_t)BUFCAP, xc, EXP_CAP, theta_s, &sh.ctr, false);
    } else {
      nx = EXP_CAP + 1u;  // reservations outran the spill share
    }
    // an overflow sends the row to the dense path: a row headed for the
    // certified tail gets this segment's share of its first pass now
    bool part = false;
    if constexpr (CERT) {
      if (nx > (uint32_t)EXP_CAP && mk_s != 0u && !fdense && plan.sampled && plan.need_rel &&
          P.version == YSKN_V3 && !P.zcheck) {
        const int64_t e1 = (int64_t)ce * WSEG < (int64_t)V ? (int64_t)ce * WSEG : (int64_t)V;
        part = cert_share<DT, PEN>(A, P, rc, row, seg, nseg, key2f(mk_s), (int64_t)cb * WSEG, e1, fl, red_f64);
      }
    }
    if (wave == 0) {
      // the segment's mass relative to its largest wave reference point
      const float mr = lane < NW ? s_mref[lane] : -__builtin_inff();
      const uint32_t mkey = wave_max_dpp(mr == -__builtin_inff() ? 0u : f2key(__float_as_uint(mr)));
      const float mr_s = mkey == 0u ? -__builtin_inff() : key2f(mkey);
      double t = 0.0;
      if (lane < NW && mr != -__builtin_inff()) t = s_mass[lane] * exp((double)mr - (double)mr_s);
      const double ms = wave_sum_f64_dpp(t);
      if (lane == 0) {
        SegMeta& m = A.exp_meta[(int64_t)row * nseg + seg];
        m.count = nx;
        m.flags = sh.flags;
        m.mkey = mk_s;
        m.theta = theta;
        m.mass = ms;
        m.mref = mr_s;
        m.part = part ? 1u : 0u;
      }
    }
    // release: the barrier completes every wave's stores of the export and
    // the record; one agent-scope release (an L2 write-back) then publishes
    // them before the arrival
    __syncthreads();
    if (tid == 0) {
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
      const uint32_t old = __hip_atomic_fetch_add(&A.segcnt[row], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      s_last = old == (uint32_t)(nseg - 1) ? 1 : 0;
      if (s_last) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    }
    __syncthreads();
    if (!s_last) return;  // (uniform: the whole block leaves)
    // ---- the row's last block: gather every segment's export ---------------
    // Every slot of every segment is requested before the segments' records
    // arrive (their counts then pick the filled slots): one round trip.
    const uint64_t* const xr = A.exp_cand + (int64_t)row * nseg * EXP_CAP;
    constexpr int IMP = SEG_MAX * EXP_CAP / NT;
    uint64_t v[IMP];
#pragma unroll
    for (int r = 0; r < IMP; ++r) {
      const int i = tid + r * NT;
      v[r] = i < nseg * EXP_CAP ? xr[i] : 0ull;
    }
    const SegMeta* const mt = A.exp_meta + (int64_t)row * nseg;
    // per-segment offsets into the buffer, then its counts; then the largest
    // segment bound, the number of entries at or above it and their keys
    // (the first 256)
    uint32_t* const s_off = (uint32_t*)fl.w;
    uint32_t* const s_hi = s_off + 2 * SEG_MAX;
    if (wave == 0) {
      // lane q reads segment q's record (one round trip for all of them)
      uint32_t c = 0u, mk = 0u, fo = 0u, ts = 0u;
      float mr = -__builtin_inff();
      double ms = 0.0;
      if (lane < nseg) {
        c = mt[lane].count;
        mk = mt[lane].mkey;
        ts = mt[lane].theta;
        fo = mt[lane].flags;
        mr = mt[lane].mref;
        ms = mt[lane].mass;
        s_mref[lane] = mr;
        s_mass[lane] = ms;
      }
      const bool over = __ballot(lane < nseg && c > (uint32_t)EXP_CAP) != 0ull;
      const uint32_t cc = c > (uint32_t)EXP_CAP ? 0u : c;
      const int incl = wave_incl_scan((int)cc, lane);
      if (lane < nseg) {
        s_off[lane] = (uint32_t)incl - cc;
        s_off[SEG_MAX + lane] = cc;
      }
      const uint32_t total = (uint32_t)__builtin_amdgcn_readlane(incl, 63);
      const uint32_t mkr = wave_max_dpp(mk);
      const uint32_t tlo = wave_max_dpp(ts);
      uint32_t fr = fo;
#pragma unroll
      for (int o = 32; o > 0; o >>= 1) fr |= (uint32_t)__shfl_xor((int)fr, o);
      if (lane == 0) {
        __hip_atomic_store(&A.segcnt[row], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);  // for the next call
        sh.bw[BW_MKEY] = mkr;
        sh.flags = fr;
        // an overflow sends the row to the dense path (a count past the spill)
        sh.count = over ? (uint32_t)BUFCAP + (uint32_t)A.dense_ld + 1u : total;
        sh.ctr = 0u;
        s_hi[0] = tlo;
        s_hi[1] = 0u;
      }
    }
    n_mass = nseg;
    __syncthreads();
    const uint32_t total = sh.count;
    if (total <= (uint32_t)BUFCAP) {
      // The row's KB-th key is among the entries at or above the largest
      // segment bound (that segment exported at least KB of them, and every
      // segment exported all of its own): at most 256 of them, one wave
      // selects it (every wave, the same); more, the whole import is ranked.
      const uint32_t tlo = s_hi[0];
#pragma unroll
      for (int r = 0; r < IMP; ++r) {
        const int i = tid + r * NT;
        const int q = i / EXP_CAP, j = i - q * EXP_CAP;
        const bool ok = q < nseg && (uint32_t)j < s_off[SEG_MAX + q];
        if (ok) fl.buf[s_off[q] + (uint32_t)j] = v[r];
        const uint32_t key = pk_key(v[r]);
        const bool hi = ok && key >= tlo;
        const uint64_t hm = __ballot(hi);
        if (hm) {
          uint32_t base = 0u;
          if (lane == 0) base = atomicAdd(&s_hi[1], (uint32_t)__popcll(hm));
          base = (uint32_t)__builtin_amdgcn_readfirstlane((int)base);
          const uint32_t slot = base + lanes_below(hm);
          if (hi && slot < 256u) s_hi[2 + slot] = key;
        }
      }
      __syncthreads();
      const uint32_t nhi = s_hi[1];
      if (total < (uint32_t)plan.KB) {
        theta = 0u;
      } else if (nhi >= (uint32_t)plan.KB && nhi <= 256u) {
        uint32_t x[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) x[q] = (uint32_t)(lane + 64 * q) < nhi ? s_hi[2 + lane + 64 * q] : 0u;
        theta = wave_kth_largest_radix4(x, plan.KB);
      } else {
        theta = lds_kth_key(fl.buf, total, (uint32_t)plan.KB, (uint32_t*)fl.cand);
      }
    } else {
      theta = 0u;
    }
    __syncthreads();
  }

  // ---- row results -----------------------------------------------------
  const float M = key2f(sh.bw[BW_MKEY]);
  const uint32_t rflags = sh.flags;
  int32_t status = ST_OK;
  if (rflags & F_INVALID) status = ST_EINVAL;
  else if (rflags & F_NONFINITE) status = ST_ENONFINITE;
  else if (A.out_ids && !s_pos_ok) status = ST_EINVAL;  // prediction position overflow

  if (status == ST_OK) {
    // Every element with key >= theta_f = row_threshold(M, theta) was
    // appended (every bound used was no larger), so the appended entries at
    // or above theta_f are exactly the row's: sorted, they hold the top-KB
    // and every relevant element, which is all the outputs and the tail read.
    const uint32_t theta_f = row_threshold(plan, P, M, theta);
    bool dense = fdense || (P.zcheck && plan.sampled);
    bool zfail = false;
    bool drawn = false;  // the certified tail made the draws
    int64_t ncand = 0;
    bool sorted = false;
    // a single draw that the wave path takes: its weights and scores can be
    // computed while the candidates are ranked
    const bool pre_draw = A.out_ids != nullptr && !P.greedy && (A.mode == MODE_VERIFY || A.n_draws == 1);
    bool have_pre = false;
    if (!dense) {
      const uint32_t cnt = sh.count;
      if (cnt <= (uint32_t)BUFCAP) {
        // every wave: order-free compaction of the buffer (one LDS atomic
        // per wave and pass; sh.ctr was cleared at the start) ...
        for (uint32_t i0 = 0; i0 < cnt; i0 += NT) {
          const uint32_t i = i0 + (uint32_t)tid;
          const uint64_t e = i < cnt ? fl.buf[i] : 0ull;
          const bool k = i < cnt && pk_key(e) >= theta_f;
          const uint64_t km = __ballot(k);
          if (km) {
            uint32_t base = 0u;
            if (lane == 0) base = atomicAdd(&sh.ctr, (uint32_t)__popcll(km));
            base = (uint32_t)__builtin_amdgcn_readfirstlane((int)base);
            const uint32_t slot = base + lanes_below(km);
            if (k && slot < (uint32_t)CAP) fl.cand[slot] = e;
          }
        }
        __syncthreads();
        const uint32_t m = sh.ctr;
        if (m <= 64u) {
          // ... then (<= 64 survivors, the common case) a rank sort: thread
          // t of waves 0..3 compares survivor t % 64 with survivors
          // 16 (t / 64) .. +15 and adds the number above it to that
          // survivor's rank. Meanwhile, for a single draw, wave 4 computes
          // each survivor's weight exp_d(z) and wave 5 its version-3 score
          // z + g (z = (l - M) / T with M the row maximum, the first sorted
          // value), in the order the draw reads them once permuted.
          const uint32_t i = (uint32_t)tid & 63u;
          const uint64_t x = i < m ? fl.cand[i] : 0ull;
          if (wave < 4) {
            const uint32_t j0 = (uint32_t)wave * 16u;
            if (i < m && j0 < m) {
              uint32_t above = 0u;
#pragma unroll
              for (uint32_t j = 0; j < 16; ++j) above += (j0 + j < m && fl.cand[j0 + j] > x) ? 1u : 0u;
              if (above) atomicAdd(&s_rank[i], above);
            }
          } else if (pre_draw && wave == 4) {
            if (i < m) s_wpre[i] = exp_d_inline(((double)key2f(pk_key(x)) - (double)M) / P.temperature);
          } else if (pre_draw && wave == 5 && P.version == YSKN_V3) {
            if (i < m) {
              const double z = ((double)key2f(pk_key(x)) - (double)M) / P.temperature;
              s_spre[i] = z + gumbel_from_key<true>(position_key(P.seed, s_pos), pk_id(x));
            }
          }
          __syncthreads();
          if ((uint32_t)tid < m) {  // wave 0 holds survivors 0..m-1
            const uint32_t r = s_rank[tid];
            fl.cand[r] = x;
            if (pre_draw) {
              fl.w[r] = s_wpre[tid];
              fl.w[64 + r] = s_spre[tid];
            }
          }
          have_pre = pre_draw;
        }
        __syncthreads();
        ncand = (int64_t)sh.ctr;
        sorted = ncand <= 64;
      } else if (cnt - (uint32_t)BUFCAP <= (uint32_t)A.dense_ld) {
        uint32_t nc = compact_entries(fl.buf, BUFCAP, fl.cand, CAP, theta_f, &sh.ctr, true);
        nc = compact_entries(spill, cnt - (uint32_t)BUFCAP, fl.cand, CAP, theta_f, &sh.ctr, false);
        ncand = (int64_t)nc;
      } else {
        ncand = (int64_t)CAP + 1;  // reservations outran the spill area: the dense path
      }
      dense = ncand > CAP || ncand < 1;
    }
    const uint64_t* cand;
    double* wbuf;
    if (!dense) {
      if (!sorted) {
        if (ncand <= NT) sort_desc_small(fl.cand, (uint64_t*)fl.w, (int)ncand);
        else sort_desc(fl.cand, (int)ncand);
      }
      cand = fl.cand;
      wbuf = fl.w;
    } else {
      const uint32_t trel = relevance_key(M, P.temperature);
      // a sampled version-3 row whose lists fit the waves' length: the cut
      // certified without sorting the row when the bounds allow it
      int64_t nc = 0;
      if constexpr (CERT) {
        if (!fdense && plan.sampled && plan.need_rel && P.version == YSKN_V3 && !P.zcheck)
          nc = dense_certified<DT, PEN>(A, P, rc, row, nseg, M, trel, plan, fl, red_f64, red_u64);
      }
      drawn = nc > 0;
      if (drawn) ncand = nc;
      cand = A.dense_a + (int64_t)row * A.dense_ld;
      wbuf = A.dense_w + (int64_t)row * A.dense_ld;
      if (!drawn) {
        ncand = dense_build<DT, PEN>(A, rc, row, trel, plan.need_rel, plan.KB, (uint32_t*)fl.cand,
                                     (uint64_t*)fl.buf);
        __syncthreads();
        if (P.zcheck && plan.sampled) {
          // The reference fails the row when any of its k candidates has a
          // non-finite z = (l - l_0) / T (output_head_sampler.rs:146-153); z
          // falls with l, so the k-th largest value decides.
          uint32_t* lw = (uint32_t*)fl.cand;
          const int64_t kk = plan.k_eff < (int64_t)V ? plan.k_eff : (int64_t)V;
          const uint32_t kkey = radix_kth_key<DT, PEN>(rc, V, kk, lw, lw + 512 + NW * 256);
          const double z = ((double)key2f(kkey) - (double)M) / P.temperature;
          zfail = !(z - z == 0.0);
          __syncthreads();
        }
        // the first 64 sorted candidates in LDS too: every output and the
        // one-wave tail read only those (LDS reads, not generic ones)
        for (int i = tid; i < 64; i += NT) fl.cand[i] = i < ncand ? cand[i] : 0ull;
      }
    }

    __syncthreads();  // the sorted candidates are visible to every thread
    // The row maximum is always a candidate: cand[0] is the argmax (larger
    // value, then smaller id).
    const uint32_t amax = pk_id(fl.cand[0]);

    // ---- outputs in raw order (wave 1, while wave 0 draws) ----------------
    // Raw values come from the keys (exact for every value but +-0, whose
    // sign the key drops, and for penalised rows, whose keys are of the
    // penalised values): only those are read again from the logits.
    const int ot = tid - 64;  // wave 1's lanes: 0..63
    // log of the mass (wave 1 alone, off the draw's path): one term per
    // wave, in lanes 0..NW-1
    // (more than 64 outputs: every wave writes them, and needs logZ)
    const bool big_out = CERT && (A.topn > 64 || A.n_lp > 64);
    double logZ = 0.0;
    if (A.want_mass && (wave == 1 || big_out)) {
      double t = 0.0;
      if (lane < n_mass && s_mref[lane] != -__builtin_inff()) t = s_mass[lane] * exp((double)s_mref[lane] - (double)M);
      logZ = log(wave_sum_f64_dpp(t));
    }
    auto raw_value = [&](uint64_t p) -> float {
      const float v = key2f(pk_key(p));
      if (PEN || v == 0.0f) return __uint_as_float(value_bits<DT, PEN>(rc, pk_id(p)));
      return v;
    };
    if (A.argmax && ot == 0) A.argmax[row] = amax;
    if (A.top8_ids && ot >= 0 && ot < 8) {
      const int i = ot;
      const bool in = i < ncand;
      A.top8_ids[(int64_t)row * 8 + i] = in ? pk_id(fl.cand[i]) : 0xffffffffu;
      A.top8_vals[(int64_t)row * 8 + i] = in ? raw_value(fl.cand[i]) : -__builtin_inff();
    }
    if (A.top20_ids && ot >= 0 && ot < 20) {
      const int i = ot;
      const bool in = i < ncand;
      A.top20_ids[(int64_t)row * 20 + i] = in ? pk_id(fl.cand[i]) : 0xffffffffu;
      A.top20_vals[(int64_t)row * 20 + i] = in ? raw_value(fl.cand[i]) : -__builtin_inff();
    }
    if (CERT && A.topn_ids && A.topn > 64) {
      for (int64_t i = tid; i < A.topn; i += NT) {
        const bool in = i < ncand;
        A.topn_ids[(int64_t)row * A.topn + i] = in ? pk_id(cand[i]) : 0xffffffffu;
        if (A.topn_vals) A.topn_vals[(int64_t)row * A.topn + i] = in ? raw_value(cand[i]) : -__builtin_inff();
      }
    } else if (A.topn_ids && ot >= 0 && ot < A.topn) {
      const int i = ot;
      const bool in = i < ncand;
      A.topn_ids[(int64_t)row * A.topn + i] = in ? pk_id(fl.cand[i]) : 0xffffffffu;
      if (A.topn_vals) A.topn_vals[(int64_t)row * A.topn + i] = in ? raw_value(fl.cand[i]) : -__builtin_inff();
    }
    if (CERT && A.n_lp > 64) {
      for (int64_t i = tid; i < A.n_lp; i += NT) {
        const bool in = i < ncand;
        double lp = -__builtin_inf();
        if (in) {
          const float l = PEN ? __uint_as_float(value_bits<DT, PEN>(rc, pk_id(cand[i]))) : key2f(pk_key(cand[i]));
          lp = ((double)l - (double)M) - logZ;
        }
        A.lp_ids[(int64_t)row * A.n_lp + i] = in ? pk_id(cand[i]) : 0xffffffffu;
        A.lp_vals[(int64_t)row * A.n_lp + i] = lp;
      }
    } else if (A.n_lp > 0 && ot >= 0 && ot < A.n_lp) {
      const int i = ot;
      const bool in = i < ncand;
      double lp = -__builtin_inf();
      if (in) {
        // (the sign of a zero does not change l - M)
        const float l = PEN ? __uint_as_float(value_bits<DT, PEN>(rc, pk_id(fl.cand[i]))) : key2f(pk_key(fl.cand[i]));
        lp = ((double)l - (double)M) - logZ;
      }
      A.lp_ids[(int64_t)row * A.n_lp + i] = in ? pk_id(fl.cand[i]) : 0xffffffffu;
      A.lp_vals[(int64_t)row * A.n_lp + i] = lp;
    }
    if (A.nll_targets && ot == 0) {
      const uint32_t t = A.nll_targets[row];
      if (t < (uint32_t)V) {
        const float l = __uint_as_float(value_bits<DT, PEN>(rc, t));
        A.nll_out[row] = ((double)M - (double)l) + logZ;
      } else {
        A.nll_out[row] = __builtin_nan("");
      }
    }
    if (A.nll_targets) {
      // an out-of-range target fails the row (every thread sees the same)
      if (A.nll_targets[row] >= (uint32_t)V) status = ST_EINVAL;
    }
    // ---- token selection ---------------------------------------------------
    if (zfail) status = ST_ENONFINITE;
    if (A.out_ids) {
      if (zfail) {
        const int nd = A.mode == MODE_VERIFY ? 1 : A.n_draws;
        for (int d = tid; d < nd; d += NT) A.out_ids[(int64_t)row * A.n_draws + d] = 0xffffffffu;
      } else if (P.greedy) {
        const int nd = A.mode == MODE_VERIFY ? 1 : A.n_draws;
        for (int d = tid; d < nd; d += NT) A.out_ids[(int64_t)row * A.n_draws + d] = amax;
      } else if (drawn) {
        // written by the certified tail
      } else if (ncand <= 64 && (A.mode == MODE_VERIFY || A.n_draws == 1)) {
        // one draw over at most 64 candidates: wave 0 alone
        if (wave == 0) {
          int c = (int)plan.k_eff < (int)ncand ? (int)plan.k_eff : (int)ncand;
          if (plan.need_rel) {
            const uint32_t trel = relevance_key(M, P.temperature);
            const int nrel = (int)__popcll(__ballot(lane < ncand && pk_key(fl.cand[lane < ncand ? lane : 0]) >= trel));
            c = (int)plan.k_eff < nrel ? (int)plan.k_eff : nrel;
          }
          sample_tail_wave(A, P, row, fl.cand, c, s_pos, fl.w, have_pre && !dense);
        }
      } else {
        int64_t c;
        if (plan.need_rel) {
          const uint32_t trel = relevance_key(M, P.temperature);
          int cr = 0;
          for (int64_t i = tid; i < ncand; i += NT) cr += (pk_key(cand[i]) >= trel) ? 1 : 0;
          const int64_t nrel = block_sum_int(cr, red_int);
          c = plan.k_eff < nrel ? plan.k_eff : nrel;
        } else {
          c = plan.k_eff;
        }
        sample_tail(A, P, row, cand, wbuf, c, &ts, red_f64, red_int, red_u64);
      }
    }
    if (tid == 0 && A.stats) {
      atomicAdd(&A.stats[STAT_ROWS], 1ull);
      if (dense) atomicAdd(&A.stats[STAT_DENSE_ROWS], 1ull);
      if (drawn) atomicAdd(&A.stats[STAT_CERT_ROWS], 1ull);
      atomicAdd(&A.stats[STAT_CANDIDATES], (unsigned long long)ncand);
    }
  } else if (A.out_ids) {
    const int nd = A.mode == MODE_VERIFY ? 1 : A.n_draws;
    for (int d = tid; d < nd; d += NT) A.out_ids[(int64_t)row * A.n_draws + d] = 0xffffffffu;
  }
  if (tid == 0) {
    A.status[row] = status;
    if (A.row_status) A.row_status[row] = status;
  }

  // ---- single-row decode: advance the device position and token ---------
  // (q35_sample.cu:206: *adv_pos += 1, *adv_tok = id). The host admits it
  // for one row only; the row's position was read before this point, so the
  // position counter may be the one the row was sampled at.
  if (A.mode == MODE_SAMPLE && A.adv_pos) {
    __syncthreads();
    if (tid == 0 && status == ST_OK) {
      const uint32_t tok = __hip_atomic_load(&A.out_ids[(int64_t)row * A.n_draws], __ATOMIC_RELAXED,
                                             __HIP_MEMORY_SCOPE_AGENT);
      *A.adv_pos += 1u;
      *A.adv_tok = tok;
    }
  }

  // ---- verify: the last finished row applies the acceptance rule --------
  // Rows are walked in order like speculation.rs:483-523: a failed row
  // fails the pass only when the walk reaches it (rows after the first
  // mismatch or EOS are never selected, :520-522). With a commit target the
  // position advances by the tokens emitted and the token becomes the last
  // of them, as Engine35::commit does on the host (engine35.cpp:1319-1329).
  if (A.mode == MODE_VERIFY) {
    __syncthreads();
    if (tid == 0) {
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
      const uint32_t old = __hip_atomic_fetch_add(A.vcount, 1u, __ATOMIC_RELAXED,
                                                  __HIP_MEMORY_SCOPE_AGENT);
      if (old == (uint32_t)(A.rows - 1)) {
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
        uint32_t emitted = 0, accepted = 0, token = 0xffffffffu;
        int32_t stop_eos = 0, vstatus = ST_OK;
        for (int j = 0; j < A.rows; ++j) {
          const int32_t sj = A.status[j];
          if (sj != ST_OK) {
            vstatus = sj;
            break;
          }
          const uint32_t sel = A.out_ids[j];
          ++emitted;
          token = sel;
          const bool matched = (j + 1 < A.rows) && A.drafts[j] == sel;
          accepted += matched ? 1u : 0u;
          for (int e = 0; e < A.n_eos; ++e)
            if (A.eos[e] == sel) stop_eos = 1;
          if (stop_eos || !matched) break;
        }
        if (vstatus != ST_OK) {
          emitted = 0;
          accepted = 0;
          token = 0xffffffffu;
          stop_eos = 0;
        }
        A.vresult[VR_ACCEPTED] = accepted;
        A.vresult[VR_EMITTED] = emitted;
        A.vresult[VR_TOKEN] = token;
        A.vresult[VR_STOP_EOS] = (uint32_t)stop_eos;
        A.vresult[VR_STATUS] = (uint32_t)vstatus;
        if (vstatus == ST_OK && A.adv_pos) {
          *A.adv_pos += emitted;
          *A.adv_tok = token;
        }
        __hip_atomic_store(A.vcount, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
  }
}
// ---------------------------------------------------------------------------
// Penalty preparation: the number of times each token occurs in the row's
// history (the frequency penalty's count; presence and repetition apply to
// any count > 0), laid out for a one-load lookup. Per row, word w of the vocabulary holds the membership bits of ids
// 32w..32w+31 and the number of distinct history ids below 32w; the counts of
// the distinct ids follow in id order, so id v's count is
// cnt[rank(w) + popcount(bits(w) below v)]. Built in LDS, a window of PW_WIN
// words at a time, with no sort: the history sits in registers (HCAP / 1024
// ids per thread), membership by LDS atomicOr, ranks by a block scan of the
// words' popcounts, counts by LDS atomicAdd at each id's rank.
// ---------------------------------------------------------------------------
constexpr int PP_NT = 1024;
constexpr int PP_PER = HCAP / PP_NT;
constexpr int PW_WIN = 8192;
constexpr int PW_PT = PW_WIN / PP_NT;
static_assert(PP_PER * PP_NT == HCAP && PW_PT * PP_NT == PW_WIN, "penalty prep geometry");

__global__ __launch_bounds__(PP_NT) void smp_penalty_prep(PenArgs A) {
  __shared__ uint32_t wb[PW_WIN];  // the window's membership bits
  __shared__ uint32_t wr[PW_WIN];  // the window's ranks
  __shared__ uint32_t cnt[HCAP];
  __shared__ uint32_t red[PP_NT / 64];
  __shared__ int s_bad;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, row = blockIdx.x;
  // (the parameters and the length are requested together: one round trip)
  const DevParams P = A.prm[A.prm_shared ? 0 : row];
  const int len = A.history_len ? A.history_len[row] : 0;
  if (!P.penalize) {
    if (tid == 0) A.len[row] = 0;
    return;
  }
  if (len < 0 || len > HCAP || (A.history_ld > 0 && (int64_t)len > A.history_ld)) {
    if (tid == 0) A.len[row] = -1;
    return;
  }
  // ids >= V are invalid; 0xffffffff (>= any V) marks an empty slot
  uint32_t h[PP_PER];
  bool bad = false;
#pragma unroll
  for (int k = 0; k < PP_PER; ++k) {
    const int i = tid + k * PP_NT;
    h[k] = 0xffffffffu;
    if (i < len) {
      h[k] = A.history[(int64_t)row * A.history_ld + i];
      bad |= h[k] >= (uint32_t)A.V;
    }
  }
  if (tid == 0) s_bad = 0;
  for (int i = tid; i < HCAP; i += PP_NT) cnt[i] = 0u;
  __syncthreads();
  if (bad) atomicOr(&s_bad, 1);
  __syncthreads();
  if (s_bad) {
    if (tid == 0) A.len[row] = -1;
    return;
  }
  const int words = (A.V + 31) >> 5;
  uint2* out = A.words + (int64_t)row * A.pw_ld;
  uint32_t carry = 0;  // distinct ids below the window
  for (int w0 = 0; w0 < words; w0 += PW_WIN) {
    const int nw = min(PW_WIN, words - w0);
#pragma unroll
    for (int j = 0; j < PW_PT; ++j) wb[tid * PW_PT + j] = 0u;
    __syncthreads();
#pragma unroll
    for (int k = 0; k < PP_PER; ++k) {
      const int w = (int)(h[k] >> 5) - w0;
      if (h[k] != 0xffffffffu && w >= 0 && w < nw) atomicOr(&wb[w], 1u << (h[k] & 31));
    }
    __syncthreads();
    uint32_t s = 0;
#pragma unroll
    for (int j = 0; j < PW_PT; ++j) s += __popc(wb[tid * PW_PT + j]);
    uint32_t inc = s;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const uint32_t y = __shfl_up(inc, o);
      if (lane >= o) inc += y;
    }
    if (lane == 63) red[wave] = inc;
    __syncthreads();
    uint32_t r = carry, tot = 0;
#pragma unroll
    for (int w = 0; w < PP_NT / 64; ++w) {
      r += (w < wave) ? red[w] : 0u;
      tot += red[w];
    }
    r += inc - s;
#pragma unroll
    for (int j = 0; j < PW_PT; ++j) {
      const int wi = tid * PW_PT + j;
      wr[wi] = r;
      r += __popc(wb[wi]);
    }
    __syncthreads();
    // coalesced: consecutive threads write consecutive words
    for (int wi = tid; wi < nw; wi += PP_NT) out[w0 + wi] = make_uint2(wb[wi], wr[wi]);
#pragma unroll
    for (int k = 0; k < PP_PER; ++k) {
      const int w = (int)(h[k] >> 5) - w0;
      if (h[k] != 0xffffffffu && w >= 0 && w < nw) {
        const uint32_t below = wb[w] & ((1u << (h[k] & 31)) - 1u);
        atomicAdd(&cnt[wr[w] + __popc(below)], 1u);
      }
    }
    carry += tot;
    __syncthreads();
  }
  uint32_t* co = A.cnt + (int64_t)row * HCAP;
  for (int i = tid; i < (int)carry; i += PP_NT) co[i] = cnt[i];
  if (tid == 0) A.len[row] = (int32_t)carry;
}

// ---------------------------------------------------------------------------
// Launches of fewer than CERT_ROWS rows, every segmented launch and every
// launch that uses a feature beyond plain sampling (verify, device
// positions, several draws, advance, NLL targets, lists longer than KBMAX,
// the forced dense path) use the general form: row segments, the certified
// dense tail, everything. The other large launches stream one row per block
// with the large form, which leaves all that out (a dense row there, rare,
// takes the sorting path): that kernel keeps the code of the stream and the
// common finish alone.
constexpr int CERT_ROWS = 192;

template <int DT, bool VEC, bool PEN>
static hipError_t launch_t(const SmpArgs& a, hipStream_t st) {
  const bool large = a.rows >= CERT_ROWS && a.nseg == 1 && a.mode == MODE_SAMPLE && a.pos_mode == POS_ARRAY &&
                     a.n_draws == 1 && a.adv_pos == nullptr && a.adv_tok == nullptr && a.nll_targets == nullptr &&
                     a.topn <= KBMAX && a.n_lp <= KBMAX && a.force_dense == 0;
  if (!large)
    hipLaunchKernelGGL((smp_row<DT, VEC, PEN, true>), dim3((unsigned)(a.rows * a.nseg)), dim3(NT), 0, st, a);
  else
    hipLaunchKernelGGL((smp_row<DT, VEC, PEN, false>), dim3((unsigned)(a.rows * a.nseg)), dim3(NT), 0, st, a);
  return hipGetLastError();
}

hipError_t launch_sample(const SmpArgs& a, int dtype, bool vec, bool pen, hipStream_t st) {
  if (dtype == 2) return pen ? launch_t<2, false, true>(a, st) : launch_t<2, false, false>(a, st);
  if (dtype == 0) {
    if (vec) return pen ? launch_t<0, true, true>(a, st) : launch_t<0, true, false>(a, st);
    return pen ? launch_t<0, false, true>(a, st) : launch_t<0, false, false>(a, st);
  }
  if (vec) return pen ? launch_t<1, true, true>(a, st) : launch_t<1, true, false>(a, st);
  return pen ? launch_t<1, false, true>(a, st) : launch_t<1, false, false>(a, st);
}

__global__ __launch_bounds__(NT) void smp_prefix_test(const double* w, double* S, int64_t c) {
  __shared__ PScanShared ps;
  exact_prefix(w, S, c, &ps);
}

hipError_t launch_prefix_test(const double* w, double* S, int64_t c, hipStream_t st) {
  hipLaunchKernelGGL(smp_prefix_test, dim3(1), dim3(NT), 0, st, w, S, c);
  return hipGetLastError();
}

hipError_t launch_penalty_prep(const PenArgs& a, hipStream_t st) {
  hipLaunchKernelGGL(smp_penalty_prep, dim3(a.rows), dim3(1024), 0, st, a);
  return hipGetLastError();
}

}  // namespace yskn
