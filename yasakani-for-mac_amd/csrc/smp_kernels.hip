// smp_kernels.hip -- gfx950 kernels of the per-step sampling path.
//
// Two launches per call (three with penalties):
//
//  smp_scan   S * rows blocks of 8 wave64s (S = ceil(V / 16,384)). Each wave
//             owns 2,048 consecutive logits of a row in registers (32 per
//             lane, coalesced 16-byte loads). Per wave: lane maxima, the wave
//             maximum, a top-KB threshold from the sorted lane maxima; one
//             block barrier shares them. The block stores its bounds in its
//             own slot (relaxed agent-scope store, no contention) and its 8
//             largest lane maxima. Each wave then keeps only the elements
//             that can matter to the reference algorithm: (a) elements whose
//             binary64 weight exp_d((l - M)/T) can reach 2^-53 (smaller
//             weights are absorbed by the reference's serial binary64 sums,
//             whose running value is >= 1) and (b) a superset of the row's
//             top-KB by value. If its block's bounds leave more than WCAP
//             elements, the wave reads the slots of the row's other blocks
//             (any subset gives valid bounds). A wave still over WCAP hands
//             over nothing and is re-read by the finisher. The wave also sums
//             exp(l - m) over the elements near its reference m for the
//             logprob normaliser.
//  smp_finish one block per row. Exact row maximum and top-KB bound from the
//             wave records and the published lane maxima give the final
//             threshold; the survivors (which do not depend on timing) are
//             gathered, sorted by (value desc, id asc) and the reference's
//             serial binary64 truncation and draw run on them
//             (output_head_sampler.rs:136-212). Rows with more survivors than
//             LDS holds take the exact "dense" path: radix select, stable LSD
//             radix sort in global scratch, same tail.
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
__device__ __forceinline__ double wave_sum_f64(double v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  return v;
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
  const uint32_t* bitmap;  // penalty bitmap of the row (or NULL)
  const uint32_t* pids;
  const uint32_t* pcnt;
  int32_t plen;
  float rep, pres, freq;
};

__device__ __forceinline__ uint32_t pen_count(const RowCtx& r, uint32_t v) {
  int lo = 0, hi = r.plen;
  while (lo < hi) {
    const int mid = (lo + hi) >> 1;
    if (r.pids[mid] < v) lo = mid + 1; else hi = mid;
  }
  return (lo < r.plen && r.pids[lo] == v) ? r.pcnt[lo] : 0u;
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

template <int DT>
__device__ __forceinline__ uint32_t raw_bits(const RowCtx& r, int64_t i) {
  if (DT == 0) return ((const uint32_t*)r.base)[i];
  return (uint32_t)((const uint16_t*)r.base)[i] << 16;
}

template <int DT, bool PEN>
__device__ __forceinline__ uint32_t value_bits(const RowCtx& r, int64_t i) {
  uint32_t b = raw_bits<DT>(r, i);
  if (PEN && r.bitmap) {
    if ((r.bitmap[i >> 5] >> (i & 31)) & 1u) b = penalize(b, pen_count(r, (uint32_t)i), r);
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
  p.need_rel = p.sampled && p.k_eff > KBMAX;
  return p;
}

__device__ __forceinline__ uint64_t position_of(const SmpArgs& A, int row, int d) {
  if (A.mode == MODE_VERIFY) return *A.base_position + (uint64_t)row + 1u;
  return A.positions[(int64_t)row * A.n_draws + d];
}

// ---------------------------------------------------------------------------
// LDS layout of the finisher (88 KB); the dense path borrows `cand`.
// ---------------------------------------------------------------------------
struct FinishLds {
  uint64_t cand[CAP];          // survivors, sorted (compact path)
  double w[CAP];               // weights of the first c candidates (compact path)
  uint32_t cnt[MAX_WAVES];     // per wave: candidates handed over (0 if re-scanned)
  uint32_t off[MAX_WAVES];     // exclusive prefix of cnt
  uint32_t res[MAX_WAVES];     // indices of the waves to re-scan
};

// ---------------------------------------------------------------------------
// Truncation and draw on the first c sorted candidates (output_head_sampler.rs
// :136-212). cand/w are generic pointers (LDS or global scratch).
// ---------------------------------------------------------------------------
struct TailShared {
  uint32_t retained;
  double mass;  // serial binary64 sum of the retained weights (version 2)
  double best;
  int pick;
};

__device__ void sample_tail(const SmpArgs& A, const DevParams& P, int row, const uint64_t* cand,
                            double* w, int64_t c, TailShared* ts, double* redd, int* redi,
                            uint64_t* redu) {
  const int tid = threadIdx.x;
  const double T = P.temperature;
  const float v0 = key2f(pk_key(cand[0]));
  // weights: widen, subtract, divide, exp_d -- in candidate order
  for (int64_t j = tid; j < c; j += NT) {
    const double z = ((double)key2f(pk_key(cand[j])) - (double)v0) / T;
    w[j] = exp_d(z);
  }
  __syncthreads();
  if (tid == 0) {
    double total = 0.0;
    for (int64_t j = 0; j < c; ++j) total = total + w[j];
    int64_t n = c;
    double prefix = 0.0;
    const double thr = P.top_p * total;
    for (int64_t j = 0; j < c; ++j) {
      prefix = prefix + w[j];
      if (prefix >= thr) {
        n = j + 1;
        break;
      }
    }
    if (P.min_p > 0.0) {
      int64_t m = 1;
      while (m < n && w[m] >= P.min_p) ++m;
      n = m;
    }
    double mass = 0.0;
    if (P.version != YSKN_V3) {
      for (int64_t j = 0; j < n; ++j) mass = mass + w[j];
    }
    ts->retained = (uint32_t)n;
    ts->mass = mass;
  }
  __syncthreads();
  const int64_t r = ts->retained;
  const int nd = A.mode == MODE_VERIFY ? 1 : A.n_draws;
  if (P.version == YSKN_V3 && nd == 1) {
    // one draw: candidates in parallel, argmax of z + g with the earliest
    // candidate winning ties (strict > in candidate order)
    const uint64_t pk = position_key(P.seed, position_of(A, row, 0));
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
    // reduce (best desc, index asc) across the block
    const int lane = tid & 63, wave = tid >> 6;
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
      redi[wave] = (int)bj;
    }
    __syncthreads();
    if (tid == 0) {
      double b = redd[0];
      int jj = redi[0];
      for (int q = 1; q < NW; ++q) {
        if (redd[q] > b || (redd[q] == b && redi[q] < jj)) {
          b = redd[q];
          jj = redi[q];
        }
      }
      const uint32_t id = pk_id(cand[jj]);
      A.out_ids[(int64_t)row * A.n_draws] = id;
    }
    __syncthreads();
    return;
  }
  // several draws (or version 2): one thread per draw, serial over candidates
  for (int d = tid; d < nd; d += NT) {
    const uint64_t pos = position_of(A, row, d);
    int64_t pick = r - 1;
    if (P.version == YSKN_V3) {
      const uint64_t pk = position_key(P.seed, pos);
      double best = -__builtin_inf();
      for (int64_t j = 0; j < r; ++j) {
        const uint64_t cj = cand[j];
        const double z = ((double)key2f(pk_key(cj)) - (double)v0) / T;
        const double s = z + gumbel_from_key(pk, pk_id(cj));
        if (s > best) {
          best = s;
          pick = j;
        }
      }
    } else {
      const double u = uniform_v2(P.seed, pos);
      const double thr = u * ts->mass;
      double prefix = 0.0;
      for (int64_t j = 0; j < r; ++j) {
        prefix = prefix + w[j];
        if (thr < prefix) {
          pick = j;
          break;
        }
      }
    }
    A.out_ids[(int64_t)row * A.n_draws + d] = pk_id(cand[pick]);
  }
  __syncthreads();
}

// ---------------------------------------------------------------------------
// Dense path: exact sorted order of every element with key >= theta_D.
// ---------------------------------------------------------------------------
template <int DT, bool PEN>
__device__ int64_t dense_build(const SmpArgs& A, const RowCtx& rc, int row, uint32_t theta_rel,
                               bool need_rel, int KB, uint32_t* lds, int* redi) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int V = A.V;
  uint32_t* hist = lds;              // 256
  uint32_t* dbase = lds + 256;       // 256
  uint32_t* wcnt = lds + 512;        // NW * 256
  uint32_t* bc = lds + 512 + NW * 256;  // broadcast words
  // (a) exact KB-th largest key: four 8-bit radix passes from the top
  uint32_t prefix = 0, mask = 0;
  int need = KB;
  for (int pass = 0; pass < 4; ++pass) {
    const int shift = 24 - 8 * pass;
    for (int i = tid; i < 256; i += NT) hist[i] = 0;
    __syncthreads();
    for (int64_t i = tid; i < V; i += NT) {
      const uint32_t k = f2key(value_bits<DT, PEN>(rc, i));
      if ((k & mask) == prefix) atomicAdd(&hist[(k >> shift) & 255u], 1u);
    }
    __syncthreads();
    if (tid == 0) {
      int cum = 0, dsel = 0;
      for (int d = 255; d >= 0; --d) {
        const int h = (int)hist[d];
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
    need = (int)bc[1];
    __syncthreads();
  }
  uint32_t theta = prefix;
  if (need_rel && theta_rel < theta) theta = theta_rel;
  if (theta < 1u) theta = 1u;
  // (b) order-preserving compaction of key >= theta into dense_a
  uint64_t* da = A.dense_a + (int64_t)row * A.dense_ld;
  uint64_t* db = A.dense_b + (int64_t)row * A.dense_ld;
  int64_t n = 0;
  for (int64_t base = 0; base < V; base += NT) {
    const int64_t i = base + tid;
    uint64_t p = 0;
    int f = 0;
    if (i < V) {
      const uint32_t k = f2key(value_bits<DT, PEN>(rc, i));
      if (k >= theta) {
        f = 1;
        p = pack(k, (uint32_t)i);
      }
    }
    int tot;
    const int off = block_excl_scan(f, redi, &tot);
    if (f) da[n + off] = p;
    n += tot;
  }
  __syncthreads();
  // (c) stable LSD radix sort on the key, descending (digit = 255 - byte)
  for (int pass = 0; pass < 4; ++pass) {
    const int shift = 32 + 8 * pass;
    uint64_t* src = (pass & 1) ? db : da;
    uint64_t* dst = (pass & 1) ? da : db;
    for (int i = tid; i < 256; i += NT) hist[i] = 0;
    __syncthreads();
    for (int64_t i = tid; i < n; i += NT) {
      const uint32_t d = 255u - (uint32_t)((src[i] >> shift) & 255u);
      atomicAdd(&hist[d], 1u);
    }
    __syncthreads();
    if (tid == 0) {
      uint32_t run = 0;
      for (int d = 0; d < 256; ++d) {
        dbase[d] = run;
        run += hist[d];
      }
    }
    __syncthreads();
    for (int64_t base = 0; base < n; base += NT) {
      const int64_t i = base + tid;
      const bool valid = i < n;
      const uint64_t p = valid ? src[i] : 0ull;
      const uint32_t d = valid ? 255u - (uint32_t)((p >> shift) & 255u) : 0u;
      for (int j = tid; j < NW * 256; j += NT) wcnt[j] = 0;
      __syncthreads();
      uint64_t peers = __ballot(valid);
#pragma unroll
      for (int b = 0; b < 8; ++b) {
        const bool bit = (d >> b) & 1u;
        const uint64_t bal = __ballot(bit);
        peers &= bit ? bal : ~bal;
      }
      const uint64_t below = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
      const uint32_t rank = (uint32_t)__popcll(peers & below);
      if (valid && rank == 0) wcnt[wave * 256 + d] = (uint32_t)__popcll(peers);
      __syncthreads();
      if (valid) {
        uint32_t off = dbase[d] + rank;
        for (int q = 0; q < wave; ++q) off += wcnt[q * 256 + d];
        dst[off] = p;
      }
      __syncthreads();
      if (tid < 256) {
        uint32_t s = 0;
        for (int q = 0; q < NW; ++q) s += wcnt[q * 256 + tid];
        dbase[tid] += s;
      }
      __syncthreads();
    }
  }
  // four passes: the sorted result is back in dense_a
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
  rc.bitmap = nullptr;
  rc.pids = nullptr;
  rc.pcnt = nullptr;
  rc.plen = 0;
  rc.rep = P.rep;
  rc.pres = P.pres;
  rc.freq = P.freq;
  if (PEN && P.penalize) {
    rc.plen = A.pen_len[row];
    if (rc.plen < 0) {
      *flags |= F_INVALID;
      rc.plen = 0;
    } else {
      rc.bitmap = A.pen_bitmap + (int64_t)row * A.bm_ld;
      rc.pids = A.pen_ids + (int64_t)row * HCAP;
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
// smp_scan: one wave per 2,048 logits.
// ---------------------------------------------------------------------------
template <int DT, bool VEC, bool PEN>
__global__ __launch_bounds__(NTS) __attribute__((amdgpu_waves_per_eu(6))) void smp_scan(SmpArgs A) {
  __shared__ uint64_t s_wmax[NWS];
  __shared__ uint32_t s_wtb[NWS];
  __shared__ uint32_t s_top[NWS * TOPS];

  // wave index and every per-wave quantity below are uniform: keep them in
  // scalar registers (readfirstlane) so the 32 keys own the vector file
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int S = A.S;
  const int32_t V = A.V;
  // Workgroups are dealt round-robin to the 8 XCDs (linear id mod 8). Groups
  // of 8 rows are laid out so that all S blocks of a row share one XCD: they
  // are dispatched together by one dispatcher and their bounds arrive early.
  int row, seg;
  {
    const int b = blockIdx.x;
    const int full = (A.rows / 8) * 8;  // rows in complete groups of 8
    if (b < full * S) {
      const int g = b / (8 * S), r8 = b - g * 8 * S;
      row = g * 8 + (r8 & 7);
      seg = r8 >> 3;
    } else {
      const int r = b - full * S;
      row = full + r / S;
      seg = r - (r / S) * S;
    }
  }
  const DevParams P = A.prm[A.prm_shared ? 0 : row];
  const RowPlan plan = make_plan(A, P);
  uint32_t wflags = 0;
  const RowCtx rc = make_rowctx<PEN>(A, P, row, DT == 0 ? 4 : 2, &wflags);

  // ---- load 32 logits per lane as raw bits ------------------------------
  // Element of (q, c) for this lane: e = ebase + q * 64 * GRP + c (32-bit:
  // V <= 4,194,304). A wave whose 2,048 elements are all inside the row
  // (every wave but the row's last) runs without per-element bounds checks.
  constexpr int GRP = (DT == 0) ? 4 : 8;  // elements per 16-byte load
  constexpr int NGRP = EPT / GRP;
  const uint32_t w0 = (uint32_t)seg * SEG + (uint32_t)wave * WSEG;
  const uint32_t ebase = w0 + (uint32_t)lane * GRP;
  const bool full = w0 + WSEG <= (uint32_t)V;
  uint32_t key[EPT];
  if (VEC && full) {
    const uint4* src = (const uint4*)(rc.base + (size_t)ebase * (DT == 0 ? 4 : 2));
#pragma unroll
    for (int q = 0; q < NGRP; ++q) {
      const uint4 v = src[q * 64];
      if (DT == 0) {
        key[q * 4 + 0] = v.x;
        key[q * 4 + 1] = v.y;
        key[q * 4 + 2] = v.z;
        key[q * 4 + 3] = v.w;
      } else {
        key[q * 8 + 0] = v.x << 16;
        key[q * 8 + 1] = v.x & 0xffff0000u;
        key[q * 8 + 2] = v.y << 16;
        key[q * 8 + 3] = v.y & 0xffff0000u;
        key[q * 8 + 4] = v.z << 16;
        key[q * 8 + 5] = v.z & 0xffff0000u;
        key[q * 8 + 6] = v.w << 16;
        key[q * 8 + 7] = v.w & 0xffff0000u;
      }
    }
  } else {
#pragma unroll
    for (int q = 0; q < NGRP; ++q) {
#pragma unroll
      for (int c = 0; c < GRP; ++c) {
        const uint32_t e = ebase + q * 64 * GRP + c;
        key[q * GRP + c] = e < (uint32_t)V ? raw_bits<DT>(rc, e) : 0u;
      }
    }
  }
  // ---- values, lane max (first index on ties: indices grow with q, c) ---
  // The hot loop works on binary32 values: IEEE comparisons treat -0 and +0
  // as equal, exactly like the canonical keys; 32-bit keys are formed only
  // for the lane maximum and for the elements handed over. Absent elements
  // (past the row's end) are -inf, which no threshold keeps.
  float val[EPT];
  bool bad = false;
  float lmax = -__builtin_inff();
  uint32_t imax = 0;
#pragma unroll
  for (int q = 0; q < NGRP; ++q) {
    uint32_t wbits = 0;
    const uint32_t e0 = ebase + q * 64 * GRP;
    if (PEN && rc.bitmap && e0 < (uint32_t)V) wbits = rc.bitmap[e0 >> 5];
#pragma unroll
    for (int c = 0; c < GRP; ++c) {
      const uint32_t e = e0 + c;
      uint32_t b = key[q * GRP + c];
      float v = -__builtin_inff();
      if (full || e < (uint32_t)V) {
        if (PEN && rc.bitmap && ((wbits >> (e & 31)) & 1u)) b = penalize(b, pen_count(rc, e), rc);
        v = __uint_as_float(b);
        bad |= __builtin_amdgcn_class(v, 0x207) != 0;  // signaling/quiet NaN, +-inf
      }
      val[q * GRP + c] = v;
      // track the offset (an immediate) rather than the index: no per-element
      // index register stays live into the hand-over below
      if (v > lmax) {
        lmax = v;
        imax = q * 64 * GRP + c;
      }
    }
  }
  imax += ebase;
  if (__ballot(bad)) wflags |= F_NONFINITE;
  const uint32_t kmax = lmax == -__builtin_inff() ? 0u : f2key(__float_as_uint(lmax));
  const uint64_t wmax = wave_max_u64(kmax ? pack(kmax, imax) : 0ull);
  // Top-KB threshold of the block: per wave the ceil(KB/8)-th largest lane
  // maximum (0 where too few lanes hold data); the minimum over the block's
  // 8 waves has at least 8 * ceil(KB/8) >= KB elements at or above it.
  const uint32_t lsorted = wave_sort_asc(kmax);
  const uint32_t wb = __shfl(lsorted, 64 - (plan.KB + NWS - 1) / NWS);
  if (lane == 0) {
    s_wmax[wave] = wmax;
    s_wtb[wave] = wb;
  }
  if (lane >= 64 - TOPS) s_top[wave * TOPS + lane - (64 - TOPS)] = lsorted;
  __syncthreads();
  // The block publishes its TOPS largest lane maxima: distinct elements of
  // the row, from which the finisher takes a row-wide top-KB bound.
  if (wave == 0) {
    const uint32_t t = wave_sort_asc(s_top[lane]);
    if (lane >= 64 - TOPS)
      A.tops[((int64_t)row * MAX_SEGMENTS + seg) * TOPS + lane - (64 - TOPS)] = t;
  }
  // lane w < 8 reads wave w's record; three shuffle steps reduce them (few
  // registers live next to the 32 keys)
  uint64_t bmax = lane < NWS ? s_wmax[lane] : 0ull;
  uint32_t thb = lane < NWS ? s_wtb[lane] : 0xffffffffu;
#pragma unroll
  for (int o = NWS / 2; o > 0; o >>= 1) {
    const uint64_t ob = __shfl_xor(bmax, o);
    const uint32_t oc = __shfl_xor(thb, o);
    bmax = ob > bmax ? ob : bmax;
    thb = oc < thb ? oc : thb;
  }
  // (readfirstlane yields int: convert through uint32_t, never sign-extend)
  bmax = ((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(bmax >> 32)) << 32) |
         (uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)bmax);
  const uint32_t th1 = (uint32_t)__builtin_amdgcn_readfirstlane(thb);
  const uint32_t key_b = pk_key(bmax);

  // ---- row bounds. Every block stores its max key and top-KB threshold in
  // its own slot; a wave first filters with its block's own bounds and reads
  // the row's slots (those of the blocks that got there first) only if it
  // would keep more than WCAP elements. Any subset of the slots gives valid
  // (if weaker) bounds, so relaxed agent-scope stores and loads suffice,
  // nothing waits, and no address is contended.
  uint64_t* const slots = A.slots + (int64_t)row * MAX_SEGMENTS;
  if (tid == 0)
    __hip_atomic_store(slots + seg, ((uint64_t)th1 << 32) | (uint64_t)key_b, __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
  uint32_t mkey = key_b;
  uint32_t theta = A.force_dense ? 0xffffffffu : row_threshold(plan, P, key2f(mkey), th1);
  // survivors of this lane as a bit mask; run = survivors of the wave
  float thf = key_threshold_float(theta);
  uint32_t keep = 0;
#pragma unroll
  for (int i = 0; i < EPT; ++i) keep |= (val[i] >= thf ? 1u : 0u) << i;
  uint32_t run = (uint32_t)__builtin_amdgcn_readfirstlane(wave_sum_int(__popc(keep)));
  // at most two reads of the slots, the second after a short sleep that lets
  // more of the row's blocks publish; a wave still over WCAP is re-read by
  // the finisher
  for (int attempt = 0; attempt < 2 && run > (uint32_t)WCAP && !A.force_dense; ++attempt) {
    if (attempt > 0) __builtin_amdgcn_s_sleep(127);
    uint32_t hm = key_b, hk = th1;
    for (int s0 = 0; s0 < S; s0 += 64) {
      if (s0 + lane < S) {
        const uint64_t v = __hip_atomic_load(slots + s0 + lane, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        hm = (uint32_t)v > hm ? (uint32_t)v : hm;
        hk = (uint32_t)(v >> 32) > hk ? (uint32_t)(v >> 32) : hk;
      }
    }
    hm = wave_max_u32(hm);
    hk = wave_max_u32(hk);
    mkey = (uint32_t)__builtin_amdgcn_readfirstlane(hm);
    theta = row_threshold(plan, P, key2f(mkey), (uint32_t)__builtin_amdgcn_readfirstlane(hk));
    thf = key_threshold_float(theta);
    keep = 0;
#pragma unroll
    for (int i = 0; i < EPT; ++i) keep |= (val[i] >= thf ? 1u : 0u) << i;
    run = (uint32_t)__builtin_amdgcn_readfirstlane(wave_sum_int(__popc(keep)));
  }
  const float m_ref = key2f(mkey);

  // ---- logprob mass relative to m_ref (terms below m_ref - ZMASS left out).
  // Terms are binary32 exponentials accumulated in binary64: next to the
  // row maximum's term (1.0) the small terms must not be rounded away, since
  // the top token's logprob is -log(1 + their sum).
  double wmass = 0.0;
  if (A.want_mass) {
    const float lo = m_ref - ZMASS;
    double acc = 0.0;
#pragma unroll
    for (int q = 0; q < NGRP; ++q) {
      bool any = false;
#pragma unroll
      for (int c = 0; c < GRP; ++c) any |= val[q * GRP + c] >= lo;
      if (__ballot(any)) {
#pragma unroll
        for (int c = 0; c < GRP; ++c) {
          const float v = val[q * GRP + c];
          const float t = v >= lo ? (v - m_ref) * 1.4426950408889634f : -__builtin_inff();
          acc += (double)__builtin_amdgcn_exp2f(t);
        }
      }
    }
    wmass = wave_sum_f64(acc);
  }

  // ---- hand over the survivors (or nothing if more than WCAP) -----------
  if (run <= (uint32_t)WCAP && run > 0) {
    const uint32_t mine = (uint32_t)__popc(keep);
    uint32_t slot = (uint32_t)wave_incl_scan((int)mine, lane) - mine;
    // uniform base, 32-bit per-lane slot: one register for the address
    uint64_t* const base = A.wave_cand + (((int64_t)row * S + seg) * NWS + wave) * WCAP;
#pragma unroll
    for (int q = 0; q < NGRP; ++q) {
#pragma unroll
      for (int c = 0; c < GRP; ++c) {
        if ((keep >> (q * GRP + c)) & 1u)
          base[slot++] = pack(f2key(__float_as_uint(val[q * GRP + c])), ebase + q * 64 * GRP + c);
      }
    }
  }
  if (lane == 0) {
    WaveRec r;
    r.maxp = wmax;
    r.mass = wmass;
    r.mref = m_ref;
    r.count = run <= (uint32_t)WCAP ? run : RESCAN;
    r.th1 = th1;
    r.flags = wflags;
    A.wave_rec[((int64_t)row * S + seg) * NWS + wave] = r;
  }
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

// ---------------------------------------------------------------------------
// smp_finish: one block per row.
// ---------------------------------------------------------------------------
template <int DT, bool PEN>
__global__ __launch_bounds__(NT) void smp_finish(SmpArgs A) {
  __shared__ FinishLds fl;
  __shared__ uint64_t red_u64[NW];
  __shared__ double red_f64[NW];
  __shared__ int red_int[NW];
  __shared__ uint32_t red_u32[NW];
  __shared__ uint32_t bc[4];
  __shared__ TailShared ts;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int row = blockIdx.x;
  const int32_t V = A.V;
  const int W = A.S * NWS;
  const DevParams P = A.prm[A.prm_shared ? 0 : row];
  const RowPlan plan = make_plan(A, P);
  uint32_t pflags = 0;
  const RowCtx rc = make_rowctx<PEN>(A, P, row, DT == 0 ? 4 : 2, &pflags);
  const WaveRec* recs = A.wave_rec + (int64_t)row * W;

  // ---- wave records: row max, top-KB threshold, flags, counts -----------
  uint64_t rmax = 0, rkb = 0;
  uint32_t rflags = pflags;
  for (int w = tid; w < W; w += NT) {
    const WaveRec r = recs[w];
    rmax = r.maxp > rmax ? r.maxp : rmax;
    rkb = r.th1 > rkb ? r.th1 : rkb;
    rflags |= r.flags;
    fl.cnt[w] = r.count == RESCAN ? 0u : r.count;
    fl.res[w] = r.count == RESCAN ? 1u : 0u;
  }
  rmax = block_max_u64(rmax, red_u64);
  rkb = block_max_u64(rkb, red_u64);
  {
    // OR of the flags across the block: every decision below (status, dense
    // or compact) must be uniform over the block's threads
    uint32_t f = rflags;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) f |= __shfl_xor(f, o);
    __syncthreads();
    if (lane == 0) red_u32[wave] = f;
    __syncthreads();
    f = 0;
#pragma unroll
    for (int w = 0; w < NW; ++w) f |= red_u32[w];
    rflags = f;
  }
  // exclusive scans of the counts and of the re-scan flags; thread t owns
  // the four records 4t .. 4t+3 (W <= MAX_WAVES = 4 * NT)
  int csum = 0, nres = 0;
  {
    uint32_t c4[4], r4[4];
    int sc = 0, sr = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int w = 4 * tid + i;
      c4[i] = w < W ? fl.cnt[w] : 0u;
      r4[i] = w < W ? fl.res[w] : 0u;
      sc += (int)c4[i];
      sr += (int)r4[i];
    }
    const int exc = block_excl_scan(sc, red_int, &csum);
    const int exr = block_excl_scan(sr, red_int, &nres);
    __syncthreads();  // every read of fl.res above precedes the list writes
    int oc = exc, orr = exr;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int w = 4 * tid + i;
      if (w < W) {
        fl.off[w] = (uint32_t)oc;
        oc += (int)c4[i];
        if (r4[i]) fl.res[orr++] = (uint32_t)w;
      }
    }
  }
  const float M = key2f(pk_key(rmax));
  double logZ = 0.0;
  if (A.want_mass) {
    double part = 0.0;
    for (int w = tid; w < W; w += NT) {
      const WaveRec r = recs[w];
      if (r.maxp) part += r.mass * exp((double)r.mref - (double)M);
    }
    logZ = log(block_sum_f64(part, red_f64));
  }
  int32_t status = ST_OK;
  if (rflags & F_INVALID) status = ST_EINVAL;
  else if (rflags & F_NONFINITE) status = ST_ENONFINITE;

  if (status == ST_OK) {
    // Final threshold from exact row quantities: every wave filtered with
    // bounds no larger than these, so the survivors gathered below are
    // exactly the row's elements with key >= theta_f, whatever the timing.
    // Row-wide top-KB bound from the lane maxima the scan blocks published
    // (distinct elements of this row, all written by this call): the KB-th
    // largest of them has at least KB elements at or above it. At most 512
    // are used: the `per` largest of each block.
    uint32_t theta_pub = 0u;
    {
      const int S = A.S;
      const int per = S * TOPS <= NT ? TOPS : (NT / S > 0 ? NT / S : 1);
      const int npub = per * S < NT ? per * S : NT;
      uint32_t* pub = (uint32_t*)fl.w;
      if (tid == 0) bc[1] = 0u;
      if (tid < npub) {
        const int sg = tid / per, k = tid - sg * per;
        pub[tid] = A.tops[((int64_t)row * MAX_SEGMENTS + sg) * TOPS + (TOPS - 1 - k)];
      }
      __syncthreads();
      if (tid < npub) {
        const uint32_t x = pub[tid];
        if (x != 0u) {
          int rank = 0;
#pragma unroll 16
          for (int i = 0; i < npub; ++i) {
            const uint32_t y = pub[i];
            rank += (y > x || (y == x && i < tid)) ? 1 : 0;
          }
          if (rank == plan.KB - 1) bc[1] = x;
        }
      }
      __syncthreads();
      theta_pub = bc[1];
    }
    const uint32_t theta_f =
        row_threshold(plan, P, M, (uint32_t)rkb > theta_pub ? (uint32_t)rkb : theta_pub);
    bool dense = A.force_dense != 0;
    const uint64_t* cand;
    double* wbuf;
    int64_t ncand = 0;
    if (!dense) {
      if (tid == 0) bc[0] = 0u;
      __syncthreads();
      const uint64_t* wc = A.wave_cand + (int64_t)row * W * WCAP;
      // (a) candidates handed over by the waves
      for (int i0 = 0; i0 < csum; i0 += NT) {
        const int idx = i0 + tid;
        bool keep = false;
        uint64_t p = 0;
        if (idx < csum) {
          int lo = 0, hi = W - 1;  // largest w with off[w] <= idx
          while (lo < hi) {
            const int mid = (lo + hi + 1) >> 1;
            if ((int)fl.off[mid] <= idx) lo = mid; else hi = mid - 1;
          }
          p = wc[(int64_t)lo * WCAP + (idx - (int)fl.off[lo])];
          keep = pk_key(p) >= theta_f;
        }
        const uint64_t m = __ballot(keep);
        uint32_t base = 0;
        if (lane == 0 && m) base = atomicAdd(&bc[0], (uint32_t)__popcll(m));
        base = __shfl(base, 0);
        const uint32_t slot = base + (uint32_t)__popcll(m & ((lane == 0) ? 0ull : (~0ull >> (64 - lane))));
        if (keep && slot < (uint32_t)CAP) fl.cand[slot] = p;
      }
      // (b) waves that handed over nothing: read their logits again, four
      // consecutive elements per thread (one 16-byte or 8-byte load when the
      // rows are aligned), two groups per iteration
      const int64_t ngrp = (int64_t)nres * (WSEG / 4);
      for (int64_t t0 = 0; t0 < ngrp; t0 += 2 * NT) {
        uint32_t kk[2][4];
        int64_t e0[2];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const int64_t t = t0 + h * NT + tid;
          e0[h] = 0;
#pragma unroll
          for (int c = 0; c < 4; ++c) kk[h][c] = 0u;
          if (t < ngrp) {
            e0[h] = (int64_t)fl.res[t / (WSEG / 4)] * WSEG + (t % (WSEG / 4)) * 4;
            if (!PEN && A.vec && e0[h] + 4 <= V) {
              uint32_t b[4];
              if (DT == 0) {
                const uint4 q = *(const uint4*)(rc.base + e0[h] * 4);
                b[0] = q.x; b[1] = q.y; b[2] = q.z; b[3] = q.w;
              } else {
                const uint2 q = *(const uint2*)(rc.base + e0[h] * 2);
                b[0] = q.x << 16; b[1] = q.x & 0xffff0000u; b[2] = q.y << 16; b[3] = q.y & 0xffff0000u;
              }
#pragma unroll
              for (int c = 0; c < 4; ++c) kk[h][c] = f2key(b[c]);
            } else {
#pragma unroll
              for (int c = 0; c < 4; ++c)
                kk[h][c] = (e0[h] + c < V) ? f2key(value_bits<DT, PEN>(rc, e0[h] + c)) : 0u;
            }
          }
        }
#pragma unroll
        for (int h = 0; h < 2; ++h) {
#pragma unroll
          for (int c = 0; c < 4; ++c) {
            const bool keep = kk[h][c] >= theta_f;
            const uint64_t m = __ballot(keep);
            uint32_t base = 0;
            if (lane == 0 && m) base = atomicAdd(&bc[0], (uint32_t)__popcll(m));
            base = __shfl(base, 0);
            const uint32_t slot = base + (uint32_t)__popcll(m & ((lane == 0) ? 0ull : (~0ull >> (64 - lane))));
            if (keep && slot < (uint32_t)CAP) fl.cand[slot] = pack(kk[h][c], (uint32_t)(e0[h] + c));
          }
        }
      }
      __syncthreads();
      ncand = (int64_t)bc[0];
      if (ncand > CAP || ncand < 1) dense = true;
    }
    if (!dense) {
      if (ncand <= NT) sort_desc_small(fl.cand, (uint64_t*)fl.w, (int)ncand);
      else sort_desc(fl.cand, (int)ncand);
      cand = fl.cand;
      wbuf = fl.w;
    } else {
      const uint32_t trel = relevance_key(M, P.temperature);
      ncand = dense_build<DT, PEN>(A, rc, row, trel, plan.need_rel, plan.KB, (uint32_t*)fl.cand,
                                   red_int);
      __syncthreads();
      cand = A.dense_a + (int64_t)row * A.dense_ld;
      wbuf = A.dense_w + (int64_t)row * A.dense_ld;
    }

    // ---- outputs in raw order ------------------------------------------
    if (A.argmax && tid == 0) A.argmax[row] = pk_id(rmax);
    if (A.top8_ids) {
      for (int i = tid; i < 8; i += NT) {
        const bool in = i < ncand;
        const uint32_t id = in ? pk_id(cand[i]) : 0xffffffffu;
        A.top8_ids[(int64_t)row * 8 + i] = id;
        A.top8_vals[(int64_t)row * 8 + i] = in ? __uint_as_float(value_bits<DT, PEN>(rc, id)) : -__builtin_inff();
      }
    }
    if (A.top20_ids) {
      for (int i = tid; i < 20; i += NT) {
        const bool in = i < ncand;
        const uint32_t id = in ? pk_id(cand[i]) : 0xffffffffu;
        A.top20_ids[(int64_t)row * 20 + i] = id;
        A.top20_vals[(int64_t)row * 20 + i] = in ? __uint_as_float(value_bits<DT, PEN>(rc, id)) : -__builtin_inff();
      }
    }
    if (A.topn_ids) {
      for (int i = tid; i < A.topn; i += NT) {
        const bool in = i < ncand;
        const uint32_t id = in ? pk_id(cand[i]) : 0xffffffffu;
        A.topn_ids[(int64_t)row * A.topn + i] = id;
        if (A.topn_vals)
          A.topn_vals[(int64_t)row * A.topn + i] = in ? __uint_as_float(value_bits<DT, PEN>(rc, id)) : -__builtin_inff();
      }
    }
    if (A.n_lp > 0) {
      for (int i = tid; i < A.n_lp; i += NT) {
        const bool in = i < ncand;
        const uint32_t id = in ? pk_id(cand[i]) : 0xffffffffu;
        double lp = -__builtin_inf();
        if (in) {
          const float l = __uint_as_float(value_bits<DT, PEN>(rc, id));
          lp = ((double)l - (double)M) - logZ;
        }
        A.lp_ids[(int64_t)row * A.n_lp + i] = id;
        A.lp_vals[(int64_t)row * A.n_lp + i] = lp;
      }
    }
    if (A.nll_targets && tid == 0) {
      const uint32_t t = A.nll_targets[row];
      if (t < (uint32_t)V) {
        const float l = __uint_as_float(value_bits<DT, PEN>(rc, t));
        A.nll_out[row] = ((double)M - (double)l) + logZ;
      } else {
        status = ST_EINVAL;
        A.nll_out[row] = __builtin_nan("");
      }
    }
    // ---- token selection ---------------------------------------------------
    if (A.out_ids) {
      if (P.greedy) {
        const int nd = A.mode == MODE_VERIFY ? 1 : A.n_draws;
        for (int d = tid; d < nd; d += NT) A.out_ids[(int64_t)row * A.n_draws + d] = pk_id(rmax);
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
      atomicAdd(&A.stats[STAT_RESCAN_WAVES], (unsigned long long)nres);
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
  // clear the row's bound slots for the next call (ordered by the kernel boundary)
  for (int sg = tid; sg < A.S; sg += NT) A.slots[(int64_t)row * MAX_SEGMENTS + sg] = 0ull;

  // ---- verify: the last finished row applies the acceptance rule --------
  if (A.mode == MODE_VERIFY) {
    __syncthreads();
    if (tid == 0) {
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
      const uint32_t old = __hip_atomic_fetch_add(A.vcount, 1u, __ATOMIC_RELAXED,
                                                  __HIP_MEMORY_SCOPE_AGENT);
      if (old == (uint32_t)(A.rows - 1)) {
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
        uint32_t emitted = 0, accepted = 0, token = 0xffffffffu;
        int32_t stop_eos = 0;
        bool ok = true;
        for (int j = 0; j < A.rows; ++j) ok = ok && (A.status[j] == ST_OK);
        if (ok) {
          for (int j = 0; j < A.rows; ++j) {
            const uint32_t sel = A.out_ids[j];
            ++emitted;
            token = sel;
            const bool matched = (j + 1 < A.rows) && A.drafts[j] == sel;
            accepted += matched ? 1u : 0u;
            for (int e = 0; e < A.n_eos; ++e)
              if (A.eos[e] == sel) stop_eos = 1;
            if (stop_eos || !matched) break;
          }
        }
        A.vresult[0] = accepted;
        A.vresult[1] = emitted;
        A.vresult[2] = token;
        A.vresult[3] = (uint32_t)stop_eos;
        __hip_atomic_store(A.vcount, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
  }
}
// ---------------------------------------------------------------------------
// Penalty preparation: per row, sorted unique history ids with counts and a
// membership bitmap over the vocabulary.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(1024) void smp_penalty_prep(PenArgs A) {
  __shared__ uint32_t h[HCAP];
  __shared__ int red[16];
  __shared__ int s_bad;
  const int tid = threadIdx.x, row = blockIdx.x;
  const DevParams P = A.prm[A.prm_shared ? 0 : row];
  if (!P.penalize) {
    if (tid == 0) A.len[row] = 0;
    return;
  }
  int len = A.history_len ? A.history_len[row] : 0;
  uint32_t* bm = A.bitmap + (int64_t)row * A.bm_ld;
  const int words = (A.V + 31) >> 5;
  for (int i = tid; i < words; i += 1024) bm[i] = 0u;
  if (tid == 0) s_bad = (len < 0 || len > HCAP) ? 1 : 0;
  __syncthreads();
  if (s_bad) {
    if (tid == 0) A.len[row] = -1;
    return;
  }
  int n2 = 1;
  while (n2 < len) n2 <<= 1;
  for (int i = tid; i < n2; i += 1024) {
    uint32_t v = 0xffffffffu;
    if (i < len) {
      v = A.history[(int64_t)row * A.history_ld + i];
      if (v >= (uint32_t)A.V) atomicOr(&s_bad, 1);
    }
    h[i] = v;
  }
  __syncthreads();
  if (s_bad) {
    if (tid == 0) A.len[row] = -1;
    return;
  }
  // bitonic sort ascending
  for (int k = 2; k <= n2; k <<= 1) {
    for (int j = k >> 1; j > 0; j >>= 1) {
      for (int i = tid; i < n2; i += 1024) {
        const int ixj = i ^ j;
        if (ixj > i) {
          const uint32_t a = h[i], b = h[ixj];
          const bool asc = (i & k) == 0;
          if (asc ? (a > b) : (a < b)) {
            h[i] = b;
            h[ixj] = a;
          }
        }
      }
      __syncthreads();
    }
  }
  // run starts: count per thread over a contiguous chunk, then scan
  const int chunk = (len + 1023) / 1024;
  const int lo = tid * chunk, hi = min(len, lo + chunk);
  int starts = 0;
  for (int i = lo; i < hi; ++i) starts += (i == 0 || h[i] != h[i - 1]) ? 1 : 0;
  // block exclusive scan (1024 threads = 16 waves)
  const int lane = tid & 63, wave = tid >> 6;
  int inc = starts;
  for (int o = 1; o < 64; o <<= 1) {
    const int y = __shfl_up(inc, o);
    if (lane >= o) inc += y;
  }
  if (lane == 63) red[wave] = inc;
  __syncthreads();
  int base = 0, tot = 0;
  for (int w = 0; w < 16; ++w) {
    base += (w < wave) ? red[w] : 0;
    tot += red[w];
  }
  int u = base + inc - starts;
  uint32_t* ids = A.ids + (int64_t)row * HCAP;
  uint32_t* cnt = A.cnt + (int64_t)row * HCAP;
  for (int i = lo; i < hi; ++i) {
    if (i == 0 || h[i] != h[i - 1]) {
      int e = i + 1;
      while (e < len && h[e] == h[i]) ++e;
      ids[u] = h[i];
      cnt[u] = (uint32_t)(e - i);
      atomicOr(&bm[h[i] >> 5], 1u << (h[i] & 31));
      ++u;
    }
  }
  if (tid == 0) A.len[row] = tot;
}

// ---------------------------------------------------------------------------
template <int DT, bool VEC, bool PEN>
static hipError_t launch_t(const SmpArgs& a, hipStream_t st) {
  hipLaunchKernelGGL((smp_scan<DT, VEC, PEN>), dim3((unsigned)(a.S * a.rows)), dim3(NTS), 0, st, a);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL((smp_finish<DT, PEN>), dim3((unsigned)a.rows), dim3(NT), 0, st, a);
  return hipGetLastError();
}

hipError_t launch_sample(const SmpArgs& a, int dtype, bool vec, bool pen, hipStream_t st) {
  if (dtype == 0) {
    if (vec) return pen ? launch_t<0, true, true>(a, st) : launch_t<0, true, false>(a, st);
    return pen ? launch_t<0, false, true>(a, st) : launch_t<0, false, false>(a, st);
  }
  if (vec) return pen ? launch_t<1, true, true>(a, st) : launch_t<1, true, false>(a, st);
  return pen ? launch_t<1, false, true>(a, st) : launch_t<1, false, false>(a, st);
}

hipError_t launch_penalty_prep(const PenArgs& a, hipStream_t st) {
  hipLaunchKernelGGL(smp_penalty_prep, dim3(a.rows), dim3(1024), 0, st, a);
  return hipGetLastError();
}

}  // namespace yskn
