// smp_kernels.hip -- gfx950 kernels of the per-step sampling path.
//
// One launch per call. S * rows blocks: block (seg, row) owns 16,384 logits of
// the row in registers (32 per thread, coalesced 16-byte loads). The path:
//
//  1. scan: order-preserving 32-bit keys, segment max, non-finite check.
//  2. row bounds: each block publishes its max key and a top-KB threshold
//     with agent-scope atomic max operations, whose return values give it
//     the row's running maxima at once. A block that would keep too many
//     elements under those bounds waits, with a bounded spin that always
//     ends, until every block of its row has published.
//  3. filter: a block keeps only elements that can matter to the reference
//     algorithm: (a) elements whose binary64 weight exp_d((l - M)/T) can
//     reach 2^-53 -- smaller weights are absorbed by the reference's serial
//     binary64 sums, whose running value is >= 1 -- and (b) a superset of the
//     row's top-KB by value. Survivors are written compactly for the row.
//  4. finish: the last block of the row gathers the survivors, sorts them in
//     LDS by (value desc, id asc) and runs the reference's serial binary64
//     truncation and draw on them (output_head_sampler.rs:136-212).
//     Rows with more survivors than LDS holds take the exact "dense" path:
//     radix select, stable LSD radix sort in global scratch, same tail.
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
// LDS layout of the finisher (32 KB), reused by the dense path.
// ---------------------------------------------------------------------------
struct FinishLds {
  uint64_t cand[CAP];  // sorted candidates (LDS path)
  double w[CAP];       // weights of the first c candidates (LDS path)
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
// The fused kernel.
// ---------------------------------------------------------------------------
template <int DT, bool VEC, bool PEN>
__global__ __launch_bounds__(NT) void smp_main(SmpArgs A) {
  __shared__ FinishLds fl;
  __shared__ uint64_t red_u64[NW];
  __shared__ double red_f64[NW];
  __shared__ int red_int[NW];
  __shared__ uint32_t red_u32[NW];
  __shared__ uint32_t bc[8];
  __shared__ TailShared ts;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int S = A.S;
  // Workgroups are dealt round-robin to the 8 XCDs (linear id mod 8). Groups
  // of 8 rows are laid out so that all S segments of a row share one XCD:
  // its segments are dispatched together by one dispatcher and the row's
  // hand-off traffic stays within one L2.
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
  const int32_t V = A.V;
  const DevParams P = A.prm[A.prm_shared ? 0 : row];
  const RowPlan plan = make_plan(A, P);

  RowCtx rc;
  rc.base = (const char*)A.logits + (int64_t)row * A.ld * (DT == 0 ? 4 : 2);
  rc.bitmap = nullptr;
  rc.pids = nullptr;
  rc.pcnt = nullptr;
  rc.plen = 0;
  rc.rep = P.rep;
  rc.pres = P.pres;
  rc.freq = P.freq;
  uint32_t seg_flags = 0;
  if (PEN && P.penalize) {
    rc.plen = A.pen_len[row];
    if (rc.plen < 0) {
      seg_flags |= F_INVALID;
      rc.plen = 0;
    } else {
      rc.bitmap = A.pen_bitmap + (int64_t)row * A.bm_ld;
      rc.pids = A.pen_ids + (int64_t)row * HCAP;
      rc.pcnt = A.pen_cnt + (int64_t)row * HCAP;
    }
  }

  // ---- 1. load the segment into registers as keys -----------------------
  const int64_t seg0 = (int64_t)seg * SEG;
  uint32_t key[EPT];
  constexpr int GRP = (DT == 0) ? 4 : 8;  // elements per 16-byte load
  constexpr int NGRP = EPT / GRP;
#pragma unroll
  for (int q = 0; q < NGRP; ++q) {
    const int64_t e0 = seg0 + (int64_t)(q * NT + tid) * GRP;
    if (VEC && e0 + GRP <= V) {
      const uint4 v = *(const uint4*)(rc.base + e0 * (DT == 0 ? 4 : 2));
      if (DT == 0) {
        key[q * 4 + 0] = v.x;
        key[q * 4 + 1] = v.y;
        key[q * 4 + 2] = v.z;
        key[q * 4 + 3] = v.w;
      } else {
        const uint32_t wv[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          key[q * 8 + 2 * c] = wv[c] << 16;
          key[q * 8 + 2 * c + 1] = wv[c] & 0xffff0000u;
        }
      }
    } else {
#pragma unroll
      for (int c = 0; c < GRP; ++c) key[q * GRP + c] = (e0 + c < V) ? raw_bits<DT>(rc, e0 + c) : 0u;
    }
  }
  bool bad = false;
  uint64_t tmax = 0;
#pragma unroll
  for (int q = 0; q < NGRP; ++q) {
    const int64_t e0 = seg0 + (int64_t)(q * NT + tid) * GRP;
    uint32_t wbits = 0;
    if (PEN && rc.bitmap && e0 < V) wbits = rc.bitmap[e0 >> 5];
#pragma unroll
    for (int c = 0; c < GRP; ++c) {
      const int64_t e = e0 + c;
      uint32_t b = key[q * GRP + c];
      if (e < V) {
        if (PEN && rc.bitmap && ((wbits >> (e & 31)) & 1u)) b = penalize(b, pen_count(rc, (uint32_t)e), rc);
        bad |= nonfinite_bits(b);
        const uint32_t k = f2key(b);
        key[q * GRP + c] = k;
        const uint64_t p = pack(k, (uint32_t)e);
        tmax = p > tmax ? p : tmax;
      } else {
        key[q * GRP + c] = 0u;
      }
    }
  }
  if (__syncthreads_or(bad)) seg_flags |= F_NONFINITE;
  const uint64_t bmax = block_max_u64(tmax, red_u64);
  const uint32_t key_b = pk_key(bmax);

  // ---- top-KB threshold: per wave the ceil(KB/8)-th largest thread max;
  // at least KB elements of the segment lie at or above the minimum over waves.
  {
    const int qp = (plan.KB + NW - 1) / NW;
    uint64_t mine = tmax, last = 0;
    for (int i = 0; i < qp; ++i) {
      const uint64_t m = wave_max_u64(mine);
      last = m;
      if (mine == m) mine = 0;
    }
    __syncthreads();
    if (lane == 0) red_u32[wave] = pk_key(last);
    __syncthreads();
  }
  uint32_t th1 = red_u32[0];
#pragma unroll
  for (int w = 1; w < NW; ++w) th1 = th1 < red_u32[w] ? th1 : red_u32[w];

  // ---- 2. row bounds -------------------------------------------------------
  // Each block publishes its max key and its top-KB threshold; fetch_max
  // returns the row's running maxima, so a block obtains bounds without
  // waiting. Only monotone bounds travel this way: any value read is a valid
  // (if weaker) bound, so relaxed atomics suffice and no cache-wide fence is
  // issued while blocks stream their segments.
  if (tid == 0) {
    RowSync* rs = A.sync + row;
    const uint32_t om = __hip_atomic_fetch_max(&rs->hint_max, key_b, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const uint32_t ok = __hip_atomic_fetch_max(&rs->hint_kb, th1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_fetch_add(&rs->arrive, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    bc[0] = om > key_b ? om : key_b;
    bc[1] = ok > th1 ? ok : th1;
    bc[2] = 0u;
  }
  __syncthreads();
  uint32_t mkey = bc[0];
  uint32_t th_kb = bc[1];
  float m_ref = key2f(mkey);

  // ---- 3. filter --------------------------------------------------------
  auto threshold = [&](float mr, uint32_t kb) {
    uint32_t t = kb;
    if (plan.need_rel) {
      const uint32_t tr = relevance_key(mr, P.temperature);
      t = tr < t ? tr : t;
    }
    if (A.force_dense) t = 0xffffffffu;  // compact path unused
    return t < 1u ? 1u : t;
  };
  uint32_t theta = threshold(m_ref, th_kb);
  int cnt = 0;
#pragma unroll
  for (int i = 0; i < EPT; ++i) cnt += (key[i] >= theta) ? 1 : 0;
  int total = block_sum_int(cnt, red_int);
  if (total > CAPSEG / 2 && A.spin_limit > 0) {
    // Too many survivors under the bounds seen so far: wait (bounded) until
    // every block of the row has published, then filter again.
    if (tid == 0) {
      RowSync* rs = A.sync + row;
      uint32_t n = 0;
      int it = 0;
      for (; it < A.spin_limit; ++it) {
        n = __hip_atomic_load(&rs->arrive, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (n >= (uint32_t)S) break;
        __builtin_amdgcn_s_sleep(2);
      }
      if (A.stats) atomicAdd(&A.stats[STAT_SPINS], (unsigned long long)it + 1ull);
      const uint32_t hm = __hip_atomic_load(&rs->hint_max, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      const uint32_t hk = __hip_atomic_load(&rs->hint_kb, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      bc[3] = hm > mkey ? hm : mkey;
      bc[4] = hk > th_kb ? hk : th_kb;
      bc[2] = n >= (uint32_t)S ? 0u : F_TIMEOUT;
    }
    __syncthreads();
    mkey = bc[3];
    th_kb = bc[4];
    m_ref = key2f(mkey);
    theta = threshold(m_ref, th_kb);
    cnt = 0;
#pragma unroll
    for (int i = 0; i < EPT; ++i) cnt += (key[i] >= theta) ? 1 : 0;
  }
  seg_flags |= bc[2];

  // mass relative to m_ref: binary32 terms, pairwise within the thread
  double mass = 0.0;
  if (A.want_mass) {
    float acc[EPT];
#pragma unroll
    for (int i = 0; i < EPT; ++i) {
      const uint32_t k = key[i];
      const float x = k ? (key2f(k) - m_ref) : -__builtin_inff();
      acc[i] = __builtin_amdgcn_exp2f(x * 1.4426950408889634f);
    }
#pragma unroll
    for (int s = EPT / 2; s > 0; s >>= 1) {
#pragma unroll
      for (int i = 0; i < s; ++i) acc[i] = acc[i] + acc[i + s];
    }
    mass = block_sum_f64((double)acc[0], red_f64);
  }

  const int off = block_excl_scan(cnt, red_int, &total);
  const bool overflow = total > CAPSEG;
  if (!overflow && cnt) {
    uint64_t* dst = A.seg_cand + ((int64_t)row * S + seg) * CAPSEG + off;
    int o = 0;
#pragma unroll
    for (int q = 0; q < NGRP; ++q) {
#pragma unroll
      for (int c = 0; c < GRP; ++c) {
        const uint32_t k = key[q * GRP + c];
        if (k >= theta) {
          const int64_t e = seg0 + (int64_t)(q * NT + tid) * GRP + c;
          dst[o++] = pack(k, (uint32_t)e);
        }
      }
    }
  }
  if (tid == 0) {
    SegInfo si;
    si.maxp = bmax;
    si.mass = mass;
    si.mref = m_ref;
    si.count = overflow ? 0u : (uint32_t)total;
    si.flags = seg_flags | (overflow ? F_OVERFLOW : 0u);
    si.th1 = th1;
    A.seg_info[(int64_t)row * S + seg] = si;
  }

  // ---- last block of the row finishes ------------------------------------
  // release: this block's candidates and SegInfo reach device-coherent memory
  // before its arrival is counted; the finisher acquires once.
  __syncthreads();
  if (tid == 0) {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
    const uint32_t old = __hip_atomic_fetch_add(&A.sync[row].done, 1u, __ATOMIC_RELAXED,
                                                __HIP_MEMORY_SCOPE_AGENT);
    bc[5] = (old == (uint32_t)(S - 1)) ? 1u : 0u;
    if (bc[5]) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
  }
  __syncthreads();
  if (!bc[5]) return;
  if (tid == 0) {
    RowSync* rs = A.sync + row;
    __hip_atomic_store(&rs->arrive, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(&rs->done, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(&rs->hint_max, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(&rs->hint_kb, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }

  // ---- 4. finish ----------------------------------------------------------
  // One parallel pass over the segment records (their counts go to LDS,
  // borrowing the weight area, which is not in use yet).
  uint32_t* s_cnt = (uint32_t*)fl.w;         // [MAX_SEGMENTS]
  uint32_t* s_off = s_cnt + MAX_SEGMENTS;    // [MAX_SEGMENTS]
  uint64_t rmax = 0, rkb = 0;
  uint32_t rflags = 0;
  for (int s = tid; s < S; s += NT) {
    const SegInfo si = A.seg_info[(int64_t)row * S + s];
    rmax = si.maxp > rmax ? si.maxp : rmax;
    rkb = si.th1 > rkb ? si.th1 : rkb;
    rflags |= si.flags;
    s_cnt[s] = si.count;
  }
  rmax = block_max_u64(rmax, red_u64);
  rkb = block_max_u64(rkb, red_u64);
  {
    // OR of the segment flags across the block: every decision below
    // (status, dense or compact) must be uniform over the block's threads
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
  int csum;
  {
    // exclusive scan of the counts; thread t owns segments 2t and 2t+1
    const int s0 = 2 * tid, s1 = 2 * tid + 1;
    const int c0 = s0 < S ? (int)s_cnt[s0] : 0, c1 = s1 < S ? (int)s_cnt[s1] : 0;
    const int ex = block_excl_scan(c0 + c1, red_int, &csum);
    if (s0 < S) s_off[s0] = (uint32_t)ex;
    if (s1 < S) s_off[s1] = (uint32_t)(ex + c0);
  }
  const float M = key2f(pk_key(rmax));
  double logZ = 0.0, rmass = 0.0;
  if (A.want_mass) {
    double part = 0.0;
    for (int s = tid; s < S; s += NT) {
      const SegInfo si = A.seg_info[(int64_t)row * S + s];
      part += si.mass * exp((double)si.mref - (double)M);
    }
    rmass = block_sum_f64(part, red_f64);
    logZ = log(rmass);
  }
  int32_t status = ST_OK;
  if (rflags & F_INVALID) status = ST_EINVAL;
  else if (rflags & F_NONFINITE) status = ST_ENONFINITE;

  if (status == ST_OK) {
    // Final threshold from exact row quantities: every block filtered with
    // bounds no larger than these, so the survivors below are exactly the
    // row's elements with key >= theta_f, whatever the rendezvous timing.
    uint32_t theta_f = (uint32_t)rkb;
    if (plan.need_rel) {
      const uint32_t tr = relevance_key(M, P.temperature);
      theta_f = tr < theta_f ? tr : theta_f;
    }
    if (theta_f < 1u) theta_f = 1u;
    bool dense = A.force_dense || (rflags & F_OVERFLOW);
    const uint64_t* cand;
    double* wbuf;
    int64_t ncand = 0;
    if (!dense) {
      // gather the survivors of every segment in one flat parallel pass
      // (order is irrelevant: sorted next)
      if (tid == 0) bc[6] = 0u;
      __syncthreads();
      const int64_t cbase = (int64_t)row * S * CAPSEG;
      for (int i0 = 0; i0 < csum; i0 += NT) {
        const int idx = i0 + tid;
        bool keep = false;
        uint64_t p = 0;
        if (idx < csum) {
          int lo = 0, hi = S - 1;  // largest s with s_off[s] <= idx
          while (lo < hi) {
            const int mid = (lo + hi + 1) >> 1;
            if ((int)s_off[mid] <= idx) lo = mid; else hi = mid - 1;
          }
          p = A.seg_cand[cbase + (int64_t)lo * CAPSEG + (idx - (int)s_off[lo])];
          keep = pk_key(p) >= theta_f;
        }
        const uint64_t m = __ballot(keep);
        uint32_t base = 0;
        if (lane == 0 && m) base = atomicAdd(&bc[6], (uint32_t)__popcll(m));
        base = __shfl(base, 0);
        const uint32_t slot = base + (uint32_t)__popcll(m & ((lane == 0) ? 0ull : (~0ull >> (64 - lane))));
        if (keep && slot < (uint32_t)CAP) fl.cand[slot] = p;
      }
      __syncthreads();
      csum = (int)bc[6];
      if (csum > CAP || csum < 1) dense = true;
    }
    if (!dense) {
      int n2 = 1;
      while (n2 < csum) n2 <<= 1;
      for (int i = csum + tid; i < n2; i += NT) fl.cand[i] = 0ull;
      __syncthreads();
      // bitonic sort, descending
      for (int k = 2; k <= n2; k <<= 1) {
        for (int j = k >> 1; j > 0; j >>= 1) {
          for (int i = tid; i < n2; i += NT) {
            const int ixj = i ^ j;
            if (ixj > i) {
              const uint64_t a = fl.cand[i], b = fl.cand[ixj];
              const bool desc = (i & k) == 0;
              if (desc ? (a < b) : (a > b)) {
                fl.cand[i] = b;
                fl.cand[ixj] = a;
              }
            }
          }
          __syncthreads();
        }
      }
      cand = fl.cand;
      wbuf = fl.w;
      ncand = csum;
    } else {
      const uint32_t trel = relevance_key(M, P.temperature);
      ncand = dense_build<DT, PEN>(A, rc, row, trel, plan.need_rel, plan.KB, (uint32_t*)fl.cand,
                                   red_int);
      __syncthreads();
      cand = A.dense_a + (int64_t)row * A.dense_ld;
      wbuf = A.dense_w + (int64_t)row * A.dense_ld;
    }

    // outputs in raw order
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
    // token selection
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
      atomicAdd(&A.stats[STAT_CANDIDATES], (unsigned long long)csum);
      if (rflags & F_TIMEOUT) atomicAdd(&A.stats[STAT_WAIT_TIMEOUTS], 1ull);
    }
  } else if (A.out_ids) {
    const int nd = A.mode == MODE_VERIFY ? 1 : A.n_draws;
    for (int d = tid; d < nd; d += NT) A.out_ids[(int64_t)row * A.n_draws + d] = 0xffffffffu;
  }
  if (tid == 0) {
    A.status[row] = status;
    if (A.row_status) A.row_status[row] = status;
  }

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
            const uint32_t sel = __hip_atomic_load(A.out_ids + j, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
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
  hipLaunchKernelGGL((smp_main<DT, VEC, PEN>), dim3((unsigned)(a.S * a.rows)), dim3(NT), 0, st, a);
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
