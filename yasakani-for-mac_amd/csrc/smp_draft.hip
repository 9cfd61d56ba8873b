// Draft-side selection: the drafter's shortlist of its approximate scores,
// the exact top 16 of the rescored shortlist, and the Gumbel-coupled choice
// among those 16 (crates/yskn-ref/src/draft_head.rs:219-379; the CUDA
// drafter's bdr_sk_hist2/collect/top16 and bdr_select(3) kernels,
// src/q35_bdraft.cu:318-475,801-898).
//
// The shortlist keeps the reference's two histogram passes (1,024 bins of the
// key's top 10 bits, then 2,048 bins of the next 11 bits inside the cut-off
// bin) and fills the tie bucket in ascending token order, as draft_head.rs
// does: the result, its order included, is a function of the scores alone
// (the CUDA collect step's atomic slot order made it vary between runs).
// One 1,024-thread block per row; the row is read three times (histogram,
// histogram inside one bin, ordered collection), each read coalesced.
#include "smp_internal.hpp"
#include "smp_math.hpp"

namespace yskn {
namespace {

constexpr int DNT = 1024;  // threads per shortlist / top-16 block
constexpr int DNW = DNT / 64;
constexpr int NB1 = 1024;  // first-pass bins: key >> 22
constexpr int NB2 = 2048;  // second-pass bins: (key >> 11) & 2047
constexpr int TILE_J = 8;  // collection tile: TILE_J * DNT elements

// Order-preserving key of a binary32 score, -0 below +0
// (draft_head.rs:219-226: no canonicalisation).
__device__ __forceinline__ uint32_t draft_key(uint32_t u) { return (u & 0x80000000u) ? ~u : (u | 0x80000000u); }

// The same with -0 taken as +0: the key of the total order the reference
// sorts by (partial_cmp: -0 == +0).
__device__ __forceinline__ uint32_t order_key(uint32_t u) {
  if (u == 0x80000000u) u = 0u;
  return draft_key(u);
}

__device__ __forceinline__ bool finite_u(uint32_t u) { return (u & 0x7f800000u) != 0x7f800000u; }

__device__ __forceinline__ uint32_t wave_incl_scan(uint32_t v) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const uint32_t t = (uint32_t)__shfl_up((int)v, o);
    if (lane >= o) v += t;
  }
  return v;
}

// Histogram increment of `bin` (bits wide) for the valid lanes of a wave:
// lanes with equal bins are found with one ballot per bit, and the lowest of
// them adds their number (one LDS atomic per distinct bin, not per lane).
__device__ __forceinline__ void hist_add(uint32_t* hist, uint32_t bin, bool valid, int bits) {
  const int lane = threadIdx.x & 63;
  uint64_t peers = __ballot(valid);
  for (int b = 0; b < bits; ++b) {
    const bool bit = (bin >> b) & 1u;
    const uint64_t bal = __ballot(bit);
    peers &= bit ? bal : ~bal;
  }
  if (valid && (peers & ((1ull << lane) - 1ull)) == 0ull) atomicAdd(&hist[bin], (uint32_t)__popcll(peers));
}

// Block-wide exclusive scan over DNT threads; red holds 2 * DNW + 1 words.
__device__ uint32_t block_excl_scan(uint32_t v, uint32_t* red, uint32_t* total) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const uint32_t inc = wave_incl_scan(v);
  if (lane == 63) red[wave] = inc;
  __syncthreads();
  if (wave == 0) {
    const uint32_t w = lane < DNW ? red[lane] : 0u;
    const uint32_t wi = wave_incl_scan(w);
    if (lane < DNW) red[DNW + 1 + lane] = wi - w;
    if (lane == DNW - 1) red[DNW] = wi;
  }
  __syncthreads();
  const uint32_t r = red[DNW + 1 + wave] + inc - v;
  *total = red[DNW];
  __syncthreads();
  return r;
}

// The highest bin b with (sum of bins above b) + hist[b] >= need, and that
// sum above (draft_head.rs:227-236): with suffix sums S(b) over bins >= b,
// the unique b with S(b) >= need > S(b + 1). Bins are taken NB / DNT per
// thread from the top down. Result in bc[0] (bin), bc[1] (above).
template <int NB>
__device__ void cutoff_bin(const uint32_t* hist, uint32_t need, uint32_t* red, uint32_t* bc) {
  constexpr int PER = NB / DNT;
  const int t = threadIdx.x;
  uint32_t h[PER], loc = 0u;
#pragma unroll
  for (int q = 0; q < PER; ++q) {
    h[q] = hist[NB - 1 - (t * PER + q)];
    loc += h[q];
  }
  uint32_t tot;
  uint32_t s = block_excl_scan(loc, red, &tot);  // sum of the bins above this thread's first
#pragma unroll
  for (int q = 0; q < PER; ++q) {
    const uint32_t above = s;
    s += h[q];
    if (s >= need && above < need) {
      bc[0] = (uint32_t)(NB - 1 - (t * PER + q));
      bc[1] = above;
    }
  }
  __syncthreads();
}

__global__ __launch_bounds__(DNT) void draft_shortlist_kernel(DraftShortlistArgs A) {
  __shared__ uint32_t h1[NB1];
  __shared__ uint32_t h2[NB2];
  __shared__ uint32_t red[2 * DNW + 1];
  __shared__ uint32_t bc[4];
  __shared__ uint32_t offs[TILE_J * DNW];  // per (j, wave) offsets: above | tie << 16
  __shared__ uint32_t ctot[2];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int row = blockIdx.x;
  const int V = A.V;
  const uint32_t count = (uint32_t)A.count;
  const uint32_t* x = (const uint32_t*)(A.scores + (int64_t)row * A.ld);
  uint32_t* out = A.out + (int64_t)row * A.out_ld;
  for (int i = tid; i < NB1; i += DNT) h1[i] = 0u;
  for (int i = tid; i < NB2; i += DNT) h2[i] = 0u;
  __syncthreads();
  // pass 1: finite check and the 1,024-bin histogram
  bool bad = false;
  for (int i0 = 0; i0 < V; i0 += 4 * DNT) {
    uint32_t u[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int i = i0 + q * DNT + tid;
      u[q] = i < V ? x[i] : 0u;
    }
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const bool v = i0 + q * DNT + tid < V;
      bad = bad || (v && !finite_u(u[q]));
      hist_add(h1, draft_key(u[q]) >> 22, v, 10);
    }
  }
  if (__syncthreads_or(bad)) {
    for (uint32_t i = (uint32_t)tid; i < count; i += DNT) out[i] = 0xffffffffu;
    if (tid == 0) {
      A.status[row] = ST_ENONFINITE;
      if (A.row_status) A.row_status[row] = ST_ENONFINITE;
    }
    return;
  }
  cutoff_bin<NB1>(h1, count, red, bc);
  const uint32_t first = bc[0], above1 = bc[1];
  // pass 2: the 2,048-bin histogram inside the first cut-off bin
  for (int i0 = 0; i0 < V; i0 += 4 * DNT) {
    uint32_t u[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int i = i0 + q * DNT + tid;
      u[q] = i < V ? x[i] : 0u;
    }
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const uint32_t k = draft_key(u[q]);
      hist_add(h2, (k >> 11) & 2047u, i0 + q * DNT + tid < V && (k >> 22) == first, 11);
    }
  }
  __syncthreads();
  cutoff_bin<NB2>(h2, count - above1, red, bc + 2);
  const uint32_t prefix = (first << 11) | bc[2];
  const uint32_t above = above1 + bc[3];  // ids with key >> 11 above the prefix: all kept
  const uint32_t ties = count - above;    // the lowest ids of the tie bucket
  // pass 3: ordered collection, tiles of TILE_J * DNT elements; element
  // (j, t) of a tile is tile + j * DNT + t (coalesced), ranked (j, wave,
  // lane): above ids go to out[rank], tie ids to out[above + rank] while
  // that is below count
  uint32_t na = 0u, nt = 0u;
  for (int base = 0; base < V; base += TILE_J * DNT) {
    uint32_t fa = 0u, ft = 0u;  // bit j: element j is above / in the tie bucket
#pragma unroll
    for (int j = 0; j < TILE_J; ++j) {
      const int i = base + j * DNT + tid;
      const uint32_t k = i < V ? (draft_key(x[i]) >> 11) : 0u;
      const bool a = i < V && k > prefix, t = i < V && k == prefix;
      fa |= (uint32_t)a << j;
      ft |= (uint32_t)t << j;
      const uint64_t ma = __ballot(a), mt = __ballot(t);
      if (lane == 0) offs[j * DNW + wave] = (uint32_t)__popcll(ma) | ((uint32_t)__popcll(mt) << 16);
    }
    __syncthreads();
    // wave 0: exclusive scan over the TILE_J * DNW (j, wave) counts in order
    if (wave == 0) {
      const uint32_t c0 = offs[2 * lane], c1 = offs[2 * lane + 1];  // TILE_J * DNW == 128
      const uint32_t loc = c0 + c1;
      const uint32_t inc = wave_incl_scan(loc);
      offs[2 * lane] = inc - loc;
      offs[2 * lane + 1] = inc - loc + c0;
      if (lane == 63) {
        ctot[0] = inc & 0xffffu;
        ctot[1] = inc >> 16;
      }
    }
    __syncthreads();
    const uint64_t below = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
#pragma unroll
    for (int j = 0; j < TILE_J; ++j) {
      const bool a = (fa >> j) & 1u, t = (ft >> j) & 1u;
      const uint64_t ma = __ballot(a), mt = __ballot(t);
      const uint32_t o = offs[j * DNW + wave];
      const uint32_t i = (uint32_t)(base + j * DNT + tid);
      if (a) out[na + (o & 0xffffu) + (uint32_t)__popcll(ma & below)] = i;
      if (t) {
        const uint32_t r = nt + (o >> 16) + (uint32_t)__popcll(mt & below);
        if (r < ties) out[above + r] = i;
      }
    }
    na += ctot[0];
    nt += ctot[1];
    __syncthreads();  // offs and ctot are written again by the next tile
    if (na >= above && nt >= ties) break;  // (block-uniform)
  }
  if (tid == 0) {
    A.status[row] = ST_OK;
    if (A.row_status) A.row_status[row] = ST_OK;
  }
}

// Ascending bitonic sort of n2 (a power of two, <= 4096) 64-bit keys with a
// 32-bit payload in LDS, by the whole block.
__device__ void bitonic_sort(uint64_t* key, uint32_t* pay, int n2) {
  for (int k = 2; k <= n2; k <<= 1) {
    for (int j = k >> 1; j > 0; j >>= 1) {
      for (int p = threadIdx.x; p < (n2 >> 1); p += DNT) {
        const int i = 2 * j * (p / j) + (p % j), l = i + j;
        const bool up = (i & k) == 0;
        const uint64_t a = key[i], b = key[l];
        if ((a > b) == up) {
          key[i] = b;
          key[l] = a;
          if (pay) {
            const uint32_t t = pay[i];
            pay[i] = pay[l];
            pay[l] = t;
          }
        }
      }
      __syncthreads();
    }
  }
}

__global__ __launch_bounds__(DNT) void draft_top16_kernel(DraftTop16Args A) {
  __shared__ uint64_t sk[TOP16_NMAX];
  __shared__ uint32_t si[TOP16_NMAX];
  __shared__ uint64_t tk[TOP16_NMAX];
  const int tid = threadIdx.x, row = blockIdx.x;
  const int n = A.n;
  int n2 = 16;
  while (n2 < n) n2 <<= 1;
  const uint32_t* sc = (const uint32_t*)(A.scores + (int64_t)row * A.ld);
  const uint32_t* tok = A.tokens + (int64_t)row * A.ld;
  bool bad = false;
  for (int i = tid; i < n2; i += DNT) {
    if (i < n) {
      const uint32_t u = sc[i], t = tok[i];
      bad = bad || !finite_u(u);
      // ascending (~key, token): score descending, then token ascending
      sk[i] = ((uint64_t)(~order_key(u)) << 32) | t;
      si[i] = (uint32_t)i;
      tk[i] = ((uint64_t)t << 32) | (uint32_t)i;
    } else {
      sk[i] = ~0ull;
      si[i] = 0xffffffffu;
      tk[i] = ~0ull;
    }
  }
  bool fail = __syncthreads_or(bad);
  if (!fail) {
    // distinct tokens are required (draft_head.rs:295-303): sorted by token,
    // equal tokens are neighbours (padding, all ones, sorts after every
    // real entry, whose low word is an index < n)
    bitonic_sort(tk, nullptr, n2);
    bool dup = false;
    for (int i = tid; i + 1 < n; i += DNT) dup = dup || (tk[i] >> 32) == (tk[i + 1] >> 32);
    fail = __syncthreads_or(dup);
  }
  if (!fail) bitonic_sort(sk, si, n2);
  if (tid < 16) {
    const int64_t o = (int64_t)row * 16 + tid;
    if (fail) {
      A.out_tokens[o] = 0xffffffffu;
      if (A.out_scores) A.out_scores[o] = -__builtin_inff();
    } else {
      const uint32_t j = si[tid];
      A.out_tokens[o] = tok[j];
      if (A.out_scores) A.out_scores[o] = __uint_as_float(sc[j]);
    }
  }
  if (tid == 0) {
    const int32_t st = fail ? ST_EINVAL : ST_OK;
    A.status[row] = st;
    if (A.row_status) A.row_status[row] = st;
  }
}

__device__ __forceinline__ double lane_f64(double x, int j) {
  const uint64_t b = (uint64_t)__double_as_longlong(x);
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)b, j);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(b >> 32), j);
  return __longlong_as_double((long long)(((uint64_t)hi << 32) | lo));
}

__device__ __forceinline__ float lane_f32(float x, int j) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), j));
}

// One wave per row; candidate i in lane i (draft_head.rs:325-379). The
// loops over candidates run lane-uniform on values read from the lanes.
__global__ __launch_bounds__(256) void draft_choose_kernel(DraftChooseArgs A) {
  const int lane = threadIdx.x & 63;
  const int row = (int)blockIdx.x * 4 + (int)(threadIdx.x >> 6);
  if (row >= A.rows) return;  // (wave-uniform)
  const bool in = lane < 16;
  const float s = in ? A.scores[(int64_t)row * A.ld + lane] : 0.0f;
  const uint32_t tok = in ? A.tokens[(int64_t)row * A.ld + lane] : 0u;
  const int64_t o = row;
  if (__ballot(in && !finite_u(__float_as_uint(s)))) {
    if (lane == 0) {
      A.out[o] = 0xffffffffu;
      if (A.alt) A.alt[o] = -1;
      if (A.alt3) A.alt3[o] = -1;
      if (A.margin) A.margin[o] = 1e30f;
      A.status[row] = ST_EINVAL;
      if (A.row_status) A.row_status[row] = ST_EINVAL;
    }
    return;
  }
  // the greedy choice: the first strictly larger score in input order
  int best = 0;
  float bs = lane_f32(s, 0);
  for (int k = 1; k < 16; ++k) {
    const float sk = lane_f32(s, k);
    if (sk > bs) {
      bs = sk;
      best = k;
    }
  }
  int b2 = -1, b3 = -1;
  double sel = 0.0, v2 = -__builtin_inf(), v3 = -__builtin_inf();
  float v2f = -__builtin_inff();
  double sval = -__builtin_inf();
  if (A.sampled) {
    // rank under (score desc, token asc); ord[r] = the lane of rank r
    int rk = 0;
    for (int k = 0; k < 16; ++k) {
      const float sk = lane_f32(s, k);
      const uint32_t tkk = (uint32_t)__builtin_amdgcn_readlane((int)tok, k);
      // (a stable sort: equal scores and tokens keep the input order)
      rk += (sk > s || (sk == s && (tkk < tok || (tkk == tok && k < lane)))) ? 1 : 0;
    }
    int ord[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) ord[r] = (int)__builtin_ctzll(__ballot(in && rk == r));
    // widen, subtract the top score, divide by the binary64 temperature
    const float stop = lane_f32(s, ord[0]);
    const double z = ((double)s - (double)stop) / A.temperature;
    const double w = in ? exp_d_inline(z) : 0.0;
    double total = 0.0;
#pragma unroll
    for (int r = 0; r < 16; ++r) total = total + lane_f64(w, ord[r]);
    // membership is decided before the candidate's own weight is added
    uint32_t member = 0u;
    double prefix = 0.0;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const double lim = 0.95 * total;
      if (prefix < lim) member |= 1u << ord[r];
      prefix = prefix + lane_f64(w, ord[r]);
    }
    if (in && ((member >> lane) & 1u)) sval = z + gumbel_from_key<true>(position_key(A.seed, A.positions[row]), tok);
    // the largest member score, the earliest in order winning ties; then
    // the runners-up the same way (q35_bdraft.cu:437-446)
    double bv = -__builtin_inf();
    for (int r = 0; r < 16; ++r) {
      const double v = lane_f64(sval, ord[r]);
      if (v > bv) {
        bv = v;
        best = ord[r];
      }
    }
    sel = bv;
    for (int r = 0; r < 16; ++r) {
      const double v = lane_f64(sval, ord[r]);
      if (ord[r] != best && v > v2) {
        v2 = v;
        b2 = ord[r];
      }
    }
    for (int r = 0; r < 16; ++r) {
      const double v = lane_f64(sval, ord[r]);
      if (ord[r] != best && ord[r] != b2 && v > v3) {
        v3 = v;
        b3 = ord[r];
      }
    }
  } else {
    // greedy runners-up in input order (q35_bdraft.cu:447-450)
    for (int k = 0; k < 16; ++k) {
      const float sk = lane_f32(s, k);
      if (k != best && sk > v2f) {
        v2f = sk;
        b2 = k;
      }
    }
    float v3f = -__builtin_inff();
    for (int k = 0; k < 16; ++k) {
      const float sk = lane_f32(s, k);
      if (k != best && k != b2 && sk > v3f) {
        v3f = sk;
        b3 = k;
      }
    }
  }
  const uint32_t tb = (uint32_t)__builtin_amdgcn_readlane((int)tok, best);
  const uint32_t t2 = b2 >= 0 ? (uint32_t)__builtin_amdgcn_readlane((int)tok, b2) : 0u;
  const uint32_t t3 = b3 >= 0 ? (uint32_t)__builtin_amdgcn_readlane((int)tok, b3) : 0u;
  if (lane == 0) {
    A.out[o] = tb;
    if (A.sampled) {
      const bool ok = b2 >= 0 && v2 > -__builtin_inf();
      if (A.alt) A.alt[o] = ok ? (int32_t)t2 : -1;
      if (A.margin) A.margin[o] = ok ? (float)(sel - v2) : 1e30f;
      if (A.alt3) A.alt3[o] = (ok && b3 >= 0 && v3 > -__builtin_inf()) ? (int32_t)t3 : -1;
    } else {
      if (A.alt) A.alt[o] = b2 >= 0 ? (int32_t)t2 : -1;
      if (A.margin) A.margin[o] = b2 >= 0 ? __fsub_rn(bs, v2f) : 1e30f;
      if (A.alt3) A.alt3[o] = (b2 >= 0 && b3 >= 0) ? (int32_t)t3 : -1;
    }
    A.status[row] = ST_OK;
    if (A.row_status) A.row_status[row] = ST_OK;
  }
}

}  // namespace

hipError_t launch_draft_shortlist(const DraftShortlistArgs& a, hipStream_t st) {
  hipLaunchKernelGGL(draft_shortlist_kernel, dim3(a.rows), dim3(DNT), 0, st, a);
  return hipGetLastError();
}

hipError_t launch_draft_top16(const DraftTop16Args& a, hipStream_t st) {
  hipLaunchKernelGGL(draft_top16_kernel, dim3(a.rows), dim3(DNT), 0, st, a);
  return hipGetLastError();
}

hipError_t launch_draft_choose(const DraftChooseArgs& a, hipStream_t st) {
  hipLaunchKernelGGL(draft_choose_kernel, dim3((a.rows + 3) / 4), dim3(256), 0, st, a);
  return hipGetLastError();
}

}  // namespace yskn
