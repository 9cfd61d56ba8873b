// smp_bench.hip -- native driver of yskn_smp_sample for profiler runs.
//
// Times the large-batch top-p workload (rows x V binary32 logits, top-k
// disabled, top-p 0.95, temperature 1.0, Gumbel draw, per-row seeds
// mix64(0x1A46E + row), positions 1..rows, top-20 logprobs) through the C ABI
// only: no Python, no torch, so that counter collection intercepts nothing but
// the HIP runtime and the sampler's own kernels. With --copy it runs a plain
// 16-byte-per-lane device copy of the same byte count instead, whose counters
// calibrate the sampler's.
//
//   smp_bench [--logits FILE] [--rows R] [--vocab V] [--steps K] [--warmup W]
//             [--top-k K] [--logprobs N] [--copy]
//
// --top-k sets every row's top-k (default 0, disabled); --logprobs the
// number of logprobs per row (default 20, 0 for none).
//
// FILE holds rows * V little-endian binary32 values (row-major). Without it
// the logits come from an on-device generator of 2 * t_3 variates (a
// counter-based SplitMix64 stream, Box-Muller normals), statistically the
// same workload. Prints one JSON line.
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <vector>

#include "../../include/yskn_smp.h"
#include "smp_math.hpp"

#define HIP_OK(x)                                                                       \
  do {                                                                                 \
    hipError_t e_ = (x);                                                               \
    if (e_ != hipSuccess) {                                                            \
      fprintf(stderr, "%s:%d %s: %s\n", __FILE__, __LINE__, #x, hipGetErrorString(e_)); \
      exit(1);                                                                         \
    }                                                                                  \
  } while (0)

namespace {

__global__ void copy16(const uint4* __restrict__ src, uint4* __restrict__ dst, size_t n) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (size_t)gridDim.x * blockDim.x)
    dst[i] = src[i];
}

__device__ __forceinline__ double unit(uint64_t key, uint64_t i) {
  // (0, 1): 53 random bits, offset by half an ulp so log() never sees 0
  return ((double)(yskn::mix64(key ^ (i * 0x9e3779b97f4a7c15ull)) >> 11) + 0.5) *
         (1.0 / 9007199254740992.0);
}

__device__ __forceinline__ double normal(uint64_t key, uint64_t i) {
  const double r = sqrt(-2.0 * log(unit(key, 2 * i)));
  return r * cos(6.283185307179586 * unit(key, 2 * i + 1));
}

// 2 * N0 / sqrt((N1^2 + N2^2 + N3^2) / 3) per element, keyed by (row, stream).
__global__ void gen_t3(float* out, int rows, int V) {
  const size_t n = (size_t)rows * V;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (size_t)gridDim.x * blockDim.x) {
    const uint64_t row = i / V, e = i % V;
    const uint64_t k = yskn::mix64(0x7A3Bull + row);
    const double n0 = normal(k ^ 1, e), n1 = normal(k ^ 2, e), n2 = normal(k ^ 3, e),
                 n3 = normal(k ^ 4, e);
    out[i] = (float)(2.0 * n0 / sqrt((n1 * n1 + n2 * n2 + n3 * n3) / 3.0));
  }
}

void check(int st, const char* what) {
  if (st != YSKN_SMP_OK) {
    fprintf(stderr, "%s failed (%d): %s\n", what, st, yskn_smp_last_error());
    exit(1);
  }
}

}  // namespace

int main(int argc, char** argv) {
  const char* path = nullptr;
  int rows = 256, V = 248320, steps = 20, warmup = 3, top_k = 0, n_lp = 20;
  bool copy = false;
  for (int i = 1; i < argc; ++i) {
    const bool more = i + 1 < argc;
    if (!strcmp(argv[i], "--logits") && more) path = argv[++i];
    else if (!strcmp(argv[i], "--rows") && more) rows = atoi(argv[++i]);
    else if (!strcmp(argv[i], "--vocab") && more) V = atoi(argv[++i]);
    else if (!strcmp(argv[i], "--steps") && more) steps = atoi(argv[++i]);
    else if (!strcmp(argv[i], "--warmup") && more) warmup = atoi(argv[++i]);
    else if (!strcmp(argv[i], "--top-k") && more) top_k = atoi(argv[++i]);
    else if (!strcmp(argv[i], "--logprobs") && more) n_lp = atoi(argv[++i]);
    else if (!strcmp(argv[i], "--copy")) copy = true;
    else {
      fprintf(stderr, "usage: %s [--logits FILE] [--rows R] [--vocab V] [--steps K] [--warmup W] [--top-k K] "
                      "[--logprobs N] [--copy]\n",
              argv[0]);
      return 2;
    }
  }
  if (rows < 1 || V < 1 || steps < 1 || warmup < 0 || top_k < 0 || n_lp < 0 || n_lp > 64) {
    fprintf(stderr, "rows, vocab and steps must be positive, top-k >= 0, logprobs in 0..64\n");
    return 2;
  }
  const size_t n = (size_t)rows * V, bytes = n * sizeof(float);
  hipStream_t st;
  HIP_OK(hipStreamCreate(&st));
  hipEvent_t e0, e1;
  HIP_OK(hipEventCreate(&e0));
  HIP_OK(hipEventCreate(&e1));

  if (copy) {
    const size_t n16 = bytes / 16;
    void *src, *dst;
    HIP_OK(hipMalloc(&src, n16 * 16));
    HIP_OK(hipMalloc(&dst, n16 * 16));
    HIP_OK(hipMemsetAsync(src, 0x3c, n16 * 16, st));
    const unsigned grid = 256 * 8 * 4;
    for (int i = 0; i < warmup; ++i)
      hipLaunchKernelGGL(copy16, dim3(grid), dim3(256), 0, st, (const uint4*)src, (uint4*)dst, n16);
    HIP_OK(hipEventRecord(e0, st));
    for (int i = 0; i < steps; ++i)
      hipLaunchKernelGGL(copy16, dim3(grid), dim3(256), 0, st, (const uint4*)src, (uint4*)dst, n16);
    HIP_OK(hipEventRecord(e1, st));
    HIP_OK(hipStreamSynchronize(st));
    float ms = 0;
    HIP_OK(hipEventElapsedTime(&ms, e0, e1));
    const double us = ms * 1e3 / steps;
    printf("{\"mode\": \"copy\", \"bytes_read\": %zu, \"bytes_written\": %zu, \"launches\": %d, "
           "\"us_per_launch\": %.3f, \"gbs\": %.1f}\n",
           n16 * 16, n16 * 16, warmup + steps, us, 2.0 * n16 * 16 / us / 1e3);
    HIP_OK(hipFree(src));
    HIP_OK(hipFree(dst));
    return 0;
  }

  // three input buffers rotate so that no step is served from the
  // Infinity Cache left warm by the previous one
  float* buf[3];
  for (auto& b : buf) HIP_OK(hipMalloc(&b, bytes));
  if (path) {
    std::vector<float> h(n);
    FILE* f = fopen(path, "rb");
    if (!f || fread(h.data(), sizeof(float), n, f) != n) {
      fprintf(stderr, "cannot read %zu binary32 values from %s\n", n, path);
      return 1;
    }
    fclose(f);
    HIP_OK(hipMemcpy(buf[0], h.data(), bytes, hipMemcpyHostToDevice));
  } else {
    hipLaunchKernelGGL(gen_t3, dim3(8192), dim3(256), 0, st, buf[0], rows, V);
    HIP_OK(hipGetLastError());
  }
  HIP_OK(hipMemcpyAsync(buf[1], buf[0], bytes, hipMemcpyDeviceToDevice, st));
  HIP_OK(hipMemcpyAsync(buf[2], buf[0], bytes, hipMemcpyDeviceToDevice, st));

  std::vector<yskn_smp_params> prm(rows);
  std::vector<uint64_t> pos(rows);
  for (int r = 0; r < rows; ++r) {
    prm[r] = yskn_smp_params{};
    prm[r].temperature_milli = 1000;
    prm[r].top_p_milli = 950;
    prm[r].top_k = (uint32_t)top_k;
    prm[r].min_p_milli = 0;
    prm[r].seed = yskn::mix64(0x1A46Eull + (uint64_t)r);
    prm[r].version = YSKN_SMP_VERSION_GUMBEL;
    prm[r].repetition_penalty = 1.0f;
    pos[r] = (uint64_t)r + 1;
  }
  yskn_smp_handle h = nullptr;
  check(yskn_smp_create(rows, V, YSKN_SMP_FLAG_EXTENDED_TOP_K, &h), "yskn_smp_create");
  check(yskn_smp_set_params(h, prm.data(), rows), "yskn_smp_set_params");
  uint64_t* d_pos;
  uint32_t *d_ids, *d_lpi;
  double* d_lp;
  int32_t* d_st;
  HIP_OK(hipMalloc(&d_pos, rows * sizeof(uint64_t)));
  HIP_OK(hipMalloc(&d_ids, rows * sizeof(uint32_t)));
  HIP_OK(hipMalloc(&d_lpi, rows * 64 * sizeof(uint32_t)));
  HIP_OK(hipMalloc(&d_lp, rows * 64 * sizeof(double)));
  HIP_OK(hipMalloc(&d_st, rows * sizeof(int32_t)));
  HIP_OK(hipMemcpy(d_pos, pos.data(), rows * sizeof(uint64_t), hipMemcpyHostToDevice));
  yskn_smp_aux aux{};
  aux.n_logprobs = n_lp;
  aux.logprob_ids = n_lp ? d_lpi : nullptr;
  aux.logprobs = n_lp ? d_lp : nullptr;
  aux.row_status = d_st;

  auto step = [&](int i) {
    check(yskn_smp_sample(h, buf[i % 3], YSKN_SMP_F32, rows, V, V, d_pos, 1, d_ids, &aux, st),
          "yskn_smp_sample");
  };
  for (int i = 0; i < warmup; ++i) step(i);
  HIP_OK(hipStreamSynchronize(st));
  std::vector<hipEvent_t> ev(2 * steps);
  for (auto& e : ev) HIP_OK(hipEventCreate(&e));
  for (int i = 0; i < steps; ++i) {
    HIP_OK(hipEventRecord(ev[2 * i], st));
    step(i);
    HIP_OK(hipEventRecord(ev[2 * i + 1], st));
  }
  HIP_OK(hipStreamSynchronize(st));
  check(yskn_smp_sync(h, st), "yskn_smp_sync");
  double tot = 0;
  for (int i = 0; i < steps; ++i) {
    float ms = 0;
    HIP_OK(hipEventElapsedTime(&ms, ev[2 * i], ev[2 * i + 1]));
    tot += ms;
  }
  const double us = tot * 1e3 / steps;
  std::vector<uint32_t> ids(rows);
  HIP_OK(hipMemcpy(ids.data(), d_ids, rows * sizeof(uint32_t), hipMemcpyDeviceToHost));
  uint64_t digest = 0;
  for (int r = 0; r < rows; ++r) digest = yskn::mix64(digest ^ ids[r]);
  uint64_t s[4] = {0, 0, 0, 0};
  if (yskn_smp_get_stats(h, s, 4) < 0) check(-1, "yskn_smp_get_stats");  // returns the count
  printf("{\"mode\": \"sample\", \"rows\": %d, \"vocab\": %d, \"steps\": %d, \"warmup\": %d, "
         "\"us_per_step\": %.3f, \"rows_per_s\": %.1f, \"hbm_gbs\": %.1f, \"ids_digest\": \"%016llx\", "
         "\"dense_rows\": %llu, \"candidates\": %llu}\n",
         rows, V, steps, warmup, us, rows / us * 1e6, (double)bytes / us / 1e3,
         (unsigned long long)digest, (unsigned long long)s[1], (unsigned long long)s[3]);
  for (auto& e : ev) HIP_OK(hipEventDestroy(e));
  yskn_smp_destroy(h);
  for (auto& b : buf) HIP_OK(hipFree(b));
  HIP_OK(hipFree(d_pos));
  HIP_OK(hipFree(d_ids));
  HIP_OK(hipFree(d_lpi));
  HIP_OK(hipFree(d_lp));
  HIP_OK(hipFree(d_st));
  return 0;
}
