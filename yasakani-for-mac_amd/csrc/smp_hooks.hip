// smp_hooks.hip -- device-math test hook of the sampling library.
//
// yskn_smp_pm_test evaluates one device primitive of the sampler on inputs
// given in host memory, so that its binary64/binary32 results can be compared
// bit for bit with the CPU restatement. It is the counterpart of the
// reference's yskn_pm_test (src/pm_test.cu:30-52; fn 10 = exp_d, fn 11 =
// log_d there as here), the tail's exact prefix-sum scan (fn 8) and the two
// bounded approximations of the certified dense tail (fn 15, 16). Not on the
// sampling path: it allocates, copies and synchronises.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/yskn_smp.h"
#include "smp_internal.hpp"
#include "smp_math.hpp"

namespace yskn {
namespace {

__global__ __launch_bounds__(256) void pm_test_kernel(int fn, uint64_t base, const uint64_t* in, void* out,
                                                      int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  uint64_t* o64 = (uint64_t*)out;
  uint32_t* o32 = (uint32_t*)out;
  switch (fn) {
    case 10: o64[i] = pm_bits(exp_d(__longlong_as_double((long long)in[i]))); break;
    case 11: o64[i] = pm_bits(log_d(__longlong_as_double((long long)in[i]))); break;
    case 12: {
      const uint64_t seed = in[3 * i], pos = in[3 * i + 1];
      const uint32_t tok = (uint32_t)in[3 * i + 2];
      o64[i] = pm_bits(gumbel_from_key(position_key(seed, pos), tok));
      break;
    }
    case 13: o64[i] = pm_bits(uniform_v2(in[2 * i], in[2 * i + 1])); break;
    case 14: o64[i] = mix64(in[i]); break;
    case 15: o64[i] = pm_bits(exp_approx(__longlong_as_double((long long)in[i]))); break;
    case 16:
      o64[i] = __float_as_uint(score_approx(__uint_as_float((uint32_t)in[3 * i]), in[3 * i + 1],
                                            (uint32_t)in[3 * i + 2]));
      break;
    case 6:
    case 7: {
      const uint32_t b = (uint32_t)(base + (uint64_t)i);
      const float x = __uint_as_float(b);
      o32[i] = __float_as_uint(fn == 6 ? rsqrt_rn_f32(x) : sqrt_rn_f32(x));
      break;
    }
    default: break;
  }
}

int words_in(int fn) {
  switch (fn) {
    case 10: case 11: case 14: case 15: return 1;
    case 12: case 16: return 3;
    case 13: return 2;
    case 8: return 1;
    case 6: case 7: return 0;
    default: return -1;
  }
}

}  // namespace
}  // namespace yskn

extern "C" int yskn_smp_pm_test(int32_t fn, uint64_t base, const void* host_in, void* host_out, int64_t n) {
  using namespace yskn;
  const int win = words_in(fn);
  if (win < 0 || n <= 0 || n > (1ll << 28) || !host_out || (win > 0 && !host_in)) return YSKN_SMP_EINVAL;
  const size_t in_bytes = (size_t)n * (size_t)win * 8u;
  const size_t out_bytes = (size_t)n * (fn >= 8 ? 8u : 4u);
  void* d = nullptr;
  hipError_t e = hipMalloc(&d, in_bytes + out_bytes + 16);
  if (e != hipSuccess) return YSKN_SMP_EDEVICE;
  uint64_t* din = (uint64_t*)d;
  void* dout = (char*)d + in_bytes;
  if (win > 0) e = hipMemcpy(din, host_in, in_bytes, hipMemcpyHostToDevice);
  if (e == hipSuccess) {
    if (fn == 8) {
      e = launch_prefix_test((const double*)din, (double*)dout, n, nullptr);
    } else {
      hipLaunchKernelGGL(pm_test_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, nullptr, fn, base, din,
                         dout, n);
      e = hipGetLastError();
    }
  }
  if (e == hipSuccess) e = hipMemcpy(host_out, dout, out_bytes, hipMemcpyDeviceToHost);
  const hipError_t f = hipFree(d);
  if (e == hipSuccess) e = f;
  return e == hipSuccess ? YSKN_SMP_OK : YSKN_SMP_EDEVICE;
}
