// Numerics self-test entry points: evaluate the device primitives every
// kernel relies on (exp_cw, sqrt_rn, silu_rn, the zero-addend dot2) over
// caller arrays, so a test can compare them bit for bit against IEEE CPU
// arithmetic. No counterpart in the reference; used by the test suite.
#include "ttsp_common.h"

namespace ttsp {

__global__ void selftest_math_kernel(const float* __restrict__ in, int n, int op, float* __restrict__ out) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const float x = in[i];
  float y;
  switch (op) {
    case 0: y = exp_cw(x); break;
    case 1: y = sqrt_rn(x); break;
    case 2: y = rsqrt_rn(x); break;
    default: y = silu_rn(x); break;
  }
  out[i] = y;
}

template <int DT>
__global__ void selftest_dot2_kernel(const uint32_t* __restrict__ a, const uint32_t* __restrict__ b, int n,
                                     float* __restrict__ out) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  out[i] = Elem<DT>::dot2(a[i], b[i]);
}

}  // namespace ttsp

using namespace ttsp;

extern "C" int ttsp_selftest_math(const float* in, int n, int op, float* out, hipStream_t stream) {
  if (n < 0 || op < 0 || op > 3) return (int)hipErrorInvalidValue;
  if (n == 0) return 0;
  hipLaunchKernelGGL(selftest_math_kernel, dim3((n + 255) / 256), dim3(256), 0, stream, in, n, op, out);
  TTSP_RETURN_LAUNCH();
}

extern "C" int ttsp_selftest_dot2(const uint32_t* a, const uint32_t* b, int n, int dtype, float* out,
                                  hipStream_t stream) {
  if (n < 0) return (int)hipErrorInvalidValue;
  if (n == 0) return 0;
  if (dtype == DT_F16)
    hipLaunchKernelGGL(selftest_dot2_kernel<DT_F16>, dim3((n + 255) / 256), dim3(256), 0, stream, a, b, n, out);
  else if (dtype == DT_BF16)
    hipLaunchKernelGGL(selftest_dot2_kernel<DT_BF16>, dim3((n + 255) / 256), dim3(256), 0, stream, a, b, n, out);
  else
    return (int)hipErrorInvalidValue;
  TTSP_RETURN_LAUNCH();
}
