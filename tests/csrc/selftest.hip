// Numerics self-test entry points - TEST INFRASTRUCTURE, built into
// tests/libttsp_selftest.so, not the product library: evaluate the device
// primitives every kernel relies on (exp_cw, sqrt_rn, silu_rn, the
// fp16-operand fma, from ttspipe_amd/csrc/ttsp_common.h) over caller arrays,
// so a test can compare them bit for bit against IEEE CPU arithmetic.
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

// out = fma(a.hi, b.hi, fma(a.lo, b.lo, c)) on packed fp16 pairs: the GEMV's
// inner step (v_fma_mix_f32 with op_sel), to be checked against IEEE fmaf.
__global__ void selftest_fma16_kernel(const uint32_t* __restrict__ a, const uint32_t* __restrict__ b,
                                      const float* __restrict__ c, int n, float* __restrict__ out) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const float t = __builtin_fmaf(h_lo(a[i]), h_lo(b[i]), c[i]);
  out[i] = __builtin_fmaf(h_hi(a[i]), h_hi(b[i]), t);
}

}  // namespace ttsp

using namespace ttsp;

extern "C" int ttsp_selftest_math(const float* in, int n, int op, float* out, hipStream_t stream) {
  if (n < 0 || op < 0 || op > 3) return (int)hipErrorInvalidValue;
  if (n == 0) return 0;
  hipLaunchKernelGGL(selftest_math_kernel, dim3((n + 255) / 256), dim3(256), 0, stream, in, n, op, out);
  TTSP_RETURN_LAUNCH();
}

extern "C" int ttsp_selftest_fma16(const uint32_t* a, const uint32_t* b, const float* c, int n,
                                   float* out, hipStream_t stream) {
  if (n < 0) return (int)hipErrorInvalidValue;
  if (n == 0) return 0;
  hipLaunchKernelGGL(selftest_fma16_kernel, dim3((n + 255) / 256), dim3(256), 0, stream, a, b, c, n, out);
  TTSP_RETURN_LAUNCH();
}
