// NF4 dequantisation (bitsandbytes layout, see nf4_gemv.hip): every code to
// round(code * scale) in fp16 / bf16 / fp32, one rounding - the values
// bitsandbytes' dequantize_4bit produces and the prefill GEMM feeds to MFMA.
#include "ttsp_common.h"

namespace ttsp {

// Dequantise n codes (flattened) to fp16/bf16/fp32: out = round(code[q] * s),
// one rounding, as bitsandbytes' dequantize_4bit. 16 codes (8 bytes) per thread.
template <int ODT, bool NESTED>
__global__ __launch_bounds__(256) void nf4_dequant_kernel(
    const uint8_t* __restrict__ W, const uint8_t* __restrict__ A8, const float* __restrict__ AMAX,
    const float* __restrict__ CODE2, float offset, const float* __restrict__ LUT,
    void* __restrict__ OUT, long long n, int bs_shift, int bs2_shift) {
  __shared__ float lut[16];
  if (threadIdx.x < 16) lut[threadIdx.x] = LUT[threadIdx.x];
  __syncthreads();
  const long long t = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  const long long k0 = t * 16;
  if (k0 >= n) return;
  const long long b = k0 >> bs_shift;  // 16 codes never straddle a block (bs >= 64)
  float s;
  if constexpr (NESTED) {
    s = __fadd_rn(__fmul_rn(CODE2[A8[b]], AMAX[b >> bs2_shift]), offset);
  } else {
    s = AMAX[b];
  }
  uint8_t bytes[8];
  const long long nb = (n - k0 + 1) / 2 < 8 ? (n - k0 + 1) / 2 : 8;
  if (nb == 8) {
    const uint2 v = *reinterpret_cast<const uint2*>(W + k0 / 2);
    *reinterpret_cast<uint2*>(bytes) = v;
  } else {
    for (int i = 0; i < 8; ++i) bytes[i] = i < nb ? W[k0 / 2 + i] : 0;
  }
  float v[16];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    v[2 * i] = __fmul_rn(lut[bytes[i] >> 4], s);
    v[2 * i + 1] = __fmul_rn(lut[bytes[i] & 15], s);
  }
  const int cnt = n - k0 < 16 ? (int)(n - k0) : 16;
  if constexpr (ODT == DT_F32) {
    float* o = (float*)OUT + k0;
    if (cnt == 16) {
#pragma unroll
      for (int i = 0; i < 4; ++i)
        reinterpret_cast<float4*>(o)[i] = make_float4(v[4 * i], v[4 * i + 1], v[4 * i + 2], v[4 * i + 3]);
    } else {
      for (int i = 0; i < cnt; ++i) o[i] = v[i];
    }
  } else {
    uint16_t* o = (uint16_t*)OUT + k0;
    uint16_t h[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) h[i] = Elem<ODT>::store(v[i]);
    if (cnt == 16) {
      reinterpret_cast<uint4*>(o)[0] = *reinterpret_cast<uint4*>(h);
      reinterpret_cast<uint4*>(o)[1] = *reinterpret_cast<uint4*>(h + 8);
    } else {
      for (int i = 0; i < cnt; ++i) o[i] = h[i];
    }
  }
}

static int dq_log2_exact(int v) {
  if (v <= 0 || (v & (v - 1))) return -1;
  int s = 0;
  while ((1 << s) < v) ++s;
  return s;
}

}  // namespace ttsp

using namespace ttsp;

extern "C" int ttsp_nf4_dequant(const uint8_t* W, const uint8_t* A8, const float* AMAX,
                                const float* CODE2, float offset, const float* LUT, void* out,
                                int out_dtype, long long n, int blocksize, int blocksize2,
                                hipStream_t stream) {
  const int bs_shift = dq_log2_exact(blocksize);
  const int bs2_shift = A8 ? dq_log2_exact(blocksize2) : 0;
  if (bs_shift < 6 || bs2_shift < 0 || n < 0) return (int)hipErrorInvalidValue;
  if (n == 0) return 0;
  const long long threads = (n + 15) / 16;
  const dim3 grid((unsigned)((threads + 255) / 256));
#define TTSP_DQ(ODT, NESTED)                                                                  \
  hipLaunchKernelGGL((nf4_dequant_kernel<ODT, NESTED>), grid, dim3(256), 0, stream, W, A8, AMAX, \
                     CODE2, offset, LUT, out, n, bs_shift, bs2_shift)
  switch (out_dtype) {
    case DT_F16: if (A8) TTSP_DQ(DT_F16, true); else TTSP_DQ(DT_F16, false); break;
    case DT_BF16: if (A8) TTSP_DQ(DT_BF16, true); else TTSP_DQ(DT_BF16, false); break;
    case DT_F32: if (A8) TTSP_DQ(DT_F32, true); else TTSP_DQ(DT_F32, false); break;
    default: return (int)hipErrorInvalidValue;
  }
#undef TTSP_DQ
  TTSP_RETURN_LAUNCH();
}
