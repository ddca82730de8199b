// Fused RMSNorm and interleaved rotary embedding (the fork's RMSNorm and
// apply_rotary_emb, one kernel each; app/engine/fusedops.py:61-133).
//
// rms_norm: y = round(round(x * r) * w), r = 1 / sqrt(sum(x^2) / D + eps), the
// two roundings the fork's `_norm(x.float()).type_as(x) * weight` makes
// (app/engine/fusedops.py:8-14, 88-93). One wave per row. The sum of squares
// goes 64 chunks (of 8 elements) at a time: each chunk's squares by an fma
// chain in element order from 0, the 64 chunk sums by the rising-distance DPP
// butterfly, and these partial sums left to right - the order the GEMV's
// folded norm uses (a wave per 64 chunks there), so the fused and unfused
// forms agree bit for bit.
// Single pass over HBM: the row is re-read for the output from L1/L2.
//
// rope: pairs (2i, 2i+1) of the last axis, y0 = x0*c - x1*s, y1 = x1*c + x0*s
// in fp32 with each product and the sum rounded separately (no fma), then
// one rounding to the activation type (app/engine/fusedops.py:125-132).
#include "ttsp_common.h"

namespace ttsp {

constexpr int NORM_THREADS = 256;

template <int DT>
__global__ __launch_bounds__(NORM_THREADS) void rms_norm_kernel(
    const uint16_t* __restrict__ X, const uint16_t* __restrict__ Wt, uint16_t* __restrict__ Y,
    int rows, int D, float eps) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * (NORM_THREADS / 64) + (threadIdx.x >> 6);
  if (row >= rows) return;  // whole waves
  const size_t base = (size_t)row * D;
  const uint4* xr = reinterpret_cast<const uint4*>(X + base);
  const int nc = D >> 3;
  float ss = 0.0f;
  for (int c0 = 0; c0 < nc; c0 += 64) {  // 64 chunks per step, steps left to right
    float acc = 0.0f;
    if (c0 + lane < nc) {
      const uint4 v = xr[c0 + lane];
      const uint32_t u[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const float a = Elem<DT>::load(u[k]), b = Elem<DT>::load(u[k] >> 16);
        acc = __builtin_fmaf(a, a, acc);
        acc = __builtin_fmaf(b, b, acc);
      }
    }
    const float part = wave_sum_dpp(acc);
    ss = c0 == 0 ? part : __fadd_rn(ss, part);
  }
  const float r = rsqrt_rn(__fadd_rn(__fdiv_rn(ss, (float)D), eps));

  const uint4* wr = reinterpret_cast<const uint4*>(Wt);
  uint4* yr = reinterpret_cast<uint4*>(Y + base);
  for (int c = lane; c < nc; c += 64) {
    const uint4 v = xr[c], g = wr[c];
    const uint32_t u[4] = {v.x, v.y, v.z, v.w}, gw[4] = {g.x, g.y, g.z, g.w};
    uint32_t o[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const float n0 = Elem<DT>::load(Elem<DT>::store(__fmul_rn(Elem<DT>::load(u[k]), r)));
      const float n1 = Elem<DT>::load(Elem<DT>::store(__fmul_rn(Elem<DT>::load(u[k] >> 16), r)));
      const uint32_t y0 = Elem<DT>::store(__fmul_rn(n0, Elem<DT>::load(gw[k])));
      const uint32_t y1 = Elem<DT>::store(__fmul_rn(n1, Elem<DT>::load(gw[k] >> 16)));
      o[k] = y0 | (y1 << 16);
    }
    yr[c] = make_uint4(o[0], o[1], o[2], o[3]);
  }
}

template <int DT>
__global__ __launch_bounds__(256) void rope_kernel(const uint16_t* __restrict__ X,
                                                   const void* __restrict__ F, int ftype,
                                                   uint16_t* __restrict__ Y, long long pairs,
                                                   int half_dim, int heads, int seq) {
  const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= pairs) return;
  const int p = (int)(i % half_dim);
  const int s = (int)((i / half_dim / heads) % seq);
  const size_t f = ((size_t)s * half_dim + p) * 2;
  const float fr = load_elem(F, f, ftype);
  const float fi = load_elem(F, f + 1, ftype);
  const uint32_t u = reinterpret_cast<const uint32_t*>(X)[i];
  const float x0 = Elem<DT>::load(u), x1 = Elem<DT>::load(u >> 16);
  const uint32_t y0 = Elem<DT>::store(__fsub_rn(__fmul_rn(x0, fr), __fmul_rn(x1, fi)));
  const uint32_t y1 = Elem<DT>::store(__fadd_rn(__fmul_rn(x1, fr), __fmul_rn(x0, fi)));
  reinterpret_cast<uint32_t*>(Y)[i] = y0 | (y1 << 16);
}

}  // namespace ttsp

using namespace ttsp;

extern "C" int ttsp_rms_norm(const void* X, const void* Wt, void* Y, int rows, int D, float eps,
                             int dtype, hipStream_t stream) {
  if (rows < 0 || D <= 0 || D % 8) return (int)hipErrorInvalidValue;
  if (rows == 0) return 0;
  const unsigned grid = (unsigned)((rows + NORM_THREADS / 64 - 1) / (NORM_THREADS / 64));
  if (dtype == DT_F16)
    hipLaunchKernelGGL(rms_norm_kernel<DT_F16>, dim3(grid), dim3(NORM_THREADS), 0, stream,
                       (const uint16_t*)X, (const uint16_t*)Wt, (uint16_t*)Y, rows, D, eps);
  else if (dtype == DT_BF16)
    hipLaunchKernelGGL(rms_norm_kernel<DT_BF16>, dim3(grid), dim3(NORM_THREADS), 0, stream,
                       (const uint16_t*)X, (const uint16_t*)Wt, (uint16_t*)Y, rows, D, eps);
  else
    return (int)hipErrorInvalidValue;
  TTSP_RETURN_LAUNCH();
}

extern "C" int ttsp_rope(const void* X, const void* F, int ftype, void* Y, long long pairs,
                         int half_dim, int heads, int seq, int dtype, hipStream_t stream) {
  if (pairs < 0 || half_dim <= 0 || heads <= 0 || seq <= 0 || ftype < 0 || ftype > 2)
    return (int)hipErrorInvalidValue;
  if (pairs == 0) return 0;
  const dim3 grid((unsigned)((pairs + 255) / 256));
  if (dtype == DT_F16)
    hipLaunchKernelGGL(rope_kernel<DT_F16>, grid, dim3(256), 0, stream, (const uint16_t*)X, F,
                       ftype, (uint16_t*)Y, pairs, half_dim, heads, seq);
  else if (dtype == DT_BF16)
    hipLaunchKernelGGL(rope_kernel<DT_BF16>, grid, dim3(256), 0, stream, (const uint16_t*)X, F,
                       ftype, (uint16_t*)Y, pairs, half_dim, heads, seq);
  else
    return (int)hipErrorInvalidValue;
  TTSP_RETURN_LAUNCH();
}
