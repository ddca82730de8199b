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
// Single pass over HBM: rows of up to 4096 elements stay in registers between
// the sum and the output; longer rows are re-read from L1/L2.
//
// rope: pairs (2i, 2i+1) of the last axis, y0 = x0*c - x1*s, y1 = x1*c + x0*s
// in fp32 with each product and the sum rounded separately (no fma), then
// one rounding to the activation type (app/engine/fusedops.py:125-132).
#include "ttsp_common.h"

namespace ttsp {

constexpr int NORM_THREADS = 256;

// One wave per row. Rows of at most NORM_REG x 512 elements are read into
// registers with all loads issued before the first wait (a row of 2560 bf16
// is five 16-byte loads a lane) and normalised from there; longer rows take
// the loop that streams 64 chunks at a time and re-reads the row for the
// output. Both give the same bits: chunk c's squares are summed by lane
// c % 64 of step c / 64.
constexpr int NORM_REG = 8;

template <int DT>
__device__ __forceinline__ float sumsq_chunk(uint4 v, float acc) {
  const uint32_t u[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const float a = Elem<DT>::load(u[k]), b = Elem<DT>::load(u[k] >> 16);
    acc = __builtin_fmaf(a, a, acc);
    acc = __builtin_fmaf(b, b, acc);
  }
  return acc;
}

template <int DT>
__device__ __forceinline__ uint4 norm_chunk(uint4 v, uint4 g, float r) {
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
  return make_uint4(o[0], o[1], o[2], o[3]);
}

template <int DT, bool REG>
__global__ __launch_bounds__(NORM_THREADS) void rms_norm_kernel(
    const uint16_t* __restrict__ X, const uint16_t* __restrict__ Wt, uint16_t* __restrict__ Y,
    int rows, int D, float eps) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * (NORM_THREADS / 64) + (threadIdx.x >> 6);
  if (row >= rows) return;  // whole waves
  const size_t base = (size_t)row * D;
  const uint4* xr = reinterpret_cast<const uint4*>(X + base);
  const uint4* wr = reinterpret_cast<const uint4*>(Wt);
  uint4* yr = reinterpret_cast<uint4*>(Y + base);
  const int nc = D >> 3;
  if constexpr (REG) {
    // chunk lane + 64 j, clamped loads (unconditional: the waits stay exact)
    uint4 v[NORM_REG], g[NORM_REG];
#pragma unroll
    for (int j = 0; j < NORM_REG; ++j) v[j] = xr[min(lane + 64 * j, nc - 1)];
#pragma unroll
    for (int j = 0; j < NORM_REG; ++j) g[j] = wr[min(lane + 64 * j, nc - 1)];
    float ss = 0.0f;
#pragma unroll
    for (int j = 0; j < NORM_REG; ++j) {
      if (64 * j >= nc) break;  // wave-uniform
      const float part = wave_sum_dpp(lane + 64 * j < nc ? sumsq_chunk<DT>(v[j], 0.0f) : 0.0f);
      ss = j == 0 ? part : __fadd_rn(ss, part);
    }
    const float r = rsqrt_rn(__fadd_rn(__fdiv_rn(ss, (float)D), eps));
#pragma unroll
    for (int j = 0; j < NORM_REG; ++j)
      if (lane + 64 * j < nc) yr[lane + 64 * j] = norm_chunk<DT>(v[j], g[j], r);
  } else {
    float ss = 0.0f;
    for (int c0 = 0; c0 < nc; c0 += 64) {  // 64 chunks per step, steps left to right
      const float acc = c0 + lane < nc ? sumsq_chunk<DT>(xr[c0 + lane], 0.0f) : 0.0f;
      const float part = wave_sum_dpp(acc);
      ss = c0 == 0 ? part : __fadd_rn(ss, part);
    }
    const float r = rsqrt_rn(__fadd_rn(__fdiv_rn(ss, (float)D), eps));
    for (int c = lane; c < nc; c += 64) yr[c] = norm_chunk<DT>(xr[c], wr[c], r);
  }
}

// One pair per thread: any half_dim and 4-byte alignment (the general form;
// the launcher takes it when the 16-byte one does not apply).
template <int DT>
__global__ __launch_bounds__(256) void rope_pair_kernel(const uint16_t* __restrict__ X,
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

// Four pairs (16 bytes of x) per thread; the pairs of a piece share their row
// (half_dim % 4 == 0), so one table load covers them (16 bytes of a 16-bit
// table, 32 of an fp32 one). Index arithmetic in 32 bits (the launcher checks
// that pairs and seq * half_dim are below 2^31).
template <int DT>
__global__ __launch_bounds__(256) void rope_kernel(const uint16_t* __restrict__ X,
                                                   const void* __restrict__ F, int ftype,
                                                   uint16_t* __restrict__ Y, unsigned pieces,
                                                   unsigned half_dim, unsigned heads, unsigned seq) {
  const unsigned i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= pieces) return;
  const unsigned pair = 4 * i;
  const unsigned p = pair % half_dim;
  const unsigned s = (pair / half_dim / heads) % seq;
  const unsigned f = s * half_dim + p;  // first pair's table entry
  float fr[4], fi[4];
  if (ftype == DT_F32) {
    const float4* t = reinterpret_cast<const float4*>(reinterpret_cast<const float*>(F) + 2 * (size_t)f);
    const float4 a = t[0], b = t[1];
    fr[0] = a.x, fi[0] = a.y, fr[1] = a.z, fi[1] = a.w, fr[2] = b.x, fi[2] = b.y, fr[3] = b.z, fi[3] = b.w;
  } else {
    const uint4 t = *reinterpret_cast<const uint4*>(reinterpret_cast<const uint16_t*>(F) + 2 * (size_t)f);
    const uint32_t w[4] = {t.x, t.y, t.z, t.w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      fr[k] = ftype == DT_F16 ? f16_to_f32(w[k] & 0xffffu) : bf16_to_f32(w[k] & 0xffffu);
      fi[k] = ftype == DT_F16 ? f16_to_f32(w[k] >> 16) : bf16_to_f32(w[k] >> 16);
    }
  }
  const uint4 xv = reinterpret_cast<const uint4*>(X)[i];
  const uint32_t u[4] = {xv.x, xv.y, xv.z, xv.w};
  uint32_t o[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const float x0 = Elem<DT>::load(u[k]), x1 = Elem<DT>::load(u[k] >> 16);
    const uint32_t y0 = Elem<DT>::store(__fsub_rn(__fmul_rn(x0, fr[k]), __fmul_rn(x1, fi[k])));
    const uint32_t y1 = Elem<DT>::store(__fadd_rn(__fmul_rn(x1, fr[k]), __fmul_rn(x0, fi[k])));
    o[k] = y0 | (y1 << 16);
  }
  reinterpret_cast<uint4*>(Y)[i] = make_uint4(o[0], o[1], o[2], o[3]);
}

}  // namespace ttsp

using namespace ttsp;

extern "C" int ttsp_rms_norm(const void* X, const void* Wt, void* Y, int rows, int D, float eps,
                             int dtype, hipStream_t stream) {
  if (rows < 0 || D <= 0 || D % 8) return (int)hipErrorInvalidValue;
  if ((uintptr_t)X % 16 || (uintptr_t)Wt % 16 || (uintptr_t)Y % 16) return (int)hipErrorInvalidValue;
  if (rows == 0) return 0;
  const unsigned grid = (unsigned)((rows + NORM_THREADS / 64 - 1) / (NORM_THREADS / 64));
  const bool reg = D <= NORM_REG * 512;
#define TTSP_N(DTV, RV)                                                                                        \
  hipLaunchKernelGGL((rms_norm_kernel<DTV, RV>), dim3(grid), dim3(NORM_THREADS), 0, stream, (const uint16_t*)X, \
                     (const uint16_t*)Wt, (uint16_t*)Y, rows, D, eps)
  if (dtype == DT_F16) {
    if (reg) TTSP_N(DT_F16, true);
    else TTSP_N(DT_F16, false);
  } else if (dtype == DT_BF16) {
    if (reg) TTSP_N(DT_BF16, true);
    else TTSP_N(DT_BF16, false);
  } else {
    return (int)hipErrorInvalidValue;
  }
#undef TTSP_N
  TTSP_RETURN_LAUNCH();
}

// pairs: elements of X / 2. Four pairs per thread where half_dim and pairs are
// multiples of 4, pairs and the table's pairs are below 2^31 and X, Y, F are
// 16-byte aligned; one pair per thread otherwise.
extern "C" int ttsp_rope(const void* X, const void* F, int ftype, void* Y, long long pairs,
                         int half_dim, int heads, int seq, int dtype, hipStream_t stream) {
  if (pairs < 0 || half_dim <= 0 || heads <= 0 || seq <= 0 || ftype < 0 || ftype > 2)
    return (int)hipErrorInvalidValue;
  if (dtype != DT_F16 && dtype != DT_BF16) return (int)hipErrorInvalidValue;
  if ((uintptr_t)X % 4 || (uintptr_t)Y % 4 || (uintptr_t)F % (ftype == DT_F32 ? 4 : 2))
    return (int)hipErrorInvalidValue;
  if (pairs == 0) return 0;
  const bool wide = half_dim % 4 == 0 && pairs % 4 == 0 && pairs < (1LL << 31) &&
                    (long long)seq * half_dim < (1LL << 31) && (uintptr_t)X % 16 == 0 &&
                    (uintptr_t)Y % 16 == 0 && (uintptr_t)F % 16 == 0;
  if (wide) {
    const unsigned pieces = (unsigned)(pairs / 4);
    const dim3 grid((pieces + 255) / 256);
#define TTSP_R(DTV)                                                                              \
  hipLaunchKernelGGL(rope_kernel<DTV>, grid, dim3(256), 0, stream, (const uint16_t*)X, F, ftype, \
                     (uint16_t*)Y, pieces, (unsigned)half_dim, (unsigned)heads, (unsigned)seq)
    if (dtype == DT_F16) TTSP_R(DT_F16);
    else TTSP_R(DT_BF16);
#undef TTSP_R
  } else {
    const dim3 grid((unsigned)((pairs + 255) / 256));
#define TTSP_R(DTV)                                                                                   \
  hipLaunchKernelGGL(rope_pair_kernel<DTV>, grid, dim3(256), 0, stream, (const uint16_t*)X, F, ftype, \
                     (uint16_t*)Y, pairs, half_dim, heads, seq)
    if (dtype == DT_F16) TTSP_R(DT_F16);
    else TTSP_R(DT_BF16);
#undef TTSP_R
  }
  TTSP_RETURN_LAUNCH();
}
