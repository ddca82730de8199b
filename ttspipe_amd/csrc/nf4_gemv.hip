// NF4 GEMV (one activation row) and NF4 dequantisation, reading the
// bitsandbytes layout in place:
//   * W is the row-major flattened weight, two 4-bit codes per byte, the HIGH
//     nibble holding the even flattened index (byte j = q[2j] << 4 | q[2j+1]);
//   * scale block b covers flattened codes [b*bs, (b+1)*bs), bs a power of two
//     >= 64, so with K % bs == 0 a block never straddles a row;
//   * plain scales are fp32 absmax[b]; nested ("double-quant") scales are
//     code2[a8[b]] * absmax2[b >> log2(bs2)] + offset, two fp32 roundings.
//
// GEMV design (HBM-bound, ~1/2 byte per weight):
//   * A row is K/8 dwords (8 codes each). Lane l of a wave owns dwords
//     l + 64*c of every row it visits, so each load instruction reads 256
//     contiguous bytes, and the 8 activations matching a dword stay in
//     registers for every row (x is read once per wave, not once per row).
//   * Each byte (two codes) becomes a packed pair of fp16 code values through
//     a 256-entry LDS table. A dword's 8 products are chained in code order
//     (v_fma_mix_f32 on the fp16 halves, the first onto +0, one IEEE rounding
//     each), and the dword's partial meets its block scale in
//     one fma into the lane accumulator: the scale multiplies the block's
//     partial sum instead of each weight (the factored form the reference
//     CPU kernel uses, app/engine/nf4cpu.py:115-129).
//   * bf16 activations are first rescaled per wave by a power of two and
//     converted to fp16 exactly, so both activation types get 11-bit codes.
//   * The scales of a workgroup's rows are contiguous; they are loaded once,
//     cooperatively, resolved (nested: code2 from an LDS copy) and parked in
//     LDS, where the 8 lanes sharing a 64-code block read one broadcast word.
//   * KS waves of a workgroup split K (chunks interleaved), RPW rows per wave
//     are issued together; all loads of a wave are in flight before the first
//     multiply. Reductions are a fixed xor-butterfly over the wave, then a
//     fixed left-to-right sum over the KS slices: the result does not depend
//     on scheduling.
#include "ttsp_common.h"

namespace ttsp {

constexpr int GEMV_THREADS = 256;
constexpr int GEMV_WAVES = GEMV_THREADS / 64;

// 256-entry table: entry v holds (code[v >> 4], code[v & 15]) rounded to the
// activation type, low half first, matching the activation pair (x[2i], x[2i+1]).
template <int DT>
__device__ __forceinline__ uint32_t lut_pair(const float* __restrict__ LUT, int v) {
  const uint32_t lo = Elem<DT>::store(LUT[v >> 4]);
  const uint32_t hi = Elem<DT>::store(LUT[v & 15]);
  return lo | (hi << 16);
}

// Output rounding as the unfused fork: the matmul result is rounded to the
// activation type, and so is each elementwise op after it (app/engine/
// nf4gemv.py:215-226): residual y' = round(R + y), gate y' = round(round(silu(R)) * y).
template <int DT>
__device__ __forceinline__ void store_row(uint16_t* __restrict__ Y, const uint16_t* __restrict__ R,
                                          int epi, int row, float acc) {
  const float y = Elem<DT>::load(Elem<DT>::store(acc));
  float o = y;
  if (epi == 1) {
    o = __fadd_rn(Elem<DT>::load(R[row]), y);
  } else if (epi == 2) {
    o = __fmul_rn(Elem<DT>::load(Elem<DT>::store(silu_rn(Elem<DT>::load(R[row])))), y);
  }
  Y[row] = Elem<DT>::store(o);
}

template <int DT, int J, int RPW, bool NESTED>
__global__ __launch_bounds__(GEMV_THREADS) void nf4_gemv_kernel(
    const uint32_t* __restrict__ W, const uint8_t* __restrict__ A8,
    const float* __restrict__ AMAX, const float* __restrict__ CODE2, float offset,
    const float* __restrict__ LUT, const uint16_t* __restrict__ X, uint16_t* __restrict__ Y,
    const uint16_t* __restrict__ R, int epi, int M, int K, int KS, int bs_shift, int bs2_shift) {
  constexpr int SL = 4;  // scale entries a thread loads per batch
  __shared__ uint32_t lut[256];
  __shared__ float code2_s[NESTED ? 256 : 1];
  __shared__ float red[GEMV_WAVES][RPW];
  extern __shared__ float srow[];  // [rows of this workgroup][nblk]

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int ks = wave % KS;
  const int rg = wave / KS;
  const int KD = K >> 3;
  const int nblk = K >> bs_shift;
  const int sh = bs_shift - 3;
  const int rows_wg = (GEMV_WAVES / KS) * RPW;
  const int wg_row0 = blockIdx.x * rows_wg;
  const int row0 = wg_row0 + rg * RPW;
  const int nsc = rows_wg * nblk;                 // scale entries of this workgroup
  const long long sc_last = (long long)M * nblk - 1;
  const long long sc0 = (long long)wg_row0 * nblk;

  // 1. first batch of this workgroup's scales (contiguous: its rows are)
  float sv[SL];
  uint32_t av[NESTED ? SL : 1];
#pragma unroll
  for (int i = 0; i < SL; ++i) {
    const long long gb = min(sc0 + tid + i * GEMV_THREADS, sc_last);
    if constexpr (NESTED) {
      av[i] = A8[gb];
      sv[i] = AMAX[gb >> bs2_shift];
    } else {
      sv[i] = AMAX[gb];
    }
  }
  // 2. every weight dword this wave reads, all its rows at once
  uint32_t w[RPW][J];
#pragma unroll
  for (int r = 0; r < RPW; ++r) {
    const uint32_t* wr = W + (size_t)min(row0 + r, M - 1) * KD;
#pragma unroll
    for (int j = 0; j < J; ++j) {
      const int d = lane + 64 * (j * KS + ks);
      w[r][j] = d < KD ? __builtin_nontemporal_load(wr + d) : 0u;
    }
  }
  // 3. activations for this lane's dwords
  uint4 xr[J];
#pragma unroll
  for (int j = 0; j < J; ++j) {
    const int d = lane + 64 * (j * KS + ks);
    xr[j] = d < KD ? *reinterpret_cast<const uint4*>(X + 8 * (size_t)d) : make_uint4(0, 0, 0, 0);
  }
  // 4. tables in LDS (fp16 code pairs for either activation type)
  lut[tid] = lut_pair<DT_F16>(LUT, tid);
  if constexpr (NESTED) {
    code2_s[tid] = CODE2[tid];
    __syncthreads();
  }
#pragma unroll
  for (int i = 0; i < SL; ++i) {
    const int e = tid + i * GEMV_THREADS;
    if (e < nsc) {
      if constexpr (NESTED) srow[e] = __fadd_rn(__fmul_rn(code2_s[av[i]], sv[i]), offset);
      else srow[e] = sv[i];
    }
  }
  for (int e0 = SL * GEMV_THREADS; e0 < nsc; e0 += SL * GEMV_THREADS) {  // wide rows only
#pragma unroll
    for (int i = 0; i < SL; ++i) {
      const long long gb = min(sc0 + e0 + tid + i * GEMV_THREADS, sc_last);
      if constexpr (NESTED) {
        av[i] = A8[gb];
        sv[i] = AMAX[gb >> bs2_shift];
      } else {
        sv[i] = AMAX[gb];
      }
    }
#pragma unroll
    for (int i = 0; i < SL; ++i) {
      const int e = e0 + tid + i * GEMV_THREADS;
      if (e < nsc) {
        if constexpr (NESTED) srow[e] = __fadd_rn(__fmul_rn(code2_s[av[i]], sv[i]), offset);
        else srow[e] = sv[i];
      }
    }
  }
  __syncthreads();

  // bf16 activations: rescale this wave's slice by 2^-e so max|x| lands in
  // [2^14, 2^15) and convert to fp16 - exact, since bf16's 8 significant bits
  // fit in fp16's 11 - then every product below is fp16 x fp16 with 11-bit
  // codes. The wave's partial sums are scaled back by 2^e (also exact).
  int xe = 0;
  if constexpr (DT == DT_BF16) {
    float m = 0.0f;
#pragma unroll
    for (int j = 0; j < J; ++j) {
      const uint32_t u[4] = {xr[j].x, xr[j].y, xr[j].z, xr[j].w};
#pragma unroll
      for (int k = 0; k < 4; ++k)
        m = fmaxf(m, fmaxf(fabsf(bf16_to_f32(u[k] & 0xffffu)), fabsf(bf16_to_f32(u[k] >> 16))));
    }
    m = wave_max(m);
    if (m > 0.0f && m <= 3.402823466e38f) xe = __builtin_amdgcn_frexp_expf(m) - 15;
#pragma unroll
    for (int j = 0; j < J; ++j) {
      uint32_t* u = reinterpret_cast<uint32_t*>(&xr[j]);
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const uint32_t lo = f32_to_f16(__builtin_ldexpf(bf16_to_f32(u[k] & 0xffffu), -xe));
        const uint32_t hi = f32_to_f16(__builtin_ldexpf(bf16_to_f32(u[k] >> 16), -xe));
        u[k] = lo | (hi << 16);
      }
    }
  }

  // 5. dot products
#pragma unroll
  for (int r = 0; r < RPW; ++r) {
    const float* srr = srow + (rg * RPW + r) * nblk;
    float acc = 0.0f;
#pragma unroll
    for (int j = 0; j < J; ++j) {
      // Past the row's end w and x are zero; the clamped index keeps the
      // scale read inside the row (a finite value times zero).
      const int d = min(lane + 64 * (j * KS + ks), KD - 1);
      const float s = srr[d >> sh];
      const uint32_t wv = w[r][j];
      const uint32_t c0 = lut[wv & 0xffu], c1 = lut[(wv >> 8) & 0xffu];
      const uint32_t c2 = lut[(wv >> 16) & 0xffu], c3 = lut[wv >> 24];
      // the dword's 8 products in code order, each an fma (the first onto +0)
      float q = __builtin_fmaf(h_lo(c0), h_lo(xr[j].x), 0.0f);
      q = __builtin_fmaf(h_hi(c0), h_hi(xr[j].x), q);
      q = __builtin_fmaf(h_lo(c1), h_lo(xr[j].y), q);
      q = __builtin_fmaf(h_hi(c1), h_hi(xr[j].y), q);
      q = __builtin_fmaf(h_lo(c2), h_lo(xr[j].z), q);
      q = __builtin_fmaf(h_hi(c2), h_hi(xr[j].z), q);
      q = __builtin_fmaf(h_lo(c3), h_lo(xr[j].w), q);
      q = __builtin_fmaf(h_hi(c3), h_hi(xr[j].w), q);
      acc = __builtin_fmaf(q, s, acc);
    }
    acc = wave_sum(acc);
    if constexpr (DT == DT_BF16) acc = __builtin_ldexpf(acc, xe);
    if (KS > 1) {
      if (lane == 0) red[wave][r] = acc;
    } else if (lane == r && row0 + r < M) {
      store_row<DT>(Y, R, epi, row0 + r, acc);
    }
  }
  if (KS > 1) {
    __syncthreads();
    if (ks == 0 && lane < RPW && row0 + lane < M) {
      float acc = red[wave][0];
#pragma unroll
      for (int r = 1; r < RPW; ++r) acc = lane == r ? red[wave][r] : acc;
      for (int k2 = 1; k2 < KS; ++k2) {
        float v = red[wave + k2][0];
#pragma unroll
        for (int r = 1; r < RPW; ++r) v = lane == r ? red[wave + k2][r] : v;
        acc = __fadd_rn(acc, v);
      }
      store_row<DT>(Y, R, epi, row0 + lane, acc);
    }
  }
}

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

// ---------------------------------------------------------------------------
// host side

static constexpr int kJ[] = {1, 2, 3, 4, 5, 6, 8, 10, 12, 16, 20, 24, 32};

// Launch shape for one row: K split over KS waves, RPW rows per wave.
// Chosen so a launch has >= ~2048 waves in flight on 256 CUs where the shape
// allows it; KS never leaves a wave without a 64-dword chunk.
struct GemvShape {
  int J, KS, RPW;
};

static GemvShape gemv_shape(int M, int K) {
  const int KD = K >> 3;
  int KS = 1;
  if (M <= 1536) KS = 4;
  else if (M <= 4096) KS = 2;
  while (KS > 1 && KD < 64 * KS) KS >>= 1;
  const int need = (KD + 64 * KS - 1) / (64 * KS);
  int J = 0;
  for (int v : kJ)
    if (v >= need) { J = v; break; }
  int RPW = 4;
  while (RPW > 1 && (long long)((M + RPW - 1) / RPW) * KS < 2048) RPW >>= 1;
  return {J, KS, RPW};
}

template <int DT, int J, int RPW, bool NESTED>
static void launch_gemv(const void* X, const uint8_t* W, const uint8_t* A8, const float* AMAX,
                        const float* CODE2, float offset, const float* LUT, void* Y, const void* R,
                        int epi, int M, int K, int KS, int bs_shift, int bs2_shift, hipStream_t st) {
  const int rows_per_wg = (GEMV_WAVES / KS) * RPW;
  const int grid = (M + rows_per_wg - 1) / rows_per_wg;
  const size_t shmem = (size_t)rows_per_wg * (K >> bs_shift) * sizeof(float);
  hipLaunchKernelGGL((nf4_gemv_kernel<DT, J, RPW, NESTED>), dim3(grid), dim3(GEMV_THREADS), shmem, st,
                     (const uint32_t*)W, A8, AMAX, CODE2, offset, LUT, (const uint16_t*)X,
                     (uint16_t*)Y, (const uint16_t*)R, epi, M, K, KS, bs_shift, bs2_shift);
}

template <int DT, int J, bool NESTED>
static void dispatch_rpw(int RPW, const void* X, const uint8_t* W, const uint8_t* A8,
                         const float* AMAX, const float* CODE2, float offset, const float* LUT,
                         void* Y, const void* R, int epi, int M, int K, int KS, int bs_shift,
                         int bs2_shift, hipStream_t st) {
  switch (RPW) {
    case 4: launch_gemv<DT, J, 4, NESTED>(X, W, A8, AMAX, CODE2, offset, LUT, Y, R, epi, M, K, KS, bs_shift, bs2_shift, st); break;
    case 2: launch_gemv<DT, J, 2, NESTED>(X, W, A8, AMAX, CODE2, offset, LUT, Y, R, epi, M, K, KS, bs_shift, bs2_shift, st); break;
    default: launch_gemv<DT, J, 1, NESTED>(X, W, A8, AMAX, CODE2, offset, LUT, Y, R, epi, M, K, KS, bs_shift, bs2_shift, st); break;
  }
}

template <int DT, bool NESTED>
static int dispatch_j(const GemvShape& g, const void* X, const uint8_t* W, const uint8_t* A8,
                      const float* AMAX, const float* CODE2, float offset, const float* LUT,
                      void* Y, const void* R, int epi, int M, int K, int bs_shift, int bs2_shift,
                      hipStream_t st) {
#define TTSP_J(JV)                                                                          \
  case JV:                                                                                   \
    dispatch_rpw<DT, JV, NESTED>(g.RPW, X, W, A8, AMAX, CODE2, offset, LUT, Y, R, epi, M, K, \
                                 g.KS, bs_shift, bs2_shift, st);                            \
    return 0;
  switch (g.J) {
    TTSP_J(1) TTSP_J(2) TTSP_J(3) TTSP_J(4) TTSP_J(5) TTSP_J(6) TTSP_J(8) TTSP_J(10)
    TTSP_J(12) TTSP_J(16) TTSP_J(20) TTSP_J(24) TTSP_J(32)
    default: return (int)hipErrorInvalidValue;
  }
#undef TTSP_J
}

static int log2_exact(int v) {
  if (v <= 0 || (v & (v - 1))) return -1;
  int s = 0;
  while ((1 << s) < v) ++s;
  return s;
}

int gemv_n1(const void* X, int dt, const uint8_t* W, const uint8_t* A8, const float* AMAX,
            const float* CODE2, float offset, const float* LUT, void* Y, const void* R, int epi,
            int M, int K, int blocksize, int blocksize2, hipStream_t st) {
  const int bs_shift = log2_exact(blocksize);
  const int bs2_shift = A8 ? log2_exact(blocksize2) : 0;
  if (bs_shift < 6 || bs2_shift < 0 || K % 128 || K % blocksize || M <= 0) return (int)hipErrorInvalidValue;
  if (epi < 0 || epi > 2 || (epi && !R)) return (int)hipErrorInvalidValue;
  const GemvShape g = gemv_shape(M, K);
  if (!g.J) return (int)hipErrorInvalidValue;
  int rc;
  if (dt == DT_F16)
    rc = A8 ? dispatch_j<DT_F16, true>(g, X, W, A8, AMAX, CODE2, offset, LUT, Y, R, epi, M, K, bs_shift, bs2_shift, st)
            : dispatch_j<DT_F16, false>(g, X, W, A8, AMAX, CODE2, offset, LUT, Y, R, epi, M, K, bs_shift, bs2_shift, st);
  else if (dt == DT_BF16)
    rc = A8 ? dispatch_j<DT_BF16, true>(g, X, W, A8, AMAX, CODE2, offset, LUT, Y, R, epi, M, K, bs_shift, bs2_shift, st)
            : dispatch_j<DT_BF16, false>(g, X, W, A8, AMAX, CODE2, offset, LUT, Y, R, epi, M, K, bs_shift, bs2_shift, st);
  else
    return (int)hipErrorInvalidValue;
  if (rc) return rc;
  TTSP_RETURN_LAUNCH();
}

}  // namespace ttsp

using namespace ttsp;

extern "C" int ttsp_gemv_shape(int M, int K, int* J, int* KS, int* RPW) {
  const GemvShape g = gemv_shape(M, K);
  if (J) *J = g.J;
  if (KS) *KS = g.KS;
  if (RPW) *RPW = g.RPW;
  return g.J ? 0 : (int)hipErrorInvalidValue;
}

extern "C" int ttsp_nf4_dequant(const uint8_t* W, const uint8_t* A8, const float* AMAX,
                                const float* CODE2, float offset, const float* LUT, void* out,
                                int out_dtype, long long n, int blocksize, int blocksize2,
                                hipStream_t stream) {
  const int bs_shift = log2_exact(blocksize);
  const int bs2_shift = A8 ? log2_exact(blocksize2) : 0;
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
