// NF4 GEMV (one activation row) and NF4 dequantisation, reading the
// bitsandbytes layout in place:
//   * W is the row-major flattened weight, two 4-bit codes per byte, the HIGH
//     nibble holding the even flattened index (byte j = q[2j] << 4 | q[2j+1]);
//   * scale block b covers flattened codes [b*bs, (b+1)*bs), bs a power of two
//     >= 64, so with K % bs == 0 a block never straddles a row;
//   * plain scales are fp32 absmax[b]; nested ("double-quant") scales are
//     code2[a8[b]] * absmax2[b >> log2(bs2)] + offset, two fp32 roundings.
//
// GEMV design. At batch 1 every weight byte is used once, so the kernel is a
// stream of W from HBM, and at decode shapes (1-25 MB) it is short enough that
// launch ramp and the per-byte instruction count, not the bus, set its time.
// Hence:
//   * Ownership. A row is K/8 dwords (8 codes each). Lane l of a wave owns
//     dwords d = l + 64*(j*KS + ks) of every row the wave visits: each load
//     instruction reads 256 contiguous bytes, and the 8 activations matching a
//     dword stay in registers for all of the wave's rows (x is read once per
//     wave, not once per row). KS waves split K; each wave takes RPW rows.
//   * Issue order. Everything small (code table, code2, the workgroup's
//     scales, the residual operand, x) is requested before the weights, so
//     waiting for it never waits for the weight stream (vector-memory counters
//     retire in order), and all RPW*J weight dwords of a lane are in flight
//     before the first barrier. The dot products start as rows arrive.
//   * Code lookup without bank conflicts. Each byte (two codes) becomes a
//     packed pair of fp16 code values through a 256-entry table that is
//     replicated 64 times in LDS, entry e of lane l at byte 256*e + 4*l: the 64
//     lanes of a lookup always hit 64 different banks, and the address is one
//     v_perm_b32 (the byte of W next to the lane's own offset). The 64 KiB
//     table is built while the weights are in flight.
//   * Arithmetic (fixed order, so a CPU restatement reproduces every bit): a
//     dword's 8 products are chained in code order (v_fma_mix_f32 on fp16
//     halves, the first onto +0), the dword's partial meets its block scale in
//     one fma into the lane accumulator - the scale multiplies the block's
//     partial sum, the factored form of the reference CPU kernel
//     (app/engine/nf4cpu.py:115-129). bf16 activations are first rescaled per
//     K-slice by a power of two and converted to fp16 exactly, so both
//     activation types meet 11-bit codes.
//   * Reductions: lanes by a DPP butterfly inside each 16-lane row (the xor
//     1, 2, 4, 8 tree: quad_perm, then half-mirror and mirror pair the same
//     partial sums) and the four row sums as (r0 + r1) + (r2 + r3); K-slices
//     left to right through LDS. No atomics anywhere.
#include "ttsp_common.h"

namespace ttsp {

constexpr int LUT_REP = 64;                    // table copies, one per lane
constexpr int LUT_BYTES = 256 * LUT_REP * 4;   // 64 KiB
constexpr int GEMV_WAVES = 8;                  // waves per workgroup
constexpr int GEMV_MAX_WAVES = GEMV_WAVES;

// Packed fp16 code pair of table entry v: low half code[v >> 4] (the even
// flattened index), high half code[v & 15], matching the activation pair
// (x[2i], x[2i+1]) of a 32-bit x word.
__device__ __forceinline__ uint32_t code_pair(float hi_code, float lo_code) {
  return (uint32_t)Elem<DT_F16>::store(hi_code) | ((uint32_t)Elem<DT_F16>::store(lo_code) << 16);
}

// Output rounding as the unfused fork: the matmul result is rounded to the
// activation type, and so is each elementwise op after it (app/engine/
// nf4gemv.py:215-226): residual y' = round(R + y), gate y' = round(round(silu(R)) * y).
template <int DT>
__device__ __forceinline__ uint16_t epilogue16(float acc, int epi, uint32_t r) {
  const float y = Elem<DT>::load(Elem<DT>::store(acc));
  float o = y;
  if (epi == 1) {
    o = __fadd_rn(Elem<DT>::load(r), y);
  } else if (epi == 2) {
    o = __fmul_rn(Elem<DT>::load(Elem<DT>::store(silu_rn(Elem<DT>::load(r)))), y);
  }
  return Elem<DT>::store(o);
}

// Every lane of a 16-lane row gets the row's sum, by the xor 1, 2, 4, 8
// butterfly tree (each step adds a partner's value; fp add is commutative, so
// the mirrored partners of steps 3 and 4 give the same bits as xor 4 and 8).
__device__ __forceinline__ float row16_sum(float v) {
  v = __fadd_rn(v, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0xB1, 0xF, 0xF, false)));
  v = __fadd_rn(v, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x4E, 0xF, 0xF, false)));
  v = __fadd_rn(v, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x141, 0xF, 0xF, false)));
  v = __fadd_rn(v, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x140, 0xF, 0xF, false)));
  return v;
}

// Sum over the wave: the butterfly's xor 16 and 32 steps on the row sums.
// The result is wave-uniform.
__device__ __forceinline__ float wave_sum_dpp(float v) {
  v = row16_sum(v);
  const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
  const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
  const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
  const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
  return __fadd_rn(__fadd_rn(r0, r1), __fadd_rn(r2, r3));
}

// Largest wave-uniform value helpers: readfirstlane makes a per-wave value a
// scalar, so row and slice offsets fold into scalar address arithmetic.
__device__ __forceinline__ int uniform(int v) { return __builtin_amdgcn_readfirstlane(v); }

// Max over the wave (every lane gets it): DPP within rows, then the 4 rows.
__device__ __forceinline__ float wave_max_dpp(float v) {
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0xB1, 0xF, 0xF, false)));
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x4E, 0xF, 0xF, false)));
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x141, 0xF, 0xF, false)));
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x140, 0xF, 0xF, false)));
  const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
  const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
  const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
  const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
  return fmaxf(fmaxf(r0, r1), fmaxf(r2, r3));
}

// bf16 pair -> fp16 pair of the same values times 2^-xe (exact for the range
// the rescale targets; below fp16's normal range the RNE conversion rounds).
__device__ __forceinline__ uint32_t bf16x2_to_f16x2(uint32_t u, int xe) {
  const uint32_t lo = f32_to_f16(__builtin_ldexpf(__uint_as_float(u << 16), -xe));
  const uint32_t hi = f32_to_f16(__builtin_ldexpf(__uint_as_float(u & 0xffff0000u), -xe));
  return lo | (hi << 16);
}

constexpr int XC_MAX = 8;  // bf16 x: 16-byte chunks a thread converts (K <= 8 * 8 * threads)

// Workgroup: 8 waves = KS * RG; wave w takes K-slice w % KS of RPW
// consecutive rows starting at blockIdx.x * RG * RPW + (w / KS) * RPW.
// LDS: the static code-pair table replicas at address 0 (so a lookup address
// is the v_perm result itself), then (dynamic) pair staging [256], code2
// [256], per-wave maxima [NW], per-wave K-slice partials [NW][RPW], the
// workgroup's scales [RG * RPW][nblk], and for bf16 the rescaled x [K] (fp16).
template <int DT, int J, int RPW, bool NESTED>
__global__ __launch_bounds__(GEMV_MAX_WAVES * 64) void nf4_gemv_kernel(
    const uint32_t* __restrict__ W, const uint8_t* __restrict__ A8,
    const float* __restrict__ AMAX, const float* __restrict__ CODE2, float offset,
    const float* __restrict__ LUT, const uint16_t* __restrict__ X, uint16_t* __restrict__ Y,
    const uint16_t* R, int epi, int M, int K, int KS, int bs_shift, int bs2_shift) {
  // Scale entries per thread: a workgroup holds (8 / KS) * RPW rows of at
  // most 8 * J * KS blocks (bs >= 64), i.e. <= 64 * RPW * J entries.
  constexpr int SL = (RPW * J + 7) / 8;
  constexpr int NW = GEMV_WAVES;
  constexpr int nthr = NW * 64;
  __shared__ __align__(16) uint32_t lut_rep[256 * LUT_REP];
  extern __shared__ __align__(16) unsigned char lds_dyn[];
  uint32_t* pair_s = reinterpret_cast<uint32_t*>(lds_dyn);
  float* code2_s = reinterpret_cast<float*>(pair_s + 256);
  float* wmax = code2_s + 256;                      // [NW]
  float* red = wmax + GEMV_MAX_WAVES;               // [NW][RPW]
  float* srow = red + GEMV_MAX_WAVES * RPW;         // [RG * RPW][nblk]
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = uniform(tid >> 6);
  const int ks = wave % KS, rg = wave / KS;
  const int RG = NW / KS;
  const int KD = K >> 3;
  const int nblk = K >> bs_shift;
  const int sh = bs_shift - 3;
  const int rows_wg = RG * RPW;
  const int wg_row0 = blockIdx.x * rows_wg;
  const int row0 = wg_row0 + rg * RPW;
  const int nsc = min(rows_wg, M - wg_row0) * nblk;  // scale entries of this workgroup
  const long long sc0 = (long long)wg_row0 * nblk;
  uint4* xs = reinterpret_cast<uint4*>(srow + ((rows_wg * nblk + 3) & ~3));  // bf16 only: [KD]

  // 1. small operands first: code table entries, code2, scales, residual, x
  float chi = 0.0f, clo = 0.0f, c2v = 0.0f;
  if (tid < 256) {
    chi = LUT[tid >> 4];
    clo = LUT[tid & 15];
    if constexpr (NESTED) c2v = CODE2[tid];
  }
  float sv[SL];
  uint32_t av[NESTED ? SL : 1];
#pragma unroll
  for (int i = 0; i < SL; ++i) {
    const long long gb = sc0 + min(tid + i * nthr, nsc - 1);
    if constexpr (NESTED) {
      av[i] = A8[gb];
      sv[i] = AMAX[gb >> bs2_shift];
    } else {
      sv[i] = AMAX[gb];
    }
  }
  const uint32_t rres = R[min(row0 + min(lane, RPW - 1), M - 1)];  // used by the epilogue only
  uint4 xr[J];
  uint4 xc[DT == DT_BF16 ? XC_MAX : 1];
  const int XN = (KD + nthr - 1) / nthr;  // bf16: x chunks per thread (uniform)
  if constexpr (DT == DT_BF16) {
#pragma unroll
    for (int i = 0; i < XC_MAX; ++i) {
      xc[i] = make_uint4(0, 0, 0, 0);
      if (i < XN) xc[i] = *reinterpret_cast<const uint4*>(X + 8 * (size_t)min(tid + i * nthr, KD - 1));
    }
  } else {
#pragma unroll
    for (int j = 0; j < J; ++j)
      xr[j] = *reinterpret_cast<const uint4*>(X + 8 * (size_t)min(lane + 64 * (j * KS + ks), KD - 1));
  }
  // 2. the weight stream: every dword of this wave's rows, all in flight
  uint32_t w[RPW][J];
#pragma unroll
  for (int r = 0; r < RPW; ++r) {
    const uint32_t* wr = W + (size_t)min(row0 + r, M - 1) * KD + 64 * ks;
#pragma unroll
    for (int j = 0; j < J; ++j)
      w[r][j] = __builtin_nontemporal_load(wr + min(64 * j * KS + lane, KD - 1 - 64 * ks));
  }


  // 3. tables: pair staging, code2 and the x maximum, then the replicated pair
  //    table, the resolved scales and the rescaled x
  if (tid < 256) {
    pair_s[tid] = code_pair(chi, clo);
    if constexpr (NESTED) code2_s[tid] = c2v;
  }
  if constexpr (DT == DT_BF16) {
    float m = 0.0f;
#pragma unroll
    for (int i = 0; i < XC_MAX; ++i) {
      if (i < XN) {
        const uint32_t u[4] = {xc[i].x, xc[i].y, xc[i].z, xc[i].w};
#pragma unroll
        for (int k = 0; k < 4; ++k)
          m = fmaxf(m, fmaxf(fabsf(bf16_to_f32(u[k] & 0xffffu)), fabsf(bf16_to_f32(u[k] >> 16))));
      }
    }
    m = wave_max_dpp(m);
    if (lane == 0) wmax[wave] = m;
  }
  __syncthreads();
  {
    constexpr int G = (int)sizeof(lut_rep) / 1024 / NW;  // 1 KiB (4 entries) per wave store
    uint32_t v[G];
#pragma unroll
    for (int i = 0; i < G; ++i) v[i] = pair_s[4 * (wave + NW * i) + (lane >> 4)];
#pragma unroll
    for (int i = 0; i < G; ++i)
      reinterpret_cast<uint4*>(lut_rep)[(wave + NW * i) * 64 + lane] = make_uint4(v[i], v[i], v[i], v[i]);
  }
#pragma unroll
  for (int i = 0; i < SL; ++i) {
    const int e = tid + i * nthr;
    if (e < nsc) {
      if constexpr (NESTED) srow[e] = __fadd_rn(__fmul_rn(code2_s[av[i]], sv[i]), offset);
      else srow[e] = sv[i];
    }
  }
  // bf16 activations: rescale x by 2^-xe so max|x| lands in [2^14, 2^15) and
  // convert to fp16 - exact, since bf16's 8 significant bits fit in fp16's 11 -
  // then every product below is fp16 x fp16 with 11-bit codes. The row sums
  // are scaled back by 2^xe (also exact).
  int xe = 0;
  if constexpr (DT == DT_BF16) {
    float m = wmax[0];
    for (int v = 1; v < NW; ++v) m = fmaxf(m, wmax[v]);
    if (m > 0.0f && m <= 3.402823466e38f) xe = __builtin_amdgcn_frexp_expf(m) - 15;
#pragma unroll
    for (int i = 0; i < XC_MAX; ++i) {
      const int c = tid + i * nthr;
      if (i < XN && c < KD)
        xs[c] = make_uint4(bf16x2_to_f16x2(xc[i].x, xe), bf16x2_to_f16x2(xc[i].y, xe),
                           bf16x2_to_f16x2(xc[i].z, xe), bf16x2_to_f16x2(xc[i].w, xe));
    }
  }
  __syncthreads();
  if constexpr (DT == DT_BF16) {
#pragma unroll
    for (int j = 0; j < J; ++j) xr[j] = xs[min(lane + 64 * (j * KS + ks), KD - 1)];
  }
  // Past the row's end (K not a multiple of 512 * KS) x is zero: the clamped
  // weight dword there is finite, so its products are exactly +0. (Only x is
  // zeroed - the weight registers may still be in flight.)
#pragma unroll
  for (int j = 0; j < J; ++j) {
    const bool in_row = lane + 64 * (j * KS + ks) < KD;
    xr[j] = make_uint4(in_row ? xr[j].x : 0u, in_row ? xr[j].y : 0u, in_row ? xr[j].z : 0u,
                       in_row ? xr[j].w : 0u);
  }

  // 4. dot products, row by row as the rows arrive
  const uint32_t lane4 = (uint32_t)lane * 4u;
  const unsigned char* lut_b = reinterpret_cast<const unsigned char*>(lut_rep);
  // block index of each of the lane's dwords (clamped inside the row past its end)
  int sblk[J];
#pragma unroll
  for (int j = 0; j < J; ++j) sblk[j] = min(lane + 64 * (j * KS + ks), KD - 1) >> sh;
  float tot[RPW];
#pragma unroll
  for (int r = 0; r < RPW; ++r) {
    const float* srr = srow + uniform((rg * RPW + r) * nblk);
    float acc = 0.0f;
#pragma unroll
    for (int j = 0; j < J; ++j) {
      const float s = srr[sblk[j]];
      const uint32_t wv = w[r][j];
      const uint32_t c0 = *reinterpret_cast<const uint32_t*>(lut_b + __builtin_amdgcn_perm(wv, lane4, 0x0C0C0400u));
      const uint32_t c1 = *reinterpret_cast<const uint32_t*>(lut_b + __builtin_amdgcn_perm(wv, lane4, 0x0C0C0500u));
      const uint32_t c2 = *reinterpret_cast<const uint32_t*>(lut_b + __builtin_amdgcn_perm(wv, lane4, 0x0C0C0600u));
      const uint32_t c3 = *reinterpret_cast<const uint32_t*>(lut_b + __builtin_amdgcn_perm(wv, lane4, 0x0C0C0700u));
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
    acc = wave_sum_dpp(acc);
    if constexpr (DT == DT_BF16) acc = __builtin_ldexpf(acc, xe);
    tot[r] = acc;
  }

  // 5. K-slices left to right, epilogue, store (lane r stores row r)
  if (KS > 1) {
    if (lane == 0) {
#pragma unroll
      for (int r = 0; r < RPW; ++r) red[wave * RPW + r] = tot[r];
    }
    __syncthreads();
    if (ks != 0) return;
#pragma unroll
    for (int r = 0; r < RPW; ++r) {
      float a = tot[r];
      for (int k2 = 1; k2 < KS; ++k2) a = __fadd_rn(a, red[(wave + k2) * RPW + r]);
      tot[r] = a;
    }
  }
  float mine = tot[0];
#pragma unroll
  for (int r = 1; r < RPW; ++r) mine = lane == r ? tot[r] : mine;
  if (lane < RPW && row0 + lane < M) Y[row0 + lane] = epilogue16<DT>(mine, epi, rres);
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

// Launch shape of the N == 1 GEMV for [M, K]: J 64-dword chunks per lane, K
// split over KS waves, RPW rows per wave, NW waves per workgroup.
struct GemvShape {
  int J, KS, RPW, NW;
};

static constexpr int kJ[] = {1, 2, 3, 4, 5, 6, 8};
static constexpr int kRPW[] = {1, 2, 3, 4, 5, 6, 8};
static constexpr int kCUs = 256;
static constexpr size_t kLdsPerCU = 160 * 1024;

// Dynamic LDS of one workgroup (the table is static).
static size_t gemv_dyn_lds(const GemvShape& g, int dt, int K, int bs_shift) {
  const size_t rows_wg = (size_t)(g.NW / g.KS) * g.RPW;
  const size_t sc = (rows_wg * (K >> bs_shift) + 3) & ~(size_t)3;
  return 4 * (256 + 256 + GEMV_MAX_WAVES + (size_t)GEMV_MAX_WAVES * g.RPW + sc) +
         (dt == DT_BF16 ? 2 * (size_t)K : 0);
}

// K is split (KS a power of two) so that a lane's chunks J <= 8 leave the
// fewest slots idle; workgroups are 8 waves wide, because every workgroup
// builds the 64 KiB table and converts x once; and RPW is the
// smallest that fits every row into one pass of the workgroups the LDS lets
// each CU hold.
static GemvShape gemv_shape(int M, int K, int dt = DT_F16, int bs_shift = 6) {
  const int chunks = (K / 8 + 63) / 64;  // 64-dword chunks per row
  int KS = 0, J = 0, waste = 1 << 30;
  for (int ks = 1; ks <= GEMV_WAVES; ks *= 2) {
    int j = 0;
    for (int v : kJ)
      if (v >= (chunks + ks - 1) / ks) { j = v; break; }
    if (j && ks * j - chunks < waste) { KS = ks; J = j; waste = ks * j - chunks; }
  }
  if (!KS) return {0, 0, 0, 0};
  const int NW = GEMV_WAVES;
  const int RG = NW / KS;
  GemvShape g{J, KS, kRPW[0], NW};
  for (int v : kRPW) {
    g.RPW = v;
    const size_t per_wg = LUT_BYTES + gemv_dyn_lds(g, dt, K, bs_shift);
    const long long slots = (long long)kCUs * (long long)(kLdsPerCU / per_wg);
    if ((long long)(M + RG * v - 1) / (RG * v) <= slots) break;
  }
  return g;
}

template <int DT, int J, int RPW, bool NESTED>
static void launch_gemv(const GemvShape& g, const void* X, const uint8_t* W, const uint8_t* A8,
                        const float* AMAX, const float* CODE2, float offset, const float* LUT,
                        void* Y, const void* R, int epi, int M, int K, int bs_shift, int bs2_shift,
                        hipStream_t st) {
  const int RG = g.NW / g.KS;
  const int rows_wg = RG * RPW;
  const int grid = (M + rows_wg - 1) / rows_wg;
  const size_t shmem = gemv_dyn_lds(g, DT, K, bs_shift);
  hipLaunchKernelGGL((nf4_gemv_kernel<DT, J, RPW, NESTED>), dim3(grid), dim3(64 * g.NW), shmem, st,
                     (const uint32_t*)W, A8, AMAX, CODE2, offset, LUT, (const uint16_t*)X,
                     (uint16_t*)Y, (const uint16_t*)R, epi, M, K, g.KS, bs_shift, bs2_shift);
}

template <int DT, int J, bool NESTED>
static int dispatch_rpw(const GemvShape& g, const void* X, const uint8_t* W, const uint8_t* A8,
                        const float* AMAX, const float* CODE2, float offset, const float* LUT,
                        void* Y, const void* R, int epi, int M, int K, int bs_shift, int bs2_shift,
                        hipStream_t st) {
#define TTSP_R(RV)                                                                                   \
  case RV:                                                                                           \
    launch_gemv<DT, J, RV, NESTED>(g, X, W, A8, AMAX, CODE2, offset, LUT, Y, R, epi, M, K, bs_shift, \
                                   bs2_shift, st);                                                   \
    return 0;
  switch (g.RPW) {
    TTSP_R(1) TTSP_R(2) TTSP_R(3) TTSP_R(4) TTSP_R(5) TTSP_R(6) TTSP_R(8)
    default: return (int)hipErrorInvalidValue;
  }
#undef TTSP_R
}

template <int DT, bool NESTED>
static int dispatch_j(const GemvShape& g, const void* X, const uint8_t* W, const uint8_t* A8,
                      const float* AMAX, const float* CODE2, float offset, const float* LUT,
                      void* Y, const void* R, int epi, int M, int K, int bs_shift, int bs2_shift,
                      hipStream_t st) {
#define TTSP_J(JV)                                                                                 \
  case JV:                                                                                         \
    return dispatch_rpw<DT, JV, NESTED>(g, X, W, A8, AMAX, CODE2, offset, LUT, Y, R, epi, M, K,   \
                                        bs_shift, bs2_shift, st);
  switch (g.J) {
    TTSP_J(1) TTSP_J(2) TTSP_J(3) TTSP_J(4) TTSP_J(5) TTSP_J(6) TTSP_J(8)
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
  if (!epi) R = Y;  // the kernel reads R unconditionally (an M-element buffer); unused without an epilogue
  const GemvShape g = gemv_shape(M, K, dt, bs_shift);
  if (!g.J || g.KS > GEMV_MAX_WAVES) return (int)hipErrorInvalidValue;
  // the workgroup's scales (and bf16 x) must fit next to the table
  if (LUT_BYTES + gemv_dyn_lds(g, dt, K, bs_shift) > 160 * 1024) return (int)hipErrorInvalidValue;
  if (dt == DT_BF16 && (K / 8 + 64 * g.NW - 1) / (64 * g.NW) > XC_MAX) return (int)hipErrorInvalidValue;
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
