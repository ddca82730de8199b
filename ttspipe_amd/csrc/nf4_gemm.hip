// NF4 GEMM for several activation rows (prompt prefill): Y[N][M] = X[N][K] . W^T
// with W the bitsandbytes NF4 weight (nf4_gemv.hip gives the layout).
//
// Each workgroup owns a BM x BN tile of the output (BM weight rows, BN input
// rows), WM x WN waves of 32x32 MFMA blocks. Per K-step of 64 codes, the
// workgroup's threads
//   * dequantise BM x 64 weights, 8 packed bytes (16 codes) each, as
//     round(code * scale) in the activation type - the exact value
//     bitsandbytes' dequantize_4bit produces, so the product is the dense
//     fork's matmul on identical weights - straight into an LDS A tile (the
//     16 code points in LDS: 64 lanes hit at most 16 banks, no conflicts; one
//     hardware pack-convert rounds two products);
//   * copy BN x 64 activations into an LDS B tile;
// and the waves run v_mfma_f32_32x32x16 over their sub-tiles, fp32
// accumulate. The packed weights, scales and activations of the next PF
// steps are in flight in registers while a step multiplies (the K loop is
// latency-bound otherwise: a lone workgroup waits a memory round trip per
// step), and LDS is double-buffered. Rows are padded to 72 elements (144 B) so
// the 16-byte operand reads of 16 consecutive rows hit disjoint banks. The
// output tile is rounded, staged in LDS and written (with the epilogue) as
// 16-byte row pieces.
//
// MFMA 32x32x16 operand layout: lane l supplies row (l % 32) of A and column
// (l % 32) of B, each as 8 consecutive k at 8 * (l / 32); accumulator r of
// lane l is D[8*(r/4) + 4*(l/32) + r%4][l % 32]. A and B only need to agree on
// which k a lane carries, so any k permutation inside a step is harmless.
#include "gemv_common.h"

namespace ttsp {

typedef __bf16 bf16x8_v __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_v __attribute__((ext_vector_type(8)));
typedef float f32x16_v __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x2_v __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2_v __attribute__((ext_vector_type(2)));
typedef float f32x2_v __attribute__((ext_vector_type(2)));

constexpr int KT = 64;        // codes per K-step (one bs=64 scale block)
constexpr int LROW = KT + 8;  // LDS row stride in elements

template <int DT>
__device__ __forceinline__ f32x16_v mfma32(uint4 a, uint4 b, f32x16_v c) {
  if constexpr (DT == DT_BF16)
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_v, a),
                                                   __builtin_bit_cast(bf16x8_v, b), c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8_v, a),
                                                  __builtin_bit_cast(f16x8_v, b), c, 0, 0, 0);
}

// Two fp32 values, each already rounded to fp32, to the activation type
// (round to nearest even, one hardware pack-convert); lo in the low half.
template <int DT>
__device__ __forceinline__ uint32_t pack2(float lo, float hi) {
  const f32x2_v v = {opaque(lo), opaque(hi)};
  if constexpr (DT == DT_BF16)
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_v));
  else
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, f16x2_v));
}

// WM x WN waves; each wave covers (BM/WM) x (BN/WN) with 32x32 MFMA blocks;
// PF K-steps of operands in flight (nsteps a multiple of PF).
template <int DT, int BM, int BN, int WM, int WN, bool NESTED, int PF>
__global__ __launch_bounds__(64 * WM * WN) void nf4_gemm_kernel(
    const uint16_t* __restrict__ X, const uint8_t* __restrict__ W, const uint8_t* __restrict__ A8,
    const float* __restrict__ AMAX, const float* __restrict__ CODE2, float offset,
    const float* __restrict__ LUT, uint16_t* __restrict__ Y, const uint16_t* __restrict__ R,
    int epi, int M, int K, int N, int bs_shift, int bs2_shift, float* __restrict__ YP) {
  constexpr int GEMM_THREADS = 64 * WM * WN;
  constexpr int TM = BM / WM / 32, TN = BN / WN / 32;  // MFMA blocks per wave
  constexpr int A_CH = BM * (KT / 16);                                  // 8-byte packed chunks (16 codes) per step
  constexpr int A_PER_T = (A_CH + GEMM_THREADS - 1) / GEMM_THREADS;     // per thread (the last partly idle)
  constexpr int B_PER_T = BN * (KT / 8) / GEMM_THREADS;                 // 16-byte activation chunks per thread
  static_assert(B_PER_T >= 1 && BN * (KT / 8) % GEMM_THREADS == 0, "tile too small for the workgroup");
  static_assert(GEMM_THREADS >= 256, "the code tables are filled one entry per thread");

  // the operand tiles (two buffers each); after the K loop the same memory
  // holds the output tile, BN rows of BM + 8 elements
  constexpr int YROW = BM + 8;
  constexpr int OPS = 2 * (BM + BN) * LROW, YS = BN * YROW;
  __shared__ __align__(16) uint16_t smem[OPS > YS ? OPS : YS];
  uint16_t (*As)[BM * LROW] = reinterpret_cast<uint16_t (*)[BM * LROW]>(smem);
  uint16_t (*Bs)[BN * LROW] = reinterpret_cast<uint16_t (*)[BN * LROW]>(smem + 2 * BM * LROW);
  __shared__ float2 lut2_s[256];  // byte -> (code of its high nibble, code of its low nibble)
  __shared__ float code2_s[NESTED ? 256 : 1];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;
  const int m0 = blockIdx.x * BM, n0 = blockIdx.y * BN;
  // split-K (gridDim.z > 1): workgroup z takes K-steps [z S, z S + S) and
  // writes its fp32 partial sums to YP[z][n][m]; a second kernel adds them
  const int nsteps = K / KT / gridDim.z, kbase = blockIdx.z * nsteps * KT;
  const size_t rowbytes = (size_t)K / 2;

  if (tid < 256) lut2_s[tid] = make_float2(LUT[tid >> 4], LUT[tid & 15]);
  if constexpr (NESTED)
    if (tid < 256) code2_s[tid] = CODE2[tid];

  struct Stage {
    uint2 w[A_PER_T];
    float s[A_PER_T];
    uint32_t a8[NESTED ? A_PER_T : 1];
    uint4 x[B_PER_T];
  };
  Stage stg[PF];

  // step clamped into range: the loads past the last step repeat it and go unused
  auto load_step = [&](Stage& sg, int step) {
    const int k0 = kbase + min(step, nsteps - 1) * KT;
#pragma unroll
    for (int i = 0; i < A_PER_T; ++i) {
      const int c = min(tid + i * GEMM_THREADS, A_CH - 1);  // chunk: row c / 4, codes 16 (c % 4) ..
      const int row = min(m0 + c / (KT / 16), M - 1);
      const int kc = k0 + (c % (KT / 16)) * 16;
      typedef uint32_t u32x2_v __attribute__((ext_vector_type(2)));
      const u32x2_v v = __builtin_nontemporal_load(
          reinterpret_cast<const u32x2_v*>(W + (size_t)row * rowbytes + kc / 2));
      sg.w[i] = make_uint2(v.x, v.y);
      const long long b = ((long long)row * K + kc) >> bs_shift;
      if constexpr (NESTED) {
        sg.a8[i] = A8[b];
        sg.s[i] = AMAX[b >> bs2_shift];
      } else {
        sg.s[i] = AMAX[b];
      }
    }
#pragma unroll
    for (int i = 0; i < B_PER_T; ++i) {
      const int c = tid + i * GEMM_THREADS;  // chunk: row c/8, 8 elements at (c%8)*8
      const int n = min(n0 + c / (KT / 8), N - 1);
      sg.x[i] = *reinterpret_cast<const uint4*>(X + (size_t)n * K + k0 + (c % (KT / 8)) * 8);
    }
  };
  auto store_step = [&](const Stage& sg, int buf) {
#pragma unroll
    for (int i = 0; i < A_PER_T; ++i) {
      const int c = tid + i * GEMM_THREADS;
      if (A_CH % GEMM_THREADS && c >= A_CH) break;
      float s = sg.s[i];
      if constexpr (NESTED) s = __fadd_rn(__fmul_rn(code2_s[sg.a8[i]], s), offset);
      const uint32_t wv[2] = {sg.w[i].x, sg.w[i].y};
      // one lookup per byte (both codes), all 8 in flight before the first
      // is used (one LDS round trip per step instead of one per byte)
      float cv[16];
#pragma unroll
      for (int q = 0; q < 2; ++q)
#pragma unroll
        for (int bb = 0; bb < 4; ++bb) {
          const float2 pc = lut2_s[(wv[q] >> (8 * bb)) & 0xffu];
          cv[2 * (q * 4 + bb)] = pc.x;
          cv[2 * (q * 4 + bb) + 1] = pc.y;
        }
      uint32_t o[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] = pack2<DT>(__fmul_rn(cv[2 * e], s), __fmul_rn(cv[2 * e + 1], s));
      uint4* dst = reinterpret_cast<uint4*>(&As[buf][(c / (KT / 16)) * LROW + (c % (KT / 16)) * 16]);
#pragma unroll
      for (int q = 0; q < 2; ++q) dst[q] = make_uint4(o[4 * q], o[4 * q + 1], o[4 * q + 2], o[4 * q + 3]);
    }
#pragma unroll
    for (int i = 0; i < B_PER_T; ++i) {
      const int c = tid + i * GEMM_THREADS;
      const int n = n0 + c / (KT / 8);
      *reinterpret_cast<uint4*>(&Bs[buf][(c / (KT / 8)) * LROW + (c % (KT / 8)) * 8]) =
          n < N ? sg.x[i] : make_uint4(0, 0, 0, 0);
    }
  };

  f32x16_v acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

#pragma unroll
  for (int i = 0; i < PF; ++i) load_step(stg[i], i);
  __syncthreads();  // lut2_s / code2_s
  store_step(stg[0], 0);
  __syncthreads();
  load_step(stg[0], PF);
  // Step s multiplies buffer s & 1 while the same waves dequantise step s + 1
  // into the other buffer (read by nobody since the previous barrier); one
  // barrier per step. The last step stages a repeat of itself, unread.
  for (int s0 = 0; s0 < nsteps; s0 += PF) {
#pragma unroll
    for (int i = 0; i < PF; ++i) {
      const int step = s0 + i;
      const int buf = step & 1;
      const uint16_t* as = As[buf];
      const uint16_t* bs = Bs[buf];
#pragma unroll
      for (int kk = 0; kk < KT / 16; ++kk) {
        const int ko = kk * 16 + (lane >> 5) * 8;
        uint4 af[TM], bf[TN];
#pragma unroll
        for (int a = 0; a < TM; ++a)
          af[a] = *reinterpret_cast<const uint4*>(as + (wm * (BM / WM) + a * 32 + (lane & 31)) * LROW + ko);
#pragma unroll
        for (int b = 0; b < TN; ++b)
          bf[b] = *reinterpret_cast<const uint4*>(bs + (wn * (BN / WN) + b * 32 + (lane & 31)) * LROW + ko);
#pragma unroll
        for (int a = 0; a < TM; ++a)
#pragma unroll
          for (int b = 0; b < TN; ++b) acc[a][b] = mfma32<DT>(af[a], bf[b], acc[a][b]);
      }
      store_step(stg[(i + 1) % PF], buf ^ 1);
      __syncthreads();
      load_step(stg[(i + 1) % PF], step + 1 + PF);
    }
  }

  if (YP) {  // split-K partials: 4 consecutive rows m per 16-byte store
    // (n * M + m is a multiple of 4 only when M is: m always is)
    float* yp = YP + (size_t)blockIdx.z * N * M;
    const bool v4 = (M & 3) == 0;
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const int n = n0 + wn * (BN / WN) + j * 32 + (lane & 31);
        if (n >= N) continue;
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int m = m0 + wm * (BM / WM) + i * 32 + 8 * g + 4 * (lane >> 5);
          if (v4 && m + 4 <= M) {
            *reinterpret_cast<float4*>(yp + (size_t)n * M + m) =
                make_float4(acc[i][j][4 * g], acc[i][j][4 * g + 1], acc[i][j][4 * g + 2], acc[i][j][4 * g + 3]);
          } else {
            for (int c = 0; c < 4 && m + c < M; ++c) yp[(size_t)n * M + m + c] = acc[i][j][4 * g + c];
          }
        }
      }
    return;
  }
  // epilogue: accumulator r of lane l is (row 8*(r/4) + 4*(l/32) + r%4, column
  // l%32); each value is rounded to the activation type and the tile goes
  // through LDS as Y rows (the operand buffers are free after the last
  // barrier), so the stores and the operand reads are 16 bytes per lane
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int nl = wn * (BN / WN) + j * 32 + (lane & 31);
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int ml = wm * (BM / WM) + i * 32 + 8 * g + 4 * (lane >> 5);
        const uint32_t lo = (uint32_t)Elem<DT>::store(acc[i][j][4 * g]) |
                            ((uint32_t)Elem<DT>::store(acc[i][j][4 * g + 1]) << 16);
        const uint32_t hi = (uint32_t)Elem<DT>::store(acc[i][j][4 * g + 2]) |
                            ((uint32_t)Elem<DT>::store(acc[i][j][4 * g + 3]) << 16);
        *reinterpret_cast<uint2*>(&smem[nl * YROW + ml]) = make_uint2(lo, hi);
      }
    }
  __syncthreads();
  const bool vec = (epi & 4) != 0;  // M % 8 == 0 and Y, R 16-byte aligned (host)
  const int ep = epi & 3;
  for (int cc = tid; cc < BN * (BM / 8); cc += GEMM_THREADS) {
    const int nl = cc / (BM / 8), ml = (cc % (BM / 8)) * 8;
    const int n = n0 + nl, m = m0 + ml;
    if (n >= N || m >= M) continue;
    const uint4 yv = *reinterpret_cast<const uint4*>(&smem[nl * YROW + ml]);
    const uint32_t yw[4] = {yv.x, yv.y, yv.z, yv.w};
    const size_t o = (size_t)n * M + m;
    if (vec && m + 8 <= M) {
      uint32_t rw[4] = {0u, 0u, 0u, 0u};
      if (ep) {
        const uint4 rv = *reinterpret_cast<const uint4*>(R + o);
        rw[0] = rv.x, rw[1] = rv.y, rw[2] = rv.z, rw[3] = rv.w;
      }
      uint32_t ow[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        uint32_t h2[2];
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          const float y = Elem<DT>::load(yw[q] >> (16 * u));
          const float r = Elem<DT>::load(rw[q] >> (16 * u));
          float v = y;
          if (ep == 1) v = __fadd_rn(r, y);
          else if (ep == 2) v = __fmul_rn(Elem<DT>::load(Elem<DT>::store(silu_rn(r))), y);
          h2[u] = Elem<DT>::store(v);
        }
        ow[q] = h2[0] | (h2[1] << 16);
      }
      *reinterpret_cast<uint4*>(Y + o) = make_uint4(ow[0], ow[1], ow[2], ow[3]);
    } else {
      for (int u = 0; u < 8 && m + u < M; ++u) {
        const float y = Elem<DT>::load(yw[u >> 1] >> (16 * (u & 1)));
        float v = y;
        if (ep == 1) v = __fadd_rn(Elem<DT>::load(R[o + u]), y);
        else if (ep == 2) v = __fmul_rn(Elem<DT>::load(Elem<DT>::store(silu_rn(Elem<DT>::load(R[o + u])))), y);
        Y[o + u] = Elem<DT>::store(v);
      }
    }
  }
}

// Y[n][m] = epilogue(round(sum over z of YP[z][n][m])), the sum in z order;
// 8 consecutive m per thread (16-byte stores when vec).
template <int DT>
__global__ __launch_bounds__(256) void nf4_gemm_reduce_kernel(const float* __restrict__ YP, int splits,
                                                              uint16_t* __restrict__ Y,
                                                              const uint16_t* __restrict__ R, int epi, int M,
                                                              int N) {
  const int chunks = (M + 7) / 8;
  const long long c = (long long)blockIdx.x * 256 + threadIdx.x;
  if (c >= (long long)chunks * N) return;
  const int n = (int)(c / chunks), m = (int)(c % chunks) * 8;
  const bool vec = (epi & 4) != 0;
  const int ep = epi & 3;
  const size_t o = (size_t)n * M + m;
  float acc[8];
  if (vec && m + 8 <= M) {
    const float4* p = reinterpret_cast<const float4*>(YP + o);
    float4 a = p[0], b = p[1];
    for (int z = 1; z < splits; ++z) {
      const float4* q = reinterpret_cast<const float4*>(YP + (size_t)z * N * M + o);
      const float4 u = q[0], v = q[1];
      a.x += u.x, a.y += u.y, a.z += u.z, a.w += u.w;
      b.x += v.x, b.y += v.y, b.z += v.z, b.w += v.w;
    }
    acc[0] = a.x, acc[1] = a.y, acc[2] = a.z, acc[3] = a.w, acc[4] = b.x, acc[5] = b.y, acc[6] = b.z, acc[7] = b.w;
    uint32_t rw[4] = {0u, 0u, 0u, 0u};
    if (ep) {
      const uint4 rv = *reinterpret_cast<const uint4*>(R + o);
      rw[0] = rv.x, rw[1] = rv.y, rw[2] = rv.z, rw[3] = rv.w;
    }
    uint32_t ow[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      uint32_t h2[2];
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const float y = Elem<DT>::load(Elem<DT>::store(acc[2 * q + u]));
        const float r = Elem<DT>::load(rw[q] >> (16 * u));
        float v = y;
        if (ep == 1) v = __fadd_rn(r, y);
        else if (ep == 2) v = __fmul_rn(Elem<DT>::load(Elem<DT>::store(silu_rn(r))), y);
        h2[u] = Elem<DT>::store(v);
      }
      ow[q] = h2[0] | (h2[1] << 16);
    }
    *reinterpret_cast<uint4*>(Y + o) = make_uint4(ow[0], ow[1], ow[2], ow[3]);
  } else {
    for (int u = 0; u < 8 && m + u < M; ++u) {
      float a = YP[o + u];
      for (int z = 1; z < splits; ++z) a += YP[(size_t)z * N * M + o + u];
      const float y = Elem<DT>::load(Elem<DT>::store(a));
      float v = y;
      if (ep == 1) v = __fadd_rn(Elem<DT>::load(R[o + u]), y);
      else if (ep == 2) v = __fmul_rn(Elem<DT>::load(Elem<DT>::store(silu_rn(Elem<DT>::load(R[o + u])))), y);
      Y[o + u] = Elem<DT>::store(v);
    }
  }
}

// The split-K reduce, its epilogue and the fork's RMSNorm of each output row
// in one launch: Y is nf4_gemm_reduce_kernel's output, YN = rms_norm(Y, G, eps)
// with rms_norm_kernel's order (chunk c of 8 values by lane c % 64 in step
// c / 64, each chunk an fma chain of squares, DPP sums, steps left to right).
// One workgroup per output row with a wave per step (64 * ceil(M / 512)
// threads, at most 8 waves): each wave issues all of its loads - the splits'
// partials, the residual and the norm weight - before using any, so the row
// costs one memory round trip; the step sums meet in LDS.
// M % 8 == 0, M <= 64 * 8 * NRM_CH.
constexpr int NRM_CH = 8;
template <int DT, int S>
__global__ __launch_bounds__(64 * NRM_CH) void nf4_gemm_reduce_norm_kernel(const float* __restrict__ YP,
                                                                          uint16_t* __restrict__ Y,
                                                                          const uint16_t* __restrict__ R, int epi,
                                                                          int M, int N,
                                                                          const uint16_t* __restrict__ G, float eps,
                                                                          uint16_t* __restrict__ YN) {
  __shared__ float step_sum[NRM_CH];
  const int lane = threadIdx.x & 63, j = threadIdx.x >> 6;  // this wave's step
  const int n = blockIdx.x;
  const int nc = M >> 3, ep = epi & 3, nsteps = (nc + 63) >> 6;
  const int c = min(lane + 64 * j, nc - 1);
  const size_t o = (size_t)n * M + 8 * (size_t)c;
  float4 p[S][2];
#pragma unroll
  for (int z = 0; z < S; ++z) {
    const float4* q = reinterpret_cast<const float4*>(YP + (size_t)z * N * M + o);
    p[z][0] = q[0];
    p[z][1] = q[1];
  }
  const uint4 rv = ep ? *reinterpret_cast<const uint4*>(R + o) : make_uint4(0, 0, 0, 0);
  const uint4 gv = *reinterpret_cast<const uint4*>(G + 8 * (size_t)c);
  const uint32_t rw[4] = {rv.x, rv.y, rv.z, rv.w};
  uint32_t ow[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    uint32_t h2[2];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int e = 2 * q + u;  // element of the chunk, in the reduce kernel's order
      float a = e < 4 ? (&p[0][0].x)[e] : (&p[0][1].x)[e - 4];
#pragma unroll
      for (int z = 1; z < S; ++z) a += e < 4 ? (&p[z][0].x)[e] : (&p[z][1].x)[e - 4];
      const float y = Elem<DT>::load(Elem<DT>::store(a));
      const float r = Elem<DT>::load(rw[q] >> (16 * u));
      float v = y;
      if (ep == 1) v = __fadd_rn(r, y);
      else if (ep == 2) v = __fmul_rn(Elem<DT>::load(Elem<DT>::store(silu_rn(r))), y);
      h2[u] = Elem<DT>::store(v);
    }
    ow[q] = h2[0] | (h2[1] << 16);
  }
  const uint4 h = make_uint4(ow[0], ow[1], ow[2], ow[3]);
  const bool own = lane + 64 * j < nc;
  if (own) *reinterpret_cast<uint4*>(Y + o) = h;
  const float part = wave_sum_dpp(own ? sumsq8<DT>(h, 0.0f) : 0.0f);
  if (lane == 0) step_sum[j] = part;
  __syncthreads();
  float ss = step_sum[0];
  for (int k = 1; k < nsteps; ++k) ss = __fadd_rn(ss, step_sum[k]);
  const float rr = rsqrt_rn(__fadd_rn(__fdiv_rn(ss, (float)M), eps));
  if (own) *reinterpret_cast<uint4*>(YN + o) = norm8<DT>(h, gv, rr);
}

template <int DT, int BM, int BN, int WM, int WN, int PF>
static void launch_gemm(const void* X, const uint8_t* W, const uint8_t* A8, const float* AMAX,
                        const float* CODE2, float offset, const float* LUT, void* Y, const void* R,
                        int epi, int M, int K, int N, int bs_shift, int bs2_shift, float* YP, int splits,
                        hipStream_t st) {
  const dim3 grid((M + BM - 1) / BM, (N + BN - 1) / BN, splits);
  if (A8)
    hipLaunchKernelGGL((nf4_gemm_kernel<DT, BM, BN, WM, WN, true, PF>), grid, dim3(64 * WM * WN), 0, st,
                       (const uint16_t*)X, W, A8, AMAX, CODE2, offset, LUT, (uint16_t*)Y,
                       (const uint16_t*)R, epi, M, K, N, bs_shift, bs2_shift, YP);
  else
    hipLaunchKernelGGL((nf4_gemm_kernel<DT, BM, BN, WM, WN, false, PF>), grid, dim3(64 * WM * WN), 0, st,
                       (const uint16_t*)X, W, A8, AMAX, CODE2, offset, LUT, (uint16_t*)Y,
                       (const uint16_t*)R, epi, M, K, N, bs_shift, bs2_shift, YP);
}

// Tile shape and K-split of a launch: 64 x 128 tiles (8 waves), unsplit when
// they give every CU a workgroup. Up to 128 tiles, the largest split (2, 4,
// 8; each split an even number of at least 8 K-steps) whose workgroups still
// fit one to a CU: a split's fp32 partial sums cost a write and a read of
// splits x N x M floats, so a second pass of workgroups only pays where each
// split keeps a long K run. Between 128 and 256 tiles no split fits one pass,
// and 4 splits pay only past 16 K-steps each. Unsplit launches take 64 x 128
// tiles down to 128 of them, 64 x 64 below. 33 to 64 rows take 64 x 64 tiles
// with a K split (below); up to SKINNY_MAX_N rows otherwise the skinny kernel
// (nf4_skinny.hip), shape 0, never split. Measured on the five
// projections of a 2560-wide layer (wqkv 6144 x 2560, wo 2560 x 4096, w1 and
// w3 9728 x 2560, w2 2560 x 9728): 187 -> 125 us at 128 rows against a rule
// that sought two workgroups a CU, 200 -> 184 us at 256 rows, equal at 512
// rows (where 64 x 128 beats 128 x 128 by 8-10 % at 9728 x 2560 and
// 2560 x 9728; unsplit tile shapes give identical bits).
struct GemmPlan {
  int shape, splits;
};
constexpr int SKINNY_MAX_N = 64;
int skinny_max_k(int N);
static bool skinny(int K, int N) { return N <= SKINNY_MAX_N && K <= skinny_max_k(N); }

static long long gemm_tiles(int M, int N, int bm, int bn) {
  return (long long)((M + bm - 1) / bm) * ((N + bn - 1) / bn);
}

static int unsplit_shape(int M, int N) { return gemm_tiles(M, N, 64, 128) >= 128 ? 2 : 3; }

// From 33 rows (where the skinny kernel's tiles double) a K split of 64 x 64
// tiles - one row tile covers every input row - beats the skinny kernel:
// 4 ways where each split keeps 8 or more K-steps, else 2. Measured at 33-64
// rows: 20-45 % faster on the five layer shapes (9728 x 2560 at 33 rows
// 20.4 against 26.0 us, 2560 x 9728 at 64 rows 25.9 against 45.6) and on
// the 1024-wide fast-transformer shapes (1024 x 3072 at 64 rows 13.1 against
// 25.2); at 28-32 rows the two tie over a layer, below that the skinny kernel
// wins (8 rows: 12.1 against 17.4 at 9728 x 2560). The unsplit entry has no
// workspace, and unsplit tiles lose to the skinny kernel there, so it keeps
// the skinny kernel up to SKINNY_MAX_N rows.
constexpr int SPLIT_SMALL_N = 32;

bool gemm_dl_fits(int M, int K, int N, int splits);
int gemm_dl(const void* X, int dt, const uint8_t* W, const uint8_t* A8, const float* AMAX, const float* CODE2,
            float offset, const float* LUT, void* Y, const void* R, int epi, int M, int K, int N, int bs_shift,
            int bs2_shift, int waves, int splits, float* YP, hipStream_t st);

// 256 to 512 rows: the direct-to-LDS kernel (nf4_gemm_dl.hip, shape 4, 64 x
// 128 tiles of 2 waves) with 4 K-splits where K has 64 or more steps and
// there are at least 75 tiles; with fewer steps unsplit from 512 tiles and
// with 2 splits from 300. Measured against the 64 x 128 kernel at its best
// split, 512 rows (bf16, nested scales): w1 / w3 9728 x 2560 71.5 -> 48.4 us,
// w2 2560 x 9728 70.1 -> 48.5, wo 2560 x 4096 40.7 -> 30.1, wqkv 6144 x 2560
// 46.6 -> 36.5; at 256 rows w1 45.8 -> 34.0, w2 48.0 -> 39.8. The 64 x 128
// kernel stays ahead or ties at 128 rows, at 4096 x 2560 and on the
// 1024-wide shapes.
constexpr int DL_MIN_N = 256, DL_MAX_N = 512;
static bool dl_plan(int M, int K, int N, GemmPlan* p) {
  if (N < DL_MIN_N || N > DL_MAX_N) return false;
  const int steps = K / KT;
  const long long t = gemm_tiles(M, N, 64, 128);
  if (steps >= 64) {
    if (t >= 75 && steps % 8 == 0 && gemm_dl_fits(M, K, N, 4)) return *p = GemmPlan{4, 4}, true;
    return false;
  }
  if (t >= 512 && gemm_dl_fits(M, K, N, 1)) return *p = GemmPlan{4, 1}, true;
  if (t >= 300 && steps % 4 == 0 && gemm_dl_fits(M, K, N, 2)) return *p = GemmPlan{4, 2}, true;
  return false;
}

static GemmPlan gemm_plan(int M, int K, int N) {
  const int steps = K / KT;
  if (N > SPLIT_SMALL_N && N <= 64)
    for (int sp = 4; sp >= 2; sp /= 2)
      if (steps % (2 * sp) == 0 && steps / sp >= 8) return {3, sp};
  if (skinny(K, N)) return {0, 1};
  GemmPlan dl;
  if (dl_plan(M, K, N, &dl)) return dl;
  const long long t = gemm_tiles(M, N, 64, 128);
  if (t >= 256) return {2, 1};
  int splits = 1;
  if (t > 128) {
    if (steps % 8 == 0 && steps / 4 > 16) splits = 4;
  } else {
    for (int sp = 2; sp <= 8; sp *= 2) {
      if (steps % (2 * sp) || steps / sp < 8 || t * sp > 256) break;
      splits = sp;
    }
  }
  return splits > 1 ? GemmPlan{2, splits} : GemmPlan{unsplit_shape(M, N), 1};
}

int gemm_mfma(const void* X, int dt, const uint8_t* W, const uint8_t* A8, const float* AMAX,
              const float* CODE2, float offset, const float* LUT, void* Y, const void* R, int epi,
              int M, int K, int N, int bs_shift, int bs2_shift, const GemmPlan& plan, float* YP,
              hipStream_t st, bool reduce = true) {
  if (K % (2 * KT)) return (int)hipErrorInvalidValue;
  const int splits = plan.splits;
  if (splits > 1 && (!YP || (K / KT) % (2 * splits))) return (int)hipErrorInvalidValue;
  float* yp = splits > 1 ? YP : nullptr;
  const bool pf4 = (K / KT / splits) % 4 == 0;
#define TTSP_G(DTV, BMV, BNV, WMV, WNV)                                                                     \
  (pf4 ? launch_gemm<DTV, BMV, BNV, WMV, WNV, 4>(X, W, A8, AMAX, CODE2, offset, LUT, Y, R, epi, M, K, N,    \
                                                 bs_shift, bs2_shift, yp, splits, st)                       \
       : launch_gemm<DTV, BMV, BNV, WMV, WNV, 2>(X, W, A8, AMAX, CODE2, offset, LUT, Y, R, epi, M, K, N,    \
                                                 bs_shift, bs2_shift, yp, splits, st))
  // 8 waves for the 64 x 128 tiles (two a SIMD: one wave's dequantisation
  // runs while the other's matrix products do), 4 for 64 x 64
  // The direct-to-LDS kernel resolves nested scales with at most one
  // second-level group boundary inside a workgroup's K range (true for
  // bitsandbytes' blocksize2 of 256); smaller groups take the 64 x 128
  // kernel with the same split.
  int shape = plan.shape;
  if (shape == 4 && A8 && (long long)(K / splits) > (1LL << (bs_shift + bs2_shift))) shape = 2;
  if (shape == 4) {
    if (int rc = gemm_dl(X, dt, W, A8, AMAX, CODE2, offset, LUT, Y, R, epi, M, K, N, bs_shift, bs2_shift, 2,
                         splits, yp, st))
      return rc;
  } else if (dt == DT_BF16) {
    if (shape == 2) TTSP_G(DT_BF16, 64, 128, 2, 4);
    else TTSP_G(DT_BF16, 64, 64, 2, 2);
  } else if (dt == DT_F16) {
    if (shape == 2) TTSP_G(DT_F16, 64, 128, 2, 4);
    else TTSP_G(DT_F16, 64, 64, 2, 2);
  } else {
    return (int)hipErrorInvalidValue;
  }
#undef TTSP_G
  if (splits > 1 && reduce) {
    const long long chunks = (long long)((M + 7) / 8) * N;
    const dim3 rg((unsigned)((chunks + 255) / 256));
    if (dt == DT_BF16)
      hipLaunchKernelGGL(nf4_gemm_reduce_kernel<DT_BF16>, rg, dim3(256), 0, st, YP, splits, (uint16_t*)Y,
                         (const uint16_t*)R, epi, M, N);
    else
      hipLaunchKernelGGL(nf4_gemm_reduce_kernel<DT_F16>, rg, dim3(256), 0, st, YP, splits, (uint16_t*)Y,
                         (const uint16_t*)R, epi, M, N);
  }
  TTSP_RETURN_LAUNCH();
}

bool gemv_fits(int M, int K, int blocksize, int N);
int gemv_rows(const void* X, int dt, const uint8_t* W, const uint8_t* A8, const float* AMAX,
              const float* CODE2, float offset, const float* LUT, void* Y, const void* R, int epi,
              int M, int K, int N, int blocksize, int blocksize2, hipStream_t st);
// Up to this many activation rows take the GEMV (each weight byte looked up
// once, one fp32 chain per row) rather than the few-row MFMA kernel: two rows
// cost 1.0-1.3x one row that way (gate 9728 x 2560: 7.5 against 9.4 us).
constexpr int GEMV_ROWS_N = 2;
int gemm_skinny(const void* X, int dt, const uint8_t* W, const uint8_t* A8, const float* AMAX, const float* CODE2,
                float offset, const float* LUT, void* Y, const void* RES, int epi, int M, int K, int N, int bs_shift,
                int bs2_shift, hipStream_t st);
int gemm_dl_swiglu(const void* X, int dt, const uint8_t* W1, const uint8_t* A8_1, const float* AMAX_1,
                   const float* CODE2_1, float offset_1, const uint8_t* W3, const uint8_t* A8_3,
                   const float* AMAX_3, const float* CODE2_3, float offset_3, const float* LUT, void* Y, int M, int K,
                   int N, int bs_shift, int bs2_shift, hipStream_t st);
int gemm_skinny_pair(const void* X, int dt, const uint8_t* W1, const uint8_t* A8_1, const float* AMAX_1,
                     const float* CODE2_1, float offset_1, const uint8_t* W3, const uint8_t* A8_3, const float* AMAX_3,
                     const float* CODE2_3, float offset_3, const float* LUT, void* Y, int M, int K, int N, int bs_shift,
                     int bs2_shift, hipStream_t st);
bool skinny_pair_fits(int K, int N);

// Whether the SwiGLU pair takes the skinny kernel's pair form: where each of
// its two GEMMs would run the skinny kernel (3 to 32 rows, unsplit; two rows
// take the GEMV, whose one-launch pair is ttsp_nf4_gemv_fused_rows).
static bool swiglu_skinny(int M, int K, int N) {
  if (M <= 0 || K <= 0 || K % 128 || N <= GEMV_ROWS_N || !skinny_pair_fits(K, N)) return false;
  const GemmPlan p = gemm_plan(M, K, N);
  return p.shape == 0 && p.splits == 1;
}

// Whether the SwiGLU pair fits one launch of the direct-to-LDS kernel: where
// each of its two GEMMs would run that kernel unsplit (so the one launch
// gives their bits).
static bool swiglu_fits(int M, int K, int N, int bs_shift, int bs2_shift, bool nested) {
  if (M <= 0 || K <= 0 || K % 128 || N <= SKINNY_MAX_N) return false;
  GemmPlan dl;
  if (!dl_plan(M, K, N, &dl) || dl.splits != 1 || dl.shape != 4) return false;
  // the plan's fallback to 64 x 128 tiles for small second-level groups
  return !(nested && (long long)K > (1LL << (bs_shift + bs2_shift)));
}

}  // namespace ttsp

using namespace ttsp;

// Argument checks shared by the entry points; fills the scale shifts.
static int gemm_args(const void* X, const uint8_t* W, const uint8_t* A8, const float* AMAX, const float* CODE2,
                     const float* LUT, void* Y, const void* R, int epi, int M, int K, int N, int blocksize,
                     int blocksize2, int* bs_shift, int* bs2_shift) {
  if (N <= 0 || M <= 0 || K <= 0 || !X || !W || !AMAX || !LUT || !Y) return (int)hipErrorInvalidValue;
  if (A8 && !CODE2) return (int)hipErrorInvalidValue;
  *bs_shift = 0, *bs2_shift = 0;
  while ((1 << *bs_shift) < blocksize) ++*bs_shift;
  if (A8)
    while ((1 << *bs2_shift) < blocksize2) ++*bs2_shift;
  if ((1 << *bs_shift) != blocksize || *bs_shift < 6 || (A8 && (1 << *bs2_shift) != blocksize2))
    return (int)hipErrorInvalidValue;
  if (K % 128 || K % blocksize || epi < 0 || epi > 2 || (epi && !R)) return (int)hipErrorInvalidValue;
  return 0;
}

// One entry for every row count: up to GEMV_ROWS_N rows take the
// bandwidth-bound GEMV (or, past the rows it holds, the kernels below), up
// to 64 rows the skinny MFMA kernel (weights streamed once), more rows the
// tiled MFMA kernel (weights read once per BN rows), unsplit.
extern "C" int ttsp_nf4_gemm(const void* X, int x_dtype, const uint8_t* W, const uint8_t* A8,
                             const float* AMAX, const float* CODE2, float offset, const float* LUT,
                             void* Y, const void* R, int epi, int M, int K, int N, int blocksize,
                             int blocksize2, hipStream_t stream) {
  if (N >= 1 && N <= GEMV_ROWS_N && M > 0 && K > 0 && X && W && AMAX && LUT && Y && (!A8 || CODE2) &&
      gemv_fits(M, K, blocksize, N))
    return gemv_rows(X, x_dtype, W, A8, AMAX, CODE2, offset, LUT, Y, R, epi, M, K, N, blocksize, blocksize2,
                     stream);
  int bs_shift, bs2_shift;
  if (int rc = gemm_args(X, W, A8, AMAX, CODE2, LUT, Y, R, epi, M, K, N, blocksize, blocksize2, &bs_shift,
                         &bs2_shift))
    return rc;
  // (one row whose K the GEMV cannot hold, K > 32768, takes the tiled kernel below)
  if (N >= 2 && skinny(K, N))
    return gemm_skinny(X, x_dtype, W, A8, AMAX, CODE2, offset, LUT, Y, R, epi, M, K, N, bs_shift, bs2_shift, stream);
  // vectorised output rows: 8 elements per 16-byte store
  const bool vec = M % 8 == 0 && (uintptr_t)Y % 16 == 0 && (!epi || (uintptr_t)R % 16 == 0);
  // unsplit: the direct-to-LDS kernel where the plan takes it unsplit, else
  // 64 x 128 tiles, or 64 x 64 when fewer than 128 of those
  GemmPlan plan{unsplit_shape(M, N), 1}, dl;
  if (dl_plan(M, K, N, &dl) && dl.splits == 1) plan = dl;
  return gemm_mfma(X, x_dtype, W, A8, AMAX, CODE2, offset, LUT, Y, R, epi | (vec ? 4 : 0), M, K, N, bs_shift,
                   bs2_shift, plan, nullptr, stream);
}

extern "C" int ttsp_nf4_gemm_splits(int M, int K, int N) {
  if (M <= 0 || K <= 0 || N <= 1 || K % 128) return 1;
  return gemm_plan(M, K, N).splits;
}

extern "C" int ttsp_nf4_gemm_split(const void* X, int x_dtype, const uint8_t* W, const uint8_t* A8,
                                   const float* AMAX, const float* CODE2, float offset, const float* LUT,
                                   void* Y, const void* R, int epi, int M, int K, int N, int blocksize,
                                   int blocksize2, float* work, int splits, hipStream_t stream) {
  if (N <= 1 || splits < 1 || splits != ttsp_nf4_gemm_splits(M, K, N))
    return (int)hipErrorInvalidValue;
  if (splits == 1)
    return ttsp_nf4_gemm(X, x_dtype, W, A8, AMAX, CODE2, offset, LUT, Y, R, epi, M, K, N, blocksize,
                         blocksize2, stream);
  int bs_shift, bs2_shift;
  if (int rc = gemm_args(X, W, A8, AMAX, CODE2, LUT, Y, R, epi, M, K, N, blocksize, blocksize2, &bs_shift,
                         &bs2_shift))
    return rc;
  if (!work || (uintptr_t)work % 16) return (int)hipErrorInvalidValue;
  const bool vec = M % 8 == 0 && (uintptr_t)Y % 16 == 0 && (!epi || (uintptr_t)R % 16 == 0);
  return gemm_mfma(X, x_dtype, W, A8, AMAX, CODE2, offset, LUT, Y, R, epi | (vec ? 4 : 0), M, K, N, bs_shift,
                   bs2_shift, gemm_plan(M, K, N), work, stream);
}

static int log2_of(int v) {
  int sh = 0;
  while (sh < 30 && (1 << sh) < v) ++sh;
  return (1 << sh) == v ? sh : -1;
}

extern "C" int ttsp_nf4_gemm_swiglu_fits(int M, int K, int N, int blocksize, int blocksize2, int nested) {
  const int bs = log2_of(blocksize), bs2 = nested ? log2_of(blocksize2) : 0;
  if (bs < 6 || bs2 < 0 || K % blocksize) return 0;
  return swiglu_skinny(M, K, N) || swiglu_fits(M, K, N, bs, bs2, nested != 0) ? 1 : 0;
}

extern "C" int ttsp_nf4_gemm_swiglu(const void* X, int x_dtype, const uint8_t* W1, const uint8_t* A8_1,
                                    const float* AMAX_1, const float* CODE2_1, float offset_1, const uint8_t* W3,
                                    const uint8_t* A8_3, const float* AMAX_3, const float* CODE2_3,
                                    float offset_3, const float* LUT, void* Y, int M, int K, int N, int blocksize,
                                    int blocksize2, hipStream_t stream) {
  int bs_shift, bs2_shift;
  if (int rc = gemm_args(X, W1, A8_1, AMAX_1, CODE2_1, LUT, Y, nullptr, 0, M, K, N, blocksize, blocksize2,
                         &bs_shift, &bs2_shift))
    return rc;
  if (!W3 || !AMAX_3 || (A8_3 != nullptr) != (A8_1 != nullptr) || (A8_3 && !CODE2_3))
    return (int)hipErrorInvalidValue;
  if ((uintptr_t)X % 16 || (uintptr_t)W1 % 16 || (uintptr_t)W3 % 16) return (int)hipErrorInvalidValue;
  if (swiglu_skinny(M, K, N))
    return gemm_skinny_pair(X, x_dtype, W1, A8_1, AMAX_1, CODE2_1, offset_1, W3, A8_3, AMAX_3, CODE2_3, offset_3, LUT,
                            Y, M, K, N, bs_shift, bs2_shift, stream);
  if (!swiglu_fits(M, K, N, bs_shift, bs2_shift, A8_1 != nullptr)) return (int)hipErrorInvalidValue;
  return gemm_dl_swiglu(X, x_dtype, W1, A8_1, AMAX_1, CODE2_1, offset_1, W3, A8_3, AMAX_3, CODE2_3, offset_3, LUT, Y,
                        M, K, N, bs_shift, bs2_shift, stream);
}

extern "C" int ttsp_nf4_gemm_partials(const void* X, int x_dtype, const uint8_t* W, const uint8_t* A8,
                                      const float* AMAX, const float* CODE2, float offset, const float* LUT, int M,
                                      int K, int N, int blocksize, int blocksize2, float* work, int splits,
                                      hipStream_t stream) {
  if (N <= 1 || splits < 2 || splits != ttsp_nf4_gemm_splits(M, K, N) || !work || (uintptr_t)work % 16)
    return (int)hipErrorInvalidValue;
  int bs_shift, bs2_shift;
  // (Y is not written: the split launch stops at its partial sums)
  if (int rc = gemm_args(X, W, A8, AMAX, CODE2, LUT, work, nullptr, 0, M, K, N, blocksize, blocksize2, &bs_shift,
                         &bs2_shift))
    return rc;
  return gemm_mfma(X, x_dtype, W, A8, AMAX, CODE2, offset, LUT, nullptr, nullptr, 0, M, K, N, bs_shift, bs2_shift,
                   gemm_plan(M, K, N), work, stream, false);
}

extern "C" int ttsp_nf4_gemm_split_norm(const void* X, int x_dtype, const uint8_t* W, const uint8_t* A8,
                                        const float* AMAX, const float* CODE2, float offset, const float* LUT,
                                        void* Y, const void* R, int epi, int M, int K, int N, int blocksize,
                                        int blocksize2, float* work, int splits, const void* G, float eps, void* YN,
                                        hipStream_t stream) {
  if (N <= 1 || splits < 2 || splits != ttsp_nf4_gemm_splits(M, K, N) || (splits != 2 && splits != 4 && splits != 8))
    return (int)hipErrorInvalidValue;
  if (M % 8 || M > 64 * 8 * NRM_CH || !G || !YN || !work) return (int)hipErrorInvalidValue;
  if ((uintptr_t)Y % 16 || (uintptr_t)YN % 16 || (uintptr_t)G % 16 || (uintptr_t)work % 16 ||
      (epi && (uintptr_t)R % 16))
    return (int)hipErrorInvalidValue;
  if (x_dtype != DT_BF16 && x_dtype != DT_F16) return (int)hipErrorInvalidValue;
  int bs_shift, bs2_shift;
  if (int rc = gemm_args(X, W, A8, AMAX, CODE2, LUT, Y, R, epi, M, K, N, blocksize, blocksize2, &bs_shift,
                         &bs2_shift))
    return rc;
  if (int rc = gemm_mfma(X, x_dtype, W, A8, AMAX, CODE2, offset, LUT, Y, R, epi, M, K, N, bs_shift, bs2_shift,
                         gemm_plan(M, K, N), work, stream, false))
    return rc;
  const dim3 grid((unsigned)N), block((unsigned)(64 * ((M / 8 + 63) / 64)));
#define TTSP_RN(DTV, SV)                                                                                      \
  hipLaunchKernelGGL((nf4_gemm_reduce_norm_kernel<DTV, SV>), grid, block, 0, stream, work, (uint16_t*)Y, \
                     (const uint16_t*)R, epi, M, N, (const uint16_t*)G, eps, (uint16_t*)YN)
#define TTSP_RS(DTV)                  \
  if (splits == 2) TTSP_RN(DTV, 2);   \
  else if (splits == 4) TTSP_RN(DTV, 4); \
  else TTSP_RN(DTV, 8);
  if (x_dtype == DT_BF16) {
    TTSP_RS(DT_BF16)
  } else {
    TTSP_RS(DT_F16)
  }
#undef TTSP_RS
#undef TTSP_RN
  TTSP_RETURN_LAUNCH();
}
