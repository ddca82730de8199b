// NF4 matmul for a few activation rows (2 <= N <= 64; the split plan takes
// 64 x 64 GEMM tiles from 33 rows, see nf4_gemm.hip): Y[N][M] = X[N][K] . W^T,
// W in the bitsandbytes layout (nf4_gemv.hip describes it).
//
// With few rows the weights are still the traffic - every weight byte is used
// by at most 64 rows - so the kernel is shaped like the GEMV: the weight is
// streamed once across the whole chip and the row dimension rides along on
// the matrix cores.
//
//   * Work split. A workgroup owns 16 R weight rows; its NW waves split K
//     into NW runs of 128-code steps (ragged when NW does not divide them).
//     Partial sums meet in LDS and are added in wave order, so results are a
//     fixed function of the inputs. Enough workgroups to cover the chip come
//     from the rows alone (M / 16 R).
//   * Loads. Per step, lane (m = l % 16, q = l / 16) of a wave reads 16 bytes
//     (32 codes) of weight row m of each of its R row tiles at byte 64 s + 16 q:
//     16 rows x 64 contiguous bytes per instruction. The activations come
//     straight from L2 (all workgroups read the same X): lane (n, q) reads 16
//     bytes of row n of each 16-row tile of X at element 128 s + 32 q + 8 t for
//     t = 0..3. Both streams run PF steps ahead of the arithmetic.
//   * Products. v_mfma_f32_16x16x32 with X as the A operand (row n, eight k
//     per lane) and the dequantised weights as B (column m, the same eight k):
//     the eight codes a lane carries for matrix product t are codes
//     128 s + 32 q + 8 t .. + 7, and its X fragment holds exactly those eight
//     activations, so A and B agree on every k (the k order inside a product
//     is irrelevant to the sum). The accumulator of lane (m, q) holds outputs
//     (4 q + i, m), i = 0..3.
//   * Dequantisation, as bitsandbytes' dequantize_4bit: each byte's two codes
//     come from one 8-byte LDS lookup in a 256-entry table of fp32 code pairs,
//     are multiplied by the block scale in fp32 and rounded to the activation
//     type by one hardware pack-convert: the same weight values the MFMA GEMM
//     and the dequant kernel produce. The lookups are the kernel's heaviest
//     traffic (8 bytes of LDS per weight byte), so the table holds 32
//     copies, entry e of copy j at byte 256 e + 8 j, and lane l reads copy
//     l % 32: a lookup's 64 lanes touch 128 dwords on 64 banks, two lanes a
//     bank pair, the minimum whatever the bytes; the address is one v_perm_b32
//     of the weight byte next to the lane's offset. The 64 KB are reused for
//     the partial sums after the loop, so two workgroups fit a CU. A lane's 32 codes of a step lie in one scale block
//     (64-code blocks start at multiples of 64).
//   * The SwiGLU pair (PAIR): each of a workgroup's R row tiles is read from
//     W1 and from W3 (2 R tile slots, two code2 tables), and the epilogue
//     rounds as the two launches do: g = W1 x stored, then
//     silu(g) rounded times (W3 x) rounded, rounded.
#include "ttsp_common.h"

namespace ttsp {

typedef __bf16 sk_bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 sk_f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 sk_bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 sk_f16x2 __attribute__((ext_vector_type(2)));
typedef float sk_f32x2 __attribute__((ext_vector_type(2)));

constexpr int SK_REP = 32;    // copies of the code-pair table (entry rows of 256 bytes)
constexpr int SK_LDS = 256 * SK_REP * 8;
static_assert(SK_REP * 8 == 256, "the lookup address is 256 e + 8 (lane % SK_REP): byte e at bits 8..15");
#ifndef SKINNY_PF
#define SKINNY_PF 2
#endif
constexpr int SK_PF = SKINNY_PF;  // steps of activations in flight
constexpr int SK_MAXS = 10;       // most 128-code steps a wave takes (its weights are all in flight at once)

template <int DT>
__device__ __forceinline__ f32x4 sk_mfma(u32x4 a, u32x4 b, f32x4 c) {
  if constexpr (DT == DT_BF16)
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(sk_bf16x8, a), __builtin_bit_cast(sk_bf16x8, b),
                                                   c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(sk_f16x8, a), __builtin_bit_cast(sk_f16x8, b),
                                                  c, 0, 0, 0);
}

// Two fp32 products to the activation type, rounded once each (RNE), lo in the low half.
template <int DT>
__device__ __forceinline__ uint32_t sk_pack2(float lo, float hi) {
  const sk_f32x2 v = {opaque(lo), opaque(hi)};
  if constexpr (DT == DT_BF16)
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, sk_bf16x2));
  else
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, sk_f16x2));
}

// MS: the wave's step budget (its K run is at most MS steps). TG: row-tile
// groups a workgroup (NW waves each, one table for all): the grid's
// workgroups split the row tiles evenly (workgroup b takes tiles
// b T / G .. (b + 1) T / G - 1, at most TG of them; a group past them repeats
// the first tile's loads and stores nothing), so a matrix of 2-3 tiles a CU
// runs in one round of workgroups instead of two and a tail.
// The second matrix of the SwiGLU pair (PAIR): its weights and scales.
struct SkinnyW3 {
  const uint8_t* W;
  const uint8_t* A8;
  const float* AMAX;
  const float* CODE2;
  float offset;
};

template <int DT, int R, int NT, int NW, int MS, bool NESTED, int TG = 1, bool PAIR = false>
__global__ __launch_bounds__(64 * NW * TG) void nf4_skinny_kernel(
    const uint16_t* __restrict__ X, const uint8_t* __restrict__ W, const uint8_t* __restrict__ A8,
    const float* __restrict__ AMAX, const float* __restrict__ CODE2, float offset, const float* __restrict__ LUT,
    uint16_t* __restrict__ Y, const uint16_t* __restrict__ RES, int epi, int M, int K, int N, int bs_shift,
    int bs2_shift, SkinnyW3 w3) {
  // byte e -> (code of its high nibble, code of its low nibble), copy j at
  // [e][j]; after the loop the same memory holds each wave's partial sums
  constexpr int NWT = NW * TG;  // waves a workgroup
  constexpr int S = PAIR ? 2 * R : R;  // tile slots: slot r < R of W, slot R + r of W3 (same rows)
  static_assert(NWT * S * NT * 64 * sizeof(f32x4) <= SK_LDS, "partial sums exceed the table's LDS");
  __shared__ __align__(16) unsigned char lds[SK_LDS];
  __shared__ __align__(16) float code2_s[NESTED ? (PAIR ? 512 : 256) : 4];
  float2 (*lut2)[SK_REP] = reinterpret_cast<float2 (*)[SK_REP]>(lds);
  f32x4 (*part)[S * NT][64] = reinterpret_cast<f32x4 (*)[S * NT][64]>(lds);

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int grp = TG > 1 ? wave / NW : 0, wk = TG > 1 ? wave % NW : wave;  // row-tile group, K run
  const int m = lane & 15, q = lane >> 4;
  int tile = blockIdx.x;
  bool own = true;  // the group has a tile of its own (its stores happen)
  if constexpr (TG > 1) {
    const int T = (M + 16 * R - 1) / (16 * R), G = (int)gridDim.x;
    const int b0 = (int)((long long)blockIdx.x * T / G), b1 = (int)((long long)(blockIdx.x + 1) * T / G);
    own = b0 + grp < b1;
    tile = own ? b0 + grp : b0;
  }
  const int row0 = tile * 16 * R;
  const int steps = K >> 7;  // 128-code steps per row
  const int s0 = wk * steps / NW, s1 = (wk + 1) * steps / NW;
  const size_t rowbytes = (size_t)K >> 1;
  const int nblk = K >> bs_shift;


  // Issue order (vector memory counters retire in order, so a wait for one
  // load is a wait for everything issued before it): the small operands the
  // tables need, then the activations of the first SK_PF steps, then the
  // wave's whole weight share (MS steps of R 16-byte pieces) and its scales,
  // step by step; nothing waits before all of it is in flight. Every load is
  // unconditional - steps past the wave's run repeat its last step, unused -
  // so no branch separates a load from its use and the compiler's wait counts
  // stay exact (a load under a branch makes it wait for everything).
  const float c16 = LUT[lane & 15];
  f32x4 c2v = {0.0f, 0.0f, 0.0f, 0.0f}, c2v3 = {0.0f, 0.0f, 0.0f, 0.0f};
  if constexpr (NESTED)
#pragma unroll
    for (int i = 0; i < 4; ++i) c2v[i] = CODE2[4 * lane + i];
  if constexpr (NESTED && PAIR)
#pragma unroll
    for (int i = 0; i < 4; ++i) c2v3[i] = w3.CODE2[4 * lane + i];
  u32x4 xq[SK_PF][NT][4];
  auto load_x = [&](u32x4 (&xs)[NT][4], int step) {
    const int st = min(step, max(s1 - 1, 0));
#pragma unroll
    for (int c = 0; c < NT; ++c) {
      const int n = min(16 * c + m, N - 1);
      const u32x4* xr = reinterpret_cast<const u32x4*>(X + (size_t)n * K + 128 * st + 32 * q);
#pragma unroll
      for (int t = 0; t < 4; ++t) xs[c][t] = xr[t];
    }
  };
  // (a wave with an empty run - K < 128 NW - loads step 0 and adds nothing)
  const int slast = max(s1 - 1, 0);
#pragma unroll
  for (int i = 0; i < SK_PF; ++i) load_x(xq[i], s0 + i);
  __builtin_amdgcn_sched_barrier(0);  // keep the issue order: the scheduler would move later loads ahead
  u32x4 wq[MS][S];
  float sq[MS][S];
  uint32_t aq[NESTED ? MS : 1][S];
#pragma unroll
  for (int j = 0; j < MS; ++j) {
    const int st = min(s0 + j, slast);
#pragma unroll
    for (int r = 0; r < S; ++r) {
      const bool m3 = PAIR && r >= R;
      const int row = min(row0 + 16 * (r % R) + m, M - 1);
      wq[j][r] = __builtin_nontemporal_load(
          reinterpret_cast<const u32x4*>((m3 ? w3.W : W) + (size_t)row * rowbytes + 64 * (size_t)st + 16 * q));
      const int b = row * nblk + ((128 * st + 32 * q) >> bs_shift);
      if constexpr (NESTED) {
        aq[j][r] = (m3 ? w3.A8 : A8)[b] + (m3 ? 256u : 0u);
        sq[j][r] = (m3 ? w3.AMAX : AMAX)[b >> bs2_shift];
      } else {
        sq[j][r] = (m3 ? w3.AMAX : AMAX)[b];
      }
    }
    __builtin_amdgcn_sched_barrier(0);
  }

  f32x4 acc[S][NT];
#pragma unroll
  for (int r = 0; r < S; ++r)
#pragma unroll
    for (int c = 0; c < NT; ++c) acc[r][c] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

  // the tables, while the operands stream: wave w writes entries w, w + NW,
  // ..., four a store instruction (lane l: entry base + l / 16, copies
  // 2 (l % 16) and 2 (l % 16) + 1), codes taken from the lanes that loaded them
  // (straight-line: a loop or a branch around these uses of loaded values
  // would make the compiler wait for every load first)
#pragma unroll
  for (int k = 0; k < (64 + NWT - 1) / NWT; ++k) {
    // (64 % NWT != 0: the last round's waves past entry group 63 rewrite it with the same values)
    const int eg = 64 % NWT == 0 ? wave + NWT * k : min(wave + NWT * k, 63);
    const int e = 4 * eg + (lane >> 4), j = 2 * (lane & 15);
    const float hi = __shfl(c16, e >> 4), lo = __shfl(c16, e & 15);
    *reinterpret_cast<float4*>(&lut2[e][j]) = make_float4(hi, lo, hi, lo);
  }
  // every wave writes the same code2 values (no branch on the wave)
  if constexpr (NESTED) reinterpret_cast<f32x4*>(code2_s)[lane] = c2v;
  if constexpr (NESTED && PAIR) reinterpret_cast<f32x4*>(code2_s + 256)[lane] = c2v3;
  // (no arithmetic on the streamed operands may move above the barrier: each
  // such use waits for its load, and the in-order counter for every load
  // issued before it)
  __builtin_amdgcn_sched_barrier(0);
  __syncthreads();
  __builtin_amdgcn_sched_barrier(0);
  const unsigned char* tab = reinterpret_cast<const unsigned char*>(&lut2[0][0]);
  const uint32_t lane8 = 8u * (uint32_t)(lane & (SK_REP - 1));
  // rows n >= N of an X tile contribute zeros (their fragments are replaced)
  bool nvalid[NT];
#pragma unroll
  for (int c = 0; c < NT; ++c) nvalid[c] = 16 * c + m < N;

  // Every budgeted step is computed - a branch around a step would let the
  // compiler sink that step's loads into it, after the barrier - and steps
  // past the wave's run add exact zeros (zero scale, zero activations).
#pragma unroll
  for (int j = 0; j < MS; ++j) {
    u32x4 (&xs)[NT][4] = xq[j % SK_PF];
    const bool live = s0 + j < s1;
#pragma unroll
    for (int r = 0; r < S; ++r) {
      float sc = sq[j][r];
      if constexpr (NESTED) sc = __fadd_rn(__fmul_rn(code2_s[aq[j][r]], sc), PAIR && r >= R ? w3.offset : offset);
      sc = live ? sc : 0.0f;
      const uint32_t wv[4] = {wq[j][r][0], wq[j][r][1], wq[j][r][2], wq[j][r][3]};
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        uint32_t bw[4];
#pragma unroll
        for (int b = 0; b < 4; ++b) {
          // entry e = byte b of the dword, at 256 e + 8 (lane % 32)
          const float2 pc = *reinterpret_cast<const float2*>(
              tab + __builtin_amdgcn_perm(wv[t], lane8, 0x0C0C0400u + ((uint32_t)b << 8)));
          bw[b] = sk_pack2<DT>(__fmul_rn(pc.x, sc), __fmul_rn(pc.y, sc));
        }
        const u32x4 bop = {bw[0], bw[1], bw[2], bw[3]};
#pragma unroll
        for (int c = 0; c < NT; ++c) {
          const u32x4 xa = live && nvalid[c] ? xs[c][t] : u32x4{0u, 0u, 0u, 0u};
          acc[r][c] = sk_mfma<DT>(xa, bop, acc[r][c]);
        }
      }
    }
    if (j + SK_PF < MS) load_x(xs, s0 + j + SK_PF);
  }

  // K runs in wave order within a group; wave w of a group finishes its row
  // tiles r with r % NW == w
  __syncthreads();  // every wave is past its last lookup: the table's memory takes the partial sums
#pragma unroll
  for (int r = 0; r < S; ++r)
#pragma unroll
    for (int c = 0; c < NT; ++c) part[wave][r * NT + c][lane] = acc[r][c];
  __syncthreads();
  const int ep = epi & 3;
#pragma unroll
  for (int r = 0; r < R; ++r) {
    if (r % NW != wk) continue;
    const int row = row0 + 16 * r + m;
#pragma unroll
    for (int c = 0; c < NT; ++c) {
      f32x4 v = part[grp * NW][r * NT + c][lane], v3 = {0.0f, 0.0f, 0.0f, 0.0f};
      if constexpr (PAIR) v3 = part[grp * NW][(R + r) * NT + c][lane];
#pragma unroll
      for (int w = 1; w < NW; ++w) {
        const f32x4 o = part[grp * NW + w][r * NT + c][lane];
#pragma unroll
        for (int i = 0; i < 4; ++i) v[i] = __fadd_rn(v[i], o[i]);
        if constexpr (PAIR) {
          const f32x4 o3 = part[grp * NW + w][(R + r) * NT + c][lane];
#pragma unroll
          for (int i = 0; i < 4; ++i) v3[i] = __fadd_rn(v3[i], o3[i]);
        }
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int n = 16 * c + 4 * q + i;
        if (n >= N || row >= M || !own) continue;
        const size_t o = (size_t)n * M + row;
        const float y = Elem<DT>::load(Elem<DT>::store(v[i]));
        float out = y;
        if constexpr (PAIR)  // W1's output as its launch stores it, then W3's gate epilogue
          out = __fmul_rn(Elem<DT>::load(Elem<DT>::store(silu_rn(y))), Elem<DT>::load(Elem<DT>::store(v3[i])));
        else if (ep == 1) out = __fadd_rn(Elem<DT>::load(RES[o]), y);
        else if (ep == 2) out = __fmul_rn(Elem<DT>::load(Elem<DT>::store(silu_rn(Elem<DT>::load(RES[o])))), y);
        Y[o] = Elem<DT>::store(out);
      }
    }
  }
}

int skinny_max_k(int N);

bool skinny_pair_fits(int K, int N);

// PAIR: the SwiGLU pair (w3 set), with half the row tiles a workgroup of the
// single form where that has several, and one with two X tiles (each tile
// slot is a tile of one matrix; a pair tile is two slots, which keeps the
// loads in flight and the registers near the single form's; two X tiles and
// four slots held one wave a SIMD: 9728 x 2560 at 32 rows 32.3 against
// 24.7 us with one tile, at 17 rows 28.1 against 20.5).
template <int DT, int RV, int NT, int NW, int MS, int TG = 1, bool PAIR = false>
static void launch_skinny(const void* X, const uint8_t* W, const uint8_t* A8, const float* AMAX, const float* CODE2,
                          float offset, const float* LUT, void* Y, const void* RES, int epi, int M, int K, int N,
                          int bs_shift, int bs2_shift, hipStream_t st, const SkinnyW3& w3) {
  constexpr int R = PAIR && RV > 1 ? (NT >= 2 ? 1 : RV / 2) : RV;
  const int tiles = (M + 16 * R - 1) / (16 * R);
  const dim3 grid((tiles + TG - 1) / TG);  // TG tiles a workgroup (the last may hold fewer)
  if (A8)
    hipLaunchKernelGGL((nf4_skinny_kernel<DT, R, NT, NW, MS, true, TG, PAIR>), grid, dim3(64 * NW * TG), 0, st,
                       (const uint16_t*)X, W, A8, AMAX, CODE2, offset, LUT, (uint16_t*)Y, (const uint16_t*)RES, epi,
                       M, K, N, bs_shift, bs2_shift, w3);
  else
    hipLaunchKernelGGL((nf4_skinny_kernel<DT, R, NT, NW, MS, false, TG, PAIR>), grid, dim3(64 * NW * TG), 0, st,
                       (const uint16_t*)X, W, A8, AMAX, CODE2, offset, LUT, (uint16_t*)Y, (const uint16_t*)RES, epi,
                       M, K, N, bs_shift, bs2_shift, w3);
}

// Launch shape. NW: the fewest waves (4, 8, 16) whose K runs fit SK_MAXS
// steps; with fewer than 256 row tiles and runs of more than 5 steps at 4
// waves, at least 8 (more waves per row tile). MS: the step budget; one row
// tile a workgroup takes the smallest of 2, 3, 4, 5, 6, 8, 10 that holds the
// run (every step past the run repeats a load: 2560 x 4096, runs of 4, 6.1
// against 7.0 us with MS = 5 at 4 rows, 7.7 against 9.1 at 16), the other
// forms 5 when the runs fit it, else SK_MAXS. R: with 512 or more
// row tiles, several tiles a workgroup (each X fragment then serves R of them:
// the activation traffic, which binds from 16 rows up, drops by R) - 4 for
// 17-32 rows and 2 otherwise with 4 waves, 2 from 9 rows with 8 - else 1.
// (Measured: at 9728 x 2560 two tiles cost 0.4-0.9 us more than one up to 8
// rows and save 0.7 at 16; 32 rows 16.8 us with R = 4 against 18.3 with 2,
// 64 rows 32.7 with R = 2 against 38.7 with 1; at 1024 x 2560 four waves take
// 5.7 / 6.4 / 9.3 us for 4 / 16 / 32 rows against 6.9 / 9.1 / 14.2 with
// eight, at 2560 x 4096 and 1024 x 3072 eight are faster.) Returns false when
// no shape fits (see skinny_max_k).
template <int DT, int NT, bool PAIR = false>
static bool skinny_shape(const void* X, const uint8_t* W, const uint8_t* A8, const float* AMAX, const float* CODE2,
                         float offset, const float* LUT, void* Y, const void* RES, int epi, int M, int K, int N,
                         int bs_shift, int bs2_shift, hipStream_t st, const SkinnyW3& w3 = SkinnyW3{}) {
  const int tiles = (M + 15) / 16, steps = K >> 7;
  int nw = (steps + SK_MAXS - 1) / SK_MAXS;
  if (nw > 16) return false;
  nw = nw <= 4 ? 4 : nw <= 8 ? 8 : 16;
  if (tiles < 256 && nw < 8 && steps > 4 * 5) nw = 8;
  const int run = (steps + nw - 1) / nw;
  const bool ms5 = run <= 5;
  const bool r2 = NT <= 2 && nw <= 8 && tiles >= 2 * 256 && N > 8;
#define TTSP_L(RV, NWV, MSV)                                                                                 \
  launch_skinny<DT, RV, NT, NWV, MSV, 1, PAIR>(X, W, A8, AMAX, CODE2, offset, LUT, Y, RES, epi, M, K, N, bs_shift, \
                                               bs2_shift, st, w3)
#define TTSP_MS(RV, NWV) \
  do {                   \
    if (ms5) TTSP_L(RV, NWV, 5); \
    else TTSP_L(RV, NWV, SK_MAXS); \
  } while (0)
#define TTSP_MS1(NWV)                    \
  do {                                   \
    if (run <= 2) TTSP_L(1, NWV, 2);     \
    else if (run <= 3) TTSP_L(1, NWV, 3); \
    else if (run <= 4) TTSP_L(1, NWV, 4); \
    else if (run <= 5) TTSP_L(1, NWV, 5); \
    else if (run <= 6) TTSP_L(1, NWV, 6); \
    else if (run <= 8) TTSP_L(1, NWV, 8); \
    else TTSP_L(1, NWV, SK_MAXS);        \
  } while (0)
  const bool many = tiles >= 2 * 256;
  // 2-3 row tiles a CU, up to 8 rows: three tiles a workgroup (12 waves, one
  // table) run in one round instead of two and a tail (9728 x 2560: 9.4
  // against 10.4 us at 4 rows, 10.5 against 10.7 at 8; 16 rows tie)
  if constexpr (NT == 1) {
    if (many && tiles < 3 * 256 && N <= 8 && nw == 4 && ms5) {
      launch_skinny<DT, 1, 1, 4, 5, 3, PAIR>(X, W, A8, AMAX, CODE2, offset, LUT, Y, RES, epi, M, K, N, bs_shift,
                                              bs2_shift, st, w3);
      return true;
    }
  }
  if constexpr (NT == 2) {
    if (many && nw == 4 && ms5) { TTSP_L(4, 4, 5); return true; }
  }
  if constexpr (NT == 4 && !PAIR) {
    if (many && nw == 4 && ms5) { TTSP_L(2, 4, 5); return true; }
  }
  if constexpr (NT <= 2) {
    if (r2 && nw == 4) { TTSP_MS(2, 4); return true; }
    if (r2) { TTSP_MS(2, 8); return true; }
  }
  if (nw == 4) TTSP_MS1(4);
  else if (nw == 8) TTSP_MS1(8);
  else if constexpr (NT == 1 && !PAIR) TTSP_MS1(16);  // 1024 threads: 128 registers a lane, enough for one X tile only
  else return false;
#undef TTSP_MS1
#undef TTSP_MS
#undef TTSP_L
  return true;
}

int gemm_skinny(const void* X, int dt, const uint8_t* W, const uint8_t* A8, const float* AMAX, const float* CODE2,
                float offset, const float* LUT, void* Y, const void* RES, int epi, int M, int K, int N, int bs_shift,
                int bs2_shift, hipStream_t st) {
  if (N < 2 || N > 64 || K % 128 || K > skinny_max_k(N) || bs_shift < 6 || (uintptr_t)X % 16 || (uintptr_t)W % 16)
    return (int)hipErrorInvalidValue;
  const int NT = (N + 15) / 16;
  bool ok;
#define TTSP_SK(DTV)                                                                                               \
  do {                                                                                                             \
    if (NT == 1) ok = skinny_shape<DTV, 1>(X, W, A8, AMAX, CODE2, offset, LUT, Y, RES, epi, M, K, N, bs_shift,      \
                                           bs2_shift, st);                                                         \
    else if (NT == 2) ok = skinny_shape<DTV, 2>(X, W, A8, AMAX, CODE2, offset, LUT, Y, RES, epi, M, K, N,          \
                                                bs_shift, bs2_shift, st);                                          \
    else ok = skinny_shape<DTV, 4>(X, W, A8, AMAX, CODE2, offset, LUT, Y, RES, epi, M, K, N, bs_shift, bs2_shift,   \
                                   st);                                                                            \
  } while (0)
  if (dt == DT_BF16) TTSP_SK(DT_BF16);
  else if (dt == DT_F16) TTSP_SK(DT_F16);
  else return (int)hipErrorInvalidValue;
#undef TTSP_SK
  if (!ok) return (int)hipErrorInvalidValue;
  TTSP_RETURN_LAUNCH();
}

// The SwiGLU pair in one launch: Y = silu(X W1^T) * (X W3^T), rounded and
// with the bits of gemm_skinny(W1) then gemm_skinny(W3, epi 2) on its output.
// Up to 32 rows (one or two X tiles) and K runs of at most 8 waves.
int gemm_skinny_pair(const void* X, int dt, const uint8_t* W1, const uint8_t* A8_1, const float* AMAX_1,
                     const float* CODE2_1, float offset_1, const uint8_t* W3, const uint8_t* A8_3, const float* AMAX_3,
                     const float* CODE2_3, float offset_3, const float* LUT, void* Y, int M, int K, int N, int bs_shift,
                     int bs2_shift, hipStream_t st) {
  if (!skinny_pair_fits(K, N) || bs_shift < 6 || (uintptr_t)X % 16 || (uintptr_t)W1 % 16 || (uintptr_t)W3 % 16)
    return (int)hipErrorInvalidValue;
  const SkinnyW3 w3{W3, A8_3, AMAX_3, CODE2_3, offset_3};
  bool ok;
#define TTSP_SK(DTV)                                                                                                \
  do {                                                                                                              \
    if (N <= 16) ok = skinny_shape<DTV, 1, true>(X, W1, A8_1, AMAX_1, CODE2_1, offset_1, LUT, Y, nullptr, 0, M, K, N, \
                                                 bs_shift, bs2_shift, st, w3);                                      \
    else ok = skinny_shape<DTV, 2, true>(X, W1, A8_1, AMAX_1, CODE2_1, offset_1, LUT, Y, nullptr, 0, M, K, N,        \
                                         bs_shift, bs2_shift, st, w3);                                              \
  } while (0)
  if (dt == DT_BF16) TTSP_SK(DT_BF16);
  else if (dt == DT_F16) TTSP_SK(DT_F16);
  else return (int)hipErrorInvalidValue;
#undef TTSP_SK
  if (!ok) return (int)hipErrorInvalidValue;
  TTSP_RETURN_LAUNCH();
}

bool skinny_pair_fits(int K, int N) { return N >= 2 && N <= 32 && K % 128 == 0 && K <= 8 * SK_MAXS * 128; }

// The longest row the skinny kernel takes for N activation rows: 16 waves of
// SK_MAXS steps for one X tile (N <= 16), 8 waves otherwise.
int skinny_max_k(int N) { return (N <= 16 ? 16 : 8) * SK_MAXS * 128; }

}  // namespace ttsp
