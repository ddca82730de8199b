// NF4 GEMM with direct global->LDS operand streams (prompt prefill, 128-row
// activation tiles): Y[N][M] = X[N][K] . W^T, the weight in the bitsandbytes
// NF4 layout (nf4_gemv.hip gives it), each dequantised weight the exact
// round(code * scale) of bitsandbytes' dequantize_4bit.
//
// A workgroup of W waves owns 32 W weight rows x 128 activation rows; each
// wave owns 32 weight rows x all 128 activation rows (four 32x32 MFMA blocks,
// v_mfma_f32_32x32x16). Per K-step of 64 codes:
//   * the activations (128 rows x 128 bytes) and each wave's packed weight
//     codes (32 rows x 32 bytes) arrive in a two-stage LDS ring by
//     buffer_load ... lds: no VGPR staging, no VALU, issued one step ahead;
//   * an activation load moves 8 whole 128-byte rows (coalesced); inside a
//     row's LDS copy the 16-byte segment s of row t sits at slot
//     s ^ ((t >> 1) & 7), so the MFMA B-fragment reads (16 consecutive rows,
//     one segment each) hit 16 distinct slots of the 256-byte bank width;
//   * each wave dequantises its own rows straight into the MFMA A operand
//     (both codes of a byte from one lookup in a 256-entry table of code
//     pairs, fp32 products, one pack-convert per pair).
// Inside a step lane half h carries codes 32h .. 32h + 31 and k-slice kk the
// MFMA's 8 of them; A and B agree, so each output sums the same products.
// Nested scales of the workgroup's K range are staged once (a8 bytes per
// (row, step), per lane its row's amax pair); plain fp32 absmax arrives with
// each step's loads. A workgroup takes at most DL_MAX_STEPS K-steps.
//
// The barrier of a step is a bare s_barrier: __syncthreads' release fence
// would also wait for the ring loads still in flight. Each wave waits for its
// own loads of the step (vmcnt) before it; its LDS reads of the stage the
// next loads refill fed its MFMAs, so they are complete. The step body takes
// its LDS stages as restrict pointers of one inlined call: the compiler then
// sees that the refill cannot change the stage being read and inserts no
// wait for it.
#include "ttsp_common.h"

namespace ttsp {

namespace {

typedef __bf16 bf16x8_v __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_v __attribute__((ext_vector_type(8)));
typedef float f32x16_v __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x2_v __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2_v __attribute__((ext_vector_type(2)));
typedef float f32x2_v __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) void* lds_ptr_t;

constexpr int KT = 64;             // codes per K-step
constexpr int CH = 1024;           // bytes of one wave-wide 16-byte-per-lane load
constexpr int BN = 128;            // activation rows per workgroup
constexpr int BSTAGE = BN * 128;   // activation bytes per step
constexpr int DL_MAX_STEPS = 64;   // K-steps a workgroup may take

// s_waitcnt bounding vmcnt only (gfx9 encoding)
#define TTSP_VMWAIT(n) __builtin_amdgcn_s_waitcnt(((n) & 15) | (((n) >> 4) << 14) | (7 << 4) | (15 << 8))

template <int DT>
__device__ __forceinline__ f32x16_v mfma32(u32x4 a, u32x4 b, f32x16_v c) {
  if constexpr (DT == DT_BF16)
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_v, a), __builtin_bit_cast(bf16x8_v, b),
                                                   c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8_v, a), __builtin_bit_cast(f16x8_v, b), c,
                                                  0, 0, 0);
}

// two fp32 products to the activation type, one hardware pack-convert
template <int DT>
__device__ __forceinline__ uint32_t pack2(float lo, float hi) {
  const f32x2_v v = {opaque(lo), opaque(hi)};
  if constexpr (DT == DT_BF16)
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_v));
  else
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, f16x2_v));
}

// One K-step: load a later step into stage dst (CPW activation loads, this
// wave's codes, and with plain scales its rows' absmax: one dword a
// lane, lane l row l % 32), then multiply the step in stage rd with scale sc
// (plain: read from the stage).
template <int DT, int W, int CPW, bool PLAIN, typename RS>
__device__ __forceinline__ void dl_step(const uint8_t* __restrict__ rd, uint8_t* __restrict__ dst,
                                        const float2* __restrict__ lut, RS xr, RS wr, RS ar,
                                        const uint32_t (&xoff)[CPW], uint32_t woff, uint32_t aoff, int xsoff,
                                        int wsoff, int asoff, int wave, int lane, float sc, f32x16_v (&acc)[4]) {
  constexpr int SOFF = BSTAGE + W * CH;  // the plain scales' 256 bytes a wave
#pragma unroll
  for (int j = 0; j < CPW; ++j)
    __builtin_amdgcn_raw_ptr_buffer_load_lds(xr, (lds_ptr_t)(dst + (wave * CPW + j) * CH), 16, xoff[j], xsoff, 0, 0);
  __builtin_amdgcn_raw_ptr_buffer_load_lds(wr, (lds_ptr_t)(dst + BSTAGE + wave * CH), 16, woff, wsoff, 0, 0);
  if constexpr (PLAIN) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(ar, (lds_ptr_t)(dst + SOFF + wave * 256), 4, aoff, asoff, 0, 0);
    sc = *reinterpret_cast<const float*>(rd + SOFF + wave * 256 + 4 * (lane & 31));
  }
  const u32x4 codes = *reinterpret_cast<const u32x4*>(rd + BSTAGE + wave * CH + lane * 16);
#pragma unroll
  for (int kk = 0; kk < 4; ++kk) {
    u32x4 bf[4];
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      const int t = 32 * b + (lane & 31), sg = 4 * (lane >> 5) + kk;
      bf[b] = *reinterpret_cast<const u32x4*>(rd + t * 128 + ((sg ^ ((t >> 1) & 7)) << 4));
    }
    const uint32_t wv = codes[kk];
    float cv[8];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float2 pc = lut[(wv >> (8 * j)) & 0xffu];  // (high nibble's code, low nibble's)
      cv[2 * j] = pc.x;
      cv[2 * j + 1] = pc.y;
    }
    u32x4 af;
#pragma unroll
    for (int e = 0; e < 4; ++e) af[e] = pack2<DT>(__fmul_rn(cv[2 * e], sc), __fmul_rn(cv[2 * e + 1], sc));
#pragma unroll
    for (int b = 0; b < 4; ++b) acc[b] = mfma32<DT>(af, bf[b], acc[b]);
  }
}

// epilogue of one value (y already rounded): ep 1 adds R, ep 2 multiplies by
// round(silu(R)); the result rounded
template <int DT>
__device__ __forceinline__ uint16_t dl_epi(float y, uint16_t r, int ep) {
  float v = y;
  if (ep == 1) v = __fadd_rn(Elem<DT>::load(r), y);
  else if (ep == 2) v = __fmul_rn(Elem<DT>::load(Elem<DT>::store(silu_rn(Elem<DT>::load(r)))), y);
  return Elem<DT>::store(v);
}

// The SwiGLU form's second weight (w3): its codes and scales as the first's.
struct DlMat {
  const uint8_t* W;
  const uint8_t* A8;
  const float* AMAX;
  const float* CODE2;
  float offset;
};

// SW: the SwiGLU form. Waves 0 .. W/2 - 1 take rows of the first weight (w1,
// the gate), waves W/2 .. W - 1 the same rows of the second (m3, w3); the
// gate's rounded outputs meet w3's in LDS and the workgroup stores
// round(round(silu(g)) * round(u)), the two launches' bits.
template <int DT, bool NESTED, int W, bool SW = false>
__global__ __launch_bounds__(64 * W) void nf4_gemm_dl_kernel(
    const uint16_t* __restrict__ X, const uint8_t* __restrict__ Wt, const uint8_t* __restrict__ A8,
    const float* __restrict__ AMAX, const float* __restrict__ CODE2, float offset, const float* __restrict__ LUT,
    uint16_t* __restrict__ Y, const uint16_t* __restrict__ R, int epi, int M, int K, int N, int bs_shift,
    int bs2_shift, float* __restrict__ YP, const DlMat m3 = DlMat{}) {
  // the buffer-resource type exists in device code only
#if defined(__HIP_DEVICE_COMPILE__)
  constexpr int BM = 32 * W;   // weight rows the waves take (SW: BM / 2 of each weight)
  constexpr int BMO = SW ? BM / 2 : BM;  // output rows a workgroup
  static_assert(!SW || W % 2 == 0, "the SwiGLU form splits the waves in two");
  constexpr int STAGE = BSTAGE + W * CH + (NESTED ? 0 : W * 256);
  static_assert(16 % W == 0, "activation loads split evenly over the waves");
  constexpr int CPW = 16 / W;
  // one LDS object per ring stage, indexed at compile time (the step body
  // reads one and refills the other)
  __shared__ __align__(16) uint8_t ring0[STAGE];
  __shared__ __align__(16) uint8_t ring1[STAGE];
  __shared__ float2 lut2_s[256];
  __shared__ float code2_s[NESTED ? (SW ? 512 : 256) : 1];
  __shared__ uint8_t a8_s[NESTED ? BM * DL_MAX_STEPS : 1];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int m0 = blockIdx.x * BMO, n0 = blockIdx.y * BN;
  // this wave's weight (SW: the second half of the waves takes w3). The
  // choice is made on the wave index read from one lane, so the compiler
  // knows it is uniform: the weight's buffer resource stays in scalar
  // registers (as a per-lane value it would wrap each load in a loop).
  const bool w3 = SW && __builtin_amdgcn_readfirstlane(wave) >= W / 2;
  const uint8_t* const Wm = w3 ? m3.W : Wt;
  const uint8_t* const A8m = w3 ? m3.A8 : A8;
  const float* const AMm = w3 ? m3.AMAX : AMAX;
  const float offm = w3 ? m3.offset : offset;
  // split-K (gridDim.z > 1): workgroup z takes K-steps [z S, z S + S) and
  // writes fp32 partial sums to YP[z][n][m]
  const int nsteps = K / KT / gridDim.z, kbase = blockIdx.z * nsteps * KT;

  for (int i = tid; i < 256; i += 64 * W) {
    lut2_s[i] = make_float2(LUT[i >> 4], LUT[i & 15]);
    if constexpr (NESTED) code2_s[i] = CODE2[i];
    if constexpr (NESTED && SW) code2_s[256 + i] = m3.CODE2[i];
  }
  // nested: the workgroup's scale bytes, entry r * DL_MAX_STEPS + j for row
  // r, step j; lane l takes step l (steps past the range repeat the last,
  // unread) of rows wave, wave + W, ...; all its loads are issued before the
  // first is stored (a loop that stored each before loading the next paid a
  // memory round trip per entry). Plain scales travel with each step's loads.
  if constexpr (NESTED) {
    static_assert(DL_MAX_STEPS == 64, "one step per lane");
    constexpr int PER = BM / W;  // rows per wave
    const int j = min(lane, nsteps - 1);
    uint32_t v[PER];
#pragma unroll
    for (int u = 0; u < PER; ++u) {
      const int vr = wave + u * W;  // (SW: rows BMO .. BM - 1 are w3's)
      const bool second = SW && vr >= BMO;
      const int row = min(m0 + vr - (second ? BMO : 0), M - 1);
      v[u] = (second ? m3.A8 : A8)[((long long)row * K + kbase + j * KT) >> bs_shift];
    }
#pragma unroll
    for (int u = 0; u < PER; ++u) a8_s[(wave + u * W) * DL_MAX_STEPS + lane] = (uint8_t)v[u];
  }
  // this lane's weight row; nested: its second-level scale for the steps
  // before jsw and from jsw on (a workgroup's K range crosses at most one
  // second-level group: 64 steps of 64 codes < one group of >= 256 blocks)
  const int rl = 32 * wave + (lane & 31);
  const int arow = min(m0 + rl - (w3 ? BMO : 0), M - 1);
  float amax_lo = 0.0f, amax_hi = 0.0f;
  int jsw = nsteps;
  if constexpr (NESTED) {
    const long long e0 = (long long)arow * K + kbase;
    const long long g0 = (e0 >> bs_shift) >> bs2_shift;
    amax_lo = AMm[g0];
    const long long enext = ((g0 + 1) << bs2_shift) << bs_shift;  // first element of the next group
    jsw = (int)min((long long)nsteps, (enext - e0 + KT - 1) / KT);
    amax_hi = jsw < nsteps ? AMm[g0 + 1] : amax_lo;
  }

  const __amdgpu_buffer_rsrc_t xr =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(X), (short)0, (int)((size_t)N * K * 2), 0x00020000);
  const __amdgpu_buffer_rsrc_t wr =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(Wm), (short)0, (int)((size_t)M * K / 2), 0x00020000);
  // activation load j of this wave: rows 8 q .. 8 q + 7 (q = wave CPW + j),
  // lane l row 8 q + l / 8 and LDS slot l % 8, i.e. segment (l % 8) ^ ((t >> 1) & 7)
  uint32_t xoff[CPW];
#pragma unroll
  for (int j = 0; j < CPW; ++j) {
    const int t = 8 * (wave * CPW + j) + (lane >> 3);
    const int sg = (lane & 7) ^ ((t >> 1) & 7);
    xoff[j] = (uint32_t)min(n0 + t, N - 1) * (uint32_t)K * 2u + (uint32_t)sg * 16u;
  }
  // this wave's code load: lane l row l % 32, bytes 16 (l / 32) .. of the step's 32
  const uint32_t woff = (uint32_t)arow * (uint32_t)(K / 2) + 16u * (lane >> 5);
  // plain: lane l's absmax of row l % 32 (block (row K + k) >> bs_shift: the
  // row's part per lane, the step's part uniform, both whole blocks)
  const __amdgpu_buffer_rsrc_t ar = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<float*>(AMm), (short)0, NESTED ? 0 : (int)(((size_t)M * K >> bs_shift) * 4), 0x00020000);
  const uint32_t aoff = (uint32_t)(((long long)arow * K) >> bs_shift) * 4u;

  f32x16_v acc[4];
#pragma unroll
  for (int b = 0; b < 4; ++b)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[b][r] = 0.0f;

  __syncthreads();  // tables
  {
    const int k0 = kbase;
#pragma unroll
    for (int j = 0; j < CPW; ++j)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(xr, (lds_ptr_t)(ring0 + (wave * CPW + j) * CH), 16, xoff[j], k0 * 2, 0,
                                               0);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(wr, (lds_ptr_t)(ring0 + BSTAGE + wave * CH), 16, woff, k0 / 2, 0, 0);
    if constexpr (!NESTED)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(ar, (lds_ptr_t)(ring0 + BSTAGE + W * CH + wave * 256), 4, aoff,
                                               (k0 >> bs_shift) * 4, 0, 0);
  }
  // step s (stage s % 2): its loads were issued one step before
  auto one = [&](int s, uint8_t* rd, uint8_t* dst) {
    TTSP_VMWAIT(0);
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    const int k0n = kbase + min(s + 1, nsteps - 1) * KT;  // the last step reloads itself, unread
    float sc = 0.0f;  // plain: read inside the step
    if constexpr (NESTED) {
      const float am = s < jsw ? amax_lo : amax_hi;
      sc = __fadd_rn(__fmul_rn(code2_s[(w3 ? 256 : 0) + a8_s[rl * DL_MAX_STEPS + s]], am), offm);
    }
    dl_step<DT, W, CPW, !NESTED>(rd, dst, lut2_s, xr, wr, ar, xoff, woff, aoff, k0n * 2, k0n / 2,
                                 (k0n >> bs_shift) * 4, wave, lane, sc, acc);
  };
  int s0 = 0;
  for (; s0 + 2 <= nsteps; s0 += 2) {  // no branch inside: the compiler's own wait counts stay exact
    one(s0, ring0, ring1);
    one(s0 + 1, ring1, ring0);
  }
  if (s0 < nsteps) one(s0, ring0, ring1);
  TTSP_VMWAIT(0);

  // accumulator r of lane l is (row 8 (r / 4) + 4 (l / 32) + r % 4, column
  // l % 32): 4 consecutive weight rows m of one activation row n per lane
  const bool v4 = (M & 3) == 0;
  if constexpr (SW) {
    // the gate waves' outputs, rounded, to LDS - in the stage the last step
    // read (free once every wave is past it; the other stage takes that
    // step's unread refill) - then w3's waves combine them with their own
    static_assert((W / 2) * 4 * 16 * 64 * 2 <= STAGE, "gate outputs exceed the ring stage");
    uint16_t* g_s = reinterpret_cast<uint16_t*>(nsteps % 2 == 0 ? ring1 : ring0);  // [W / 2][4][16][64]
    const int hw = w3 ? wave - W / 2 : wave;
    __syncthreads();
    if (!w3) {
#pragma unroll
      for (int b = 0; b < 4; ++b)
#pragma unroll
        for (int r = 0; r < 16; ++r) g_s[((hw * 4 + b) * 16 + r) * 64 + lane] = Elem<DT>::store(acc[b][r]);
    }
    __syncthreads();
    if (!w3) return;
    const bool vec = v4 && (epi & 8);  // Y 8-byte aligned (host)
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      const int n = n0 + 32 * b + (lane & 31);
      if (n >= N) continue;
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int m = m0 + 32 * hw + 8 * g + 4 * (lane >> 5);
        const size_t o = (size_t)n * M + m;
        uint16_t ov[4];
#pragma unroll
        for (int c = 0; c < 4; ++c)
          ov[c] = dl_epi<DT>(Elem<DT>::load(Elem<DT>::store(acc[b][4 * g + c])),
                             g_s[((hw * 4 + b) * 16 + 4 * g + c) * 64 + lane], 2);
        if (vec && m + 4 <= M) {
          *reinterpret_cast<uint2*>(Y + o) =
              make_uint2((uint32_t)ov[0] | ((uint32_t)ov[1] << 16), (uint32_t)ov[2] | ((uint32_t)ov[3] << 16));
        } else {
          for (int c = 0; c < 4 && m + c < M; ++c) Y[o + c] = ov[c];
        }
      }
    }
    return;
  }
  // Two-wave tiles' outputs leave as whole rows: staged as [n][m] in the
  // stage the last step read (no load refills it; the other stage takes that
  // step's unread refill, which is not written into) and stored 16 bytes a
  // lane, so each store instruction writes whole 128-byte lines of output
  // rows instead of 8- or 16-byte pieces of 32 rows.
  uint8_t* const rd_last = nsteps % 2 == 0 ? ring1 : ring0;
  if constexpr (W == 2) {
    __syncthreads();
    if (YP) {
      // fp32 partials, 64 activation rows at a time (a 64 x 64 block at a
      // 68-float row pitch fills the stage): both waves stage, then store
      constexpr int FR = 68;
      static_assert(64 * FR * 4 <= STAGE, "the partial block exceeds the ring stage");
      float* f_s = reinterpret_cast<float*>(rd_last);
      float* yp = YP + (size_t)blockIdx.z * N * M;
#pragma unroll
      for (int half = 0; half < 2; ++half) {
#pragma unroll
        for (int bb = 0; bb < 2; ++bb)
#pragma unroll
          for (int g = 0; g < 4; ++g) {
            const int b = 2 * half + bb;
            *reinterpret_cast<float4*>(f_s + (32 * bb + (lane & 31)) * FR + 32 * wave + 8 * g + 4 * (lane >> 5)) =
                make_float4(acc[b][4 * g], acc[b][4 * g + 1], acc[b][4 * g + 2], acc[b][4 * g + 3]);
          }
        __syncthreads();
#pragma unroll
        for (int k = 0; k < 64 * 64 / 4 / 128; ++k) {
          const int e = tid + 128 * k, nl = e >> 4, ml = (e & 15) * 4;
          const int n = n0 + 64 * half + nl, m = m0 + ml;
          if (n < N) {
            const float4 v = *reinterpret_cast<const float4*>(f_s + nl * FR + ml);
            const size_t o = (size_t)n * M + m;
            if (v4 && m + 4 <= M) {
              *reinterpret_cast<float4*>(yp + o) = v;
            } else {
              const float vv[4] = {v.x, v.y, v.z, v.w};
              for (int c = 0; c < 4 && m + c < M; ++c) yp[o + c] = vv[c];
            }
          }
        }
        __syncthreads();  // the block's reads before the next half's writes
      }
      return;
    }
    // the rounded outputs at a 72-element row pitch (both waves' 32 columns)
    constexpr int HR = 72;
    static_assert(BN * HR * 2 <= STAGE, "the output block exceeds the ring stage");
    uint16_t* h_s = reinterpret_cast<uint16_t*>(rd_last);
#pragma unroll
    for (int b = 0; b < 4; ++b)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const uint32_t lo = (uint32_t)Elem<DT>::store(acc[b][4 * g]) | ((uint32_t)Elem<DT>::store(acc[b][4 * g + 1]) << 16);
        const uint32_t hi =
            (uint32_t)Elem<DT>::store(acc[b][4 * g + 2]) | ((uint32_t)Elem<DT>::store(acc[b][4 * g + 3]) << 16);
        *reinterpret_cast<uint2*>(h_s + (32 * b + (lane & 31)) * HR + 32 * wave + 8 * g + 4 * (lane >> 5)) =
            make_uint2(lo, hi);
      }
    __syncthreads();
    const int ep = epi & 3;
    const bool vec = (M & 7) == 0 && (epi & 16);  // rows of Y and R 16-byte aligned (host: Y, R)
#pragma unroll
    for (int k = 0; k < BN * 64 / 8 / 128; ++k) {
      const int e = tid + 128 * k, nl = e >> 3, ml = (e & 7) * 8;
      const int n = n0 + nl, m = m0 + ml;
      if (n >= N) continue;
      const uint4 v = *reinterpret_cast<const uint4*>(h_s + nl * HR + ml);
      const size_t o = (size_t)n * M + m;
      const uint32_t vw[4] = {v.x, v.y, v.z, v.w};
      if (vec && m + 8 <= M) {
        uint4 rv = make_uint4(0u, 0u, 0u, 0u);
        if (ep) rv = *reinterpret_cast<const uint4*>(R + o);
        const uint32_t rw[4] = {rv.x, rv.y, rv.z, rv.w};
        uint32_t owd[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const uint16_t lo = dl_epi<DT>(Elem<DT>::load(vw[q] & 0xffffu), (uint16_t)rw[q], ep);
          const uint16_t hi = dl_epi<DT>(Elem<DT>::load(vw[q] >> 16), (uint16_t)(rw[q] >> 16), ep);
          owd[q] = (uint32_t)lo | ((uint32_t)hi << 16);
        }
        *reinterpret_cast<uint4*>(Y + o) = make_uint4(owd[0], owd[1], owd[2], owd[3]);
      } else {
        for (int c = 0; c < 8 && m + c < M; ++c)
          Y[o + c] = dl_epi<DT>(Elem<DT>::load((uint16_t)(vw[c >> 1] >> (16 * (c & 1)))), ep ? R[o + c] : (uint16_t)0,
                                ep);
      }
    }
    return;
  }
  if (YP) {
    float* yp = YP + (size_t)blockIdx.z * N * M;
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      const int n = n0 + 32 * b + (lane & 31);
      if (n >= N) continue;
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int m = m0 + 32 * wave + 8 * g + 4 * (lane >> 5);
        if (v4 && m + 4 <= M) {
          *reinterpret_cast<float4*>(yp + (size_t)n * M + m) =
              make_float4(acc[b][4 * g], acc[b][4 * g + 1], acc[b][4 * g + 2], acc[b][4 * g + 3]);
        } else {
          for (int c = 0; c < 4 && m + c < M; ++c) yp[(size_t)n * M + m + c] = acc[b][4 * g + c];
        }
      }
    }
    return;
  }
  const int ep = epi & 3;
  const bool vec = v4 && (epi & 8);  // Y (and R) 8-byte aligned (host)
#pragma unroll
  for (int b = 0; b < 4; ++b) {
    const int n = n0 + 32 * b + (lane & 31);
    if (n >= N) continue;
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int m = m0 + 32 * wave + 8 * g + 4 * (lane >> 5);
      const size_t o = (size_t)n * M + m;
      if (vec && m + 4 <= M) {
        uint32_t rw[2] = {0u, 0u};
        if (ep) {
          const uint2 rv = *reinterpret_cast<const uint2*>(R + o);
          rw[0] = rv.x, rw[1] = rv.y;
        }
        uint32_t ow[2];
#pragma unroll
        for (int q = 0; q < 2; ++q) {
          const uint16_t lo = dl_epi<DT>(Elem<DT>::load(Elem<DT>::store(acc[b][4 * g + 2 * q])), (uint16_t)rw[q], ep);
          const uint16_t hi =
              dl_epi<DT>(Elem<DT>::load(Elem<DT>::store(acc[b][4 * g + 2 * q + 1])), (uint16_t)(rw[q] >> 16), ep);
          ow[q] = (uint32_t)lo | ((uint32_t)hi << 16);
        }
        *reinterpret_cast<uint2*>(Y + o) = make_uint2(ow[0], ow[1]);
      } else {
        for (int c = 0; c < 4 && m + c < M; ++c)
          Y[o + c] = dl_epi<DT>(Elem<DT>::load(Elem<DT>::store(acc[b][4 * g + c])), ep ? R[o + c] : (uint16_t)0, ep);
      }
    }
  }
#endif
}

template <int DT, int W>
int launch_dl(const void* X, const uint8_t* Wt, const uint8_t* A8, const float* AMAX, const float* CODE2,
              float offset, const float* LUT, void* Y, const void* R, int epi, int M, int K, int N, int bs_shift,
              int bs2_shift, int splits, float* YP, hipStream_t st) {
  constexpr int BM = 32 * W;
  const dim3 grid((M + BM - 1) / BM, (N + BN - 1) / BN, splits);
  if (A8)
    hipLaunchKernelGGL((nf4_gemm_dl_kernel<DT, true, W>), grid, dim3(64 * W), 0, st, (const uint16_t*)X, Wt, A8,
                       AMAX, CODE2, offset, LUT, (uint16_t*)Y, (const uint16_t*)R, epi, M, K, N, bs_shift,
                       bs2_shift, YP, DlMat{});
  else
    hipLaunchKernelGGL((nf4_gemm_dl_kernel<DT, false, W>), grid, dim3(64 * W), 0, st, (const uint16_t*)X, Wt, A8,
                       AMAX, CODE2, offset, LUT, (uint16_t*)Y, (const uint16_t*)R, epi, M, K, N, bs_shift,
                       bs2_shift, YP, DlMat{});
  TTSP_RETURN_LAUNCH();
}

// The SwiGLU form: 4 waves, 64 output rows of both weights a workgroup.
template <int DT>
int launch_dl_swiglu(const void* X, const uint8_t* W1, const uint8_t* A8, const float* AMAX, const float* CODE2,
                     float offset, const DlMat& m3, const float* LUT, void* Y, int epi, int M, int K, int N,
                     int bs_shift, int bs2_shift, hipStream_t st) {
  constexpr int W = 4, BMO = 32 * W / 2;
  const dim3 grid((M + BMO - 1) / BMO, (N + BN - 1) / BN, 1);
  if (A8)
    hipLaunchKernelGGL((nf4_gemm_dl_kernel<DT, true, W, true>), grid, dim3(64 * W), 0, st, (const uint16_t*)X, W1,
                       A8, AMAX, CODE2, offset, LUT, (uint16_t*)Y, (const uint16_t*)nullptr, epi, M, K, N, bs_shift,
                       bs2_shift, (float*)nullptr, m3);
  else
    hipLaunchKernelGGL((nf4_gemm_dl_kernel<DT, false, W, true>), grid, dim3(64 * W), 0, st, (const uint16_t*)X, W1,
                       A8, AMAX, CODE2, offset, LUT, (uint16_t*)Y, (const uint16_t*)nullptr, epi, M, K, N, bs_shift,
                       bs2_shift, (float*)nullptr, m3);
  TTSP_RETURN_LAUNCH();
}

}  // namespace

// Whether the kernel takes this launch: whole K-steps per split, at most
// DL_MAX_STEPS of them, byte offsets of X and W below 2^31.
bool gemm_dl_fits(int M, int K, int N, int splits) {
  if (splits < 1 || K % KT || (K / KT) % splits || K / KT / splits > DL_MAX_STEPS) return false;
  return (long long)N * K * 2 < (1ll << 31) && (long long)M * K / 2 < (1ll << 31);
}

// waves: 2 (64 weight rows a workgroup) or 4 (128). splits > 1 writes fp32
// partials to YP (the caller reduces them and applies the epilogue); else
// epi as nf4_gemm_kernel's (bit 2: vectorised output; 8- and 16-byte
// alignment of Y and R is checked here).
int gemm_dl(const void* X, int dt, const uint8_t* W, const uint8_t* A8, const float* AMAX, const float* CODE2,
            float offset, const float* LUT, void* Y, const void* R, int epi, int M, int K, int N, int bs_shift,
            int bs2_shift, int waves, int splits, float* YP, hipStream_t st) {
  if (!gemm_dl_fits(M, K, N, splits) || (splits > 1 && !YP)) return (int)hipErrorInvalidValue;
  const bool al8 = (uintptr_t)Y % 8 == 0 && (!(epi & 3) || (uintptr_t)R % 8 == 0);
  const bool al16 = (uintptr_t)Y % 16 == 0 && (!(epi & 3) || (uintptr_t)R % 16 == 0);
  const int e = (epi & 3) | (al8 ? 8 : 0) | (al16 ? 16 : 0);
  float* yp = splits > 1 ? YP : nullptr;
  if (dt == DT_BF16) {
    if (waves == 2)
      return launch_dl<DT_BF16, 2>(X, W, A8, AMAX, CODE2, offset, LUT, Y, R, e, M, K, N, bs_shift, bs2_shift, splits,
                                   yp, st);
    return launch_dl<DT_BF16, 4>(X, W, A8, AMAX, CODE2, offset, LUT, Y, R, e, M, K, N, bs_shift, bs2_shift, splits,
                                 yp, st);
  }
  if (dt == DT_F16) {
    if (waves == 2)
      return launch_dl<DT_F16, 2>(X, W, A8, AMAX, CODE2, offset, LUT, Y, R, e, M, K, N, bs_shift, bs2_shift, splits,
                                  yp, st);
    return launch_dl<DT_F16, 4>(X, W, A8, AMAX, CODE2, offset, LUT, Y, R, e, M, K, N, bs_shift, bs2_shift, splits,
                                yp, st);
  }
  return (int)hipErrorInvalidValue;
}

// Y = round(round(silu(X . W1^T)) * round(X . W3^T)) in one unsplit launch
// (the two launches' bits where they run this kernel unsplit: the caller
// checks the plan). Both weights share blocksize and nesting.
int gemm_dl_swiglu(const void* X, int dt, const uint8_t* W1, const uint8_t* A8_1, const float* AMAX_1,
                   const float* CODE2_1, float offset_1, const uint8_t* W3, const uint8_t* A8_3,
                   const float* AMAX_3, const float* CODE2_3, float offset_3, const float* LUT, void* Y, int M, int K,
                   int N, int bs_shift, int bs2_shift, hipStream_t st) {
  if (!gemm_dl_fits(M, K, N, 1)) return (int)hipErrorInvalidValue;
  const DlMat m3{W3, A8_3, AMAX_3, CODE2_3, offset_3};
  const int e = (uintptr_t)Y % 8 == 0 ? 8 : 0;
  if (dt == DT_BF16)
    return launch_dl_swiglu<DT_BF16>(X, W1, A8_1, AMAX_1, CODE2_1, offset_1, m3, LUT, Y, e, M, K, N, bs_shift,
                                     bs2_shift, st);
  if (dt == DT_F16)
    return launch_dl_swiglu<DT_F16>(X, W1, A8_1, AMAX_1, CODE2_1, offset_1, m3, LUT, Y, e, M, K, N, bs_shift,
                                    bs2_shift, st);
  return (int)hipErrorInvalidValue;
}

}  // namespace ttsp
