// Device helpers shared by the NF4 GEMV (nf4_gemv.hip) and the persistent
// fast-transformer step (fast_step.hip): the replicated code-pair table, the
// 16-bit conversions, the fork's epilogue roundings, the folded RMSNorm's
// chunk arithmetic, and the attention-prologue LDS layout. Both kernels use
// these so their results are the same bits.
#pragma once
#include "attn_common.h"

namespace ttsp {

constexpr int LUT_REP = 64;                    // table copies, one per lane
constexpr int LUT_BYTES = 256 * LUT_REP * 4;   // 64 KiB
constexpr int GEMV_WAVES = 8;                  // waves per workgroup
constexpr int GEMV_THREADS = GEMV_WAVES * 64;

// LDS of the attention prologue after x: q [8][128] fp32, p [8][64] fp32,
// then per kv head R16 staged K rows (KPAD stride) and R16 V rows, R16 the
// cache length rounded up to 16 (the PV loop reads rows 16 at a time).
static constexpr int ATT_MAX_HEADS = 8;
__host__ __device__ constexpr int att_r16(int max_len) { return (max_len + 15) & ~15; }
__host__ __device__ constexpr size_t att_lds(int nkv, int max_len) {
  return 4 * (size_t)ATT_MAX_HEADS * (HD + ACHUNK) + 2 * (size_t)nkv * att_r16(max_len) * (KPAD + HD);
}
constexpr int ATT_PER = 4;  // staged 16-byte pieces per thread: nkv * R16 * 16 <= 4 * 512

__device__ __forceinline__ int uniform(int v) { return __builtin_amdgcn_readfirstlane(v); }

__device__ __forceinline__ float ld16(int dt, uint32_t h) {
  return dt == DT_BF16 ? bf16_to_f32(h & 0xffffu) : f16_to_f32(h & 0xffffu);
}
__device__ __forceinline__ uint32_t st16(int dt, float f) {
  return dt == DT_BF16 ? f32_to_bf16(f) : f32_to_f16(opaque(f));
}

// Output rounding as the unfused fork: the matmul result is rounded to the
// activation type, and so is each elementwise op after it (app/engine/
// nf4gemv.py:215-226): residual y' = round(R + y), gate y' = round(round(silu(R)) * y).
__device__ __forceinline__ uint16_t epilogue16(int dt, float acc, int epi, uint32_t r) {
  const float y = ld16(dt, st16(dt, acc));
  float o = y;
  if (epi == 1) o = __fadd_rn(ld16(dt, r), y);
  else if (epi == 2) o = __fmul_rn(ld16(dt, st16(dt, silu_rn(ld16(dt, r)))), y);
  return (uint16_t)st16(dt, o);
}

// Per-type steps on 8-value chunks (uint4 of 16-bit elements).
template <int DT>
__device__ __forceinline__ float sumsq8(uint4 v, float acc) {  // element order, fma chain
  const uint32_t u[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const float a = Elem<DT>::load(u[k]), b = Elem<DT>::load(u[k] >> 16);
    acc = __builtin_fmaf(a, a, acc);
    acc = __builtin_fmaf(b, b, acc);
  }
  return acc;
}

// The fork's RMSNorm of 8 values: round(round(x * r) * w), the standalone kernel's arithmetic.
template <int DT>
__device__ __forceinline__ uint4 norm8(uint4 v, uint4 g, float r) {
  uint32_t u[4] = {v.x, v.y, v.z, v.w};
  const uint32_t gw[4] = {g.x, g.y, g.z, g.w};
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const float n0 = Elem<DT>::load(Elem<DT>::store(__fmul_rn(Elem<DT>::load(u[k]), r)));
    const float n1 = Elem<DT>::load(Elem<DT>::store(__fmul_rn(Elem<DT>::load(u[k] >> 16), r)));
    u[k] = (uint32_t)Elem<DT>::store(__fmul_rn(n0, Elem<DT>::load(gw[k]))) |
           ((uint32_t)Elem<DT>::store(__fmul_rn(n1, Elem<DT>::load(gw[k] >> 16))) << 16);
  }
  return make_uint4(u[0], u[1], u[2], u[3]);
}

struct F8 {
  float v[8];
};

template <int DT>
__device__ __forceinline__ F8 to_f32(uint4 c) {
  const uint32_t u[4] = {c.x, c.y, c.z, c.w};
  F8 o;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    o.v[2 * k] = Elem<DT>::load(u[k]);
    o.v[2 * k + 1] = Elem<DT>::load(u[k] >> 16);
  }
  return o;
}

// The replicated code-pair table: entry e (a weight byte, two codes) of lane
// l at byte 256 e + 4 l holds fp16(code[e >> 4]) | fp16(code[e & 15]) << 16,
// so the 64 lanes of a lookup hit 64 different banks.
__device__ __forceinline__ uint32_t code_pair_entry(const float* code, int e) {
  return (uint32_t)f32_to_f16(code[e >> 4]) | ((uint32_t)f32_to_f16(code[e & 15]) << 16);
}

}  // namespace ttsp
