// Device-side helpers shared by every kernel of libttsp_hip.so (gfx950 only).
//
// Element types travel as raw 16-bit patterns (uint16_t) so one kernel body
// serves fp16 and bf16; the arithmetic type is fp32 throughout.
//
// Every floating-point operation whose rounding matters is spelled out:
// the library is compiled with -ffp-contract=off, fused multiply-adds are
// written as __builtin_fmaf where they are meant, and the two transcendental
// functions the decode path needs (exp, sqrt) are the deterministic routines
// below rather than the hardware approximations, so a CPU restatement that
// performs the same IEEE operations in the same order reproduces every bit.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>

namespace ttsp {

enum : int { DT_F16 = 0, DT_BF16 = 1, DT_F32 = 2 };

// Plain vector types for 16-byte values held in registers (HIP's uint4 is a
// union-backed struct that can keep a small local array out of registers).
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float bf16_to_f32(uint32_t h) { return __uint_as_float(h << 16); }

// Round to nearest even; NaN stays a (quiet) NaN.
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

__device__ __forceinline__ float f16_to_f32(uint32_t h) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)h);
}

// v_cvt_f16_f32: round to nearest even, overflow to inf, subnormals kept.
__device__ __forceinline__ uint16_t f32_to_f16(float f) {
  return __builtin_bit_cast(uint16_t, (_Float16)f);
}

template <int DT> struct Elem;

// Rounding to a 16-bit type happens exactly where the source says, from an
// fp32 value: `opaque` hides the value's origin from instruction selection,
// which would otherwise fuse a preceding fp32 multiply into the conversion
// (v_fma_mixlo_f16: one rounding of the exact product instead of two).
__device__ __forceinline__ float opaque(float f) {
  asm("" : "+v"(f));
  return f;
}

template <> struct Elem<DT_F16> {
  __device__ static __forceinline__ float load(uint32_t h) { return f16_to_f32(h & 0xffffu); }
  __device__ static __forceinline__ uint16_t store(float f) { return f32_to_f16(opaque(f)); }
};

template <> struct Elem<DT_BF16> {
  __device__ static __forceinline__ float load(uint32_t h) { return bf16_to_f32(h & 0xffffu); }
  __device__ static __forceinline__ uint16_t store(float f) { return f32_to_bf16(f); }
};

// Halves of a packed fp16 pair as fp32 (exact). Fed to fmaf, they select
// v_fma_mix_f32 with op_sel: an IEEE fma on fp16 operands, one instruction.
__device__ __forceinline__ float h_lo(uint32_t u) { return f16_to_f32(u & 0xffffu); }
__device__ __forceinline__ float h_hi(uint32_t u) { return f16_to_f32(u >> 16); }

__device__ __forceinline__ float load_elem(const void* p, size_t i, int dt) {
  if (dt == DT_F32) return ((const float*)p)[i];
  const uint32_t h = ((const uint16_t*)p)[i];
  return dt == DT_F16 ? f16_to_f32(h) : bf16_to_f32(h);
}

// Correctly rounded square root of a positive normal float.
// v_sqrt_f32 is within 1 ulp; the two fma residual tests below move it to the
// neighbour that brackets the exact root (the standard fix-up for a faithful
// estimate), so the result equals IEEE sqrtf.
__device__ __forceinline__ float sqrt_rn(float x) {
  const float s0 = __builtin_amdgcn_sqrtf(x);
  const float down = __uint_as_float(__float_as_uint(s0) - 1u);
  const float up = __uint_as_float(__float_as_uint(s0) + 1u);
  const float below = __builtin_fmaf(-down, s0, x);
  const float above = __builtin_fmaf(-up, s0, x);
  float s = s0;
  if (below <= 0.0f) s = down;
  if (above > 0.0f) s = up;
  return s;
}

// 1 / sqrt(x), two IEEE operations: correctly rounded sqrt, then a correctly
// rounded divide (HIP's '/' on float lowers to the exact division sequence).
__device__ __forceinline__ float rsqrt_rn(float x) { return __fdiv_rn(1.0f, sqrt_rn(x)); }

// exp(x) by Cody-Waite reduction and the Cephes single-precision polynomial
// (S. L. Moshier, Cephes Math Library, expf.c): x = n ln2 + r, |r| <= ln2/2,
// e^r = 1 + r + r^2 P(r), then scaled by 2^n. Every step is an IEEE mul, add
// or fma, so the same sequence on a CPU gives the same bits. Max error ~2 ulp.
// Inputs below -87 return 0, so no result is subnormal (exp(-87) ~ 1.6e-38).
__device__ __forceinline__ float exp_cw(float x) {
  if (x > 88.72283935546875f) return __uint_as_float(0x7f800000u);
  if (x < -87.0f) return 0.0f;
  const float n = __builtin_rintf(__fmul_rn(x, 1.44269502162933349609375f));
  float r = __builtin_fmaf(n, -0.693359375f, x);
  r = __builtin_fmaf(n, 2.12194440e-4f, r);
  const float z = __fmul_rn(r, r);
  float p = 1.9875691500e-4f;
  p = __builtin_fmaf(p, r, 1.3981999507e-3f);
  p = __builtin_fmaf(p, r, 8.3334519073e-3f);
  p = __builtin_fmaf(p, r, 4.1665795894e-2f);
  p = __builtin_fmaf(p, r, 1.6666665459e-1f);
  p = __builtin_fmaf(p, r, 5.0000001201e-1f);
  p = __builtin_fmaf(p, z, r);
  p = __fadd_rn(p, 1.0f);
  return __builtin_ldexpf(p, (int)n);
}

// silu(a) = a / (1 + exp(-a)), each step one IEEE rounding.
__device__ __forceinline__ float silu_rn(float a) {
  return __fdiv_rn(a, __fadd_rn(1.0f, exp_cw(-a)));
}

// v + (v of the DPP partner); rows outside ROWS add +0 and are not read after.
template <int CTRL, int ROWS>
__device__ __forceinline__ float dpp_add(float v) {
  return __fadd_rn(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, ROWS, 0xF, false)));
}

// Sum over the 64 lanes with the partner distance rising: the xor 1, 2, 4, 8
// butterfly inside each 16-lane row (quad_perm, then half-mirror and mirror,
// which pair the same partial sums as xor 4 and 8), then row sums r1 += r0,
// r3 += r2 and r3 += r1 by row broadcasts: lane 63 holds (r3 + r2) + (r1 + r0),
// the same bits as the xor 16, 32 steps. The result is wave-uniform.
__device__ __forceinline__ float wave_sum_dpp(float v) {
  v = dpp_add<0xB1, 0xF>(v);
  v = dpp_add<0x4E, 0xF>(v);
  v = dpp_add<0x141, 0xF>(v);
  v = dpp_add<0x140, 0xF>(v);
  v = dpp_add<0x142, 0xA>(v);
  v = dpp_add<0x143, 0xC>(v);
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

}  // namespace ttsp

// Launch-error plumbing for the extern "C" entry points: each returns the
// hipError_t of its launch (0 on success) and never allocates.
#define TTSP_RETURN_LAUNCH() return (int)hipGetLastError()
