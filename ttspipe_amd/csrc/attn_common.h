// Attention helpers shared by the attention kernels (fusedlayer.hip) and the
// NF4 GEMV's attention prologue (nf4_gemv.hip): one 128-wide head per wave,
// fixed operation orders (the oracle restates them), LDS-staged K/V rows.
#pragma once

#include "ttsp_common.h"

namespace ttsp {

constexpr int HD = 128;        // head dim
constexpr int ACHUNK = 64;     // positions per attention chunk
// LDS row stride of the staged K rows (elements): 272 bytes, so rows are
// 16-byte aligned and the 16 lanes of a 16-byte read hit 64 distinct banks.
constexpr int KPAD = HD + 8;

// Max over the wave by DPP steps and row broadcasts (exact in any order);
// the result is wave-uniform.
__device__ __forceinline__ float wave_max_u(float v) {
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(v), __float_as_int(v), 0xB1, 0xF, 0xF, false)));
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(v), __float_as_int(v), 0x4E, 0xF, 0xF, false)));
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(v), __float_as_int(v), 0x141, 0xF, 0xF, false)));
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(v), __float_as_int(v), 0x140, 0xF, 0xF, false)));
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(v), __float_as_int(v), 0x142, 0xA, 0xF, false)));
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(v), __float_as_int(v), 0x143, 0xC, 0xF, false)));
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

// q . k of one position: four fma chains over the element pairs i = c, c + 4,
// ... (pair i = elements 2i, 2i + 1 in order), then (s0 + s1) + (s2 + s3).
// qg (the wave's query, broadcast) and kr (this lane's K row) are LDS rows,
// read 16 bytes at a time; each 32-element block's reads are issued together.
template <int DT>
__device__ __forceinline__ float score4(const float* __restrict__ qg, const uint16_t* __restrict__ kr) {
  const f32x4* q4 = reinterpret_cast<const f32x4*>(qg);
  const u32x4* k4 = reinterpret_cast<const u32x4*>(kr);
  float a[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int b = 0; b < HD / 32; ++b) {
    u32x4 kk[4];
    f32x4 qq[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) kk[i] = k4[4 * b + i];
#pragma unroll
    for (int i = 0; i < 8; ++i) qq[i] = q4[8 * b + i];
#pragma unroll
    for (int t = 0; t < 16; ++t) {  // pair i = 16 b + t
      const uint32_t k2 = kk[t >> 2][t & 3];
      const f32x4 q = qq[t >> 1];
      const float qa = (t & 1) ? q[2] : q[0], qb = (t & 1) ? q[3] : q[1];
      a[t & 3] = __builtin_fmaf(qa, Elem<DT>::load(k2), a[t & 3]);
      a[t & 3] = __builtin_fmaf(qb, Elem<DT>::load(k2 >> 16), a[t & 3]);
    }
  }
  return __fadd_rn(__fadd_rn(a[0], a[1]), __fadd_rn(a[2], a[3]));
}

// p . V for dims 2 lane, 2 lane + 1: four fma chains over the positions
// j = c, c + 4, ... below nvalid, then (a0 + a1) + (a2 + a3). pg is the
// wave's own probability row (LDS, broadcast), v_s the staged V rows; each
// block of 16 positions has its reads issued together.
template <int DT>
__device__ __forceinline__ void pv4(const float* __restrict__ pg, const uint16_t* __restrict__ v_s, int nvalid,
                                    int lane, float& y0, float& y1) {
  float a[4] = {0.0f, 0.0f, 0.0f, 0.0f}, b[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  const uint32_t* vcol = reinterpret_cast<const uint32_t*>(v_s) + lane;
  const f32x4* p4 = reinterpret_cast<const f32x4*>(pg);
#pragma unroll
  for (int jb = 0; jb < ACHUNK; jb += 16) {
    if (jb >= nvalid) break;
    uint32_t vv[16];
    f32x4 pp[4];
#pragma unroll
    for (int t = 0; t < 16; ++t) vv[t] = vcol[(jb + t) * (HD / 2)];
#pragma unroll
    for (int t = 0; t < 4; ++t) pp[t] = p4[jb / 4 + t];
    if (jb + 16 <= nvalid) {
#pragma unroll
      for (int t = 0; t < 16; ++t) {
        const float pj = pp[t >> 2][t & 3];
        a[t & 3] = __builtin_fmaf(pj, Elem<DT>::load(vv[t]), a[t & 3]);
        b[t & 3] = __builtin_fmaf(pj, Elem<DT>::load(vv[t] >> 16), b[t & 3]);
      }
    } else {
#pragma unroll
      for (int t = 0; t < 16; ++t) {
        if (jb + t < nvalid) {
          const float pj = pp[t >> 2][t & 3];
          a[t & 3] = __builtin_fmaf(pj, Elem<DT>::load(vv[t]), a[t & 3]);
          b[t & 3] = __builtin_fmaf(pj, Elem<DT>::load(vv[t] >> 16), b[t & 3]);
        }
      }
    }
  }
  y0 = __fadd_rn(__fadd_rn(a[0], a[1]), __fadd_rn(a[2], a[3]));
  y1 = __fadd_rn(__fadd_rn(b[0], b[1]), __fadd_rn(b[2], b[3]));
}

// Rotary factors of the pair that holds lanes l and l + 64 of a head: the
// pair's (cos, sin) for the low half, then for the high half.
struct RopeF {
  float rl, il, rh, ih;
};
// Branch-free: the pair is one dword of a 16-bit table or two of an fp32 one,
// so every lane issues the same two dword loads per half whatever ftype is.
__device__ __forceinline__ RopeF load_rope(const void* __restrict__ F, int ftype, int lane) {
  const uint32_t* fw = reinterpret_cast<const uint32_t*>(F);
  const int es = ftype == DT_F32 ? 1 : 0;
  const int e = lane & ~1;  // the pair's even element (lo half; the hi half is e + 64)
  const int wl = (e << es) >> 1, wh = ((e + 64) << es) >> 1;
  const uint32_t l0 = fw[wl], l1 = fw[wl + es], h0 = fw[wh], h1 = fw[wh + es];
  const bool f16 = ftype == DT_F16;
  // all three decodings computed, one selected (no branch on the loaded data)
  auto dec = [&](uint32_t a, uint32_t b, bool second) {
    const uint32_t h = second ? a >> 16 : a & 0xffffu;
    const float x16 = f16_to_f32(h), xb = __uint_as_float(h << 16), x32 = __uint_as_float(second ? b : a);
    return es ? x32 : (f16 ? x16 : xb);
  };
  return RopeF{dec(l0, l1, false), dec(l0, l1, true), dec(h0, h1, false), dec(h0, h1, true)};
}

// Head norm and rotary of one 128-wide head held by a wave (lane l: elements
// l and l + 64), used by every kernel that writes q/k heads: the norm's sum is
// the two 64-element halves (rising DPP sums) added, one rounding after x * r * w;
// rotary pairs (2i, 2i+1) with the partner in lane l ^ 1, separately rounded
// products and sum. Returns the rotated values, not yet rounded. nwl, nwh
// are the norm weights of elements l and l + 64 (unused when norm is false).
template <int DT>
__device__ __forceinline__ void head_norm_rope(float& lo, float& hi, bool norm, uint16_t nwl, uint16_t nwh,
                                               float eps, const RopeF& f, int lane) {
  if (norm) {
    const float ss = __fadd_rn(wave_sum_dpp(__fmul_rn(lo, lo)), wave_sum_dpp(__fmul_rn(hi, hi)));
    const float r = rsqrt_rn(__fadd_rn(__fdiv_rn(ss, (float)HD), eps));
    lo = Elem<DT>::load(Elem<DT>::store(__fmul_rn(__fmul_rn(lo, r), Elem<DT>::load(nwl))));
    hi = Elem<DT>::load(Elem<DT>::store(__fmul_rn(__fmul_rn(hi, r), Elem<DT>::load(nwh))));
  }
  const float plo = __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(lo), 0xB1, 0xF, 0xF, false));
  const float phi = __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(hi), 0xB1, 0xF, 0xF, false));
  const float frl = f.rl, fil = f.il, frh = f.rh, fih = f.ih;
  if (lane & 1) {
    lo = __fadd_rn(__fmul_rn(lo, frl), __fmul_rn(plo, fil));
    hi = __fadd_rn(__fmul_rn(hi, frh), __fmul_rn(phi, fih));
  } else {
    lo = __fsub_rn(__fmul_rn(lo, frl), __fmul_rn(plo, fil));
    hi = __fsub_rn(__fmul_rn(hi, frh), __fmul_rn(phi, fih));
  }
}

}  // namespace ttsp
