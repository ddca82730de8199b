/*
 * CPU oracle for the NF4 decode hot path. TEST INFRASTRUCTURE ONLY: nothing in
 * the product (ttspipe_amd/) links, loads or calls this; tests, the smoke
 * check and the benchmark's CPU-baseline leg do, as the checker.
 *
 * Two kinds of function:
 *   *_ref   the reference's arithmetic with fp64 accumulation - the bar the
 *           kernels' results are held to within tolerance;
 *   *_emul  the same arithmetic with the kernels' documented fixed reduction
 *           order, so the GPU result must equal it bit for bit (every
 *           operation below is one IEEE-754 fp32 operation; the file is built
 *           with -ffp-contract=off and fmaf() is written where an fma is meant).
 *
 * Citations are into the reference tree (bitNtech/ttspipe).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

enum { DT_F16 = 0, DT_BF16 = 1, DT_F32 = 2 };

/* ---------------------------------------------------------------- rounding */

/* bf16: round to nearest even (app/engine/nf4cpu.py:71-76), NaN kept quiet. */
uint16_t orc_f32_to_bf16(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

float orc_bf16_to_f32(uint16_t h) {
  uint32_t u = (uint32_t)h << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

/* IEEE binary16, round to nearest even, overflow to inf, subnormals kept
 * (the cvt.rn.f16.f32 of app/engine/nvrtc.py:213-217). */
uint16_t orc_f32_to_f16(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  const uint32_t sign = (u >> 16) & 0x8000u;
  const uint32_t absu = u & 0x7fffffffu;
  if (absu > 0x7f800000u) return (uint16_t)(sign | 0x7e00u | ((absu >> 13) & 0x3ffu));
  if (absu >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); /* >= 65520: inf */
  if (absu < 0x38800000u) {                                  /* below 2^-14: subnormal */
    if (absu < 0x33000000u) return (uint16_t)sign;          /* below 2^-25: zero */
    const int e = (int)(absu >> 23);
    const uint32_t m = (absu & 0x7fffffu) | 0x800000u;
    const int shift = 126 - e; /* 14..24 */
    const uint32_t q = m >> shift;
    const uint32_t rem = m & ((1u << shift) - 1u);
    const uint32_t half = 1u << (shift - 1);
    uint32_t r = q + ((rem > half) || (rem == half && (q & 1u)));
    return (uint16_t)(sign | r);
  }
  uint32_t h = ((absu - 0x38000000u) >> 13);
  const uint32_t rem = absu & 0x1fffu;
  h += (rem > 0x1000u) || (rem == 0x1000u && (h & 1u));
  return (uint16_t)(sign | h);
}

float orc_f16_to_f32(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  const uint32_t e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
  uint32_t u;
  if (e == 0) {
    if (m == 0) {
      u = sign;
    } else { /* subnormal: m * 2^-24 */
      float f = (float)m * 5.9604644775390625e-08f;
      memcpy(&u, &f, 4);
      u |= sign;
    }
  } else if (e == 31) {
    u = sign | 0x7f800000u | (m << 13);
  } else {
    u = sign | ((e + 112u) << 23) | (m << 13);
  }
  float f;
  memcpy(&f, &u, 4);
  return f;
}

static inline float ld(const void* p, size_t i, int dt) {
  if (dt == DT_F32) return ((const float*)p)[i];
  const uint16_t h = ((const uint16_t*)p)[i];
  return dt == DT_F16 ? orc_f16_to_f32(h) : orc_bf16_to_f32(h);
}

static inline uint16_t st16(float f, int dt) {
  return dt == DT_F16 ? orc_f32_to_f16(f) : orc_f32_to_bf16(f);
}

static inline float rnd(float f, int dt) { return dt == DT_F32 ? f : ld(&(uint16_t){st16(f, dt)}, 0, dt); }

/* ------------------------------------------------------------ math kernels */

/* exp by Cody-Waite reduction and the Cephes expf polynomial (S. L. Moshier,
 * Cephes Math Library, expf.c), every step an IEEE operation. Inputs below
 * -87 return 0 so results are never subnormal. */
float orc_exp_cw(float x) {
  if (x > 88.72283935546875f) return INFINITY;
  if (x < -87.0f) return 0.0f;
  const float n = rintf(x * 1.44269502162933349609375f);
  float r = fmaf(n, -0.693359375f, x);
  r = fmaf(n, 2.12194440e-4f, r);
  const float z = r * r;
  float p = 1.9875691500e-4f;
  p = fmaf(p, r, 1.3981999507e-3f);
  p = fmaf(p, r, 8.3334519073e-3f);
  p = fmaf(p, r, 4.1665795894e-2f);
  p = fmaf(p, r, 1.6666665459e-1f);
  p = fmaf(p, r, 5.0000001201e-1f);
  p = fmaf(p, z, r);
  p = p + 1.0f;
  return ldexpf(p, (int)n);
}

float orc_rsqrt_rn(float x) { return 1.0f / sqrtf(x); }

/* fma(a.hi, b.hi, fma(a.lo, b.lo, c)) on packed fp16 pairs, IEEE fmaf. */
void orc_fma16_chain(const uint32_t* a, const uint32_t* b, const float* c, int n, float* out) {
  for (int i = 0; i < n; ++i) {
    const float t = fmaf(orc_f16_to_f32((uint16_t)(a[i] & 0xffffu)), orc_f16_to_f32((uint16_t)(b[i] & 0xffffu)), c[i]);
    out[i] = fmaf(orc_f16_to_f32((uint16_t)(a[i] >> 16)), orc_f16_to_f32((uint16_t)(b[i] >> 16)), t);
  }
}

static inline float silu_rn(float a) { return a / (1.0f + orc_exp_cw(-a)); }

/* Sum of 64 lane values as the kernels' xor butterfly with the partner
 * distance rising 1, 2, ..., 32 (their DPP reduction: within 16-lane rows
 * first, then across rows). */
static float butterfly64_up(float* v) {
  for (int off = 1; off <= 32; off <<= 1) {
    float t[64];
    for (int l = 0; l < 64; ++l) t[l] = v[l] + v[l ^ off];
    memcpy(v, t, sizeof t);
  }
  return v[0];
}

/* ----------------------------------------------------------------- NF4 scale */

/* Scale of flattened block b: plain absmax[b], or nested
 * code2[a8[b]] * absmax2[b >> log2(bs2)] + offset with two fp32 roundings
 * (app/engine/nf4gemv.py:154-167; tests/test_nf4gemv.py:95-111). */
static inline float scale_of(long long b, const uint8_t* A8, const float* AMAX, const float* CODE2,
                             float offset, int bs2) {
  if (!A8) return AMAX[b];
  const float c = CODE2[A8[b]] * AMAX[b / bs2];
  return c + offset;
}

/* Dequantised value of flattened code k: round(code[q] * s) in out dtype, one
 * rounding (app/engine/nf4gemv.py:39-42, 185-188). High nibble = even k. */
void orc_nf4_dequant(const uint8_t* W, const uint8_t* A8, const float* AMAX, const float* CODE2,
                     float offset, const float* LUT, void* out, int out_dtype, long long n, int bs,
                     int bs2) {
  for (long long k = 0; k < n; ++k) {
    const uint8_t byte = W[k >> 1];
    const int q = (k & 1) ? (byte & 15) : (byte >> 4);
    const float v = LUT[q] * scale_of(k / bs, A8, AMAX, CODE2, offset, bs2);
    if (out_dtype == DT_F32) ((float*)out)[k] = v;
    else ((uint16_t*)out)[k] = st16(v, out_dtype);
  }
}

/* ------------------------------------------------------------------- GEMV */

/* Reference product: Y[n][m] = sum_k w[m][k] * X[n][k] in fp64, unrounded.
 * wdt >= 0: w = round(code*s) to that type - the dequantise-then-matmul
 * arithmetic the reference's tests hold the kernel to (bitsandbytes' forward,
 * tests/test_nf4gemv.py:130-141); wdt < 0: w = code*s exactly (fp32 product). */
void orc_nf4_gemm_ref(const void* X, int dt, const uint8_t* W, const uint8_t* A8, const float* AMAX,
                      const float* CODE2, float offset, const float* LUT, double* Y, int M, int K, int N,
                      int bs, int bs2, int wdt) {
#pragma omp parallel for schedule(static)
  for (int m = 0; m < M; ++m) {
    double* acc = calloc((size_t)N, sizeof(double));
    for (int k = 0; k < K; ++k) {
      const long long fk = (long long)m * K + k;
      const uint8_t byte = W[fk >> 1];
      const int q = (fk & 1) ? (byte & 15) : (byte >> 4);
      const float wf = LUT[q] * scale_of(fk / bs, A8, AMAX, CODE2, offset, bs2);
      const float w = wdt >= 0 ? rnd(wf, wdt) : wf;
      for (int n = 0; n < N; ++n) acc[n] += (double)w * (double)ld(X, (size_t)n * K + k, dt);
    }
    for (int n = 0; n < N; ++n) Y[(size_t)n * M + m] = acc[n];
    free(acc);
  }
}

/* The kernel's epilogue with the fork's rounding points
 * (app/engine/nf4gemv.py:215-226). */
static inline float epilogue(float acc, int epi, float r, int dt) {
  const float y = rnd(acc, dt);
  if (epi == 1) return rnd(r + y, dt);
  if (epi == 2) return rnd(rnd(silu_rn(r), dt) * y, dt);
  return y;
}

/* The GPU GEMV's arithmetic, in its order (ttspipe_amd/csrc/nf4_gemv.hip):
 * lane l of K-slice ks owns dwords d = l + 64*(j*KS + ks); per dword the 8
 * codes (the code points rounded to fp16, multiplied by the activations as
 * fp32 - fp16 and bf16 values are both exact in fp32, so every product is
 * exact) are chained q = fma(c_k, x_k, q) from q = +0 in code order, then
 * acc = fma(q, s_block, acc); lanes are summed by the xor butterfly, slices
 * left to right; then the epilogue. */
void orc_gemv_emul(const void* X, int dt, const uint8_t* W, const uint8_t* A8, const float* AMAX,
                   const float* CODE2, float offset, const float* LUT, uint16_t* Y, const void* R,
                   int epi, int M, int K, int bs, int bs2, int KS, int J) {
  const int KD = K / 8, nblk = K / bs;
  float lutv[16];
  for (int i = 0; i < 16; ++i) lutv[i] = rnd(LUT[i], DT_F16); /* fp16 codes for both types */
  /* fp16 and bf16 activations are exact in fp32: the kernel multiplies the
   * fp16 code by the fp32 activation (one exact product per fma) */
  float* xv = malloc(sizeof(float) * (size_t)K);
  for (int k = 0; k < K; ++k) xv[k] = ld(X, (size_t)k, dt);
#pragma omp parallel for schedule(static)
  for (int m = 0; m < M; ++m) {
    const uint32_t* wr = (const uint32_t*)(W + (size_t)m * (K / 2));
    float total = 0.0f;
    for (int ks = 0; ks < KS; ++ks) {
      float lanes[64];
      for (int l = 0; l < 64; ++l) {
        float acc = 0.0f;
        for (int j = 0; j < J; ++j) {
          const int d = l + 64 * (j * KS + ks);
          const int dc = d < KD ? d : KD - 1;
          const float s = scale_of((long long)m * nblk + (dc * 8) / bs, A8, AMAX, CODE2, offset, bs2);
          float q = 0.0f;
          for (int b = 0; b < 4; ++b) {
            float x0 = 0.0f, x1 = 0.0f;
            int byte = 0;
            if (d < KD) {
              byte = (wr[d] >> (8 * b)) & 0xff;
              x0 = xv[8 * d + 2 * b];
              x1 = xv[8 * d + 2 * b + 1];
            }
            q = fmaf(lutv[byte >> 4], x0, q);
            q = fmaf(lutv[byte & 15], x1, q);
          }
          acc = fmaf(q, s, acc);
        }
        lanes[l] = acc;
      }
      const float ws = butterfly64_up(lanes);
      total = ks == 0 ? ws : total + ws;
    }
    const float r = epi ? ld(R, (size_t)m, dt) : 0.0f;
    Y[m] = st16(epilogue(total, epi, r, dt), dt);
  }
  free(xv);
}

/* ---------------------------------------------------------------- RMSNorm */

/* fp64 reference of the fork's RMSNorm (app/engine/fusedops.py:8-14):
 * round(round(x * r) * w) with r from the exact mean of squares. */
void orc_rms_norm_ref(const void* X, const void* Wt, double* Y, int rows, int D, float eps, int dt) {
  for (int row = 0; row < rows; ++row) {
    double ss = 0.0;
    for (int i = 0; i < D; ++i) {
      const double v = ld(X, (size_t)row * D + i, dt);
      ss += v * v;
    }
    const double r = 1.0 / sqrt(ss / D + (double)eps);
    for (int i = 0; i < D; ++i) {
      const float n = rnd((float)(ld(X, (size_t)row * D + i, dt) * r), dt);
      Y[(size_t)row * D + i] = rnd(n * ld(Wt, (size_t)i, dt), dt);
    }
  }
}

/* The kernels' order (ttspipe_amd/csrc/fusedops.hip, and the GEMV's folded
 * norm): 64 chunks of 8 elements at a time, each chunk's squares by an fma
 * chain in element order from 0, the 64 chunk sums by the rising-distance
 * butterfly, these partial sums left to right; r = 1 / sqrt(ss/D + eps). */
void orc_rms_norm_emul(const void* X, const void* Wt, uint16_t* Y, int rows, int D, float eps, int dt) {
  const int nc = D / 8;
  for (int row = 0; row < rows; ++row) {
    const size_t base = (size_t)row * D;
    float ss = 0.0f;
    for (int c0 = 0; c0 < nc; c0 += 64) {
      float lanes[64];
      for (int l = 0; l < 64; ++l) {
        float acc = 0.0f;
        if (c0 + l < nc)
          for (int k = 0; k < 8; ++k) {
            const float a = ld(X, base + 8 * (size_t)(c0 + l) + k, dt);
            acc = fmaf(a, a, acc);
          }
        lanes[l] = acc;
      }
      const float part = butterfly64_up(lanes);
      ss = c0 == 0 ? part : ss + part;
    }
    const float r = orc_rsqrt_rn(ss / (float)D + eps);
    for (int i = 0; i < D; ++i) {
      const float n = rnd(ld(X, base + i, dt) * r, dt);
      Y[base + i] = st16(n * ld(Wt, (size_t)i, dt), dt);
    }
  }
}

/* ------------------------------------------------------------------- rope */

/* Interleaved-pair rotary, no fma, one rounding (app/engine/fusedops.py:103-133). */
void orc_rope(const void* X, const void* F, int ftype, uint16_t* Y, long long pairs, int half_dim,
              int heads, int seq, int dt) {
  for (long long i = 0; i < pairs; ++i) {
    const int p = (int)(i % half_dim);
    const int s = (int)((i / half_dim / heads) % seq);
    const size_t f = ((size_t)s * half_dim + p) * 2;
    const float fr = ld(F, f, ftype), fi = ld(F, f + 1, ftype);
    const float x0 = ld(X, (size_t)(2 * i), dt), x1 = ld(X, (size_t)(2 * i + 1), dt);
    const float a = x0 * fr, b = x1 * fi, c = x1 * fr, e = x0 * fi;
    Y[2 * i] = st16(a - b, dt);
    Y[2 * i + 1] = st16(c + e, dt);
  }
}

/* --------------------------------------------------- qk norm + rope + KV write */

/* app/engine/fusedlayer.py:56-92: per head, optional norm over 128 with one
 * rounding round((x * r) * w) (r from the sum of x*x: each 64-element half by
 * the rising butterfly, then the halves added),
 * rotary, then Q or the K cache at pos; V heads copied to the V cache. */
void orc_qk_rope_kv(const uint16_t* QKV, const uint16_t* QW, const uint16_t* KW, float eps,
                    const void* F, int ftype, long long pos, uint16_t* Q, uint16_t* KC, uint16_t* VC,
                    int nh, int nkv, int max_len, int dt) {
  if (pos < 0 || pos >= max_len) return;
  for (int head = 0; head < nh + 2 * nkv; ++head) {
    if (head >= nh + nkv) {
      const int vh = head - nh - nkv;
      memcpy(VC + ((size_t)vh * max_len + pos) * 128, QKV + (size_t)head * 128, 256);
      continue;
    }
    const int is_q = head < nh;
    const uint16_t* w = is_q ? QW : KW;
    float x[128];
    for (int d = 0; d < 128; ++d) x[d] = ld(QKV, (size_t)head * 128 + d, dt);
    if (w) {
      float v0[64], v1[64];
      for (int l = 0; l < 64; ++l) {
        v0[l] = x[l] * x[l];
        v1[l] = x[64 + l] * x[64 + l];
      }
      const float ss = butterfly64_up(v0) + butterfly64_up(v1);
      const float r = orc_rsqrt_rn(ss / 128.0f + eps);
      for (int d = 0; d < 128; ++d) x[d] = rnd((x[d] * r) * ld(w, (size_t)d, dt), dt);
    }
    uint16_t* dst = is_q ? Q + (size_t)head * 128 : KC + ((size_t)(head - nh) * max_len + pos) * 128;
    for (int d = 0; d < 128; d += 2) {
      const float fr = ld(F, (size_t)d, ftype), fi = ld(F, (size_t)d + 1, ftype);
      const float x0 = x[d], x1 = x[d + 1];
      dst[d] = st16((x0 * fr) - (x1 * fi), dt);
      dst[d + 1] = st16((x1 * fr) + (x0 * fi), dt);
    }
  }
}

/* -------------------------------------------------------------- attention */

/* fp64 grouped-query decode attention over positions [0, L) (the reference's
 * decode_attention, app/engine/fastpath.py:133-174, without intermediate
 * rounding): query head i reads KV head i / (nh / nkv). */
void orc_attn_ref(const uint16_t* Q, const uint16_t* KC, const uint16_t* VC, long long L, double* Y,
                  int nh, int nkv, int max_len, float scale, int dt) {
  const int groups = nh / nkv;
  double* sc = malloc(sizeof(double) * (size_t)(L > 0 ? L : 1));
  for (int qh = 0; qh < nh; ++qh) {
    const int kh = qh / groups;
    double mx = -INFINITY;
    for (long long j = 0; j < L; ++j) {
      double s = 0.0;
      for (int d = 0; d < 128; ++d)
        s += (double)ld(Q, (size_t)qh * 128 + d, dt) * ld(KC, ((size_t)kh * max_len + j) * 128 + d, dt);
      sc[j] = s * scale;
      if (sc[j] > mx) mx = sc[j];
    }
    double den = 0.0;
    for (long long j = 0; j < L; ++j) {
      sc[j] = exp(sc[j] - mx);
      den += sc[j];
    }
    for (int d = 0; d < 128; ++d) {
      double num = 0.0;
      for (long long j = 0; j < L; ++j) num += sc[j] * ld(VC, ((size_t)kh * max_len + j) * 128 + d, dt);
      Y[(size_t)qh * 128 + d] = num / den;
    }
  }
  free(sc);
}

/* The kernels' order (ttspipe_amd/csrc/fusedlayer.hip): chunks of 64
 * positions; q * scale rounded; score = four fma chains, chain c over the
 * element pairs i = c, c + 4, ... (elements 2i, 2i + 1), summed (s0 + s1) +
 * (s2 + s3); chunk max; p = exp_cw(s - max); l = rising butterfly sum;
 * acc[d] = four fma chains, chain c over positions j = c, c + 4, ..., summed
 * (a0 + a1) + (a2 + a3); chunks merged in order with w = exp_cw(m_c - M),
 * den += l*w, num += acc*w. */
void orc_attn_emul(const uint16_t* Q, const uint16_t* KC, const uint16_t* VC, long long pos, uint16_t* Y,
                   int nh, int nkv, int max_len, int nchunk, float scale, int dt) {
  const int groups = nh / nkv;
  long long L = pos + 1;
  if (L > max_len) L = max_len;
#pragma omp parallel for schedule(static)
  for (int qh = 0; qh < nh; ++qh) {
    float* pm = malloc(sizeof(float) * (size_t)nchunk);
    float* pl = malloc(sizeof(float) * (size_t)nchunk);
    float* pacc = malloc(sizeof(float) * (size_t)nchunk * 128);
    const int kh = qh / groups;
    float q[128];
    for (int d = 0; d < 128; ++d) q[d] = ld(Q, (size_t)qh * 128 + d, dt) * scale;
    for (int c = 0; c < nchunk; ++c) {
      const long long j0 = (long long)c * 64;
      if (j0 >= L) {
        pm[c] = -1e30f;
        pl[c] = 0.0f;
        continue;
      }
      const int nvalid = (int)((L - j0) < 64 ? (L - j0) : 64);
      float s[64], p[64], mx = -3.0e38f;
      for (int l = 0; l < 64; ++l) {
        float acc = 0.0f;
        if (l < nvalid) {
          const uint16_t* kr = KC + ((size_t)kh * max_len + j0 + l) * 128;
          float ch[4] = {0.0f, 0.0f, 0.0f, 0.0f};
          for (int i = 0; i < 64; ++i) {
            ch[i & 3] = fmaf(q[2 * i], ld(kr, (size_t)(2 * i), dt), ch[i & 3]);
            ch[i & 3] = fmaf(q[2 * i + 1], ld(kr, (size_t)(2 * i + 1), dt), ch[i & 3]);
          }
          acc = (ch[0] + ch[1]) + (ch[2] + ch[3]);
        }
        s[l] = acc;
        if (l < nvalid && acc > mx) mx = acc;
      }
      for (int l = 0; l < 64; ++l) p[l] = l < nvalid ? orc_exp_cw(s[l] - mx) : 0.0f;
      float pw[64];
      memcpy(pw, p, sizeof pw);
      pm[c] = mx;
      pl[c] = butterfly64_up(pw);
      for (int d = 0; d < 128; ++d) {
        float ch[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        for (int j = 0; j < nvalid; ++j)
          ch[j & 3] = fmaf(p[j], ld(VC, ((size_t)kh * max_len + j0 + j) * 128 + d, dt), ch[j & 3]);
        pacc[(size_t)c * 128 + d] = (ch[0] + ch[1]) + (ch[2] + ch[3]);
      }
    }
    float M = -3.0e38f;
    for (int c = 0; c < nchunk; ++c) M = fmaxf(M, pm[c]);
    for (int d = 0; d < 128; ++d) {
      float num = 0.0f, den = 0.0f;
      for (int c = 0; c < nchunk; ++c) {
        if (pl[c] == 0.0f) continue;
        const float w = orc_exp_cw(pm[c] - M);
        den = den + pl[c] * w;
        num = num + pacc[(size_t)c * 128 + d] * w;
      }
      Y[(size_t)qh * 128 + d] = st16(num / den, dt);
    }
    free(pm);
    free(pl);
    free(pacc);
  }
}

/* ---------------------------------------------------- decode-loop helpers */

/* splitmix64 (Steele, Lea, Flood 2014) over seed-mixed counters; the
 * synthetic weights of the Dual-AR decode are this function of (seed, index). */
static inline uint64_t mix64(uint64_t z) {
  z += 0x9e3779b97f4a7c15ull;
  z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
  z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
  return z ^ (z >> 31);
}

void orc_synth_fill(void* out, long long n, uint64_t seed, int kind, float scale, float offset) {
  const uint64_t ms = mix64(seed);
#pragma omp parallel for schedule(static)
  for (long long i = 0; i < n; ++i) {
    const uint64_t h = mix64(ms ^ (uint64_t)i);
    if (kind == 0) {
      ((uint8_t*)out)[i] = (uint8_t)(h >> 56);
      continue;
    }
    const float u = (float)(uint32_t)(h >> 40) * 1.1920928955078125e-07f - 1.0f;
    const float v = u * scale + offset;
    if (kind == 1) ((uint16_t*)out)[i] = orc_f32_to_bf16(v);
    else if (kind == 2) ((uint16_t*)out)[i] = orc_f32_to_f16(v);
    else ((float*)out)[i] = v;
  }
}

void orc_embed_sum(const uint16_t* E, const int* tok, int ntok, int vocab, int D, uint16_t* out, int dt) {
  for (int d = 0; d < D; ++d) {
    float acc = 0.0f;
    for (int c = 0; c < ntok; ++c) {
      int t = tok[c];
      t = t < 0 ? 0 : (t >= vocab ? vocab - 1 : t);
      acc = acc + ld(E, ((size_t)c * vocab + t) * D + d, dt);
    }
    out[d] = st16(acc, dt);
  }
}

int orc_argmax(const uint16_t* X, int n, int dt) {
  float best = -INFINITY;
  int idx = 0;
  for (int i = 0; i < n; ++i) {
    const float v = ld(X, (size_t)i, dt);
    if (v > best) {
      best = v;
      idx = i;
    }
  }
  return idx;
}
