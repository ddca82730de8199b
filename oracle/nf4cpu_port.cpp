// CPU baseline: the reference's CPU NF4 GEMV algorithm (app/engine/nf4cpu.py:
// 86-146, 256-270), restated, and a decode block built on it (the structure of
// nf4cpu.py:479-617). TEST/BENCH INFRASTRUCTURE ONLY - the benchmark's
// cpu_baseline leg times it on the GPU box's host cores; nothing in the
// product calls it.
//
// Per weight row and 64-code block (32 packed bytes):
//   * widen the bytes to 16-bit lanes; high nibbles are the even codes, low
//     nibbles the odd ones;
//   * look each nibble up in the 16-entry bf16 code table (one vpermw each);
//   * dot against the activation split once into even / odd halves with two
//     vdpbf16ps (32 bf16 pairs -> 16 fp32 sums);
//   * fma the block's partial by its bf16 absmax into the row accumulator;
// then a horizontal sum, rounded to bf16. Four rows share each activation
// load (register blocking); groups of rows are spread over OpenMP threads.
// Hosts without AVX512-BF16 take a scalar loop with the same operations.
#include <immintrin.h>
#include <omp.h>
#include <stdint.h>
#include <string.h>

#include <cmath>
#include <vector>

namespace {

inline float bf2f(uint16_t h) {
  uint32_t u = (uint32_t)h << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

inline uint16_t f2bf(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

template <int R>
__attribute__((target("avx512f,avx512bw,avx512bf16"))) void rows_avx(
    const uint16_t* xs, int64_t H, int64_t NB, const uint8_t* qp, const uint16_t* ap, int64_t n0,
    __m512i lut, uint16_t* y) {
  const __m512i mask = _mm512_set1_epi16(15);
  __m512 acc[R];
  for (int r = 0; r < R; ++r) acc[r] = _mm512_setzero_ps();
  for (int64_t b = 0; b < NB; ++b) {
    const __m512bh xe = (__m512bh)_mm512_loadu_si512(xs + b * 32);
    const __m512bh xo = (__m512bh)_mm512_loadu_si512(xs + H + b * 32);
    for (int r = 0; r < R; ++r) {
      const uint8_t* row = qp + (n0 + r) * H;
      const __m512i v = _mm512_cvtepu8_epi16(_mm256_loadu_si256((const __m256i*)(row + b * 32)));
      const __m512bh we = (__m512bh)_mm512_permutexvar_epi16(_mm512_srli_epi16(v, 4), lut);
      const __m512bh wo = (__m512bh)_mm512_permutexvar_epi16(_mm512_and_si512(v, mask), lut);
      __m512 p = _mm512_dpbf16_ps(_mm512_setzero_ps(), we, xe);
      p = _mm512_dpbf16_ps(p, wo, xo);
      acc[r] = _mm512_fmadd_ps(p, _mm512_set1_ps(bf2f(ap[(n0 + r) * NB + b])), acc[r]);
    }
  }
  for (int r = 0; r < R; ++r) y[n0 + r] = f2bf(_mm512_reduce_add_ps(acc[r]));
}

__attribute__((target("avx512f,avx512bw,avx512bf16"))) void gemv_avx(
    const uint16_t* xs, int64_t K, const uint8_t* qp, const uint16_t* ap, const uint16_t* code,
    int64_t n_out, uint16_t* y, int threads) {
  const int64_t H = K / 2, NB = K / 64;
  uint16_t lut_h[32];
  for (int i = 0; i < 32; ++i) lut_h[i] = code[i & 15];
  const __m512i lut = _mm512_loadu_si512(lut_h);
  const int64_t groups = (n_out + 3) / 4;
#pragma omp parallel for num_threads(threads) schedule(static)
  for (int64_t g = 0; g < groups; ++g) {
    const int64_t n = g * 4;
    if (n + 4 <= n_out) {
      rows_avx<4>(xs, H, NB, qp, ap, n, lut, y);
    } else {
      for (int64_t t = n; t < n_out; ++t) rows_avx<1>(xs, H, NB, qp, ap, t, lut, y);
    }
  }
}

void gemv_scalar(const uint16_t* xs, int64_t K, const uint8_t* qp, const uint16_t* ap,
                 const uint16_t* code, int64_t n_out, uint16_t* y, int threads) {
  const int64_t H = K / 2, NB = K / 64;
  float c[16];
  for (int i = 0; i < 16; ++i) c[i] = bf2f(code[i]);
#pragma omp parallel for num_threads(threads) schedule(static)
  for (int64_t n = 0; n < n_out; ++n) {
    const uint8_t* row = qp + n * H;
    float acc = 0.0f;
    for (int64_t b = 0; b < NB; ++b) {
      float p = 0.0f;
      for (int j = 0; j < 32; ++j) {
        const uint8_t v = row[b * 32 + j];
        p += c[v >> 4] * bf2f(xs[b * 32 + j]) + c[v & 15] * bf2f(xs[H + b * 32 + j]);
      }
      acc += p * bf2f(ap[n * NB + b]);
    }
    y[n] = f2bf(acc);
  }
}

}  // namespace

extern "C" int cpu_has_avx512bf16(void) { return __builtin_cpu_supports("avx512bf16") ? 1 : 0; }

// y[n] = sum_k x[k] * code[q[n][k]] * absmax[n][k/64], bf16 in and out; x is
// split into even / odd halves here, once per call, as the reference does.
extern "C" void cpu_nf4_gemv(const uint16_t* x, int64_t K, const uint8_t* packed,
                             const uint16_t* absmax, const uint16_t* code16, int64_t n_out,
                             uint16_t* y, int threads, int force_scalar) {
  const int64_t H = K / 2;
  std::vector<uint16_t> xs(K);
  for (int64_t j = 0; j < H; ++j) {
    xs[j] = x[2 * j];
    xs[H + j] = x[2 * j + 1];
  }
  if (!force_scalar && cpu_has_avx512bf16())
    gemv_avx(xs.data(), K, packed, absmax, code16, n_out, y, threads);
  else
    gemv_scalar(xs.data(), K, packed, absmax, code16, n_out, y, threads);
}

namespace {

inline float round_bf(float f) { return bf2f(f2bf(f)); }

// q . k over 128 (fp32 q, bf16 k) and o += p * v, AVX-512 where the host has it
__attribute__((target("avx512f"))) float dot128_avx(const float* q, const uint16_t* k) {
  __m512 s0 = _mm512_setzero_ps(), s1 = _mm512_setzero_ps();
  for (int i = 0; i < 128; i += 32) {
    const __m512 k0 = _mm512_castsi512_ps(_mm512_slli_epi32(_mm512_cvtepu16_epi32(_mm256_loadu_si256((const __m256i*)(k + i))), 16));
    const __m512 k1 = _mm512_castsi512_ps(_mm512_slli_epi32(_mm512_cvtepu16_epi32(_mm256_loadu_si256((const __m256i*)(k + i + 16))), 16));
    s0 = _mm512_fmadd_ps(_mm512_loadu_ps(q + i), k0, s0);
    s1 = _mm512_fmadd_ps(_mm512_loadu_ps(q + i + 16), k1, s1);
  }
  return _mm512_reduce_add_ps(_mm512_add_ps(s0, s1));
}
__attribute__((target("avx512f"))) void axpy128_avx(float p, const uint16_t* v, float* o) {
  const __m512 pv = _mm512_set1_ps(p);
  for (int i = 0; i < 128; i += 16) {
    const __m512 vv = _mm512_castsi512_ps(_mm512_slli_epi32(_mm512_cvtepu16_epi32(_mm256_loadu_si256((const __m256i*)(v + i))), 16));
    _mm512_storeu_ps(o + i, _mm512_fmadd_ps(pv, vv, _mm512_loadu_ps(o + i)));
  }
}
float dot128(const float* q, const uint16_t* k, bool avx) {
  if (avx) return dot128_avx(q, k);
  float d = 0.0f;
  for (int i = 0; i < 128; ++i) d += q[i] * bf2f(k[i]);
  return d;
}
void axpy128(float p, const uint16_t* v, float* o, bool avx) {
  if (avx) return axpy128_avx(p, v, o);
  for (int i = 0; i < 128; ++i) o[i] += p * bf2f(v[i]);
}

void gemv_bf(const uint16_t* x, int64_t K, const uint8_t* packed, const uint16_t* absmax,
             const uint16_t* code16, int64_t n_out, uint16_t* y, int threads) {
  cpu_nf4_gemv(x, K, packed, absmax, code16, n_out, y, threads, 0);
}

// fork RMSNorm on fp32 values: r = 1/sqrt(mean(x^2) + eps), y = bf16(bf16(x r) w)
void rms_norm_bf(const float* x, int64_t D, const uint16_t* w, float eps, uint16_t* y) {
  double ss = 0.0;
  for (int64_t i = 0; i < D; ++i) ss += (double)x[i] * x[i];
  const float r = 1.0f / std::sqrt((float)(ss / D) + eps);
  for (int64_t i = 0; i < D; ++i) y[i] = f2bf(round_bf(x[i] * r) * bf2f(w[i]));
}

}  // namespace

// One decode position through one transformer block (batch 1, head_dim 128):
// norm -> wqkv -> q/k head norms (when given) -> interleaved rotary -> K/V
// written at pos -> grouped attention over positions [0, pos] (heads spread
// over the threads) -> wo + residual -> norm -> w1|w3 (one weight of 2*inter
// rows) -> silu(a) * b -> w2 + residual. bf16 in and out, fp32 between,
// rounded to bf16 where the fork rounds. freqs: the position's 64 (cos, sin)
// pairs in fp32.
extern "C" void cpu_decode_block(const uint16_t* x, uint16_t* out, int64_t D, int64_t nh, int64_t nkv,
                                 int64_t inter, const uint16_t* attn_norm, const uint16_t* ffn_norm,
                                 const uint16_t* qn, const uint16_t* kn, float eps, const uint8_t* qkv_p,
                                 const uint16_t* qkv_a, const uint8_t* wo_p, const uint16_t* wo_a,
                                 const uint8_t* w13_p, const uint16_t* w13_a, const uint8_t* w2_p,
                                 const uint16_t* w2_a, const uint16_t* code16, uint16_t* kc, uint16_t* vc,
                                 int64_t pos, int64_t max_len, const float* freqs, int threads) {
  const int64_t HD = 128, qs = nh * HD, kvs = nkv * HD, nqkv = qs + 2 * kvs;
  std::vector<float> xf(D), q(nqkv);
  std::vector<uint16_t> hb(D > 2 * inter ? D : 2 * inter), qkvb(nqkv), att(qs), yb(2 * inter > D ? 2 * inter : D);
  for (int64_t i = 0; i < D; ++i) xf[i] = bf2f(x[i]);
  rms_norm_bf(xf.data(), D, attn_norm, eps, hb.data());
  gemv_bf(hb.data(), D, qkv_p, qkv_a, code16, nqkv, qkvb.data(), threads);
  for (int64_t i = 0; i < nqkv; ++i) q[i] = bf2f(qkvb[i]);
  auto head_norm = [&](float* t, const uint16_t* w) {
    double ss = 0.0;
    for (int64_t i = 0; i < HD; ++i) ss += (double)t[i] * t[i];
    const float r = 1.0f / std::sqrt((float)(ss / HD) + eps);
    for (int64_t i = 0; i < HD; ++i) t[i] = round_bf(t[i] * r * bf2f(w[i]));
  };
  auto rope = [&](float* t) {
    for (int64_t i = 0; i < HD / 2; ++i) {
      const float a = t[2 * i], b = t[2 * i + 1], c = freqs[2 * i], s = freqs[2 * i + 1];
      t[2 * i] = round_bf(a * c - b * s);
      t[2 * i + 1] = round_bf(b * c + a * s);
    }
  };
  for (int64_t h = 0; h < nh + nkv; ++h) {
    float* t = q.data() + h * HD;
    if (qn) head_norm(t, h < nh ? qn : kn);
    rope(t);
  }
  for (int64_t h = 0; h < nkv; ++h)
    for (int64_t i = 0; i < HD; ++i) {
      kc[(h * max_len + pos) * HD + i] = f2bf(q[qs + h * HD + i]);
      vc[(h * max_len + pos) * HD + i] = f2bf(q[qs + kvs + h * HD + i]);
    }
  const int64_t L = pos + 1, groups = nh / nkv;
  const float scale = 1.0f / std::sqrt((float)HD);
  const bool avx = __builtin_cpu_supports("avx512f");
#pragma omp parallel for num_threads(threads) schedule(static)
  for (int64_t hq = 0; hq < nh; ++hq) {
    std::vector<float> sc(L), o(HD, 0.0f);
    const float* qr = q.data() + hq * HD;
    const uint16_t* kb = kc + (hq / groups) * max_len * HD;
    const uint16_t* vb = vc + (hq / groups) * max_len * HD;
    float mx = -INFINITY;
    for (int64_t l = 0; l < L; ++l) {
      sc[l] = round_bf(dot128(qr, kb + l * HD, avx)) * scale;
      mx = sc[l] > mx ? sc[l] : mx;
    }
    double sum = 0.0;
    for (int64_t l = 0; l < L; ++l) {
      sc[l] = std::exp(sc[l] - mx);
      sum += sc[l];
    }
    for (int64_t l = 0; l < L; ++l) {
      axpy128(round_bf((float)(sc[l] / sum)), vb + l * HD, o.data(), avx);
    }
    for (int64_t i = 0; i < HD; ++i) att[hq * HD + i] = f2bf(o[i]);
  }
  gemv_bf(att.data(), qs, wo_p, wo_a, code16, D, yb.data(), threads);
  for (int64_t i = 0; i < D; ++i) xf[i] = round_bf(xf[i] + bf2f(yb[i]));
  rms_norm_bf(xf.data(), D, ffn_norm, eps, hb.data());
  gemv_bf(hb.data(), D, w13_p, w13_a, code16, 2 * inter, yb.data(), threads);
  for (int64_t i = 0; i < inter; ++i) {
    const float a = bf2f(yb[i]), b = bf2f(yb[inter + i]);
    hb[i] = f2bf(round_bf(a / (1.0f + std::exp(-a))) * b);
  }
  gemv_bf(hb.data(), inter, w2_p, w2_a, code16, D, yb.data(), threads);
  for (int64_t i = 0; i < D; ++i) out[i] = f2bf(xf[i] + bf2f(yb[i]));
}

// argmax over n bf16 logits (first maximum)
extern "C" int64_t cpu_argmax_bf16(const uint16_t* x, int64_t n) {
  int64_t best = 0;
  float bv = bf2f(x[0]);
  for (int64_t i = 1; i < n; ++i)
    if (bf2f(x[i]) > bv) {
      bv = bf2f(x[i]);
      best = i;
    }
  return best;
}
