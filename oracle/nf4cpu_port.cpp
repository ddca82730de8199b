// CPU baseline: the reference's CPU NF4 GEMV algorithm (app/engine/nf4cpu.py:
// 86-146, 256-270), restated. TEST/BENCH INFRASTRUCTURE ONLY - the benchmark's
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
