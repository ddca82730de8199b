// Top-k / top-p sampling of one logit row in one workgroup (the reference's
// fused sampler, app/engine/fusedsample.py:28-223, restated for wave64):
//   * M = max of the row, Z = sum of exp(l - M) over the whole row (the
//     softmax normaliser of the untempered logits);
//   * the K-th largest logit by a two-pass radix select over the 16-bit keys
//     (high byte, then low byte; histograms in LDS), the K candidates =
//     everything above the threshold plus the lowest-index ties at it;
//   * one wave sorts the candidates (value descending, then index ascending;
//     a bitonic network over 128 slots, two per lane), accumulates their
//     probabilities exp(v - M) / Z in that order, keeps the first and every
//     one whose inclusive cumulative probability is <= top_p, and draws
//     argmax over the kept of v / temperature - log(-log(u_i)) with u_i the
//     caller's uniform number for vocabulary index i (the Gumbel form of the
//     fork's argmax(probs / Exp(1)): exact sampling from the tempered,
//     truncated distribution); ties go to the lowest index.
// Everything is deterministic for given inputs: fixed reduction orders, and
// the candidates are sorted before anything order-dependent reads them.
#include "ttsp_common.h"

namespace ttsp {

constexpr int SAMPLE_THREADS = 1024;
constexpr int SAMPLE_KMAX = 64;   // the largest top_k served
constexpr int SAMPLE_CAND = 128;  // candidate slots (KMAX plus room); two per lane of one wave

// 16-bit float bits -> an unsigned key ordered like the value (fp16 and bf16
// share the sign-magnitude layout).
__device__ __forceinline__ uint32_t key16(uint32_t h) { return (h & 0x8000u) ? (~h & 0xFFFFu) : (h | 0x8000u); }

template <int DT>
__global__ __launch_bounds__(SAMPLE_THREADS) void sample_topk_kernel(
    const uint16_t* __restrict__ L, int V, const uint16_t* __restrict__ TEMP, const uint16_t* __restrict__ TOPP,
    const long long* __restrict__ TOPK, const float* __restrict__ U, int* __restrict__ OUT) {
  __shared__ uint32_t hist[256];
  __shared__ float red[SAMPLE_THREADS / 64];
  __shared__ float cval[SAMPLE_CAND];
  __shared__ int cidx[SAMPLE_CAND];
  __shared__ int ccount, above, thr, need;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  constexpr int NW = SAMPLE_THREADS / 64;
  int K = (int)min(max(TOPK[0], 1LL), (long long)SAMPLE_KMAX);
  K = min(K, V);

  // max, then the normaliser (per-thread strided partials, waves by DPP,
  // waves left to right)
  float m = -__builtin_inff();
  for (int i = tid; i < V; i += SAMPLE_THREADS) m = fmaxf(m, Elem<DT>::load(L[i]));
  for (int off = 32; off >= 1; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, 64));
  if (lane == 0) red[wave] = m;
  for (int b = tid; b < 256; b += SAMPLE_THREADS) hist[b] = 0;
  if (tid == 0) ccount = 0;
  __syncthreads();
  float M = red[0];
  for (int w = 1; w < NW; ++w) M = fmaxf(M, red[w]);
  __syncthreads();
  float z = 0.0f;
  for (int i = tid; i < V; i += SAMPLE_THREADS) z = __fadd_rn(z, exp_cw(__fsub_rn(Elem<DT>::load(L[i]), M)));
  z = wave_sum_dpp(z);
  if (lane == 0) red[wave] = z;
  // radix select, high byte
  for (int i = tid; i < V; i += SAMPLE_THREADS) atomicAdd(&hist[key16(L[i]) >> 8], 1u);
  __syncthreads();
  float Z = red[0];
  for (int w = 1; w < NW; ++w) Z = __fadd_rn(Z, red[w]);
  if (tid == 0) {
    int acc = 0, b = 255;
    for (; b > 0 && acc + (int)hist[b] < K; --b) acc += (int)hist[b];
    above = acc;
    thr = b;
  }
  __syncthreads();
  const uint32_t hi = (uint32_t)thr;
  const int above_hi = above;
  __syncthreads();
  for (int b = tid; b < 256; b += SAMPLE_THREADS) hist[b] = 0;
  __syncthreads();
  // low byte among the keys whose high byte is the threshold's
  for (int i = tid; i < V; i += SAMPLE_THREADS) {
    const uint32_t k = key16(L[i]);
    if ((k >> 8) == hi) atomicAdd(&hist[k & 0xFFu], 1u);
  }
  __syncthreads();
  if (tid == 0) {
    int acc = above_hi, b = 255;
    for (; b > 0 && acc + (int)hist[b] < K; --b) acc += (int)hist[b];
    thr = (int)((hi << 8) | (uint32_t)b);
    need = K - acc;  // entries equal to the threshold that make the cut
  }
  __syncthreads();
  const uint32_t T = (uint32_t)thr;
  // everything strictly above the threshold (fewer than K of them), in any order
  for (int i = tid; i < V; i += SAMPLE_THREADS) {
    if (key16(L[i]) > T) {
      const int s = atomicAdd(&ccount, 1);
      if (s < SAMPLE_CAND) {
        cval[s] = Elem<DT>::load(L[i]);
        cidx[s] = i;
      }
    }
  }
  __syncthreads();
  // ties at the threshold, lowest indices first (one wave, in index order)
  if (wave == 0) {
    const int base_n = ccount;
    int taken = 0;
    for (int base = 0; base < V && taken < need; base += 64) {
      const int i = base + lane;
      const bool eq = i < V && key16(L[i]) == T;
      const uint64_t mask = __ballot(eq);
      const int rank = __popcll(mask & ((1ull << lane) - 1ull));
      if (eq && taken + rank < need) {
        const int s = base_n + taken + rank;
        if (s < SAMPLE_CAND) {
          cval[s] = Elem<DT>::load(L[i]);
          cidx[s] = i;
        }
      }
      taken += __popcll(mask);
    }
  }
  __syncthreads();

  if (wave == 0) {
    const int n = min(K, SAMPLE_CAND);
    constexpr int R = SAMPLE_CAND / 64;
    float v[R];
    int ix[R];
#pragma unroll
    for (int j = 0; j < R; ++j) {
      const int s = j * 64 + lane;
      v[j] = s < n ? cval[s] : -__builtin_inff();
      ix[j] = s < n ? cidx[s] : 0x7fffffff;
    }
    // bitonic sort, slot s = 64 j + lane: value descending, then index ascending
#pragma unroll
    for (int size = 2; size <= SAMPLE_CAND; size <<= 1) {
#pragma unroll
      for (int stride = size >> 1; stride > 0; stride >>= 1) {
        if (stride >= 64) {
          const int d = stride >> 6;  // partner: register j ^ d, same lane
#pragma unroll
          for (int j = 0; j < R; ++j) {
            if (j & d) continue;
            const int s = j * 64 + lane;
            const bool desc = (s & size) == 0;
            const bool lower_better = v[j] > v[j | d] || (v[j] == v[j | d] && ix[j] < ix[j | d]);
            if (lower_better != desc) {
              const float tv = v[j];
              v[j] = v[j | d];
              v[j | d] = tv;
              const int ti = ix[j];
              ix[j] = ix[j | d];
              ix[j | d] = ti;
            }
          }
        } else {
#pragma unroll
          for (int j = 0; j < R; ++j) {
            const int s = j * 64 + lane;
            const float pv = __shfl_xor(v[j], stride, 64);
            const int pi = __shfl_xor(ix[j], stride, 64);
            const bool lower = (s & stride) == 0;
            const bool desc = (s & size) == 0;
            const bool mine_better = v[j] > pv || (v[j] == pv && ix[j] < pi);
            const bool keep = (lower == desc) ? mine_better : !mine_better;
            if (!keep) {
              v[j] = pv;
              ix[j] = pi;
            }
          }
        }
      }
    }
    // inclusive cumulative probability in the sorted order, the cut, the draw
    const float temp = fmaxf(Elem<DT>::load(TEMP[0]), 1e-5f);
    const float topp = Elem<DT>::load(TOPP[0]);
    float best = -__builtin_inff();
    int best_i = ix[0];
    float carry = 0.0f;
#pragma unroll
    for (int j = 0; j < R; ++j) {
      const int s = j * 64 + lane;
      const float p = s < n ? __fdiv_rn(exp_cw(__fsub_rn(v[j], M)), Z) : 0.0f;
      float c = p;
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) {
        const float t = __shfl_up(c, o, 64);
        if (lane >= o) c = __fadd_rn(c, t);
      }
      c = __fadd_rn(c, carry);
      carry = __shfl(c, 63, 64);
      const bool kept = s < n && (s == 0 || c <= topp);
      if (kept) {
        const float u = fmaxf(U[ix[j]], 1e-20f);
        const float score = __fsub_rn(__fdiv_rn(v[j], temp), logf(-logf(u)));
        if (score > best || (score == best && ix[j] < best_i)) {
          best = score;
          best_i = ix[j];
        }
      }
    }
    for (int off = 32; off >= 1; off >>= 1) {
      const float ob = __shfl_xor(best, off, 64);
      const int oi = __shfl_xor(best_i, off, 64);
      if (ob > best || (ob == best && oi < best_i)) {
        best = ob;
        best_i = oi;
      }
    }
    if (lane == 0) OUT[0] = best_i;
  }
}

}  // namespace ttsp

using namespace ttsp;

extern "C" int ttsp_sample_max_top_k(void) { return SAMPLE_KMAX; }

extern "C" int ttsp_sample_topk(const void* L, int V, int dtype, const void* TEMP, const void* TOPP,
                                const long long* TOPK, const float* U, int* OUT, hipStream_t stream) {
  if (!L || !TEMP || !TOPP || !TOPK || !U || !OUT || V <= 0) return (int)hipErrorInvalidValue;
#define TTSP_S(DTV)                                                                                    \
  hipLaunchKernelGGL(sample_topk_kernel<DTV>, dim3(1), dim3(SAMPLE_THREADS), 0, stream, (const uint16_t*)L, \
                     V, (const uint16_t*)TEMP, (const uint16_t*)TOPP, TOPK, U, OUT)
  if (dtype == DT_F16) TTSP_S(DT_F16);
  else if (dtype == DT_BF16) TTSP_S(DT_BF16);
  else return (int)hipErrorInvalidValue;
#undef TTSP_S
  TTSP_RETURN_LAUNCH();
}
