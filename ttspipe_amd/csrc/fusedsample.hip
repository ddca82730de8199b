// Top-k / top-p / temperature draw of one logit row in one workgroup.
//
// Result (what the reference's fused sampler returns, app/engine/
// fusedsample.py:1-19): take the k = min(max(TOPK, 1), 64, V) largest logits,
// ties to the lowest index, in descending order; keep the first and every one
// whose inclusive cumulative probability under softmax(row) is <= TOPP; draw
// argmax over the kept of l / max(T, 1e-5) - log(-log(max(u, 1e-20))), with u
// the caller's uniform number of that vocabulary index (the Gumbel form of the
// fork's argmax(probs / Exp(1))), ties to the lowest index.
//
// Design (one workgroup of 4 waves; the row lives in LDS):
//   1. The row is copied into LDS as order-preserving 16-bit keys (a float's
//      bit pattern with the sign bit flipped, all bits flipped for negative
//      values: unsigned key order is float order), coalesced, while each
//      thread keeps its running max; the block max M and the softmax
//      normaliser Z = sum exp(l - M) follow (fixed order: thread, wave, then
//      the four waves in turn).
//   2. The k-th largest key t is built bit by bit from the top: a candidate
//      prefix survives when at least k keys are >= it. Counting is by wave
//      ballots - one popcount per key slot, summed in scalar registers - and
//      the four wave counts meet in LDS; 16 rounds, one barrier each.
//   3. Every key > t (fewer than k) and the first k - #(> t) keys equal to t in
//      index order are compacted into a k-entry candidate list: each thread
//      owns a contiguous range of the row, so an exclusive prefix sum of the
//      per-thread counts gives index-ordered slots.
//   4. The k candidates are ordered by rank counting: candidate c's rank is the
//      number of candidates that beat it (larger key, or equal key and lower
//      index), so ranks are a permutation and no sorting network is needed.
//   5. One wave finishes: lane j holds the j-th candidate's probability, an
//      inclusive scan gives the cumulative mass, the top-p cut and the scores
//      follow, and a butterfly over (score, index) picks the draw.
#include "ttsp_common.h"

namespace ttsp {

constexpr int SMP_THREADS = 256;
constexpr int SMP_WAVES = SMP_THREADS / 64;
constexpr int SMP_MAX_K = 64;
constexpr int SMP_MAX_V = 32768;  // LDS holds the whole row as 16-bit keys (64 KB)

__device__ __forceinline__ uint32_t key_of(uint32_t h) { return (h & 0x8000u) ? (~h & 0xffffu) : (h | 0x8000u); }
__device__ __forceinline__ uint32_t bits_of(uint32_t k) { return (k & 0x8000u) ? (k & 0x7fffu) : (~k & 0xffffu); }

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) v = fmaxf(v, __shfl_xor(v, d));
  return v;
}

// Inclusive prefix sum over the 64 lanes (Hillis-Steele, fixed order).
template <typename T>
__device__ __forceinline__ T wave_scan(T v, int lane) {
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const T o = __shfl_up(v, d);
    if (lane >= d) v = v + o;
  }
  return v;
}

template <int DT>
__global__ __launch_bounds__(SMP_THREADS) void sample_topk_kernel(const uint16_t* __restrict__ L, int V,
                                                                  const uint16_t* __restrict__ TEMP,
                                                                  const uint16_t* __restrict__ TOPP,
                                                                  const long long* __restrict__ TOPK,
                                                                  const float* __restrict__ U, int* __restrict__ OUT) {
  __shared__ __align__(16) uint16_t keys[SMP_MAX_V];
  __shared__ float red[SMP_WAVES];
  __shared__ int cnt[2][SMP_WAVES];
  __shared__ int scan_gt[SMP_WAVES], scan_eq[SMP_WAVES];
  __shared__ int cand[SMP_MAX_K], sorted[SMP_MAX_K];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int k = (int)min(min(max(TOPK[0], 1LL), (long long)SMP_MAX_K), (long long)V);

  // 1. keys into LDS, block max, normaliser
  float mx = -__builtin_inff();
  for (int i = tid; i < V; i += SMP_THREADS) {
    const uint32_t h = L[i];
    keys[i] = (uint16_t)key_of(h);
    mx = fmaxf(mx, Elem<DT>::load(h));
  }
  mx = wave_max(mx);
  if (lane == 0) red[wave] = mx;
  __syncthreads();
  float M = red[0];
#pragma unroll
  for (int w = 1; w < SMP_WAVES; ++w) M = fmaxf(M, red[w]);
  float z = 0.0f;
  for (int i = tid; i < V; i += SMP_THREADS) z = __fadd_rn(z, exp_cw(__fsub_rn(Elem<DT>::load(bits_of(keys[i])), M)));
  z = wave_sum_dpp(z);
  __syncthreads();  // every wave has read red[] as maxima
  if (lane == 0) red[wave] = z;

  // 2. the k-th largest key (counting reads the row lane-strided: 64 lanes
  // read 128 consecutive bytes, no bank conflicts)
  uint32_t t = 0;
  for (int bit = 15; bit >= 0; --bit) {
    const uint32_t c = t | (1u << bit);
    int n = 0;  // wave-uniform: the wave's keys >= c, one ballot per slot
    for (int i = tid; i - lane < V; i += SMP_THREADS) {
      const bool ge = i < V && keys[i] >= c;
      n += __popcll(__ballot(ge));
    }
    if (lane == 0) cnt[bit & 1][wave] = n;
    __syncthreads();
    int total = 0;
#pragma unroll
    for (int w = 0; w < SMP_WAVES; ++w) total += cnt[bit & 1][w];
    if (total >= k) t = c;
  }
  float Z = red[0];
#pragma unroll
  for (int w = 1; w < SMP_WAVES; ++w) Z = __fadd_rn(Z, red[w]);

  // 3. index-ordered compaction: all keys > t, then the first `need` keys == t;
  // thread tid owns the contiguous range [lo, hi)
  const int per = (V + SMP_THREADS - 1) / SMP_THREADS;
  const int lo = min(tid * per, V), hi = min(lo + per, V);
  int ngt = 0, neq = 0;
  for (int i = lo; i < hi; ++i) {
    ngt += keys[i] > t;
    neq += keys[i] == t;
  }
  const int igt = wave_scan(ngt, lane), ieq = wave_scan(neq, lane);
  if (lane == 63) scan_gt[wave] = igt, scan_eq[wave] = ieq;
  __syncthreads();
  int off_gt = igt - ngt, off_eq = ieq - neq, total_gt = 0;
#pragma unroll
  for (int w = 0; w < SMP_WAVES; ++w) {
    total_gt += scan_gt[w];
    if (w < wave) off_gt += scan_gt[w], off_eq += scan_eq[w];
  }
  const int need = k - total_gt;  // >= 1 by the choice of t
  for (int i = lo; i < hi; ++i) {
    const uint32_t key = keys[i];
    if (key > t) cand[off_gt++] = i;
    else if (key == t && off_eq < need) cand[total_gt + off_eq++] = i;
  }
  __syncthreads();

  // 4. rank counting
  if (tid < k) {
    const int me = cand[tid];
    const uint32_t mk = keys[me];
    int rank = 0;
    for (int j = 0; j < k; ++j) {
      const int o = cand[j];
      const uint32_t ok = keys[o];
      rank += ok > mk || (ok == mk && o < me);
    }
    sorted[rank] = me;
  }
  __syncthreads();

  // 5. cumulative mass, top-p cut, draw (wave 0)
  if (wave != 0) return;
  const float T = fmaxf(Elem<DT>::load(TEMP[0]), 1e-5f);
  const float P = Elem<DT>::load(TOPP[0]);
  int idx = 0x7fffffff;
  float p = 0.0f, l = 0.0f;
  if (lane < k) {
    idx = sorted[lane];
    l = Elem<DT>::load(bits_of(keys[idx]));
    p = __fdiv_rn(exp_cw(__fsub_rn(l, M)), Z);
  }
  const float c = wave_scan(p, lane);
  const bool keep = lane < k && (lane == 0 || c <= P);
  float score = -__builtin_inff();
  if (keep) {
    const float g = -logf(-logf(fmaxf(U[idx], 1e-20f)));
    score = __fadd_rn(__fdiv_rn(l, T), g);
  } else {
    idx = 0x7fffffff;
  }
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const float os = __shfl_xor(score, d);
    const int oi = __shfl_xor(idx, d);
    if (os > score || (os == score && oi < idx)) score = os, idx = oi;
  }
  if (lane == 0) OUT[0] = idx;
}

}  // namespace ttsp

using namespace ttsp;

extern "C" int ttsp_sample_max_top_k(void) { return SMP_MAX_K; }

extern "C" int ttsp_sample_max_vocab(void) { return SMP_MAX_V; }

extern "C" int ttsp_sample_topk(const void* L, int V, int dtype, const void* TEMP, const void* TOPP,
                                const long long* TOPK, const float* U, int* OUT, void* stream) {
  if (!L || !TEMP || !TOPP || !TOPK || !U || !OUT || V <= 0 || V > SMP_MAX_V) return (int)hipErrorInvalidValue;
  hipStream_t st = (hipStream_t)stream;
  if (dtype == DT_BF16)
    hipLaunchKernelGGL(sample_topk_kernel<DT_BF16>, dim3(1), dim3(SMP_THREADS), 0, st, (const uint16_t*)L, V,
                       (const uint16_t*)TEMP, (const uint16_t*)TOPP, TOPK, U, OUT);
  else if (dtype == DT_F16)
    hipLaunchKernelGGL(sample_topk_kernel<DT_F16>, dim3(1), dim3(SMP_THREADS), 0, st, (const uint16_t*)L, V,
                       (const uint16_t*)TEMP, (const uint16_t*)TOPP, TOPK, U, OUT);
  else
    return (int)hipErrorInvalidValue;
  TTSP_RETURN_LAUNCH();
}
