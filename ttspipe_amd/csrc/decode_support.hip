// Small kernels a greedy Dual-AR decode step needs between the transformer
// blocks (the synthetic frame of app/engine/graphs.py:76-132 with argmax in
// place of sampling): summed codebook-embedding gather, greedy argmax (alone,
// or with the embedding row it selects), the frame's bookkeeping, and a
// counter-based fill that materialises seeded synthetic weights on the device.
#include "ttsp_common.h"

#include <type_traits>

namespace ttsp {

// out[r][d] = round(sum_{c < ntok} E[(c * vocab + t) * D + d]) with t =
// tok[c * tok_stride + r] clamped into [0, vocab): each row's fp32 sum in
// codebook order (one row: a decode step's embedding sum). V = 8: a
// thread per 8 consecutive values (16-byte loads; D % 8 == 0 and E, out
// 16-byte aligned), V = 1: a thread per value. Up to EMB_ROWS_T tables the
// token loads, then the table loads, are all issued before the first add.
constexpr int EMB_ROWS_T = 16;
template <int DT, int V>
__global__ __launch_bounds__(256) void embed_sum_rows_kernel(const uint16_t* __restrict__ E,
                                                            const int* __restrict__ tok, long long tok_stride,
                                                            int ntok, int rows, int vocab, int D,
                                                            uint16_t* __restrict__ out) {
  using Vec = typename std::conditional<V == 8, uint4, uint16_t>::type;
  const int per_row = D / V;
  const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (long long)per_row * rows) return;
  const int r = (int)(i / per_row), d = (int)(i % per_row) * V;
  float acc[V];
#pragma unroll
  for (int k = 0; k < V; ++k) acc[k] = 0.0f;
  auto add = [&](const Vec& w) {
    if constexpr (V == 8) {
      const uint32_t u[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        acc[2 * k] = __fadd_rn(acc[2 * k], Elem<DT>::load(u[k]));
        acc[2 * k + 1] = __fadd_rn(acc[2 * k + 1], Elem<DT>::load(u[k] >> 16));
      }
    } else {
      acc[0] = __fadd_rn(acc[0], Elem<DT>::load(w));
    }
  };
  auto row_of = [&](int c) {
    int t = tok[c * tok_stride + r];
    t = t < 0 ? 0 : (t >= vocab ? vocab - 1 : t);
    return reinterpret_cast<const Vec*>(E + ((size_t)c * vocab + t) * D + d);
  };
  if (ntok <= EMB_ROWS_T) {
    const Vec* src[EMB_ROWS_T];
    Vec w[EMB_ROWS_T];
#pragma unroll
    for (int c = 0; c < EMB_ROWS_T; ++c)
      if (c < ntok) src[c] = row_of(c);
#pragma unroll
    for (int c = 0; c < EMB_ROWS_T; ++c)
      if (c < ntok) w[c] = *src[c];
#pragma unroll
    for (int c = 0; c < EMB_ROWS_T; ++c)
      if (c < ntok) add(w[c]);
  } else {
    for (int c = 0; c < ntok; ++c) add(*row_of(c));
  }
  uint16_t* o = out + (size_t)r * D + d;
  if constexpr (V == 8) {
    uint32_t w[4];
#pragma unroll
    for (int k = 0; k < 4; ++k)
      w[k] = (uint32_t)Elem<DT>::store(acc[2 * k]) | ((uint32_t)Elem<DT>::store(acc[2 * k + 1]) << 16);
    *reinterpret_cast<uint4*>(o) = make_uint4(w[0], w[1], w[2], w[3]);
  } else {
    o[0] = Elem<DT>::store(acc[0]);
  }
}

// Index of the largest of X[0..n), the lowest index on ties (NaN never wins;
// 0 when nothing beats -inf), valid in thread 0 after the call. One workgroup.
// A thread scans 8-element chunks (16-byte loads when X is 16-byte aligned),
// four chunks' loads issued before the first compare, in rising index order.
template <int DT>
__device__ __forceinline__ int block_argmax(const uint16_t* __restrict__ X, int n) {
  __shared__ float bv[16];
  __shared__ int bi[16];
  const int tid = threadIdx.x, nthr = blockDim.x;
  float best = -__builtin_inff();
  int idx = 0x7fffffff;
  if ((reinterpret_cast<uintptr_t>(X) & 15) == 0) {
    const int nch = n >> 3;  // whole chunks; the tail below
    constexpr int U = 4;
    for (int c0 = tid; c0 < nch; c0 += U * nthr) {
      uint4 v[U];
#pragma unroll
      for (int u = 0; u < U; ++u) v[u] = *reinterpret_cast<const uint4*>(X + 8 * (size_t)min(c0 + u * nthr, nch - 1));
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int c = c0 + u * nthr;
        if (c >= nch) break;
        const uint32_t w[4] = {v[u].x, v[u].y, v[u].z, v[u].w};
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float x = Elem<DT>::load((uint16_t)(w[e >> 1] >> (16 * (e & 1))));
          if (x > best) { best = x; idx = 8 * c + e; }
        }
      }
    }
    for (int i = 8 * nch + tid; i < n; i += nthr) {
      const float x = Elem<DT>::load(X[i]);
      if (x > best) { best = x; idx = i; }
    }
  } else {
    for (int i = tid; i < n; i += nthr) {
      const float x = Elem<DT>::load(X[i]);
      if (x > best) { best = x; idx = i; }
    }
  }
  for (int off = 32; off >= 1; off >>= 1) {
    const float ov = __shfl_xor(best, off, 64);
    const int oi = __shfl_xor(idx, off, 64);
    if (ov > best || (ov == best && oi < idx)) { best = ov; idx = oi; }
  }
  if ((tid & 63) == 0) { bv[tid >> 6] = best; bi[tid >> 6] = idx; }
  __syncthreads();
  if (tid == 0) {
    const int nw = (blockDim.x + 63) >> 6;
    for (int w = 1; w < nw; ++w)
      if (bv[w] > best || (bv[w] == best && bi[w] < idx)) { best = bv[w]; idx = bi[w]; }
  }
  return idx == 0x7fffffff ? 0 : idx;
}

template <int DT>
__global__ __launch_bounds__(1024) void argmax_kernel(const uint16_t* __restrict__ X, int n,
                                                     int* __restrict__ out) {
  const int idx = block_argmax<DT>(X, n);
  if (threadIdx.x == 0) out[0] = idx;
}

// The greedy token and the embedding row it selects, in one launch (argmax
// then a one-row embed_sum): tok[0] = argmax(X[0..n)), t = that clamped into
// [0, vocab), tok2[0] = t when tok2 is given, out[d] = round(0 + E[t D + d])
// (embed_sum's arithmetic for one row).
template <int DT>
__global__ __launch_bounds__(1024) void argmax_embed_kernel(const uint16_t* __restrict__ X, int n,
                                                           int* __restrict__ tok, int* __restrict__ tok2,
                                                           const uint16_t* __restrict__ E, int vocab, int D,
                                                           uint16_t* __restrict__ out) {
  __shared__ int t_s;
  const int idx = block_argmax<DT>(X, n);
  if (threadIdx.x == 0) {
    const int t = idx < 0 ? 0 : (idx >= vocab ? vocab - 1 : idx);
    tok[0] = idx;
    if (tok2) tok2[0] = t;
    t_s = t;
  }
  __syncthreads();
  const uint16_t* row = E + (size_t)t_s * D;
  for (int d = threadIdx.x; d < D; d += blockDim.x) out[d] = Elem<DT>::store(__fadd_rn(0.0f, Elem<DT>::load(row[d])));
}

// A decode frame's bookkeeping in one launch: history[step] = tokens (ntok
// entries; nothing once step is outside [0, rows)), step += 1, pos += 1, and
// the next frame's rotary row frow = F[pos] (row_elems 16-bit values; pos
// clamped into [0, npos)). Every thread reads step and pos before thread 0
// writes them.
__global__ __launch_bounds__(256) void frame_advance_kernel(const int* __restrict__ tokens, int ntok,
                                                            int* __restrict__ history, int rows,
                                                            long long* __restrict__ step, long long* __restrict__ pos,
                                                            const uint16_t* __restrict__ F, int npos, int row_elems,
                                                            uint16_t* __restrict__ frow) {
  const long long s = step[0], p = pos[0] + 1;
  const long long pr = p < 0 ? 0 : (p >= npos ? npos - 1 : p);
  for (int i = threadIdx.x; i < ntok; i += blockDim.x)
    if (s >= 0 && s < rows) history[s * ntok + i] = tokens[i];
  for (int i = threadIdx.x; i < row_elems; i += blockDim.x) frow[i] = F[pr * row_elems + i];
  __syncthreads();
  if (threadIdx.x == 0) {
    step[0] = s + 1;
    pos[0] = p;
  }
}

// splitmix64 (Steele, Lea, Flood 2014) of seed-mixed counters.
__device__ __forceinline__ uint64_t mix64(uint64_t z) {
  z += 0x9e3779b97f4a7c15ull;
  z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
  z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
  return z ^ (z >> 31);
}

__device__ __forceinline__ uint64_t hash_at(uint64_t seed, uint64_t i) {
  return mix64(mix64(seed) ^ i);
}

// kind 0: bytes (top 8 bits); kind 1/2/3: value = u * scale + offset with
// u = (h >> 40) / 2^23 - 1 in [-1, 1) (exact in fp32), one rounding per op,
// stored as bf16 / fp16 / fp32.
__global__ __launch_bounds__(256) void synth_fill_kernel(void* __restrict__ out, long long n,
                                                         unsigned long long seed, int kind,
                                                         float scale, float offset) {
  const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const uint64_t h = hash_at(seed, (uint64_t)i);
  if (kind == 0) {
    ((uint8_t*)out)[i] = (uint8_t)(h >> 56);
    return;
  }
  const float u = __fsub_rn(__fmul_rn((float)(uint32_t)(h >> 40), 1.1920928955078125e-07f), 1.0f);
  const float v = __fadd_rn(__fmul_rn(u, scale), offset);
  if (kind == 1) ((uint16_t*)out)[i] = f32_to_bf16(v);
  else if (kind == 2) ((uint16_t*)out)[i] = f32_to_f16(v);
  else ((float*)out)[i] = v;
}

}  // namespace ttsp

using namespace ttsp;

extern "C" int ttsp_embed_sum_rows(const void* E, const int* tok, long long tok_stride, int ntok, int rows,
                                   int vocab, int D, void* out, int dtype, hipStream_t stream) {
  if (ntok <= 0 || rows <= 0 || vocab <= 0 || D <= 0 || tok_stride < rows || !E || !tok || !out)
    return (int)hipErrorInvalidValue;
  const bool vec = D % 8 == 0 && (uintptr_t)E % 16 == 0 && (uintptr_t)out % 16 == 0;
  const long long threads = (long long)(vec ? D / 8 : D) * rows;
  if (threads > (1LL << 31) - 256) return (int)hipErrorInvalidValue;
  const dim3 grid((unsigned)((threads + 255) / 256));
#define TTSP_ER(DTV, VV)                                                                                    \
  hipLaunchKernelGGL((embed_sum_rows_kernel<DTV, VV>), grid, dim3(256), 0, stream, (const uint16_t*)E, tok, \
                     tok_stride, ntok, rows, vocab, D, (uint16_t*)out)
  if (dtype == DT_F16) {
    if (vec) TTSP_ER(DT_F16, 8);
    else TTSP_ER(DT_F16, 1);
  } else if (dtype == DT_BF16) {
    if (vec) TTSP_ER(DT_BF16, 8);
    else TTSP_ER(DT_BF16, 1);
  } else {
    return (int)hipErrorInvalidValue;
  }
#undef TTSP_ER
  TTSP_RETURN_LAUNCH();
}

// one position: the rows kernel with one row (every token load, then every
// table load, issued before the first add)
extern "C" int ttsp_embed_sum(const void* E, const int* tok, int ntok, int vocab, int D, void* out,
                              int dtype, hipStream_t stream) {
  return ttsp_embed_sum_rows(E, tok, 1, ntok, 1, vocab, D, out, dtype, stream);
}

extern "C" int ttsp_argmax_embed(const void* X, int n, int dtype, int* tok, int* tok2, const void* E, int vocab,
                                 int D, void* out, hipStream_t stream) {
  if (n <= 0 || vocab <= 0 || D <= 0 || !X || !tok || !E || !out) return (int)hipErrorInvalidValue;
  if (dtype == DT_F16)
    hipLaunchKernelGGL(argmax_embed_kernel<DT_F16>, dim3(1), dim3(1024), 0, stream, (const uint16_t*)X, n, tok, tok2,
                       (const uint16_t*)E, vocab, D, (uint16_t*)out);
  else if (dtype == DT_BF16)
    hipLaunchKernelGGL(argmax_embed_kernel<DT_BF16>, dim3(1), dim3(1024), 0, stream, (const uint16_t*)X, n, tok, tok2,
                       (const uint16_t*)E, vocab, D, (uint16_t*)out);
  else
    return (int)hipErrorInvalidValue;
  TTSP_RETURN_LAUNCH();
}

extern "C" int ttsp_frame_advance(const int* tokens, int ntok, int* history, int rows, long long* step,
                                  long long* pos, const void* F, int npos, int row_elems, void* frow,
                                  hipStream_t stream) {
  if (ntok <= 0 || rows <= 0 || npos <= 0 || row_elems <= 0 || !tokens || !history || !step || !pos || !F || !frow)
    return (int)hipErrorInvalidValue;
  hipLaunchKernelGGL(frame_advance_kernel, dim3(1), dim3(256), 0, stream, tokens, ntok, history, rows, step, pos,
                     (const uint16_t*)F, npos, row_elems, (uint16_t*)frow);
  TTSP_RETURN_LAUNCH();
}

extern "C" int ttsp_argmax(const void* X, int n, int dtype, int* out, hipStream_t stream) {
  if (n <= 0) return (int)hipErrorInvalidValue;
  if (dtype == DT_F16)
    hipLaunchKernelGGL(argmax_kernel<DT_F16>, dim3(1), dim3(1024), 0, stream, (const uint16_t*)X, n, out);
  else if (dtype == DT_BF16)
    hipLaunchKernelGGL(argmax_kernel<DT_BF16>, dim3(1), dim3(1024), 0, stream, (const uint16_t*)X, n, out);
  else
    return (int)hipErrorInvalidValue;
  TTSP_RETURN_LAUNCH();
}

extern "C" int ttsp_synth_fill(void* out, long long n, unsigned long long seed, int kind, float scale,
                               float offset, hipStream_t stream) {
  if (n < 0 || kind < 0 || kind > 3) return (int)hipErrorInvalidValue;
  if (n == 0) return 0;
  hipLaunchKernelGGL(synth_fill_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream, out,
                     n, seed, kind, scale, offset);
  TTSP_RETURN_LAUNCH();
}
