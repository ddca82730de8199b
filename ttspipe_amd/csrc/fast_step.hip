// The fast transformer's codebook steps in one launch (the Dual-AR frame's
// inner loop, reference app/engine/graphs.py:126-131): for each codebook step,
// every fast layer - [RMSNorm + wqkv], [q/k head norms + rotary + KV write +
// attention, then wo + residual], [RMSNorm + w1/w3 SwiGLU], [w2 + residual] -
// then [final norm + head], then the greedy token and its embedding row, which
// is the next step's input. Launched as kernels, that is 18 launches a step,
// each paying the launch gap and its own start-up; here it is 17 phases a step
// separated by grid barriers, with each phase's weights and scales requested
// before the barrier that releases its input.
//
// Results are the launched kernels' bits: every phase is the NF4 GEMV's
// arithmetic (nf4_gemv.hip: the same replicated code-pair table, lane l owning
// dwords l + 64 j of each row, the 8-product fp32 chain per dword and its block
// scale, the DPP lane sum, the same epilogue roundings, the folded RMSNorm's
// chunk and wave order), the attention is the attention-prologue form's, and
// the token is argmax_embed_kernel's (largest logit, lowest index on ties).
// Only phases whose matrices the GEMV runs unsplit along K (KS = 1) are
// served; the host declines the rest.
//
// Workgroups exchange activations through global memory with device-scope
// (write-through, L2-bypassing) stores and loads, and meet at grid barriers:
// each workgroup waits for its own stores to complete, then one thread adds to
// a counter; waiters poll it. Every wait is bounded: past FS_SPIN polls the
// workgroup stops waiting and counts the failure in sync[128] (the results are
// then garbage and the host reports an error; no wave ever waits forever).
// The grid is one workgroup per CU at most, all resident at once (the launch
// before this one has drained: same stream).
#include <mutex>

#include "gemv_common.h"
#define TTSP_HIP_TYPES_ONLY
#include "../../include/ttsp_hip.h"

extern "C" int ttsp_gemv_shape(int M, int K, int* J, int* KS, int* RPW);

namespace ttsp {

constexpr int FS_MAX_LAYERS = 4;
constexpr unsigned FS_SPIN = 1u << 18;  // polls of a barrier before giving up (each a memory round trip: > 0.1 s)

struct FsLin {
  const uint32_t* W;
  const uint8_t* A8;   // nested: scale indices; plain: AMAX again (read, unused)
  const float* AMAX;
  const float* CODE2;  // nested: 256 fp32; plain: the LUT (read, unused)
  float offset;
};

struct FsLayer {
  FsLin wqkv, wo, w1, w3, w2;
  const uint16_t *an, *fn, *qn, *kn;  // norm weights (qn / kn: any readable memory when unused)
  uint16_t *KC, *VC;                  // [nkv][max_len][128]
};

struct FsArgs {
  FsLayer L[FS_MAX_LAYERS];
  FsLin head;
  const uint16_t* hn;       // the final (fast) norm weight
  const uint16_t* emb;      // embeddings [vocab][D]
  const float* LUT;         // the 16 NF4 code points
  const void* freqs;        // rotary table, rows [max_len][64][2] of ftype
  const uint16_t* x0;       // the first step's input row [D]
  uint16_t *qkv, *h, *g, *x, *logits;  // exchanged activations
  int* tokens;              // tokens[step + 1] = the step's greedy token
  unsigned* sync;           // [0] barrier counter, [64] exit counter, [128] failed waits; zero at launch
  int D, nh, nkv, inter, vocab, nl, max_len, step0, nsteps;
  int ftype, dt, bs_shift, bs2_shift, nested, qn, kn;
  float eps, scale;
};

// device-scope (cross-XCD coherent) accesses
// (global address space: the loads are global_load rather than flat_load)
typedef __attribute__((address_space(1))) uint32_t gu32;
typedef __attribute__((address_space(1))) uint16_t gu16;
__device__ __forceinline__ uint32_t ld_dev(const void* p) {
  return __hip_atomic_load((gu32*)(const_cast<void*>(p)), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ u32x4 ld_dev4(const void* p) {
  const uint32_t* q = reinterpret_cast<const uint32_t*>(p);
  return u32x4{ld_dev(q), ld_dev(q + 1), ld_dev(q + 2), ld_dev(q + 3)};
}
__device__ __forceinline__ uint16_t ld_dev16(const uint16_t* p) {
  const uintptr_t a = reinterpret_cast<uintptr_t>(p);
  const uint32_t w = ld_dev(reinterpret_cast<const void*>(a & ~(uintptr_t)3));
  return (uint16_t)(a & 2 ? w >> 16 : w);
}
__device__ __forceinline__ void st_dev16(uint16_t* p, uint16_t v) {
  __hip_atomic_store((gu16*)p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// The grid barrier: arrive after every store of the workgroup completed
// (each arrival raises the count the next wait needs by G); wait until the
// counter reaches it. `ok` turns false for good after a wait that gave up.
struct FsSync {
  unsigned* cnt;
  unsigned* fail;
  unsigned target;
  bool ok;
};
__device__ __forceinline__ void fs_arrive(FsSync& s) {
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (threadIdx.x == 0) __hip_atomic_fetch_add(s.cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  s.target += gridDim.x;
}
__device__ __forceinline__ void fs_wait(FsSync& s, int* ok_s) {
  if (threadIdx.x == 0) {
    bool ok = s.ok;
    if (ok) {
      unsigned it = 0;
      while (ld_dev(s.cnt) < s.target) {
        if (++it > FS_SPIN) {
          ok = false;
          __hip_atomic_fetch_add(s.fail, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          break;
        }
        __builtin_amdgcn_s_sleep(1);
      }
    }
    *ok_s = ok;
  }
  __syncthreads();
  s.ok = *ok_s != 0;
}

// One phase's weight side, requested before the barrier: the wave's RPW rows
// of NM weights, J dwords each, and each dword's raw scale.
template <int J, int RPW, int NM>
struct FsW {
  uint32_t w[NM][RPW][J];
  uint32_t a8[NM][RPW][J];
  float am[NM][RPW][J];
  u32x4 c2[NM];
};

template <int J, int RPW, int NM>
__device__ __forceinline__ void fs_issue(FsW<J, RPW, NM>& f, const FsLin* L, int M, int K, int row0, bool nested,
                                         int bs_shift, int bs2_shift, int lane) {
  const int KD = K >> 3, nblk = K >> bs_shift, sh = bs_shift - 3;
#pragma unroll
  for (int m = 0; m < NM; ++m) {
    f.c2[m] = *reinterpret_cast<const u32x4*>(L[m].CODE2 + (nested ? 4 * lane : 0));
#pragma unroll
    for (int r = 0; r < RPW; ++r) {
      const uint32_t row = (uint32_t)uniform(min(row0 + r, M - 1));
      const uint32_t* wr = L[m].W + (size_t)row * KD;
#pragma unroll
      for (int j = 0; j < J; ++j) {
        const int d = min(lane + 64 * j, KD - 1);
        f.w[m][r][j] = __builtin_nontemporal_load(wr + d);
        const uint32_t b = row * (uint32_t)nblk + (uint32_t)(d >> sh);
        f.a8[m][r][j] = L[m].A8[b];
        f.am[m][r][j] = L[m].AMAX[nested ? b >> bs2_shift : b];
      }
    }
  }
}

// LDS of the kernel: the table (static), then code2 [2][256], norm partials
// [8], x [K <= 4096], the attention prologue's buffers.
struct FsLds {
  float* code2;
  float* wpart;
  uint4* xs;
  unsigned char* att;
};

// The GEMV of one phase on the staged x (LDS): rows row0 .. row0 + RPW - 1 of
// the wave, result stored with the epilogue (device-scope stores).
template <int J, int RPW, int NM>
__device__ __forceinline__ void fs_dot(const FsW<J, RPW, NM>& f, const FsLds& s, const uint32_t* lut_rep,
                                       const FsLin* L, int M, int K, int row0, int dt, bool nested, int epi,
                                       const uint16_t* R, bool r_emb, uint16_t* Y, int lane) {
  const int KD = K >> 3;
  // scales (code2 already in LDS): two fp32 roundings, as the standalone kernel
  float sc[NM][RPW][J];
#pragma unroll
  for (int m = 0; m < NM; ++m)
#pragma unroll
    for (int r = 0; r < RPW; ++r)
#pragma unroll
      for (int j = 0; j < J; ++j)
        sc[m][r][j] = nested ? __fadd_rn(__fmul_rn(s.code2[m * 256 + f.a8[m][r][j]], f.am[m][r][j]), L[m].offset)
                             : f.am[m][r][j];
  F8 xf[J];
#pragma unroll
  for (int j = 0; j < J; ++j) {
    const int d = lane + 64 * j;
    const uint4 v = s.xs[min(d, KD - 1)];
    const uint4 xz = d < KD ? v : make_uint4(0, 0, 0, 0);
    xf[j] = dt == DT_BF16 ? to_f32<DT_BF16>(xz) : to_f32<DT_F16>(xz);
  }
  const uint32_t lane4 = (uint32_t)lane * 4u;
  const unsigned char* lut_b = reinterpret_cast<const unsigned char*>(lut_rep);
  float tot[NM][RPW];
#pragma unroll
  for (int m = 0; m < NM; ++m)
#pragma unroll
    for (int r = 0; r < RPW; ++r) {
      float acc = 0.0f;
#pragma unroll
      for (int j = 0; j < J; ++j) {
        uint32_t cp[4];
#pragma unroll
        for (int b = 0; b < 4; ++b)
          cp[b] = *reinterpret_cast<const uint32_t*>(lut_b + __builtin_amdgcn_perm(f.w[m][r][j], lane4,
                                                                                  0x0C0C0400u + (b << 8)));
        float q = __builtin_fmaf(h_lo(cp[0]), xf[j].v[0], 0.0f);
        q = __builtin_fmaf(h_hi(cp[0]), xf[j].v[1], q);
        q = __builtin_fmaf(h_lo(cp[1]), xf[j].v[2], q);
        q = __builtin_fmaf(h_hi(cp[1]), xf[j].v[3], q);
        q = __builtin_fmaf(h_lo(cp[2]), xf[j].v[4], q);
        q = __builtin_fmaf(h_hi(cp[2]), xf[j].v[5], q);
        q = __builtin_fmaf(h_lo(cp[3]), xf[j].v[6], q);
        q = __builtin_fmaf(h_hi(cp[3]), xf[j].v[7], q);
        acc = __builtin_fmaf(q, sc[m][r][j], acc);
      }
      tot[m][r] = wave_sum_dpp(acc);
    }
  float mine[NM];
#pragma unroll
  for (int m = 0; m < NM; ++m) {
    mine[m] = tot[m][0];
#pragma unroll
    for (int r = 1; r < RPW; ++r) mine[m] = lane == r ? tot[m][r] : mine[m];
  }
  const int row = row0 + lane;
  if (lane < RPW && row < M) {
    if (NM == 1) {
      uint32_t rv = epi ? ld_dev16(R + row) : 0u;
      if (r_emb) rv = st16(dt, __fadd_rn(0.0f, ld16(dt, rv)));
      st_dev16(Y + row, epilogue16(dt, mine[0], epi, rv));
    } else {  // SwiGLU: w1's row gates w3's, as the two-launch form rounds it
      st_dev16(Y + row, epilogue16(dt, mine[NM - 1], 2, st16(dt, mine[0])));
    }
  }
}

// x into LDS from global (device-scope loads): chunk tid (8 values) per thread;
// with a norm weight G the fork's RMSNorm on the way (nf4_gemv.hip's folded
// norm: per-chunk fma chain, DPP wave sums, wave partials left to right).
// emb: x is an embedding row, taken as the one-row embed_sum gives it,
// round(0 + e) (a negative zero becomes +0).
__device__ __forceinline__ uint32_t emb16x2(int dt, uint32_t w) {
  return st16(dt, __fadd_rn(0.0f, ld16(dt, w))) | (st16(dt, __fadd_rn(0.0f, ld16(dt, w >> 16))) << 16);
}

__device__ __forceinline__ void fs_stage_x(const FsLds& s, const uint16_t* X, bool emb, const uint16_t* G, int K,
                                           float eps, int dt, int tid, int lane, int wave) {
  const int KD = K >> 3;
  u32x4 v = tid < KD ? ld_dev4(X + 8 * tid) : u32x4{0u, 0u, 0u, 0u};
  if (emb) v = u32x4{emb16x2(dt, v[0]), emb16x2(dt, v[1]), emb16x2(dt, v[2]), emb16x2(dt, v[3])};
  const uint4 xc = make_uint4(v[0], v[1], v[2], v[3]);
  if (!G) {
    if (tid < KD) s.xs[tid] = xc;
    __syncthreads();
    return;
  }
  const uint4 gc = *reinterpret_cast<const uint4*>(G + 8 * min(tid, KD - 1));
  float sq = 0.0f;
  if (tid < KD) sq = dt == DT_BF16 ? sumsq8<DT_BF16>(xc, 0.0f) : sumsq8<DT_F16>(xc, 0.0f);
  sq = wave_sum_dpp(sq);
  if (lane == 0) s.wpart[wave] = sq;
  __syncthreads();
  float ss = s.wpart[0];
#pragma unroll
  for (int w2 = 1; w2 < GEMV_WAVES; ++w2) ss = __fadd_rn(ss, s.wpart[w2]);
  const float r = rsqrt_rn(__fadd_rn(__fdiv_rn(ss, (float)K), eps));
  if (tid < KD) s.xs[tid] = dt == DT_BF16 ? norm8<DT_BF16>(xc, gc, r) : norm8<DT_F16>(xc, gc, r);
  __syncthreads();
}

// The attention prologue (nf4_gemv.hip's ATT form: all heads of one position
// over a cache of at most one chunk), its output rounded into x (LDS). The
// cached rows and the per-head constants are requested before the barrier;
// QKV after it. Workgroup 0 writes the new K/V row (device-scope stores).
struct FsAttPre {
  uint16_t aqw0, aqw1, akw0, akw1;
  RopeF rf;
  u32x4 kq[ATT_PER], vq[ATT_PER];
};

__device__ __forceinline__ void fs_att_issue(FsAttPre& a, const FsArgs& p, const FsLayer& Ly, int pos, int tid,
                                             int lane) {
  a.aqw0 = Ly.qn[lane];
  a.aqw1 = Ly.qn[lane + 64];
  a.akw0 = Ly.kn[lane];
  a.akw1 = Ly.kn[lane + 64];
  a.rf = load_rope(reinterpret_cast<const unsigned char*>(p.freqs) + (size_t)pos * HD * (p.ftype == DT_F32 ? 4 : 2),
                   p.ftype, lane);
  const int npc = p.nkv * p.max_len * (HD / 8);
#pragma unroll
  for (int i = 0; i < ATT_PER; ++i) {
    const int t = min(tid + i * GEMV_THREADS, npc - 1);
    const int kvh = t / (p.max_len * (HD / 8)), j = (t / (HD / 8)) % p.max_len, e = (t % (HD / 8)) * 8;
    const size_t off = ((size_t)kvh * p.max_len + j) * HD + e;
    a.kq[i] = ld_dev4(Ly.KC + off);
    a.vq[i] = ld_dev4(Ly.VC + off);
  }
}

__device__ __forceinline__ void fs_attention(const FsAttPre& a, const FsArgs& p, const FsLayer& Ly, const FsLds& s,
                                             int pos, int tid, int lane, int wave) {
  const int dt = p.dt, nh = p.nh, nkv = p.nkv, groups = p.nh / p.nkv, max_len = p.max_len;
  const int Rl = att_r16(max_len);
  const int head = min(wave, nh - 1), kvh = head / groups;
  float* q_s = reinterpret_cast<float*>(s.att);                           // [8][128]
  float* p_s = q_s + ATT_MAX_HEADS * HD;                                  // [8][64]
  uint16_t* k_s = reinterpret_cast<uint16_t*>(p_s + ATT_MAX_HEADS * ACHUNK);  // [nkv][R16][KPAD]
  uint16_t* v_s = k_s + (size_t)nkv * Rl * KPAD;                          // [nkv][R16][HD]
  const uint16_t* qr = p.qkv + (size_t)head * HD;
  const uint16_t* kr = p.qkv + (size_t)(nh + kvh) * HD;
  const uint16_t* vr = p.qkv + (size_t)(nh + nkv + kvh) * HD;
  const uint16_t aq0 = ld_dev16(qr + lane), aq1 = ld_dev16(qr + lane + 64);
  const uint16_t ak0 = ld_dev16(kr + lane), ak1 = ld_dev16(kr + lane + 64);
  const uint16_t av0 = ld_dev16(vr + lane), av1 = ld_dev16(vr + lane + 64);
  const bool pos_ok = pos >= 0 && pos < max_len;
  const int jpos = pos_ok ? pos : 0, nvalid = jpos + 1;
  const bool qwave = wave < nh, newrow = qwave && wave % groups == 0;
  uint16_t klo = 0, khi = 0;
  if (qwave) {
    float lo = ld16(dt, aq0), hi = ld16(dt, aq1);
    if (dt == DT_BF16) head_norm_rope<DT_BF16>(lo, hi, p.qn, a.aqw0, a.aqw1, p.eps, a.rf, lane);
    else head_norm_rope<DT_F16>(lo, hi, p.qn, a.aqw0, a.aqw1, p.eps, a.rf, lane);
    q_s[wave * HD + lane] = __fmul_rn(ld16(dt, st16(dt, lo)), p.scale);
    q_s[wave * HD + lane + 64] = __fmul_rn(ld16(dt, st16(dt, hi)), p.scale);
  }
  if (newrow) {
    float lo = ld16(dt, ak0), hi = ld16(dt, ak1);
    if (dt == DT_BF16) head_norm_rope<DT_BF16>(lo, hi, p.kn, a.akw0, a.akw1, p.eps, a.rf, lane);
    else head_norm_rope<DT_F16>(lo, hi, p.kn, a.akw0, a.akw1, p.eps, a.rf, lane);
    klo = (uint16_t)st16(dt, lo);
    khi = (uint16_t)st16(dt, hi);
    uint16_t* kd = k_s + ((size_t)kvh * Rl + jpos) * KPAD;
    uint16_t* vd = v_s + ((size_t)kvh * Rl + jpos) * HD;
    kd[lane] = klo;
    kd[lane + 64] = khi;
    vd[lane] = av0;
    vd[lane + 64] = av1;
  }
  const int npc = nkv * max_len * (HD / 8);
#pragma unroll
  for (int i = 0; i < ATT_PER; ++i) {
    const int t = tid + i * GEMV_THREADS;
    const int kh = t / (max_len * (HD / 8)), j = (t / (HD / 8)) % max_len, e = (t % (HD / 8)) * 8;
    if (t < npc && j != jpos) {
      *reinterpret_cast<u32x4*>(k_s + ((size_t)kh * Rl + j) * KPAD + e) = a.kq[i];
      *reinterpret_cast<u32x4*>(v_s + ((size_t)kh * Rl + j) * HD + e) = a.vq[i];
    }
  }
  __syncthreads();
  if (qwave) {
    const uint16_t* krow = k_s + ((size_t)kvh * Rl + min(lane, max_len - 1)) * KPAD;
    const float sc = dt == DT_BF16 ? score4<DT_BF16>(q_s + wave * HD, krow) : score4<DT_F16>(q_s + wave * HD, krow);
    const bool valid = lane < nvalid;
    const float m = wave_max_u(valid ? sc : -3.0e38f);
    const float pr = valid ? exp_cw(__fsub_rn(sc, m)) : 0.0f;
    const float l = wave_sum_dpp(pr);
    p_s[wave * ACHUNK + lane] = pr;  // read back by this wave only
    float a0, a1;
    const uint16_t* vs = v_s + (size_t)kvh * Rl * HD;
    if (dt == DT_BF16) pv4<DT_BF16>(p_s + wave * ACHUNK, vs, nvalid, lane, a0, a1);
    else pv4<DT_F16>(p_s + wave * ACHUNK, vs, nvalid, lane, a0, a1);
    const float wt = exp_cw(__fsub_rn(m, m));
    const float den = __fadd_rn(0.0f, __fmul_rn(l, wt));
    const float y0 = __fdiv_rn(__fadd_rn(0.0f, __fmul_rn(a0, wt)), den);
    const float y1 = __fdiv_rn(__fadd_rn(0.0f, __fmul_rn(a1, wt)), den);
    reinterpret_cast<uint32_t*>(s.xs)[wave * 64 + lane] = st16(dt, y0) | (st16(dt, y1) << 16);
  }
  if (newrow && pos_ok && blockIdx.x == 0) {
    const size_t row = ((size_t)kvh * max_len + pos) * HD;
    st_dev16(Ly.KC + row + lane, klo);
    st_dev16(Ly.KC + row + lane + 64, khi);
    st_dev16(Ly.VC + row + lane, av0);
    st_dev16(Ly.VC + row + lane + 64, av1);
  }
  __syncthreads();
}

// Greedy token of the step's logits (device-scope loads), as argmax_embed_kernel:
// the largest value, the lowest index on ties, NaN never wins, 0 when nothing
// beats -inf. The same in every workgroup.
__device__ __forceinline__ int fs_argmax(const uint16_t* X, int n, int dt, float* bv, int* bi, int tid, int lane,
                                         int wave) {
  float best = -__builtin_inff();
  int idx = 0x7fffffff;
  for (int i = tid; i < n; i += GEMV_THREADS) {
    const float v = ld16(dt, ld_dev16(X + i));
    if (v > best) { best = v; idx = i; }
  }
  for (int off = 32; off >= 1; off >>= 1) {
    const float ov = __shfl_xor(best, off, 64);
    const int oi = __shfl_xor(idx, off, 64);
    if (ov > best || (ov == best && oi < idx)) { best = ov; idx = oi; }
  }
  if (lane == 0) { bv[wave] = best; bi[wave] = idx; }
  __syncthreads();
  best = bv[0];
  idx = bi[0];
  for (int w = 1; w < GEMV_WAVES; ++w)
    if (bv[w] > best || (bv[w] == best && bi[w] < idx)) { best = bv[w]; idx = bi[w]; }
  __syncthreads();
  return idx == 0x7fffffff ? 0 : idx;
}

// Per-phase launch shape: J chunks a lane (K split 1) and RPW rows a wave.
template <int JQ_, int JO_, int J13_, int J2_, int JH_, int RQ_, int RO_, int R13_, int R2_, int RH_>
struct FsShape {
  static constexpr int JQ = JQ_, JO = JO_, J13 = J13_, J2 = J2_, JH = JH_;
  static constexpr int RQ = RQ_, RO = RO_, R13 = R13_, R2 = R2_, RH = RH_;
};

template <class S>
__global__ __launch_bounds__(GEMV_THREADS) void fast_steps_kernel(const FsArgs p) {
  __shared__ __align__(16) uint32_t lut_rep[256 * LUT_REP];
  extern __shared__ __align__(16) unsigned char lds_dyn[];
  __shared__ float code_s[16];
  __shared__ int ok_s;
  __shared__ float am_v[GEMV_WAVES];
  __shared__ int am_i[GEMV_WAVES];
  const int tid = threadIdx.x, lane = tid & 63, wave = uniform(tid >> 6);
  const int b = blockIdx.x;
  FsLds s;
  s.code2 = reinterpret_cast<float*>(lds_dyn);   // [2][256]
  s.wpart = s.code2 + 512;                       // [8]
  s.xs = reinterpret_cast<uint4*>(s.wpart + 8);  // [512] (K <= 4096)
  s.att = reinterpret_cast<unsigned char*>(s.xs + 512);
  const int dt = p.dt, bsh = p.bs_shift, b2sh = p.bs2_shift;
  const bool nested = p.nested;
  FsSync sy{p.sync, p.sync + 128, 0u, true};  // target: arrivals the next wait needs

  // the code-pair table, once for every phase (visible after the first
  // phase's staging barrier)
  if (tid < 16) code_s[tid] = p.LUT[tid];
  __syncthreads();
  for (int i = tid; i < 256 * LUT_REP; i += GEMV_THREADS) lut_rep[i] = code_pair_entry(code_s, i >> 6);

  const int D = p.D, qkv_rows = (p.nh + 2 * p.nkv) * HD, wrow = b * GEMV_WAVES + wave;
  const uint16_t* xin = p.x0;  // the step's input row: x0, then the last token's embedding row
  int tok = 0;
  bool first = true;           // the launch's first phase waits for nothing
  for (int st = 0; st < p.nsteps; ++st) {
    const int step = p.step0 + st, pos = step;  // codebook step i runs at fast position i
    if (st > 0) xin = p.emb + (size_t)tok * D;
    for (int l = 0; l < p.nl; ++l) {
      const FsLayer& Ly = p.L[l];
      const uint16_t* xl = l == 0 ? xin : p.x;  // the layer's input (and attention residual)
      {  // [norm + wqkv] -> qkv
        FsW<S::JQ, S::RQ, 1> f;
        const int row0 = wrow * S::RQ;
        fs_issue(f, &Ly.wqkv, qkv_rows, D, row0, nested, bsh, b2sh, lane);
        reinterpret_cast<u32x4*>(s.code2)[lane] = f.c2[0];
        if (!first && l > 0) fs_wait(sy, &ok_s);  // (layer 0 reads only its own token's row)
        first = false;
        fs_stage_x(s, xl, l == 0, Ly.an, D, p.eps, dt, tid, lane, wave);
        fs_dot(f, s, lut_rep, &Ly.wqkv, qkv_rows, D, row0, dt, nested, 0, nullptr, false, p.qkv, lane);
        fs_arrive(sy);
      }
      {  // [attention + wo + residual] -> h
        FsW<S::JO, S::RO, 1> f;
        FsAttPre a;
        const int row0 = wrow * S::RO;
        fs_issue(f, &Ly.wo, D, p.nh * HD, row0, nested, bsh, b2sh, lane);
        fs_att_issue(a, p, Ly, pos, tid, lane);
        reinterpret_cast<u32x4*>(s.code2)[lane] = f.c2[0];
        fs_wait(sy, &ok_s);
        fs_attention(a, p, Ly, s, pos, tid, lane, wave);
        fs_dot(f, s, lut_rep, &Ly.wo, D, p.nh * HD, row0, dt, nested, 1, xl, l == 0, p.h, lane);
        fs_arrive(sy);
      }
      {  // [norm + w1, w3 SwiGLU] -> g
        FsW<S::J13, S::R13, 2> f;
        const FsLin pair[2] = {Ly.w1, Ly.w3};
        const int row0 = wrow * S::R13;
        fs_issue(f, pair, p.inter, D, row0, nested, bsh, b2sh, lane);
        reinterpret_cast<u32x4*>(s.code2)[lane] = f.c2[0];
        reinterpret_cast<u32x4*>(s.code2 + 256)[lane] = f.c2[1];
        fs_wait(sy, &ok_s);
        fs_stage_x(s, p.h, false, Ly.fn, D, p.eps, dt, tid, lane, wave);
        fs_dot(f, s, lut_rep, pair, p.inter, D, row0, dt, nested, 0, nullptr, false, p.g, lane);
        fs_arrive(sy);
      }
      {  // [w2 + residual] -> x
        FsW<S::J2, S::R2, 1> f;
        const int row0 = wrow * S::R2;
        fs_issue(f, &Ly.w2, D, p.inter, row0, nested, bsh, b2sh, lane);
        reinterpret_cast<u32x4*>(s.code2)[lane] = f.c2[0];
        fs_wait(sy, &ok_s);
        fs_stage_x(s, p.g, false, nullptr, p.inter, p.eps, dt, tid, lane, wave);
        fs_dot(f, s, lut_rep, &Ly.w2, D, p.inter, row0, dt, nested, 1, p.h, false, p.x, lane);
        fs_arrive(sy);
      }
    }
    {  // [final norm + head] -> logits
      FsW<S::JH, S::RH, 1> f;
      const int row0 = wrow * S::RH;
      fs_issue(f, &p.head, p.vocab, D, row0, nested, bsh, b2sh, lane);
      reinterpret_cast<u32x4*>(s.code2)[lane] = f.c2[0];
      fs_wait(sy, &ok_s);
      fs_stage_x(s, p.x, false, p.hn, D, p.eps, dt, tid, lane, wave);
      fs_dot(f, s, lut_rep, &p.head, p.vocab, D, row0, dt, nested, 0, nullptr, false, p.logits, lane);
      fs_arrive(sy);
    }
    // the greedy token, in every workgroup; its embedding row is the next input
    fs_wait(sy, &ok_s);
    const int idx = fs_argmax(p.logits, p.vocab, dt, am_v, am_i, tid, lane, wave);
    if (b == 0 && tid == 0) p.tokens[step + 1] = idx;
    tok = idx < 0 ? 0 : (idx >= p.vocab ? p.vocab - 1 : idx);
  }

  // the last workgroup out resets the barrier for the next launch
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (tid == 0) {
    const unsigned old = __hip_atomic_fetch_add(p.sync + 64, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (old == gridDim.x - 1) {
      __hip_atomic_store(p.sync, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(p.sync + 64, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
}

// The served shapes: each phase's J (64-dword chunks a lane, K split 1) and
// rows a wave. J is fixed by K; the rows a wave set the grid.
using FsFast1024 = FsShape<2, 2, 2, 6, 2, 2, 1, 3, 1, 4>;  // D 1024, nh * 128 = 1024, FFN 3072
using FsFast512 = FsShape<1, 1, 1, 1, 1, 1, 1, 1, 1, 1>;   // D, nh * 128 and FFN at most 512

constexpr int FS_SYNC_WORDS = 192;

static size_t fs_dyn_lds(int nkv, int max_len) {
  return 4 * (512 + GEMV_WAVES) + 16 * 512 + att_lds(nkv, max_len);
}

template <class S>
static int fs_grid(int qkv, int D, int o_k, int inter, int vocab) {
  (void)o_k;
  auto g = [](int M, int R) { return (M + GEMV_WAVES * R - 1) / (GEMV_WAVES * R); };
  return std::max(std::max(g(qkv, S::RQ), g(D, S::RO)), std::max(std::max(g(inter, S::R13), g(D, S::R2)),
                                                                 g(vocab, S::RH)));
}

// kind 1: FsFast1024, 2: FsFast512, 0: not served.
struct FsPlan {
  int kind, grid;
};

static FsPlan fs_plan(int D, int nh, int nkv, int inter, int vocab, int max_len, int n_layers, int blocksize) {
  const FsPlan none{0, 0};
  if (n_layers < 1 || n_layers > FS_MAX_LAYERS || D <= 0 || inter <= 0 || vocab <= 0 || vocab > (1 << 20))
    return none;
  if (nh <= 0 || nkv <= 0 || nh > ATT_MAX_HEADS || nh % nkv || max_len <= 0 || max_len > ACHUNK ||
      nkv * max_len * (HD / 8) > ATT_PER * GEMV_THREADS)
    return none;
  if (blocksize < 64 || (blocksize & (blocksize - 1)) || D % 128 || inter % 128 || D % blocksize ||
      inter % blocksize || (nh * HD) % blocksize || D > 4096 || inter > 4096)
    return none;
  const int qkv = (nh + 2 * nkv) * HD;
  // each phase as the one-row GEMV launches it: unsplit along K (KS = 1)
  const int MK[5][2] = {{qkv, D}, {D, nh * HD}, {inter, D}, {D, inter}, {vocab, D}};
  int J[5];
  for (int i = 0; i < 5; ++i) {
    int j = 0, ks = 0;
    if (ttsp_gemv_shape(MK[i][0], MK[i][1], &j, &ks, nullptr) != 0 || ks != 1) return none;
    J[i] = j;
  }
  auto is = [&](int a, int b, int c, int d, int e) {
    return J[0] == a && J[1] == b && J[2] == c && J[3] == d && J[4] == e;
  };
  int kind = 0, grid = 0;
  if (is(FsFast1024::JQ, FsFast1024::JO, FsFast1024::J13, FsFast1024::J2, FsFast1024::JH)) {
    kind = 1;
    grid = fs_grid<FsFast1024>(qkv, D, nh * HD, inter, vocab);
  } else if (is(FsFast512::JQ, FsFast512::JO, FsFast512::J13, FsFast512::J2, FsFast512::JH)) {
    kind = 2;
    grid = fs_grid<FsFast512>(qkv, D, nh * HD, inter, vocab);
  }
  if (!kind || grid > 256) return none;
  return {kind, grid};
}

// Workgroups the device holds at once for a kernel (per device, cached).
static std::mutex fs_cap_mu;
static int fs_cap[64][3];

static int fs_capacity(int kind, const void* fn, size_t lds) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
  std::lock_guard<std::mutex> lock(fs_cap_mu);
  if (fs_cap[dev][kind] == 0) {
    int per_cu = 0, cus = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, GEMV_THREADS, lds) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
      return 0;
    fs_cap[dev][kind] = std::max(per_cu, 0) * std::max(cus, 0);
  }
  return fs_cap[dev][kind];
}

static FsLin fs_lin(const ttsp_nf4_weight& w) {
  // plain scales: the nested-only operands point at AMAX (read, unused)
  const bool nested = w.A8 != nullptr;
  return FsLin{reinterpret_cast<const uint32_t*>(w.W), nested ? w.A8 : reinterpret_cast<const uint8_t*>(w.AMAX),
               w.AMAX, nested ? w.CODE2 : w.AMAX, w.offset};
}

static bool fs_weight_ok(const ttsp_nf4_weight& w, bool nested) {
  return w.W && w.AMAX && (w.A8 != nullptr) == nested && (!nested || w.CODE2) &&
         (reinterpret_cast<uintptr_t>(w.W) & 15) == 0;
}

}  // namespace ttsp

using namespace ttsp;

extern "C" int ttsp_fast_steps_grid(int dim, int n_head, int n_kv, int inter, int vocab, int max_len, int n_layers,
                                    int blocksize) {
  return fs_plan(dim, n_head, n_kv, inter, vocab, max_len, n_layers, blocksize).grid;
}

extern "C" int ttsp_fast_steps_work_bytes(int dim, int n_head, int n_kv, int inter) {
  if (dim <= 0 || n_head <= 0 || n_kv <= 0 || inter <= 0) return 0;
  auto r = [](long long e) { return (2 * e + 255) / 256 * 256; };
  const long long b = r((long long)(n_head + 2 * n_kv) * HD) + 2 * r(dim) + r(inter);
  return b > (1 << 30) ? 0 : (int)b;
}

extern "C" int ttsp_fast_steps(const ttsp_fast_layer* layers, int n_layers, const ttsp_nf4_weight* head,
                               const void* fast_norm, const void* emb, const float* LUT, const void* freqs,
                               int ftype, const void* x0, void* work, unsigned* sync, void* logits, int* tokens,
                               int dim, int n_head, int n_kv, int inter, int vocab, int max_len, int step0,
                               int n_steps, float eps, int blocksize, int blocksize2, int dtype,
                               hipStream_t stream) {
  if (!layers || !head || !fast_norm || !emb || !LUT || !freqs || !x0 || !work || !sync || !logits || !tokens)
    return (int)hipErrorInvalidValue;
  if ((dtype != DT_F16 && dtype != DT_BF16) || ftype < 0 || ftype > 2 || n_steps < 1 || step0 < 0 ||
      (long long)step0 + n_steps > max_len)
    return (int)hipErrorInvalidValue;
  const FsPlan plan = fs_plan(dim, n_head, n_kv, inter, vocab, max_len, n_layers, blocksize);
  if (!plan.kind) return (int)hipErrorInvalidValue;
  const bool nested = head->A8 != nullptr;
  int bs2_shift = 0;
  if (nested) {
    if (blocksize2 <= 0 || (blocksize2 & (blocksize2 - 1))) return (int)hipErrorInvalidValue;
    while ((1 << bs2_shift) < blocksize2) ++bs2_shift;
  }
  int bs_shift = 0;
  while ((1 << bs_shift) < blocksize) ++bs_shift;
  if (!fs_weight_ok(*head, nested) || (reinterpret_cast<uintptr_t>(x0) & 15) ||
      (reinterpret_cast<uintptr_t>(emb) & 15) || ((size_t)dim * 2) % 16)
    return (int)hipErrorInvalidValue;
  FsArgs p{};
  for (int l = 0; l < n_layers; ++l) {
    const ttsp_fast_layer& s = layers[l];
    if (!fs_weight_ok(s.wqkv, nested) || !fs_weight_ok(s.wo, nested) || !fs_weight_ok(s.w1, nested) ||
        !fs_weight_ok(s.w3, nested) || !fs_weight_ok(s.w2, nested) || !s.attention_norm || !s.ffn_norm ||
        !s.k_cache || !s.v_cache || (!s.q_norm) != (!layers[0].q_norm) || (!s.k_norm) != (!layers[0].k_norm))
      return (int)hipErrorInvalidValue;
    FsLayer& d = p.L[l];
    d.wqkv = fs_lin(s.wqkv);
    d.wo = fs_lin(s.wo);
    d.w1 = fs_lin(s.w1);
    d.w3 = fs_lin(s.w3);
    d.w2 = fs_lin(s.w2);
    d.an = (const uint16_t*)s.attention_norm;
    d.fn = (const uint16_t*)s.ffn_norm;
    d.qn = (const uint16_t*)(s.q_norm ? s.q_norm : s.attention_norm);
    d.kn = (const uint16_t*)(s.k_norm ? s.k_norm : s.attention_norm);
    d.KC = (uint16_t*)s.k_cache;
    d.VC = (uint16_t*)s.v_cache;
  }
  p.head = fs_lin(*head);
  p.hn = (const uint16_t*)fast_norm;
  p.emb = (const uint16_t*)emb;
  p.LUT = LUT;
  p.freqs = freqs;
  p.x0 = (const uint16_t*)x0;
  auto r = [](long long e) { return (2 * e + 255) / 256 * 256; };
  unsigned char* wb = (unsigned char*)work;
  p.qkv = (uint16_t*)wb;
  p.h = (uint16_t*)(wb + r((long long)(n_head + 2 * n_kv) * HD));
  p.x = (uint16_t*)((unsigned char*)p.h + r(dim));
  p.g = (uint16_t*)((unsigned char*)p.x + r(dim));
  p.logits = (uint16_t*)logits;
  p.tokens = tokens;
  p.sync = sync;
  p.D = dim;
  p.nh = n_head;
  p.nkv = n_kv;
  p.inter = inter;
  p.vocab = vocab;
  p.nl = n_layers;
  p.max_len = max_len;
  p.step0 = step0;
  p.nsteps = n_steps;
  p.ftype = ftype;
  p.dt = dtype;
  p.bs_shift = bs_shift;
  p.bs2_shift = bs2_shift;
  p.nested = nested;
  p.qn = layers[0].q_norm != nullptr;
  p.kn = layers[0].k_norm != nullptr;
  p.eps = eps;
  p.scale = 1.0f / sqrtf((float)HD);
  const size_t lds = fs_dyn_lds(n_kv, max_len);
  const void* fn = plan.kind == 1 ? reinterpret_cast<const void*>(&fast_steps_kernel<FsFast1024>)
                                  : reinterpret_cast<const void*>(&fast_steps_kernel<FsFast512>);
  // every workgroup must be resident at once (they wait for each other)
  if (fs_capacity(plan.kind, fn, lds) < plan.grid) return (int)hipErrorInvalidValue;
  if (plan.kind == 1)
    hipLaunchKernelGGL(fast_steps_kernel<FsFast1024>, dim3(plan.grid), dim3(GEMV_THREADS), lds, stream, p);
  else
    hipLaunchKernelGGL(fast_steps_kernel<FsFast512>, dim3(plan.grid), dim3(GEMV_THREADS), lds, stream, p);
  TTSP_RETURN_LAUNCH();
}
