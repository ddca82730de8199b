// Grouped-query attention over a run of new positions (a prefill), flash
// style on the matrix cores. It computes what the reference computes for
// S > 1 queries with a boolean mask (app/engine/fastpath.py:133-174 for
// S <= 64 and torch's scaled_dot_product_attention with attn_mask beyond,
// fastpath.py:244-268): softmax over the keys the mask allows of
// q . k * scale, times v, query head h reading kv head h / (nh / nkv).
//
// Workgroup = (kv head kh, block of 32 queries): one wave per query head of
// the group, times NS key splits (split s takes key blocks s, s + NS, ...;
// the splits merge through LDS at the end). Keys go through LDS in blocks of
// 32: the K and V rows as they are and the 32 x 32 mask tile. Each wave computes the transposed score tile S^T = K Q^T (32
// keys x 32 queries, 8 MFMA 32x32x16 over the 128 dims; Q stays in
// registers), so one lane holds 16 keys of one query and a query's online
// softmax needs only its own lane and lane ^ 32. P^T then feeds
// O^T += V^T P^T straight from registers: the V^T fragments come from V's
// row-major tile through the transposing LDS read, in the key order the
// score layout gives P^T, so neither V nor P is transposed by hand. Scores, running max and sum are fp32 (in log2 units: the scale and
// log2 e fold into one multiply-add before the hardware exp2); the
// reference max the exponentials subtract moves only when a query's running
// max outgrows it by more than 8 (so terms stay below 2^8 and O is rarely
// rescaled); probabilities are rounded to the activation type for the matrix
// core; O is divided by the sum once at the end.
//
// Staging is a two-deep pipeline: block group t + 2 is loaded into registers
// (buffer loads, never under a branch, so the waits count them exactly)
// while group t is computed, and group t + 1 is written to the other LDS
// buffer after it. A group whose mask tile allows every key is flagged while
// it is staged, and skips the per-key masking. A first pass over the
// workgroup's 32 mask rows finds the last key any of them may see, so a
// causal mask costs only the blocks on and below the diagonal.
//
// MFMA 32x32x16 layout: lane l supplies row (l % 32) of A and column (l % 32)
// of B, each as 8 consecutive k at 8 * (l / 32) (any k permutation both
// operands agree on is fine); accumulator r of lane l is
// D[8*(r/4) + 4*(l/32) + r%4][l % 32].
#include "attn_common.h"

namespace ttsp {

typedef __bf16 pa_bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 pa_f16x8 __attribute__((ext_vector_type(8)));
typedef float pa_f32x16 __attribute__((ext_vector_type(16)));
typedef short pa_s16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) pa_s16x4 pa_lds_s16x4;

constexpr int PA_QB = 32;            // queries per workgroup
constexpr int PA_KB = 32;            // keys per block
constexpr int PA_KROW = HD + 8;      // K tile row stride (elements): 272 B
constexpr int PA_VROW = HD + 32;     // V tile row stride (elements): 320 B, see the transposed reads
constexpr int PA_MROW = PA_KB + 16;  // mask tile row stride (bytes)
constexpr int PA_MAX_GROUPS = 8;
#define PA_SPLITS(G) ((G) == 1 || (G) == 2 || (G) == 4 ? 2 : 1)

template <int DT>
__device__ __forceinline__ pa_f32x16 pa_mfma(u32x4 a, u32x4 b, pa_f32x16 c) {
  if constexpr (DT == DT_BF16)
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(pa_bf16x8, a),
                                                   __builtin_bit_cast(pa_bf16x8, b), c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(pa_f16x8, a),
                                                  __builtin_bit_cast(pa_f16x8, b), c, 0, 0, 0);
}

constexpr float PA_LOG2E = 1.4426950408889634f;

__device__ __forceinline__ float pa_exp2(float x) { return __builtin_amdgcn_exp2f(x); }  // -inf -> 0

// two fp32 values rounded to nearest-even into a packed pair of DT (the
// hardware conversion: one instruction for the pair on gfx950)
template <int DT>
__device__ __forceinline__ uint32_t pa_pack(float lo, float hi) {
  typedef float f32x2 __attribute__((ext_vector_type(2)));
  if constexpr (DT == DT_BF16) {
    typedef __bf16 b16x2 __attribute__((ext_vector_type(2)));
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){lo, hi}, b16x2));
  } else {
    typedef _Float16 h16x2 __attribute__((ext_vector_type(2)));
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){lo, hi}, h16x2));
  }
}

// ds_read_b64_tr_b16 (gfx950): within each group of 16 lanes, lane j's result
// element k is element j % 4 of the 8 bytes lane 4 k + j / 4 addresses. Four
// lanes addressing 4 consecutive dims of one key row, for 4 key rows, thus
// hand each lane of the group one dim at 4 consecutive keys: a column of V
// read straight from V's row-major tile.
__device__ __forceinline__ uint2 pa_ld_tr(const uint8_t* lds_base, uint32_t off) {
  const pa_lds_s16x4* p = (const pa_lds_s16x4*)((__attribute__((address_space(3))) const uint8_t*)lds_base + off);
  return __builtin_bit_cast(uint2, __builtin_amdgcn_ds_read_tr16_b64_v4i16(const_cast<pa_lds_s16x4*>(p)));
}

// A raw buffer over [base, base + bytes): 32-bit byte offsets, and loads past
// the end return zeros instead of touching memory.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t pa_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ u32x4 pa_ld16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
}

// Mask bytes past column L cleared, for the 16 bytes from column c; applied
// where the value is used, so the load's wait is not pulled forward.
__device__ __forceinline__ u32x4 pa_mask_tail(u32x4 v, int c, int L) {
  if (c + 16 > L) {  // rare: the piece reaches past L
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const int valid = L - c - 4 * w;  // bytes of this word before L
      v[w] &= valid >= 4 ? 0xffffffffu : valid <= 0 ? 0u : (1u << (8 * valid)) - 1u;
    }
  }
  return v;
}
// whether all 16 bytes are nonzero
__device__ __forceinline__ bool pa_all_set(u32x4 v) {
  uint32_t z = 0;
#pragma unroll
  for (int w = 0; w < 4; ++w) z |= (v[w] - 0x01010101u) & ~v[w] & 0x80808080u;
  return z == 0;
}

struct PrefillArgs {
  const uint16_t* Q;   // [S][nh][128] via q_ss / q_sh
  const uint16_t* K;   // [L][nkv][128] via k_ss / k_sh
  const uint16_t* V;   // via v_ss / v_sh
  const uint8_t* M;    // [S][L] bytes (nonzero: allowed), row stride m_ss
  uint16_t* Y;         // [S][nh][128], contiguous
  long long q_ss, q_sh;
  int k_ss, k_sh, v_ss, v_sh, m_ss;  // elements (bytes for the mask); the host bounds them
  int S, nh, nkv, L;
  float scale2;  // scale * log2(e): scores in log2 units
  float* WO;     // SPLIT: unnormalised O [z][i][head][128], then m, l [z][i][head]
  const long long* POS;  // CAUSAL: the S query rows' positions (M unused)
};

// LDS of one staged key block: K rows, V rows, mask tile (bytes)
constexpr int PA_KT = PA_KB * PA_KROW * 2;
constexpr int PA_VT = PA_KB * PA_VROW * 2;
constexpr int PA_MT = PA_QB * PA_MROW;
constexpr int PA_BLK = PA_KT + PA_VT + PA_MT;

// SPLIT: gridDim.z workgroups share each (kv head, query block), split z
// taking the z-th of gridDim.z equal runs of the key blocks that hold keys
// 0 .. last (the mask scan's result, the same in every split), and writing
// partials to WO; its first staging loads then wait for the scan.
// CAUSAL: the mask is the causal one at the rows' positions (row i allows
// keys 0 .. POS[i], and none at or past L), so it is computed instead of
// read: no mask tiles, no scan, each wave takes the workgroup's last key
// (and the first key some row may not see) from its own 32 position loads.
// The same keys are masked and the same blocks flagged whole as with the
// causal mask's bytes, so the results are those bits.
// GW: the query heads a workgroup takes, of the G that share a kv head
// (G / GW workgroups a kv head and query block, each staging the kv head's
// keys for its own heads).
template <int DT, int G, int NS, bool SPLIT, bool CAUSAL = false, int GW = G>
__global__ __launch_bounds__(64 * GW * NS) void prefill_attn_kernel(const PrefillArgs a) {
  static_assert(G % GW == 0, "a kv head's query heads split evenly over its workgroups");
  static_assert((NS & (NS - 1)) == 0, "the key splits merge in halving rounds");
  constexpr int NT = 64 * GW * NS, NW = NT / 64;
  constexpr int NKP = NS * PA_KB * (HD / 8), NVP = NKP, NMP = CAUSAL ? 0 : NS * PA_QB * 2;
  constexpr int KPT = (NKP + NT - 1) / NT, VPT = (NVP + NT - 1) / NT, MPT = NMP ? (NMP + NT - 1) / NT : 1;
  constexpr int BLK = CAUSAL ? PA_KT + PA_VT : PA_BLK;  // LDS of one staged key block
  constexpr int STAGE = 2 * NS * BLK;
  // the first merge round's slots: each giving split's o (64 floats), m, l per lane
  constexpr int MERGE = NS > 1 ? (NS / 2) * GW * 66 * 64 * 4 : 0;
  constexpr int OROW = HD + 8;  // the staged output tile's row stride (elements): 272 bytes
  constexpr int FROW = HD + 4;  // SPLIT: the staged fp32 partial rows' stride (floats): 528 bytes
  // after the merge slots: each head's 32 output rows (SPLIT: its 32 fp32 partial rows)
  constexpr int OUT = SPLIT ? GW * PA_QB * FROW * 4 : GW * PA_QB * OROW * 2;
  __shared__ __align__(16) uint8_t lds[STAGE > MERGE + OUT ? STAGE : MERGE + OUT];
  __shared__ int wmax[CAUSAL ? 1 : NW];  // the mask scan's per-wave result
  __shared__ int full[CAUSAL ? 1 : 3];   // per block group (mod 3): every key of its mask tiles allowed
  const int kh = blockIdx.x / (G / GW), q0 = blockIdx.y * PA_QB;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int gw = wave % GW, split = wave / GW;
  const int h = lane >> 5, ql = lane & 31;
  const int head = kh * G + (int)(blockIdx.x % (G / GW)) * GW + gw;
  const int i = q0 + ql;  // this lane's query
  const int nq = min(PA_QB, a.S - q0);
  const int L = a.L;
  const int z = blockIdx.z;
  int kb0 = 0;  // first key of this workgroup's run (SPLIT: set after the mask scan)
  const __amdgpu_buffer_rsrc_t kr = pa_rsrc(a.K + (size_t)kh * a.k_sh, (uint32_t)((L - 1) * a.k_ss + HD) * 2);
  const __amdgpu_buffer_rsrc_t vr = pa_rsrc(a.V + (size_t)kh * a.v_sh, (uint32_t)((L - 1) * a.v_ss + HD) * 2);
  // the mask buffer ends with the 16-byte piece holding the last row's byte
  // L - 1 (bounds are checked per dword; the piece lies in the same page as
  // that byte, and its bytes past L are cleared)
  const __amdgpu_buffer_rsrc_t mr =
      pa_rsrc(CAUSAL ? nullptr : a.M + (size_t)q0 * a.m_ss, CAUSAL ? 0u : (uint32_t)((nq - 1) * a.m_ss + ((L + 15) & ~15)));

  // the mask scan's first step, issued before everything else: thread
  // (row r, k) reads the k-th 16-byte piece from the end of row r
  // (CAUSAL: this lane's row position instead)
  constexpr int PER = NT / PA_QB;
  const int ncg = (L + 15) / 16, srow = tid % PA_QB, scg0 = ncg - 1 - tid / PA_QB;
  u32x4 scan0 = {0u, 0u, 0u, 0u};
  long long pos_i = 0;
  if constexpr (CAUSAL) pos_i = a.POS[min(i, a.S - 1)];
  else scan0 = pa_ld16(mr, (uint32_t)(min(srow, nq - 1) * a.m_ss + 16 * max(scg0, 0)));
  __builtin_amdgcn_sched_barrier(0);  // keep it first, so waiting for it waits for nothing else

  // Q^T fragments (B operand): column = query ql, dims 16 kc + 8 h .. + 7
  u32x4 qf[HD / 16];
  {
    const uint16_t* qr = a.Q + (size_t)min(i, a.S - 1) * a.q_ss + (size_t)head * a.q_sh;
#pragma unroll
    for (int kc = 0; kc < HD / 16; ++kc) qf[kc] = *reinterpret_cast<const u32x4*>(qr + 16 * kc + 8 * h);
  }
  __builtin_amdgcn_sched_barrier(0);

  // staging of block group t (blocks NS t .. NS t + NS - 1): K and V rows
  // (16-byte pieces), mask pieces. Group t is loaded into register set t % 2 two groups ahead
  // and written to LDS buffer t % 2 at the end of the iteration before it.
  // Rows are clamped into [0, L): keys past L then hold finite values, which
  // their zero probabilities cancel.
  struct Regs {
    u32x4 k[KPT], v[VPT], m[MPT];
  };
  Regs rs[2];
  auto load = [&](Regs& r, int t) {
#pragma unroll
    for (int n = 0; n < KPT; ++n) {
      const int p = min(tid + n * NT, NKP - 1), blk = p / (PA_KB * (HD / 8)), q = p % (PA_KB * (HD / 8));
      const int j = min(kb0 + NS * t * PA_KB + blk * PA_KB + q / (HD / 8), L - 1), e = (q % (HD / 8)) * 8;
      r.k[n] = pa_ld16(kr, (uint32_t)(j * a.k_ss + e) * 2);
    }
#pragma unroll
    for (int n = 0; n < VPT; ++n) {
      const int p = min(tid + n * NT, NVP - 1), blk = p / (PA_KB * (HD / 8)), q = p % (PA_KB * (HD / 8));
      const int j = min(kb0 + NS * t * PA_KB + blk * PA_KB + q / (HD / 8), L - 1), e = (q % (HD / 8)) * 8;
      r.v[n] = pa_ld16(vr, (uint32_t)(j * a.v_ss + e) * 2);
    }
    if constexpr (!CAUSAL) {
#pragma unroll
      for (int n = 0; n < MPT; ++n) {
        const int p = min(tid + n * NT, NMP - 1), blk = p / (PA_QB * 2), q = p % (PA_QB * 2);
        const int c = min(kb0 + NS * t * PA_KB + blk * PA_KB + 16 * (q & 1), 16 * (ncg - 1));
        r.m[n] = pa_ld16(mr, (uint32_t)(min(q >> 1, nq - 1) * a.m_ss + c));
      }
    }
  };
  auto store = [&](const Regs& r, int t) {
    const int buf = t & 1;
#pragma unroll
    for (int n = 0; n < KPT; ++n) {
      const int p = tid + n * NT, blk = p / (PA_KB * (HD / 8)), q = p % (PA_KB * (HD / 8));
      if (NKP % NT == 0 || p < NKP) {
        uint8_t* base = lds + (size_t)(buf * NS + blk) * BLK;
        *reinterpret_cast<u32x4*>(base + 2 * ((q / (HD / 8)) * PA_KROW + (q % (HD / 8)) * 8)) = r.k[n];
      }
    }
#pragma unroll
    for (int n = 0; n < VPT; ++n) {
      const int p = tid + n * NT, blk = p / (PA_KB * (HD / 8)), q = p % (PA_KB * (HD / 8));
      if (NVP % NT == 0 || p < NVP) {
        uint8_t* base = lds + (size_t)(buf * NS + blk) * BLK + PA_KT;
        *reinterpret_cast<u32x4*>(base + 2 * ((q / (HD / 8)) * PA_VROW + (q % (HD / 8)) * 8)) = r.v[n];
      }
    }
    if constexpr (!CAUSAL) {
#pragma unroll
      for (int n = 0; n < MPT; ++n) {
        const int p = tid + n * NT, blk = p / (PA_QB * 2), q = p % (PA_QB * 2);
        if (NMP % NT == 0 || p < NMP) {
          const u32x4 m = pa_mask_tail(r.m[n], kb0 + NS * t * PA_KB + blk * PA_KB + 16 * (q & 1), L);
          *reinterpret_cast<u32x4*>(lds + (size_t)(buf * NS + blk) * BLK + PA_KT + PA_VT + (q >> 1) * PA_MROW +
                                    16 * (q & 1)) = m;
          if ((q >> 1) < nq && !pa_all_set(m)) full[t % 3] = 0;  // rows past nq are never used
        }
      }
    }
  };
  if constexpr (!SPLIT) {
    load(rs[0], 0);
    __builtin_amdgcn_sched_barrier(0);
    load(rs[1], 1);
    __builtin_amdgcn_sched_barrier(0);
  }

  // the last key any of the workgroup's queries may see: the first step's
  // piece, then (only where it holds no allowed key) the rest of the row
  // backwards; the maximum over the workgroup through one slot per wave
  int hit = -1;
  // CAUSAL: the last key this lane's row sees (-1: none), and the lowest such
  // key over the workgroup's rows, below which every block is whole
  const int klast = CAUSAL ? (int)min(pos_i, (long long)L - 1) : 0;
  int kwhole = 0;
  if constexpr (CAUSAL) {
    hit = klast;
    kwhole = ql < nq ? klast : L;
#pragma unroll
    for (int o = 16; o >= 1; o >>= 1) kwhole = min(kwhole, __shfl_xor(kwhole, o, 64));
  } else if (srow < nq && scg0 >= 0) {
    u32x4 v = pa_mask_tail(scan0, 16 * scg0, L);
    for (int cg = scg0;;) {
#pragma unroll
      for (int w = 3; w >= 0; --w)
        if (hit < 0 && v[w]) hit = 16 * cg + 4 * w + (31 - __builtin_clz(v[w])) / 8;
      cg -= PER;
      if (hit >= 0 || cg < 0) break;
      v = pa_mask_tail(pa_ld16(mr, (uint32_t)(srow * a.m_ss + 16 * cg)), 16 * cg, L);
    }
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) hit = max(hit, __shfl_xor(hit, o, 64));
  int last = hit;  // CAUSAL: every wave holds the workgroup's value
  if constexpr (!CAUSAL) {
    if (lane == 0) wmax[wave] = hit;
    if (tid == 0) full[0] = full[1] = 1;
    __syncthreads();
    last = -1;
#pragma unroll
    for (int w = 0; w < NW; ++w) last = max(last, wmax[w]);
  }
  // this workgroup's key blocks: all blocks holding keys 0 .. last, or split
  // z's run of them
  const int live = (last + PA_KB) / PA_KB;
  int nkb = live;
  if constexpr (SPLIT) {
    const int bps = (live + (int)gridDim.z - 1) / (int)gridDim.z;
    kb0 = z * bps * PA_KB;
    nkb = max(0, min(live, (z + 1) * bps) - z * bps);
    load(rs[0], 0);
    __builtin_amdgcn_sched_barrier(0);
    load(rs[1], 1);
    __builtin_amdgcn_sched_barrier(0);
  }
  const int nit = (nkb + NS - 1) / NS;
  // wait for Q here: a wait inside the loop would also wait for the
  // prefetch loads issued after it
#pragma unroll
  for (int kc = 0; kc < HD / 16; ++kc) asm volatile("" ::"v"(qf[kc]));

  pa_f32x16 o[HD / 32];
#pragma unroll
  for (int d = 0; d < HD / 32; ++d)
#pragma unroll
    for (int r = 0; r < 16; ++r) o[d][r] = 0.0f;
  float mrun = -__builtin_inff(), lrun = 0.0f;

  if (nit > 0) store(rs[0], 0);
  __syncthreads();
  // one step of the pipeline: load group t + 2 into set rl, compute group t,
  // write group t + 1 (set rw) to the other LDS buffer
  auto step = [&](int t, Regs& rl, const Regs& rw) {
    const int buf = t & 1, b = NS * t + split;
    load(rl, t + 2);  // also past the last group: clamped rows, never stored
    if (!CAUSAL && tid == 0) full[(t + 2) % 3] = 1;  // group t - 1 used this slot before the last barrier
    if (b < nkb) {
      const uint8_t* base = lds + (size_t)(buf * NS + split) * BLK;
      const uint16_t* ks = reinterpret_cast<const uint16_t*>(base);
      const uint8_t* ms = base + PA_KT + PA_VT;
      // (CAUSAL: the group's blocks whole when its last key is below every row's
      // last key, as the causal mask's tiles are then all set)
      const int gend = kb0 + (NS * t + NS) * PA_KB - 1;
      const bool all = CAUSAL ? gend <= kwhole : __builtin_amdgcn_readfirstlane(full[t % 3]) != 0;
      // S^T = K Q^T for keys 32 b .. 32 b + 31
      pa_f32x16 s;
#pragma unroll
      for (int r = 0; r < 16; ++r) s[r] = 0.0f;
      const uint16_t* krow = ks + ql * PA_KROW + 8 * h;
#pragma unroll
      for (int kc = 0; kc < HD / 16; ++kc)
        s = pa_mfma<DT>(*reinterpret_cast<const u32x4*>(krow + 16 * kc), qf[kc], s);
      // V^T fragments (A operand of the second product: dim 32 d + ql at keys
      // 16 c + {4h .. 4h + 3, 8 + 4h .. 8 + 4h + 3}), read transposed while
      // the scores are computed: lane 4 k + q of each 16-lane group (dims
      // 16 db .. 16 db + 15) addresses key 16 c + 4 h + k (+ 8), dims 4 q ..
      u32x4 vf[HD / 32][2];
      {
        const int g = lane >> 4, li = lane & 15;
        const uint32_t vo = (uint32_t)(PA_KT + ((4 * (g >> 1) + (li >> 2)) * PA_VROW + 16 * (g & 1) + 4 * (li & 3)) * 2);
#pragma unroll
        for (int d = 0; d < HD / 32; ++d)
#pragma unroll
          for (int c = 0; c < 2; ++c) {
            const uint2 lo = pa_ld_tr(base, vo + (16 * c * PA_VROW + 32 * d) * 2);
            const uint2 hi = pa_ld_tr(base, vo + ((16 * c + 8) * PA_VROW + 32 * d) * 2);
            vf[d][c] = (u32x4){lo.x, lo.y, hi.x, hi.y};
          }
      }
      // keys 8 g + 4 h + 0..3 of the block (g = r / 4) masked to -inf unless
      // the whole group is allowed; the online softmax of query ql over this
      // lane and lane ^ 32, in log2 units
      if (!all) {
        if constexpr (CAUSAL) {
          const int k0 = kb0 + b * PA_KB + 4 * h;  // key of s[0]
#pragma unroll
          for (int g = 0; g < 4; ++g)
#pragma unroll
            for (int c = 0; c < 4; ++c)
              if (k0 + 8 * g + c > klast) s[4 * g + c] = -__builtin_inff();
        } else {
          const uint8_t* mrow = ms + ql * PA_MROW + 4 * h;
#pragma unroll
          for (int g = 0; g < 4; ++g) {
            const uint32_t mw = *reinterpret_cast<const uint32_t*>(mrow + 8 * g);
#pragma unroll
            for (int c = 0; c < 4; ++c)
              if (((mw >> (8 * c)) & 0xffu) == 0) s[4 * g + c] = -__builtin_inff();
          }
        }
      }
      float bm = -__builtin_inff();
#pragma unroll
      for (int r = 0; r < 16; ++r) bm = fmaxf(bm, s[r]);
      bm = fmaxf(bm, __shfl_xor(bm, 32, 64)) * a.scale2;
      // the reference max moves only when the running max outgrows it by more
      // than 2^8 (terms then stay below 256), so O's rescale is rare
      const float mnew = fmaxf(mrun, bm);
      const float mkeep = mnew > mrun + 8.0f ? mnew : mrun;
      const float mref = mkeep == -__builtin_inff() ? 0.0f : mkeep;  // nothing seen yet: all terms 0
      const float alpha = pa_exp2(mrun - mref);
      float ps = 0.0f;
      u32x4 pf[2];  // P^T fragments (B operand): keys 16 c + {4h .. 4h + 3, 8 + 4h .. 8 + 4h + 3}
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        float pv[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          pv[u] = pa_exp2(__builtin_fmaf(s[8 * c + u], a.scale2, -mref));
          ps += pv[u];
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) pf[c][u] = pa_pack<DT>(pv[2 * u], pv[2 * u + 1]);
      }
      ps += __shfl_xor(ps, 32, 64);
      lrun = lrun * alpha + ps;
      mrun = mkeep;
      // O^T = alpha O^T + V^T P^T (the rescale skipped while no lane's reference moved)
      if (__any(alpha != 1.0f)) {
#pragma unroll
        for (int d = 0; d < HD / 32; ++d)
#pragma unroll
          for (int r = 0; r < 16; ++r) o[d][r] *= alpha;
      }
#pragma unroll
      for (int d = 0; d < HD / 32; ++d)
#pragma unroll
        for (int c = 0; c < 2; ++c) o[d] = pa_mfma<DT>(vf[d][c], pf[c], o[d]);
    }
    if (t + 1 < nit) store(rw, t + 1);  // the other buffer: last read before the previous barrier
    __syncthreads();
  };
  for (int t = 0; t < nit; t += 2) {
    step(t, rs[0], rs[1]);
    if (t + 1 < nit) step(t + 1, rs[1], rs[0]);
  }
  if constexpr (NS > 1) {
    // splits st .. 2 st - 1 hand their o, m, l to splits 0 .. st - 1 through
    // LDS (same lane layout in both), st halving down to 1, then split 0
    // writes; the staging buffers are free after the loop's last barrier.
    // Every wave takes every barrier; only split 0 goes on.
#pragma unroll
    for (int st = NS / 2; st >= 1; st /= 2) {
      const bool give = split >= st && split < 2 * st, take = split < st;
      float* mg = reinterpret_cast<float*>(lds) + (size_t)((give ? split - st : split) * GW + gw) * 66 * 64 + lane;
      if (give) {
#pragma unroll
        for (int d = 0; d < HD / 32; ++d)
#pragma unroll
          for (int r = 0; r < 16; ++r) mg[(16 * d + r) * 64] = o[d][r];
        mg[64 * 64] = mrun;
        mg[65 * 64] = lrun;
      }
      __syncthreads();
      if (take) {
        const float m2 = mg[64 * 64], l2 = mg[65 * 64];
        const float mm = fmaxf(mrun, m2);
        const float mref = mm == -__builtin_inff() ? 0.0f : mm;
        const float f1 = pa_exp2(mrun - mref), f2 = pa_exp2(m2 - mref);
        lrun = lrun * f1 + l2 * f2;
        mrun = mm;  // o and lrun are now relative to the merged max (the key-split merge reads it)
#pragma unroll
        for (int d = 0; d < HD / 32; ++d)
#pragma unroll
          for (int r = 0; r < 16; ++r) o[d][r] = o[d][r] * f1 + mg[(16 * d + r) * 64] * f2;
      }
      if (st > 1) __syncthreads();  // the next round writes the slots again
    }
    if (split != 0) return;
  }
  if constexpr (SPLIT) {  // O unnormalised, max and sum of this split, for the merge kernel
    // O staged as this head's 32 rows in LDS (read back by this wave only)
    // and stored as whole 512-byte rows, 16 bytes a lane
    float* of = reinterpret_cast<float*>(lds + MERGE) + (size_t)gw * PA_QB * FROW;
#pragma unroll
    for (int d = 0; d < HD / 32; ++d)
#pragma unroll
      for (int g = 0; g < 4; ++g)
        *reinterpret_cast<float4*>(of + ql * FROW + 32 * d + 8 * g + 4 * h) =
            make_float4(o[d][4 * g], o[d][4 * g + 1], o[d][4 * g + 2], o[d][4 * g + 3]);
#pragma unroll
    for (int k = 0; k < PA_QB * HD / 4 / 64; ++k) {
      const int e = lane + 64 * k, r = e >> 5, cc = (e & 31) * 4;
      const float4 v = *reinterpret_cast<const float4*>(of + r * FROW + cc);
      if (q0 + r < a.S)
        *reinterpret_cast<float4*>(a.WO + (((size_t)z * a.S + q0 + r) * a.nh + head) * HD + cc) = v;
    }
    if (i < a.S && h == 0) {
      float* ml = a.WO + (size_t)gridDim.z * a.S * a.nh * HD + (((size_t)z * a.S + i) * a.nh + head) * 2;
      *reinterpret_cast<float2*>(ml) = make_float2(mrun, lrun);
    }
    return;
  }
  // Y[i][head][dim] = O^T[dim][i] / l (a row with no allowed key: 0 / 0, as the reference's softmax),
  // staged as this head's 32 rows in LDS (the wave reads back only what it
  // wrote: no barrier) and stored as whole 256-byte rows, 16 bytes a lane
  {
    const float inv = 1.0f / lrun;
    uint16_t* ot = reinterpret_cast<uint16_t*>(lds + MERGE) + (size_t)gw * PA_QB * OROW;
#pragma unroll
    for (int d = 0; d < HD / 32; ++d)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        uint2 w;
        w.x = pa_pack<DT>(o[d][4 * g] * inv, o[d][4 * g + 1] * inv);
        w.y = pa_pack<DT>(o[d][4 * g + 2] * inv, o[d][4 * g + 3] * inv);
        *reinterpret_cast<uint2*>(ot + ql * OROW + 32 * d + 8 * g + 4 * h) = w;
      }
#pragma unroll
    for (int k = 0; k < PA_QB * HD / 8 / 64; ++k) {
      const int e = lane + 64 * k, r = e >> 4, cc = (e & 15) * 8;
      const uint4 v = *reinterpret_cast<const uint4*>(ot + r * OROW + cc);
      if (q0 + r < a.S) *reinterpret_cast<uint4*>(a.Y + ((size_t)(q0 + r) * a.nh + head) * HD + cc) = v;
    }
  }
}

// Y[i][head][8 dims] from the splits' partials: weights 2^(m_z - max m),
// sums in split order, O / l rounded once (a row with no allowed key in any
// split: 0 / 0). Every split's loads are issued before the first is used
// (SPM >= splits slots, indices clamped, weight 0 past the last split), so
// the kernel costs one memory round trip whatever the split count.
template <int DT, int SPM>
__global__ __launch_bounds__(256) void prefill_merge_kernel(const float* __restrict__ WO, int splits, int S, int nh,
                                                            uint16_t* __restrict__ Y) {
  const long long t = (long long)blockIdx.x * 256 + threadIdx.x;
  if (t >= (long long)S * nh * (HD / 8)) return;
  const int d0 = (int)(t % (HD / 8)) * 8;
  const long long ih = t / (HD / 8);  // i * nh + head
  const size_t plane = (size_t)S * nh;  // (query, head) pairs per split
  const float* ml = WO + (size_t)splits * plane * HD;
  float2 mlz[SPM];
  float4 u[SPM], v[SPM];
#pragma unroll
  for (int z = 0; z < SPM; ++z) {
    const size_t zi = (size_t)min(z, splits - 1) * plane + ih;
    mlz[z] = *reinterpret_cast<const float2*>(ml + zi * 2);
    u[z] = *reinterpret_cast<const float4*>(WO + zi * HD + d0);
    v[z] = *reinterpret_cast<const float4*>(WO + zi * HD + d0 + 4);
  }
  __builtin_amdgcn_sched_barrier(0);  // all loads in flight before the first use
  float mx = -__builtin_inff();
#pragma unroll
  for (int z = 0; z < SPM; ++z) mx = fmaxf(mx, mlz[z].x);  // clamped slots repeat the last split
  const float mref = mx == -__builtin_inff() ? 0.0f : mx;
  float num[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f}, den = 0.0f;
#pragma unroll
  for (int z = 0; z < SPM; ++z) {
    const float w = z < splits ? pa_exp2(mlz[z].x - mref) : 0.0f;
    den = __builtin_fmaf(w, mlz[z].y, den);
    num[0] = __builtin_fmaf(w, u[z].x, num[0]), num[1] = __builtin_fmaf(w, u[z].y, num[1]);
    num[2] = __builtin_fmaf(w, u[z].z, num[2]), num[3] = __builtin_fmaf(w, u[z].w, num[3]);
    num[4] = __builtin_fmaf(w, v[z].x, num[4]), num[5] = __builtin_fmaf(w, v[z].y, num[5]);
    num[6] = __builtin_fmaf(w, v[z].z, num[6]), num[7] = __builtin_fmaf(w, v[z].w, num[7]);
  }
  const float inv = 1.0f / den;
  uint4 out;
  out.x = pa_pack<DT>(num[0] * inv, num[1] * inv);
  out.y = pa_pack<DT>(num[2] * inv, num[3] * inv);
  out.z = pa_pack<DT>(num[4] * inv, num[5] * inv);
  out.w = pa_pack<DT>(num[6] * inv, num[7] * inv);
  *reinterpret_cast<uint4*>(Y + (size_t)ih * HD + d0) = out;
}

// Key splits for a launch: none for fewer than 16 key blocks (the merge
// launch costs about what 4 pipeline steps save) or once the (kv head,
// 32-query) workgroups number 256; two for 128-255 workgroups over a cached
// prefix of at least 1024 keys (the keys before the run, which every query
// sees: without them a causal run's diagonal work is too uneven to gain);
// otherwise doubled up to 16 while the workgroups stay under 256 and each
// split keeps at least 3 key blocks.
static int prefill_splits(int S, int nkv, int L) {
  const long long wg = (long long)nkv * ((S + PA_QB - 1) / PA_QB);
  const int blocks = (L + PA_KB - 1) / PA_KB;
  if (blocks < 16 || wg >= 256) return 1;
  if (wg >= 128) return L - S >= 1024 ? 2 : 1;
  int sp = 1;
  while (wg * sp < 256 && sp < 16 && blocks / (2 * sp) >= 3) sp *= 2;
  return sp;
}

}  // namespace ttsp

using namespace ttsp;

extern "C" int ttsp_prefill_max_groups() { return PA_MAX_GROUPS; }

// the kernel for `groups` query heads per kv head: two key splits for 1, 2
// and 4 heads per kv head (at most 8 waves, two a SIMD at ~240 registers),
// one otherwise. The causal form with 4 heads per kv head and no key split
// over workgroups, once the (kv head, query block) pairs fill half the CUs,
// takes two workgroups of 2 heads and 4 key splits each instead (its LDS
// holds four key blocks a stage without the mask tiles): all CUs busy and
// half the serial key steps, for twice the key staging (512 causal rows,
// 32 / 8 heads: 14.5 against 15.9 us; with fewer rows, or with key splits,
// the staging costs more than it saves).
template <int DT, bool CAUSAL>
static int prefill_dispatch(int groups, dim3 grid, int splits, const PrefillArgs& a, hipStream_t stream) {
  if constexpr (CAUSAL) {
    if (groups == 4 && splits == 1 && (long long)grid.x * grid.y >= 128) {
      grid.x *= 2;
      hipLaunchKernelGGL((prefill_attn_kernel<DT, 4, 4, false, true, 2>), grid, dim3(64 * 2 * 4), 0, stream, a);
      return 0;
    }
  }
#define TTSP_PA_G(G)                                                                                         \
  case G:                                                                                                    \
    if (splits > 1)                                                                                          \
      hipLaunchKernelGGL((prefill_attn_kernel<DT, G, PA_SPLITS(G), true, CAUSAL>), grid,                     \
                         dim3(64 * G * PA_SPLITS(G)), 0, stream, a);                                         \
    else                                                                                                     \
      hipLaunchKernelGGL((prefill_attn_kernel<DT, G, PA_SPLITS(G), false, CAUSAL>), grid,                    \
                         dim3(64 * G * PA_SPLITS(G)), 0, stream, a);                                         \
    return 0;
  switch (groups) {
    TTSP_PA_G(1)
    TTSP_PA_G(2)
    TTSP_PA_G(3)
    TTSP_PA_G(4)
    TTSP_PA_G(5)
    TTSP_PA_G(6)
    TTSP_PA_G(7)
    TTSP_PA_G(8)
    default:
      return (int)hipErrorInvalidValue;
  }
#undef TTSP_PA_G
}

// mask: bool rows (mask_row_stride bytes apart), or null with pos, the S
// rows' positions, for the causal mask at those positions
static int prefill_launch(const void* Q, long long q_seq_stride, long long q_head_stride, const void* K,
                          long long k_seq_stride, long long k_head_stride, const void* V, long long v_seq_stride,
                          long long v_head_stride, const void* mask, long long mask_row_stride, const long long* pos,
                          void* Y, int S, int nh, int nkv, int L, float scale, int dtype, float* work, int splits,
                          hipStream_t stream) {
  const bool causal = pos != nullptr;
  if (causal) mask = nullptr, mask_row_stride = 0;
  if (!Q || !K || !V || (!causal && !mask) || !Y || S <= 0 || nh <= 0 || nkv <= 0 || nh % nkv || L <= 0 ||
      nh / nkv > PA_MAX_GROUPS || S > (1 << 20) || (!causal && mask_row_stride < L) || splits < 1 || splits > 16)
    return (int)hipErrorInvalidValue;
  // 16-byte pieces: every row start and the bases aligned
  const long long st[6] = {q_seq_stride, q_head_stride, k_seq_stride, k_head_stride, v_seq_stride, v_head_stride};
  for (long long s : st)
    if (s < 0 || s % 8) return (int)hipErrorInvalidValue;
  if (mask_row_stride % 16 || (uintptr_t)Q % 16 || (uintptr_t)K % 16 || (uintptr_t)V % 16 ||
      (uintptr_t)mask % 16 || (uintptr_t)Y % 16 || (splits > 1 && (!work || (uintptr_t)work % 16)))
    return (int)hipErrorInvalidValue;
  // K, V (one kv head) and the mask rows of one workgroup are addressed with
  // 32-bit byte offsets
  const long long lim = (1LL << 31) - 1;
  if (((L - 1) * k_seq_stride + 128) * 2 > lim || ((L - 1) * v_seq_stride + 128) * 2 > lim ||
      k_head_stride > lim || v_head_stride > lim || 31 * mask_row_stride + L > lim)
    return (int)hipErrorInvalidValue;
  PrefillArgs a{(const uint16_t*)Q, (const uint16_t*)K, (const uint16_t*)V, (const uint8_t*)mask, (uint16_t*)Y,
                q_seq_stride, q_head_stride, (int)k_seq_stride, (int)k_head_stride, (int)v_seq_stride,
                (int)v_head_stride, (int)mask_row_stride, S, nh, nkv, L, scale * PA_LOG2E,
                splits > 1 ? work : nullptr, pos};
  const int groups = nh / nkv;
  const dim3 grid(nkv, (S + PA_QB - 1) / PA_QB, splits);
  int rc;
  if (dtype == DT_F16)
    rc = causal ? prefill_dispatch<DT_F16, true>(groups, grid, splits, a, stream)
                : prefill_dispatch<DT_F16, false>(groups, grid, splits, a, stream);
  else if (dtype == DT_BF16)
    rc = causal ? prefill_dispatch<DT_BF16, true>(groups, grid, splits, a, stream)
                : prefill_dispatch<DT_BF16, false>(groups, grid, splits, a, stream);
  else
    return (int)hipErrorInvalidValue;
  if (rc) return rc;
  if (splits > 1) {
    const long long n = (long long)S * nh * (HD / 8);
    const dim3 mg((unsigned)((n + 255) / 256));
#define TTSP_PM(DTV, SPM) \
  hipLaunchKernelGGL((prefill_merge_kernel<DTV, SPM>), mg, dim3(256), 0, stream, work, splits, S, nh, (uint16_t*)Y)
#define TTSP_PM_SP(DTV)          \
  if (splits <= 2)               \
    TTSP_PM(DTV, 2);             \
  else if (splits <= 4)          \
    TTSP_PM(DTV, 4);             \
  else if (splits <= 8)          \
    TTSP_PM(DTV, 8);             \
  else                           \
    TTSP_PM(DTV, 16);
    if (dtype == DT_F16) {
      TTSP_PM_SP(DT_F16)
    } else {
      TTSP_PM_SP(DT_BF16)
    }
#undef TTSP_PM_SP
#undef TTSP_PM
  }
  TTSP_RETURN_LAUNCH();
}

extern "C" int ttsp_prefill_attention(const void* Q, long long q_seq_stride, long long q_head_stride,
                                      const void* K, long long k_seq_stride, long long k_head_stride,
                                      const void* V, long long v_seq_stride, long long v_head_stride,
                                      const void* mask, long long mask_row_stride, void* Y, int S, int nh,
                                      int nkv, int L, float scale, int dtype, hipStream_t stream) {
  return prefill_launch(Q, q_seq_stride, q_head_stride, K, k_seq_stride, k_head_stride, V, v_seq_stride,
                        v_head_stride, mask, mask_row_stride, nullptr, Y, S, nh, nkv, L, scale, dtype, nullptr, 1,
                        stream);
}

extern "C" int ttsp_prefill_attention_splits(int S, int nkv, int L) {
  if (S <= 0 || nkv <= 0 || L <= 0) return 1;
  return prefill_splits(S, nkv, L);
}

extern "C" int ttsp_prefill_attention_split(const void* Q, long long q_seq_stride, long long q_head_stride,
                                            const void* K, long long k_seq_stride, long long k_head_stride,
                                            const void* V, long long v_seq_stride, long long v_head_stride,
                                            const void* mask, long long mask_row_stride, void* Y, int S, int nh,
                                            int nkv, int L, float scale, int dtype, float* work, int splits,
                                            hipStream_t stream) {
  return prefill_launch(Q, q_seq_stride, q_head_stride, K, k_seq_stride, k_head_stride, V, v_seq_stride,
                        v_head_stride, mask, mask_row_stride, nullptr, Y, S, nh, nkv, L, scale, dtype, work, splits,
                        stream);
}

extern "C" int ttsp_prefill_attention_causal(const void* Q, long long q_seq_stride, long long q_head_stride,
                                             const void* K, long long k_seq_stride, long long k_head_stride,
                                             const void* V, long long v_seq_stride, long long v_head_stride,
                                             const long long* pos, void* Y, int S, int nh, int nkv, int L,
                                             float scale, int dtype, float* work, int splits, hipStream_t stream) {
  if (!pos) return (int)hipErrorInvalidValue;
  return prefill_launch(Q, q_seq_stride, q_head_stride, K, k_seq_stride, k_head_stride, V, v_seq_stride,
                        v_head_stride, nullptr, 0, pos, Y, S, nh, nkv, L, scale, dtype, work, splits, stream);
}
