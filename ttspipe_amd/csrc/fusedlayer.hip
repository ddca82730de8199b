// The three non-matmul kernels of a decode step through a transformer block
// (app/engine/fusedlayer.py:56-159): per-head norm + rotary + KV-cache write,
// then grouped-query attention as split-K over fixed chunks of the cache.
//
// Layouts (batch 1): QKV is [nh + 2*nkv][128] (q heads, k heads, v heads),
// the caches are [nkv][max_len][128], Q and Y are [nh][128]. Query head i
// reads KV head i / (nh / nkv).
//
// attn_partial: one workgroup per (kv head, chunk of 64 positions), one wave
// per query head of the group. The chunk's K and V rows are staged in LDS with
// coalesced loads; lane j scores position j (fp32 fma over d = 0..127 against
// q * 1/sqrt(128)), the wave takes the chunk max and sum of exp(s - max), and
// lane l accumulates dims 2l, 2l+1 over the chunk's positions in order.
// attn_combine merges chunks with the log-sum-exp rule, chunks in order.
//
// attn_qkv fuses the three: each workgroup of the split-K attention reads its
// query heads straight from QKV and applies the head norm and rotary itself
// (the arithmetic of qk_rope_kv, one wave per head, lane l holding elements l
// and l + 64), the workgroup whose chunk holds the new position also computes
// that K/V row, writes it to the cache and uses it from registers; with one
// chunk (a short cache) the workgroup finishes the merge in place, so the
// whole attention of a decode step is one launch (two for long caches).
// All of these are deterministic: no atomics, fixed orders.
#include "attn_common.h"

#include <mutex>

namespace ttsp {

// Head norms, rotary and the KV-cache write of one or more positions: one
// wave per head (QKV_WAVES heads a workgroup, any mix of q, k and v heads),
// lane l holding elements l and l + 64 - the decode attention's own head
// arithmetic (head_norm_rope), so both paths give the same bits. A q head goes
// to Q, a k head to KC[kv][pos], a v head is copied to VC[kv][pos]. Row
// blockIdx.y reads its own QKV row, rotary row and position; the rotary table
// is read a dword at a time (4-byte aligned). P: the row is a K-split GEMM's
// fp32 partial sums (split z of row r at YP[(z * rows + r) * qkv_rs]), added
// in split order and rounded as the split GEMM's own reduce does.
constexpr int QKV_WAVES = 4;

template <int DT, bool P = false>
__global__ __launch_bounds__(64 * QKV_WAVES) void qk_rope_kv_kernel(
    const uint16_t* __restrict__ QKV, const uint16_t* __restrict__ QW,
    const uint16_t* __restrict__ KW, float eps, const void* __restrict__ F, int ftype,
    const long long* __restrict__ POS, uint16_t* __restrict__ Q, uint16_t* __restrict__ KC,
    uint16_t* __restrict__ VC, int nh, int nkv, int max_len, int qkv_rs, const float* __restrict__ YP = nullptr,
    int splits = 0) {
  const int lane = threadIdx.x & 63;
  const int head = blockIdx.x * QKV_WAVES + (threadIdx.x >> 6);
  const int row = blockIdx.y;
  if (head >= nh + 2 * nkv) return;
  const long long pos = POS[row];
  if (pos < 0 || pos >= max_len) return;  // no cache slot to write: leave everything untouched
  float lo, hi;
  if constexpr (P) {
    const size_t o = (size_t)row * qkv_rs + (size_t)head * HD, zs = (size_t)gridDim.y * qkv_rs;
    lo = YP[o + lane];
    hi = YP[o + lane + 64];
    for (int z = 1; z < splits; ++z) {
      lo += YP[z * zs + o + lane];
      hi += YP[z * zs + o + lane + 64];
    }
    lo = Elem<DT>::load(Elem<DT>::store(lo));
    hi = Elem<DT>::load(Elem<DT>::store(hi));
  }
  const uint16_t* src = P ? nullptr : QKV + (size_t)row * qkv_rs + (size_t)head * HD;
  if (head >= nh + nkv) {
    uint16_t* v = VC + ((long long)(head - nh - nkv) * max_len + pos) * HD;
    v[lane] = P ? (uint16_t)Elem<DT>::store(lo) : src[lane];
    v[lane + 64] = P ? (uint16_t)Elem<DT>::store(hi) : src[lane + 64];
    return;
  }
  const bool is_q = head < nh;
  const uint16_t* w = is_q ? QW : KW;
  const RopeF f = load_rope((const uint8_t*)F + (size_t)row * HD * (ftype == DT_F32 ? 4 : 2), ftype, lane);
  if constexpr (!P) {
    lo = Elem<DT>::load(src[lane]);
    hi = Elem<DT>::load(src[lane + 64]);
  }
  const uint16_t nwl = w ? w[lane] : 0, nwh = w ? w[lane + 64] : 0;
  head_norm_rope<DT>(lo, hi, w != nullptr, nwl, nwh, eps, f, lane);
  uint16_t* dst = is_q ? Q + (size_t)row * nh * HD + (size_t)head * HD
                       : KC + ((long long)(head - nh) * max_len + pos) * HD;
  dst[lane] = Elem<DT>::store(lo);
  dst[lane + 64] = Elem<DT>::store(hi);
}

template <int DT>
__global__ __launch_bounds__(1024) void attn_partial_kernel(
    const uint16_t* __restrict__ Q, const uint16_t* __restrict__ KC,
    const uint16_t* __restrict__ VC, const long long* __restrict__ POS, float* __restrict__ PM,
    float* __restrict__ PL, float* __restrict__ PACC, int groups, int max_len, int nchunk,
    float scale) {
  extern __shared__ __align__(16) float smem[];
  float* q_s = smem;                                         // [groups][HD]
  float* p_s = q_s + groups * HD;                            // [groups][ACHUNK]
  uint16_t* k_s = reinterpret_cast<uint16_t*>(p_s + groups * ACHUNK);  // [ACHUNK][KPAD]
  uint16_t* v_s = k_s + ACHUNK * KPAD;                       // [ACHUNK][HD]

  const int kh = blockIdx.x, c = blockIdx.y;
  const int row = blockIdx.z;  // query row of the rows form: Q, POS and the partials by row (0: one position)
  const int tid = threadIdx.x, nthr = blockDim.x;
  const int g = tid >> 6, lane = tid & 63;
  const int qh = kh * groups + g, nh = (int)gridDim.x * groups;
  Q += (size_t)row * nh * HD;
  // Positions [0, L) are live; the cache holds max_len of them.
  const long long L = min(POS[row] + 1, (long long)max_len);
  const long long j0 = (long long)c * ACHUNK;
  const size_t slot = ((size_t)row * nh + qh) * nchunk + c;
  if (j0 >= L) {
    if (lane == 0) {
      PM[slot] = -1e30f;
      PL[slot] = 0.0f;
    }
    return;
  }
  const int nvalid = (int)min((long long)ACHUNK, L - j0);

  for (int t = tid; t < groups * HD; t += nthr)
    q_s[t] = __fmul_rn(Elem<DT>::load(Q[(size_t)(kh * groups) * HD + t]), scale);
  // K and V rows of the chunk: 16 bytes per thread per step, coalesced.
  const uint16_t* kb = KC + ((size_t)kh * max_len + j0) * HD;
  const uint16_t* vb = VC + ((size_t)kh * max_len + j0) * HD;
  for (int t = tid; t < ACHUNK * (HD / 8); t += nthr) {
    const int j = t / (HD / 8), e = (t % (HD / 8)) * 8;
    u32x4 kv = {0u, 0u, 0u, 0u}, vv = {0u, 0u, 0u, 0u};
    if (j < nvalid) {
      kv = *reinterpret_cast<const u32x4*>(kb + (size_t)j * HD + e);
      vv = *reinterpret_cast<const u32x4*>(vb + (size_t)j * HD + e);
    }
    *reinterpret_cast<u32x4*>(k_s + j * KPAD + e) = kv;
    *reinterpret_cast<u32x4*>(v_s + j * HD + e) = vv;
  }
  __syncthreads();

  // score of position `lane` for query head g
  const float s = score4<DT>(q_s + g * HD, k_s + lane * KPAD);
  const bool valid = lane < nvalid;
  const float m = wave_max_u(valid ? s : -3.0e38f);
  const float p = valid ? exp_cw(__fsub_rn(s, m)) : 0.0f;
  const float l = wave_sum_dpp(p);
  p_s[g * ACHUNK + lane] = p;  // read back by this wave only: no barrier

  float a0, a1;
  pv4<DT>(p_s + g * ACHUNK, v_s, nvalid, lane, a0, a1);
  if (lane == 0) {
    PM[slot] = m;
    PL[slot] = l;
  }
  reinterpret_cast<float2*>(PACC + slot * HD)[lane] = make_float2(a0, a1);
}

// Merge of the chunk partials of one query head: with M the largest chunk
// maximum, chunk weights w_c = exp(m_c - M) (0 for chunks with l = 0, past
// the live positions) are computed once per chunk into LDS, then every
// thread (one output dimension) folds the chunks in order: den += l_c * w_c,
// num += acc_c[d] * w_c, skipping chunks with l = 0; y = num / den. The
// partial sums are read in batches of CMB chunks, each batch requested
// before the previous one is folded (the first before the chunk maxima).
constexpr int CMB = 16;
constexpr int CMAX = 4 * HD;  // chunks the merge takes (a 32768-position cache)
template <int DT>
__global__ __launch_bounds__(HD) void attn_combine_kernel(const float* __restrict__ PM,
                                                          const float* __restrict__ PL,
                                                          const float* __restrict__ PACC,
                                                          uint16_t* __restrict__ Y, int nchunk) {
  __shared__ __align__(16) float wl_s[CMAX][2];  // per chunk: w_c, l_c
  __shared__ float mx_s[2];
  // head blockIdx.x of query row blockIdx.y (the rows form; 0 for one position)
  const int qh = blockIdx.y * gridDim.x + blockIdx.x, d = threadIdx.x, lane = d & 63;
  const float* acc = PACC + (size_t)qh * nchunk * HD + d;
  float cur[CMB];
#pragma unroll
  for (int k = 0; k < CMB; ++k) cur[k] = acc[(size_t)min(k, nchunk - 1) * HD];
  const float* pm = PM + (size_t)qh * nchunk;
  const float* pl = PL + (size_t)qh * nchunk;
  constexpr int PC = CMAX / HD;  // chunks per thread
  float m[PC], l[PC];
#pragma unroll
  for (int k = 0; k < PC; ++k) {
    const int c = d + k * HD;
    m[k] = c < nchunk ? pm[c] : -3.0e38f;
    l[k] = c < nchunk ? pl[c] : 0.0f;
  }
  float mx = fmaxf(fmaxf(m[0], m[1]), fmaxf(m[2], m[3]));
  mx = wave_max_u(mx);
  if (lane == 0) mx_s[d >> 6] = mx;
  __syncthreads();
  const float M = fmaxf(mx_s[0], mx_s[1]);  // a max: exact in any order
#pragma unroll
  for (int k = 0; k < PC; ++k) {
    const int c = d + k * HD;
    if (c < nchunk) {
      wl_s[c][0] = l[k] == 0.0f ? 0.0f : exp_cw(__fsub_rn(m[k], M));
      wl_s[c][1] = l[k];
    }
  }
  __syncthreads();
  float num = 0.0f, den = 0.0f;
  for (int c0 = 0; c0 < nchunk; c0 += CMB) {
    float nxt[CMB];
#pragma unroll
    for (int k = 0; k < CMB; ++k) nxt[k] = acc[(size_t)min(c0 + CMB + k, nchunk - 1) * HD];
    f32x4 wl[CMB / 2];
#pragma unroll
    for (int k = 0; k < CMB / 2; ++k) wl[k] = *reinterpret_cast<const f32x4*>(&wl_s[min(c0 + 2 * k, CMAX - 2)][0]);
#pragma unroll
    for (int k = 0; k < CMB; ++k) {
      const float w = wl[k >> 1][(k & 1) * 2], lc = wl[k >> 1][(k & 1) * 2 + 1];
      const bool take = c0 + k < nchunk && lc != 0.0f;
      const float den1 = __fadd_rn(den, __fmul_rn(lc, w));
      const float num1 = __fadd_rn(num, __fmul_rn(cur[k], w));
      den = take ? den1 : den;
      num = take ? num1 : num;
    }
#pragma unroll
    for (int k = 0; k < CMB; ++k) cur[k] = nxt[k];
  }
  Y[(size_t)qh * HD + d] = Elem<DT>::store(__fdiv_rn(num, den));
}

// Attention of one decode position straight from QKV (see the file comment).
// Workgroup (kv head kh, chunk c), one wave per query head of the group.
template <int DT>
__global__ __launch_bounds__(1024) void attn_qkv_kernel(
    const uint16_t* __restrict__ QKV, const uint16_t* __restrict__ QW, const uint16_t* __restrict__ KW,
    float eps, const void* __restrict__ F, int ftype, const long long* __restrict__ POS,
    uint16_t* __restrict__ KC, uint16_t* __restrict__ VC, float* __restrict__ PM, float* __restrict__ PL,
    float* __restrict__ PACC, uint16_t* __restrict__ Y, int nh, int nkv, int groups, int max_len, int nchunk,
    float scale) {
  extern __shared__ __align__(16) float smem[];
  float* q_s = smem;                                                   // [groups][HD]
  float* p_s = q_s + groups * HD;                                      // [groups][ACHUNK]
  uint16_t* k_s = reinterpret_cast<uint16_t*>(p_s + groups * ACHUNK);  // [ACHUNK][KPAD]
  uint16_t* v_s = k_s + ACHUNK * KPAD;                                 // [ACHUNK][HD]

  const int kh = blockIdx.x, c = blockIdx.y;
  const int tid = threadIdx.x, nthr = blockDim.x;
  const int g = tid >> 6, lane = tid & 63;
  // All kernel arguments the loads need are fetched at once, here (otherwise
  // the compiler fetches them one branch at a time, each with its own wait).
  const long long pos0 = POS[0];  // issued first, waited for only after the loads below are issued
  asm volatile("" ::"s"(QKV), "s"(QW), "s"(KW), "s"(F), "s"(ftype), "s"(KC), "s"(VC), "s"(nh), "s"(nkv),
               "s"(max_len));
  const int qh = kh * groups + g;
  const long long j0 = (long long)c * ACHUNK;

  // Every global load of the workgroup is issued before the position is
  // known: this wave's query head with its norm weights and rotary factors,
  // the new K/V row (wave 0; used by the chunk that holds the position), then
  // the chunk's cached K and V rows, clamped into the cache allocation (rows
  // at or past the live range are staged but never read).
  // No load depends on a branch: absent norm weights read QKV instead (and
  // are not used), every wave reads the new K/V row.
  const bool qn = QW != nullptr, kn = KW != nullptr;
  const uint16_t* qwp = qn ? QW : QKV;
  const uint16_t* kwp = kn ? KW : QKV;
  const uint16_t* qr = QKV + (size_t)qh * HD;
  const uint16_t* kr_ = QKV + (size_t)(nh + kh) * HD;
  const uint16_t* vr = QKV + (size_t)(nh + nkv + kh) * HD;
  const uint16_t q0 = qr[lane], q1 = qr[lane + 64];
  const uint16_t qw0 = qwp[lane], qw1 = qwp[lane + 64];
  const RopeF rf = load_rope(F, ftype, lane);
  const uint16_t k0 = kr_[lane], k1 = kr_[lane + 64];
  const uint16_t v0 = vr[lane], v1 = vr[lane + 64];
  const uint16_t kw0 = kwp[lane], kw1 = kwp[lane + 64];
  const uint16_t* kb = KC + (size_t)kh * max_len * HD;
  const uint16_t* vb = VC + (size_t)kh * max_len * HD;
  constexpr int NT = ACHUNK * (HD / 8);  // 16-byte pieces of the chunk's K (and of its V)
  constexpr int PER = NT / 256;  // pieces per thread issued here: all of them with 4 or more waves
  u32x4 kq[PER], vq[PER];
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int t = min(tid + i * nthr, NT - 1);
    const long long row = min(j0 + t / (HD / 8), (long long)max_len - 1);
    const int e = (t % (HD / 8)) * 8;
    kq[i] = *reinterpret_cast<const u32x4*>(kb + (size_t)row * HD + e);
    vq[i] = *reinterpret_cast<const u32x4*>(vb + (size_t)row * HD + e);
  }
  __builtin_amdgcn_sched_barrier(0);
  const long long pos = pos0;

  if (pos < 0 || pos >= max_len) return;  // no cache slot for it: nothing is written
  const long long L = pos + 1;
  const size_t slot = (size_t)qh * nchunk + c;
  if (j0 >= L) {  // a chunk past the live positions (only with nchunk > 1)
    if (lane == 0) {
      PM[slot] = -1e30f;
      PL[slot] = 0.0f;
    }
    return;
  }
  const int nvalid = (int)min((long long)ACHUNK, L - j0);
  const int jpos = (int)(pos - j0);  // the new row's place in this chunk, if < ACHUNK
  const bool newrow = jpos < ACHUNK && g == 0;

  // this wave's query head: norm, rotary, rounded as the stored Q, scaled
  {
    float lo = Elem<DT>::load(q0), hi = Elem<DT>::load(q1);
    head_norm_rope<DT>(lo, hi, qn, qw0, qw1, eps, rf, lane);
    q_s[g * HD + lane] = __fmul_rn(Elem<DT>::load(Elem<DT>::store(lo)), scale);
    q_s[g * HD + lane + 64] = __fmul_rn(Elem<DT>::load(Elem<DT>::store(hi)), scale);
  }
  // the new position's K/V row: into the staged chunk now, into the cache
  // at the end (no later step of this launch reads it from there)
  uint16_t klo = 0, khi = 0;
  if (newrow) {
    float lo = Elem<DT>::load(k0), hi = Elem<DT>::load(k1);
    head_norm_rope<DT>(lo, hi, kn, kw0, kw1, eps, rf, lane);
    klo = Elem<DT>::store(lo);
    khi = Elem<DT>::store(hi);
    k_s[jpos * KPAD + lane] = klo;
    k_s[jpos * KPAD + lane + 64] = khi;
    v_s[jpos * HD + lane] = v0;
    v_s[jpos * HD + lane + 64] = v1;
  }
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int t = tid + i * nthr;
    const int j = t / (HD / 8), e = (t % (HD / 8)) * 8;
    if (t < NT && j != jpos) {
      *reinterpret_cast<u32x4*>(k_s + j * KPAD + e) = kq[i];
      *reinterpret_cast<u32x4*>(v_s + j * HD + e) = vq[i];
    }
  }
  for (int t = tid + PER * nthr; t < NT; t += nthr) {  // the rest, with fewer than 4 waves
    const int j = t / (HD / 8), e = (t % (HD / 8)) * 8;
    if (j == jpos) continue;
    const long long jr = j0 + min(j, nvalid - 1);
    *reinterpret_cast<u32x4*>(k_s + j * KPAD + e) = *reinterpret_cast<const u32x4*>(kb + (size_t)jr * HD + e);
    *reinterpret_cast<u32x4*>(v_s + j * HD + e) = *reinterpret_cast<const u32x4*>(vb + (size_t)jr * HD + e);
  }
  __syncthreads();

  // score of position `lane` for query head g (as attn_partial_kernel)
  const float s = score4<DT>(q_s + g * HD, k_s + lane * KPAD);
  const bool valid = lane < nvalid;
  const float m = wave_max_u(valid ? s : -3.0e38f);
  const float p = valid ? exp_cw(__fsub_rn(s, m)) : 0.0f;
  const float l = wave_sum_dpp(p);
  p_s[g * ACHUNK + lane] = p;  // read back by this wave only: no barrier

  float a0, a1;
  pv4<DT>(p_s + g * ACHUNK, v_s, nvalid, lane, a0, a1);
  if (newrow) {
    const size_t row = ((size_t)kh * max_len + pos) * HD;
    KC[row + lane] = klo;
    KC[row + lane + 64] = khi;
    VC[row + lane] = v0;
    VC[row + lane + 64] = v1;
  }
  if (nchunk == 1) {
    // the merge of a single chunk, as attn_combine_kernel computes it
    const float w = exp_cw(__fsub_rn(m, m));
    const float den = __fadd_rn(0.0f, __fmul_rn(l, w));
    const float y0 = __fdiv_rn(__fadd_rn(0.0f, __fmul_rn(a0, w)), den);
    const float y1 = __fdiv_rn(__fadd_rn(0.0f, __fmul_rn(a1, w)), den);
    reinterpret_cast<uint32_t*>(Y + (size_t)qh * HD)[lane] =
        (uint32_t)Elem<DT>::store(y0) | ((uint32_t)Elem<DT>::store(y1) << 16);
    return;
  }
  if (lane == 0) {
    PM[slot] = m;
    PL[slot] = l;
  }
  reinterpret_cast<float2*>(PACC + slot * HD)[lane] = make_float2(a0, a1);
}

// The rows form of attn_qkv_kernel, for a short causal span: rows r = 0 ..
// nrows - 1 at positions POS[r], QKV row r at QKV + r qkv_rs and rotary row
// r at F + r HD. Workgroup (kv head kh, chunk c, row r) takes query head
// kh groups + w of row r in wave w, and stages every span row whose position
// falls in its chunk from that row's QKV K/V heads (norm and rotary, as
// qk_rope_kv_kernel), so no workgroup reads a cache row that another writes in
// this launch; the wave that computes span row r in the chunk holding POS[r]
// writes it to the cache. Partials go to slot (r nh + qh) nchunk + c for
// attn_combine_kernel's rows form. The bits are those of qk_rope_kv_kernel
// over the rows followed by attn_partial_kernel's rows form.
constexpr int ATT_ROWS_MAX = 8;
template <int DT>
__global__ __launch_bounds__(1024) void attn_qkv_rows_kernel(
    const uint16_t* __restrict__ QKV, int qkv_rs, const uint16_t* __restrict__ QW, const uint16_t* __restrict__ KW,
    float eps, const void* __restrict__ F, int ftype, const long long* __restrict__ POS, int nrows,
    uint16_t* __restrict__ KC, uint16_t* __restrict__ VC, float* __restrict__ PM, float* __restrict__ PL,
    float* __restrict__ PACC, int nh, int nkv, int groups, int max_len, int nchunk, float scale) {
  extern __shared__ __align__(16) float smem[];
  float* q_s = smem;                                                   // [groups][HD]
  float* p_s = q_s + groups * HD;                                      // [groups][ACHUNK]
  uint16_t* k_s = reinterpret_cast<uint16_t*>(p_s + groups * ACHUNK);  // [ACHUNK][KPAD]
  uint16_t* v_s = k_s + ACHUNK * KPAD;                                 // [ACHUNK][HD]

  const int kh = blockIdx.x, c = blockIdx.y, r = blockIdx.z;
  const int tid = threadIdx.x, nthr = blockDim.x;
  const int g = tid >> 6, lane = tid & 63;
  const int qh = kh * groups + g;
  const long long j0 = (long long)c * ACHUNK;
  const int fs = ftype == DT_F32 ? 4 : 2;  // bytes a rotary element
  // every position of the span (lane j: row j), the query head with its norm
  // weights and rotary row, then the chunk's cached K and V rows
  const long long posl = POS[min(lane, nrows - 1)];
  const bool qn = QW != nullptr, kn = KW != nullptr;
  const uint16_t* qwp = qn ? QW : QKV;
  const uint16_t* kwp = kn ? KW : QKV;
  const uint16_t* qr = QKV + (size_t)r * qkv_rs + (size_t)qh * HD;
  const uint16_t q0 = qr[lane], q1 = qr[lane + 64];
  const uint16_t qw0 = qwp[lane], qw1 = qwp[lane + 64];
  const uint16_t kw0 = kwp[lane], kw1 = kwp[lane + 64];
  const RopeF rf = load_rope((const uint8_t*)F + (size_t)r * HD * fs, ftype, lane);
  const uint16_t* kb = KC + (size_t)kh * max_len * HD;
  const uint16_t* vb = VC + (size_t)kh * max_len * HD;
  constexpr int NT = ACHUNK * (HD / 8);
  constexpr int PER = NT / 256;
  u32x4 kq[PER], vq[PER];
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int t = min(tid + i * nthr, NT - 1);
    const long long row = min(j0 + t / (HD / 8), (long long)max_len - 1);
    const int e = (t % (HD / 8)) * 8;
    kq[i] = *reinterpret_cast<const u32x4*>(kb + (size_t)row * HD + e);
    vq[i] = *reinterpret_cast<const u32x4*>(vb + (size_t)row * HD + e);
  }
  const long long pos = __shfl(posl, r, 64);
  if (pos < 0 || pos >= max_len) return;  // no cache slot for it: nothing is written
  const long long L = pos + 1;
  const size_t slot = ((size_t)r * nh + qh) * nchunk + c;
  if (j0 >= L) {  // a chunk past the row's live positions
    if (lane == 0) {
      PM[slot] = -1e30f;
      PL[slot] = 0.0f;
    }
    return;
  }
  const int nvalid = (int)min((long long)ACHUNK, L - j0);
  // chunk rows holding a span row (their cached values are stale: computed here instead)
  uint64_t span = 0;
  for (int j = 0; j < nrows; ++j) {
    const long long pj = __shfl(posl, j, 64);
    if (pj >= j0 && pj < j0 + ACHUNK && pj < max_len) span |= 1ull << (int)(pj - j0);
  }

  // this wave's query head of row r: norm, rotary, rounded as the stored Q, scaled
  {
    float lo = Elem<DT>::load(q0), hi = Elem<DT>::load(q1);
    head_norm_rope<DT>(lo, hi, qn, qw0, qw1, eps, rf, lane);
    q_s[g * HD + lane] = __fmul_rn(Elem<DT>::load(Elem<DT>::store(lo)), scale);
    q_s[g * HD + lane + 64] = __fmul_rn(Elem<DT>::load(Elem<DT>::store(hi)), scale);
  }
  // the span rows in this chunk, wave w taking rows w, w + groups, ...: K
  // normed and rotated as qk_rope_kv_kernel stores it, V as it is
  for (int j = g; j < nrows; j += groups) {
    const long long pj = __shfl(posl, j, 64);
    if (pj < j0 || pj >= j0 + ACHUNK || pj >= max_len) continue;
    const uint16_t* kr = QKV + (size_t)j * qkv_rs + (size_t)(nh + kh) * HD;
    const uint16_t* vr = QKV + (size_t)j * qkv_rs + (size_t)(nh + nkv + kh) * HD;
    const RopeF fj = load_rope((const uint8_t*)F + (size_t)j * HD * fs, ftype, lane);
    float lo = Elem<DT>::load(kr[lane]), hi = Elem<DT>::load(kr[lane + 64]);
    const uint16_t v0 = vr[lane], v1 = vr[lane + 64];
    head_norm_rope<DT>(lo, hi, kn, kw0, kw1, eps, fj, lane);
    const uint16_t klo = Elem<DT>::store(lo), khi = Elem<DT>::store(hi);
    const int jj = (int)(pj - j0);
    k_s[jj * KPAD + lane] = klo;
    k_s[jj * KPAD + lane + 64] = khi;
    v_s[jj * HD + lane] = v0;
    v_s[jj * HD + lane + 64] = v1;
    if (j == r) {  // row r's K/V into the cache (read by no workgroup of this launch)
      const size_t row = ((size_t)kh * max_len + pj) * HD;
      KC[row + lane] = klo;
      KC[row + lane + 64] = khi;
      VC[row + lane] = v0;
      VC[row + lane + 64] = v1;
    }
  }
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int t = tid + i * nthr;
    const int j = t / (HD / 8), e = (t % (HD / 8)) * 8;
    if (t < NT && !((span >> j) & 1ull)) {
      *reinterpret_cast<u32x4*>(k_s + j * KPAD + e) = kq[i];
      *reinterpret_cast<u32x4*>(v_s + j * HD + e) = vq[i];
    }
  }
  for (int t = tid + PER * nthr; t < NT; t += nthr) {  // the rest, with fewer than 4 waves
    const int j = t / (HD / 8), e = (t % (HD / 8)) * 8;
    if ((span >> j) & 1ull) continue;
    const long long jr = j0 + min(j, nvalid - 1);
    *reinterpret_cast<u32x4*>(k_s + j * KPAD + e) = *reinterpret_cast<const u32x4*>(kb + (size_t)jr * HD + e);
    *reinterpret_cast<u32x4*>(v_s + j * HD + e) = *reinterpret_cast<const u32x4*>(vb + (size_t)jr * HD + e);
  }
  __syncthreads();

  const float s = score4<DT>(q_s + g * HD, k_s + lane * KPAD);
  const bool valid = lane < nvalid;
  const float m = wave_max_u(valid ? s : -3.0e38f);
  const float p = valid ? exp_cw(__fsub_rn(s, m)) : 0.0f;
  const float l = wave_sum_dpp(p);
  p_s[g * ACHUNK + lane] = p;  // read back by this wave only: no barrier
  float a0, a1;
  pv4<DT>(p_s + g * ACHUNK, v_s, nvalid, lane, a0, a1);
  if (lane == 0) {
    PM[slot] = m;
    PL[slot] = l;
  }
  reinterpret_cast<float2*>(PACC + slot * HD)[lane] = make_float2(a0, a1);
}

}  // namespace ttsp

using namespace ttsp;

extern "C" int ttsp_attn_chunk(void) { return ACHUNK; }

extern "C" int ttsp_qk_rope_kv(const void* QKV, const void* QW, const void* KW, float eps,
                               const void* F, int ftype, const long long* POS, void* Q, void* KC,
                               void* VC, int nh, int nkv, int max_len, int dtype,
                               hipStream_t stream) {
  if (nh <= 0 || nkv <= 0 || max_len <= 0 || ftype < 0 || ftype > 2 || (uintptr_t)F % 4)
    return (int)hipErrorInvalidValue;
#define TTSP_QK(DTV)                                                                            \
  hipLaunchKernelGGL(qk_rope_kv_kernel<DTV>, dim3((nh + 2 * nkv + QKV_WAVES - 1) / QKV_WAVES), dim3(64 * QKV_WAVES), \
                     0, stream,                                                                 \
                     (const uint16_t*)QKV, (const uint16_t*)QW, (const uint16_t*)KW, eps, F, ftype, \
                     POS, (uint16_t*)Q, (uint16_t*)KC, (uint16_t*)VC, nh, nkv, max_len, 0)
  if (dtype == DT_F16) TTSP_QK(DT_F16);
  else if (dtype == DT_BF16) TTSP_QK(DT_BF16);
  else return (int)hipErrorInvalidValue;
#undef TTSP_QK
  TTSP_RETURN_LAUNCH();
}

extern "C" int ttsp_qk_rope_kv_rows(const void* QKV, long long qkv_row_stride, const void* QW, const void* KW,
                                    float eps, const void* F, int ftype, const long long* POS, void* Q, void* KC,
                                    void* VC, int nh, int nkv, int max_len, int rows, int dtype,
                                    hipStream_t stream) {
  if (nh <= 0 || nkv <= 0 || max_len <= 0 || ftype < 0 || ftype > 2 || rows <= 0 || rows > 65535 ||
      qkv_row_stride < (long long)(nh + 2 * nkv) * HD || qkv_row_stride > (1LL << 30) || (uintptr_t)F % 4)
    return (int)hipErrorInvalidValue;
#define TTSP_QKR(DTV)                                                                            \
  hipLaunchKernelGGL(qk_rope_kv_kernel<DTV>, dim3((nh + 2 * nkv + QKV_WAVES - 1) / QKV_WAVES, rows),          \
                     dim3(64 * QKV_WAVES), 0, stream,                                           \
                     (const uint16_t*)QKV, (const uint16_t*)QW, (const uint16_t*)KW, eps, F, ftype, \
                     POS, (uint16_t*)Q, (uint16_t*)KC, (uint16_t*)VC, nh, nkv, max_len, (int)qkv_row_stride)
  if (dtype == DT_F16) TTSP_QKR(DT_F16);
  else if (dtype == DT_BF16) TTSP_QKR(DT_BF16);
  else return (int)hipErrorInvalidValue;
#undef TTSP_QKR
  TTSP_RETURN_LAUNCH();
}

extern "C" int ttsp_qk_rope_kv_rows_partials(const float* YP, int splits, const void* QW, const void* KW, float eps,
                                             const void* F, int ftype, const long long* POS, void* Q, void* KC,
                                             void* VC, int nh, int nkv, int max_len, int rows, int dtype,
                                             hipStream_t stream) {
  if (nh <= 0 || nkv <= 0 || max_len <= 0 || ftype < 0 || ftype > 2 || rows <= 0 || rows > 65535 || !YP ||
      splits < 2 || splits > 8 || (uintptr_t)F % 4)
    return (int)hipErrorInvalidValue;
  const int qkv_rs = (nh + 2 * nkv) * HD;
#define TTSP_QKP(DTV)                                                                                           \
  hipLaunchKernelGGL((qk_rope_kv_kernel<DTV, true>), dim3((nh + 2 * nkv + QKV_WAVES - 1) / QKV_WAVES, rows),      \
                     dim3(64 * QKV_WAVES), 0, stream, nullptr, (const uint16_t*)QW, (const uint16_t*)KW, eps, F, \
                     ftype, POS, (uint16_t*)Q, (uint16_t*)KC, (uint16_t*)VC, nh, nkv, max_len, qkv_rs, YP, splits)
  if (dtype == DT_F16) TTSP_QKP(DT_F16);
  else if (dtype == DT_BF16) TTSP_QKP(DT_BF16);
  else return (int)hipErrorInvalidValue;
#undef TTSP_QKP
  TTSP_RETURN_LAUNCH();
}

extern "C" int ttsp_attn_decode_rows(const void* Q, const void* KC, const void* VC, const long long* POS,
                                     float* PM, float* PL, float* PACC, void* Y, int nh, int nkv, int max_len,
                                     int nchunk, float scale, int rows, int dtype, hipStream_t stream) {
  if (nh <= 0 || nkv <= 0 || nh % nkv || nchunk <= 0 || max_len <= 0 || rows <= 0 || rows > 65535 || !Q || !KC ||
      !VC || !POS || !PM || !PL || !PACC || !Y)
    return (int)hipErrorInvalidValue;
  const int groups = nh / nkv;
  if (groups > 16 || nchunk > CMAX) return (int)hipErrorInvalidValue;
  const size_t shmem = sizeof(float) * (size_t)groups * (HD + ACHUNK) +
                       sizeof(uint16_t) * (size_t)ACHUNK * (KPAD + HD);
#define TTSP_AR(DTV)                                                                                    \
  do {                                                                                                  \
    hipLaunchKernelGGL(attn_partial_kernel<DTV>, dim3(nkv, nchunk, rows), dim3(64 * groups), shmem, stream, \
                       (const uint16_t*)Q, (const uint16_t*)KC, (const uint16_t*)VC, POS, PM, PL, PACC,    \
                       groups, max_len, nchunk, scale);                                                 \
    hipLaunchKernelGGL(attn_combine_kernel<DTV>, dim3(nh, rows), dim3(HD), 0, stream, PM, PL, PACC,     \
                       (uint16_t*)Y, nchunk);                                                           \
  } while (0)
  if (dtype == DT_F16) TTSP_AR(DT_F16);
  else if (dtype == DT_BF16) TTSP_AR(DT_BF16);
  else return (int)hipErrorInvalidValue;
#undef TTSP_AR
  TTSP_RETURN_LAUNCH();
}

extern "C" int ttsp_attn_decode_qkv_rows(const void* QKV, int qkv_rs, const void* QW, const void* KW, float eps,
                                         const void* F, int ftype, const long long* POS, void* KC, void* VC,
                                         float* PM, float* PL, float* PACC, void* Y, int nh, int nkv, int max_len,
                                         int nchunk, float scale, int rows, int dtype, hipStream_t stream) {
  if (!QKV || !F || !POS || !KC || !VC || !PM || !PL || !PACC || !Y || nh <= 0 || nkv <= 0 || nh % nkv ||
      max_len <= 0 || nchunk <= 0 || rows < 1 || rows > ATT_ROWS_MAX || ftype < 0 || ftype > 2 || (uintptr_t)F % 4 ||
      qkv_rs < (nh + 2 * nkv) * HD)
    return (int)hipErrorInvalidValue;
  const int groups = nh / nkv;
  if (groups > 16 || nchunk > CMAX) return (int)hipErrorInvalidValue;
  const size_t shmem = sizeof(float) * (size_t)groups * (HD + ACHUNK) +
                       sizeof(uint16_t) * (size_t)ACHUNK * (KPAD + HD);
  const uint16_t* qw = (const uint16_t*)QW;
  const uint16_t* kw = (const uint16_t*)KW;
#define TTSP_AQR(DTV)                                                                                           \
  do {                                                                                                          \
    hipLaunchKernelGGL(attn_qkv_rows_kernel<DTV>, dim3(nkv, nchunk, rows), dim3(64 * groups), shmem, stream,     \
                       (const uint16_t*)QKV, qkv_rs, qw, kw, eps, F, ftype, POS, rows, (uint16_t*)KC,             \
                       (uint16_t*)VC, PM, PL, PACC, nh, nkv, groups, max_len, nchunk, scale);                    \
    hipLaunchKernelGGL(attn_combine_kernel<DTV>, dim3(nh, rows), dim3(HD), 0, stream, PM, PL, PACC,             \
                       (uint16_t*)Y, nchunk);                                                                   \
  } while (0)
  if (dtype == DT_F16) TTSP_AQR(DT_F16);
  else if (dtype == DT_BF16) TTSP_AQR(DT_BF16);
  else return (int)hipErrorInvalidValue;
#undef TTSP_AQR
  TTSP_RETURN_LAUNCH();
}

extern "C" int ttsp_attn_decode(const void* Q, const void* KC, const void* VC,
                                const long long* POS, float* PM, float* PL, float* PACC, void* Y,
                                int nh, int nkv, int max_len, int nchunk, float scale, int dtype,
                                hipStream_t stream) {
  if (nh <= 0 || nkv <= 0 || nh % nkv || nchunk <= 0 || max_len <= 0) return (int)hipErrorInvalidValue;
  const int groups = nh / nkv;
  if (groups > 16 || nchunk > CMAX) return (int)hipErrorInvalidValue;
  const size_t shmem = sizeof(float) * (size_t)groups * (HD + ACHUNK) +
                       sizeof(uint16_t) * (size_t)ACHUNK * (KPAD + HD);
#define TTSP_AT(DTV)                                                                            \
  do {                                                                                          \
    hipLaunchKernelGGL(attn_partial_kernel<DTV>, dim3(nkv, nchunk), dim3(64 * groups), shmem,    \
                       stream, (const uint16_t*)Q, (const uint16_t*)KC, (const uint16_t*)VC, POS, \
                       PM, PL, PACC, groups, max_len, nchunk, scale);                           \
    hipLaunchKernelGGL(attn_combine_kernel<DTV>, dim3(nh), dim3(HD), 0, stream, PM, PL, PACC,   \
                       (uint16_t*)Y, nchunk);                                                   \
  } while (0)
  if (dtype == DT_F16) TTSP_AT(DT_F16);
  else if (dtype == DT_BF16) TTSP_AT(DT_BF16);
  else return (int)hipErrorInvalidValue;
#undef TTSP_AT
  TTSP_RETURN_LAUNCH();
}

extern "C" int ttsp_attn_decode_qkv(const void* QKV, const void* QW, const void* KW, float eps,
                                    const void* F, int ftype, const long long* POS, void* KC, void* VC,
                                    float* PM, float* PL, float* PACC, void* Y, int nh, int nkv,
                                    int max_len, int nchunk, float scale, int dtype, hipStream_t stream) {
  if (nh <= 0 || nkv <= 0 || nh % nkv || nchunk <= 0 || max_len <= 0 || ftype < 0 || ftype > 2)
    return (int)hipErrorInvalidValue;
  const int groups = nh / nkv;
  if (groups > 16 || nchunk > CMAX || (nchunk > 1 && (!PM || !PL || !PACC))) return (int)hipErrorInvalidValue;
  const size_t shmem = sizeof(float) * (size_t)groups * (HD + ACHUNK) +
                       sizeof(uint16_t) * (size_t)ACHUNK * (KPAD + HD);
#define TTSP_AQ(DTV)                                                                                  \
  do {                                                                                                \
    hipLaunchKernelGGL(attn_qkv_kernel<DTV>, dim3(nkv, nchunk), dim3(64 * groups), shmem, stream,     \
                       (const uint16_t*)QKV, (const uint16_t*)QW, (const uint16_t*)KW, eps, F, ftype, \
                       POS, (uint16_t*)KC, (uint16_t*)VC, PM, PL, PACC, (uint16_t*)Y, nh, nkv, groups, \
                       max_len, nchunk, scale);                                                       \
    if (nchunk > 1)                                                                                   \
      hipLaunchKernelGGL(attn_combine_kernel<DTV>, dim3(nh), dim3(HD), 0, stream, PM, PL, PACC,       \
                         (uint16_t*)Y, nchunk);                                                       \
  } while (0)
  if (dtype == DT_F16) TTSP_AQ(DT_F16);
  else if (dtype == DT_BF16) TTSP_AQ(DT_BF16);
  else return (int)hipErrorInvalidValue;
#undef TTSP_AQ
  TTSP_RETURN_LAUNCH();
}

// ---------------------------------------------------------------------------
// The allocation-free form of ttsp_attn_decode_qkv: the split-K partials live
// in a file-scope device array (one copy per GPU, held until the process
// ends) instead of caller buffers. Host code never passes the array's name to
// a kernel: its device address is looked up once per device with that device
// current (hipGetSymbolAddress) and kept in attn_scratch_ptr.
constexpr int NOALLOC_SLOTS = 4096;  // nh * nchunk: e.g. 32 heads over a 8192-position cache
constexpr int NOALLOC_FLOATS = NOALLOC_SLOTS * (2 + HD);  // PM, PL, then PACC [slots][128]
static __device__ __align__(256) float scratch[NOALLOC_FLOATS];

namespace {
constexpr int kMaxDevices = 64;
std::mutex attn_scratch_mu;
float* attn_scratch_ptr[kMaxDevices];

// The scratch array's address on the device `stream` runs on (the current
// device for the null stream); set up on the first call for that device.
int attn_scratch(hipStream_t stream, float** out) {
  int dev = 0;
  hipError_t rc = stream ? hipStreamGetDevice(stream, &dev) : hipGetDevice(&dev);
  if (rc != hipSuccess) return (int)rc;
  if (dev < 0 || dev >= kMaxDevices) return (int)hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lock(attn_scratch_mu);
  if (!attn_scratch_ptr[dev]) {
    int cur = 0;
    if ((rc = hipGetDevice(&cur)) != hipSuccess) return (int)rc;
    if (cur != dev && (rc = hipSetDevice(dev)) != hipSuccess) return (int)rc;
    void* p = nullptr;
    rc = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (cur != dev) {
      const hipError_t back = hipSetDevice(cur);
      if (rc == hipSuccess) rc = back;
    }
    if (rc != hipSuccess) return (int)rc;
    attn_scratch_ptr[dev] = static_cast<float*>(p);
  }
  *out = attn_scratch_ptr[dev];
  return 0;
}
}  // namespace

extern "C" int ttsp_attn_decode_qkv_noalloc(const void* QKV, const void* QW, const void* KW, float eps,
                                            const void* F, int ftype, const long long* POS, void* KC, void* VC,
                                            void* Y, int nh, int nkv, int max_len, int nchunk, float scale,
                                            int dtype, hipStream_t stream) {
  if (nh <= 0 || nchunk <= 0 || (long long)nh * nchunk > NOALLOC_SLOTS) return (int)hipErrorInvalidValue;
  float* s = nullptr;
  if (int rc = attn_scratch(stream, &s)) return rc;
  return ttsp_attn_decode_qkv(QKV, QW, KW, eps, F, ftype, POS, KC, VC, s, s + NOALLOC_SLOTS, s + 2 * NOALLOC_SLOTS, Y,
                              nh, nkv, max_len, nchunk, scale, dtype, stream);
}

extern "C" int ttsp_attn_decode_qkv_noalloc_max_slots(void) { return NOALLOC_SLOTS; }
