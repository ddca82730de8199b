// NF4 GEMV (one activation row), reading the bitsandbytes layout in place:
//   * W is the row-major flattened weight, two 4-bit codes per byte, the HIGH
//     nibble holding the even flattened index (byte j = q[2j] << 4 | q[2j+1]);
//   * scale block b covers flattened codes [b*bs, (b+1)*bs), bs a power of two
//     >= 64, so with K % bs == 0 a block never straddles a row;
//   * plain scales are fp32 absmax[b]; nested ("double-quant") scales are
//     code2[a8[b]] * absmax2[b >> log2(bs2)] + offset, two fp32 roundings.
//
// One kernel serves three forms of a decode-block matmul:
//   * plain      y = epi(x . W^T)              (the reference's nf4_mma at N=1)
//   * + norm     y = epi(rmsnorm(x) . W^T)     (the fork's RMSNorm folded in)
//   * SwiGLU     y = round(round(silu(round(x.W1^T))) * round(x.W3^T)), two
//                weights of one shape streamed by the same waves (w1 and w3).
//
// Design. At batch 1 every weight byte is used once, so the kernel is a
// stream of W from HBM, and at decode shapes (1-25 MB) it is short enough that
// launch latency and the per-byte instruction count, not the bus, set its time.
//   * Ownership. A row is K/8 dwords (8 codes each). Lane l of a wave owns
//     dwords d = l + 64*(j*KS + ks) of every row the wave visits: each load
//     instruction reads 256 contiguous bytes, and the 8 activations matching a
//     dword stay in registers for all of the wave's rows. 8 waves per
//     workgroup: KS of them split K, 8 / KS row groups of RPW rows.
//   * Issue order. Everything small (code table, code2, the workgroup's
//     scales, the residual operand, x, the norm weight) is requested before the
//     weights, so waiting for it never waits for the weight stream (vector
//     memory counters retire in order), and every weight dword of a wave is in
//     flight before anything waits. All loads are unconditional (clamped
//     addresses, dummy pointers for absent operands): no branch ever separates
//     a load from its use, which keeps the compiler's wait counts exact, so the
//     dot products start as rows arrive.
//   * One pass of set-up while the weights stream, two barriers: each lane
//     writes its share of the code table straight from the 16 code points (no
//     staging), code2 goes to LDS and - with a norm - waves 0..J-1 each
//     normalise 64 chunks of x for the workgroup (every wave holds all of x at
//     KS == 1, so the sum of squares needs no barrier); after the first
//     barrier the scales are resolved once per workgroup and x is read as fp32.
//   * Code lookup without bank conflicts. Each byte (two codes) becomes a
//     packed pair of fp16 code values through a 256-entry table replicated 64
//     times in LDS, entry e of lane l at byte 256*e + 4*l: the 64 lanes of a
//     lookup always hit 64 different banks, and the address is one v_perm_b32
//     (the byte of W next to the lane's own offset).
//   * Arithmetic (fixed order, so a CPU restatement reproduces every bit): a
//     dword's 8 products are chained in code order (v_fma_mix_f32: fp16 code
//     times fp32 activation, exact, the first onto +0), the dword's partial
//     meets its block scale in one fma into the lane accumulator - the scale
//     multiplies the block's partial sum, the factored form of the reference
//     CPU kernel (app/engine/nf4cpu.py:115-129). fp16 and bf16 activations are
//     both exact in fp32, so one loop serves both.
//   * Reductions: lanes by DPP adds (the xor 1, 2, 4, 8 tree inside 16-lane
//     rows, then the row sums as (r3 + r2) + (r1 + r0)); K-slices left to
//     right through LDS. No atomics anywhere.
#include "gemv_common.h"

namespace ttsp {

constexpr int XC_MAX = 3;                      // x chunks per thread held in registers (K <= 3 * 512 * 8)
#ifndef GEMV_LOOKAHEAD
#define GEMV_LOOKAHEAD 3                       // (row, chunk) items whose code lookups run ahead
#endif
#ifndef GEMV_PREFETCH_ROWS
#define GEMV_PREFETCH_ROWS 2                   // weight rows in flight before the barrier
#endif

// One NF4 weight. For plain scales A8 and CODE2 point at any readable memory
// (AMAX): the kernel reads them unconditionally and discards the values.
struct Nf4Mat {
  const uint32_t* W;
  const uint8_t* A8;
  const float* AMAX;
  const float* CODE2;
  float offset;
};

// The attention whose output is the GEMV's x (the attention-prologue form):
// one decode position, all query heads, a cache of at most one chunk.
struct AttnSrc {
  const uint16_t* QKV;    // [nh + 2 nkv][128]
  const uint16_t* QW;     // q / k head-norm weights, or QKV (hcfg says which are used)
  const uint16_t* KW;
  const void* F;          // the position's rotary row
  const long long* POS;
  uint16_t* KC;           // [nkv][max_len][128]
  uint16_t* VC;
  float eps, scale;
  int max_len;            // <= 64
  uint32_t hcfg;          // nh | nkv << 8 | groups << 16 | ftype << 24 | qn << 28 | kn << 29
};

struct GemvParams {
  Nf4Mat mat[2];          // mat[1]: the SwiGLU form's second weight (w3)
  const float* LUT;       // the 16 NF4 code points
  const uint16_t* X;      // [N][K]
  const uint16_t* G;      // RMSNorm weight [K], or readable dummy
  const uint16_t* R;      // epilogue operand [N][M], or readable dummy
  uint16_t* Y;            // [N][M]
  float eps;
  int M, K, N, KS, bs_shift, bs2_shift;  // N: activation rows (1, or up to NR of the rows form)
  int dt;                 // DT_F16 / DT_BF16
  int nested, norm, epi;  // flags; epi: 0 none, 1 residual, 2 silu gate
  AttnSrc att;            // the attention-prologue form only
};



// Dynamic LDS after the static table: code2 [NM][256], norm partials [NR][8],
// K-slice partials [8][NM*NR*RPW], the resolved scales [8 waves][NM][RPW][8 J]
// (16-byte aligned), then x as staged [NR][K/8].
// The leading scalar arguments are what the first loads need (weight 0's
// stream and scales, x, the code tables, the sizes): the command processor
// preloads them into SGPRs, so those loads issue at wave start; the rest of
// GemvParams is fetched once they are in flight. mk = M | (K / 128) << 20,
// cfg = KS | bs_shift << 4 | bs2_shift << 8 | dt << 12 | nested << 14 |
// norm << 15.
template <int J, int RPW, int NM, bool ATT = false, int NR = 1>
__global__ __launch_bounds__(GEMV_THREADS) void nf4_gemv_kernel(
    const uint32_t* __restrict__ W0, const uint16_t* __restrict__ X, const float* __restrict__ LUT,
    const uint8_t* __restrict__ A80, const float* __restrict__ AM0, const float* __restrict__ C20, uint32_t mk,
    uint32_t cfg, const GemvParams p) {
  constexpr int NW = GEMV_WAVES;
  constexpr int nthr = GEMV_THREADS;
  constexpr int G = 256 * LUT_REP / (4 * 64 * NW);  // table stores (16 bytes) per lane
  static_assert(NW % 4 == 0, "table entry split assumes 4 | waves");
  // Scale entries per thread: a workgroup holds (8 / KS) * RPW rows of at
  // most 8 * J * KS blocks (bs >= 64), i.e. <= 64 * RPW * J entries per weight.
  constexpr int SL = (NM * RPW * J + 7) / 8;
  constexpr int PF = RPW < GEMV_PREFETCH_ROWS ? RPW : GEMV_PREFETCH_ROWS;
  __shared__ __align__(16) uint32_t lut_rep[256 * LUT_REP];
  extern __shared__ __align__(16) unsigned char lds_dyn[];
  float* code2_s = reinterpret_cast<float*>(lds_dyn);  // [NM][256]
  float* wpart = code2_s + NM * 256;                   // [NR][NW] norm partial sums
  float* red = wpart + NR * NW;                        // [NW][NM*NR*RPW]
  float* srow = red + NW * NM * NR * RPW;              // [NW][NM][RPW][8 J] scale slots

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = uniform(tid >> 6);
  const int KS = (int)(cfg & 15u), ks = wave % KS, rg = wave / KS;
  const int bs_shift = (int)((cfg >> 4) & 15u), bs2_shift = (int)((cfg >> 8) & 15u);
  const int RG = NW / KS;
  const int M = (int)(mk & 0xfffffu), K = (int)(mk >> 20) * 128, KD = K >> 3;
  const int nblk = K >> bs_shift, sh = bs_shift - 3;
  const int rows_wg = RG * RPW;
  const int wg_row0 = blockIdx.x * rows_wg;
  const int row0 = wg_row0 + rg * RPW;
  const int dt = (int)((cfg >> 12) & 3u);
  const bool nested = (cfg >> 14) & 1u, norm = (cfg >> 15) & 1u;
  // weight m's operands: m = 0 from the preloaded arguments (the SwiGLU
  // form's second weight comes from GemvParams, fetched here)
  const uint32_t* W1 = NM == 2 ? p.mat[1].W : W0;
  const uint8_t* A81 = NM == 2 ? p.mat[1].A8 : A80;
  const float* AM1 = NM == 2 ? p.mat[1].AMAX : AM0;
  const float* C21 = NM == 2 ? p.mat[1].CODE2 : C20;
  uint4* xs = reinterpret_cast<uint4*>(srow + NW * NM * RPW * 8 * J);  // [KD]

  // 1. small operands first. The table entries this lane writes are
  //    e_i = 4 * (wave + NW * i) + (lane >> 4): low half code[e_i >> 4] =
  //    code[NW / 4 * i + wave / 4] (wave-uniform, read from lane e_i >> 4 of
  //    a load of the 16 codes), high half code[e_i & 15] = code[4 * (wave % 4)
  //    + lane / 16].
  const float cl16 = LUT[lane & 15];
  const float clo = LUT[4 * (wave & 3) + (lane >> 4)];
  u32x4 c2q[NM];  // code2 entries 4 * lane .. 4 * lane + 3 (every wave writes the whole table)
#pragma unroll
  for (int m = 0; m < NM; ++m) c2q[m] = *reinterpret_cast<const u32x4*>((m ? C21 : C20) + (nested ? 4 * lane : 0));
  // Scales, per wave and read by that wave only (no barrier): slot
  // (m, r, 8 j + g) holds the scale of block g of the wave's chunk j in row r
  // of weight m (8 slots per chunk; with bs > 64 the chunk has 64 / (bs / 8)
  // blocks and the other slots go unread), so a lane's scale sits at a fixed
  // offset per row and chunk. Lane l loads slots l + 64 i.
  constexpr int SW = NM * RPW * 8 * J;  // slots per wave
  const int spc = sh <= 6 ? 64 >> sh : 1;  // blocks per 64-dword chunk
  float sv[SL];
  uint32_t av[SL];
#pragma unroll
  for (int i = 0; i < SL; ++i) {
    const int sl = min(lane + 64 * i, SW - 1);
    const int mr = sl / (8 * J), jg = sl % (8 * J);
    const int m = mr / RPW, r = mr % RPW, j = jg >> 3, g = min(jg & 7, spc - 1);
    const int d = min(64 * (j * KS + ks) + (g << sh), KD - 1);
    const uint32_t gb = (uint32_t)min(row0 + r, M - 1) * (uint32_t)nblk + (uint32_t)(d >> sh);
    av[i] = (m ? A81 : A80)[gb];
    sv[i] = (m ? AM1 : AM0)[nested ? gb >> bs2_shift : gb];
  }
  // x (and the norm weight): staged once per workgroup, chunk c = tid + 512 i
  // of each activation row by thread tid (one chunk per thread unless
  // K > 4096, where there is no norm); rows past N repeat row N - 1 (the rows
  // form: NR > 1, a norm of each row if any)
  const int XN = uniform((KD + nthr - 1) / nthr);
  uint4 xc[XC_MAX][NR];
  // (chunks past XN stay unset and unread: a zero-initialised chunk would make
  // the branch's join wait for the load)
  if constexpr (!ATT) {
#pragma unroll
    for (int n = 0; n < NR; ++n) {
      // (row 0 needs no argument beyond the preloaded ones: its loads issue at wave start)
      const uint16_t* xrow = n == 0 ? X : X + (size_t)min(n, p.N - 1) * K;
      xc[0][n] = *reinterpret_cast<const uint4*>(xrow + 8 * (size_t)min(tid, KD - 1));
#pragma unroll
      for (int i = 1; i < XC_MAX; ++i)
        if (i < XN) xc[i][n] = *reinterpret_cast<const uint4*>(xrow + 8 * (size_t)min(tid + i * nthr, KD - 1));
    }
  }

  // 2. the first PF rows of the weight stream; the rest is requested row by
  //    row during the dot products, PF rows ahead, so no wave's barrier
  //    waits for its whole stream to be accepted by the memory system
  uint32_t w[NM][RPW][J];
  uint32_t woff[J];  // byte offset of the lane's dword j in the wave's K-slice (clamped inside the row)
#pragma unroll
  for (int j = 0; j < J; ++j) woff[j] = 4u * (uint32_t)min(64 * j * KS + lane, KD - 1 - 64 * ks);
  auto load_row = [&](int r) {
#pragma unroll
    for (int m = 0; m < NM; ++m) {
      const char* wr = reinterpret_cast<const char*>((m ? W1 : W0) + (size_t)uniform(min(row0 + r, M - 1)) * KD + 64 * ks);
#pragma unroll
      for (int j = 0; j < J; ++j)
        w[m][r][j] = __builtin_nontemporal_load(reinterpret_cast<const uint32_t*>(wr + woff[j]));
    }
  };
#pragma unroll
  for (int r = 0; r < PF; ++r) load_row(r);
  // the remaining arguments, in one round trip while those loads fly
  asm volatile("" ::"s"(p.G), "s"(p.R), "s"(p.Y), "s"(p.mat[0].offset), "s"(p.mat[NM - 1].offset), "s"(p.eps));
  uint32_t rres[NR];  // epilogue operands
#pragma unroll
  for (int n = 0; n < NR; ++n)
    rres[n] = p.R[(n == 0 ? 0 : (size_t)min(n, p.N - 1) * M) + min(row0 + min(lane, RPW - 1), M - 1)];
  const uint4 gc = *reinterpret_cast<const uint4*>(p.G + 8 * (size_t)(norm ? min(tid, KD - 1) : 0));

  // 2b. (attention prologue) every load of the attention, before any waits:
  //     wave w takes query head min(w, nh - 1) (waves past nh duplicate the
  //     last head's loads and compute nothing), its kv head's new K/V row and
  //     norm weights, and the workgroup stages all nkv * max_len cached rows
  //     (row pos, stale, is replaced by the computed row).
  const AttnSrc& at = p.att;
  const int a_nh = (int)(at.hcfg & 255u), a_nkv = (int)((at.hcfg >> 8) & 255u);
  const int a_groups = (int)((at.hcfg >> 16) & 255u), a_ftype = (int)((at.hcfg >> 24) & 15u);
  const bool a_qn = (at.hcfg >> 28) & 1u, a_kn = (at.hcfg >> 29) & 1u;
  const int a_R = att_r16(at.max_len);
  const int a_head = min(wave, a_nh - 1), a_kvh = a_head / a_groups;
  uint16_t aq0 = 0, aq1 = 0, aqw0 = 0, aqw1 = 0, ak0 = 0, ak1 = 0, av0 = 0, av1 = 0, akw0 = 0, akw1 = 0;
  RopeF arf{};
  u32x4 akq[ATT_PER], avq[ATT_PER];
  long long apos0 = 0;
  if constexpr (ATT) {
    apos0 = at.POS[0];
    const uint16_t* qr = at.QKV + (size_t)a_head * HD;
    const uint16_t* kr = at.QKV + (size_t)(a_nh + a_kvh) * HD;
    const uint16_t* vr = at.QKV + (size_t)(a_nh + a_nkv + a_kvh) * HD;
    aq0 = qr[lane];
    aq1 = qr[lane + 64];
    aqw0 = at.QW[lane];
    aqw1 = at.QW[lane + 64];
    arf = load_rope(at.F, a_ftype, lane);
    ak0 = kr[lane];
    ak1 = kr[lane + 64];
    av0 = vr[lane];
    av1 = vr[lane + 64];
    akw0 = at.KW[lane];
    akw1 = at.KW[lane + 64];
    const int npc = a_nkv * at.max_len * (HD / 8);  // pieces to stage
#pragma unroll
    for (int i = 0; i < ATT_PER; ++i) {
      const int t = min(tid + i * nthr, npc - 1);
      const int kvh = t / (at.max_len * (HD / 8)), j = (t / (HD / 8)) % at.max_len, e = (t % (HD / 8)) * 8;
      const size_t off = ((size_t)kvh * at.max_len + j) * HD + e;
      akq[i] = *reinterpret_cast<const u32x4*>(at.KC + off);
      avq[i] = *reinterpret_cast<const u32x4*>(at.VC + off);
    }
  }

  // 3. set-up while those stream: the replicated code table, code2 (each wave
  //    its own full copy: identical values, so no barrier), the resolved
  //    scales, x staged (or, with a norm, each wave's sum of squares)
  {
    const uint32_t hi = (uint32_t)f32_to_f16(clo) << 16;
    const uint32_t c16 = f32_to_f16(cl16);
#pragma unroll
    for (int i = 0; i < G; ++i) {
      const uint32_t v = (uint32_t)__builtin_amdgcn_readlane((int)c16, NW / 4 * i + (wave >> 2)) | hi;
      reinterpret_cast<uint4*>(lut_rep)[(wave + NW * i) * 64 + lane] = make_uint4(v, v, v, v);
    }
  }
#pragma unroll
  for (int m = 0; m < NM; ++m) reinterpret_cast<u32x4*>(code2_s + m * 256)[lane] = c2q[m];
#pragma unroll
  for (int i = 0; i < SL; ++i) {
    const int sl = lane + 64 * i;
    const int m = sl / (8 * J * RPW);
    const float off = m ? p.mat[NM - 1].offset : p.mat[0].offset;
    if (sl < SW) srow[wave * SW + sl] = nested ? __fadd_rn(__fmul_rn(code2_s[m * 256 + av[i]], sv[i]), off) : sv[i];
  }
  if constexpr (ATT) {
    // 3b. the attention (attn_qkv_kernel's arithmetic, one chunk), its
    //     output rounded into x
    float* q_s = reinterpret_cast<float*>(xs + KD);                         // [8][128]
    float* p_s = q_s + ATT_MAX_HEADS * HD;                                  // [8][64]
    uint16_t* k_s = reinterpret_cast<uint16_t*>(p_s + ATT_MAX_HEADS * ACHUNK);  // [nkv][R16][KPAD]
    uint16_t* v_s = k_s + (size_t)a_nkv * a_R * KPAD;                       // [nkv][R16][HD]
    const long long pos = apos0;
    const bool pos_ok = pos >= 0 && pos < at.max_len;
    const int jpos = pos_ok ? (int)pos : 0, nvalid = jpos + 1;
    const bool qwave = wave < a_nh, newrow = qwave && wave % a_groups == 0;
    uint16_t klo = 0, khi = 0;
    if (qwave) {
      float lo = ld16(dt, aq0), hi = ld16(dt, aq1);
      if (dt == DT_BF16) head_norm_rope<DT_BF16>(lo, hi, a_qn, aqw0, aqw1, at.eps, arf, lane);
      else head_norm_rope<DT_F16>(lo, hi, a_qn, aqw0, aqw1, at.eps, arf, lane);
      q_s[wave * HD + lane] = __fmul_rn(ld16(dt, st16(dt, lo)), at.scale);
      q_s[wave * HD + lane + 64] = __fmul_rn(ld16(dt, st16(dt, hi)), at.scale);
    }
    if (newrow) {
      float lo = ld16(dt, ak0), hi = ld16(dt, ak1);
      if (dt == DT_BF16) head_norm_rope<DT_BF16>(lo, hi, a_kn, akw0, akw1, at.eps, arf, lane);
      else head_norm_rope<DT_F16>(lo, hi, a_kn, akw0, akw1, at.eps, arf, lane);
      klo = (uint16_t)st16(dt, lo);
      khi = (uint16_t)st16(dt, hi);
      uint16_t* kd = k_s + ((size_t)a_kvh * a_R + jpos) * KPAD;
      uint16_t* vd = v_s + ((size_t)a_kvh * a_R + jpos) * HD;
      kd[lane] = klo;
      kd[lane + 64] = khi;
      vd[lane] = av0;
      vd[lane + 64] = av1;
    }
    const int npc = a_nkv * at.max_len * (HD / 8);
#pragma unroll
    for (int i = 0; i < ATT_PER; ++i) {
      const int t = tid + i * nthr;
      const int kvh = t / (at.max_len * (HD / 8)), j = (t / (HD / 8)) % at.max_len, e = (t % (HD / 8)) * 8;
      if (t < npc && j != jpos) {
        *reinterpret_cast<u32x4*>(k_s + ((size_t)kvh * a_R + j) * KPAD + e) = akq[i];
        *reinterpret_cast<u32x4*>(v_s + ((size_t)kvh * a_R + j) * HD + e) = avq[i];
      }
    }
    __syncthreads();
    if (qwave) {
      const uint16_t* kr = k_s + ((size_t)a_kvh * a_R + min(lane, at.max_len - 1)) * KPAD;
      const float sc = dt == DT_BF16 ? score4<DT_BF16>(q_s + wave * HD, kr) : score4<DT_F16>(q_s + wave * HD, kr);
      const bool valid = lane < nvalid;
      const float m = wave_max_u(valid ? sc : -3.0e38f);
      const float pr = valid ? exp_cw(__fsub_rn(sc, m)) : 0.0f;
      const float l = wave_sum_dpp(pr);
      p_s[wave * ACHUNK + lane] = pr;  // read back by this wave only
      float a0, a1;
      const uint16_t* vs = v_s + (size_t)a_kvh * a_R * HD;
      if (dt == DT_BF16) pv4<DT_BF16>(p_s + wave * ACHUNK, vs, nvalid, lane, a0, a1);
      else pv4<DT_F16>(p_s + wave * ACHUNK, vs, nvalid, lane, a0, a1);
      // the merge of a single chunk, as attn_combine_kernel computes it
      const float wt = exp_cw(__fsub_rn(m, m));
      const float den = __fadd_rn(0.0f, __fmul_rn(l, wt));
      const float y0 = __fdiv_rn(__fadd_rn(0.0f, __fmul_rn(a0, wt)), den);
      const float y1 = __fdiv_rn(__fadd_rn(0.0f, __fmul_rn(a1, wt)), den);
      reinterpret_cast<uint32_t*>(xs)[wave * 64 + lane] = st16(dt, y0) | (st16(dt, y1) << 16);
    }
    // the new row into the cache, once (workgroup 0)
    if (newrow && pos_ok && blockIdx.x == 0) {
      const size_t row = ((size_t)a_kvh * at.max_len + pos) * HD;
      at.KC[row + lane] = klo;
      at.KC[row + lane + 64] = khi;
      at.VC[row + lane] = av0;
      at.VC[row + lane + 64] = av1;
    }
  } else if (!norm) {
#pragma unroll
    for (int n = 0; n < NR; ++n) {
#pragma unroll
      for (int i = 0; i < XC_MAX; ++i) {
        const int c = tid + i * nthr;
        if (i < XN && c < KD) xs[n * KD + c] = xc[i][n];
      }
      // rows longer than XC_MAX chunks a thread (K > 12288): the rest of x is
      // loaded here, after the weight rows were requested, so this wait also
      // waits for them - only those long rows pay it
      for (int i = XC_MAX; i < XN; ++i) {
        const int c = tid + i * nthr;
        if (c < KD)
          xs[n * KD + c] = *reinterpret_cast<const uint4*>(X + (n == 0 ? 0 : (size_t)min(n, p.N - 1) * K) + 8 * (size_t)c);
      }
    }
  } else {  // each activation row's sum of squares, wave w taking its chunks 64 w .. 64 w + 63
#pragma unroll
    for (int n = 0; n < NR; ++n) {
      float sq = 0.0f;
      if (tid < KD) sq = dt == DT_BF16 ? sumsq8<DT_BF16>(xc[0][n], 0.0f) : sumsq8<DT_F16>(xc[0][n], 0.0f);
      sq = wave_sum_dpp(sq);
      if (lane == 0) wpart[n * NW + wave] = sq;
    }
  }
  __syncthreads();
  if (norm) {  // per row: the 64-chunk partial sums left to right, then each thread's chunk
#pragma unroll
    for (int n = 0; n < NR; ++n) {
      float ss = wpart[n * NW];
#pragma unroll
      for (int w2 = 1; w2 < NW; ++w2) ss = __fadd_rn(ss, wpart[n * NW + w2]);
      const float r = rsqrt_rn(__fadd_rn(__fdiv_rn(ss, (float)K), p.eps));
      if (tid < KD)
        xs[n * KD + tid] = dt == DT_BF16 ? norm8<DT_BF16>(xc[0][n], gc, r) : norm8<DT_F16>(xc[0][n], gc, r);
    }
    __syncthreads();
  }

  // x as fp32 (zero past the row's end: the clamped weight dword there is
  // finite, so its products are exactly +0)
  F8 xf[NR][J];
#pragma unroll
  for (int n = 0; n < NR; ++n) {
    uint4 xz[J];
#pragma unroll
    for (int j = 0; j < J; ++j) {
      const int d = lane + 64 * (j * KS + ks);
      const uint4 v = xs[n * KD + min(d, KD - 1)];
      xz[j] = d < KD ? v : make_uint4(0, 0, 0, 0);
    }
    if (dt == DT_BF16) {
#pragma unroll
      for (int j = 0; j < J; ++j) xf[n][j] = to_f32<DT_BF16>(xz[j]);
    } else {
#pragma unroll
      for (int j = 0; j < J; ++j) xf[n][j] = to_f32<DT_F16>(xz[j]);
    }
  }

  // 4. dot products, row by row as the rows arrive: a dword's 8 products in
  //    code order, each an fma (the first onto +0), then its block scale
  const uint32_t lane4 = (uint32_t)lane * 4u;
  const unsigned char* lut_b = reinterpret_cast<const unsigned char*>(lut_rep);
  const unsigned char* srow_b = reinterpret_cast<const unsigned char*>(srow);
  int sblk4[J];  // byte offset of each of the lane's chunks' scale slot in row 0 of weight 0
#pragma unroll
  for (int j = 0; j < J; ++j) sblk4[j] = 4 * (wave * SW + 8 * j + (lane >> sh));
  // The (row, chunk) items in order, the code lookups LA items ahead of the
  // arithmetic (sched_barrier keeps the compiler from pulling them back), the
  // next weight row requested at each row's start. A lookup may only reach
  // rows already requested: row r + PF is requested when row r starts, so the
  // lookahead stays within PF rows of items (with one chunk per lane and three
  // or more rows a wave, three items ahead would read a row before its load).
  constexpr int T = NM * RPW * J;
  constexpr int LA0 = GEMV_LOOKAHEAD < T ? GEMV_LOOKAHEAD : T;
  constexpr int LA = LA0 < PF * J ? LA0 : PF * J;
  float sc[T];
  uint32_t cp[T][4];
  auto lookup = [&](int t) {
    const int j = t % J, mr = t / J, m = mr / RPW, r = mr % RPW;
    sc[t] = *reinterpret_cast<const float*>(srow_b + sblk4[j] + 4 * 8 * J * (m * RPW + r));
#pragma unroll
    for (int b = 0; b < 4; ++b)
      cp[t][b] = *reinterpret_cast<const uint32_t*>(lut_b + __builtin_amdgcn_perm(w[m][r][j], lane4, 0x0C0C0400u + (b << 8)));
  };
#pragma unroll
  for (int t = 0; t < LA; ++t) lookup(t);
  // outputs per weight row: NM weights (SwiGLU) or NR activation rows
  constexpr int NO = NM * NR;
  float tot[NO][RPW];
#pragma unroll
  for (int m = 0; m < NM; ++m)
#pragma unroll
    for (int r = 0; r < RPW; ++r) {
      if (m == 0 && r + PF < RPW) load_row(r + PF);
      float acc[NR];
#pragma unroll
      for (int n = 0; n < NR; ++n) acc[n] = 0.0f;
#pragma unroll
      for (int j = 0; j < J; ++j) {
        const int t = (m * RPW + r) * J + j;
        if (t + LA < T) lookup(t + LA);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int n = 0; n < NR; ++n) {  // each activation row: the one-row chain
          float q = __builtin_fmaf(h_lo(cp[t][0]), xf[n][j].v[0], 0.0f);
          q = __builtin_fmaf(h_hi(cp[t][0]), xf[n][j].v[1], q);
          q = __builtin_fmaf(h_lo(cp[t][1]), xf[n][j].v[2], q);
          q = __builtin_fmaf(h_hi(cp[t][1]), xf[n][j].v[3], q);
          q = __builtin_fmaf(h_lo(cp[t][2]), xf[n][j].v[4], q);
          q = __builtin_fmaf(h_hi(cp[t][2]), xf[n][j].v[5], q);
          q = __builtin_fmaf(h_lo(cp[t][3]), xf[n][j].v[6], q);
          q = __builtin_fmaf(h_hi(cp[t][3]), xf[n][j].v[7], q);
          acc[n] = __builtin_fmaf(q, sc[t], acc[n]);
        }
      }
#pragma unroll
      for (int n = 0; n < NR; ++n) tot[m * NR + n][r] = wave_sum_dpp(acc[n]);
    }

  // 5. K-slices left to right, epilogue, store (lane r stores row r)
  if (KS > 1) {
    if (lane == 0) {
#pragma unroll
      for (int o = 0; o < NO; ++o)
#pragma unroll
        for (int r = 0; r < RPW; ++r) red[wave * NO * RPW + o * RPW + r] = tot[o][r];
    }
    __syncthreads();
    if (ks != 0) return;
#pragma unroll
    for (int o = 0; o < NO; ++o)
#pragma unroll
      for (int r = 0; r < RPW; ++r) {
        float a = tot[o][r];
        for (int k2 = 1; k2 < KS; ++k2) a = __fadd_rn(a, red[(wave + k2) * NO * RPW + o * RPW + r]);
        tot[o][r] = a;
      }
  }
  float mine[NO];
#pragma unroll
  for (int o = 0; o < NO; ++o) {
    mine[o] = tot[o][0];
#pragma unroll
    for (int r = 1; r < RPW; ++r) mine[o] = lane == r ? tot[o][r] : mine[o];
  }
  if (lane < RPW && row0 + lane < M) {
    if constexpr (NM == 1) {
#pragma unroll
      for (int n = 0; n < NR; ++n)
        if (n < p.N) p.Y[(size_t)n * M + row0 + lane] = epilogue16(dt, mine[n], p.epi, rres[n]);
    } else {
      // SwiGLU: w1's row is the gate operand of w3's row, as the two-launch form rounds it
#pragma unroll
      for (int n = 0; n < NR; ++n)
        if (n < p.N) p.Y[(size_t)n * M + row0 + lane] = epilogue16(dt, mine[NR + n], 2, st16(dt, mine[n]));
    }
  }
}

// ---------------------------------------------------------------------------
// host side

// Launch shape: J 64-dword chunks per lane, K split over KS waves, RPW rows
// per wave (8 waves per workgroup).
struct GemvShape {
  int J, KS, RPW;
};

static constexpr int kJ[] = {1, 2, 3, 4, 5, 6, 8};
static constexpr int kRPW1[] = {1, 2, 3, 4, 5, 6, 8};
static constexpr int kRPW2[] = {1, 2, 3, 4, 5};
#ifndef GEMV_WG_SLOTS
#define GEMV_WG_SLOTS 256
#endif
static constexpr int kCUs = GEMV_WG_SLOTS;  // workgroups resident at once
static constexpr size_t kLdsPerCU = 160 * 1024;  // a workgroup's LDS must fit

// Dynamic LDS of one workgroup (the table is static); nr activation rows.
static size_t gemv_dyn_lds(const GemvShape& g, int nm, int K, int bs_shift, int nr = 1) {
  const size_t sc = (size_t)GEMV_WAVES * nm * g.RPW * 8 * g.J;  // scale slots
  return 4 * (256 * (size_t)nm + (size_t)GEMV_WAVES * nr + (size_t)GEMV_WAVES * nm * nr * g.RPW + sc) +
         2 * (size_t)K * nr;
}

// K is split (KS a power of two) so that a lane's chunks J <= 8 leave the
// fewest slots idle; RPW is the smallest that fits every row into one
// workgroup per CU (every workgroup builds the 64 KiB table and stages x once,
// so fewer, fuller workgroups pay less of that - measured faster than two
// half-full workgroups per CU at every decode shape).
// The rows form (nr > 1 activation rows) holds x as fp32 for its J chunks of
// every row through the dot loop: J * nr <= 20 keeps that within 160 VGPRs.
// Two rows: every J fits, so the K split is the one-row launch's and each
// row's result equals a one-row launch bit for bit. (Four rows a launch were
// built and measured: faster than the few-row MFMA kernel only on the
// smallest matrices, 10-35 % slower on the large ones.)
static constexpr int kRowsXMax = 20;
constexpr int GEMV_MAX_ROWS = 2;

static GemvShape gemv_shape(int M, int K, int nm = 1, int bs_shift = 6, int nr = 1) {
  const int chunks = (K / 8 + 63) / 64;  // 64-dword chunks per row
  int KS = 0, J = 0, waste = 1 << 30;
  for (int ks = 1; ks <= GEMV_WAVES; ks *= 2) {
    int j = 0;
    for (int v : kJ)
      if (v >= (chunks + ks - 1) / ks) { j = v; break; }
    if (j && (nr == 1 || j * nr <= kRowsXMax) && ks * j - chunks < waste) { KS = ks; J = j; waste = ks * j - chunks; }
  }
  if (!KS) return {0, 0, 0};
  const int RG = GEMV_WAVES / KS;
  GemvShape g{J, KS, 1};
  const int* rpw = nm == 1 ? kRPW1 : kRPW2;
  const int nrpw = nm == 1 ? (int)(sizeof(kRPW1) / sizeof(int)) : (int)(sizeof(kRPW2) / sizeof(int));
  for (int i = 0; i < nrpw; ++i) {
    g.RPW = rpw[i];
    if ((long long)(M + RG * g.RPW - 1) / (RG * g.RPW) <= kCUs) break;
  }
  return g;
}

template <int J, int RPW, int NM, bool ATT = false, int NR = 1>
static void launch_gemv(const GemvShape& g, const GemvParams& p, hipStream_t st, size_t extra_lds = 0) {
  const int rows_wg = (GEMV_WAVES / g.KS) * RPW;
  const int grid = (p.M + rows_wg - 1) / rows_wg;
  const uint32_t mk = (uint32_t)p.M | ((uint32_t)(p.K / 128) << 20);
  const uint32_t cfg = (uint32_t)g.KS | ((uint32_t)p.bs_shift << 4) | ((uint32_t)p.bs2_shift << 8) |
                       ((uint32_t)p.dt << 12) | ((uint32_t)p.nested << 14) | ((uint32_t)p.norm << 15);
  hipLaunchKernelGGL((nf4_gemv_kernel<J, RPW, NM, ATT, NR>), dim3(grid), dim3(GEMV_THREADS),
                     gemv_dyn_lds(g, NM, p.K, p.bs_shift, NR) + extra_lds, st, p.mat[0].W, p.X, p.LUT,
                     p.mat[0].A8, p.mat[0].AMAX, p.mat[0].CODE2, mk, cfg, p);
}

template <int J, int NM, int NR = 1>
static int dispatch_rpw(const GemvShape& g, const GemvParams& p, hipStream_t st) {
#define TTSP_R(RV) \
  case RV: launch_gemv<J, RV, NM, false, NR>(g, p, st); return 0;
  if constexpr (NM == 1) {
    switch (g.RPW) {
      TTSP_R(1) TTSP_R(2) TTSP_R(3) TTSP_R(4) TTSP_R(5) TTSP_R(6) TTSP_R(8)
      default: return (int)hipErrorInvalidValue;
    }
  } else {
    switch (g.RPW) {
      TTSP_R(1) TTSP_R(2) TTSP_R(3) TTSP_R(4) TTSP_R(5)
      default: return (int)hipErrorInvalidValue;
    }
  }
#undef TTSP_R
}

template <int NM, int NR = 1>
static int dispatch_j(const GemvShape& g, const GemvParams& p, hipStream_t st) {
#define TTSP_J(JV)                                                            \
  case JV:                                                                    \
    if constexpr (NR == 1 || JV * NR <= kRowsXMax) return dispatch_rpw<JV, NM, NR>(g, p, st); \
    else return (int)hipErrorInvalidValue;
  switch (g.J) {
    TTSP_J(1) TTSP_J(2) TTSP_J(3) TTSP_J(4) TTSP_J(5) TTSP_J(6) TTSP_J(8)
    default: return (int)hipErrorInvalidValue;
  }
#undef TTSP_J
}

// The attention-prologue form: one weight, K = nh * 128 <= 1024, so KS = 1,
// J <= 2 and any RPW the row count needs up to 4 (beyond that: declined).
static int dispatch_att(const GemvShape& g, const GemvParams& p, hipStream_t st, size_t extra) {
  if (g.KS != 1) return (int)hipErrorInvalidValue;
#define TTSP_A(JV, RV) \
  if (g.J == JV && g.RPW == RV) { launch_gemv<JV, RV, 1, true>(g, p, st, extra); return 0; }
  TTSP_A(1, 1) TTSP_A(1, 2) TTSP_A(1, 3) TTSP_A(1, 4)
  TTSP_A(2, 1) TTSP_A(2, 2) TTSP_A(2, 3) TTSP_A(2, 4)
#undef TTSP_A
  return (int)hipErrorInvalidValue;
}

static int log2_exact(int v) {
  if (v <= 0 || (v & (v - 1))) return -1;
  int s = 0;
  while ((1 << s) < v) ++s;
  return s;
}

// Validates, fills GemvParams and launches. mat3 == nullptr: one weight with
// epilogue `epi`; otherwise the SwiGLU pair (epi must be 0). G != nullptr
// folds the RMSNorm prologue in.
static int gemv_launch(const void* X, int dt, const void* G, float eps, const Nf4Mat& mat1,
                       const Nf4Mat* mat3, bool nested, const float* LUT, void* Y, const void* R,
                       int epi, int M, int K, int blocksize, int blocksize2, hipStream_t st,
                       const AttnSrc* att = nullptr, int N = 1) {
  const int bs_shift = log2_exact(blocksize);
  const int bs2_shift = nested ? log2_exact(blocksize2) : 0;
  if (bs_shift < 6 || bs_shift > 15 || bs2_shift < 0 || bs2_shift > 15 || K % 128 || K % blocksize || M <= 0 ||
      M >= (1 << 20) || K / 128 >= (1 << 12))
    return (int)hipErrorInvalidValue;  // the sizes travel packed: M < 2^20, K / 128 < 2^12
  if (dt != DT_F16 && dt != DT_BF16) return (int)hipErrorInvalidValue;
  if (epi < 0 || epi > 2 || (epi && !R) || (mat3 && epi)) return (int)hipErrorInvalidValue;
  const int nm = mat3 ? 2 : 1;
  if (N < 1 || N > GEMV_MAX_ROWS || (N > 1 && att)) return (int)hipErrorInvalidValue;
  const int nr = N;
  const GemvShape g = gemv_shape(M, K, nm, bs_shift, nr);
  if (!g.J) return (int)hipErrorInvalidValue;
  if (G && K / 8 > GEMV_THREADS) return (int)hipErrorInvalidValue;  // the norm: one chunk per thread
  const size_t att_bytes = att ? att_lds((int)((att->hcfg >> 8) & 255u), att->max_len) : 0;
  if (LUT_BYTES + gemv_dyn_lds(g, nm, K, bs_shift, nr) + att_bytes > kLdsPerCU) return (int)hipErrorInvalidValue;
  if (att && (G || mat3)) return (int)hipErrorInvalidValue;
  if (nested && ((uintptr_t)mat1.CODE2 % 16 || (mat3 && (uintptr_t)mat3->CODE2 % 16)))
    return (int)hipErrorInvalidValue;  // code2 is read 16 bytes per lane
  GemvParams p;
  p.mat[0] = mat1;
  p.mat[1] = mat3 ? *mat3 : mat1;
  for (Nf4Mat& m : p.mat) {
    if (!nested) {  // unused operands point at readable memory
      m.A8 = reinterpret_cast<const uint8_t*>(m.AMAX);
      m.CODE2 = LUT;  // 16 bytes of it are read
      m.offset = 0.0f;
    }
  }
  p.LUT = LUT;
  p.X = (const uint16_t*)X;
  p.G = G ? (const uint16_t*)G : (const uint16_t*)X;
  p.Y = (uint16_t*)Y;
  p.R = epi ? (const uint16_t*)R : (const uint16_t*)Y;  // read unconditionally, used by the epilogue only
  p.eps = eps;
  p.M = M;
  p.K = K;
  p.N = N;
  p.KS = g.KS;
  p.bs_shift = bs_shift;
  p.bs2_shift = bs2_shift;
  p.dt = dt;
  p.nested = nested ? 1 : 0;
  p.norm = G ? 1 : 0;
  p.epi = epi;
  p.att = att ? *att : AttnSrc{};
  const int rc = att     ? dispatch_att(g, p, st, att_bytes)
                 : nm == 2 ? (nr == 1 ? dispatch_j<2>(g, p, st) : dispatch_j<2, 2>(g, p, st))
                 : nr == 1 ? dispatch_j<1>(g, p, st)
                           : dispatch_j<1, 2>(g, p, st);
  if (rc) return rc;
  TTSP_RETURN_LAUNCH();
}

// Whether the GEMV takes a one-weight launch of this shape for N activation
// rows (no norm): rows of at most 64 chunks a lane-set (K <= 32768; fewer
// with several activation rows) whose LDS fits a CU. Larger rows go to the
// tiled kernel.
bool gemv_fits(int M, int K, int blocksize, int N) {
  const int bs_shift = log2_exact(blocksize);
  if (bs_shift < 6 || bs_shift > 15 || M <= 0 || K <= 0 || K % 128 || K % blocksize || M >= (1 << 20)) return false;
  if (N < 1 || N > GEMV_MAX_ROWS) return false;
  const GemvShape g = gemv_shape(M, K, 1, bs_shift, N);
  return g.J && LUT_BYTES + gemv_dyn_lds(g, 1, K, bs_shift, N) <= kLdsPerCU;
}

// N (1..GEMV_MAX_ROWS) activation rows through the GEMV: every weight byte's
// codes are looked up once, and each row gets the one-row arithmetic (its
// result equals a one-row launch, bit for bit).
int gemv_rows(const void* X, int dt, const uint8_t* W, const uint8_t* A8, const float* AMAX,
              const float* CODE2, float offset, const float* LUT, void* Y, const void* R, int epi,
              int M, int K, int N, int blocksize, int blocksize2, hipStream_t st) {
  const Nf4Mat m{reinterpret_cast<const uint32_t*>(W), A8, AMAX, CODE2, offset};
  return gemv_launch(X, dt, nullptr, 0.0f, m, nullptr, A8 != nullptr, LUT, Y, R, epi, M, K, blocksize,
                     blocksize2, st, nullptr, N);
}

}  // namespace ttsp

using namespace ttsp;

extern "C" int ttsp_gemv_shape(int M, int K, int* J, int* KS, int* RPW) {
  const GemvShape g = gemv_shape(M, K);
  if (J) *J = g.J;
  if (KS) *KS = g.KS;
  if (RPW) *RPW = g.RPW;
  return g.J ? 0 : (int)hipErrorInvalidValue;
}

extern "C" int ttsp_gemv_rows_shape(int M, int K, int N, int* J, int* KS, int* RPW) {
  const bool ok = gemv_fits(M, K, 64, N);
  const GemvShape g = ok ? gemv_shape(M, K, 1, 6, N) : GemvShape{0, 0, 0};
  if (J) *J = g.J;
  if (KS) *KS = g.KS;
  if (RPW) *RPW = g.RPW;
  return ok ? 0 : (int)hipErrorInvalidValue;
}

extern "C" int ttsp_nf4_gemv_fused(const void* X, int x_dtype, const void* NORM_W, float eps,
                                   const uint8_t* W1, const uint8_t* A8_1, const float* AMAX_1,
                                   const float* CODE2_1, float offset_1, const uint8_t* W3,
                                   const uint8_t* A8_3, const float* AMAX_3, const float* CODE2_3,
                                   float offset_3, const float* LUT, void* Y, const void* R, int epi,
                                   int M, int K, int blocksize, int blocksize2, hipStream_t stream) {
  if (!X || !W1 || !AMAX_1 || !LUT || !Y || M <= 0 || K <= 0) return (int)hipErrorInvalidValue;
  const bool nested = A8_1 != nullptr;
  if (nested && !CODE2_1) return (int)hipErrorInvalidValue;
  const Nf4Mat m1{reinterpret_cast<const uint32_t*>(W1), A8_1, AMAX_1, CODE2_1, offset_1};
  if (!W3) return gemv_launch(X, x_dtype, NORM_W, eps, m1, nullptr, nested, LUT, Y, R, epi, M, K, blocksize,
                              blocksize2, stream);
  if (!AMAX_3 || (A8_3 != nullptr) != nested || (nested && !CODE2_3)) return (int)hipErrorInvalidValue;
  const Nf4Mat m3{reinterpret_cast<const uint32_t*>(W3), A8_3, AMAX_3, CODE2_3, offset_3};
  return gemv_launch(X, x_dtype, NORM_W, eps, m1, &m3, nested, LUT, Y, R, epi, M, K, blocksize, blocksize2,
                     stream);
}

extern "C" int ttsp_nf4_gemv_fused_rows(const void* X, int x_dtype, const void* NORM_W, float eps,
                                        const uint8_t* W1, const uint8_t* A8_1, const float* AMAX_1,
                                        const float* CODE2_1, float offset_1, const uint8_t* W3,
                                        const uint8_t* A8_3, const float* AMAX_3, const float* CODE2_3,
                                        float offset_3, const float* LUT, void* Y, const void* R, int epi, int M,
                                        int K, int N, int blocksize, int blocksize2, hipStream_t stream) {
  if (!X || !W1 || !AMAX_1 || !LUT || !Y || M <= 0 || K <= 0 || N < 1 || N > GEMV_MAX_ROWS)
    return (int)hipErrorInvalidValue;
  const bool nested = A8_1 != nullptr;
  if (nested && !CODE2_1) return (int)hipErrorInvalidValue;
  const Nf4Mat m1{reinterpret_cast<const uint32_t*>(W1), A8_1, AMAX_1, CODE2_1, offset_1};
  if (!W3)
    return gemv_launch(X, x_dtype, NORM_W, eps, m1, nullptr, nested, LUT, Y, R, epi, M, K, blocksize, blocksize2,
                       stream, nullptr, N);
  if (!AMAX_3 || (A8_3 != nullptr) != nested || (nested && !CODE2_3)) return (int)hipErrorInvalidValue;
  const Nf4Mat m3{reinterpret_cast<const uint32_t*>(W3), A8_3, AMAX_3, CODE2_3, offset_3};
  return gemv_launch(X, x_dtype, NORM_W, eps, m1, &m3, nested, LUT, Y, R, epi, M, K, blocksize, blocksize2, stream,
                     nullptr, N);
}

extern "C" int ttsp_attn_nf4_gemv(const void* QKV, const void* QW, const void* KW, float eps, const void* F,
                                  int ftype, const long long* POS, void* KC, void* VC, int nh, int nkv,
                                  int max_len, float scale, const uint8_t* W, const uint8_t* A8,
                                  const float* AMAX, const float* CODE2, float offset, const float* LUT,
                                  void* Y, const void* R, int epi, int M, int blocksize, int blocksize2,
                                  int dtype, hipStream_t stream) {
  if (!QKV || !F || !POS || !KC || !VC || !W || !AMAX || !LUT || !Y) return (int)hipErrorInvalidValue;
  if (nh <= 0 || nkv <= 0 || nh > ATT_MAX_HEADS || nh % nkv || ftype < 0 || ftype > 2) return (int)hipErrorInvalidValue;
  if (max_len <= 0 || max_len > ACHUNK || nkv * max_len * (HD / 8) > ATT_PER * GEMV_THREADS)
    return (int)hipErrorInvalidValue;
  const bool nested = A8 != nullptr;
  if (nested && !CODE2) return (int)hipErrorInvalidValue;
  AttnSrc a;
  a.QKV = (const uint16_t*)QKV;
  a.QW = QW ? (const uint16_t*)QW : (const uint16_t*)QKV;
  a.KW = KW ? (const uint16_t*)KW : (const uint16_t*)QKV;
  a.F = F;
  a.POS = POS;
  a.KC = (uint16_t*)KC;
  a.VC = (uint16_t*)VC;
  a.eps = eps;
  a.scale = scale;
  a.max_len = max_len;
  a.hcfg = (uint32_t)nh | ((uint32_t)nkv << 8) | ((uint32_t)(nh / nkv) << 16) | ((uint32_t)ftype << 24) |
           ((QW ? 1u : 0u) << 28) | ((KW ? 1u : 0u) << 29);
  const Nf4Mat m{reinterpret_cast<const uint32_t*>(W), A8, AMAX, CODE2, offset};
  return gemv_launch(QKV, dtype, nullptr, 0.0f, m, nullptr, nested, LUT, Y, R, epi, M, nh * HD, blocksize,
                     blocksize2, stream, &a);
}
