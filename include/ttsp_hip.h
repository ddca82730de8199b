/*
 * C-ABI of libttsp_hip.so - the MI355X (gfx950) NF4 decode hot path.
 *
 * Every entry point takes raw device pointers, sizes and a hipStream_t
 * (passed as void*), launches on that stream, returns a hipError_t (0 on
 * success, hipErrorInvalidValue = 1 for arguments it rejects) and allocates
 * nothing. Scratch memory is always caller-provided.
 *
 * Element types: TTSP_F16 = 0, TTSP_BF16 = 1, TTSP_F32 = 2 (16-bit types are
 * passed as raw bit patterns).
 *
 * NF4 layout (bitsandbytes): W is the row-major flattened [M, K] weight, two
 * codes per byte with the even flattened index in the high nibble; scale
 * block b covers flattened codes [b*bs, (b+1)*bs). Plain scales: fp32
 * AMAX[b]. Nested (double-quant) scales: A8 uint8 [M*K/bs], AMAX = fp32
 * absmax2 [ceil(M*K/bs / bs2)], CODE2 = fp32 [256], plus `offset`:
 * s_b = CODE2[A8[b]] * AMAX[b / bs2] + offset. LUT = the 16 fp32 NF4 codes.
 *
 * Citations are into the reference tree (bitNtech/ttspipe); the reference
 * reaches its CUDA kernels through NVRTC + cuLaunchKernel via ctypes
 * (app/engine/nvrtc.py:118-198), and these functions are what its ctypes
 * argument blocks would bind instead.
 */
#ifndef TTSP_HIP_H
#define TTSP_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { TTSP_F16 = 0, TTSP_BF16 = 1, TTSP_F32 = 2 };
enum { TTSP_EPI_NONE = 0, TTSP_EPI_RESIDUAL = 1, TTSP_EPI_SILU_GATE = 2 };

/* One NF4 weight as ttsp_nf4_gemm takes it (A8 == NULL: plain scales). */
typedef struct ttsp_nf4_weight {
  const uint8_t* W;
  const uint8_t* A8;
  const float* AMAX;
  const float* CODE2;
  float offset;
} ttsp_nf4_weight;

/* One fast-transformer layer for ttsp_fast_steps: its weights, RMSNorm
 * weights (q_norm / k_norm NULL without head norms) and KV cache
 * [n_kv][max_len][128]. */
typedef struct ttsp_fast_layer {
  ttsp_nf4_weight wqkv, wo, w1, w3, w2;
  const void* attention_norm;
  const void* ffn_norm;
  const void* q_norm;
  const void* k_norm;
  void* k_cache;
  void* v_cache;
} ttsp_fast_layer;

/* ttsp_fast_steps' barrier words: TTSP_FAST_SYNC_WORDS uint32, zero before the
 * first launch; a launch leaves them zero except word TTSP_FAST_SYNC_FAILED,
 * the count of barrier waits that gave up (sticky until the caller clears it). */
enum { TTSP_FAST_SYNC_WORDS = 192, TTSP_FAST_SYNC_FAILED = 128 };

#ifndef TTSP_HIP_TYPES_ONLY

/* Y[N][M] = epi(X[N][K] . dequant(W)^T). N == 1 runs the HBM-bound GEMV (rows
 * of up to 32768 codes; a longer row takes the tiled kernel), N > 1 the MFMA
 * GEMM (LDS-staged dequantisation; from 256 to 512 rows on large shapes,
 * direct-to-LDS operand streams). epi 1: Y = round(R + round(XW)); epi 2:
 * Y = round(round(silu(R)) * round(XW)); R has Y's shape. Requires K % 128 == 0,
 * K % blocksize == 0, blocksize a power of two >= 64, blocksize2 a power of two
 * (nested only), 16-byte aligned X and W. A8 == NULL selects plain scales.
 * Replaces: the nf4_mma kernel and its launch, app/engine/nf4gemv.py:108-229,
 * 459-477 (argument block built at nf4gemv.py:385-405). */
int ttsp_nf4_gemm(const void* X, int x_dtype, const uint8_t* W, const uint8_t* A8,
                  const float* AMAX, const float* CODE2, float offset, const float* LUT, void* Y,
                  const void* R, int epi, int M, int K, int N, int blocksize, int blocksize2,
                  void* stream);

/* How many K splits ttsp_nf4_gemm_split uses for this shape (1: none, then no
 * workspace is needed). The split is chosen so the output tiles times the
 * splits give every CU a workgroup; from 256 to 512 rows on large or long-K
 * shapes it is the direct-to-LDS kernel's (1, 2 or 4, at most 64 K-steps of
 * 64 codes per split). Host-only. Replaces: the reference's
 * slicing of the rows into MAX_N = 32 launches (app/engine/nf4gemv.py:460-477),
 * which it does instead of splitting K. */
int ttsp_nf4_gemm_splits(int M, int K, int N);

/* ttsp_nf4_gemm with the K loop split `splits` ways (exactly
 * ttsp_nf4_gemm_splits(M, K, N), N > 1): each split writes fp32 partial sums
 * to `work` (splits * N * M floats, 16-byte aligned, the caller's), and a
 * second kernel adds them in split order, rounds and applies the epilogue.
 * splits == 1 is ttsp_nf4_gemm. Replaces: as ttsp_nf4_gemm. */
int ttsp_nf4_gemm_split(const void* X, int x_dtype, const uint8_t* W, const uint8_t* A8,
                        const float* AMAX, const float* CODE2, float offset, const float* LUT,
                        void* Y, const void* R, int epi, int M, int K, int N, int blocksize,
                        int blocksize2, float* work, int splits, void* stream);

/* The K-split launch of ttsp_nf4_gemm_split without its reduce: work gets
 * the fp32 partial sums, split z of output row n at work + (z*N + n)*M, for
 * a consumer that adds them in split order (ttsp_qk_rope_kv_rows_partials).
 * splits must equal ttsp_nf4_gemm_splits(M, K, N) > 1; work 16-byte aligned.
 * Replaces: as ttsp_nf4_gemm_split. */
int ttsp_nf4_gemm_partials(const void* X, int x_dtype, const uint8_t* W, const uint8_t* A8,
                           const float* AMAX, const float* CODE2, float offset, const float* LUT, int M,
                           int K, int N, int blocksize, int blocksize2, float* work, int splits, void* stream);

/* ttsp_nf4_gemm_split (splits > 1) whose reduce also writes the RMSNorm of
 * each output row: Y as ttsp_nf4_gemm_split, and YN[n] = rms_norm(Y[n], G,
 * eps), bit-identical to ttsp_rms_norm on Y. The reduce, the epilogue and the
 * norm are one launch (a workgroup per row). Requires M % 8 == 0, M <= 4096 and
 * 16-byte aligned Y, YN, G, work (and R with an epilogue); else
 * hipErrorInvalidValue. Replaces: wo / w2 of a multi-row block
 * (nf4gemv.matmul, app/engine/nf4gemv.py:460-477) followed by the next
 * RMSNorm launch (fusedops.rms_norm, app/engine/fusedops.py:169-196). */
int ttsp_nf4_gemm_split_norm(const void* X, int x_dtype, const uint8_t* W, const uint8_t* A8,
                             const float* AMAX, const float* CODE2, float offset, const float* LUT,
                             void* Y, const void* R, int epi, int M, int K, int N, int blocksize,
                             int blocksize2, float* work, int splits, const void* G, float eps,
                             void* YN, void* stream);

/* The SwiGLU pair of a multi-row forward in one launch:
 * Y[N][M] = round(round(silu(round(X . W1^T))) * round(X . W3^T)), W1 and W3
 * of one shape [M, K] with the same blocksize and nesting, every value the
 * bits of ttsp_nf4_gemm(W1) then ttsp_nf4_gemm(W3, epi 2, R = the first's
 * output). Served where both of those would run the direct-to-LDS kernel
 * unsplit (ttsp_nf4_gemm_swiglu_fits; e.g. 385-512 rows of 9728 x 2560) or
 * the few-row kernel unsplit (3-32 rows, K up to 10240); other shapes return
 * hipErrorInvalidValue and the caller runs the two launches.
 * 16-byte aligned X, W1, W3. Replaces: w1 then w3 with the SwiGLU gate in
 * the fork's FeedForward for S > 1 (the unfused block the reference runs
 * there, fastpath.py:207-271, through nf4gemv.matmul twice). */
int ttsp_nf4_gemm_swiglu(const void* X, int x_dtype, const uint8_t* W1, const uint8_t* A8_1,
                         const float* AMAX_1, const float* CODE2_1, float offset_1, const uint8_t* W3,
                         const uint8_t* A8_3, const float* AMAX_3, const float* CODE2_3, float offset_3,
                         const float* LUT, void* Y, int M, int K, int N, int blocksize, int blocksize2,
                         void* stream);

/* 1 where ttsp_nf4_gemm_swiglu serves [M, K] weights over N rows (nested:
 * double-quant scales), else 0. Host-only. Replaces: nothing separate. */
int ttsp_nf4_gemm_swiglu_fits(int M, int K, int N, int blocksize, int blocksize2, int nested);

/* The batch-1 matmuls of a decode block in one launch each (K <= 32768,
 * K <= 4096 with NORM_W; ttsp_gemv_shape says whether a shape fits):
 *   W3 == NULL: Y = epi(n(X) . dequant(W1)^T), epi as ttsp_nf4_gemm;
 *   W3 != NULL: Y = round(round(silu(round(n(X) . W1^T))) * round(n(X) . W3^T)),
 *               W1 and W3 of one shape [M, K] (the SwiGLU gate, epi must be 0);
 * n(X) = X, or with NORM_W != NULL the fork's RMSNorm with weight NORM_W and
 * eps, bit-identical to ttsp_rms_norm. Scale arguments as ttsp_nf4_gemm (both
 * weights plain or both nested). Results equal the unfused sequence
 * ttsp_rms_norm -> ttsp_nf4_gemm (-> ttsp_nf4_gemm with epi 2) bit for bit.
 * Replaces: the rms_norm -> nf4_mma and w1 -> w3(silu gate) launch pairs of the
 * reference's decode block (app/engine/fusedlayer.py:222-225, 262-267). */
int ttsp_nf4_gemv_fused(const void* X, int x_dtype, const void* NORM_W, float eps, const uint8_t* W1,
                        const uint8_t* A8_1, const float* AMAX_1, const float* CODE2_1, float offset_1,
                        const uint8_t* W3, const uint8_t* A8_3, const float* AMAX_3,
                        const float* CODE2_3, float offset_3, const float* LUT, void* Y,
                        const void* R, int epi, int M, int K, int blocksize, int blocksize2,
                        void* stream);

/* ttsp_nf4_gemv_fused for N = 1 or 2 activation rows (X [N][K], R and Y
 * [N][M]): each row normalised with NORM_W (if given) as ttsp_rms_norm does,
 * with one weight or the SwiGLU pair (W3 != NULL, epi 0), every weight
 * byte's codes looked up once for both rows, each row's result bit for bit
 * its own one-row launch. Replaces: the rms_norm -> matmul and w1 -> w3
 * (silu gate) launches of the unfused block the reference runs for a short
 * prompt span (app/engine/fastpath.py:207-271 with
 * app/engine/nf4gemv.py:459-477). */
int ttsp_nf4_gemv_fused_rows(const void* X, int x_dtype, const void* NORM_W, float eps, const uint8_t* W1,
                             const uint8_t* A8_1, const float* AMAX_1, const float* CODE2_1, float offset_1,
                             const uint8_t* W3, const uint8_t* A8_3, const float* AMAX_3,
                             const float* CODE2_3, float offset_3, const float* LUT, void* Y,
                             const void* R, int epi, int M, int K, int N, int blocksize, int blocksize2,
                             void* stream);

/* out[k] = round(LUT[q_k] * s_{k / blocksize}) for the n flattened codes, one
 * rounding, out_dtype TTSP_F16/BF16/F32. Replaces: the dequantisation inside
 * nf4_mma (app/engine/nf4gemv.py:154-188) and bitsandbytes' dequantize_4bit
 * that the reference's fallback calls (tests/test_nf4gemv.py:77-80). */
int ttsp_nf4_dequant(const uint8_t* W, const uint8_t* A8, const float* AMAX, const float* CODE2,
                     float offset, const float* LUT, void* out, int out_dtype, long long n,
                     int blocksize, int blocksize2, void* stream);

/* Launch shape the N == 1 GEMV uses for [M, K]: J 64-dword chunks per lane,
 * K split over KS waves, RPW rows per wave. The arithmetic order depends on KS
 * only. Returns nonzero (and zeros) when the GEMV cannot hold the rows
 * (K > 32768). Host-only query; no GPU needed. Replaces: _config (app/engine/
 * nf4gemv.py:234-246). */
int ttsp_gemv_shape(int M, int K, int* J, int* KS, int* RPW);

/* Launch shape ttsp_nf4_gemm uses for N = 1 or 2 activation rows through the
 * GEMV (each weight byte's codes looked up once, one fp32 chain per row; row
 * n's result equals a one-row launch, bit for bit). Returns nonzero (and
 * zeros) when those rows take the MFMA kernels instead (N > 2, or rows longer
 * than the GEMV holds).
 * Host-only query. Replaces: _config for small N (app/engine/nf4gemv.py:
 * 234-246), whose N <= 8 launches are the reference's near-N=1 design point
 * (nf4gemv.py:20-28). */
int ttsp_gemv_rows_shape(int M, int K, int N, int* J, int* KS, int* RPW);

/* Fork RMSNorm over the last axis: Y = round(round(X * r) * Wt),
 * r = 1 / sqrt(sum(X^2) / D + eps); rows x D, D % 8 == 0, dtype F16/BF16,
 * X, Wt and Y 16-byte aligned.
 * Replaces: rms_norm kernel + launch, app/engine/fusedops.py:61-94, 169-196. */
int ttsp_rms_norm(const void* X, const void* Wt, void* Y, int rows, int D, float eps, int dtype,
                  void* stream);

/* Interleaved-pair rotary of X [B, S, heads, 2*half_dim] against
 * F [S, half_dim, 2] (cos, sin) of type ftype: y0 = x0*c - x1*s, y1 = x1*c + x0*s,
 * no fma, one rounding. pairs = X elements / 2; X and Y 4-byte aligned
 * (16-byte aligned with half_dim % 4 == 0 takes the four-pairs-a-thread form).
 * Replaces: rope kernel + launch, app/engine/fusedops.py:103-133, 199-236. */
int ttsp_rope(const void* X, const void* F, int ftype, void* Y, long long pairs, int half_dim,
              int heads, int seq, int dtype, void* stream);

/* Per head of QKV [(nh + 2*nkv) * 128]: optional head norm (QW / KW may be
 * NULL), rotary with F [64, 2], write Q [nh*128] or KC[kv][POS[0]][:], copy V to
 * VC[kv][POS[0]][:]. Caches are [nkv][max_len][128]; POS is one int64 on the
 * device; nothing is written if POS[0] is outside [0, max_len).
 * Replaces: qk_rope_kv, app/engine/fusedlayer.py:56-92, 233-242. */
int ttsp_qk_rope_kv(const void* QKV, const void* QW, const void* KW, float eps, const void* F,
                    int ftype, const long long* POS, void* Q, void* KC, void* VC, int nh, int nkv,
                    int max_len, int dtype, void* stream);

/* ttsp_qk_rope_kv for `rows` positions at once (a prompt prefill): row r
 * reads QKV + r*qkv_row_stride (elements, >= (nh + 2*nkv)*128), its rotary
 * row F + r*128 elements and POS[r], and writes Q + r*nh*128 and cache
 * position POS[r]; rows <= 65535. Same arithmetic per row as the one-position
 * entry. Replaces: the q/k head norms, apply_rotary_emb and KVCache.update of
 * the block's forward for S > 1 (fastpath.py:216-234), which the reference
 * runs as torch ops. */
int ttsp_qk_rope_kv_rows(const void* QKV, long long qkv_row_stride, const void* QW, const void* KW,
                         float eps, const void* F, int ftype, const long long* POS, void* Q, void* KC,
                         void* VC, int nh, int nkv, int max_len, int rows, int dtype, void* stream);

/* ttsp_qk_rope_kv_rows reading a K-split GEMM's fp32 partial sums instead of
 * its output: split z of row r at YP + (z*rows + r)*(nh + 2*nkv)*128 (what
 * ttsp_nf4_gemm_partials writes), summed in split order and rounded as
 * ttsp_nf4_gemm_split's reduce rounds them, so every write equals
 * ttsp_nf4_gemm_split then ttsp_qk_rope_kv_rows bit for bit; 2 <= splits <= 8.
 * Replaces: as ttsp_qk_rope_kv_rows, with the wqkv GEMM's reduce folded in. */
int ttsp_qk_rope_kv_rows_partials(const float* YP, int splits, const void* QW, const void* KW, float eps,
                                  const void* F, int ftype, const long long* POS, void* Q, void* KC, void* VC,
                                  int nh, int nkv, int max_len, int rows, int dtype, void* stream);

/* Grouped-query decode attention of Q [nh*128] over cache positions
 * [0, min(POS[0] + 1, max_len)), split into nchunk chunks of
 * ttsp_attn_chunk() positions, then merged: Y [nh*128]. Scratch (caller's):
 * PM, PL [nh * nchunk] and PACC [nh * nchunk * 128], fp32. nh % nkv == 0,
 * nh / nkv <= 16, nchunk <= 512 (a 32768-position cache); larger values
 * return hipErrorInvalidValue. Replaces: attn_partial + attn_combine,
 * app/engine/fusedlayer.py:95-159, 244-261. */
int ttsp_attn_decode(const void* Q, const void* KC, const void* VC, const long long* POS, float* PM,
                     float* PL, float* PACC, void* Y, int nh, int nkv, int max_len, int nchunk,
                     float scale, int dtype, void* stream);

/* ttsp_attn_decode for `rows` query rows at once: row r reads Q + r*nh*128
 * and POS[r], attends over cache positions [0, min(POS[r] + 1, max_len)) and
 * writes Y + r*nh*128; scratch PM, PL [rows * nh * nchunk], PACC
 * [rows * nh * nchunk * 128]. Each row's result is the one-position entry's
 * for that row, bit for bit (a causal prompt span whose K/V rows are already
 * in the cache). Replaces: the grouped decode attention the reference runs for
 * a span of up to 64 positions (fastpath.py:133-174, 243-250), for a causal
 * mask. */
int ttsp_attn_decode_rows(const void* Q, const void* KC, const void* VC, const long long* POS, float* PM,
                          float* PL, float* PACC, void* Y, int nh, int nkv, int max_len, int nchunk,
                          float scale, int rows, int dtype, void* stream);

/* ttsp_qk_rope_kv_rows then ttsp_attn_decode_rows, for up to 8 rows, in one
 * attention launch and its merge: QKV row r at QKV + r*qkv_rs (the wqkv
 * output, qkv_rs >= (nh + 2 nkv) * 128), rotary row r at F + r*128 values
 * (F 4-byte aligned, ftype as ttsp_rope), positions POS[rows]. Each
 * (kv head, chunk, row) workgroup computes its row's query head and every span
 * row its chunk holds (q/k head norms with QW / KW if given, rotary), and
 * writes its own row's K/V to the cache; Y and the cache rows are bit for bit
 * those of the two entry points. Scratch as ttsp_attn_decode_rows.
 * Replaces: the same reference steps as those two (a short causal prompt
 * span, fusedlayer.py:56-92 and fastpath.py:133-174). */
int ttsp_attn_decode_qkv_rows(const void* QKV, int qkv_rs, const void* QW, const void* KW, float eps,
                              const void* F, int ftype, const long long* POS, void* KC, void* VC, float* PM,
                              float* PL, float* PACC, void* Y, int nh, int nkv, int max_len, int nchunk,
                              float scale, int rows, int dtype, void* stream);

/* qk_rope_kv and the decode attention in one pass: the head norms and rotary
 * of the query heads are applied inside the attention workgroups (from QKV),
 * the new position's K/V row is computed, written to KC/VC[kv][POS[0]] and used
 * by the chunk that holds it; Y [nh*128] as ttsp_attn_decode. With nchunk == 1
 * the merge happens in place (PM/PL/PACC may be NULL); otherwise a second
 * launch merges the chunks. Nothing is written if POS[0] is outside
 * [0, max_len). Results equal ttsp_qk_rope_kv followed by ttsp_attn_decode
 * bit for bit. Replaces: qk_rope_kv + attn_partial + attn_combine,
 * app/engine/fusedlayer.py:56-159, 233-261. */
int ttsp_attn_decode_qkv(const void* QKV, const void* QW, const void* KW, float eps, const void* F,
                         int ftype, const long long* POS, void* KC, void* VC, float* PM, float* PL,
                         float* PACC, void* Y, int nh, int nkv, int max_len, int nchunk, float scale,
                         int dtype, void* stream);

/* ttsp_attn_decode_qkv without scratch arguments, for callers that cannot
 * allocate (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc); it has no counterpart in the reference. The split-K
 * partials live in a device array inside the library, one per GPU, allocated
 * with the library and held until the process ends: nh * nchunk <=
 * ttsp_attn_decode_qkv_noalloc_max_slots() (4096, about 2.1 MB), larger
 * requests return hipErrorInvalidValue. Nothing is allocated and nothing needs
 * clearing (every slot the merge reads is written by the same call). All calls
 * on one GPU share that array: calls that overlap on one GPU (two streams)
 * race. The first call on a device looks the array up and must not be the
 * first thing captured into a graph on a device that has never run it.
 * Results equal ttsp_attn_decode_qkv bit for bit. */
int ttsp_attn_decode_qkv_noalloc(const void* QKV, const void* QW, const void* KW, float eps, const void* F,
                                 int ftype, const long long* POS, void* KC, void* VC, void* Y, int nh, int nkv,
                                 int max_len, int nchunk, float scale, int dtype, void* stream);

/* The largest nh * nchunk ttsp_attn_decode_qkv_noalloc serves (4096). */
int ttsp_attn_decode_qkv_noalloc_max_slots(void);

/* ttsp_attn_decode_qkv for a cache of at most one chunk, and the attention
 * output projection, in one launch: every workgroup of the NF4 GEMV that
 * computes Y = epi(attention . W^T) first computes the whole attention (all
 * nh <= 8 query heads; nkv * max_len <= 128, max_len <= 64) in its own LDS,
 * with ttsp_attn_decode_qkv's arithmetic, rounds it to dtype as x, and the
 * first workgroup writes the new K/V row to KC/VC[kv][POS[0]]. W/A8/AMAX/
 * CODE2/offset/LUT/R/epi/M/blocksize/blocksize2 as ttsp_nf4_gemm with K =
 * nh * 128. Results equal ttsp_attn_decode_qkv followed by ttsp_nf4_gemm
 * (N = 1) bit for bit; with POS[0] outside [0, max_len) nothing is written to
 * the cache and Y is unspecified. Replaces: attention + wo in decode_block,
 * app/engine/fusedlayer.py:233-261 (the fast transformer's short caches). */
int ttsp_attn_nf4_gemv(const void* QKV, const void* QW, const void* KW, float eps, const void* F,
                       int ftype, const long long* POS, void* KC, void* VC, int nh, int nkv, int max_len,
                       float scale, const uint8_t* W, const uint8_t* A8, const float* AMAX,
                       const float* CODE2, float offset, const float* LUT, void* Y, const void* R, int epi,
                       int M, int blocksize, int blocksize2, int dtype, void* stream);

/* Top-k / top-p sampling of one row L [V] (fp16 or bf16 as dtype, V up to
 * ttsp_sample_max_vocab()): the largest top_k = TOPK[0] entries
 * (1..ttsp_sample_max_top_k(), ties by lowest index), sorted; the first and
 * every one whose inclusive cumulative probability under softmax(L) is <=
 * TOPP[0] are kept; OUT[0] = the kept index maximising
 * L[i] / max(TEMP[0], 1e-5) - log(-log(U[i])) (U: one uniform float per
 * index), ties to the lowest index. TEMP and TOPP have L's dtype. One
 * workgroup. Replaces: sample_topk, app/engine/fusedsample.py:28-223. */
int ttsp_sample_topk(const void* L, int V, int dtype, const void* TEMP, const void* TOPP,
                     const long long* TOPK, const float* U, int* OUT, void* stream);

/* The largest top_k ttsp_sample_topk serves (64). Replaces: MAX_TOP_K,
 * app/engine/fusedsample.py:26. */
int ttsp_sample_max_top_k(void);

/* The longest row ttsp_sample_topk serves (32768: the row is held in LDS).
 * The reference's kernel streams rows of any length; a longer row here is
 * declined and the caller's sampler runs (app/engine/fusedsample.py:226-238
 * is that fallback for top_k above MAX_TOP_K). */
int ttsp_sample_max_vocab(void);

/* Cache positions per attention chunk (64). Replaces: CHUNK,
 * app/engine/fusedlayer.py:40. */
int ttsp_attn_chunk(void);

/* Grouped-query attention of S new positions at once (a prefill): for query
 * i and head hd (kv head hd / (nh / nkv)),
 *   Y[i][hd][:] = softmax_j(Q[i][hd] . K[j] * scale, over j < L with
 *                 mask[i][j] != 0) . V[j].
 * Q element (i, hd, d) at Q + i*q_seq_stride + hd*q_head_stride + d, K/V
 * (j, kv, d) likewise with their strides (elements; all multiples of 8),
 * mask one byte per (i, j) at mask + i*mask_row_stride + j (a multiple of
 * 16, >= L), Y [S][nh][128] contiguous; head dim 128, fp16 or bf16 (dtype),
 * nh / nkv <= ttsp_prefill_max_groups(), S <= 2^20, 16-byte aligned bases;
 * other values return hipErrorInvalidValue. A row with no allowed key gives
 * NaN (0/0), as a softmax over all -inf. Replaces: decode_attention for
 * S <= 64 and scaled_dot_product_attention(attn_mask=mask, enable_gqa=True)
 * beyond, app/engine/fastpath.py:133-174 and 244-268. */
int ttsp_prefill_attention(const void* Q, long long q_seq_stride, long long q_head_stride,
                           const void* K, long long k_seq_stride, long long k_head_stride,
                           const void* V, long long v_seq_stride, long long v_head_stride,
                           const void* mask, long long mask_row_stride, void* Y, int S, int nh,
                           int nkv, int L, float scale, int dtype, void* stream);

/* Largest query heads per kv head ttsp_prefill_attention takes (8). */
int ttsp_prefill_max_groups(void);

/* Key splits for ttsp_prefill_attention_split at (S, nkv, L): 1 when the
 * (kv head, 32-query) workgroups already fill the GPU or the keys are few
 * (under 16 blocks of 32), 2 for half a GPU of workgroups over a cached
 * prefix of 1024+ keys, else up to 16 so that a short run of positions over
 * a long cached prefix still spreads over the CUs. Host only. Replaces: nothing (the reference's SDPA picks its own split,
 * app/engine/fastpath.py:244-268). */
int ttsp_prefill_attention_splits(int S, int nkv, int L);

/* ttsp_prefill_attention with the keys split into `splits` (1..16) ranges of
 * whole 32-key blocks over separate workgroups, each writing its unnormalised
 * output, running max and sum to `work` (fp32, 16-byte aligned,
 * splits * S * nh * 130 floats), then one merge launch writing Y. splits = 1
 * is ttsp_prefill_attention (work unused). Same results to rounding: the
 * splits merge in fp32 before the one division. Replaces: the same call as
 * ttsp_prefill_attention. */
int ttsp_prefill_attention_split(const void* Q, long long q_seq_stride, long long q_head_stride,
                                 const void* K, long long k_seq_stride, long long k_head_stride,
                                 const void* V, long long v_seq_stride, long long v_head_stride,
                                 const void* mask, long long mask_row_stride, void* Y, int S, int nh,
                                 int nkv, int L, float scale, int dtype, float* work, int splits,
                                 void* stream);

/* ttsp_prefill_attention_split with the causal mask at the rows' positions:
 * pos (int64, S entries on the device) in place of the mask, query i
 * allowing keys j <= min(pos[i], L - 1). The mask is computed in the kernel
 * rather than read (no mask rows, no scan of them), and the same keys are
 * masked, so Y is bit for bit ttsp_prefill_attention_split's with mask row i
 * = causal_mask[pos[i]][0 .. L), except with nh / nkv = 4, splits = 1 and
 * nkv * ceil(S / 32) >= 128, where four key splits a workgroup merge (the
 * same attention to fp32 rounding). Null pos returns hipErrorInvalidValue.
 * Replaces: scaled_dot_product_attention with the mask forward_generate
 * builds, causal_mask[..., input_pos, :max_seq_len] (app/engine/fastpath.py:9,
 * 244-268; the prefill of app/engine/graphs.py:219-228). */
int ttsp_prefill_attention_causal(const void* Q, long long q_seq_stride, long long q_head_stride,
                                  const void* K, long long k_seq_stride, long long k_head_stride,
                                  const void* V, long long v_seq_stride, long long v_head_stride,
                                  const long long* pos, void* Y, int S, int nh, int nkv, int L, float scale,
                                  int dtype, float* work, int splits, void* stream);

/* out[d] = round(sum_{c < ntok} E[(c*vocab + tok[c]) * D + d]) (tok int32 on the
 * device, clamped into [0, vocab)). Replaces: the codebook-embedding lookup of
 * a decode step (app/engine/graphs.py:124-131 via the fork's _fast_embed /
 * embed). */
int ttsp_embed_sum(const void* E, const int* tok, int ntok, int vocab, int D, void* out, int dtype,
                   void* stream);

/* ttsp_embed_sum for `rows` positions: out[r][d] = round(sum_{c < ntok}
 * E[(c*vocab + tok[c*tok_stride + r]) * D + d]) (tok int32 [ntok][tok_stride]
 * on the device, each clamped into [0, vocab)); row r has the bits of a
 * one-position ttsp_embed_sum of column r. Replaces: the summed codebook
 * embeddings of a prompt span (the prompt's embed in the fork's
 * forward_generate, reached through app/engine/graphs.py:219-231). */
int ttsp_embed_sum_rows(const void* E, const int* tok, long long tok_stride, int ntok, int rows, int vocab,
                        int D, void* out, int dtype, void* stream);

/* out[0] = argmax(X[0..n)), lowest index on ties: greedy decoding in place of
 * the sampler (app/engine/graphs.py:57-73, fusedsample.py). */
int ttsp_argmax(const void* X, int n, int dtype, int* out, void* stream);

/* ttsp_argmax and a one-row ttsp_embed_sum in one launch, the same bits:
 * tok[0] = argmax(X[0..n)), t = that clamped into [0, vocab), tok2[0] = t
 * unless tok2 is NULL, out[0..D) = row t of E [vocab][D]. Replaces: a frame's
 * greedy token and its codebook embedding, app/engine/graphs.py:121-131
 * (_sample, the clamp into the codebook, _fast_embed). */
int ttsp_argmax_embed(const void* X, int n, int dtype, int* tok, int* tok2, const void* E, int vocab, int D,
                      void* out, void* stream);

/* A decode frame's bookkeeping in one launch: history[step[0]] = tokens
 * (int32 [rows][ntok]; skipped when step[0] is outside [0, rows)), step[0] += 1,
 * pos[0] += 1, and the next frame's rotary row frow = F[pos[0]] (row_elems
 * 16-bit values per row of F [npos]; pos clamped into [0, npos)). step and pos
 * are int64. Replaces: the frame advance of app/engine/graphs.py:197-217
 * (codes into the history, pos.add_(1)) and the rotary-row lookup at the
 * next frame's start. */
int ttsp_frame_advance(const int* tokens, int ntok, int* history, int rows, long long* step, long long* pos,
                       const void* F, int npos, int row_elems, void* frow, void* stream);

/* Deterministic synthetic data: element i of a tensor seeded `seed` is a
 * function of splitmix64(splitmix64(seed) ^ i). kind 0: uint8 (top byte);
 * 1/2/3: u*scale + offset as bf16/f16/f32 with u uniform in [-1, 1).
 * No counterpart in the reference: it materialises the random-init weights
 * of the synthetic benchmark model on the device. */
int ttsp_synth_fill(void* out, long long n, unsigned long long seed, int kind, float scale,
                    float offset, void* stream);

/* The fast transformer's codebook steps in one launch: for step i = step0 ..
 * step0 + n_steps - 1 (fast position i, rotary row F[i] of ftype), the
 * n_layers decode blocks (ttsp_nf4_gemv_fused with the norm, the attention
 * and wo as ttsp_attn_nf4_gemv, w1/w3 SwiGLU, w2 with the residual), the
 * final norm (fast_norm) and head, then tokens[i + 1] = argmax of the logits
 * (lowest index on ties), whose clamped row of emb [vocab][dim] is the next
 * step's input; x0 [dim] is the first step's input. logits [vocab] keeps the
 * last step's. The same bits as that launch sequence (one launch per block
 * half, head and ttsp_argmax_embed per step). Workgroups meet at grid
 * barriers in `sync` (TTSP_FAST_SYNC_WORDS words, zero before the first
 * launch); a wait is bounded, and one that gives up counts in
 * sync[TTSP_FAST_SYNC_FAILED] (the results are then not valid). work:
 * ttsp_fast_steps_work_bytes() bytes of activations. Served shapes:
 * ttsp_fast_steps_grid() > 0 (every phase unsplit along K as the GEMV runs
 * it: dim and n_head * 128 of 1024 with FFN 3072, or all of them at most
 * 512; <= 4 layers, <= 8 query heads, max_len <= 64); others, and grids the
 * device cannot hold at once, return hipErrorInvalidValue. Positions must lie
 * in [0, max_len). All weights share blocksize and nesting. Replaces: the
 * codebook loop of sample_frame, app/engine/graphs.py:126-131 (per step:
 * _fast_step over the fast layers and head, _sample, _fast_embed), greedy. */
int ttsp_fast_steps(const ttsp_fast_layer* layers, int n_layers, const ttsp_nf4_weight* head,
                    const void* fast_norm, const void* emb, const float* LUT, const void* F, int ftype,
                    const void* x0, void* work, unsigned* sync, void* logits, int* tokens, int dim, int n_head,
                    int n_kv, int inter, int vocab, int max_len, int step0, int n_steps, float eps,
                    int blocksize, int blocksize2, int dtype, void* stream);

/* Workgroups ttsp_fast_steps launches for these shapes, 0 when it does not
 * serve them (host-only). Replaces: nothing separate (the reference always
 * runs the loop as separate launches). */
int ttsp_fast_steps_grid(int dim, int n_head, int n_kv, int inter, int vocab, int max_len, int n_layers,
                         int blocksize);

/* Bytes of ttsp_fast_steps' activation workspace (host-only). Replaces: the
 * fast transformer's activation buffers inside the captured frame
 * (graphs.py:126-131). */
int ttsp_fast_steps_work_bytes(int dim, int n_head, int n_kv, int inter);

#endif /* TTSP_HIP_TYPES_ONLY */

#ifdef __cplusplus
}
#endif

#endif /* TTSP_HIP_H */
